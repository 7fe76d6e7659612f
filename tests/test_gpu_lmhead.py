"""The MFMA LM head and its fused greedy selection on the GPU.

Logits: against a float64 product of the same bf16 inputs, within the
float32 accumulation bound K * 2^-24 * sum |x w| per entry.  Greedy: the
fused kernel's tokens must equal the lowest-index argmax of the unfused
logits and the oracle's temperature-0 selection on them, including exact
ties (duplicated weight rows).  Sampled rows through lm_head_sample must be
the oracle's tokens on the GPU's logits."""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def announce(msg):
    sys.stderr.write(f"[gpu-case] {msg}\n")
    sys.stderr.flush()


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from whallm_amd import _lib

    _lib.lib()
    return torch.device("cuda:0")


def _inputs(dev, M, K, V, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = (torch.randn(M, K, device=dev, generator=g) * 0.5).to(torch.bfloat16)
    w = (torch.randn(V, K, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    return x, w


# V = 129,280 and 131,000 take 8-wave workgroups at M <= 32 (their grids
# spread evenly over the CUs), 131,000 with a part-filled last workgroup;
# the others take 4 waves, or two x row blocks at M > 32
@pytest.mark.parametrize("M,K,V", [(1, 256, 1000), (7, 2560, 151936), (33, 512, 5003), (64, 2560, 151936),
                                   (16, 4096, 129280), (32, 64, 129), (3, 512, 131000), (32, 256, 131000)])
def test_lm_head_logits_and_greedy(dev, oracle, M, K, V):
    from whallm_amd.lmhead import lm_head, lm_head_greedy

    x, w = _inputs(dev, M, K, V, M * 7 + K)
    if V > 200:
        w[V - 100] = w[17]  # exact tie with a lower index
        w[V // 2] = w[V - 3]
    announce(f"wh_lmhead_logits M={M} K={K} V={V}")
    got = lm_head(x, w)
    xd, wd = x.double(), w.double()
    ref = xd @ wd.T
    bound = K * 2.0 ** -24 * (xd.abs() @ wd.abs().T) + 1e-30
    err = (got.double() - ref).abs()
    assert bool((err <= bound).all()), float((err / bound).max())
    announce(f"wh_lmhead_greedy M={M} K={K} V={V}")
    tok = lm_head_greedy(x, w).cpu().numpy()
    lg = got.cpu().numpy()
    assert np.array_equal(tok, np.argmax(lg, axis=1).astype(np.int32))  # numpy: first maximum
    ot, _ = oracle.sample(lg, oracle.make_params(M, temperature=0.0), np.zeros(M, np.float32))
    assert np.array_equal(tok, ot)


def test_lm_head_greedy_exact_ties(dev):
    """Rows of x that make two vocabulary entries tie exactly: the lower
    index wins, also when it lies in a later workgroup's columns' reach."""
    from whallm_amd.lmhead import lm_head, lm_head_greedy

    M, K, V = 5, 512, 40000
    x, w = _inputs(dev, M, K, V, 99)
    hot = torch.ones(K, device=dev, dtype=torch.bfloat16)
    for v in (31000, 129, 39999, 7):
        w[v] = hot  # identical rows: identical logits
    x[:] = 0.25
    announce("wh_lmhead_greedy ties")
    tok = lm_head_greedy(x, w).cpu().numpy()
    lg = lm_head(x, w).cpu().numpy()
    assert np.all(lg[:, 7] == lg[:, 31000])
    assert np.all(tok == 7)


def test_lm_head_sample_paths(dev, oracle):
    from whallm_amd.lmhead import lm_head, lm_head_sample

    M, K, V = 24, 1024, 151936
    x, w = _inputs(dev, M, K, V, 5)
    rng = np.random.default_rng(3)
    u = rng.random(M, dtype=np.float32)
    lg = lm_head(x, w).cpu().numpy()
    kw = dict(temperature=0.9, top_p=0.9, top_k=40, min_p=0.05)
    announce("lm_head_sample sampled")
    t = lm_head_sample(x, w, uniforms=torch.from_numpy(u).to(dev), **kw).cpu().numpy()
    ot, _ = oracle.sample(lg, oracle.make_params(M, chain=0, **kw), u)
    assert np.array_equal(t, ot)
    announce("lm_head_sample greedy (fused)")
    t0 = lm_head_sample(x, w, temperature=0.0).cpu().numpy()
    assert np.array_equal(t0, np.argmax(lg, axis=1))


def test_lm_head_rejects(dev):
    from whallm_amd.lmhead import lm_head

    x = torch.zeros(2, 100, device=dev, dtype=torch.bfloat16)
    w = torch.zeros(10, 100, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        lm_head(x, w)  # K not a multiple of 64
    with pytest.raises(ValueError):
        lm_head(torch.zeros(65, 128, device=dev, dtype=torch.bfloat16),
                torch.zeros(10, 128, device=dev, dtype=torch.bfloat16))


@pytest.mark.parametrize("M,K,V", [(1, 2560, 151936), (16, 1024, 129280), (64, 2560, 151936), (33, 512, 5003),
                                   (5, 512, 131000)])
def test_lm_head_sample_fused_wide(dev, oracle, M, K, V):
    """Rows filtered by top-p alone (or not at all): the product emits the
    sampler's slice maxima.  Tokens equal lm_head() then sample(), and the
    oracle on the same logits; the logits themselves are the product's."""
    from whallm_amd import sampling
    from whallm_amd.lmhead import lm_head, lm_head_sample

    x, w = _inputs(dev, M, K, V, 300 + M)
    ref = lm_head(x, w)
    lg = ref.cpu().numpy()
    rng = np.random.default_rng(M + V)
    for chain, T, top_p in ((0, 0.2, 0.98), (1, 1.0, 0.9), (0, 0.7, 1.0)):
        u = rng.random(M, dtype=np.float32)
        ut = torch.from_numpy(u).to(dev)
        kw = dict(temperature=T, top_p=top_p, chain="mlx" if chain == 0 else "whallm")
        announce(f"wh_lmhead_sample fused M={M} K={K} V={V} {kw}")
        tok, logits = lm_head_sample(x, w, uniforms=ut, return_logits=True, **kw)
        assert torch.equal(logits, ref)
        assert set(sampling.last_paths(dev, M).cpu().numpy().tolist()) <= {6, 1}
        unf = sampling.sample(ref, uniforms=ut, **kw)
        ot, _ = oracle.sample(lg, oracle.make_params(M, temperature=T, top_p=top_p, chain=chain), u)
        assert np.array_equal(tok.cpu().numpy(), unf.cpu().numpy())
        assert np.array_equal(tok.cpu().numpy(), ot)


def test_lm_head_sample_unfused_routes(dev, oracle):
    """Penalties (the epilogue sees raw logits) take the product, then the
    sampler; the tokens still match the oracle."""
    from whallm_amd.lmhead import lm_head, lm_head_sample

    M, K, V = 8, 512, 30000
    x, w = _inputs(dev, M, K, V, 41)
    lg = lm_head(x, w).cpu().numpy()
    rng = np.random.default_rng(2)
    hist = rng.integers(0, V, (M, 64)).astype(np.int32)
    u = rng.random(M, dtype=np.float32)
    kw = dict(temperature=0.8, top_p=0.95, presence_penalty=0.5, presence_context=32)
    announce("wh_lmhead_sample with penalties")
    tok = lm_head_sample(x, w, uniforms=torch.from_numpy(u).to(dev), history=torch.from_numpy(hist).to(dev), **kw)
    ot, _ = oracle.sample(lg, oracle.make_params(M, chain=0, **kw), u, hist)
    assert np.array_equal(tok.cpu().numpy(), ot)
