"""wh_sample_noalloc (the entry point that allocates nothing) against
wh_sample with a caller workspace, through the C ABI: two calls in a row,
the second on a smaller input, then the first shape again; results must be
identical to the existing entry point's and to the oracle's."""
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


def _case(big, seed):
    from whallm_amd import synth

    rng = np.random.default_rng(seed)
    if big:
        B, V, H = 64, synth.V_QWEN, 2048
        bits = synth.f32_to_bf16_bits(rng.normal(0, 3, (B, V)).astype(np.float32))
        x = synth.bf16_bits_to_f32(bits)
        kw = dict(temperature=1.0, top_p=0.9, min_p=0.05, presence_penalty=0.5, frequency_penalty=0.3,
                  presence_context=0, frequency_context=0, chain=0)
    else:
        B, V, H = 8, 20000, 100
        bits = None
        x = (2.5 * rng.standard_t(3, (B, V))).astype(np.float32)
        kw = dict(temperature=0.9, top_k=40, top_p=0.95, repetition_penalty=1.1, chain=1)
    hist = rng.integers(0, V, (B, H)).astype(np.int32)
    u = rng.random(B, dtype=np.float32)
    return x, bits, hist, u, kw


@pytest.mark.parametrize("order", [(True, False, True)])
def test_noalloc_matches_workspace_entry_point(dev, oracle, order):
    from whallm_amd import sampling

    for i, big in enumerate(order):
        x, bits, hist, u, kw = _case(big, 3000 + i)
        B = x.shape[0]
        xt = torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16) if bits is not None \
            else torch.from_numpy(x).to(dev)
        args = dict(history=torch.from_numpy(hist).to(dev), uniforms=torch.from_numpy(u).to(dev), return_kept=True, **kw)
        announce(f"wh_sample_noalloc call {i}: B={B} V={x.shape[1]} {kw}")
        t_na, k_na = sampling.sample(xt, engine="noalloc", **args)
        t_ws, k_ws = sampling.sample(xt, engine="auto", **args)
        t_na, k_na, t_ws, k_ws = (v.cpu().numpy() for v in (t_na, k_na, t_ws, k_ws))
        assert np.array_equal(t_na, t_ws) and np.array_equal(k_na, k_ws), i
        p = oracle.make_params(B, **kw)
        ot, ok = oracle.sample(x, p, u, hist)
        assert np.array_equal(t_na, ot) and np.array_equal(k_na, ok), i


def test_noalloc_rejects_beyond_its_scratch(dev):
    from whallm_amd import sampling

    x = torch.zeros(2048, 151936, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="WH_NOALLOC_SCRATCH_BYTES"):
        sampling.sample(x, temperature=1.0, top_p=0.9, engine="noalloc", uniforms=torch.zeros(2048, device=dev))
