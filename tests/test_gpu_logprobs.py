"""wh_top_logprobs on the GPU against the oracle's top-n (value descending,
id ascending; logsumexp in float64).  Ids must match exactly; logprobs within
2e-6 absolute (1e-5 relative in probability would allow 1e-5)."""
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


def _rows(rng, B, V, kind):
    x = rng.normal(0, 3, (B, V))
    if kind == "ties":
        x = np.round(x * 2) / 2
    elif kind == "masked":
        x[rng.random((B, V)) < 0.6] = -np.inf
    elif kind == "peaked":
        x[:, rng.integers(0, V, 3)] += 25.0
    return x.astype(np.float32)


def _check(oracle, x, ids, lps, n):
    oi, ol = oracle.top_logprobs(x, n)
    assert np.array_equal(ids, oi), np.nonzero((ids != oi).any(1))[0][:5]
    fin = np.isfinite(ol)
    assert np.array_equal(np.isfinite(lps), fin)
    assert np.all(lps[~fin] == ol[~fin])
    assert np.allclose(lps[fin], ol[fin], rtol=0, atol=2e-6)


@pytest.mark.parametrize("V,n,kind", [
    (1, 1, "normal"), (5, 5, "ties"), (4096, 20, "normal"), (4097, 64, "ties"), (20000, 7, "masked"),
    (151936, 20, "ties"), (129280, 64, "peaked"), (262144, 64, "normal"), (262144, 1, "ties"),
])
def test_top_logprobs_f32(dev, oracle, V, n, kind):
    from whallm_amd.logprobs import top_logprobs

    rng = np.random.default_rng(V + n)
    B = 5
    x = _rows(rng, B, V, kind)
    tok = rng.integers(-1, V + 1, B).astype(np.int32)
    announce(f"wh_top_logprobs f32 B={B} V={V} n={n} {kind}")
    ids, lps, tlp = top_logprobs(torch.from_numpy(x).to(dev), n, tokens=torch.from_numpy(tok).to(dev))
    _check(oracle, x, ids.cpu().numpy(), lps.cpu().numpy(), n)
    tlp = tlp.cpu().numpy()
    for b in range(B):
        if 0 <= tok[b] < V and np.isfinite(x[b, tok[b]]):
            r = x[b].astype(np.float64)
            m = r.max()
            want = x[b, tok[b]] - (m + np.log(np.sum(np.exp(r - m))))
            assert abs(tlp[b] - want) <= 2e-6
        else:
            assert tlp[b] == -np.inf


def test_top_logprobs_bf16_and_strided(dev, oracle):
    from whallm_amd.logprobs import top_logprobs
    from whallm_amd.synth import bf16_bits_to_f32, f32_to_bf16_bits

    rng = np.random.default_rng(31)
    B, V, n = 64, 151936, 20
    bits = f32_to_bf16_bits(_rows(rng, B, V, "normal"))
    x = bf16_bits_to_f32(bits)
    announce(f"wh_top_logprobs bf16 B={B} V={V} n={n}")
    t = torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)
    ids, lps, _ = top_logprobs(t, n)
    _check(oracle, x, ids.cpu().numpy(), lps.cpu().numpy(), n)
    # rows of a wider buffer (row_stride > V)
    wide = torch.from_numpy(_rows(rng, 6, 5000, "ties")).to(dev)
    view = wide[:, :4321]
    announce("wh_top_logprobs strided rows")
    ids, lps, _ = top_logprobs(view, 9)
    _check(oracle, np.ascontiguousarray(view.cpu().numpy()), ids.cpu().numpy(), lps.cpu().numpy(), 9)


def test_top_logprobs_all_neg_inf_row(dev, oracle):
    from whallm_amd.logprobs import top_logprobs

    x = np.full((3, 9000), -np.inf, np.float32)
    x[1, 4444] = 1.5
    x[2, ::7] = 0.0
    announce("wh_top_logprobs -inf rows")
    ids, lps, _ = top_logprobs(torch.from_numpy(x).to(dev), 10)
    _check(oracle, x, ids.cpu().numpy(), lps.cpu().numpy(), 10)
    assert ids[0].tolist() == list(range(10))
    assert lps[1, 0].item() == 0.0


def test_top_logprobs_rejects(dev):
    from whallm_amd.logprobs import top_logprobs

    x = torch.zeros(2, 100, device=dev)
    with pytest.raises(ValueError):
        top_logprobs(x, 0)
    with pytest.raises(ValueError):
        top_logprobs(x, 65)
    with pytest.raises(ValueError):
        top_logprobs(torch.zeros(2, 10, device=dev), 11)
