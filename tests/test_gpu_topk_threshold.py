"""GPU parity for the slice kernel's top-k candidate threshold.

The threshold comes from histograms of the group maxima: for k <= 64 one
over the 8 nats below the slice max (1024 bins of 1/128 nat), else (or when
that holds fewer than k values) the ladder's rungs and one histogram over
the bracketing interval.  A bin counts only the values that reach its lower
edge, so the threshold must leave at least k elements at or above it
whatever the rounding.  The rows below put values exactly on bin edges, tie
the k-th value, move the k-th value far below an outlier (the first
histogram falls short and the ladder runs), spread large k over a
heavy-tailed row, and let penalised (listed) elements take part.  Tokens and
kept-set sizes must equal the oracle's, and at most a few rows may take the
exact engine (the fast engine's own threshold is what is checked; a top-p
cut the normaliser bounds cannot settle on such flat rows is such a row,
before and after the histograms alike).
"""
import sys
import zlib

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
V = 151936


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


def _rows(kind, rng, B):
    x = rng.normal(0.0, 2.0, (B, V))
    if kind == "edges":
        # values on the 1/128-nat grid below each row's max: every candidate
        # lies exactly on a bin edge of the near histogram
        top = 9.0
        x = np.minimum(x, top - 0.5)
        for r in range(B):
            ids = rng.choice(V, 400, replace=False)
            x[r, ids] = top - rng.integers(0, 900, 400) / 128.0
            x[r, ids[0]] = top
    elif kind == "ties":
        # a long run of exact ties around the k-th value
        for r in range(B):
            ids = rng.choice(V, 300, replace=False)
            x[r, ids] = 7.0
            x[r, ids[:10]] = 7.25
    elif kind == "outlier":
        # one value 40 nats above the rest: fewer than k values within 8
        # nats of some slices' max, so the ladder finds the bracket
        for r in range(B):
            x[r, rng.integers(0, V)] = 48.0
    elif kind == "heavy":
        # t(3) tails: large k reached deep below the max
        x = 3.0 * rng.standard_t(3, (B, V))
    return x.astype(np.float32)


CASES = [("edges", 20, "f32"), ("edges", 64, "bf16"), ("ties", 50, "f32"), ("ties", 200, "bf16"),
         ("outlier", 30, "f32"), ("outlier", 500, "bf16"), ("heavy", 700, "f32"), ("heavy", 12, "bf16")]


@pytest.mark.parametrize("kind,k,dtype", CASES)
def test_topk_threshold_parity(dev, oracle, kind, k, dtype):
    from whallm_amd import sampling, synth

    rng = np.random.default_rng(zlib.crc32(f"{kind}-{k}-{dtype}".encode()))
    B = 16
    x = _rows(kind, rng, B)
    if dtype == "bf16":
        bits = synth.f32_to_bf16_bits(x)
        x = synth.bf16_bits_to_f32(bits)
        xd = torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        xd = torch.from_numpy(x).to(dev)
    u = rng.random(B, dtype=np.float32)
    ud = torch.from_numpy(u).to(dev)
    for chain, extra in ((0, dict(top_p=0.9, min_p=0.0)), (1, dict(top_p=1.0, min_p=0.01))):
        kw = dict(temperature=0.8, top_k=k, **extra)
        p = oracle.make_params(B, chain=chain, **kw)
        ot, ok = oracle.sample(x, p, u, None, None)
        announce(f"wh_sample top-k threshold {kind} k={k} {dtype} chain={chain}")
        tok, kept = sampling.sample(xd, uniforms=ud, return_kept=True, chain=chain, **kw)
        paths = sampling.last_paths(dev, B).cpu().numpy()
        assert np.array_equal(kept.cpu().numpy(), ok), (kind, k, dtype, chain)
        assert np.array_equal(tok.cpu().numpy(), ot), (kind, k, dtype, chain)
        assert np.sum((paths == 1) | (paths == 3)) <= 2, paths


def test_topk_threshold_with_penalised_elements(dev, oracle):
    """History ids on the highest logits: penalised elements are listed apart
    from the groups and enter both histograms as single values."""
    from whallm_amd import sampling, synth

    rng = np.random.default_rng(77)
    B, H = 16, 512
    x = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    hist = np.empty((B, H), np.int32)
    for r in range(B):
        top = np.argsort(-x[r])[:300]
        hist[r] = np.concatenate([top, rng.choice(V, H - 300, replace=False)]).astype(np.int32)
    bits = synth.f32_to_bf16_bits(x)
    x = synth.bf16_bits_to_f32(bits)
    xd = torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)
    hl = np.full(B, H, np.int32)
    u = rng.random(B, dtype=np.float32)
    for k in (20, 300):
        kw = dict(temperature=0.7, top_k=k, top_p=0.9, min_p=0.0, repetition_penalty=1.3, presence_penalty=0.5,
                  frequency_penalty=0.25, repetition_context=H, presence_context=H, frequency_context=H)
        p = oracle.make_params(B, chain=1, **kw)
        ot, ok = oracle.sample(x, p, u, hist, hl)
        announce(f"wh_sample top-k threshold with penalties k={k}")
        tok, kept = sampling.sample(xd, uniforms=torch.from_numpy(u).to(dev), history=torch.from_numpy(hist).to(dev),
                                    history_len=torch.from_numpy(hl).to(dev), return_kept=True, chain=1, **kw)
        paths = sampling.last_paths(dev, B).cpu().numpy()
        assert np.array_equal(kept.cpu().numpy(), ok), k
        assert np.array_equal(tok.cpu().numpy(), ot), k
        assert np.sum((paths == 1) | (paths == 3)) <= 2, paths
