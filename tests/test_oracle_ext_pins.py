"""Pins for the oracle's draft-step and top-n logprob functions
(oracle/wh_oracle_ext.c).

The Markov bias (runtime/deepseek_v4_ssd/dspark.py:157-165) is checked
against a float64 matrix-vector product under a rounding-error bound, exactly
on integer-valued weights (where every float32 order gives the exact sum), and
across weight formats (bf16 bits widened must equal the float32 path on the
same values).  A swapped operand, a row/column transpose, an off-by-one in
`prev` or a dropped chunk all miss these by orders of magnitude.  The top-n
output is checked against numpy's stable lexicographic sort and a float64
logsumexp, and against hand-written tie and -inf cases.
"""
import numpy as np
import pytest

from whallm_amd.synth import bf16_bits_to_f32, f32_to_bf16_bits


@pytest.mark.parametrize("rank", [8, 64, 256])
def test_markov_matches_float64_within_rounding_bound(oracle, rank):
    rng = np.random.default_rng(rank)
    V = 3001
    w1 = rng.normal(0, 0.05, (V, rank)).astype(np.float32)
    w2 = rng.normal(0, 0.08, (V, rank)).astype(np.float32)
    base = rng.normal(0, 2.0, V).astype(np.float32)
    for prev in (0, 1234, V - 1):
        got = oracle.markov_logits(base, w1, w2, prev).astype(np.float64)
        e = w1[prev].astype(np.float64)
        exact = base.astype(np.float64) + w2.astype(np.float64) @ e
        # float32 accumulation of rank products plus the final add
        bound = (rank + 2) * 2.0 ** -24 * (np.abs(w2.astype(np.float64)) @ np.abs(e) + np.abs(exact))
        assert np.all(np.abs(got - exact) <= bound), prev
        # a neighbouring row's embedding is far outside the bound
        wrong = base.astype(np.float64) + w2.astype(np.float64) @ w1[(prev + 1) % V].astype(np.float64)
        assert np.mean(np.abs(wrong - exact) > bound) > 0.9


def test_markov_exact_on_integer_weights(oracle):
    """Small integers: every partial sum is exact in float32, so any correct
    order gives the exact integer result."""
    rng = np.random.default_rng(5)
    V, rank = 500, 256
    w1 = rng.integers(-8, 9, (V, rank)).astype(np.float32)
    w2 = rng.integers(-8, 9, (V, rank)).astype(np.float32)
    base = rng.integers(-100, 101, V).astype(np.float32)
    for prev in (3, 499):
        got = oracle.markov_logits(base, w1, w2, prev)
        want = base.astype(np.int64) + w2.astype(np.int64) @ w1[prev].astype(np.int64)
        assert np.array_equal(got.astype(np.int64), want)


def test_markov_bf16_bits_equal_float32_path(oracle):
    rng = np.random.default_rng(6)
    V, rank = 1024, 256
    b1 = f32_to_bf16_bits(rng.normal(0, 0.05, (V, rank)).astype(np.float32))
    b2 = f32_to_bf16_bits(rng.normal(0, 0.08, (V, rank)).astype(np.float32))
    base = rng.normal(0, 2.0, V).astype(np.float32)
    got = oracle.markov_logits(base, b1, b2, 17)
    want = oracle.markov_logits(base, bf16_bits_to_f32(b1), bf16_bits_to_f32(b2), 17)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_markov_rejects_bad_shapes(oracle):
    w = np.zeros((10, 12), np.float32)  # rank not a multiple of 8
    with pytest.raises(ValueError):
        oracle.markov_logits(np.zeros(10, np.float32), w, w, 0)
    w = np.zeros((10, 16), np.float32)
    with pytest.raises(ValueError):
        oracle.markov_logits(np.zeros(10, np.float32), w, w, 10)  # prev out of range


def _np_top(x, n):
    order = np.lexsort((np.arange(x.size), -x.astype(np.float64)))
    m = np.max(x.astype(np.float64))
    lse = m + np.log(np.sum(np.exp(x.astype(np.float64) - m)))
    return order[:n], (x[order[:n]].astype(np.float64) - lse).astype(np.float32)


def test_top_logprobs_against_numpy(oracle):
    rng = np.random.default_rng(8)
    B, V, n = 6, 20000, 20
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    x[1] = np.round(x[1])  # many exact ties: ids break them, lowest first
    x[2, rng.random(V) < 0.5] = -np.inf
    ids, lps = oracle.top_logprobs(x, n)
    for b in range(B):
        wi, wl = _np_top(x[b], n)
        assert np.array_equal(ids[b], wi), b
        assert np.allclose(lps[b], wl, rtol=0, atol=2e-6), b
    # the logprobs of the whole row would sum to one in probability
    full_ids, full = oracle.top_logprobs(x[:1], V)
    assert abs(np.sum(np.exp(full.astype(np.float64))) - 1.0) < 1e-5
    assert np.array_equal(np.sort(full_ids[0]), np.arange(V))


def test_top_logprobs_hand_cases(oracle):
    x = np.array([1.0, 3.0, 3.0, 2.0, -np.inf], np.float32)
    ids, lps = oracle.top_logprobs(x, 5)
    assert ids[0].tolist() == [1, 2, 3, 0, 4]
    lse = np.log(np.exp(1.0) + 2 * np.exp(3.0) + np.exp(2.0))
    assert np.allclose(lps[0][:4], np.array([3.0, 3.0, 2.0, 1.0]) - lse, atol=1e-6)
    assert lps[0][4] == -np.inf
    ids, lps = oracle.top_logprobs(np.full(4, -np.inf, np.float32), 2)
    assert ids[0].tolist() == [0, 1] and np.all(lps == -np.inf)
    with pytest.raises(ValueError):
        oracle.top_logprobs(x, 6)
