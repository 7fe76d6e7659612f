"""Pins for the faithful float32 replay of the reference's op order
(oracle/wh_oracle.c: who_sample_rows_faithful, who_verify_faithful).

The faithful replay is what the GPU's results are compared against for the
boundary-mismatch report, so each of its reference-specific choices gets a
check that a plausible mistake fails:

  * the strict `cumulative > 1 - top_p` of mlx_lm apply_top_p and the tie
    order of its ascending stable argsort (dspark.py:369 calls it);
  * the two temperature forms: `logprobs * (1 / T)` in mlx_lm make_sampler
    (chain A) and `logprobs / max(T, 1e-5)` in sampling_logprobs
    (dspark.py:374, chain B), each on a row where the other form draws a
    different token;
  * min-p compared on the normalised logprobs (dspark.py:370-371 passes
    logprobs), on a row where comparing raw logits keeps a different set;
  * _verify (dspark.py:857-898): the reference's known answers, the closed
    forms (p == q always accepts, disjoint supports resample p, a zero
    residual falls back to the target row) and the speculative-sampling
    identity;
  * agreement with the contract oracle everywhere except within 1e-6 of a
    cumulative-probability boundary (tests/boundary.py restates those
    boundaries in float64).

The small emulations below replay the faithful op sequence in numpy float32
scalars with libm's expf / logf (the functions the oracle calls), so that a
row can be built on which two candidate op orders disagree; the assertion is
then which of the two the oracle follows.
"""
import ctypes
import ctypes.util
import json
import math
import os

import numpy as np
import pytest

from boundary import sample_margins, verify_margin

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = json.load(open(os.path.join(HERE, "golden", "reference_cases.json")))
F = np.float32
_m = ctypes.CDLL(ctypes.util.find_library("m"))
_m.expf.restype = ctypes.c_float
_m.expf.argtypes = [ctypes.c_float]
_m.logf.restype = ctypes.c_float
_m.logf.argtypes = [ctypes.c_float]


def expf(x):
    return F(_m.expf(float(x)))


def logf(x):
    return F(_m.logf(float(x)))


def lse_f32(v):
    m = max(v)
    if m == F(-np.inf):
        return m
    s = F(0.0)
    for x in v:
        s = F(s + expf(F(x - m)))
    return F(m + logf(s))


def draw_f32(z, u):
    """The replay's draw: float32 weights expf(z - max), accumulated in float64."""
    m = max(z)
    tot = 0.0
    for x in z:
        tot += float(expf(F(x - m)))
    tgt = float(F(u)) * tot
    c = 0.0
    last = 0
    for i, x in enumerate(z):
        w = expf(F(x - m))
        if w == 0:
            continue
        c += float(w)
        last = i
        if c > tgt:
            return i
    return last


def emulate_token(x, T, u, form):
    """The faithful row with no filters: logprobs, then the temperature
    `form` -- 'recip' lp * fp32(1/T) or 'div' lp / fp32(max(T, 1e-5)), with
    '_renorm' a second logsumexp subtracted -- then the draw."""
    x = [F(v) for v in x]
    lse = lse_f32(x)
    lp = [F(v - lse) for v in x]
    if form.startswith("recip"):
        inv = F(1.0 / T)
        z = [F(v * inv) for v in lp]
    else:
        tc = F(max(T, 1e-5))
        z = [F(v / tc) for v in lp]
    if form.endswith("_renorm"):
        l2 = lse_f32(z)
        z = [F(v - l2) for v in z]
    return draw_f32(z, u)


def first_u_of_token1(x, T, form):
    """Smallest float32 u in [0, 1) at which the 2-token row draws token 1."""
    lo, hi = 0, int(np.float32(0.99999994).view(np.uint32))
    if emulate_token(x, T, np.uint32(hi).view(np.float32), form) == 0:
        return None
    while lo < hi:
        mid = (lo + hi) // 2
        if emulate_token(x, T, np.uint32(mid).view(np.float32), form) == 1:
            hi = mid
        else:
            lo = mid + 1
    return np.uint32(lo).view(np.float32)


# --------------------------------------------------------------------------
# top-p: strict inequality and the ascending-stable tie order
# --------------------------------------------------------------------------
def _faithful_sweep(oracle, x, p, n=2048):
    u = (np.arange(n, dtype=np.float64) / n).astype(np.float32)
    X = np.repeat(np.asarray(x, np.float32)[None], n, 0)
    return oracle.sample_faithful(X, np.repeat(p, n), u)[0]


@pytest.mark.parametrize("chain", [0, 1])
def test_faithful_top_p_ties_keep_higher_ids(oracle, chain):
    # 8 equal logits: every probability is exactly 1/8 and every cumulative
    # sum exact.  The ascending stable sort orders ids 0..7, so the nucleus
    # of 0.5 (keep cum > 0.5) is ids 4..7; a descending or unstable order
    # would keep lower ids.
    x = np.zeros(8, np.float32)
    p = oracle.make_params(1, temperature=1.0, top_p=0.5, chain=chain)
    assert oracle.sample_faithful(x, p, 0.3)[1][0] == 4
    assert set(_faithful_sweep(oracle, x, p).tolist()) == {4, 5, 6, 7}


@pytest.mark.parametrize("chain", [0, 1])
def test_faithful_top_p_cut_is_strict(oracle, chain):
    # top_p = 0.625: theta = fp32(1 - 0.625) = 0.375 exactly, and id 2's
    # ascending cumulative sum is exactly 3/8: `>` drops it, `>=` would keep it
    x = np.zeros(8, np.float32)
    p = oracle.make_params(1, temperature=1.0, top_p=0.625, chain=chain)
    assert oracle.sample_faithful(x, p, 0.3)[1][0] == 5
    assert set(_faithful_sweep(oracle, x, p).tolist()) == {3, 4, 5, 6, 7}


def theta_split_row(oracle):
    """A row of 8 zeros and one value d < 0 whose contract mass W makes the
    last token's share W / Z fall in (0.1f, 0.100000024f]: kept under MLX's
    threshold fp32(1 - 0.9) = 0.1f, dropped under fp32(1 - fp32(0.9))."""
    lo, hi = float(np.float32(0.1)), float(np.nextafter(np.float32(0.1), np.float32(1)) + 2 * 7.450580596923828e-09)
    assert np.float32(hi) == np.float32(1.0 - np.float32(0.9))
    d = np.float32(-0.1178)
    for _ in range(20000):
        W = int(oracle.exp_fix44(np.array([d], np.float32))[0])
        Z = 8 * (1 << 44) + W
        r = W / Z
        if lo < r <= hi and W > math.floor(lo * Z) and W <= math.floor(hi * Z):
            return np.array([0.0] * 8 + [float(d)], np.float32)
        d = np.nextafter(d, np.float32(0.0) if r < lo else np.float32(-1.0), dtype=np.float32)
    raise AssertionError("no row found")


def test_top_p_threshold_comes_from_the_double(oracle):
    # MLX forms 1 - top_p in double and rounds it to float32: top_p = 0.9
    # gives 0.1f, not fp32(1 - fp32(0.9)) = 0.100000024f
    x = theta_split_row(oracle)
    for chain in (0, 1):
        p = oracle.make_params(1, temperature=1.0, top_p=0.9, chain=chain)
        assert oracle.sample(x, p, 0.5)[1][0] == 9
        p = oracle.make_params(1, temperature=1.0, top_p=float(np.float32(0.9)), chain=chain)
        assert oracle.sample(x, p, 0.5)[1][0] == 8


# --------------------------------------------------------------------------
# the two temperature forms
# --------------------------------------------------------------------------
def _find_form_split(want, other, seed):
    rng = np.random.default_rng(seed)
    for _ in range(4000):
        T = float(rng.uniform(0.2, 2.5))
        x = [F(0.0), F(-rng.uniform(0.05, 3.0))]
        ua = first_u_of_token1(x, T, want)
        ub = first_u_of_token1(x, T, other)
        if ua is None or ub is None or ua == ub:
            continue
        u = min(ua, ub)
        ta, tb = emulate_token(x, T, u, want), emulate_token(x, T, u, other)
        if ta != tb:
            return np.array(x, np.float32), T, u, ta
    raise AssertionError("no row found on which the two temperature forms draw differently")


FORMS = ("recip", "div", "recip_renorm", "div_renorm")


@pytest.mark.parametrize("chain,form", [(0, "recip"), (1, "div_renorm")])
def test_faithful_temperature_form_decides_the_draw(oracle, chain, form):
    # chain A: categorical(logprobs * (1 / T)) (mlx_lm make_sampler);
    # chain B: scaled = logprobs / max(T, 1e-5), scaled - logsumexp(scaled)
    # (dspark.py:374-375).  Against each other form, a row and a uniform on
    # which the two draw different tokens: the oracle must draw `form`'s.
    for k, other in enumerate(f for f in FORMS if f != form):
        x, T, u, tok = _find_form_split(form, other, seed=41 + 7 * chain + k)
        p = oracle.make_params(1, temperature=T, chain=chain)
        assert oracle.sample_faithful(x, p, np.float32(u))[0][0] == tok, other


def test_faithful_top_p_threshold_comes_from_the_double(oracle):
    # 8 zeros and one value d whose float32 probability expf(d - lse) lies in
    # (0.1f, 0.100000024f]: its ascending cumulative sum (it is the smallest)
    # exceeds fp32(1 - 0.9) = 0.1f but not fp32(1 - fp32(0.9))
    lo, hi = np.float32(0.1), np.float32(1.0 - np.float32(0.9))
    d = np.float32(-0.1178)
    for _ in range(50000):
        x = [F(0.0)] * 8 + [d]
        pr = expf(F(d - lse_f32(x)))
        if lo < pr <= hi:
            break
        d = np.nextafter(d, np.float32(0.0) if pr < lo else np.float32(-1.0), dtype=np.float32)
    else:
        raise AssertionError("no row found")
    x = np.array(x, np.float32)
    for chain in (0, 1):
        assert oracle.sample_faithful(x, oracle.make_params(1, temperature=1.0, top_p=0.9, chain=chain), 0.5)[1][0] == 9
        p32 = oracle.make_params(1, temperature=1.0, top_p=float(np.float32(0.9)), chain=chain)
        assert oracle.sample_faithful(x, p32, 0.5)[1][0] == 8


# --------------------------------------------------------------------------
# min-p on the normalised logprobs
# --------------------------------------------------------------------------
def _minp_keep(x, min_p, on_logprobs):
    x = [F(v) for v in x]
    c = F(math.log(min_p))
    if on_logprobs:
        lse = lse_f32(x)
        v = [F(a - lse) for a in x]
    else:
        v = x
    thr = F(max(v) + c)
    return sum(1 for a in v if not a < thr)


def test_faithful_min_p_compares_logprobs(oracle):
    rng = np.random.default_rng(43)
    found = 0
    for _ in range(20000):
        min_p = float(rng.uniform(0.01, 0.9))
        c = F(math.log(min_p))
        # one token sits a few ulps from the min-p threshold of the max (0)
        a = np.nextafter(c, F(0.0) if rng.random() < 0.5 else F(-1.0), dtype=np.float32)
        for _k in range(int(rng.integers(0, 3))):
            a = np.nextafter(a, F(-1.0), dtype=np.float32)
        x = [F(0.0), F(a), F(-6.0), F(rng.uniform(-9.0, -7.0))]
        kl, kr = _minp_keep(x, min_p, True), _minp_keep(x, min_p, False)
        if kl == kr:
            continue
        p = oracle.make_params(1, temperature=1.0, min_p=min_p, chain=1)
        assert oracle.sample_faithful(np.array(x, np.float32), p, 0.5)[1][0] == kl
        found += 1
        if found >= 5:
            break
    assert found >= 1


# --------------------------------------------------------------------------
# _verify: known answers, closed forms, the sampling identity
# --------------------------------------------------------------------------
def _rows(a):
    return np.array([[float("-inf") if v == "-inf" else float(v) for v in r] for r in a], np.float32)


def test_verify_faithful_reference_cases(oracle):
    c = CASES["greedy_verify_first_mismatch"]   # runtime/tests/test_runtime.py:1514-1532
    acc, tok = oracle.verify_faithful(_rows(c["draft_logprobs"])[None], _rows(c["target"])[None],
                                      np.array([c["draft_tokens"]]), np.zeros((1, 3), np.float32), 0.0)
    assert (acc[0], tok[0]) == (c["expected_accepted"], c["expected_token"])
    c = CASES["sampling_verify_identical"]      # runtime/tests/test_runtime.py:1534-1542
    for u in (0.0, 0.5, 0.999):
        acc, tok = oracle.verify_faithful(_rows(c["draft_logprobs"])[None], _rows(c["target"])[None],
                                          np.array([c["draft_tokens"]]), np.full((1, 2), u, np.float32), 1.0)
        assert (acc[0], tok[0]) == (c["expected_accepted"], c["expected_token"])
    c = CASES["mtp_disjoint_supports"]          # runtime/tests/test_qwen.py:420-442
    V = c["vocab"]
    tgt = np.full((1, 2, V), -np.inf, np.float32)
    tgt[..., c["target_support"]] = 0.0
    dr = np.full((1, 1, V), -np.inf, np.float32)
    dr[..., c["draft_support"]] = 0.0
    for u in (0.3, 0.99):
        acc, tok = oracle.verify_faithful(dr, tgt, np.array([c["draft_support"][:1]]), np.full((1, 2), u, np.float32), 1.0)
        assert (acc[0], tok[0]) == (c["expected_accepted"], c["expected_token"])
    c = CASES["mtp_identical_supports"]         # runtime/tests/test_qwen.py:387-418
    V = c["vocab"]
    logits = np.full((2, V), -np.inf, np.float32)
    logits[:, c["support"]] = 0.0
    p = oracle.make_params(2, temperature=c["temperature"], top_p=c["top_p"], top_k=c["top_k"], chain=1)
    _, _, rows = oracle.sample_faithful(logits, p, np.array([0.2, 0.6], np.float32), want_rows=True)
    for u in (0.1, 0.5, 0.99):
        for t in c["support"]:
            acc, _ = oracle.verify_faithful(rows[:1][None], rows[None], np.array([[t]]),
                                            np.full((1, 2), u, np.float32), c["temperature"])
            assert acc[0] == c["expected_accepted"]


def test_verify_faithful_closed_forms(oracle):
    rng = np.random.default_rng(44)
    B, n, V = 32, 4, 50
    lp = rng.normal(0, 2, (B, n + 1, V))
    lp = (lp - np.log(np.exp(lp).sum(-1, keepdims=True))).astype(np.float32)
    toks = rng.integers(0, V, (B, n)).astype(np.int32)
    # p == q: the ratio is 1 and u <= 1 never rejects; the bonus row is drawn
    u = np.full((B, n + 1), np.float32(0.99999994))
    acc, tok = oracle.verify_faithful(lp[:, :n], lp, toks, u, 1.0)
    assert (acc == n).all()
    # disjoint supports: every test rejects (u > 0 = ratio) and the residual
    # max(p - q, 0) is p itself: the draw sweeps p's support in order
    tgt = np.full((1, 2, 6), -np.inf, np.float32)
    tgt[0, :, :3] = np.log(np.array([0.5, 0.25, 0.25], np.float32))
    dr = np.full((1, 1, 6), -np.inf, np.float32)
    dr[0, 0, 3:] = np.log(np.float32(1 / 3))
    got = [oracle.verify_faithful(dr, tgt, np.array([[4]]), np.array([[0.5, uu]], np.float32), 1.0)
           for uu in (0.1, 0.49, 0.51, 0.74, 0.76, 0.99)]
    assert [int(a[0]) for a, _ in got] == [0] * 6
    assert [int(t[0]) for _, t in got] == [0, 0, 1, 1, 2, 2]
    # zero residual: the draft puts slightly more mass than the target on the
    # drafted token (3 ulps of its logprob) and no less anywhere, so
    # u = 0.99999994 rejects (ratio ~ 1 - 1.8e-7) yet every max(p - q, 0) is
    # 0; the reference draws from the target row instead (dspark.py:889-894)
    half = np.log(np.float32(0.5))
    d0 = half
    for _ in range(3):
        d0 = np.nextafter(d0, np.float32(0), dtype=np.float32)
    tgt = np.array([[[half, half], [half, half]]], np.float32)
    dr = np.array([[[d0, half]]], np.float32)
    u0 = np.float32(0.99999994)
    for u_n, want in ((0.3, 0), (0.7, 1)):
        acc, tok = oracle.verify_faithful(dr, tgt, np.array([[0]]), np.array([[u0, u_n]], np.float32), 1.0)
        assert (acc[0], tok[0]) == (0, want)
        acc_c, tok_c = oracle.verify_logprobs(dr, tgt, np.array([[0]]), np.array([[u0, u_n]], np.float32), 1.0)
        assert (acc_c[0], tok_c[0]) == (0, want)


def test_verify_faithful_output_distribution_equals_target(oracle):
    """Leviathan et al. 2023 / Chen et al. 2023: with t ~ q, accept-or-resample
    emits a token distributed as p."""
    rng = np.random.default_rng(45)
    V = 6
    p = rng.dirichlet(np.ones(V) * 0.8)
    q = rng.dirichlet(np.ones(V) * 0.8)
    lp, lq = np.log(p).astype(np.float32), np.log(q).astype(np.float32)
    N = 200000
    t = rng.choice(V, size=N, p=q).astype(np.int32)
    u = rng.random((N, 2), dtype=np.float32)
    acc, tok = oracle.verify_faithful(np.repeat(lq[None, None], N, 0), np.repeat(np.stack([lp, lp])[None], N, 0),
                                      t[:, None], u, 1.0)
    first = np.where(acc == 1, t, tok)
    freq = np.bincount(first, minlength=V) / N
    assert (((freq - p) ** 2) / p).sum() * N < 30.0  # df 5


# --------------------------------------------------------------------------
# faithful vs contract: disagreements only at boundaries
# --------------------------------------------------------------------------
@pytest.mark.parametrize("case", ["plain", "topk_topp", "mtp_ties"])
def test_faithful_and_contract_differ_only_near_boundaries(oracle, case):
    rng = np.random.default_rng({"plain": 9, "topk_topp": 10, "mtp_ties": 11}[case])
    B, V = 96, 6000
    if case == "plain":
        x = rng.normal(0, 3, (B, V))
        kw = dict(temperature=1.0, top_p=0.9, min_p=0.05, presence_penalty=0.5, frequency_penalty=0.3, chain=0)
    elif case == "topk_topp":
        x = 2.5 * rng.standard_t(3, (B, V))
        kw = dict(temperature=0.7, top_k=50, top_p=0.95, repetition_penalty=1.1, chain=0)
    else:
        x = np.round(rng.normal(0, 2, (B, V)) / 0.125) * 0.125
        kw = dict(temperature=0.6, top_k=20, top_p=0.8, min_p=0.02, repetition_penalty=1.05, presence_penalty=0.4,
                  frequency_penalty=0.2, chain=1)
    x = x.astype(np.float32)
    hist = rng.integers(0, V, (B, 256)).astype(np.int32)
    p = oracle.make_params(B, repetition_context=0, presence_context=0, frequency_context=0, **kw)
    u = rng.random(B, dtype=np.float32)
    a, ka = oracle.sample(x, p, u, hist)
    b, kb = oracle.sample_faithful(x, p, u, hist)
    marg = sample_margins(oracle.penalize(x, p, hist), p, u)
    bad = np.nonzero((a != b) & (marg >= 1e-6))[0]
    assert bad.size == 0, (bad[:5], marg[bad[:5]], a[bad[:5]], b[bad[:5]])
    assert np.mean(a == b) >= 0.9


def test_verify_faithful_and_contract_differ_only_near_boundaries(oracle):
    rng = np.random.default_rng(46)
    B, n, V, T = 48, 6, 3000, 0.8
    x = rng.normal(0, 2.5, (B, n + 1, V)).astype(np.float32)
    dl = x[:, :n].astype(np.float64) + rng.normal(0, 0.5, (B, n, V))
    q = np.exp(dl / T - (dl / T).max(-1, keepdims=True))
    q /= q.sum(-1, keepdims=True)
    toks = np.array([[rng.choice(V, p=q[b, j]) for j in range(n)] for b in range(B)], np.int32)
    q = q.astype(np.float32)
    u = rng.random((B, n + 1), dtype=np.float32)
    a, t = oracle.verify_fused(x, q, toks, u, T)
    # the reference's target rows: sampling_logprobs(logits, T, top_p=1)
    pr = oracle.make_params(B * (n + 1), temperature=T, chain=1)
    _, _, tlp = oracle.sample_faithful(x.reshape(-1, V), pr, np.zeros(B * (n + 1), np.float32), want_rows=True)
    tlp = tlp.reshape(B, n + 1, V)
    dlp = np.log(q)
    fa, ft = oracle.verify_faithful(dlp, tlp, toks, u, T)
    x64 = x.astype(np.float64) / T
    tl64 = x64 - np.log(np.exp(x64 - x64.max(-1, keepdims=True)).sum(-1, keepdims=True)) - x64.max(-1, keepdims=True)
    for bb in np.nonzero((a != fa) | (t != ft))[0]:
        assert verify_margin(tl64[bb], np.log(q[bb].astype(np.float64)), toks[bb], u[bb], T) < 1e-6, bb
    assert np.mean((a == fa) & (t == ft)) >= 0.9
