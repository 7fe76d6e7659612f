"""Pins for the CPU oracle (oracle/wh_oracle.c).

Each check is chosen so that a plausible mistake in the oracle (a dropped
term, a wrong tie direction, a transposed operand, an off-by-one in a window)
fails it: known answers transcribed from the reference's own tests
(tests/golden/reference_cases.json), hand-computed cases, exact rational
arithmetic (Python Fractions) for the integer helpers, an independent
float64 restatement for kept sets away from cumulative boundaries, and
Monte-Carlo checks of the draw and of the speculative-sampling identity.
"""
import json
import math
import os
from fractions import Fraction

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = json.load(open(os.path.join(HERE, "golden", "reference_cases.json")))
NEG_INF = float("-inf")


def _f(v):
    return NEG_INF if v == "-inf" else float(v)


# --------------------------------------------------------------------------
# contract exponential
# --------------------------------------------------------------------------
def test_exp_fix44_accuracy_against_float64(oracle):
    rng = np.random.default_rng(0)
    d = np.concatenate([
        -rng.random(1 << 20, dtype=np.float32) * 31.0,
        -np.linspace(0, 1, 1 << 18, dtype=np.float32),
        np.array([0.0, -0.0, -1e-30, -1e-7], dtype=np.float32),
    ]).astype(np.float32)
    w = oracle.exp_fix44(d).astype(np.float64) * 2.0 ** -44
    ref = np.exp(d.astype(np.float64))
    t = np.abs(d.astype(np.float64)) * 1.4426950408889634
    bound = ref * (t + 2.0) * 2.0 ** -23 + 2.0 ** -44
    assert np.all(np.abs(w - ref) <= bound)
    near = np.abs(d) <= 1.0
    rel = np.abs(w[near] - ref[near]) / ref[near]
    assert rel.max() < 3e-7
    assert oracle.exp_fix44(np.float32(0.0))[()] == 1 << 44
    assert oracle.exp_fix44(np.array([NEG_INF, -100.0], np.float32)).tolist() == [0, 0]


# --------------------------------------------------------------------------
# exact integer helpers, against Python Fractions
# --------------------------------------------------------------------------
def test_gt_theta_matches_exact_rationals(oracle):
    rng = np.random.default_rng(1)
    for _ in range(3000):
        Z = int(rng.integers(1, 1 << 62))
        theta = np.float32(rng.random() ** 3)
        A = int(rng.integers(0, Z + 1)) if rng.random() < 0.5 else int(Fraction(float(theta)) * Z) + int(rng.integers(-2, 3))
        A = max(A, 0)
        assert oracle.gt_theta(A, theta, Z) == (Fraction(A) > Fraction(float(theta)) * Z)
    # theta == 0 (top_p rounding to 1): keep iff A > 0
    assert oracle.gt_theta(1, 0.0, 10) and not oracle.gt_theta(0, 0.0, 10)


def test_floor_qz_and_reject_fused_match_exact_rationals(oracle):
    rng = np.random.default_rng(2)
    for _ in range(3000):
        Z = int(rng.integers(1, 1 << 62))
        q = np.float32(rng.random() ** 4)
        assert oracle.floor_qz(q, Z) == math.floor(Fraction(float(q)) * Z)
        u = np.float32(rng.random())
        W = int(rng.integers(0, 1 << 45))
        if rng.random() < 0.3:
            W = int(Fraction(float(u)) * Fraction(float(q)) * Z) + int(rng.integers(-1, 2))
            W = max(W, 0)
        expect = Fraction(float(u)) * Fraction(float(q)) * Z > W
        assert oracle.reject_fused(u, q, Z, W) == expect


def test_reject_lp_reference_cases(oracle):
    # ratio = min(1, exp(g - d)); reject iff u > ratio (dspark.py:880-884)
    assert not oracle.reject_lp(0.99, -1.0, -2.0)        # ratio 1
    assert not oracle.reject_lp(0.0, -10.0, -1.0)        # u = 0 never rejects
    assert oracle.reject_lp(0.5, NEG_INF, -1.0)          # target gives the token no mass
    assert not oracle.reject_lp(0.5, -1.0, NEG_INF)      # draft gave it no mass: ratio inf
    assert not oracle.reject_lp(0.5, NEG_INF, NEG_INF)   # NaN ratio: comparison false
    r = math.exp(-0.7)
    assert oracle.reject_lp(np.float32(r + 1e-4), -1.0, -0.3)
    assert not oracle.reject_lp(np.float32(r - 1e-4), -1.0, -0.3)


# --------------------------------------------------------------------------
# penalties: hand-computed known answers
# --------------------------------------------------------------------------
def _pen(oracle, l, hist, **kw):
    p = oracle.make_params(1, **kw)
    return oracle.penalize(np.array(l, np.float32), p, np.array(hist, np.int32))[0].tolist()


def test_penalties_known_answers(oracle):
    l = [2.0, -2.0, 1.0, 0.5]
    h = [0, 1, 0]
    assert _pen(oracle, l, h, repetition_penalty=2.0) == [1.0, -4.0, 1.0, 0.5]
    assert _pen(oracle, l, h, presence_penalty=0.5) == [1.5, -2.5, 1.0, 0.5]   # once per unique id
    assert _pen(oracle, l, h, frequency_penalty=0.5) == [1.0, -2.5, 1.0, 0.5]  # per occurrence
    # processor order repetition -> presence: 2/2 - 1 = 0 (presence first would give 0.5)
    assert _pen(oracle, l, h, repetition_penalty=2.0, presence_penalty=1.0)[0] == 0.0
    # windows: context 1 keeps only the last id (0); context 0 means the whole history
    assert _pen(oracle, l, h, repetition_penalty=2.0, repetition_context=1) == [1.0, -2.0, 1.0, 0.5]
    assert _pen(oracle, l, h, repetition_penalty=2.0, repetition_context=0) == [1.0, -4.0, 1.0, 0.5]
    assert _pen(oracle, l, h, frequency_penalty=0.5, frequency_context=2) == [1.5, -2.5, 1.0, 0.5]
    # ids outside [0, V) are ignored
    assert _pen(oracle, l, [7, -1, 3], presence_penalty=1.0) == [2.0, -2.0, 1.0, -0.5]
    # repetition 1.0 is a no-op
    assert _pen(oracle, l, h, repetition_penalty=1.0) == l


# --------------------------------------------------------------------------
# sampler
# --------------------------------------------------------------------------
def test_greedy_reference_case(oracle):
    c = CASES["greedy_sampler"]
    x = np.linspace(*c["linspace"][:2], c["linspace"][2], dtype=np.float32)
    for chain in (0, 1):
        p = oracle.make_params(1, temperature=0.0, chain=chain)
        assert oracle.sample(x, p, 0.5)[0][0] == c["expected_token"]


def test_noop_filters_keep_everything(oracle):
    rng = np.random.default_rng(3)
    x = rng.normal(0, 2, (4, 300)).astype(np.float32)
    for chain in (0, 1):
        p = oracle.make_params(4, temperature=0.8, top_p=1.0, top_k=0, min_p=0.0, chain=chain)
        _, kept = oracle.sample(x, p, 0.3)
        assert kept.tolist() == [300] * 4


def _sweep_tokens(oracle, x, p, n=4096):
    u = (np.arange(n, dtype=np.float64) / n).astype(np.float32)
    X = np.repeat(np.asarray(x, np.float32)[None], n, 0)
    P = np.repeat(p, n)
    return oracle.sample(X, P, u)[0]


def test_tie_rules_known_answers(oracle):
    x = np.zeros(8, np.float32)
    # top-p alone (chain B): ascending stable sort puts higher ids last, so the
    # nucleus of 0.5 over 8 equal tokens is ids 4..7
    p = oracle.make_params(1, temperature=1.0, top_p=0.5, chain=1)
    assert set(_sweep_tokens(oracle, x, p).tolist()) == {4, 5, 6, 7}
    # top-k alone: lower ids win ties
    p = oracle.make_params(1, temperature=1.0, top_k=3, chain=1)
    assert set(_sweep_tokens(oracle, x, p).tolist()) == {0, 1, 2}
    # chain A, k=3 then p=0.5: the top-3 mass 3/8 never exceeds 1-p, so every
    # token is masked and the all -inf row yields index 0 with an empty kept set
    p = oracle.make_params(1, temperature=1.0, top_k=3, top_p=0.5, chain=0)
    tok, kept = oracle.sample(x, p, 0.7)
    assert (tok[0], kept[0]) == (0, 0)
    # chain B, p=0.5 then k=3: k takes the three lowest ids of the nucleus 4..7
    p = oracle.make_params(1, temperature=1.0, top_k=3, top_p=0.5, chain=1)
    assert set(_sweep_tokens(oracle, x, p).tolist()) == {4, 5, 6}


def test_min_p_threshold_known_answer(oracle):
    # min_p keeps l >= max + ln(min_p): ln 0.5 = -0.693
    x = np.array([0.0, -0.5, -0.69, -0.7, -3.0], np.float32)
    p = oracle.make_params(1, temperature=1.0, min_p=0.5, chain=1)
    assert oracle.sample(x, p, 0.1)[1][0] == 3
    p = oracle.make_params(1, temperature=1.0, min_p=1.0, chain=1)
    assert oracle.sample(x, p, 0.9)[0][0] == 0


def _kept_float64(l, T, top_p, top_k, min_p, chain):
    """Independent float64 restatement of the filter chain on a logit row;
    returns (kept mask, boundary margin of the top-p decision)."""
    V = l.size
    lp = l.astype(np.float64) - (np.log(np.sum(np.exp(l - l.max()))) + l.max())
    alive = np.ones(V, bool)
    margin = np.inf
    order_k = np.lexsort((np.arange(V), -lp))            # value desc, id asc
    order_p = np.lexsort((-np.arange(V), -lp))           # value desc, id desc

    def do_k():
        idx = [i for i in order_k if alive[i]]
        for i in idx[top_k:]:
            alive[i] = False

    def do_p():
        nonlocal margin
        pr = np.where(alive, np.exp(lp), 0.0)
        S = pr.sum()
        head = 0.0
        for i in order_p:
            if not alive[i]:
                continue
            val = S - head
            margin = min(margin, abs(val - (1.0 - top_p)))
            head += pr[i]
            if not val > float(np.float32(1.0 - top_p)):
                alive[i] = False

    def do_m():
        mx = lp[alive].max() if alive.any() else -np.inf
        thr = np.float32(np.float32(mx) + np.float32(math.log(min_p)))
        for i in range(V):
            if alive[i] and not (np.float32(lp[i]) >= thr):
                alive[i] = False

    steps = {"k": (top_k > 0 and top_k < V, do_k), "p": (0 < top_p < 1, do_p), "m": (min_p != 0, do_m)}
    for s in ("kpm" if chain == 0 else "pmk"):
        if steps[s][0]:
            steps[s][1]()
    return alive, margin


def test_kept_sets_match_float64_restatement(oracle):
    rng = np.random.default_rng(4)
    checked = 0
    for trial in range(60):
        V = int(rng.integers(50, 3000))
        kind = trial % 3
        if kind == 0:
            x = rng.normal(0, 2.5, V)
        elif kind == 1:
            x = 3 * rng.standard_t(3, V)
        else:
            x = np.round(rng.normal(0, 2, V) / 0.125) * 0.125
        x = x.astype(np.float32)
        T = float(rng.choice([0.6, 1.0, 1.3]))
        top_p = float(rng.choice([1.0, 0.95, 0.8, 0.5]))
        top_k = int(rng.choice([0, 1, 5, 20, 200]))
        min_p = float(rng.choice([0.0, 0.02, 0.1]))
        for chain in (0, 1):
            if chain == 0 and top_k >= V:
                continue
            p = oracle.make_params(1, temperature=T, top_p=top_p, top_k=top_k, min_p=min_p, chain=chain)
            alive, margin = _kept_float64(x, T, top_p, top_k, min_p, chain)
            if margin < 1e-6:
                continue
            if chain == 1:
                _, kept, rows = oracle.sample(x, p, 0.5, want_rows=True)
                assert np.array_equal(np.isfinite(rows[0]), alive), (trial, chain)
            else:
                _, kept = oracle.sample(x, p, 0.5)
            assert kept[0] == alive.sum(), (trial, chain)
            checked += 1
    assert checked > 80


def test_draw_matches_tempered_probabilities(oracle):
    """Inverse-CDF over a uniform sweep reproduces exp(s*(l-m)) over the kept
    set in vocab order; both temperature forms (x * (1/T) and x / T)."""
    rng = np.random.default_rng(5)
    for chain in (0, 1):
        x = rng.normal(0, 1.5, 40).astype(np.float32)
        T = 0.7
        p = oracle.make_params(1, temperature=T, top_k=12, chain=chain)
        n = 1 << 16
        toks = _sweep_tokens(oracle, x, p, n)
        assert np.all(np.diff(toks) >= 0)  # vocab order CDF: monotone in u
        keep = np.argsort(-x, kind="stable")[:12]
        w = np.zeros(40)
        w[keep] = np.exp((x[keep].astype(np.float64) - x.max()) / T)
        w /= w.sum()
        freq = np.bincount(toks, minlength=40) / n
        assert np.abs(freq - w).max() < 2.0 / n + 1e-6


def test_chi_square_of_random_uniforms(oracle):
    rng = np.random.default_rng(6)
    x = rng.normal(0, 1, 16).astype(np.float32)
    p = oracle.make_params(1, temperature=1.0, top_p=0.9, chain=1)
    n = 200000
    u = rng.random(n, dtype=np.float32)
    toks = oracle.sample(np.repeat(x[None], n, 0), np.repeat(p, n), u)[0]
    _, _, rows = oracle.sample(x, p, 0.5, want_rows=True)
    prob = np.exp(rows[0].astype(np.float64))
    cnt = np.bincount(toks, minlength=16)
    m = prob > 0
    assert cnt[~m].sum() == 0
    chi2 = (((cnt[m] - n * prob[m]) ** 2) / (n * prob[m])).sum()
    assert chi2 < 45.0  # df <= 15; p ~ 1e-4 tail


def test_reproducible_and_non_constant_draws(oracle):
    """Build analogue of runtime/tests/test_sampling.py:22-38: fixed uniform
    streams reproduce, differ across streams and are not constant."""
    logits = np.linspace(-1, 1, 128, dtype=np.float32)
    lp = (logits - (np.log(np.exp(logits - 1).sum()) + 1)).astype(np.float32)
    for prof in CASES["sampler_profiles"]["profiles"]:
        p = oracle.make_params(64, temperature=prof["temp"], top_p=prof.get("top_p", 1.0),
                               top_k=prof.get("top_k", 0), min_p=prof.get("min_p", 0.0), chain=0)
        X = np.repeat(lp[None], 64, 0)
        a = oracle.sample(X, p, np.random.default_rng(20260906).random(64, dtype=np.float32))[0]
        b = oracle.sample(X, p, np.random.default_rng(20260906).random(64, dtype=np.float32))[0]
        c = oracle.sample(X, p, np.random.default_rng(20260907).random(64, dtype=np.float32))[0]
        assert len(set(a.tolist())) > 1
        assert a.tolist() == b.tolist()
        assert a.tolist() != c.tolist()


def test_chain_orders_differ_on_mtp_shape(oracle):
    """k=20, p=0.8 on a wide row: chain A (k first) leaves a top-20 mass far
    below 1-p and masks everything; chain B keeps 20."""
    rng = np.random.default_rng(7)
    x = (np.round(rng.normal(0, 2, 20000) / 0.125) * 0.125).astype(np.float32)
    pa = oracle.make_params(1, temperature=0.6, top_k=20, top_p=0.8, min_p=0.02, chain=0)
    pb = oracle.make_params(1, temperature=0.6, top_k=20, top_p=0.8, min_p=0.02, chain=1)
    assert oracle.sample(x, pa, 0.4)[1][0] == 0
    assert oracle.sample(x, pb, 0.4)[1][0] == 20


def test_parameter_validation(oracle):
    x = np.zeros((1, 10), np.float32)
    with pytest.raises(ValueError):
        oracle.sample(x, oracle.make_params(1, temperature=1.0, top_k=10, chain=0), 0.5)
    # chain B guards 0 < k < V instead of raising (dspark.py:372)
    assert oracle.sample(x, oracle.make_params(1, temperature=1.0, top_k=10, chain=1), 0.5)[1][0] == 10
    with pytest.raises(ValueError):
        oracle.sample(x, oracle.make_params(1, temperature=1.0, min_p=1.5), 0.5)
    with pytest.raises(ValueError):
        oracle.sample(x, oracle.make_params(1, temperature=-1.0), 0.5)


# --------------------------------------------------------------------------
# verifier
# --------------------------------------------------------------------------
def _rows(a):
    return np.array([[_f(v) for v in r] for r in a], np.float32)


def test_verify_reference_cases(oracle):
    c = CASES["greedy_verify_first_mismatch"]
    acc, tok = oracle.verify_logprobs(_rows(c["draft_logprobs"])[None], _rows(c["target"])[None],
                                      np.array([c["draft_tokens"]]), np.zeros((1, 3), np.float32), 0.0)
    assert (acc[0], tok[0]) == (c["expected_accepted"], c["expected_token"])
    c = CASES["sampling_verify_identical"]
    for u in (0.0, 0.5, 0.999):
        acc, tok = oracle.verify_logprobs(_rows(c["draft_logprobs"])[None], _rows(c["target"])[None],
                                          np.array([c["draft_tokens"]]), np.full((1, 2), u, np.float32), 1.0)
        assert (acc[0], tok[0]) == (c["expected_accepted"], c["expected_token"])


def test_verify_disjoint_and_identical_supports(oracle):
    c = CASES["mtp_disjoint_supports"]
    V = c["vocab"]
    tgt = np.full((1, 2, V), NEG_INF, np.float32)
    tgt[..., c["target_support"]] = 0.0
    dr = np.full((1, 1, V), NEG_INF, np.float32)
    dr[..., c["draft_support"]] = 0.0
    for u in (0.0, 0.3, 0.99):
        acc, tok, row = oracle.verify_logprobs(dr, tgt, np.array([c["draft_support"][:1]]),
                                               np.full((1, 2), u, np.float32), 1.0, want_rows=True)
        # u = 0 accepts (u > ratio is false); otherwise the residual max(p - q, 0) = p
        exp_acc = 1 if u == 0.0 else c["expected_accepted"]
        assert acc[0] == exp_acc
        if exp_acc == 0:
            assert tok[0] == c["expected_token"]
            assert row[0][0] == 0.0 and np.isneginf(row[0][1:]).all()
    c = CASES["mtp_identical_supports"]
    V = c["vocab"]
    logits = np.full((2, V), NEG_INF, np.float32)
    logits[:, c["support"]] = 0.0
    p = oracle.make_params(2, temperature=c["temperature"], top_p=c["top_p"], top_k=c["top_k"], chain=1)
    _, _, rows = oracle.sample(logits, p, np.array([0.2, 0.6], np.float32), want_rows=True)
    for u in (0.1, 0.5, 0.99):
        for t in c["support"]:
            acc, _ = oracle.verify_logprobs(rows[:1][None], rows[None], np.array([[t]]),
                                            np.full((1, 2), u, np.float32), c["temperature"])
            assert acc[0] == c["expected_accepted"]


def test_verify_output_distribution_equals_target(oracle):
    """Speculative sampling identity (Leviathan et al. 2023, Chen et al. 2023):
    with t ~ q, accept-or-resample emits a token distributed as p."""
    rng = np.random.default_rng(8)
    V = 6
    p = rng.dirichlet(np.ones(V) * 0.8)
    q = rng.dirichlet(np.ones(V) * 0.8)
    lp = np.log(p).astype(np.float32)
    lq = np.log(q).astype(np.float32)
    n = 200000
    t = rng.choice(V, size=n, p=q).astype(np.int32)
    u = rng.random((n, 2), dtype=np.float32)
    tgt = np.repeat(np.stack([lp, lp])[None], n, 0)
    dr = np.repeat(lq[None, None], n, 0)
    acc, tok = oracle.verify_logprobs(dr, tgt, t[:, None], u, 1.0)
    first = np.where(acc == 1, t, tok)
    freq = np.bincount(first, minlength=V) / n
    chi2 = (((freq - p) ** 2) / p).sum() * n
    assert chi2 < 30.0  # df 5
    # fused form on the same distributions
    X = np.repeat(np.stack([lp, lp])[None], n, 0)  # logits = log p, T = 1
    Q = np.repeat(q.astype(np.float32)[None, None], n, 0)
    acc2, tok2 = oracle.verify_fused(X, Q, t[:, None], u, 1.0)
    first2 = np.where(acc2 == 1, t, tok2)
    freq2 = np.bincount(first2, minlength=V) / n
    assert (((freq2 - p) ** 2) / p).sum() * n < 30.0
    assert np.mean(acc == acc2) > 0.999


def test_verify_zero_residual_falls_back_to_target(oracle):
    V = 5
    lp = np.log(np.array([0.1, 0.2, 0.3, 0.2, 0.2])).astype(np.float32)
    # draft dominates target everywhere it matters -> residual sum 0 only if p == q;
    # force a rejection with p == q by making u exceed the ratio 1: impossible, so
    # use a draft with more mass on every token's support ordering: q = p exactly
    tgt = np.stack([lp, lp])[None]
    acc, _ = oracle.verify_logprobs(lp[None, None], tgt, np.array([[2]]), np.array([[0.99, 0.5]], np.float32), 1.0)
    assert acc[0] == 1
    # all draft mass on a token the target does not support, with the target's
    # support a subset of the draft's: residual is p itself
    q = np.log(np.array([0.05, 0.05, 0.05, 0.05, 0.8])).astype(np.float32)
    p = np.log(np.array([0.0, 0.0, 0.5, 0.5, 0.0]) + 1e-30).astype(np.float32)
    acc, tok = oracle.verify_logprobs(q[None, None], np.stack([p, p])[None], np.array([[4]]),
                                      np.array([[0.5, 0.75]], np.float32), 1.0)
    assert acc[0] == 0 and tok[0] in (2, 3)
