"""The drop-in mirrors and the less common kernel branches on the GPU, each
against the CPU oracle.

  * mlx_lm names (whallm_amd/sample_utils.py): the Sampler returned by
    make_sampler, categorical_sampling, make_logits_processors with the
    reference's default profiles (runtime/tests/test_sampling.py:23-24,
    runtime/tests/test_advanced_defaults.py:18-24);
  * Whallm's dspark helpers (whallm_amd/dspark.py): _sample, _verify with
    DraftResult, on the reference's verify cases and on random rows;
  * a token and its sampling_logprobs row from one call (the draft step of
    runtime/deepseek_v4_ssd/dspark.py:319-330 needs both);
  * penalty windows over histories longer than the slice kernel's prefetch
    (4,096 ids), float32 and bfloat16;
  * bfloat16 rows with ties, -inf entries, top-k and vocabularies that are
    not a multiple of 8; vocabularies of a few dozen ids on the fast engine;
  * the greedy MTP rounds of runtime/tests/test_qwen.py:360-385 and 468-490
    driven through the verifier;
  * pre-bound calls reading buffers the caller refills between steps.
"""
import json
import os
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
CASES = json.load(open(os.path.join(HERE, "golden", "reference_cases.json")))


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


def _lp(x):
    x = x.astype(np.float64)
    m = x.max(-1, keepdims=True)
    return (x - m - np.log(np.exp(x - m).sum(-1, keepdims=True))).astype(np.float32)


def _bf16(x):
    from whallm_amd.synth import bf16_bits_to_f32, f32_to_bf16_bits

    bits = f32_to_bf16_bits(x)
    return bits, bf16_bits_to_f32(bits)


def _tbf16(bits, dev):
    return torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)


# --------------------------------------------------------------------------
# mlx_lm mirrors
# --------------------------------------------------------------------------
@pytest.mark.parametrize("prof", range(3))
def test_make_sampler_profiles(dev, oracle, prof):
    from whallm_amd import sample_utils as su

    c = CASES["sampler_profiles"]["profiles"][prof]
    rng = np.random.default_rng(1000 + prof)
    B, V = 32, 151936
    x = _lp(rng.normal(0, 2.5, (B, V)).astype(np.float32))
    u = rng.random(B, dtype=np.float32)
    sampler = su.make_sampler(temp=c["temp"], top_p=c.get("top_p", 0.0), min_p=c.get("min_p", 0.0),
                              top_k=c.get("top_k", 0))
    announce(f"make_sampler profile {c}")
    got = sampler(torch.from_numpy(x).to(dev), uniforms=torch.from_numpy(u).to(dev)).cpu().numpy()
    p = oracle.make_params(B, temperature=c["temp"], top_p=c.get("top_p", 1.0) or 1.0, min_p=c.get("min_p", 0.0),
                           top_k=c.get("top_k", 0), chain=0)
    want, _ = oracle.sample(x, p, u)
    assert np.array_equal(got, want)
    # a 1-D row returns a 0-d token, as mlx_lm's sampler does for [V]
    one = sampler(torch.from_numpy(x[0]).to(dev), uniforms=torch.from_numpy(u[:1]).to(dev))
    assert one.dim() == 0 and int(one) == want[0]


@pytest.mark.parametrize("mode", ["chat", "thinking"])
def test_qwen_chat_defaults_through_processors(dev, oracle, mode):
    """Whallm's Qwen defaults (runtime/tests/test_advanced_defaults.py:18-24)
    through make_logits_processors then make_sampler, as generation.py:1280-1293
    wires them: presence over the last 20 ids (mlx_lm's default window)."""
    from whallm_amd import sample_utils as su

    c = CASES["qwen_chat_defaults"][mode]
    rng = np.random.default_rng(1100 + (mode == "chat"))
    B, V, H = 16, 151936, 300
    x = rng.normal(0, 2.5, (B, V)).astype(np.float32)
    hist = rng.integers(0, V, (B, H)).astype(np.int32)
    hist[:, -5:] = np.argsort(-x, axis=1)[:, :5]  # the current leaders are in the window
    u = rng.random(B, dtype=np.float32)
    procs = su.make_logits_processors(presence_penalty=c["presence_penalty"] or None)
    sampler = su.make_sampler(temp=c["temperature"], top_p=c["top_p"], top_k=c["top_k"])
    announce(f"qwen {mode} defaults {c}")
    t = torch.from_numpy(x.copy()).to(dev)
    ht = torch.from_numpy(hist).to(dev)
    for pr in procs:
        t = pr(ht, t)
    lp = t - torch.logsumexp(t, dim=-1, keepdim=True)
    got = sampler(lp, uniforms=torch.from_numpy(u).to(dev)).cpu().numpy()
    p_pen = oracle.make_params(B, presence_penalty=c["presence_penalty"], presence_context=20)
    xp = oracle.penalize(x, p_pen, hist)
    lpo = lp.cpu().numpy()
    # the sampler's input is the device's float32 logprob row; the oracle
    # samples that same row
    assert np.array_equal(np.isfinite(lpo), np.isfinite(xp))
    p = oracle.make_params(B, temperature=c["temperature"], top_p=c["top_p"], top_k=c["top_k"], chain=0)
    want, _ = oracle.sample(lpo, p, u)
    assert np.array_equal(got, want)


def test_categorical_sampling(dev, oracle):
    from whallm_amd import sample_utils as su

    rng = np.random.default_rng(1200)
    B, V = 40, 20000
    x = rng.normal(0, 3, (B, V)).astype(np.float32)
    u = rng.random(B, dtype=np.float32)
    announce("categorical_sampling")
    for temp in (0.5, 1.0, 1.7):
        got = su.categorical_sampling(torch.from_numpy(x).to(dev), temp, uniforms=torch.from_numpy(u).to(dev))
        want, _ = oracle.sample(x, oracle.make_params(B, temperature=temp, chain=0), u)
        assert np.array_equal(got.cpu().numpy(), want), temp


# --------------------------------------------------------------------------
# dspark mirrors
# --------------------------------------------------------------------------
def test_dspark_sample(dev, oracle):
    from whallm_amd import dspark

    rng = np.random.default_rng(1300)
    V = 129280
    announce("dspark._sample")
    for i in range(6):
        row = _lp(rng.normal(0, 2, V).astype(np.float32))
        u = float(rng.random())
        t = torch.from_numpy(row).to(dev)
        assert dspark._sample(t, 0.0) == int(np.argmax(row))
        got = dspark._sample(t, 0.8, uniform=u)
        # the row is already tempered: a categorical draw from it (T = 1)
        want, _ = oracle.sample(row, oracle.make_params(1, temperature=1.0, chain=1), np.float32(u))
        assert got == want[0]


def _rows(a):
    return np.array([[float("-inf") if v == "-inf" else float(v) for v in r] for r in a], np.float32)


def test_dspark_verify_reference_cases(dev):
    from whallm_amd import dspark

    announce("dspark._verify reference cases")
    c = CASES["greedy_verify_first_mismatch"]
    d = dspark.DraftResult(tokens=c["draft_tokens"], logprobs=[torch.from_numpy(r).to(dev) for r in _rows(c["draft_logprobs"])],
                           confidence=[1.0] * 2, seconds=0.0)
    acc, tok, row = dspark._verify(d, torch.from_numpy(_rows(c["target"])).to(dev), 0.0)
    assert (acc, tok) == (c["expected_accepted"], c["expected_token"])
    c = CASES["sampling_verify_identical"]
    d = dspark.DraftResult(tokens=c["draft_tokens"], logprobs=[torch.from_numpy(r).to(dev) for r in _rows(c["draft_logprobs"])],
                           confidence=[1.0], seconds=0.0)
    for u in (0.0, 0.5, 0.999):
        acc, tok, _ = dspark._verify(d, torch.from_numpy(_rows(c["target"])).to(dev), 1.0,
                                     uniforms=torch.tensor([u, u], dtype=torch.float32))
        assert (acc, tok) == (c["expected_accepted"], c["expected_token"])
    c = CASES["mtp_disjoint_supports"]
    V = c["vocab"]
    tgt = np.full((2, V), -np.inf, np.float32)
    tgt[:, c["target_support"]] = 0.0
    dr = np.full((V,), -np.inf, np.float32)
    dr[c["draft_support"]] = 0.0
    d = dspark.DraftResult(tokens=c["draft_support"][:1], logprobs=[torch.from_numpy(dr).to(dev)], confidence=[1.0],
                           seconds=0.0)
    for u in (0.3, 0.99):
        acc, tok, row = dspark._verify(d, torch.from_numpy(tgt).to(dev), 1.0, uniforms=torch.tensor([u, u]))
        assert (acc, tok) == (c["expected_accepted"], c["expected_token"])
        r = row.cpu().numpy()
        assert r[0] == 0.0 and np.isneginf(r[1:]).all()  # the residual row is p itself


@pytest.mark.parametrize("seed", range(4))
def test_dspark_verify_random(dev, oracle, seed):
    from whallm_amd import dspark

    rng = np.random.default_rng(1400 + seed)
    n, V = int(rng.integers(1, 6)), int(rng.choice([300, 129280]))
    T = float(rng.choice([0.0, 0.7, 1.0]))
    tl = _lp(rng.normal(0, 2, (n + 1, V)).astype(np.float32))
    dl = _lp(tl[:n] + rng.normal(0, 0.6, (n, V)).astype(np.float32))
    toks = [int(rng.choice(V, p=np.exp(dl[j].astype(np.float64)) / np.exp(dl[j].astype(np.float64)).sum()))
            for j in range(n)]
    u = rng.random(n + 1, dtype=np.float32)
    d = dspark.DraftResult(tokens=toks, logprobs=[torch.from_numpy(r).to(dev) for r in dl], confidence=[1.0] * n,
                           seconds=0.0)
    announce(f"dspark._verify random seed={seed} n={n} V={V} T={T}")
    acc, tok, row = dspark._verify(d, torch.from_numpy(tl).to(dev), T, uniforms=torch.from_numpy(u))
    oa, ot, orow = oracle.verify_logprobs(dl[None], tl[None], np.array([toks], np.int32), u[None], T, want_rows=True)
    assert (acc, tok) == (int(oa[0]), int(ot[0]))
    if T > 0:
        r = row.cpu().numpy()
        m = np.isfinite(orow[0])
        assert np.array_equal(np.isfinite(r), m)
        assert np.allclose(np.exp(r[m].astype(np.float64)), np.exp(orow[0][m].astype(np.float64)), rtol=1e-5, atol=1e-12)


def test_token_and_row_from_one_call(dev, oracle):
    """A draft step keeps the drawn token and its sampling_logprobs row
    (dspark.py:319-330): both from one wh_sample call."""
    from whallm_amd import sampling

    rng = np.random.default_rng(1500)
    B, V = 5, 129280
    x = rng.normal(0, 2.5, (B, V)).astype(np.float32)
    u = rng.random(B, dtype=np.float32)
    announce("sample(return_logprobs=True), chain whallm")
    for engine in ("auto", "exact"):
        tok, rows = sampling.sample(torch.from_numpy(x).to(dev), temperature=0.8, top_p=0.95, chain="whallm",
                                    uniforms=torch.from_numpy(u).to(dev), return_logprobs=True, engine=engine)
        p = oracle.make_params(B, temperature=0.8, top_p=0.95, chain=1)
        ot, _, orow = oracle.sample(x, p, u, want_rows=True)
        assert np.array_equal(tok.cpu().numpy(), ot), engine
        r = rows.cpu().numpy()
        m = np.isfinite(orow)
        assert np.array_equal(np.isfinite(r), m)
        assert np.allclose(np.exp(r[m].astype(np.float64)), np.exp(orow[m].astype(np.float64)), rtol=1e-5, atol=1e-12)


# --------------------------------------------------------------------------
# unreached branches
# --------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("H", [5000, 12000, 20000])
def test_long_history_windows(dev, oracle, dtype, H):
    """Histories longer than the slice kernel's 4,096-id prefetch: the
    windows are suffixes of at most 4,096 ids (default context 20, and
    4,096), per-row lengths below and above the prefetch."""
    from whallm_amd import sampling

    rng = np.random.default_rng(1600 + H + (dtype == "bf16"))
    B, V = 6, 151936
    x = rng.normal(0, 2.5, (B, V)).astype(np.float32)
    bits = None
    if dtype == "bf16":
        bits, x = _bf16(x)
    hist = rng.integers(0, V, (B, H)).astype(np.int32)
    hist[:, -300:] = np.argsort(-x, axis=1)[:, :300]  # penalise the leaders too
    hlen = np.array([H, H - 1, H - 4097, 4097, 4096, min(H, 4200)], np.int32)
    u = rng.random(B, dtype=np.float32)
    xt = _tbf16(bits, dev) if bits is not None else torch.from_numpy(x).to(dev)
    for ctx in ((20, 20, 20), (4096, 4096, 4096), (4096, 20, 1000)):
        pen = dict(repetition_penalty=1.3, presence_penalty=0.5, frequency_penalty=0.25, repetition_context=ctx[0],
                   presence_context=ctx[1], frequency_context=ctx[2])
        p = oracle.make_params(B, temperature=0.9, top_p=0.95, min_p=0.02, chain=0, **pen)
        ot, ok = oracle.sample(x, p, u, hist, hlen)
        for engine in ("auto", "exact"):
            announce(f"long history {dtype} H={H} ctx={ctx} engine={engine}")
            tok, kept = sampling.sample(xt, temperature=0.9, top_p=0.95, min_p=0.02, chain="mlx",
                                        history=torch.from_numpy(hist).to(dev),
                                        history_len=torch.from_numpy(hlen).to(dev),
                                        uniforms=torch.from_numpy(u).to(dev), return_kept=True, engine=engine, **pen)
            assert np.array_equal(kept.cpu().numpy(), ok), (ctx, engine)
            assert np.array_equal(tok.cpu().numpy(), ot), (ctx, engine)


def _bf16_case(rng, B, V):
    kind = rng.integers(0, 4)
    if kind == 0:
        x = rng.normal(0, rng.uniform(0.5, 4.0), (B, V))
    elif kind == 1:
        x = 3 * rng.standard_t(3, (B, V))
    elif kind == 2:
        x = np.round(rng.normal(0, 2, (B, V)) / 0.25) * 0.25   # dense ties
    else:
        x = rng.normal(0, 2, (B, V))
        x[rng.random((B, V)) < 0.3] = -np.inf                  # masked entries
    return _bf16(x.astype(np.float32))


@pytest.mark.parametrize("seed", range(16))
def test_bf16_random_parity(dev, oracle, seed):
    from whallm_amd import sampling

    rng = np.random.default_rng(1700 + seed)
    B = int(rng.integers(1, 40))
    V = int(rng.choice([40, 72, 1000, 4099, 20000, 151936]))  # 4099: not a multiple of 8 (exact engine)
    bits, x = _bf16_case(rng, B, V)
    chain = int(rng.integers(0, 2))
    T = float(rng.choice([0.0, 0.3, 0.7, 1.0, 1.5]))
    top_p = float(rng.choice([1.0, 0.99, 0.9, 0.5, 0.1]))
    top_k = int(rng.choice([0, 1, 3, 20, 200, min(1024, V - 1)]))
    if chain == 0 and top_k >= V:
        top_k = V - 1
    min_p = float(rng.choice([0.0, 0.01, 0.1, 0.5]))
    H = int(rng.integers(1, 300))
    hist = rng.integers(-2, V + 2, (B, H)).astype(np.int32)
    hlen = rng.integers(0, H + 1, B).astype(np.int32)
    pen = dict(repetition_penalty=float(rng.choice([0.0, 1.3, 0.8])), presence_penalty=float(rng.choice([0.0, 0.5])),
               frequency_penalty=float(rng.choice([0.0, 0.25])), repetition_context=int(rng.integers(0, 50)),
               presence_context=int(rng.integers(0, 50)), frequency_context=int(rng.integers(0, 50)))
    u = rng.random(B, dtype=np.float32)
    u[: max(1, B // 8)] = np.float32(0.0)
    p = oracle.make_params(B, temperature=T, top_p=top_p, top_k=top_k, min_p=min_p, chain=chain, **pen)
    ot, ok = oracle.sample(x, p, u, hist, hlen)
    for engine in ("auto", "exact"):
        announce(f"bf16 random seed={seed} engine={engine} B={B} V={V} chain={chain} T={T} p={top_p} k={top_k} "
                 f"minp={min_p} {pen}")
        tok, kept = sampling.sample(_tbf16(bits, dev), temperature=T, top_p=top_p, top_k=top_k, min_p=min_p,
                                    chain=chain, history=torch.from_numpy(hist).to(dev),
                                    history_len=torch.from_numpy(hlen).to(dev), uniforms=torch.from_numpy(u).to(dev),
                                    return_kept=True, engine=engine, **pen)
        if T > 0:
            assert np.array_equal(kept.cpu().numpy(), ok), engine
        assert np.array_equal(tok.cpu().numpy(), ot), engine


@pytest.mark.parametrize("dtype,V", [("bf16", 8), ("bf16", 40), ("bf16", 72), ("f32", 4), ("f32", 12), ("f32", 36)])
def test_tiny_vocab_fast_engine(dev, oracle, dtype, V):
    """A few dozen ids on the sliced engine: the plan must not cut slices
    that start past the row (bf16 V = 40 rounds to slices of 16)."""
    from whallm_amd import sampling

    rng = np.random.default_rng(1800 + V)
    B = 3
    x = rng.normal(0, 1.5, (B, V)).astype(np.float32)
    bits = None
    if dtype == "bf16":
        bits, x = _bf16(x)
    hist = rng.integers(0, V, (B, 10)).astype(np.int32)
    u = rng.random(B, dtype=np.float32)
    xt = _tbf16(bits, dev) if bits is not None else torch.from_numpy(x).to(dev)
    for kw in (dict(temperature=1.0, top_p=0.9, min_p=0.05, chain=0), dict(temperature=0.7, top_k=2, chain=1),
               dict(temperature=0.0, chain=0)):
        announce(f"tiny vocab {dtype} V={V} {kw}")
        tok, kept = sampling.sample(xt, uniforms=torch.from_numpy(u).to(dev), history=torch.from_numpy(hist).to(dev),
                                    presence_penalty=0.5, return_kept=True, **kw)
        p = oracle.make_params(B, presence_penalty=0.5, **kw)
        ot, ok = oracle.sample(x, p, u, hist)
        assert np.array_equal(tok.cpu().numpy(), ot), kw
        if kw["temperature"] > 0:
            assert np.array_equal(kept.cpu().numpy(), ok), kw


# --------------------------------------------------------------------------
# greedy MTP rounds through the verifier
# --------------------------------------------------------------------------
def _greedy_mtp(dev, prompt, max_tokens, reject_input=None, block=5, V=32):
    """runtime/tests/test_qwen.py's fakes, on the device: the target maps
    input t to +1000 at (t + 1) mod V and -1000 elsewhere; the drafter does
    the same except after `reject_input`.  Each round drafts
    min(block, remaining - 1) tokens and verifies them greedily
    (dspark.py:864-876), committing the accepted prefix and the target's
    token.  Returns the tokens and the (drafted, accepted) of each round."""
    from whallm_amd import sampling

    def target_rows(inputs):
        t = torch.as_tensor(inputs, device=dev)
        rows = torch.full((len(inputs), V), -1000.0, device=dev)
        rows[torch.arange(len(inputs), device=dev), (t + 1) % V] = 1000.0
        return rows - torch.logsumexp(rows, -1, keepdim=True)

    def draft(t):
        return (t + 2) % V if t == reject_input else (t + 1) % V

    out = [int(torch.argmax(target_rows([prompt[-1]])[0]))]
    rounds = []
    while len(out) < max_tokens:
        n = min(block, max_tokens - len(out) - 1)
        if n == 0:
            out.append(int(torch.argmax(target_rows([out[-1]])[0])))
            continue
        drafts = []
        for _ in range(n):
            drafts.append(draft(drafts[-1] if drafts else out[-1]))
        tgt = target_rows([out[-1], *drafts]).reshape(1, n + 1, V)
        acc, tok = sampling.verify_logprobs(tgt, None, torch.tensor([drafts], dtype=torch.int32, device=dev), 0.0)
        a, t = int(acc[0]), int(tok[0])
        out += drafts[:a] + [t]
        rounds.append((n, a))
    return out[:max_tokens], rounds


def test_greedy_mtp_rounds(dev):
    announce("greedy MTP rounds (test_qwen.py:360-385, 468-490)")
    c = CASES["greedy_mtp_chain"]
    toks, rounds = _greedy_mtp(dev, [1, 2], len(c["expected_tokens"]))
    assert toks == c["expected_tokens"] and list(rounds[0]) == c["expected_round"]
    c = CASES["greedy_mtp_partial"]
    toks, rounds = _greedy_mtp(dev, [1, 2], len(c["expected_tokens"]), reject_input=5)
    assert toks == c["expected_tokens"] and list(rounds[0]) == c["expected_round"]


# --------------------------------------------------------------------------
# pre-bound calls
# --------------------------------------------------------------------------
def test_prebound_calls_read_refilled_buffers(dev, oracle):
    from whallm_amd import sampling

    rng = np.random.default_rng(1900)
    B, V, H = 8, 151936, 512
    bits, x = _bf16(rng.normal(0, 3, (B, V)).astype(np.float32))
    xt = _tbf16(bits, dev)
    hist = torch.from_numpy(rng.integers(0, V, (B, H)).astype(np.int32)).to(dev)
    hlen = torch.full((B,), H, dtype=torch.int32, device=dev)
    u = torch.from_numpy(rng.random(B, dtype=np.float32)).to(dev)
    kw = dict(temperature=1.0, top_p=0.9, min_p=0.05, presence_penalty=0.5, frequency_penalty=0.3,
              presence_context=0, frequency_context=0)
    call = sampling.SampleCall(xt, history=hist, history_len=hlen, uniforms=u, **kw)
    p = oracle.make_params(B, chain=0, **kw)
    announce("SampleCall refills")
    for step in range(3):
        bits2, x2 = _bf16(rng.normal(0, 3, (B, V)).astype(np.float32))
        h2 = rng.integers(0, V, (B, H)).astype(np.int32)
        l2 = rng.integers(1, H + 1, B).astype(np.int32)
        u2 = rng.random(B, dtype=np.float32)
        xt.copy_(_tbf16(bits2, dev))
        hist.copy_(torch.from_numpy(h2))
        hlen.copy_(torch.from_numpy(l2))
        u.copy_(torch.from_numpy(u2))
        got = call().cpu().numpy()
        want, _ = oracle.sample(x2, p, u2, h2, l2)
        assert np.array_equal(got, want), step
    # buffers a pre-bound call would have to copy are refused
    with pytest.raises(ValueError):
        sampling.SampleCall(xt, history=hist.long(), history_len=hlen, uniforms=u, **kw)
    with pytest.raises(ValueError):
        sampling.SampleCall(xt, history=hist, history_len=hlen, uniforms=u.double(), **kw)
    with pytest.raises(ValueError):
        sampling.SampleCall(xt, history=hist[0], history_len=hlen, uniforms=u, **kw)
    with pytest.raises(ValueError):
        sampling.SampleCall(xt.half(), uniforms=u, temperature=1.0)
    # VerifyCall
    Bv, n, Vv, T = 4, 3, 4096, 0.8
    tgt = torch.zeros(Bv, n + 1, Vv, device=dev)
    q = torch.zeros(Bv, n, Vv, device=dev)
    dt = torch.zeros(Bv, n, dtype=torch.int32, device=dev)
    uv = torch.zeros(Bv, n + 1, device=dev)
    vc = sampling.VerifyCall(tgt, q, dt, T, uv)
    announce("VerifyCall refills")
    for step in range(2):
        x3 = rng.normal(0, 2.5, (Bv, n + 1, Vv)).astype(np.float32)
        q3 = rng.dirichlet(np.ones(Vv), (Bv, n)).astype(np.float32)
        t3 = rng.integers(0, Vv, (Bv, n)).astype(np.int32)
        u3 = rng.random((Bv, n + 1), dtype=np.float32)
        tgt.copy_(torch.from_numpy(x3))
        q.copy_(torch.from_numpy(q3))
        dt.copy_(torch.from_numpy(t3))
        uv.copy_(torch.from_numpy(u3))
        a, t = vc()
        oa, ot = oracle.verify_fused(x3, q3, t3, u3, T)
        assert np.array_equal(a.cpu().numpy(), oa) and np.array_equal(t.cpu().numpy(), ot), step
    with pytest.raises(ValueError):
        sampling.VerifyCall(tgt, q, dt.long(), T, uv)
