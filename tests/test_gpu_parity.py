"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle.

Token ids, accept counts and kept-set sizes must be bit-identical to the
contract oracle; float rows (sampling_logprobs, residual rows) agree within
1e-5 relative in probability.  The float32 "faithful" replay of the
reference's op order is compared separately and its agreement rate printed.
Every GPU step first prints the case it is about to run.
"""
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


@pytest.fixture(scope="module")
def S(dev):
    from whallm_amd import sampling

    return sampling


def logits_tensor(w, dev):
    if w.dtype == "bf16":
        return torch.from_numpy(w.logits_bits.view(np.int16)).to(dev).view(torch.bfloat16)
    return torch.from_numpy(w.logits_f32).to(dev)


def run_gpu_sample(S, w, dev, **extra):
    p = dict(w.params)
    kw = dict(temperature=p.get("temperature", 0.0), top_p=p.get("top_p", 1.0), top_k=p.get("top_k", 0),
              min_p=p.get("min_p", 0.0), chain=p.get("chain", "mlx"),
              repetition_penalty=p.get("repetition_penalty", 0.0), presence_penalty=p.get("presence_penalty", 0.0),
              frequency_penalty=p.get("frequency_penalty", 0.0), repetition_context=p.get("repetition_context", 20),
              presence_context=p.get("presence_context", 20), frequency_context=p.get("frequency_context", 20))
    kw.update(extra)
    hist = None if w.history is None else torch.from_numpy(w.history).to(dev)
    hl = None if w.history_len is None else torch.from_numpy(w.history_len).to(dev)
    kr = None if w.top_k_rows is None else torch.from_numpy(w.top_k_rows).to(dev)
    u = torch.from_numpy(w.uniforms).to(dev)
    tok, kept = S.sample(logits_tensor(w, dev), history=hist, history_len=hl, uniforms=u, top_k_rows=kr,
                         return_kept=True, **kw)
    torch.cuda.synchronize()
    return tok.cpu().numpy(), kept.cpu().numpy()


def test_exp_fix44_bit_exact(S, dev, oracle):
    rng = np.random.default_rng(11)
    d = np.concatenate([-rng.random(1 << 20, dtype=np.float32) * 40.0,
                        -rng.random(1 << 16, dtype=np.float32) * 1e-3,
                        np.array([0.0, -0.0, -np.inf, -31.19, -31.2, -100.0, 1e-8], np.float32)]).astype(np.float32)
    announce(f"wh_exp_fix44 n={d.size}")
    got = S.exp_fix44(torch.from_numpy(d).to(dev)).cpu().numpy().astype(np.uint64)
    assert np.array_equal(got, oracle.exp_fix44(d))


@pytest.mark.parametrize("engine", ["auto", "exact"])
@pytest.mark.parametrize("idx", [1, 2, 4, 5])
def test_workload_parity_full_size(S, dev, oracle, idx, engine):
    from whallm_amd import synth

    w = synth.SAMPLE_WORKLOADS[idx]()
    p = synth.oracle_params(w, oracle.make_params)
    ot, ok = oracle.sample(w.logits_f32, p, w.uniforms, w.history, w.history_len)
    announce(f"wh_sample workload {idx} engine={engine}: {w.name}")
    gt, gk = run_gpu_sample(S, w, dev, engine=engine)
    assert np.array_equal(gk, ok), f"kept mismatch rows {np.nonzero(gk != ok)[0][:10]}"
    assert np.array_equal(gt, ot), f"token mismatch rows {np.nonzero(gt != ot)[0][:10]}"
    ft, _ = oracle.sample_faithful(w.logits_f32, p, w.uniforms, w.history, w.history_len)
    print(f"workload {idx}: GPU vs faithful float32 replay agreement {np.mean(gt == ft):.6f} over {w.B} rows")


def _random_case(rng, B, V):
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
    return x.astype(np.float32)


@pytest.mark.parametrize("seed", range(40))
def test_random_parameters_parity(S, dev, oracle, seed):
    rng = np.random.default_rng(100 + seed)
    B = int(rng.integers(1, 40))
    V = int(rng.choice([17, 256, 1000, 4099, 20000]))
    x = _random_case(rng, B, V)
    chain = int(rng.integers(0, 2))
    T = float(rng.choice([0.0, 0.3, 0.7, 1.0, 1.5]))
    top_p = float(rng.choice([1.0, 0.99, 0.9, 0.5, 0.1]))
    top_k = int(rng.choice([0, 1, 3, 20, V - 1]))
    if chain == 0 and top_k >= V:
        top_k = V - 1  # mlx_lm apply_top_k rejects k >= V
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
        announce(f"wh_sample random seed={seed} engine={engine} B={B} V={V} chain={chain} T={T} p={top_p} "
                 f"k={top_k} minp={min_p} {pen}")
        tok, kept = S.sample(torch.from_numpy(x).to(dev), temperature=T, top_p=top_p, top_k=top_k, min_p=min_p,
                             chain=chain, history=torch.from_numpy(hist).to(dev),
                             history_len=torch.from_numpy(hlen).to(dev), uniforms=torch.from_numpy(u).to(dev),
                             return_kept=True, engine=engine, **pen)
        tok, kept = tok.cpu().numpy(), kept.cpu().numpy()
        if T > 0:
            assert np.array_equal(kept, ok), engine
        assert np.array_equal(tok, ot), engine


@pytest.mark.parametrize("seed", range(6))
def test_small_topk_then_topp(S, dev, oracle, seed):
    """mlx_lm order with a small top-k before top-p: the register merge cuts
    top-p over at most 64 alive candidates.  Quantised logits give dense value
    ties (ids break them); kept-set sizes and tokens must match exactly."""
    rng = np.random.default_rng(900 + seed)
    B, V = 24, 151936
    k = (8, 33, 64)[seed % 3]
    top_p = (0.5, 0.8, 0.95)[seed // 2 % 3]
    T = (0.7, 1.0)[seed % 2]
    x = rng.normal(0.0, 2.5, (B, V))
    if seed % 2 == 0:
        x = np.round(x * 2) / 2  # many equal values among the top candidates
    x[:, rng.choice(V, 12, replace=False)] += 6.0
    x = x.astype(np.float32)
    u = rng.random(B, dtype=np.float32)
    p = oracle.make_params(B, temperature=T, top_p=top_p, top_k=k, min_p=0.0, chain=0)
    ot, ok = oracle.sample(x, p, u, None, None)
    announce(f"wh_sample small top-k then top-p seed={seed} k={k} p={top_p} T={T}")
    tok, kept = S.sample(torch.from_numpy(x).to(dev), temperature=T, top_p=top_p, top_k=k, min_p=0.0, chain=0,
                         uniforms=torch.from_numpy(u).to(dev), return_kept=True)
    assert np.array_equal(kept.cpu().numpy(), ok)
    assert np.array_equal(tok.cpu().numpy(), ot)


@pytest.mark.parametrize("seed", range(3))
def test_dense_block_and_ties_full_vocab(S, dev, oracle, seed):
    """Full-vocabulary rows built to reach the rarer steps of the register
    merge: hundreds of near-max candidates inside one 4096-id block (the
    draw's block has more than 16 members, so both the speculative and the
    filtered draw take the radix levels), rows of exact ties under top-k
    (a radix bucket of count one ends the select early only when it is
    unique), and a temperature != 1 so the draw weights differ from the
    masses."""
    rng = np.random.default_rng(700 + seed)
    B, V = 24, 151936
    x = rng.normal(0, 1.5, (B, V)).astype(np.float32) - 6.0
    for r in range(B):
        kind = r % 3
        if kind == 0:   # a dense block of near-max candidates
            blk = int(rng.integers(0, V // 4096)) * 4096
            ids = blk + rng.choice(4096, 300, replace=False)
            x[r, ids] = rng.uniform(2.0, 2.4, 300).astype(np.float32)
        elif kind == 1:  # exact ties around the k-th value
            ids = rng.choice(V, 64, replace=False)
            x[r, ids] = np.float32(3.0)
            x[r, ids[:5]] = np.float32(3.5)
        else:            # a few clear leaders and a tied tail
            ids = rng.choice(V, 40, replace=False)
            x[r, ids] = np.round(rng.uniform(1.0, 3.0, 40) * 4).astype(np.float32) / 4
    u = rng.random(B, dtype=np.float32)
    cases = [dict(temperature=0.7, top_p=0.9, top_k=0, min_p=0.05, chain=1),
             dict(temperature=1.3, top_p=1.0, top_k=20, min_p=0.0, chain=0),
             dict(temperature=0.8, top_p=0.95, top_k=7, min_p=0.02, chain=1)]
    for c in cases:
        p = oracle.make_params(B, **c)
        ot, ok = oracle.sample(x, p, u)
        announce(f"wh_sample dense-block/ties seed={seed} B={B} V={V} {c}")
        tok, kept = S.sample(torch.from_numpy(x).to(dev), uniforms=torch.from_numpy(u).to(dev), return_kept=True, **c)
        tok, kept = tok.cpu().numpy(), kept.cpu().numpy()
        assert np.array_equal(kept, ok), c
        assert np.array_equal(tok, ot), c


@pytest.mark.parametrize("seed", range(4))
def test_per_row_parameters_parity(S, dev, oracle, seed):
    rng = np.random.default_rng(200 + seed)
    B, V = 48, 3000
    x = _random_case(rng, B, V)
    T = rng.choice([0.0, 0.5, 1.0], B).astype(np.float32)
    pp = rng.choice([1.0, 0.9, 0.6], B).astype(np.float32)
    mp = rng.choice([0.0, 0.05], B).astype(np.float32)
    kk = rng.choice([0, 1, 10, V + 5], B).astype(np.int32)
    u = rng.random(B, dtype=np.float32)
    chain = seed % 2
    p = oracle.make_params(B, temperature=T, top_p=pp, min_p=mp, top_k=np.where(kk >= V, 0, kk), chain=chain)
    ot, ok = oracle.sample(x, p, u)
    announce(f"wh_sample per-row params seed={seed} chain={chain}")
    tok, kept = S.sample(torch.from_numpy(x).to(dev), chain=chain, uniforms=torch.from_numpy(u).to(dev),
                         temperature_rows=torch.from_numpy(T).to(dev), top_p_rows=torch.from_numpy(pp).to(dev),
                         min_p_rows=torch.from_numpy(mp).to(dev), top_k_rows=torch.from_numpy(kk).to(dev),
                         return_kept=True)
    tok, kept = tok.cpu().numpy(), kept.cpu().numpy()
    assert np.array_equal(tok, ot)
    assert np.array_equal(kept[T > 0], ok[T > 0])


def test_sampling_logprobs_rows(S, dev, oracle):
    from whallm_amd import dspark, synth

    w = synth.workload5(B=16)
    p = synth.oracle_params(w, oracle.make_params)
    _, _, orows = oracle.sample(w.logits_f32, p, w.uniforms, w.history, w.history_len, want_rows=True)
    announce("filter_rows WHALLM chain, workload 5 at B=16")
    hist = torch.from_numpy(w.history).to(dev)
    prm = dict(w.params)
    prm.pop("chain")
    rows = S.filter_rows(logits_tensor(w, dev), chain="whallm", history=hist,
                         history_len=torch.from_numpy(w.history_len).to(dev), **prm).cpu().numpy()
    assert np.array_equal(np.isfinite(rows), np.isfinite(orows))
    m = np.isfinite(orows)
    po, pg = np.exp(orows[m].astype(np.float64)), np.exp(rows[m].astype(np.float64))
    assert np.all(np.abs(pg - po) <= 1e-5 * po + 1e-12)
    # the dspark mirror (no penalties: Whallm's DSpark path passes none)
    x = torch.from_numpy(w.logits_f32[:4]).to(dev)
    r2 = dspark.sampling_logprobs(x, 0.8, 0.9, 20, 0.02).cpu().numpy()
    p2 = oracle.make_params(4, temperature=0.8, top_p=0.9, top_k=20, min_p=0.02, chain=1)
    _, _, o2 = oracle.sample(w.logits_f32[:4], p2, np.zeros(4, np.float32), want_rows=True)
    assert np.array_equal(np.isfinite(r2), np.isfinite(o2))
    assert np.allclose(np.exp(r2[np.isfinite(o2)]), np.exp(o2[np.isfinite(o2)]), rtol=1e-5, atol=1e-12)
    assert dspark.sampling_logprobs(x, 0.0, 0.9) is x


def test_masked_filters_match_oracle(S, dev, oracle):
    from whallm_amd import sample_utils as su

    rng = np.random.default_rng(300)
    B, V = 8, 5000
    x = np.round(rng.normal(0, 2, (B, V)) / 0.125) * 0.125
    lp = (x - np.log(np.exp(x - x.max(1, keepdims=True)).sum(1, keepdims=True)) - x.max(1, keepdims=True))
    lp = lp.astype(np.float32)
    t = torch.from_numpy(lp).to(dev)
    announce("apply_top_k / apply_top_p / apply_min_p")
    for name, fn, kw in [("k", su.apply_top_k, dict(top_k=37)), ("p", su.apply_top_p, dict(top_p=0.7)),
                         ("m", su.apply_min_p, dict(min_p=0.05))]:
        out = fn(t, *kw.values()).cpu().numpy()
        p = oracle.make_params(B, temperature=1.0, chain=1, **kw)
        _, kept, rows = oracle.sample(lp, p, np.zeros(B, np.float32), want_rows=True)
        assert np.array_equal(np.isfinite(out), np.isfinite(rows)), name
        assert np.array_equal(out[np.isfinite(out)], lp[np.isfinite(out)]), name


def test_penalty_processors_in_place(S, dev, oracle):
    from whallm_amd import sample_utils as su

    rng = np.random.default_rng(400)
    B, V, H = 4, 2000, 500
    x = rng.normal(0, 2, (B, V)).astype(np.float32)
    hist = rng.integers(0, V, (B, H)).astype(np.int32)
    hist[:, :50] = hist[:, :1]  # repeats
    procs = su.make_logits_processors(repetition_penalty=1.3, presence_penalty=0.5, frequency_penalty=0.2,
                                      repetition_context_size=100, presence_context_size=0,
                                      frequency_context_size=300)
    announce("make_logits_processors float32 and bf16 in place")
    t = torch.from_numpy(x.copy()).to(dev)
    ht = torch.from_numpy(hist).to(dev)
    for pr in procs:
        t = pr(ht, t)
    p = oracle.make_params(B, repetition_penalty=1.3, presence_penalty=0.5, frequency_penalty=0.2,
                           repetition_context=100, presence_context=0, frequency_context=300)
    want = oracle.penalize(x, p, hist)
    assert np.array_equal(t.cpu().numpy(), want)
    from whallm_amd.synth import bf16_bits_to_f32, f32_to_bf16_bits

    bits = f32_to_bf16_bits(x)
    tb = torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)
    tb = procs[0](ht, tb)
    p1 = oracle.make_params(B, repetition_penalty=1.3, repetition_context=100)
    want_b = f32_to_bf16_bits(oracle.penalize(bf16_bits_to_f32(bits), p1, hist))
    assert np.array_equal(tb.view(torch.int16).cpu().numpy().view(np.uint16), want_b)


@pytest.mark.parametrize("seed", range(6))
def test_verify_logprobs_parity(S, dev, oracle, seed):
    rng = np.random.default_rng(500 + seed)
    B = int(rng.integers(1, 20))
    n = int(rng.integers(0, 7))
    V = int(rng.choice([5, 300, 4000, 30000]))
    T = float(rng.choice([0.0, 0.6, 1.0]))
    tl = rng.normal(0, 2, (B, n + 1, V))
    tl = (tl - np.log(np.exp(tl).sum(-1, keepdims=True))).astype(np.float32)
    dl = tl[:, :n] + rng.normal(0, 0.7, (B, n, V))
    dl = (dl - np.log(np.exp(dl).sum(-1, keepdims=True))).astype(np.float32)
    if seed % 3 == 2:
        dl[rng.random(dl.shape) < 0.2] = -np.inf
        tl[rng.random(tl.shape) < 0.2] = -np.inf
    toks = np.empty((B, n), np.int32)
    for b in range(B):
        for j in range(n):
            pr = np.exp(dl[b, j].astype(np.float64))
            toks[b, j] = rng.choice(V, p=pr / pr.sum())
    u = rng.random((B, n + 1), dtype=np.float32)
    oa, ot, orow = oracle.verify_logprobs(dl, tl, toks, u, T, want_rows=True)
    announce(f"wh_verify_logprobs seed={seed} B={B} n={n} V={V} T={T}")
    a, t, row = S.verify_logprobs(torch.from_numpy(tl).to(dev), torch.from_numpy(dl).to(dev),
                                  torch.from_numpy(toks).to(dev), T, uniforms=torch.from_numpy(u).to(dev),
                                  return_row=True)
    assert np.array_equal(a.cpu().numpy(), oa)
    assert np.array_equal(t.cpu().numpy(), ot)
    row = row.cpu().numpy()
    assert np.array_equal(np.isfinite(row), np.isfinite(orow))
    m = np.isfinite(orow)
    assert np.allclose(np.exp(row[m].astype(np.float64)), np.exp(orow[m].astype(np.float64)), rtol=1e-5, atol=1e-12)


def test_verify_fused_workload3_full_size(S, dev, oracle):
    from whallm_amd import synth

    w = synth.workload3()
    oa, ot = oracle.verify_fused(w.target_logits, w.draft_q, w.draft_tokens, w.uniforms, w.temperature)
    announce(f"wh_verify_fused workload 3: {w.name}")
    a, t = S.verify_fused(torch.from_numpy(w.target_logits).to(dev), torch.from_numpy(w.draft_q).to(dev),
                          torch.from_numpy(w.draft_tokens).to(dev), w.temperature,
                          uniforms=torch.from_numpy(w.uniforms).to(dev))
    assert np.array_equal(a.cpu().numpy(), oa)
    assert np.array_equal(t.cpu().numpy(), ot)


@pytest.mark.gpu
@pytest.mark.parametrize("force_exact", [False, True])
@pytest.mark.parametrize("seed", range(12))
def test_verify_fused_sliced(S, dev, oracle, seed, force_exact):
    """The sliced verifier (T > 0, V % 4 == 0): bounds-decided ratio tests,
    exact residual draw; with wh_verify_force_exact every entry takes the
    exact per-row algorithm that undecided entries use.  Seeds 10 and 11 use
    long drafts (n = 17, 63: the most the sliced form takes)."""
    rng = np.random.default_rng(700 + seed)
    B, n = int(rng.integers(1, 20)), int(rng.integers(1, 11))
    if seed >= 10:
        B, n = int(rng.integers(1, 4)), (17, 63)[seed - 10]
    V = int(rng.choice([4096, 20000, 129280])) if seed < 8 else 129280
    T = float(rng.choice([0.3, 0.8, 1.0, 2.0]))
    x = rng.normal(0, 2.5, (B, n + 1, V)).astype(np.float32)
    if seed % 4 == 1:
        x = (np.round(x * 4) / 4).astype(np.float32)  # dense ties
    dl = x[:, :n].astype(np.float64) + rng.normal(0, 0.5, (B, n, V))
    z = dl / T
    z -= z.max(-1, keepdims=True)
    q = np.exp(z)
    q /= q.sum(-1, keepdims=True)
    cdf = np.cumsum(q, -1)
    toks = np.array([[min(int(np.searchsorted(cdf[b, j], rng.random() * cdf[b, j, -1], side="right")), V - 1)
                      for j in range(n)] for b in range(B)], np.int32)
    q = q.astype(np.float32)
    if seed % 4 == 2:
        x[rng.random(x.shape) < 0.3] = -np.inf
        x[0, 0, :] = -np.inf  # a row with no finite logit
    if seed % 4 == 3:
        q[rng.random(q.shape) < 0.1] = 0.0
    if seed % 5 == 0:
        toks[0, 0] = V  # out of range: rejected
    u = rng.random((B, n + 1), dtype=np.float32)
    from whallm_amd import _lib

    _lib.lib().wh_verify_force_exact(1 if force_exact else 0)
    oa, ot = oracle.verify_fused(x, q, toks, u, T)
    announce(f"wh_verify_fused sliced seed={seed} B={B} n={n} V={V} T={T} force_exact={force_exact}")
    try:
        a, t = S.verify_fused(torch.from_numpy(x).to(dev), torch.from_numpy(q).to(dev),
                              torch.from_numpy(toks).to(dev), T, uniforms=torch.from_numpy(u).to(dev))
    finally:
        _lib.lib().wh_verify_force_exact(0)
    assert np.array_equal(a.cpu().numpy(), oa)
    assert np.array_equal(t.cpu().numpy(), ot)


@pytest.mark.parametrize("seed", range(4))
def test_verify_fused_random(S, dev, oracle, seed):
    rng = np.random.default_rng(600 + seed)
    B, n, V = int(rng.integers(1, 12)), int(rng.integers(0, 6)), int(rng.choice([7, 500, 20000]))
    T = float(rng.choice([0.0, 0.5, 1.0]))
    x = rng.normal(0, 2, (B, n + 1, V)).astype(np.float32)
    q = rng.dirichlet(np.ones(V) * 0.5, (B, n)).astype(np.float32) if n else np.zeros((B, 0, V), np.float32)
    toks = rng.integers(0, V, (B, n)).astype(np.int32)
    u = rng.random((B, n + 1), dtype=np.float32)
    oa, ot = oracle.verify_fused(x, q, toks, u, T)
    announce(f"wh_verify_fused random seed={seed} B={B} n={n} V={V} T={T}")
    a, t = S.verify_fused(torch.from_numpy(x).to(dev), torch.from_numpy(q).to(dev), torch.from_numpy(toks).to(dev),
                          T, uniforms=torch.from_numpy(u).to(dev))
    assert np.array_equal(a.cpu().numpy(), oa)
    assert np.array_equal(t.cpu().numpy(), ot)


@pytest.mark.parametrize("chain", [0, 1])
def test_confident_rows_settle_on_fast_engine(S, dev, oracle, chain):
    """Rows where one token holds most of the mass (a confident model), with
    top-p and min-p together: min-p sets the slices' thresholds, so the
    slices take no float sums and the candidates' normaliser bounds cannot
    place the top-p cut.  The merge's second pass (a float sum over the row)
    must settle every row on the fast engine (path 7 or 8, no exact-engine
    fallback), with tokens and kept sizes equal to the oracle's."""
    rng = np.random.default_rng(1300 + chain)
    B, V = 32, 151936
    x = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    lead = rng.integers(0, V, B)
    x[np.arange(B), lead] += np.float32(12.0) + rng.uniform(0.0, 6.0, B).astype(np.float32)
    u = rng.random(B, dtype=np.float32)
    c = (dict(temperature=1.0, top_p=0.9, top_k=0, min_p=0.05) if chain == 0
         else dict(temperature=0.7, top_p=0.95, top_k=20, min_p=0.01))
    p = oracle.make_params(B, chain=chain, **c)
    ot, ok = oracle.sample(x, p, u)
    announce(f"wh_sample confident rows chain={chain} {c}")
    tok, kept = S.sample(torch.from_numpy(x).to(dev), uniforms=torch.from_numpy(u).to(dev), return_kept=True,
                         chain=chain, **c)
    paths = S.last_paths(dev, B).cpu().numpy()
    assert np.array_equal(kept.cpu().numpy(), ok)
    assert np.array_equal(tok.cpu().numpy(), ot)
    assert not np.any((paths == 1) | (paths == 3)), paths
    assert np.any((paths == 7) | (paths == 8)), paths  # the second pass ran


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_confident_rows_with_penalties_settle(S, dev, oracle, dtype):
    """The merge's second bounds pass with a penalty table (built after the
    candidates in LDS): confident bf16 and float32 rows, penalties over a
    history that holds the leading token in half the rows, Whallm's order
    with top-p, min-p and top-k.  Tokens and kept sizes equal to the oracle's,
    no exact-engine fallback."""
    from whallm_amd import synth

    rng = np.random.default_rng(1400 + (dtype == "bf16"))
    B, V, H = 32, 151936, 256
    x = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    lead = rng.integers(0, V, B)
    x[np.arange(B), lead] += np.float32(12.0) + rng.uniform(0.0, 6.0, B).astype(np.float32)
    hist = rng.integers(0, V, (B, H)).astype(np.int32)
    hist[::2, :8] = lead[::2, None]
    hl = np.full(B, H, np.int32)
    if dtype == "bf16":
        bits = synth.f32_to_bf16_bits(x)
        x = synth.bf16_bits_to_f32(bits)
        xd = torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        xd = torch.from_numpy(x).to(dev)
    u = rng.random(B, dtype=np.float32)
    c = dict(temperature=0.8, top_p=0.95, top_k=40, min_p=0.01, repetition_penalty=1.2, presence_penalty=0.3,
             frequency_penalty=0.1, repetition_context=H, presence_context=H, frequency_context=H)
    p = oracle.make_params(B, chain=1, **c)
    ot, ok = oracle.sample(x, p, u, hist, hl)
    announce(f"wh_sample confident rows with penalties {dtype}")
    tok, kept = S.sample(xd, uniforms=torch.from_numpy(u).to(dev), history=torch.from_numpy(hist).to(dev),
                         history_len=torch.from_numpy(hl).to(dev), return_kept=True, chain=1, **c)
    paths = S.last_paths(dev, B).cpu().numpy()
    assert np.array_equal(kept.cpu().numpy(), ok)
    assert np.array_equal(tok.cpu().numpy(), ot)
    assert not np.any((paths == 1) | (paths == 3)), paths
    assert np.any((paths == 7) | (paths == 8)), paths  # the second pass ran


@pytest.mark.parametrize("B,dtype", [(8, "bf16"), (24, "f32"), (40, "bf16"), (7, "f32"), (9, "bf16")])
def test_slice_placement_batches(S, dev, oracle, B, dtype):
    """Batch sizes that are multiples of 8 run the slice grid that puts a
    row's slices on one XCD (row 8 y + x % 8, slice x / 8); others run the
    plain (slice, row) grid.  Per-row histories with all three penalties,
    top-k, top-p and min-p: tokens and kept counts equal the oracle's on the
    fast engine, for every row (a misplaced row or slice would read another
    row's logits or history)."""
    from whallm_amd import synth

    rng = np.random.default_rng(900 + B)
    V, H = 151936 if dtype == "bf16" else 129280, 512
    x = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    x[np.arange(B), rng.integers(0, V, B)] += 9.0  # a distinct leader per row
    hist = rng.integers(0, V, (B, H)).astype(np.int32)
    hlen = rng.integers(H // 2, H + 1, B).astype(np.int32)
    if dtype == "bf16":
        bits = synth.f32_to_bf16_bits(x)
        x = synth.bf16_bits_to_f32(bits)
        xd = torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        xd = torch.from_numpy(x).to(dev)
    u = rng.random(B, dtype=np.float32)
    kw = dict(temperature=0.8, top_k=40, top_p=0.9, min_p=0.02, repetition_penalty=1.2, presence_penalty=0.4,
              frequency_penalty=0.2, repetition_context=H, presence_context=64, frequency_context=H)
    p = oracle.make_params(B, chain=1, **kw)
    ot, ok = oracle.sample(x, p, u, hist, hlen)
    announce(f"wh_sample slice placement B={B} {dtype}")
    tok, kept = S.sample(xd, chain=1, history=torch.from_numpy(hist).to(dev),
                         history_len=torch.from_numpy(hlen).to(dev), uniforms=torch.from_numpy(u).to(dev),
                         return_kept=True, **kw)
    paths = S.last_paths(dev, B).cpu().numpy()
    assert not np.any((paths == 1) | (paths == 3)), paths
    assert np.array_equal(kept.cpu().numpy(), ok)
    assert np.array_equal(tok.cpu().numpy(), ot)
