"""The decode-step glue on the GPU: device-resident history (wh_history_append)
and TokenSelector / generate() against the oracle run as generate_step does
it (runtime/deepseek_v4_ssd/generation.py:1279-1293, 1465-1475): the history
is the prompt plus every generated id, the processors read its last
`context` ids, and the sampler picks the next id.  The model is a fixed table
lookup (logits = table[last id mod 64]) so both sides see the same rows.
Tokens must be identical at every step."""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
V = 32000


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


def _table(seed):
    rng = np.random.default_rng(seed)
    t = rng.normal(0, 2.0, (64, V)).astype(np.float32)
    # a few strong ids per row make repeats (and so the penalties) matter
    for r in range(64):
        t[r, rng.integers(0, V, 4)] += 6.0
    return t


def _oracle_run(oracle, table, prompts, steps, U, params):
    hist = [list(p) for p in prompts]
    last = [p[-1] for p in prompts]
    out = []
    for s in range(steps):
        x = table[np.array(last) % 64]
        H = max(len(h) for h in hist)
        ha = np.zeros((len(hist), H), np.int32)
        for b, h in enumerate(hist):
            ha[b, :len(h)] = h
        tok, _ = oracle.sample(x, params, U[s], ha, np.array([len(h) for h in hist], np.int32))
        out.append(tok.tolist())
        for b, t in enumerate(tok):
            hist[b].append(int(t))
        last = tok.tolist()
    return out, hist


PROMPTS = [[5, 9, 9, 1, 17], list(range(100, 130)), [7], [3, 3, 3, 3, 2, 2, 40, 41, 42, 43, 44, 45]]


@pytest.mark.parametrize("case", ["windowed", "whole_history", "greedy", "whallm_chain"])
def test_generate_matches_oracle_loop(dev, oracle, case):
    from whallm_amd.decode import TokenSelector, generate

    table = _table(7)
    B, steps = len(PROMPTS), 60
    rng = np.random.default_rng(11)
    U = rng.random((steps, B), dtype=np.float32)
    kw = dict(temperature=0.8, top_p=0.9, top_k=50, min_p=0.02, repetition_penalty=1.3, repetition_context=20,
              presence_penalty=0.5, presence_context=12, frequency_penalty=0.25, frequency_context=16)
    chain = 0
    if case == "whole_history":
        kw.update(presence_context=0)
    elif case == "greedy":
        kw.update(temperature=0.0)
    elif case == "whallm_chain":
        chain = 1
    sel = TokenSelector(chain="mlx" if chain == 0 else "whallm", **kw)
    state = sel.make_state(PROMPTS, dev, capacity=0 if case == "whole_history" else 40)
    p = oracle.make_params(B, chain=chain, **kw)
    want, full = _oracle_run(oracle, table, PROMPTS, steps, U, p)
    tab = torch.from_numpy(table).to(dev)
    Ud = torch.from_numpy(U).to(dev)
    announce(f"decode loop {case} B={B} steps={steps} capacity={state.capacity} keep={state.keep}")
    got = list(generate(lambda last: tab[last.long() % 64], PROMPTS, max_tokens=steps, selector=sel,
                        uniforms=lambda s: Ud[s], state=state))
    assert got == want
    # the device history is the tail of the full one, at least `keep` long
    for b, row in enumerate(state.rows()):
        assert row == full[b][-len(row):]
        if state.keep is not None:
            assert len(row) >= min(state.keep, len(full[b]))
        else:
            assert row == full[b]


def test_top_logprobs_path_same_tokens(dev, oracle):
    """With top_logprobs the selector penalises a float32 copy, then samples
    it without history: the tokens must equal the fused call's, and the top-n
    must be the oracle's top-n of the penalised row."""
    from whallm_amd.decode import TokenSelector

    table = _table(8)
    B, steps, n = len(PROMPTS), 25, 8
    rng = np.random.default_rng(12)
    U = torch.from_numpy(rng.random((steps, B), dtype=np.float32)).to(dev)
    kw = dict(temperature=0.7, top_p=0.95, repetition_penalty=1.25, presence_penalty=0.4, frequency_penalty=0.1)
    fused, withlp = TokenSelector(**kw), TokenSelector(top_logprobs=n, **kw)
    s1 = fused.make_state(PROMPTS, dev, capacity=48)
    s2 = withlp.make_state(PROMPTS, dev, capacity=48)
    p = oracle.make_params(B, chain=0, repetition_context=20, presence_context=20, frequency_context=20, **kw)
    tab_bf16 = torch.from_numpy(table).to(dev).to(torch.bfloat16)
    last = torch.tensor([q[-1] for q in PROMPTS], dtype=torch.int32, device=dev)
    for s in range(steps):
        x = tab_bf16[last.long() % 64]
        announce(f"selector step {s} (bf16 logits, top_logprobs={n})")
        hist_before = s2.rows()
        t1 = fused(x, s1, uniforms=U[s])
        t2, (ids, lps, tlp) = withlp(x, s2, uniforms=U[s])
        assert torch.equal(t1, t2), s
        H = max(len(h) for h in hist_before)
        ha = np.zeros((B, H), np.int32)
        for b, h in enumerate(hist_before):
            ha[b, :len(h)] = h
        pen = oracle.penalize(x.float().cpu().numpy(), p, ha, np.array([len(h) for h in hist_before], np.int32))
        oi, ol = oracle.top_logprobs(pen, n)
        assert np.array_equal(ids.cpu().numpy(), oi)
        assert np.allclose(lps.cpu().numpy(), ol, atol=2e-6, rtol=0)
        last = t1
    assert s1.rows() == s2.rows()


def test_history_append_mtp_commit(dev):
    """The MTP commit (qwen4_exp.py:1143-1149): accepted drafts, then the next
    token; rows that fill keep their last `keep` ids."""
    from whallm_amd.decode import DecodeState

    rng = np.random.default_rng(13)
    B, n, cap, keep = 6, 5, 32, 20
    prompts = [list(rng.integers(0, 1000, int(rng.integers(1, 30)))) for _ in range(B)]
    st = DecodeState.from_prompts(prompts, cap, keep, dev, max_append=n)
    model = [list(p)[-keep:] for p in prompts]
    for r in range(40):
        drafts = rng.integers(0, 1000, (B, n)).astype(np.int32)
        acc = rng.integers(-1, n + 2, B).astype(np.int32)  # clamped to [0, n] on the device
        nxt = rng.integers(0, 1000, B).astype(np.int32)
        announce(f"wh_history_append mtp round {r}")
        st.append(torch.from_numpy(drafts).to(dev), counts=torch.from_numpy(acc).to(dev),
                  tail=torch.from_numpy(nxt).to(dev))
        for b in range(B):
            new = list(drafts[b, :min(max(acc[b], 0), n)]) + [int(nxt[b])]
            model[b] = model[b] + new if len(model[b]) + len(new) <= cap else model[b][-keep:] + new
    assert st.rows() == [[int(v) for v in row] for row in model]


def test_default_options_loop_matches_oracle(dev, oracle):
    """The reference's default request (T 0.2, top-p 0.98, no top-k / min-p;
    generation.py:109-118) at V = 151,936, one sequence: the rows take the
    wide exact engine; tokens identical to the oracle at every step."""
    from whallm_amd.decode import GenerationOptions, TokenSelector, generate

    Vq = 151936
    rng = np.random.default_rng(21)
    table = rng.normal(0, 2.0, (16, Vq)).astype(np.float32)
    opts = GenerationOptions(presence_penalty=0.3, repetition_penalty=1.1)
    sel = TokenSelector.from_options(opts)
    steps = 24
    U = rng.random((steps, 1), dtype=np.float32)
    prompt = [[11, 12, 13, 11]]
    p = oracle.make_params(1, chain=0, temperature=0.2, top_p=0.98, presence_penalty=0.3, repetition_penalty=1.1,
                           presence_context=20, repetition_context=20)
    hist = list(prompt[0])
    want = []
    last = prompt[0][-1]
    for s in range(steps):
        x = table[last % 16][None]
        tok, _ = oracle.sample(x, p, U[s], np.array([hist], np.int32), np.array([len(hist)], np.int32))
        want.append([int(tok[0])])
        hist.append(int(tok[0]))
        last = int(tok[0])
    tab = torch.from_numpy(table).to(dev)
    Ud = torch.from_numpy(U).to(dev)
    announce("decode loop, default options, V=151936")
    got = list(generate(lambda l: tab[l.long() % 16], prompt, max_tokens=steps, selector=sel,
                        uniforms=lambda s: Ud[s]))
    assert got == want
