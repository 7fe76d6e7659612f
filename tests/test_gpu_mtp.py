"""MTP verification rows (runtime/deepseek_v4_ssd/qwen4_exp.py:946-958,
1083-1099) on the GPU at workload 5's shape: 32 batch entries x (4 drafts +
the bonus position), V = 151,936 bf16, 4,096 committed history ids per
entry, repetition 1.05 + presence 0.4 + frequency 0.2 over the last 4,096
ids, T 0.6, top-k 20, top-p 0.8, min-p 0.02.

Row i of an entry is penalised over committed + drafts[:i]; the oracle
builds each row's history explicitly.  The rows must match the oracle's
within 1e-5 (probabilities) with identical kept sets, and the verifier fed
with them must give the oracle's accepted counts and tokens on the same rows.
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


@pytest.mark.parametrize("seed", range(2))
def test_mtp_target_rows_and_verify(dev, oracle, seed):
    from whallm_amd import mtp, synth

    rng = np.random.default_rng(2000 + seed)
    B, n, V, H = 32, 4, synth.V_QWEN, 4096
    T, top_p, top_k, min_p = 0.6, 0.8, 20, 0.02
    pen = dict(repetition_penalty=1.05, presence_penalty=0.4, frequency_penalty=0.2, repetition_context=H,
               presence_context=H, frequency_context=H)
    x = (np.round(rng.normal(0.0, 2.0, (B, n + 1, V)) / 0.125) * 0.125).astype(np.float32)
    bits = synth.f32_to_bf16_bits(x)
    committed = synth.zipf_ids(rng, 1.1, (B, H), V, rng.permutation(V))
    clen = rng.integers(H - 64, H + 1, B).astype(np.int32)
    drafts = np.argsort(-x[:, :n], axis=-1)[:, :, 0].astype(np.int32)  # the drafts are the leaders
    drafts[:, 1::2] = rng.integers(0, V, (B, (n + 1) // 2))
    # the oracle's rows: each (entry, position) with its own explicit history
    hx = np.zeros((B * (n + 1), H + n), np.int32)
    hl = np.zeros(B * (n + 1), np.int32)
    for b in range(B):
        for i in range(n + 1):
            seq = np.concatenate([committed[b, :clen[b]], drafts[b, :i]])
            hx[b * (n + 1) + i, :seq.size] = seq
            hl[b * (n + 1) + i] = seq.size
    p = oracle.make_params(B * (n + 1), temperature=T, top_p=top_p, top_k=top_k, min_p=min_p, chain=1, **pen)
    _, okept, orows = oracle.sample(x.reshape(-1, V), p, np.zeros(B * (n + 1), np.float32), hx, hl, want_rows=True)
    # the device: one shared history row per entry, with room for the drafts
    hist = torch.zeros(B, H + n + 8, dtype=torch.int32, device=dev)
    hist[:, :H] = torch.from_numpy(committed).to(dev)
    hlen = torch.from_numpy(clen).to(dev)
    xt = torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)
    dl = rng.normal(0, 2, (B, n, V)).astype(np.float32)
    dl[np.arange(B)[:, None], np.arange(n)[None, :], drafts] += 4.0
    dl = (dl - np.log(np.exp(dl.astype(np.float64)).sum(-1, keepdims=True))).astype(np.float32)
    u = rng.random((B, n + 1), dtype=np.float32)
    announce(f"mtp target rows + verify seed={seed} B={B} n={n} V={V} H={H}")
    acc, tok, rows = mtp.verify_block(xt, hist, hlen, torch.from_numpy(drafts).to(dev), torch.from_numpy(dl).to(dev),
                                      temperature=T, top_p=top_p, top_k=top_k, min_p=min_p,
                                      uniforms=torch.from_numpy(u).to(dev), **pen)
    r = rows.cpu().numpy().reshape(-1, V)
    assert np.array_equal(np.isfinite(r), np.isfinite(orows))
    assert np.array_equal(np.isfinite(r).sum(-1), okept)
    m = np.isfinite(orows)
    assert np.allclose(np.exp(r[m].astype(np.float64)), np.exp(orows[m].astype(np.float64)), rtol=1e-5, atol=1e-12)
    # the drafts landed in the shared history rows
    h = hist.cpu().numpy()
    for b in range(B):
        assert np.array_equal(h[b, clen[b]:clen[b] + n], drafts[b])
    oa, ot = oracle.verify_logprobs(dl, r.reshape(B, n + 1, V), drafts, u, T)
    assert np.array_equal(acc.cpu().numpy(), oa)
    assert np.array_equal(tok.cpu().numpy(), ot)


def test_mtp_rows_qwen_vocabulary(dev, oracle):
    """The MTP target rows at Qwen's production vocabulary (V = 248,320,
    qwen4_exp.py:44): penalties over history + drafts[:i], chain B."""
    from whallm_amd import mtp

    rng = np.random.default_rng(248)
    B, n, V, H = 2, 3, 248320, 40
    logits = rng.normal(0, 2.0, (B, n + 1, V)).astype(np.float32)
    hist = rng.integers(0, V, (B, H + n)).astype(np.int32)  # room for the drafts after the committed ids
    hlen = np.array([H, 17], np.int32)
    drafts = rng.integers(0, V, (B, n)).astype(np.int32)
    kw = dict(temperature=0.6, top_p=0.8, top_k=20, min_p=0.02, repetition_penalty=1.05, presence_penalty=0.4)
    sys.stderr.write("[gpu-case] mtp rows V=248320\n")
    rows = mtp.adjusted_logprobs_rows(torch.from_numpy(logits).to(dev), torch.from_numpy(hist).to(dev),
                                      torch.from_numpy(hlen).to(dev), torch.from_numpy(drafts).to(dev), **kw)
    rows = rows.cpu().numpy().reshape(B, n + 1, V)
    p = oracle.make_params(1, chain=1, temperature=0.6, top_p=0.8, top_k=20, min_p=0.02, repetition_penalty=1.05,
                           presence_penalty=0.4, repetition_context=20, presence_context=20)
    for b in range(B):
        for i in range(n + 1):
            h = np.concatenate([hist[b, :hlen[b]], drafts[b, :i]]).astype(np.int32)
            _, _, orow = oracle.sample(logits[b, i][None], p, np.zeros(1, np.float32), h[None],
                                       np.array([h.size], np.int32), want_rows=True)
            fin = np.isfinite(orow[0])
            assert np.array_equal(np.isfinite(rows[b, i]), fin)
            assert np.allclose(np.exp(rows[b, i][fin].astype(np.float64)), np.exp(orow[0][fin].astype(np.float64)),
                               rtol=1e-5, atol=1e-12)
