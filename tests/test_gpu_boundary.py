"""GPU vs the faithful float32 replay of the reference's op order, at the
full size of every workload.

The HIP kernels reproduce the contract oracle bit for bit (asserted here
again).  Against the faithful replay (oracle/wh_oracle.c, who_*_faithful:
logsumexp, stable argsort, sequential float32 cumsum for top-p, as
runtime/deepseek_v4_ssd/dspark.py:358-375 and 857-904 and mlx_lm run them)
every disagreement must lie within 1e-6 of a cumulative-probability boundary
(tests/boundary.py computes the distance in float64).  The agreement rate per
workload goes to the run's summary.
"""
import sys

import numpy as np
import pytest

from boundary import sample_margins, verify_margin

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
TOL = 1e-6


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


def _logits(w, dev):
    if w.dtype == "bf16":
        return torch.from_numpy(w.logits_bits.view(np.int16)).to(dev).view(torch.bfloat16)
    return torch.from_numpy(w.logits_f32).to(dev)


@pytest.mark.parametrize("idx", [1, 2, 4, 5])
def test_sample_mismatches_lie_on_boundaries(dev, oracle, report, idx):
    from whallm_amd import sampling, synth

    w = synth.SAMPLE_WORKLOADS[idx]()
    p = synth.oracle_params(w, oracle.make_params)
    announce(f"boundary check, workload {idx}: {w.name}")
    prm = dict(w.params)
    tok = sampling.sample(_logits(w, dev), uniforms=torch.from_numpy(w.uniforms).to(dev),
                          history=None if w.history is None else torch.from_numpy(w.history).to(dev),
                          history_len=None if w.history_len is None else torch.from_numpy(w.history_len).to(dev),
                          top_k_rows=None if w.top_k_rows is None else torch.from_numpy(w.top_k_rows).to(dev), **prm)
    got = tok.cpu().numpy()
    want, _ = oracle.sample(w.logits_f32, p, w.uniforms, w.history, w.history_len)
    assert np.array_equal(got, want)
    faithful, _ = oracle.sample_faithful(w.logits_f32, p, w.uniforms, w.history, w.history_len)
    diff = np.nonzero(got != faithful)[0]
    if diff.size:
        pen = oracle.penalize(w.logits_f32[diff], p[diff], None if w.history is None else w.history[diff],
                              None if w.history_len is None else w.history_len[diff]) if w.history is not None \
            else w.logits_f32[diff]
        marg = sample_margins(pen, p[diff], w.uniforms[diff])
        far = diff[marg >= TOL]
        assert far.size == 0, f"rows {far[:8].tolist()} differ from the faithful replay away from any boundary"
    report(f"workload {idx}: GPU vs faithful float32 replay, {w.B - diff.size}/{w.B} rows agree "
           f"(mismatch rate {diff.size / w.B:.4f}; every mismatch within {TOL:g} of a boundary)")


def test_verify_mismatches_lie_on_boundaries(dev, oracle, report):
    from whallm_amd import sampling, synth

    w = synth.workload3()
    B, n, V, T = w.B, w.n, w.V, w.temperature
    announce(f"boundary check, workload 3: {w.name}")
    a, t = sampling.verify_fused(torch.from_numpy(w.target_logits).to(dev), torch.from_numpy(w.draft_q).to(dev),
                                 torch.from_numpy(w.draft_tokens).to(dev), T,
                                 uniforms=torch.from_numpy(w.uniforms).to(dev))
    a, t = a.cpu().numpy(), t.cpu().numpy()
    oa, ot = oracle.verify_fused(w.target_logits, w.draft_q, w.draft_tokens, w.uniforms, T)
    assert np.array_equal(a, oa) and np.array_equal(t, ot)
    # the reference's inputs to _verify: target rows sampling_logprobs(x, T,
    # top_p=1) (dspark.py:663-670) and the draft's logprob rows log q
    pr = oracle.make_params(B * (n + 1), temperature=T, chain=1)
    _, _, tlp = oracle.sample_faithful(w.target_logits.reshape(-1, V), pr, np.zeros(B * (n + 1), np.float32),
                                       want_rows=True)
    with np.errstate(divide="ignore"):
        dlp = np.log(w.draft_q)
    fa, ft = oracle.verify_faithful(dlp, tlp.reshape(B, n + 1, V), w.draft_tokens, w.uniforms, T)
    diff = np.nonzero((a != fa) | (t != ft))[0]
    for b in diff:
        x = w.target_logits[b].astype(np.float64) / T
        tl = x - (np.log(np.exp(x - x.max(-1, keepdims=True)).sum(-1, keepdims=True)) + x.max(-1, keepdims=True))
        with np.errstate(divide="ignore"):
            dl = np.log(w.draft_q[b].astype(np.float64))
        assert verify_margin(tl, dl, w.draft_tokens[b], w.uniforms[b], T) < TOL, f"entry {b}"
    report(f"workload 3: GPU vs faithful float32 replay of _verify, {B - diff.size}/{B} entries agree "
           f"(mismatch rate {diff.size / B:.4f}; every mismatch within {TOL:g} of a boundary)")


def test_top_p_threshold_from_the_double(dev, oracle):
    """top_p = 0.9 (a Python float) gives MLX's threshold fp32(1 - 0.9) =
    0.1f on the GPU too: a row whose last token's share lies in
    (0.1f, 0.100000024f] keeps it, on both engines and both chains."""
    from test_faithful_pins import theta_split_row
    from whallm_amd import sampling

    x = theta_split_row(oracle)
    V = 4096  # pad to the fast engine's alignment with -inf entries
    row = np.full((1, V), -np.inf, np.float32)
    row[0, :x.size] = x
    t = torch.from_numpy(row).to(dev)
    announce("top-p threshold from the double (0.9)")
    for chain in ("mlx", "whallm"):
        for engine in ("auto", "exact"):
            _, kept = sampling.sample(t, temperature=1.0, top_p=0.9, chain=chain, engine=engine,
                                      uniforms=torch.full((1,), 0.5, device=dev), return_kept=True)
            assert int(kept[0]) == 9, (chain, engine)
            _, kept = sampling.sample(t, temperature=1.0, top_p=float(np.float32(0.9)), chain=chain, engine=engine,
                                      uniforms=torch.full((1,), 0.5, device=dev), return_kept=True)
            assert int(kept[0]) == 8, (chain, engine)
