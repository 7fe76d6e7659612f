"""The DSpark draft block on the GPU (runtime/deepseek_v4_ssd/dspark.py:
315-344, deepseek_v41/dspark.py:128-142) against the CPU oracle.

wh_markov_logits must reproduce the oracle's Markov-biased logits bit for bit
(float32 and bf16 weights, V = 129,280, rank 256); a 5-position draft block
must give the oracle's tokens exactly and its sampling_logprobs rows within
1e-5 (probabilities), with every position's previous token read on the
device.
"""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
V, RANK = 129280, 256


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


def _weights(rng, dtype, dev):
    from whallm_amd.synth import bf16_bits_to_f32, f32_to_bf16_bits

    w1 = rng.normal(0, 0.05, (V, RANK)).astype(np.float32)
    w2 = rng.normal(0, 0.08, (V, RANK)).astype(np.float32)
    if dtype == "bf16":
        b1, b2 = f32_to_bf16_bits(w1), f32_to_bf16_bits(w2)
        t1 = torch.from_numpy(b1.view(np.int16)).to(dev).view(torch.bfloat16)
        t2 = torch.from_numpy(b2.view(np.int16)).to(dev).view(torch.bfloat16)
        return b1, b2, t1, t2
    return w1, w2, torch.from_numpy(w1).to(dev), torch.from_numpy(w2).to(dev)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_markov_logits_bit_exact(dev, oracle, dtype):
    from whallm_amd import draft

    rng = np.random.default_rng(2100 + (dtype == "bf16"))
    o1, o2, t1, t2 = _weights(rng, dtype, dev)
    base = rng.normal(0, 2.5, V).astype(np.float32)
    for prev in (0, 777, V - 1):
        announce(f"wh_markov_logits {dtype} prev={prev}")
        got = draft.markov_logits(torch.from_numpy(base).to(dev), t1, t2,
                                  torch.tensor([prev], dtype=torch.int32, device=dev)).cpu().numpy()
        want = oracle.markov_logits(base, o1, o2, prev)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), prev


@pytest.mark.parametrize("T", [0.0, 0.8])
def test_draft_block_matches_oracle(dev, oracle, T):
    from whallm_amd import draft

    rng = np.random.default_rng(2200 + int(T * 10))
    block, top_p, anchor = 5, 0.95, 4321
    o1, o2, t1, t2 = _weights(rng, "bf16", dev)
    base = rng.normal(0, 2.5, (block, V)).astype(np.float32)
    u = rng.random(block, dtype=np.float32)
    announce(f"draft block T={T} block={block}")
    toks, rows = draft.draft_block(torch.from_numpy(base).to(dev), t1, t2, anchor, T, top_p,
                                   uniforms=torch.from_numpy(u).to(dev))
    toks, rows = toks.cpu().numpy(), rows.cpu().numpy()
    prev = anchor
    p = oracle.make_params(1, temperature=T, top_p=top_p, chain=1)
    for i in range(block):
        lg = oracle.markov_logits(base[i], o1, o2, prev)
        ot, _, orow = oracle.sample(lg, p, u[i:i + 1], want_rows=True)
        assert toks[i] == ot[0], i
        if T == 0:
            assert np.array_equal(rows[i], lg)  # sampling_logprobs returns the logits at T == 0
        else:
            m = np.isfinite(orow[0])
            assert np.array_equal(np.isfinite(rows[i]), m)
            assert np.allclose(np.exp(rows[i][m].astype(np.float64)), np.exp(orow[0][m].astype(np.float64)),
                               rtol=1e-5, atol=1e-12)
        prev = int(ot[0])
    # the DraftResult mirror: Python ints, rows on the device
    d = draft.draft(torch.from_numpy(base).to(dev), t1, t2, anchor, T, top_p, uniforms=torch.from_numpy(u).to(dev))
    assert d.tokens == [int(t) for t in toks]
    assert len(d.logprobs) == block
