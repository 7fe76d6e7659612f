"""Seeded synthetic inputs for the five token-selection workloads.

numpy PCG64, seed 20261201 + workload index; uniforms come from a separate
stream (seed + 1000).  Zipf(1.1) history ranks are truncated to [1, V] by
rejection and mapped through a fixed seeded permutation of the vocabulary.
bf16 logits are produced by round-to-nearest-even from float32 and returned
as raw uint16 bit patterns (plus their exact float32 widening).

Workloads (index: description):
  1  plain decode, B=1, V=129,280 fp32 N(0, 2.5^2), 20 ids boosted +8,
     repetition 1.1 over 256 uniform history ids, T 0.7, top-k 50,
     top-p 0.95, mlx_lm chain (k -> p -> min-p).
  2  plain decode, B=64, V=151,936 bf16 N(0, 3^2), 2,048 Zipf history ids
     per row, presence 0.5 + frequency 0.3, T 1.0, top-p 0.9, min-p 0.05,
     mlx_lm chain.
  3  speculative verify, B=16, n=8, V=129,280 fp32 target logits
     N(0, 2.5^2) [16, 9, V]; draft logits = target[:, :8] + N(0, 0.5^2),
     q = softmax(draft / 0.8); draft ids drawn from q; T 0.8; u [16, 9].
  4  B=256, V=129,280 fp32 3 * Student-t(3); per-row top-k log-uniform in
     [1, 1024] (k = 1 is greedy); T 0.9; no penalties; mlx_lm chain.
  5  MTP rows, 128 x V=151,936 bf16 on a 0.125 grid from N(0, 2^2),
     4,096 Zipf history ids per row, repetition 1.05 + presence 0.4 +
     frequency 0.2, T 0.6, top-k 20, top-p 0.8, min-p 0.02, Whallm chain
     (p -> min-p -> k); dense ties at both cutoffs.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

SEED0 = 20261201
V_DSV4 = 129_280
V_QWEN = 151_936


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = (b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def zipf_ids(rng: np.random.Generator, a: float, size, V: int, perm: np.ndarray) -> np.ndarray:
    n = int(np.prod(size))
    out = np.empty(n, dtype=np.int64)
    filled = 0
    while filled < n:
        z = rng.zipf(a, size=2 * (n - filled) + 16)
        z = z[z <= V]
        take = min(len(z), n - filled)
        out[filled:filled + take] = z[:take]
        filled += take
    return perm[out - 1].astype(np.int32).reshape(size)


@dataclass
class SampleWorkload:
    name: str
    B: int
    V: int
    dtype: str                 # "f32" or "bf16"
    logits_f32: np.ndarray     # exact float32 values [B, V]
    logits_bits: np.ndarray | None  # bf16 bit patterns when dtype == "bf16"
    history: np.ndarray | None
    history_len: np.ndarray | None
    uniforms: np.ndarray
    params: dict = field(default_factory=dict)
    top_k_rows: np.ndarray | None = None

    def bytes_per_call(self) -> int:
        """Algorithmic bytes: every input read once, every output written once."""
        elem = 4 if self.dtype == "f32" else 2
        b = self.B * self.V * elem + self.B * 4 + self.B * 4
        if self.history is not None:
            b += self.history.size * 4
        if self.top_k_rows is not None:
            b += self.B * 4
        return b


@dataclass
class VerifyWorkload:
    name: str
    B: int
    n: int
    V: int
    target_logits: np.ndarray  # [B, n+1, V] f32
    draft_q: np.ndarray        # [B, n, V] f32
    draft_tokens: np.ndarray   # [B, n] int32
    uniforms: np.ndarray       # [B, n+1]
    temperature: float

    def bytes_per_call(self) -> int:
        """Algorithmic bytes: target logits and draft probabilities of every
        position, draft ids and uniforms read once; accepted count and token
        written once."""
        B, n, V = self.B, self.n, self.V
        return B * (n + 1) * V * 4 + B * n * V * 4 + B * n * 4 + B * (n + 1) * 4 + B * 8

    def must_read_bytes(self, accepted) -> int:
        """Bytes a verifier that stops at each entry's first rejection must
        move: every target row (each position's normaliser), the draft
        probability q(t_j) of every tested draft, the whole q row at a
        rejection (the residual), ids, uniforms and outputs."""
        B, n, V = self.B, self.n, self.V
        rejected = int(sum(1 for a in accepted if a < n))
        tested = int(sum(min(int(a) + 1, n) for a in accepted))
        return B * (n + 1) * V * 4 + tested * 4 + rejected * V * 4 + B * n * 4 + B * (n + 1) * 4 + B * 8


def _rngs(idx: int):
    return np.random.Generator(np.random.PCG64(SEED0 + idx)), np.random.Generator(np.random.PCG64(SEED0 + idx + 1000))


def workload1(B: int = 1, V: int = V_DSV4) -> SampleWorkload:
    rng, urng = _rngs(1)
    x = rng.normal(0.0, 2.5, (B, V)).astype(np.float32)
    for b in range(B):
        ids = rng.choice(V, size=20, replace=False)
        x[b, ids] += np.float32(8.0)
    hist = rng.integers(0, V, (B, 256)).astype(np.int32)
    u = urng.random(B, dtype=np.float32)
    return SampleWorkload("plain-decode B=%d V=%d fp32 k50 p0.95 rep1.1" % (B, V), B, V, "f32", x, None, hist,
                          np.full(B, 256, np.int32), u,
                          dict(temperature=0.7, top_k=50, top_p=0.95, min_p=0.0, repetition_penalty=1.1,
                               repetition_context=256, chain="mlx"))


def workload2(B: int = 64, V: int = V_QWEN, H: int = 2048) -> SampleWorkload:
    rng, urng = _rngs(2)
    x = rng.normal(0.0, 3.0, (B, V)).astype(np.float32)
    bits = f32_to_bf16_bits(x)
    perm = rng.permutation(V)
    hist = zipf_ids(rng, 1.1, (B, H), V, perm)
    u = urng.random(B, dtype=np.float32)
    return SampleWorkload("plain-decode B=%d V=%d bf16 p0.9 minp0.05 pres0.5 freq0.3 H=%d" % (B, V, H), B, V, "bf16",
                          bf16_bits_to_f32(bits), bits, hist, np.full(B, H, np.int32), u,
                          dict(temperature=1.0, top_k=0, top_p=0.9, min_p=0.05, presence_penalty=0.5,
                               frequency_penalty=0.3, presence_context=H, frequency_context=H, chain="mlx"))


def workload3(B: int = 16, n: int = 8, V: int = V_DSV4, T: float = 0.8) -> VerifyWorkload:
    rng, urng = _rngs(3)
    tgt = rng.normal(0.0, 2.5, (B, n + 1, V)).astype(np.float32)
    dl = tgt[:, :n] + rng.normal(0.0, 0.5, (B, n, V)).astype(np.float32)
    z = dl.astype(np.float64) / T
    z -= z.max(axis=-1, keepdims=True)
    q = np.exp(z)
    q /= q.sum(axis=-1, keepdims=True)
    toks = np.empty((B, n), np.int32)
    cdf = np.cumsum(q, axis=-1)
    r = rng.random((B, n))
    for b in range(B):
        for j in range(n):
            toks[b, j] = min(int(np.searchsorted(cdf[b, j], r[b, j] * cdf[b, j, -1], side="right")), V - 1)
    u = urng.random((B, n + 1), dtype=np.float32)
    return VerifyWorkload("verify B=%d n=%d V=%d fp32 T%.1f" % (B, n, V, T), B, n, V, tgt, q.astype(np.float32),
                          toks, u, T)


def workload4(B: int = 256, V: int = V_DSV4) -> SampleWorkload:
    rng, urng = _rngs(4)
    x = (3.0 * rng.standard_t(3, (B, V))).astype(np.float32)
    k = np.rint(np.exp(rng.uniform(0.0, np.log(1024.0), B))).astype(np.int32)
    k = np.clip(k, 1, 1024)
    u = urng.random(B, dtype=np.float32)
    return SampleWorkload("top-k B=%d V=%d fp32 t3 k in [1,1024]" % (B, V), B, V, "f32", x, None, None, None, u,
                          dict(temperature=0.9, top_k=0, top_p=1.0, min_p=0.0, chain="mlx"), top_k_rows=k)


def workload5(B: int = 128, V: int = V_QWEN, H: int = 4096) -> SampleWorkload:
    rng, urng = _rngs(5)
    x = (np.round(rng.normal(0.0, 2.0, (B, V)) / 0.125) * 0.125).astype(np.float32)
    bits = f32_to_bf16_bits(x)
    perm = rng.permutation(V)
    hist = zipf_ids(rng, 1.1, (B, H), V, perm)
    u = urng.random(B, dtype=np.float32)
    return SampleWorkload("mtp B=%d V=%d bf16 grid0.125 k20 p0.8 minp0.02 rep1.05 pres0.4 freq0.2 H=%d" % (B, V, H),
                          B, V, "bf16", bf16_bits_to_f32(bits), bits, hist, np.full(B, H, np.int32), u,
                          dict(temperature=0.6, top_k=20, top_p=0.8, min_p=0.02, repetition_penalty=1.05,
                               presence_penalty=0.4, frequency_penalty=0.2, repetition_context=H,
                               presence_context=H, frequency_context=H, chain="whallm"))


SAMPLE_WORKLOADS = {1: workload1, 2: workload2, 4: workload4, 5: workload5}


def oracle_params(w: SampleWorkload, make_params):
    """Per-row oracle parameter records for a sample workload."""
    p = w.params
    kw = dict(temperature=p.get("temperature", 0.0), top_p=p.get("top_p", 1.0), min_p=p.get("min_p", 0.0),
              repetition_penalty=p.get("repetition_penalty", 0.0), presence_penalty=p.get("presence_penalty", 0.0),
              frequency_penalty=p.get("frequency_penalty", 0.0),
              repetition_context=p.get("repetition_context", 20), presence_context=p.get("presence_context", 20),
              frequency_context=p.get("frequency_context", 20), chain=0 if p.get("chain", "mlx") == "mlx" else 1)
    kw["top_k"] = w.top_k_rows if w.top_k_rows is not None else p.get("top_k", 0)
    return make_params(w.B, **kw)
