"""ctypes front end of oracle/wh_oracle.c (test infrastructure only).

The contract functions (sample, verify_logprobs, verify_fused) define the
exact results the HIP kernels must reproduce; the faithful functions replay
mlx_lm / Whallm's float32 op order (runtime/deepseek_v4_ssd/dspark.py:358-375,
857-904 and third-party mlx_lm.sample_utils) for mismatch reporting and as the
timed CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "build", "libwh_oracle.so")

CHAIN_KPM = 0  # mlx_lm make_sampler: top_k -> top_p -> min_p, logprobs * (1/T)
CHAIN_PMK = 1  # Whallm sampling_logprobs: top_p -> min_p -> top_k, logprobs / max(T, 1e-5)

# who_params: temperature, top_p and min_p are the caller's doubles, as the
# reference's Python floats are.
PARAMS_DTYPE = np.dtype(
    [
        ("temperature", np.float64),
        ("top_p", np.float64),
        ("min_p", np.float64),
        ("top_k", np.int32),
        ("repetition_penalty", np.float32),
        ("presence_penalty", np.float32),
        ("frequency_penalty", np.float32),
        ("repetition_context", np.int32),
        ("presence_context", np.int32),
        ("frequency_context", np.int32),
        ("chain", np.int32),
    ]
)
assert PARAMS_DTYPE.itemsize == 56

_lib = None


def build() -> None:
    """Compile oracle/wh_oracle.c with its Makefile (gcc, OpenMP)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i32, i64, f32 = ctypes.c_int, ctypes.c_long, ctypes.c_float
        L.who_exp_fix44.restype = ctypes.c_uint64
        L.who_exp_fix44.argtypes = [f32]
        L.who_exp_fix44_batch.argtypes = [P, P, i64]
        L.who_exp_fix44_batch.restype = None
        for name in ("who_sample_rows", "who_sample_rows_faithful"):
            fn = getattr(L, name)
            fn.restype = i32
            fn.argtypes = [P, i32, i32, i64, P, i64, P, P, P, P, P, P, i32]
        L.who_verify_logprobs.restype = i32
        L.who_verify_logprobs.argtypes = [P, P, P, P, i32, i32, i32, f32, P, P, P, i32]
        L.who_verify_faithful.restype = i32
        L.who_verify_faithful.argtypes = [P, P, P, P, i32, i32, i32, f32, P, P, i32]
        L.who_verify_fused.restype = i32
        L.who_verify_fused.argtypes = [P, P, P, P, i32, i32, i32, f32, P, P, i32]
        L.who_gt_theta_export.restype = i32
        L.who_gt_theta_export.argtypes = [ctypes.c_uint64, f32, ctypes.c_uint64]
        L.who_floor_qz_export.restype = ctypes.c_uint64
        L.who_floor_qz_export.argtypes = [f32, ctypes.c_uint64]
        L.who_reject_fused_export.restype = i32
        L.who_reject_fused_export.argtypes = [f32, f32, ctypes.c_uint64, ctypes.c_uint64]
        L.who_reject_lp_export.restype = i32
        L.who_reject_lp_export.argtypes = [f32, f32, f32]
        L.who_markov_logits.restype = i32
        L.who_markov_logits.argtypes = [P, P, P, i32, i32, i32, i32, P]
        L.who_top_logprobs.restype = i32
        L.who_top_logprobs.argtypes = [P, i32, i32, i64, i32, P, P]
        L.who_penalize_rows.restype = None
        L.who_penalize_rows.argtypes = [P, i32, i32, i64, P, i64, P, P]
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact widening of bfloat16 bit patterns (uint16) to float32."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def make_params(B: int, **kw) -> np.ndarray:
    """Per-row parameter records; keyword values may be scalars or length-B arrays."""
    p = np.zeros(B, dtype=PARAMS_DTYPE)
    p["top_p"] = 1.0
    for k, v in kw.items():
        p[k] = v
    return p


def exp_fix44(d) -> np.ndarray:
    d = np.ascontiguousarray(d, dtype=np.float32)
    out = np.empty(d.shape, dtype=np.uint64)
    lib().who_exp_fix44_batch(_ptr(d), _ptr(out), d.size)
    return out


def _hist_args(hist, hist_len, B):
    if hist is None:
        return None, 0, None
    hist = np.ascontiguousarray(hist, dtype=np.int32)
    if hist.ndim == 1:
        hist = hist[None, :].repeat(B, 0)
    if hist_len is None:
        hist_len = np.full(B, hist.shape[1], dtype=np.int32)
    return hist, hist.shape[1], np.ascontiguousarray(hist_len, dtype=np.int32)


def _sample(fn, logits, params, u, hist=None, hist_len=None, want_rows=False, threads=None):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    if logits.ndim == 1:
        logits = logits[None, :]
    B, V = logits.shape
    params = np.ascontiguousarray(params, dtype=PARAMS_DTYPE)
    assert params.shape == (B,)
    u = np.ascontiguousarray(np.broadcast_to(np.asarray(u, dtype=np.float32), (B,)))
    h, hld, hl = _hist_args(hist, hist_len, B)
    tokens = np.empty(B, dtype=np.int32)
    kept = np.empty(B, dtype=np.int32)
    rows = np.empty((B, V), dtype=np.float32) if want_rows else None
    nthreads = threads or min(8, os.cpu_count() or 1)
    rc = fn(_ptr(logits), B, V, V, _ptr(h), hld, _ptr(hl), _ptr(params), _ptr(u), _ptr(tokens), _ptr(kept),
            _ptr(rows), nthreads)
    if rc != 0:
        raise ValueError(f"oracle rejected the arguments (code {rc})")
    return (tokens, kept, rows) if want_rows else (tokens, kept)


def sample(logits, params, u, hist=None, hist_len=None, want_rows=False, threads=None):
    """Contract sampler: exact token ids the GPU must reproduce."""
    return _sample(lib().who_sample_rows, logits, params, u, hist, hist_len, want_rows, threads)


def sample_faithful(logits, params, u, hist=None, hist_len=None, want_rows=False, threads=None):
    """float32 replay of the reference op order (mismatch reporting, CPU baseline)."""
    return _sample(lib().who_sample_rows_faithful, logits, params, u, hist, hist_len, want_rows, threads)


def penalize(logits, params, hist, hist_len=None):
    logits = np.array(logits, dtype=np.float32, copy=True)
    if logits.ndim == 1:
        logits = logits[None, :]
    B, V = logits.shape
    h, hld, hl = _hist_args(hist, hist_len, B)
    params = np.ascontiguousarray(params, dtype=PARAMS_DTYPE)
    lib().who_penalize_rows(_ptr(logits), B, V, V, _ptr(h), hld, _ptr(hl), _ptr(params))
    return logits


def verify_logprobs(draft_lp, target_lp, draft_tok, u, temperature, want_rows=False, threads=None):
    draft_lp = np.ascontiguousarray(draft_lp, dtype=np.float32)
    target_lp = np.ascontiguousarray(target_lp, dtype=np.float32)
    draft_tok = np.ascontiguousarray(draft_tok, dtype=np.int32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    B, n1, V = target_lp.shape
    n = n1 - 1
    assert draft_lp.shape == (B, n, V) and draft_tok.shape == (B, n) and u.shape == (B, n1)
    acc = np.empty(B, dtype=np.int32)
    tok = np.empty(B, dtype=np.int32)
    rows = np.empty((B, V), dtype=np.float32) if want_rows else None
    rc = lib().who_verify_logprobs(_ptr(draft_lp), _ptr(target_lp), _ptr(draft_tok), _ptr(u), B, n, V,
                                   float(temperature), _ptr(acc), _ptr(tok), _ptr(rows),
                                   threads or min(8, os.cpu_count() or 1))
    if rc != 0:
        raise ValueError(f"oracle rejected the arguments (code {rc})")
    return (acc, tok, rows) if want_rows else (acc, tok)


def verify_faithful(draft_lp, target_lp, draft_tok, u, temperature, threads=None):
    draft_lp = np.ascontiguousarray(draft_lp, dtype=np.float32)
    target_lp = np.ascontiguousarray(target_lp, dtype=np.float32)
    draft_tok = np.ascontiguousarray(draft_tok, dtype=np.int32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    B, n1, V = target_lp.shape
    acc = np.empty(B, dtype=np.int32)
    tok = np.empty(B, dtype=np.int32)
    rc = lib().who_verify_faithful(_ptr(draft_lp), _ptr(target_lp), _ptr(draft_tok), _ptr(u), B, n1 - 1, V,
                                   float(temperature), _ptr(acc), _ptr(tok), threads or min(8, os.cpu_count() or 1))
    if rc != 0:
        raise ValueError(f"oracle rejected the arguments (code {rc})")
    return acc, tok


def verify_fused(target_logits, draft_q, draft_tok, u, temperature, threads=None):
    target_logits = np.ascontiguousarray(target_logits, dtype=np.float32)
    draft_q = np.ascontiguousarray(draft_q, dtype=np.float32)
    draft_tok = np.ascontiguousarray(draft_tok, dtype=np.int32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    B, n1, V = target_logits.shape
    acc = np.empty(B, dtype=np.int32)
    tok = np.empty(B, dtype=np.int32)
    rc = lib().who_verify_fused(_ptr(target_logits), _ptr(draft_q), _ptr(draft_tok), _ptr(u), B, n1 - 1, V,
                                float(temperature), _ptr(acc), _ptr(tok), threads or min(8, os.cpu_count() or 1))
    if rc != 0:
        raise ValueError(f"oracle rejected the arguments (code {rc})")
    return acc, tok


def markov_logits(base_row, w1, w2, prev: int):
    """DSpark draft step logits: base_row + markov_w2 @ float32(markov_w1[prev])
    in the contract's summation order (wh_oracle_ext.c).  w1, w2: [V, rank]
    float32 arrays or bfloat16 bit patterns (uint16)."""
    base_row = np.ascontiguousarray(base_row, dtype=np.float32)
    dtype = 1 if w1.dtype == np.uint16 else 0
    w1 = np.ascontiguousarray(w1)
    w2 = np.ascontiguousarray(w2)
    V, rank = w2.shape
    out = np.empty(V, np.float32)
    rc = lib().who_markov_logits(_ptr(base_row), _ptr(w1), _ptr(w2), dtype, V, rank, int(prev), _ptr(out))
    if rc != 0:
        raise ValueError("oracle rejected the Markov arguments")
    return out


def top_logprobs(logits, n: int):
    """Top-n (ids, logprobs) per row: (value desc, id asc), logprob in float64."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    if logits.ndim == 1:
        logits = logits[None]
    B, V = logits.shape
    ids = np.empty((B, n), np.int32)
    lps = np.empty((B, n), np.float32)
    rc = lib().who_top_logprobs(_ptr(logits), B, V, V, int(n), _ptr(ids), _ptr(lps))
    if rc != 0:
        raise ValueError("oracle rejected the top-logprob arguments")
    return ids, lps


def gt_theta(A: int, theta: float, Z: int) -> bool:
    return bool(lib().who_gt_theta_export(A, theta, Z))


def floor_qz(q: float, Z: int) -> int:
    return int(lib().who_floor_qz_export(q, Z))


def reject_fused(u: float, q: float, Z: int, W: int) -> bool:
    return bool(lib().who_reject_fused_export(u, q, Z, W))


def reject_lp(u: float, g: float, d: float) -> bool:
    return bool(lib().who_reject_lp_export(u, g, d))
