"""ctypes binding of libwh_sample.so (include/wh_sample.h).

The library is loaded from this package directory; if it is missing the
import fails loudly -- there is no CPU or PyTorch fallback for the product
path.  Tensors cross the boundary as raw device pointers plus the current HIP
stream of their device.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libwh_sample.so")

WH_OK = 0
WH_EINVAL = -1
WH_EHIP = -2
WH_ELIMIT = -3
DTYPE_F32 = 0
DTYPE_BF16 = 1
CHAIN_MLX = 0
CHAIN_WHALLM = 1
OUT_LOGPROBS = 0
OUT_MASKED = 1
MAX_VOCAB = 262144
MAX_TOP_LOGPROBS = 64
LMHEAD_MAX_ROWS = 64
MAX_WINDOW = 4096
NOALLOC_SCRATCH_BYTES = 32 << 20

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_f64 = ctypes.c_double


class SampleArgs(ctypes.Structure):
    _fields_ = [
        ("logits", _p), ("dtype", _i32), ("B", _i32), ("V", _i32), ("chain", _i32), ("row_stride", _i64),
        ("history", _p), ("history_stride", _i64), ("history_len", _p),
        ("uniforms", _p),
        ("temperature", _f64), ("top_p", _f64), ("min_p", _f64), ("top_k", _i32), ("history_share", _i32),
        ("temperature_rows", _p), ("top_p_rows", _p), ("min_p_rows", _p), ("top_k_rows", _p),
        ("repetition_penalty", _f32), ("presence_penalty", _f32), ("frequency_penalty", _f32),
        ("repetition_context", _i32), ("presence_context", _i32), ("frequency_context", _i32),
        ("tokens", _p), ("kept_count", _p), ("logprobs_out", _p), ("out_mode", _i32), ("reserved", _i32),
        ("workspace", _p), ("workspace_bytes", ctypes.c_size_t),
    ]


class VerifyArgs(ctypes.Structure):
    _fields_ = [
        ("B", _i32), ("n", _i32), ("V", _i32), ("temperature", _f32),
        ("target", _p), ("draft", _p), ("draft_tokens", _p), ("uniforms", _p),
        ("accepted", _p), ("token", _p), ("row_out", _p), ("workspace", _p), ("workspace_bytes", ctypes.c_size_t),
    ]


class MarkovArgs(ctypes.Structure):
    _fields_ = [
        ("base", _p), ("embed", _p), ("proj", _p), ("dtype", _i32), ("V", _i32), ("rank", _i32), ("reserved", _i32),
        ("prev", _p), ("logits_out", _p),
    ]


class TopLogprobsArgs(ctypes.Structure):
    _fields_ = [
        ("logits", _p), ("dtype", _i32), ("B", _i32), ("V", _i32), ("n", _i32), ("row_stride", _i64),
        ("token", _p), ("top_ids", _p), ("top_logprobs", _p), ("token_logprob", _p),
        ("workspace", _p), ("workspace_bytes", ctypes.c_size_t),
    ]


class HistoryArgs(ctypes.Structure):
    _fields_ = [
        ("history", _p), ("history_stride", _i64), ("history_len", _p), ("B", _i32), ("capacity", _i32),
        ("keep", _i32), ("m", _i32), ("tokens", _p), ("counts", _p), ("tail", _p),
    ]


class LmHeadArgs(ctypes.Structure):
    _fields_ = [
        ("x", _p), ("weight", _p), ("M", _i32), ("K", _i32), ("V", _i32), ("reserved", _i32),
        ("logits_out", _p), ("logits_stride", _i64), ("tokens", _p), ("workspace", _p),
        ("workspace_bytes", ctypes.c_size_t),
    ]


class WhError(RuntimeError):
    pass


_lib = None


def lib() -> ctypes.CDLL:
    """Load libwh_sample.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m whallm_amd.build` "
                "(there is no CPU fallback for the token-selection path)")
        L = ctypes.CDLL(LIB_PATH)
        L.wh_sample.argtypes = [ctypes.POINTER(SampleArgs), _p]
        L.wh_sample.restype = ctypes.c_int
        L.wh_sample_noalloc.argtypes = [ctypes.POINTER(SampleArgs), _p]
        L.wh_sample_noalloc.restype = ctypes.c_int
        L.wh_apply_penalties.argtypes = [ctypes.POINTER(SampleArgs), _p]
        L.wh_apply_penalties.restype = ctypes.c_int
        L.wh_sample_workspace_bytes.argtypes = [_i32, _i32]
        L.wh_sample_workspace_bytes.restype = ctypes.c_size_t
        L.wh_verify_logprobs.argtypes = [ctypes.POINTER(VerifyArgs), _p]
        L.wh_verify_logprobs.restype = ctypes.c_int
        L.wh_verify_fused.argtypes = [ctypes.POINTER(VerifyArgs), _p]
        L.wh_verify_fused.restype = ctypes.c_int
        L.wh_verify_workspace_bytes.argtypes = [_i32, _i32, _i32]
        L.wh_verify_workspace_bytes.restype = ctypes.c_size_t
        L.wh_markov_logits.argtypes = [ctypes.POINTER(MarkovArgs), _p]
        L.wh_markov_logits.restype = ctypes.c_int
        L.wh_top_logprobs.argtypes = [ctypes.POINTER(TopLogprobsArgs), _p]
        L.wh_top_logprobs.restype = ctypes.c_int
        L.wh_top_logprobs_workspace_bytes.argtypes = [_i32, _i32, _i32]
        L.wh_top_logprobs_workspace_bytes.restype = ctypes.c_size_t
        L.wh_history_append.argtypes = [ctypes.POINTER(HistoryArgs), _p]
        L.wh_history_append.restype = ctypes.c_int
        L.wh_lmhead_logits.argtypes = [ctypes.POINTER(LmHeadArgs), _p]
        L.wh_lmhead_logits.restype = ctypes.c_int
        L.wh_lmhead_greedy.argtypes = [ctypes.POINTER(LmHeadArgs), _p]
        L.wh_lmhead_greedy.restype = ctypes.c_int
        L.wh_lmhead_sample.argtypes = [ctypes.POINTER(LmHeadArgs), ctypes.POINTER(SampleArgs), _p]
        L.wh_lmhead_sample.restype = ctypes.c_int
        L.wh_lmhead_greedy_workspace_bytes.argtypes = [_i32, _i32]
        L.wh_lmhead_greedy_workspace_bytes.restype = ctypes.c_size_t
        L.wh_verify_force_exact.argtypes = [ctypes.c_int]
        L.wh_verify_force_exact.restype = ctypes.c_int
        L.wh_exp_fix44.argtypes = [_p, _p, _i64, _p]
        L.wh_exp_fix44.restype = ctypes.c_int
        L.wh_last_error.argtypes = []
        L.wh_last_error.restype = ctypes.c_char_p
        L.wh_version.argtypes = []
        L.wh_version.restype = ctypes.c_char_p
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc == WH_OK:
        return
    msg = lib().wh_last_error().decode(errors="replace")
    if rc in (WH_EINVAL, WH_ELIMIT):
        raise ValueError(msg)
    raise WhError(f"libwh_sample error {rc}: {msg}")


def stream_of(t: torch.Tensor) -> int:
    """Raw hipStream_t of the current torch stream on t's device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t) -> int | None:
    if t is None:
        return None
    return t.data_ptr()


def require_device(*tensors) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
            raise ValueError("whallm_amd kernels take HIP device tensors (device='cuda')")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all tensors must be on the same device")
    return dev


_workspaces: dict = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Cached device workspace per device and stream (grown on demand)."""
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
        _workspaces[key] = buf
    return buf
