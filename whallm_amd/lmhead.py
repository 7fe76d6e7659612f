"""The LM head on MFMA, alone or fused with greedy selection.

The logits the token selection consumes come from the LM head
(runtime/deepseek_v4_ssd/model.py:716 `model.lm_head(output)`, dspark.py:313,
qwen4_exp.py:960-961).  lm_head() computes them (wh_lmhead_logits, bf16
inputs, float32 accumulation); lm_head_greedy() fuses the product with
temperature-0 selection (wh_lmhead_greedy: argmax, lowest index among equal
maxima) so the logits never reach memory; lm_head_sample() takes sample()'s
arguments: temperature 0 without penalties takes the fused greedy kernel,
rows filtered by top-p alone (or not at all) take the product with the
sampler's first step in its epilogue, the rest the product then the sampler.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib as L
from . import sampling as S


def _args(x: torch.Tensor, weight: torch.Tensor) -> L.LmHeadArgs:
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("x and weight must be bfloat16")
    if x.dim() != 2 or weight.dim() != 2 or x.shape[1] != weight.shape[1]:
        raise ValueError("x must be [M, K] and weight [V, K]")
    if not (x.is_contiguous() and weight.is_contiguous()):
        raise ValueError("x and weight must be contiguous")
    L.require_device(x, weight)
    a = L.LmHeadArgs()
    a.x = x.data_ptr()
    a.weight = weight.data_ptr()
    a.M, a.K = x.shape
    a.V = weight.shape[0]
    return a


def lm_head(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """logits [M, V] float32 = x [M, K] @ weight[V, K]^T (bf16 in)."""
    a = _args(x, weight)
    if out is None:
        out = torch.empty(a.M, a.V, dtype=torch.float32, device=x.device)
    if out.dtype != torch.float32 or out.dim() != 2 or out.shape[0] != a.M or out.shape[1] != a.V or out.stride(1) != 1:
        raise ValueError("out must be float32 [M, V] with unit stride in V")
    a.logits_out = out.data_ptr()
    a.logits_stride = out.stride(0) if a.M > 1 else a.V
    L.check(L.lib().wh_lmhead_logits(ctypes.byref(a), ctypes.c_void_p(L.stream_of(x))))
    return out


def lm_head_greedy(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """int32 [M]: per row the lowest index among the largest logits, without
    materialising the logits."""
    a = _args(x, weight)
    tokens = torch.empty(a.M, dtype=torch.int32, device=x.device)
    if a.M == 0:
        return tokens
    ws = L.workspace(x.device, L.lib().wh_lmhead_greedy_workspace_bytes(a.M, a.V))
    a.tokens = tokens.data_ptr()
    a.workspace = ws.data_ptr()
    a.workspace_bytes = ws.numel()
    L.check(L.lib().wh_lmhead_greedy(ctypes.byref(a), ctypes.c_void_p(L.stream_of(x))))
    return tokens


_PENALTIES = ("repetition_penalty", "presence_penalty", "frequency_penalty")


def lm_head_sample(x: torch.Tensor, weight: torch.Tensor, *, temperature: float = 0.0, top_p: float = 1.0,
                   top_k: int = 0, min_p: float = 0.0, chain="mlx", uniforms: torch.Tensor | None = None,
                   generator: torch.Generator | None = None, return_logits: bool = False, **kw):
    """sample(lm_head(x, weight), ...) in one call (wh_lmhead_sample).

    Temperature 0 without penalties or row-wise parameters takes the fused
    greedy kernel (no logits written).  Rows filtered by top-p alone or not
    at all, without penalties, take the fused sampled form: the product also
    emits the sampler's per-slice maxima.  Otherwise the product, then the
    sampler.  Returns int32 tokens [M] (and the float32 logits with
    return_logits)."""
    plain = not any(kw.get(k) for k in _PENALTIES) and not any(
        kw.get(k) is not None for k in ("temperature_rows", "top_p_rows", "min_p_rows", "top_k_rows"))
    if not (temperature > 0.0) and plain and not return_logits and not any(kw.values()):
        return lm_head_greedy(x, weight)
    a = _args(x, weight)
    M, V = a.M, a.V
    dev = x.device
    logits = torch.empty(M, V, dtype=torch.float32, device=dev)
    a.logits_out = logits.data_ptr()
    a.logits_stride = V
    if uniforms is None:
        uniforms = torch.rand(M, device=dev, dtype=torch.float32, generator=generator)
    uniforms = torch.as_tensor(uniforms, dtype=torch.float32, device=dev).reshape(M).contiguous()
    tokens = torch.empty(M, dtype=torch.int32, device=dev)
    sa = L.SampleArgs()
    rows = (S._rows_param(kw.pop("temperature_rows", None), M, torch.float64, dev),
            S._rows_param(kw.pop("top_p_rows", None), M, torch.float64, dev),
            S._rows_param(kw.pop("min_p_rows", None), M, torch.float64, dev),
            S._rows_param(kw.pop("top_k_rows", None), M, torch.int32, dev))
    keep = S._fill_args(sa, logits, L.DTYPE_F32, chain, kw.pop("history", None), kw.pop("history_len", None),
                        temperature, top_p, top_k, min_p, kw.pop("repetition_penalty", 0.0),
                        kw.pop("presence_penalty", 0.0), kw.pop("frequency_penalty", 0.0),
                        kw.pop("repetition_context", 20), kw.pop("presence_context", 20),
                        kw.pop("frequency_context", 20), rows)
    if kw:
        raise TypeError(f"unexpected arguments: {sorted(kw)}")
    sa.uniforms = uniforms.data_ptr()
    sa.tokens = tokens.data_ptr()
    sa.out_mode = L.OUT_LOGPROBS
    ws = L.workspace(dev, L.lib().wh_sample_workspace_bytes(M, V))
    sa.workspace = ws.data_ptr()
    sa.workspace_bytes = ws.numel()
    L.check(L.lib().wh_lmhead_sample(ctypes.byref(a), ctypes.byref(sa), ctypes.c_void_p(L.stream_of(x))))
    del keep
    return (tokens, logits) if return_logits else tokens
