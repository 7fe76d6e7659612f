"""The LM head on MFMA, alone or fused with greedy selection.

The logits the token selection consumes come from the LM head
(runtime/deepseek_v4_ssd/model.py:716 `model.lm_head(output)`, dspark.py:313,
qwen4_exp.py:960-961).  lm_head() computes them (wh_lmhead_logits, bf16
inputs, float32 accumulation); lm_head_greedy() fuses the product with
temperature-0 selection (wh_lmhead_greedy: argmax, lowest index among equal
maxima) so the logits never reach memory; lm_head_sample() takes sample()'s
arguments and uses the fused path where it applies (temperature 0, no
penalties), otherwise lm_head() then sample().
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


def lm_head_sample(x: torch.Tensor, weight: torch.Tensor, **sample_kwargs) -> torch.Tensor:
    """sample(lm_head(x, weight), **sample_kwargs); temperature 0 without
    penalties (and no row-wise parameters) takes the fused greedy kernel."""
    greedy = not (sample_kwargs.get("temperature", 0.0) > 0.0)
    plain = not any(sample_kwargs.get(k) for k in _PENALTIES) and not any(
        sample_kwargs.get(k) is not None for k in ("temperature_rows", "top_p_rows", "min_p_rows", "top_k_rows"))
    extra = sample_kwargs.get("return_logprobs") or sample_kwargs.get("return_kept")
    if greedy and plain and not extra:
        return lm_head_greedy(x, weight)
    return S.sample(lm_head(x, weight), **sample_kwargs)
