"""Top-n logprob output (the OpenAI `logprobs` / `top_logprobs` fields).

runtime/deepseek_v4_ssd/server.py:1110-1111 rejects these fields today; the
value they carry is mlx_lm's per-step `logprobs = logits - logsumexp(logits)`
(the row generate_step hands to the sampler, generation.py:1465-1475), of
which a response returns the chosen token's entry and the n most likely ones.
wh_top_logprobs computes both on the device in one pass over the row.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib as L


def top_logprobs(logits: torch.Tensor, n: int, tokens: Optional[torch.Tensor] = None):
    """Top-n of each row's log-softmax.

    logits: [B, V] (or [V]) float32 / bfloat16 device tensor, unit stride in
    V.  Returns (ids int32 [B, n], logprobs float32 [B, n], token_logprobs
    float32 [B] or None).  Order: logprob descending, lower ids first among
    equal values; logprob = float32(l - logsumexp(row)) with the logsumexp in
    float64.  tokens [B] (int32/int64): also return each row's logprob of
    that token (-inf outside [0, V))."""
    if logits.dim() == 1:
        logits = logits.unsqueeze(0)
    if logits.dim() != 2 or logits.stride(-1) != 1:
        raise ValueError("logits must be [B, V] with unit stride in V")
    if logits.dtype == torch.float32:
        dt = L.DTYPE_F32
    elif logits.dtype == torch.bfloat16:
        dt = L.DTYPE_BF16
    else:
        raise ValueError("logits must be float32 or bfloat16")
    dev = L.require_device(logits, tokens)
    B, V = logits.shape
    n = int(n)
    if not 1 <= n <= min(V, L.MAX_TOP_LOGPROBS):
        raise ValueError(f"n must be in [1, {min(V, L.MAX_TOP_LOGPROBS)}], got {n}")
    ids = torch.empty(B, n, dtype=torch.int32, device=dev)
    lps = torch.empty(B, n, dtype=torch.float32, device=dev)
    tlp = None
    if tokens is not None:
        tokens = tokens.reshape(-1).to(torch.int32).contiguous()
        if tokens.numel() != B:
            raise ValueError(f"tokens must hold one id per row ({B}), got {tokens.numel()}")
        tlp = torch.empty(B, dtype=torch.float32, device=dev)
    if B == 0:
        return ids, lps, tlp
    a = L.TopLogprobsArgs()
    a.logits = logits.data_ptr()
    a.dtype = dt
    a.B = B
    a.V = V
    a.n = n
    a.row_stride = logits.stride(0) if B > 1 else V
    a.token = L.ptr(tokens)
    a.top_ids = ids.data_ptr()
    a.top_logprobs = lps.data_ptr()
    a.token_logprob = L.ptr(tlp)
    ws = L.workspace(dev, L.lib().wh_top_logprobs_workspace_bytes(B, V, n))
    a.workspace = ws.data_ptr()
    a.workspace_bytes = ws.numel()
    L.check(L.lib().wh_top_logprobs(ctypes.byref(a), ctypes.c_void_p(L.stream_of(logits))))
    return ids, lps, tlp
