"""The DSpark draft block on the device.

runtime/deepseek_v4_ssd/dspark.py:315-344 (and deepseek_v41/dspark.py:
128-142) draft a block of tokens one position at a time:

    previous = anchor
    for position in range(block_size):
        bias, embedding = markov_head(previous)          # markov_w2 @ w1[previous]
        logprobs = sampling_logprobs(base_logits[:, position] + bias, T, top_p)
        token = argmax(logprobs) if T == 0 else categorical(logprobs)
        ...; previous = token
    tokens = [int(t.item()) for t in token_arrays]       # one host sync per token

Here each position is two launches on the caller's stream -- wh_markov_logits
(which reads `previous` from device memory) and wh_sample's chain
WH_CHAIN_WHALLM writing the token and its sampling_logprobs row -- and the
whole block runs without a host round trip.  draft() synchronises once, to
hand back Python ints as DraftResult does.
"""
from __future__ import annotations

import ctypes
import time
from typing import Optional

import torch

from . import _lib as L
from . import sampling as S
from .dspark import DraftResult


def _weights_dtype(w1: torch.Tensor, w2: torch.Tensor) -> int:
    if w1.dtype != w2.dtype or w1.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("markov_w1 and markov_w2 must both be float32 or both bfloat16")
    if w1.dim() != 2 or w2.dim() != 2 or w1.shape != w2.shape:
        raise ValueError("markov_w1 and markov_w2 must be [V, rank] (markov_w2 as nn.Linear(rank, V).weight)")
    if not (w1.is_contiguous() and w2.is_contiguous()):
        raise ValueError("Markov weights must be contiguous")
    return L.DTYPE_F32 if w1.dtype == torch.float32 else L.DTYPE_BF16


def markov_logits(base_row: torch.Tensor, markov_w1: torch.Tensor, markov_w2: torch.Tensor, prev: torch.Tensor,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """base_row [V] float32 + markov_w2 @ float32(markov_w1[prev]); prev is
    an int32 [1] device tensor (read on the device)."""
    dt = _weights_dtype(markov_w1, markov_w2)
    V, rank = markov_w2.shape
    if base_row.dtype != torch.float32 or base_row.numel() != V or not base_row.is_contiguous():
        raise ValueError("base_row must be a contiguous float32 [V] tensor")
    if prev.dtype != torch.int32 or prev.numel() < 1:
        raise ValueError("prev must be an int32 device tensor")
    L.require_device(base_row, markov_w1, markov_w2, prev)
    if out is None:
        out = torch.empty(V, dtype=torch.float32, device=base_row.device)
    a = L.MarkovArgs()
    a.base = base_row.data_ptr()
    a.embed = markov_w1.data_ptr()
    a.proj = markov_w2.data_ptr()
    a.dtype = dt
    a.V = V
    a.rank = rank
    a.prev = prev.data_ptr()
    a.logits_out = out.data_ptr()
    L.check(L.lib().wh_markov_logits(ctypes.byref(a), ctypes.c_void_p(L.stream_of(base_row))))
    return out


def draft_block(base_logits: torch.Tensor, markov_w1: torch.Tensor, markov_w2: torch.Tensor, anchor,
                temperature: float, top_p: float, uniforms: Optional[torch.Tensor] = None,
                generator: Optional[torch.Generator] = None):
    """Draft len(base_logits) positions on the device.

    base_logits: [block, V] (or [1, block, V]) float32, the draft head's
    logits (dspark.py:313); anchor: the last committed token (int or int32
    device tensor).  Returns (tokens int32 [block], rows float32 [block, V])
    on the device: rows[i] is position i's sampling_logprobs row (at T == 0,
    its logits, as sampling_logprobs returns them).  uniforms [block] drive
    the draws (torch.rand when None)."""
    if base_logits.dim() == 3:
        base_logits = base_logits[0]
    if base_logits.dim() != 2 or base_logits.dtype != torch.float32:
        raise ValueError("base_logits must be float32 [block, V]")
    base_logits = base_logits.contiguous()
    block, V = base_logits.shape
    dev = base_logits.device
    if markov_w2.shape[0] != V:
        raise ValueError("markov weights and base_logits disagree on V")
    tokens = torch.empty(block + 1, dtype=torch.int32, device=dev)
    tokens[0] = torch.as_tensor(anchor, dtype=torch.int32, device=dev).reshape(())
    rows = torch.empty(block, V, dtype=torch.float32, device=dev)
    logits = torch.empty(block, V, dtype=torch.float32, device=dev)
    if uniforms is None:
        uniforms = torch.rand(block, device=dev, dtype=torch.float32, generator=generator)
    u = torch.as_tensor(uniforms, dtype=torch.float32, device=dev).reshape(block).contiguous()
    ws = L.workspace(dev, L.lib().wh_sample_workspace_bytes(1, V))
    stream = ctypes.c_void_p(L.stream_of(base_logits))
    for i in range(block):
        markov_logits(base_logits[i], markov_w1, markov_w2, tokens[i:i + 1], out=logits[i])
        a = L.SampleArgs()
        keep = S._fill_args(a, logits[i:i + 1], L.DTYPE_F32, "whallm", None, None, temperature, top_p, 0, 0.0,
                            0.0, 0.0, 0.0, 20, 20, 20, (None, None, None, None))
        a.uniforms = u[i:i + 1].data_ptr()
        a.tokens = tokens[i + 1:i + 2].data_ptr()
        a.logprobs_out = rows[i].data_ptr()
        a.out_mode = L.OUT_LOGPROBS
        a.workspace = ws.data_ptr()
        a.workspace_bytes = ws.numel()
        L.check(L.lib().wh_sample(ctypes.byref(a), stream))
        del keep
    return tokens[1:], rows


def draft(base_logits: torch.Tensor, markov_w1: torch.Tensor, markov_w2: torch.Tensor, anchor: int,
          temperature: float, top_p: float, uniforms: Optional[torch.Tensor] = None,
          confidence: Optional[list] = None) -> DraftResult:
    """draft_block, then one synchronisation: a DraftResult with Python int
    tokens and the per-position rows (dspark.py:338-344; the confidence head
    belongs to the model and is passed through)."""
    started = time.perf_counter()
    toks, rows = draft_block(base_logits, markov_w1, markov_w2, anchor, temperature, top_p, uniforms)
    tokens = [int(t) for t in toks.tolist()]
    logprobs = [rows[i] for i in range(len(tokens))] if temperature else [torch.empty(0) for _ in tokens]
    conf = list(confidence) if confidence is not None else [1.0] * len(tokens)
    return DraftResult(tokens=tokens, logprobs=logprobs, confidence=conf, seconds=time.perf_counter() - started)
