"""MTP verification rows: the per-position target distributions Whallm's
Qwen MTP loop builds before it verifies a draft block.

runtime/deepseek_v4_ssd/qwen4_exp.py:946-958 defines
adjusted_logprobs(logits, tokens): the logits processors (penalties) over
`tokens`, then sampling_logprobs(logits, T, top_p, top_k, min_p) (chain B).
qwen4_exp.py:1083-1092 stacks it over the n+1 verified positions, position i
penalised over sampling_tokens + draft_tokens[:i], and hands the stack to
_verify (qwen4_exp.py:1099).

Here the n+1 rows of a batch entry share one device history row that holds
the committed ids followed by the drafts; row i reads it with length
committed + i (wh_sample_args.history_share = n + 1).  One wh_sample launch
builds every row of every entry; nothing synchronises with the host.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib as L
from . import sampling as S


def adjusted_logprobs_rows(verified_logits: torch.Tensor, history: torch.Tensor, history_len: torch.Tensor,
                           draft_tokens: torch.Tensor, *, temperature: float, top_p: float, top_k: int = 0,
                           min_p: float = 0.0, repetition_penalty: float = 0.0, presence_penalty: float = 0.0,
                           frequency_penalty: float = 0.0, repetition_context: int = 20, presence_context: int = 20,
                           frequency_context: int = 20) -> torch.Tensor:
    """Target rows [B, n+1, V] (float32 sampling_logprobs rows) for B batch
    entries of n drafts.

    verified_logits: [B, n+1, V] float32 or bfloat16, the target model's
    logits at [anchor, *drafts]; history: int32 [B, Hcap] device buffer whose
    first history_len[b] ids are entry b's committed ids (sampling_tokens);
    draft_tokens: int32 [B, n].  The drafts are written into history at
    positions history_len[b] .. history_len[b] + n - 1 (Hcap must leave room
    for them: positions past the buffer are clamped to its last column).
    Penalty contexts are windows over the end of each row's history, as in
    mlx_lm's processors (context 0: the whole history).
    """
    if verified_logits.dim() == 2:
        verified_logits = verified_logits.unsqueeze(0)
    if verified_logits.dim() != 3:
        raise ValueError("verified_logits must be [n+1, V] or [B, n+1, V]")
    B, n1, V = verified_logits.shape
    n = n1 - 1
    dev = verified_logits.device
    if history.dtype != torch.int32 or history.dim() != 2 or history.shape[0] != B or not history.is_contiguous():
        raise ValueError("history must be a contiguous int32 [B, Hcap] device buffer")
    if history_len.dtype != torch.int32 or tuple(history_len.shape) != (B,):
        raise ValueError("history_len must be an int32 [B] device tensor")
    draft_tokens = torch.as_tensor(draft_tokens, device=dev)
    if draft_tokens.dtype != torch.int32 or tuple(draft_tokens.shape) != (B, n):
        raise ValueError("draft_tokens must be an int32 [B, n] tensor")
    L.require_device(verified_logits, history, history_len, draft_tokens)
    Hcap = history.shape[1]
    if n > 0:
        pos = (history_len.long().unsqueeze(1) + torch.arange(n, device=dev)).clamp_(0, Hcap - 1)
        history.scatter_(1, pos, draft_tokens)
    lens = (history_len.unsqueeze(1) + torch.arange(n1, device=dev, dtype=torch.int32)).reshape(-1).contiguous()
    rows, dt = S._as_rows(verified_logits.reshape(B * n1, V))
    out = torch.empty(B * n1, V, dtype=torch.float32, device=dev)
    a = L.SampleArgs()
    keep = S._fill_args(a, rows, dt, "whallm", None, None, temperature, top_p, top_k, min_p, repetition_penalty,
                        presence_penalty, frequency_penalty, repetition_context, presence_context, frequency_context,
                        (None, None, None, None))
    a.history = history.data_ptr()
    a.history_stride = Hcap
    a.history_len = lens.data_ptr()
    a.history_share = n1
    a.logprobs_out = out.data_ptr()
    a.out_mode = L.OUT_LOGPROBS
    ws = L.workspace(dev, L.lib().wh_sample_workspace_bytes(B * n1, V))
    a.workspace = ws.data_ptr()
    a.workspace_bytes = ws.numel()
    L.check(L.lib().wh_sample(ctypes.byref(a), ctypes.c_void_p(L.stream_of(rows))))
    del keep
    return out.reshape(B, n1, V)


def verify_block(verified_logits: torch.Tensor, history: torch.Tensor, history_len: torch.Tensor,
                 draft_tokens: torch.Tensor, draft_logprobs: torch.Tensor | None, *, temperature: float,
                 top_p: float, top_k: int = 0, min_p: float = 0.0, uniforms: torch.Tensor | None = None,
                 **penalties):
    """qwen4_exp.py:1083-1099 for B entries: the adjusted target rows, then
    _verify against the drafts' logprob rows [B, n, V].  Returns
    (accepted [B], token [B], target rows [B, n+1, V])."""
    rows = adjusted_logprobs_rows(verified_logits, history, history_len, draft_tokens, temperature=temperature,
                                  top_p=top_p, top_k=top_k, min_p=min_p, **penalties)
    # at T == 0 sampling_logprobs returns the (penalised) logits themselves;
    # the greedy verify needs only their argmax
    acc, tok = S.verify_logprobs(rows, draft_logprobs, draft_tokens, temperature, uniforms=uniforms)
    return acc, tok, rows
