"""Drop-in mirror of Whallm's token-selection helpers in
runtime/deepseek_v4_ssd/dspark.py: DraftResult (179-185),
sampling_logprobs (358-375), _verify (857-898) and _sample (901-904).

Same names, arguments and return types, over torch tensors on a HIP device;
_sample and _verify return Python ints (synchronising, as the reference's
.item() calls do).  Each draw consumes a uniform in [0, 1): pass `uniform=` /
`uniforms=` for parity runs, otherwise torch.rand supplies them.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib as L
from . import sampling as S


@dataclass(frozen=True)
class DraftResult:
    tokens: list
    logprobs: list
    confidence: list
    seconds: float


def sampling_logprobs(logits: torch.Tensor, temperature: float, top_p: float, top_k: int = 0,
                      min_p: float = 0.0) -> torch.Tensor:
    """T == 0: logits unchanged.  Otherwise normalise, top_p -> min_p ->
    top_k, divide by max(T, 1e-5) and renormalise; returns the full row(s)."""
    if temperature == 0:
        return logits
    out = S.filter_rows(logits, chain="whallm", temperature=temperature, top_p=top_p, top_k=top_k, min_p=min_p,
                        out_mode=L.OUT_LOGPROBS)
    return out.reshape(logits.shape)


def _sample(logprobs: torch.Tensor, temperature: float, uniform: Optional[float] = None) -> int:
    """T == 0: argmax; otherwise a categorical draw from the (already
    tempered) logprob row."""
    row = logprobs.reshape(1, -1)
    if temperature == 0:
        tok = S.sample(row, temperature=0.0, chain="whallm")
    else:
        u = None if uniform is None else torch.tensor([uniform], dtype=torch.float32, device=row.device)
        tok = S.sample(row, temperature=1.0, chain="whallm", uniforms=u)
    return int(tok[0].item())


def _verify(draft: DraftResult, target_logprobs: torch.Tensor, temperature: float,
            uniforms: Optional[torch.Tensor] = None):
    """Greedy prefix match (T == 0) or the ratio test u > min(1, p/q) with
    residual max(p - q, 0) resampling; returns (accepted, token, row)."""
    n = len(draft.tokens)
    target = target_logprobs[: n + 1].reshape(1, n + 1, -1)
    dev = target.device
    toks = torch.tensor([draft.tokens], dtype=torch.int32, device=dev).reshape(1, n)
    if temperature == 0 or n == 0:
        dl = None
    else:
        dl = torch.stack([d.reshape(-1) for d in draft.logprobs[:n]]).reshape(1, n, -1)
    if uniforms is not None:
        uniforms = torch.as_tensor(uniforms, dtype=torch.float32, device=dev).reshape(1, n + 1)
    acc, tok, row = S.verify_logprobs(target, dl, toks, temperature, uniforms=uniforms, return_row=True)
    return int(acc[0].item()), int(tok[0].item()), row[0]
