"""Drop-in mirror of the mlx_lm.sample_utils names Whallm uses.

Whallm builds its plain-decode sampler and processors here:
runtime/deepseek_v4_ssd/generation.py:19 imports make_sampler and
make_logits_processors, generation.py:1280-1293 calls them, and
runtime/deepseek_v4_ssd/dspark.py:14 imports apply_top_k / apply_top_p /
apply_min_p.  The names, argument meanings and ValueError behaviour follow
mlx_lm (third party, mlx-lm @ 5c10538); the arithmetic runs in
libwh_sample.so on the GPU.  Tensors are torch tensors on a HIP device
instead of mx.array.

Randomness: mlx_lm draws from MLX's global PRNG.  Here every draw consumes a
uniform in [0, 1): pass `uniforms=` for reproducible parity, otherwise one
is drawn with torch.rand on the logits' device (seed with
torch.manual_seed, the analogue of mx.random.seed).
"""
from __future__ import annotations

from typing import Callable, Dict, List, Optional

import torch

from . import _lib as L
from . import sampling as S


class Sampler:
    """The callable make_sampler returns: sampler(logprobs) -> token ids."""

    def __init__(self, temp: float, top_p: float, min_p: float, top_k: int):
        self.temp = float(temp)
        self.top_p = float(top_p)
        self.min_p = float(min_p)
        self.top_k = int(top_k)

    def __call__(self, logprobs: torch.Tensor, uniforms: Optional[torch.Tensor] = None,
                 generator: Optional[torch.Generator] = None) -> torch.Tensor:
        squeeze = logprobs.dim() == 1
        tok = S.sample(logprobs, temperature=self.temp, top_p=self.top_p, top_k=self.top_k, min_p=self.min_p,
                       chain="mlx", uniforms=uniforms, generator=generator)
        return tok[0] if squeeze else tok

    def __repr__(self) -> str:
        return f"Sampler(temp={self.temp}, top_p={self.top_p}, min_p={self.min_p}, top_k={self.top_k})"


def make_sampler(temp: float = 0.0, top_p: float = 0.0, min_p: float = 0.0, min_tokens_to_keep: int = 1,
                 top_k: int = 0, xtc_probability: float = 0.0, xtc_threshold: float = 0.0,
                 xtc_special_tokens: List[int] = []) -> Callable[..., torch.Tensor]:
    """temp == 0 -> argmax; otherwise top_k (if > 0) -> top_p (if 0 < p < 1)
    -> min_p (if != 0) on the logprobs, then categorical(logprobs * (1/temp))."""
    if min_tokens_to_keep != 1:
        raise NotImplementedError("min_tokens_to_keep != 1 is not supported (Whallm always uses 1)")
    if xtc_probability > 0.0:
        raise NotImplementedError("XTC sampling is not part of Whallm's sampler")
    if not (0.0 <= float(min_p) <= 1.0):
        raise ValueError(f"`min_p` has to be a float in the [0, 1] interval, but is {min_p}")
    return Sampler(temp, top_p, min_p, top_k)


class _Penalty:
    """One logits processor: processor(tokens, logits) -> logits (in place)."""

    def __init__(self, kind: str, penalty: float, context_size: Optional[int]):
        self.kind = kind
        self.penalty = float(penalty)
        self.context_size = 0 if context_size is None else int(context_size)

    def __call__(self, tokens, logits: torch.Tensor) -> torch.Tensor:
        tokens = torch.as_tensor(tokens, device=logits.device)
        if tokens.numel() == 0:
            return logits
        kw = {"repetition_penalty": 0.0, "presence_penalty": 0.0, "frequency_penalty": 0.0}
        kw[self.kind + "_penalty"] = self.penalty
        ctx = {self.kind + "_context": self.context_size}
        B = logits.shape[0] if logits.dim() == 2 else 1
        hist = tokens if tokens.dim() == 2 else tokens.reshape(1, -1).expand(B, -1)
        return S.apply_penalties(logits, hist, **kw, **ctx)


def make_repetition_penalty(penalty: float, context_size: int = 20):
    if penalty < 0 or not isinstance(penalty, (int, float)):
        raise ValueError(f"penalty must be a non-negative float, got {penalty}")
    return _Penalty("repetition", penalty, context_size)


def make_presence_penalty(penalty: float, context_size: int = 20):
    return _Penalty("presence", penalty, context_size)


def make_frequency_penalty(penalty: float, context_size: int = 20):
    return _Penalty("frequency", penalty, context_size)


def make_logits_processors(logit_bias: Optional[Dict[int, float]] = None,
                           repetition_penalty: Optional[float] = None, repetition_context_size: Optional[int] = 20,
                           presence_penalty: Optional[float] = None, presence_context_size: Optional[int] = 20,
                           frequency_penalty: Optional[float] = None, frequency_context_size: Optional[int] = 20):
    """Processors in mlx_lm's append order: repetition, presence, frequency."""
    if logit_bias:
        raise NotImplementedError("logit_bias is not used by Whallm and is not implemented")
    procs = []
    if repetition_penalty and repetition_penalty != 0.0:
        procs.append(make_repetition_penalty(repetition_penalty, repetition_context_size))
    if presence_penalty and presence_penalty != 0.0:
        procs.append(make_presence_penalty(presence_penalty, presence_context_size))
    if frequency_penalty and frequency_penalty != 0.0:
        procs.append(make_frequency_penalty(frequency_penalty, frequency_context_size))
    return procs


def apply_top_k(logprobs: torch.Tensor, top_k: int) -> torch.Tensor:
    """Keep the top_k largest entries (ties: lower id first), others -inf."""
    V = logprobs.shape[-1]
    if not isinstance(top_k, int) or not (0 < top_k < V):
        raise ValueError(f"`top_k` has to be an integer in the (0, {V}] interval, but is {top_k}.")
    out = S.filter_rows(logprobs, top_k=top_k, out_mode=L.OUT_MASKED)
    return out.reshape(logprobs.shape)


def apply_top_p(logprobs: torch.Tensor, top_p: float) -> torch.Tensor:
    """Nucleus filter on a normalised logprob row: keep i iff the ascending
    cumulative probability at i exceeds 1 - top_p."""
    out = S.filter_rows(logprobs, top_p=top_p, out_mode=L.OUT_MASKED)
    return out.reshape(logprobs.shape)


def apply_min_p(logprobs: torch.Tensor, min_p: float, min_tokens_to_keep: int = 1) -> torch.Tensor:
    """Keep i iff logprob_i >= max + ln(min_p)."""
    if not (0 <= min_p <= 1.0):
        raise ValueError(f"`min_p` has to be a float in the [0, 1] interval, but is {min_p}")
    if not isinstance(min_tokens_to_keep, int) or (min_tokens_to_keep < 1):
        raise ValueError(f"`min_tokens_to_keep` has to be a positive integer, but is {min_tokens_to_keep}")
    if min_tokens_to_keep != 1:
        raise NotImplementedError("min_tokens_to_keep != 1 is not supported")
    if min_p == 0:
        return logprobs.float().clone()
    out = S.filter_rows(logprobs, min_p=min_p, out_mode=L.OUT_MASKED)
    return out.reshape(logprobs.shape)


def categorical_sampling(logits: torch.Tensor, temp: float, uniforms: Optional[torch.Tensor] = None) -> torch.Tensor:
    """categorical(logits * (1/temp)) via the inverse CDF of a uniform."""
    squeeze = logits.dim() == 1
    tok = S.sample(logits, temperature=temp, chain="mlx", uniforms=uniforms)
    return tok[0] if squeeze else tok
