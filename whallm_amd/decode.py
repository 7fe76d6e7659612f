"""Decode-step glue: device-resident history and the per-token selection.

The reference wires token selection into mlx_lm's loop:
runtime/deepseek_v4_ssd/generation.py:1279-1293 builds
`sampler = make_sampler(temp, top_p, top_k, min_p)` and
`logits_processors = make_logits_processors(presence_penalty,
repetition_penalty)` (each only when it differs from its neutral value), and
generation.py:1465-1475 hands both to `stream_generate`, whose generate_step
does per token

    tokens = concat([tokens, y])                     # the history, host side
    for processor in logits_processors: logits = processor(tokens, logits)
    logprobs = logits - logsumexp(logits)
    y = sampler(logprobs); yield y.item(), logprobs

Here the history is a device buffer (DecodeState, extended by
wh_history_append), TokenSelector is the sampler and the processors as one
wh_sample launch over that buffer, and generate() is the loop.  A step is two
launches (select, append) and no host round trip; generate() synchronises
once per step to yield Python ints, as generate_step's `.item()` does.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Callable, Iterator, Optional, Sequence

import torch

from . import _lib as L
from . import sampling as S
from .logprobs import top_logprobs as _top_logprobs


@dataclass(frozen=True)
class GenerationOptions:
    """The sampling fields of the reference's per-request options
    (runtime/deepseek_v4_ssd/generation.py:109-118), same names and
    defaults: temperature 0.2, top-p 0.98, no top-k or min-p, presence 0,
    repetition 1."""

    max_tokens: int = 272_000
    temperature: float = 0.2
    top_p: float = 0.98
    top_k: int = 0
    min_p: float = 0.0
    presence_penalty: float = 0.0
    repetition_penalty: float = 1.0


class DecodeState:
    """Token histories of B sequences on the device: int32 [B, capacity]
    and lengths [B], in the layout wh_sample reads.  A full row keeps its last
    `keep` ids (keep must cover every penalty context in use); keep=None
    means never compact, and an append that could overflow raises."""

    def __init__(self, B: int, capacity: int, keep: Optional[int], device, max_append: int = 1):
        if keep is not None and not 0 <= keep <= 4096:
            raise ValueError("keep must be in [0, 4096]")
        if keep is not None and keep + max_append + 1 > capacity:
            raise ValueError("capacity must exceed keep + the ids one append adds")
        self.B, self.capacity, self.keep = B, capacity, keep
        self.device = torch.device(device)
        self.history = torch.zeros(B, capacity, dtype=torch.int32, device=self.device)
        self.history_len = torch.zeros(B, dtype=torch.int32, device=self.device)
        self._bound = 0  # host-side upper bound on any row's length (keep=None)

    @classmethod
    def from_prompts(cls, prompts: Sequence[Sequence[int]], capacity: int, keep: Optional[int], device,
                     max_append: int = 1) -> "DecodeState":
        """Seed each row with its prompt's last `keep` ids (all of them for
        keep=None) -- the history generate_step starts from."""
        st = cls(len(prompts), capacity, keep, device, max_append)
        rows = [list(p)[-keep:] if keep else list(p) for p in prompts] if keep != 0 else [[] for _ in prompts]
        longest = max((len(r) for r in rows), default=0)
        if longest > capacity:
            raise ValueError(f"a prompt ({longest} ids) does not fit the history capacity ({capacity})")
        host = torch.zeros(st.B, capacity, dtype=torch.int32)
        for b, r in enumerate(rows):
            if r:
                host[b, :len(r)] = torch.tensor(r, dtype=torch.int32)
        st.history.copy_(host)
        st.history_len.copy_(torch.tensor([len(r) for r in rows], dtype=torch.int32))
        st._bound = longest
        return st

    def append(self, tokens: torch.Tensor, counts: Optional[torch.Tensor] = None,
               tail: Optional[torch.Tensor] = None) -> None:
        """Row b gets tokens[b, :counts[b]] (all of tokens[b] without counts),
        then tail[b]: for MTP, the drafts with the accepted counts and the
        verifier's next token."""
        tok = tokens.reshape(self.B, -1) if tokens.numel() else tokens.reshape(self.B, 0)
        m = tok.shape[1]
        if self.keep is None and self._bound + m + (tail is not None) > self.capacity:
            raise ValueError("history capacity exhausted (keep=None never drops ids)")
        if self.keep is not None and self.keep + m + (tail is not None) > self.capacity:
            raise ValueError("capacity must exceed keep + the ids one append adds")
        tok = tok.to(torch.int32).contiguous()
        cnt = None if counts is None else counts.reshape(self.B).to(torch.int32).contiguous()
        tl = None if tail is None else tail.reshape(self.B).to(torch.int32).contiguous()
        L.require_device(self.history, tok, cnt, tl)
        a = L.HistoryArgs()
        a.history = self.history.data_ptr()
        a.history_stride = self.capacity
        a.history_len = self.history_len.data_ptr()
        a.B = self.B
        a.capacity = self.capacity
        a.keep = 0 if self.keep is None else self.keep  # keep=None: the bound above means no row fills
        a.m = m
        a.tokens = tok.data_ptr() if m else None
        a.counts = L.ptr(cnt)
        a.tail = L.ptr(tl)
        L.check(L.lib().wh_history_append(ctypes.byref(a), ctypes.c_void_p(L.stream_of(self.history))))
        self._bound += m + (tail is not None)

    def rows(self) -> list:
        """The histories as Python lists (synchronises; for inspection)."""
        h, n = self.history.cpu(), self.history_len.cpu()
        return [h[b, :int(n[b])].tolist() for b in range(self.B)]


class TokenSelector:
    """make_sampler(temp, top_p, top_k, min_p) + make_logits_processors(...)
    as one device call over a DecodeState (generation.py:1279-1293).

    Penalties follow generation.py:1286-1291: a processor is active only when
    it differs from its neutral value (repetition 1.0, presence and frequency
    0).  chain "mlx" is make_sampler's order; "whallm" is sampling_logprobs'.
    With top_logprobs = n, each call also returns the n most likely entries of
    the penalised row's log-softmax (generate_step's `logprobs`) and the
    chosen token's; tokens are the same either way."""

    def __init__(self, *, temperature: float = 0.0, top_p: float = 1.0, top_k: int = 0, min_p: float = 0.0,
                 repetition_penalty: float = 1.0, presence_penalty: float = 0.0, frequency_penalty: float = 0.0,
                 repetition_context: int = 20, presence_context: int = 20, frequency_context: int = 20,
                 chain: str = "mlx", top_logprobs: int = 0):
        self.kw = dict(temperature=temperature, top_p=top_p, top_k=top_k, min_p=min_p, chain=chain)
        self.pen = dict(
            repetition_penalty=0.0 if repetition_penalty in (None, 1.0) else float(repetition_penalty),
            presence_penalty=float(presence_penalty or 0.0), frequency_penalty=float(frequency_penalty or 0.0),
            repetition_context=repetition_context, presence_context=presence_context,
            frequency_context=frequency_context)
        self.top_logprobs = int(top_logprobs)
        ctxs = [c for p, c in ((self.pen["repetition_penalty"], repetition_context),
                               (self.pen["presence_penalty"], presence_context),
                               (self.pen["frequency_penalty"], frequency_context)) if p]
        # ids the history must keep: None = the whole history (a context of 0)
        self.window = None if any(c <= 0 for c in ctxs) else max(ctxs, default=0)

    @classmethod
    def from_options(cls, options: GenerationOptions, **kw) -> "TokenSelector":
        """The sampler and processors generation.py:1279-1293 builds from a
        request's options: make_sampler(temp, top_p, top_k, min_p), plus
        presence / repetition processors when they differ from 0 / 1 (the
        processors' default window of 20 ids)."""
        return cls(temperature=options.temperature, top_p=options.top_p, top_k=options.top_k,
                   min_p=options.min_p, presence_penalty=options.presence_penalty,
                   repetition_penalty=options.repetition_penalty, chain="mlx", **kw)

    @property
    def penalised(self) -> bool:
        return any(self.pen[k] for k in ("repetition_penalty", "presence_penalty", "frequency_penalty"))

    def make_state(self, prompts: Sequence[Sequence[int]], device, capacity: int = 0,
                   max_append: int = 1) -> DecodeState:
        """A DecodeState sized for this selector's penalty window."""
        keep = self.window
        if capacity <= 0:
            # a context of 0 reads the whole history: wh_sample takes at most
            # WH_MAX_WINDOW (4096) history entries per row
            capacity = max(2 * (keep or 0) + max_append + 1, 64) if keep is not None else 4096
        return DecodeState.from_prompts(prompts, capacity, keep, device, max_append)

    def __call__(self, logits: torch.Tensor, state: Optional[DecodeState] = None,
                 uniforms: Optional[torch.Tensor] = None, generator: Optional[torch.Generator] = None,
                 append: bool = True):
        """Select one token per row of logits [B, V]; append it to `state`.
        Returns tokens int32 [B] (device), or (tokens, (ids, logprobs,
        token_logprobs)) with top_logprobs."""
        hist = dict(history=state.history, history_len=state.history_len) if (state and self.penalised) else {}
        extra = None
        if self.top_logprobs:
            rows = logits.reshape(-1, logits.shape[-1]).float()  # the f32 values the fused call would penalise
            if rows.data_ptr() == logits.data_ptr():
                rows = rows.clone()
            if hist:
                S.apply_penalties(rows, **hist, **self.pen)
            tok = S.sample(rows, uniforms=uniforms, generator=generator, **self.kw)
            ids, lps, tlp = _top_logprobs(rows, self.top_logprobs, tokens=tok)
            extra = (ids, lps, tlp)
        else:
            tok = S.sample(logits, uniforms=uniforms, generator=generator, **self.kw, **(self.pen if hist else {}),
                           **hist)
        if state is not None and append:
            state.append(tok)
        return tok if extra is None else (tok, extra)


def generate(model_step: Callable[[torch.Tensor], torch.Tensor], prompts: Sequence[Sequence[int]], *,
             max_tokens: int, selector: TokenSelector, device="cuda", eos_token_ids: Sequence[int] = (),
             uniforms: Optional[Callable[[int], torch.Tensor]] = None,
             state: Optional[DecodeState] = None) -> Iterator[list]:
    """stream_generate's decode loop (generation.py:1465-1475) over device
    state.  model_step(last_tokens int32 [B]) -> logits [B, V] is the model;
    each step yields the B chosen ids as Python ints (one synchronisation, as
    generate_step's `.item()`).  A row that emitted one of eos_token_ids keeps
    being stepped but is reported as finished by yielding None for it.
    uniforms(step) -> float32 [B] device tensor drives the draws when given."""
    dev = torch.device(device)
    if state is None:
        state = selector.make_state(prompts, dev)
    last = torch.tensor([p[-1] for p in prompts], dtype=torch.int32, device=dev)
    done = [False] * len(prompts)
    eos = set(int(e) for e in eos_token_ids)
    for step in range(max_tokens):
        logits = model_step(last)
        out = selector(logits, state, uniforms=None if uniforms is None else uniforms(step))
        last = out[0] if isinstance(out, tuple) else out
        ids = last.tolist()
        yield [None if done[b] else ids[b] for b in range(len(ids))]
        for b, t in enumerate(ids):
            if t in eos:
                done[b] = True
        if all(done):
            return
