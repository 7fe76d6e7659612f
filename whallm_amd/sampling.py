"""Tensor-level entry points over libwh_sample.so.

These are the batched calls the drop-in mirrors (sample_utils.py, dspark.py)
are built on, and the fused decode-step API: one kernel launch applies the
penalty processors, the filter chain, the temperature and the draw.

Every function is asynchronous on the current HIP stream of its inputs and
returns device tensors; nothing here synchronises with the host.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib as L

_CHAINS = {"mlx": L.CHAIN_MLX, "whallm": L.CHAIN_WHALLM, L.CHAIN_MLX: L.CHAIN_MLX, L.CHAIN_WHALLM: L.CHAIN_WHALLM}


def _as_rows(logits: torch.Tensor):
    if logits.dim() == 1:
        logits = logits.unsqueeze(0)
    if logits.dim() != 2:
        raise ValueError("logits must be [V] or [B, V]")
    if logits.dtype == torch.float32:
        dt = L.DTYPE_F32
    elif logits.dtype == torch.bfloat16:
        dt = L.DTYPE_BF16
    elif logits.dtype == torch.float16:
        logits = logits.float()  # exact widening
        dt = L.DTYPE_F32
    else:
        raise ValueError(f"unsupported logits dtype {logits.dtype}")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    return logits, dt


def _rows_param(x, B, dtype, device):
    if x is None:
        return None
    t = torch.as_tensor(x, dtype=dtype, device=device)
    if t.dim() == 0:
        t = t.expand(B)
    t = t.contiguous()
    if t.shape != (B,):
        raise ValueError("per-row parameters must have shape [B]")
    return t


def _history(history, history_len, B, device):
    if history is None:
        return None, 0, None
    h = torch.as_tensor(history, device=device)
    if h.dtype != torch.int32:
        h = h.to(torch.int32)
    if h.dim() == 1:
        h = h.unsqueeze(0).expand(B, -1)
    if h.dim() != 2 or h.shape[0] != B:
        raise ValueError("history must be [H] or [B, H]")
    h = h.contiguous()
    if history_len is None:
        hl = torch.full((B,), h.shape[1], dtype=torch.int32, device=device)
    else:
        hl = torch.as_tensor(history_len, dtype=torch.int32, device=device)
        if hl.dim() == 0:
            hl = hl.expand(B)
        hl = hl.contiguous()
    return h, h.shape[1], hl


def _fill_args(a: L.SampleArgs, logits, dt, chain, history, history_len, temperature, top_p, top_k, min_p,
               repetition_penalty, presence_penalty, frequency_penalty, repetition_context, presence_context,
               frequency_context, rows):
    B, V = logits.shape
    a.logits = logits.data_ptr()
    a.dtype = dt
    a.B = B
    a.V = V
    a.chain = _CHAINS[chain]
    a.row_stride = logits.stride(0) if B > 1 else V
    h, hs, hl = _history(history, history_len, B, logits.device)
    a.history = L.ptr(h)
    a.history_stride = hs
    a.history_len = L.ptr(hl)
    a.temperature = float(temperature)
    a.top_p = float(top_p)
    a.top_k = int(top_k)
    a.min_p = float(min_p)
    a.repetition_penalty = float(repetition_penalty or 0.0)
    a.presence_penalty = float(presence_penalty or 0.0)
    a.frequency_penalty = float(frequency_penalty or 0.0)
    a.repetition_context = int(repetition_context or 0)
    a.presence_context = int(presence_context or 0)
    a.frequency_context = int(frequency_context or 0)
    tr, pr, mr, kr = rows
    a.temperature_rows = L.ptr(tr)
    a.top_p_rows = L.ptr(pr)
    a.min_p_rows = L.ptr(mr)
    a.top_k_rows = L.ptr(kr)
    return (h, hl)  # keep alive until launch


def sample(logits: torch.Tensor, *, temperature: float = 0.0, top_p: float = 1.0, top_k: int = 0,
           min_p: float = 0.0, chain="mlx", history=None, history_len=None,
           repetition_penalty: float = 0.0, presence_penalty: float = 0.0, frequency_penalty: float = 0.0,
           repetition_context: int = 20, presence_context: int = 20, frequency_context: int = 20,
           uniforms: torch.Tensor | None = None, generator: torch.Generator | None = None,
           temperature_rows=None, top_p_rows=None, min_p_rows=None, top_k_rows=None,
           return_logprobs: bool = False, return_kept: bool = False, engine: str = "auto"):
    """Fused decode-step token selection for B rows (one kernel launch).

    chain "mlx": mlx_lm make_sampler order (top_k -> top_p -> min_p, then
    categorical(logprobs * (1/T))); chain "whallm": Whallm sampling_logprobs
    order (top_p -> min_p -> top_k, logprobs / max(T, 1e-5)).  Penalties
    (repetition -> presence -> frequency over the last *_context ids of
    `history`; context 0 = the whole history) are applied first.  `uniforms`
    [B] in [0, 1) drive the inverse-CDF draw; when None they are drawn with
    torch.rand on the logits' device (optionally from `generator`).

    Returns int32 tokens [B]; with return_logprobs (chain "whallm" only) also
    the sampling_logprobs rows [B, V]; with return_kept the kept-set sizes.
    engine "exact" forces the multi-pass engine (no workspace) -- both
    engines return identical results; "auto" picks the sliced single-read one;
    "noalloc" calls wh_sample_noalloc, which uses the library's own device
    scratch instead of a workspace (same results, no allocation).
    """
    logits, dt = _as_rows(logits)
    L.require_device(logits)
    B, V = logits.shape
    dev = logits.device
    rows = (_rows_param(temperature_rows, B, torch.float64, dev), _rows_param(top_p_rows, B, torch.float64, dev),
            _rows_param(min_p_rows, B, torch.float64, dev), _rows_param(top_k_rows, B, torch.int32, dev))
    if uniforms is None:
        uniforms = torch.rand(B, device=dev, dtype=torch.float32, generator=generator)
    else:
        uniforms = torch.as_tensor(uniforms, dtype=torch.float32, device=dev).reshape(B).contiguous()
    tokens = torch.empty(B, dtype=torch.int32, device=dev)
    kept = torch.empty(B, dtype=torch.int32, device=dev) if return_kept else None
    out = torch.empty(B, V, dtype=torch.float32, device=dev) if return_logprobs else None
    a = L.SampleArgs()
    keep = _fill_args(a, logits, dt, chain, history, history_len, temperature, top_p, top_k, min_p,
                      repetition_penalty, presence_penalty, frequency_penalty, repetition_context,
                      presence_context, frequency_context, rows)
    a.uniforms = uniforms.data_ptr()
    a.tokens = tokens.data_ptr()
    a.kept_count = L.ptr(kept)
    a.logprobs_out = L.ptr(out)
    a.out_mode = L.OUT_LOGPROBS
    fn = L.lib().wh_sample
    if engine == "noalloc":
        fn = L.lib().wh_sample_noalloc
    elif engine != "exact":
        nb = L.lib().wh_sample_workspace_bytes(B, V)
        ws = L.workspace(dev, nb)
        a.workspace = ws.data_ptr()
        a.workspace_bytes = ws.numel()
    L.check(fn(ctypes.byref(a), ctypes.c_void_p(L.stream_of(logits))))
    del keep
    res = [tokens]
    if return_logprobs:
        res.append(out)
    if return_kept:
        res.append(kept)
    return tokens if len(res) == 1 else tuple(res)


def _bound(name, t, dtype, shape):
    """A buffer a pre-bound call reads on every invocation: it must already be
    exactly what the kernel reads, or later refills by the caller would not
    reach the kernel (a converted copy would be read instead)."""
    if t is None:
        return None
    if not isinstance(t, torch.Tensor) or t.dtype != dtype or tuple(t.shape) != tuple(shape) or not t.is_contiguous():
        got = f"{t.dtype} {tuple(t.shape)}" if isinstance(t, torch.Tensor) else type(t).__name__
        raise ValueError(f"{name} must be a contiguous {dtype} tensor of shape {tuple(shape)} (got {got}): "
                         "a pre-bound call reads the caller's buffer itself on every call")
    return t


class SampleCall:
    """A wh_sample launch bound to fixed device buffers.

    For decode loops that refill the same logits / history / uniform buffers
    every step: the C argument struct is built once, and each call is one
    ctypes call into wh_sample on the stream current at construction.  Takes
    the keyword arguments of sample(); `uniforms` is required.  Every buffer
    must already be in the layout the kernel reads -- logits float32 or
    bfloat16 [B, V] with unit last stride, history int32 [B, H], history_len
    int32 [B], uniforms float32 [B], per-row parameters float64 / int32 [B] --
    because the call keeps reading the caller's buffers (a ValueError names
    the first that is not).  The outputs are the attributes `tokens` (and
    `kept` with return_kept).
    """

    def __init__(self, logits: torch.Tensor, *, uniforms: torch.Tensor, temperature: float = 0.0,
                 top_p: float = 1.0, top_k: int = 0, min_p: float = 0.0, chain="mlx", history=None,
                 history_len=None, repetition_penalty: float = 0.0, presence_penalty: float = 0.0,
                 frequency_penalty: float = 0.0, repetition_context: int = 20, presence_context: int = 20,
                 frequency_context: int = 20, temperature_rows=None, top_p_rows=None, min_p_rows=None,
                 top_k_rows=None, return_kept: bool = False, engine: str = "auto"):
        if not isinstance(logits, torch.Tensor) or logits.dim() != 2 or logits.stride(1) != 1 or \
                logits.dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("logits must be a float32 or bfloat16 [B, V] tensor with unit last stride")
        dt = L.DTYPE_F32 if logits.dtype == torch.float32 else L.DTYPE_BF16
        L.require_device(logits)
        B, V = logits.shape
        dev = logits.device
        rows = (_bound("temperature_rows", temperature_rows, torch.float64, (B,)),
                _bound("top_p_rows", top_p_rows, torch.float64, (B,)),
                _bound("min_p_rows", min_p_rows, torch.float64, (B,)),
                _bound("top_k_rows", top_k_rows, torch.int32, (B,)))
        u = _bound("uniforms", uniforms, torch.float32, (B,))
        if history is not None:
            _bound("history", history, torch.int32, (B, history.shape[-1] if isinstance(history, torch.Tensor) else -1))
            _bound("history_len", history_len, torch.int32, (B,))
            if history_len is None:
                raise ValueError("history_len must be given with history in a pre-bound call")
        L.require_device(u, history, history_len, *rows)
        self.tokens = torch.empty(B, dtype=torch.int32, device=dev)
        self.kept = torch.empty(B, dtype=torch.int32, device=dev) if return_kept else None
        self.args = L.SampleArgs()
        keep = _fill_args(self.args, logits, dt, chain, history, history_len, temperature, top_p, top_k, min_p,
                          repetition_penalty, presence_penalty, frequency_penalty, repetition_context,
                          presence_context, frequency_context, rows)
        if history is not None and (keep[0].data_ptr() != history.data_ptr() or
                                    keep[1].data_ptr() != history_len.data_ptr()):
            raise ValueError("history buffers were copied: pass int32 [B, H] history and int32 [B] history_len")
        self.args.uniforms = u.data_ptr()
        self.args.tokens = self.tokens.data_ptr()
        self.args.kept_count = L.ptr(self.kept)
        self.args.out_mode = L.OUT_LOGPROBS
        self._ws = None
        if engine != "exact":
            self._ws = L.workspace(dev, L.lib().wh_sample_workspace_bytes(B, V))
            self.args.workspace = self._ws.data_ptr()
            self.args.workspace_bytes = self._ws.numel()
        self._alive = (logits, u, rows, keep)
        self._stream = ctypes.c_void_p(L.stream_of(logits))
        self._fn = L.lib().wh_sample
        self._ref = ctypes.byref(self.args)

    def __call__(self) -> torch.Tensor:
        L.check(self._fn(self._ref, self._stream))
        return self.tokens


def last_paths(device, B: int) -> torch.Tensor:
    """Per-row engine path of the last workspace call on the current
    stream: 0 merged from candidates, 1 exact engine (candidate or list
    overflow), 2 greedy, 3 exact engine (top-p cut not settled by the
    normaliser bounds), 4 merged from candidates through LDS (large sets),
    6 wide exact engine (top-p alone or no filter), 7 merged from candidates
    after a float sum over the row settled the top-p cut.
    Diagnostics only: results are identical."""
    ws = L.workspace(torch.device(device), 0)
    return ws[:4 * B].view(torch.int32).clone()


def filter_rows(logits: torch.Tensor, *, chain="whallm", temperature: float = 1.0, top_p: float = 1.0,
                top_k: int = 0, min_p: float = 0.0, out_mode: int = L.OUT_LOGPROBS,
                history=None, history_len=None, repetition_penalty: float = 0.0, presence_penalty: float = 0.0,
                frequency_penalty: float = 0.0, repetition_context: int = 20, presence_context: int = 20,
                frequency_context: int = 20, engine: str = "auto") -> torch.Tensor:
    """Filtered rows without a draw: OUT_LOGPROBS gives Whallm's
    sampling_logprobs row, OUT_MASKED the input row with filtered entries -inf."""
    logits, dt = _as_rows(logits)
    L.require_device(logits)
    B, V = logits.shape
    out = torch.empty(B, V, dtype=torch.float32, device=logits.device)
    a = L.SampleArgs()
    keep = _fill_args(a, logits, dt, chain, history, history_len, temperature, top_p, top_k, min_p,
                      repetition_penalty, presence_penalty, frequency_penalty, repetition_context,
                      presence_context, frequency_context, (None, None, None, None))
    a.logprobs_out = out.data_ptr()
    a.out_mode = out_mode
    if engine != "exact":
        ws = L.workspace(logits.device, L.lib().wh_sample_workspace_bytes(B, V))
        a.workspace = ws.data_ptr()
        a.workspace_bytes = ws.numel()
    L.check(L.lib().wh_sample(ctypes.byref(a), ctypes.c_void_p(L.stream_of(logits))))
    del keep
    return out


def apply_penalties(logits: torch.Tensor, history, history_len=None, *, repetition_penalty: float = 0.0,
                    presence_penalty: float = 0.0, frequency_penalty: float = 0.0, repetition_context: int = 20,
                    presence_context: int = 20, frequency_context: int = 20) -> torch.Tensor:
    """Penalty processors in place (float32 or bf16 logits); returns logits."""
    rows, dt = _as_rows(logits)
    if rows.data_ptr() != logits.data_ptr():
        raise ValueError("apply_penalties works in place on float32/bfloat16 logits with unit last stride")
    L.require_device(rows)
    a = L.SampleArgs()
    keep = _fill_args(a, rows, dt, "mlx", history, history_len, 1.0, 1.0, 0, 0.0, repetition_penalty,
                      presence_penalty, frequency_penalty, repetition_context, presence_context, frequency_context,
                      (None, None, None, None))
    L.check(L.lib().wh_apply_penalties(ctypes.byref(a), ctypes.c_void_p(L.stream_of(rows))))
    del keep
    return logits


def _verify_args(target, draft, draft_tokens, uniforms, temperature, B, n, V):
    a = L.VerifyArgs()
    a.B, a.n, a.V = B, n, V
    a.temperature = float(temperature)
    a.target = target.data_ptr()
    a.draft = L.ptr(draft)
    a.draft_tokens = L.ptr(draft_tokens)
    a.uniforms = L.ptr(uniforms)
    return a


def verify_logprobs(target_logprobs: torch.Tensor, draft_logprobs: torch.Tensor | None, draft_tokens: torch.Tensor,
                    temperature: float, uniforms: torch.Tensor | None = None, generator=None,
                    return_row: bool = False):
    """Batched _verify over logprob rows: target [B, n+1, V], draft [B, n, V]
    (may be None when temperature == 0), draft_tokens [B, n], uniforms
    [B, n+1] (u[:, j<n] accept tests, u[:, n] the final draw).
    Returns (accepted [B], token [B]) [+ row [B, V]]."""
    target = target_logprobs.float().contiguous()
    B, n1, V = target.shape
    n = n1 - 1
    dev = target.device
    draft = None if (draft_logprobs is None or n == 0) else draft_logprobs.float().contiguous()
    if draft is not None and draft.shape != (B, n, V):
        raise ValueError("draft logprobs must be [B, n, V]")
    toks = torch.as_tensor(draft_tokens, dtype=torch.int32, device=dev).reshape(B, n).contiguous()
    L.require_device(target, draft, toks)
    if uniforms is None and temperature > 0:
        uniforms = torch.rand(B, n1, device=dev, dtype=torch.float32, generator=generator)
    if uniforms is not None:
        uniforms = torch.as_tensor(uniforms, dtype=torch.float32, device=dev).reshape(B, n1).contiguous()
    acc = torch.empty(B, dtype=torch.int32, device=dev)
    tok = torch.empty(B, dtype=torch.int32, device=dev)
    row = torch.empty(B, V, dtype=torch.float32, device=dev) if return_row else None
    a = _verify_args(target, draft, toks, uniforms, temperature, B, n, V)
    a.accepted = acc.data_ptr()
    a.token = tok.data_ptr()
    a.row_out = L.ptr(row)
    L.check(L.lib().wh_verify_logprobs(ctypes.byref(a), ctypes.c_void_p(L.stream_of(target))))
    return (acc, tok, row) if return_row else (acc, tok)


def verify_fused(target_logits: torch.Tensor, draft_probs: torch.Tensor, draft_tokens: torch.Tensor,
                 temperature: float, uniforms: torch.Tensor | None = None, generator=None):
    """Fused verifier: target logits [B, n+1, V] (p = softmax(x / T) is formed
    inside), draft probabilities q [B, n, V], draft_tokens [B, n], uniforms
    [B, n+1].  Returns (accepted [B], token [B])."""
    target = target_logits.float().contiguous()
    B, n1, V = target.shape
    n = n1 - 1
    dev = target.device
    q = draft_probs.float().contiguous() if n > 0 else None
    toks = torch.as_tensor(draft_tokens, dtype=torch.int32, device=dev).reshape(B, n).contiguous()
    L.require_device(target, q, toks)
    if uniforms is None and temperature > 0:
        uniforms = torch.rand(B, n1, device=dev, dtype=torch.float32, generator=generator)
    if uniforms is not None:
        uniforms = torch.as_tensor(uniforms, dtype=torch.float32, device=dev).reshape(B, n1).contiguous()
    acc = torch.empty(B, dtype=torch.int32, device=dev)
    tok = torch.empty(B, dtype=torch.int32, device=dev)
    a = _verify_args(target, q, toks, uniforms, temperature, B, n, V)
    a.accepted = acc.data_ptr()
    a.token = tok.data_ptr()
    nb = L.lib().wh_verify_workspace_bytes(B, n, V)
    ws = L.workspace(dev, nb)
    a.workspace = ws.data_ptr()
    a.workspace_bytes = ws.numel()
    L.check(L.lib().wh_verify_fused(ctypes.byref(a), ctypes.c_void_p(L.stream_of(target))))
    return acc, tok


class VerifyCall:
    """A wh_verify_fused launch bound to fixed device buffers (target logits
    float32 [B, n+1, V], draft probabilities float32 [B, n, V], draft tokens
    int32 [B, n], uniforms float32 [B, n+1], all contiguous: the call keeps
    reading the caller's buffers, so a buffer in any other layout raises
    ValueError instead of being copied).  Each call is one ctypes call on the
    stream current at construction; outputs are the attributes `accepted`
    and `token`."""

    def __init__(self, target_logits: torch.Tensor, draft_probs: torch.Tensor, draft_tokens: torch.Tensor,
                 temperature: float, uniforms: torch.Tensor):
        if not isinstance(target_logits, torch.Tensor) or target_logits.dim() != 3:
            raise ValueError("target logits must be a float32 [B, n+1, V] tensor")
        B, n1, V = target_logits.shape
        n = n1 - 1
        dev = target_logits.device
        target = _bound("target logits", target_logits, torch.float32, (B, n1, V))
        q = _bound("draft probabilities", draft_probs, torch.float32, (B, n, V)) if n > 0 else None
        toks = _bound("draft tokens", draft_tokens, torch.int32, (B, n))
        u = _bound("uniforms", uniforms, torch.float32, (B, n1))
        L.require_device(target, q, toks, u)
        self.accepted = torch.empty(B, dtype=torch.int32, device=dev)
        self.token = torch.empty(B, dtype=torch.int32, device=dev)
        self.args = _verify_args(target, q, toks, u, temperature, B, n, V)
        self.args.accepted = self.accepted.data_ptr()
        self.args.token = self.token.data_ptr()
        self._ws = L.workspace(dev, L.lib().wh_verify_workspace_bytes(B, n, V))
        self.args.workspace = self._ws.data_ptr()
        self.args.workspace_bytes = self._ws.numel()
        self._alive = (target, q, toks, u)
        self._stream = ctypes.c_void_p(L.stream_of(target))
        self._fn = L.lib().wh_verify_fused
        self._ref = ctypes.byref(self.args)

    def __call__(self):
        L.check(self._fn(self._ref, self._stream))
        return self.accepted, self.token


def exp_fix44(d: torch.Tensor) -> torch.Tensor:
    """Device contract exponential floor(2^44 exp(d)) as int64 (test hook)."""
    d = d.float().contiguous()
    L.require_device(d)
    out = torch.empty(d.shape, dtype=torch.int64, device=d.device)
    L.check(L.lib().wh_exp_fix44(d.data_ptr(), out.data_ptr(), d.numel(), ctypes.c_void_p(L.stream_of(d))))
    return out
