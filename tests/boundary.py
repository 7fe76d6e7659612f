"""Float64 distance of a sampling or verify outcome from the nearest
cumulative-probability boundary (test infrastructure).

The contract oracle and the HIP kernels compute every cut and draw exactly
(fixed-point masses); the faithful replay of the reference's op order
(oracle/wh_oracle.c, who_*_faithful) rounds in float32 along a sequential
cumsum.  The two may disagree only where a decision lies within float32
rounding of its boundary.  These functions restate, in float64 and
independently of both, where each decision's boundary lies, so a test can
assert that every disagreement is within 1e-6 of one:

  * top-p: keep i iff S - head_excl(i) > fp32(1 - top_p)
    (runtime/deepseek_v4_ssd/dspark.py:369 via mlx_lm apply_top_p), the
    distance |S - head_excl(i) - theta| for every element whose final status
    the decision sets;
  * min-p: keep i iff lp_i >= lp_max + fp32(ln min_p), the distance in nats;
  * top-k: the gap between the k-th and (k+1)-th values (float32 rounding of
    the logprobs can only reorder values closer than that);
  * the draw: |u - C_j / Z| over the kept set's cumulative sums in vocab order;
  * verify (dspark.py:880-896): |u_j - min(1, p_j(t) / q_j(t))| for every
    tested position, and the residual draw's |u_n - C_j / Z|.
"""
from __future__ import annotations

import math

import numpy as np

INF = float("inf")


def _lse(x):
    m = np.max(x)
    if m == -np.inf:
        return -np.inf
    return m + math.log(np.sum(np.exp(x - m)))


def _draw_margin(w, u):
    """min_j |u - C_j / Z| over the positive weights w (vocab order)."""
    w = w[w > 0]
    if w.size == 0:
        return INF
    c = np.cumsum(w)
    return float(np.min(np.abs(float(u) - c / c[-1])))


def sample_margin(l, *, temperature, top_p=1.0, top_k=0, min_p=0.0, chain=0, u=0.5):
    """Margin of one row.  l: the penalised float32 logits of the row."""
    l = np.asarray(l, np.float64)
    V = l.size
    margins = [INF]
    if not temperature > 0:
        # argmax: the faithful chain A takes it over float32 logprobs, where
        # two close logits can round to one value
        s = np.sort(l[np.isfinite(l)])
        if s.size >= 2 and s[-1] != s[-2]:
            margins.append((s[-1] - s[-2]) / max(1.0, abs(s[-1])))
        return min(margins)
    if not np.isfinite(l).any():
        return INF
    lp = l - _lse(l)
    alive = np.isfinite(lp)
    use_k = 0 < top_k < V
    use_p = 0.0 < top_p < 1.0
    use_m = min_p != 0.0
    theta = float(np.float32(1.0 - top_p))
    cmin = float(np.float32(math.log(min_p))) if use_m else -INF
    steps = "kpm" if chain == 0 else "pmk"
    order_k = np.lexsort((np.arange(V), -lp))     # value desc, id asc
    order_p = np.lexsort((-np.arange(V), -lp))    # value desc, id desc
    p_decisions = []                              # (id, margin) of each top-p decision

    for si, s in enumerate(steps):
        later = steps[si + 1:]
        if s == "k" and use_k:
            idx = [i for i in order_k if alive[i]]
            if len(idx) > top_k:
                gap = lp[idx[top_k - 1]] - lp[idx[top_k]]
                if gap > 0:
                    margins.append(gap)
                for i in idx[top_k:]:
                    alive[i] = False
        elif s == "p" and use_p:
            pr = np.where(alive, np.exp(lp), 0.0)
            S = pr.sum()
            head = 0.0
            for i in order_p:
                if not alive[i]:
                    continue
                val = S - head
                p_decisions.append((i, abs(val - theta), later))
                head += pr[i]
                if not val > theta:
                    alive[i] = False
        elif s == "m" and use_m and alive.any():
            thr = lp[alive].max() + cmin
            d = np.abs(lp[alive] - thr)
            margins.append(float(d.min()))
            alive &= ~(lp < thr)
    # a top-p decision matters when the element would survive the later filters
    if p_decisions:
        thr_m = (lp[np.isfinite(lp)].max() + cmin) if use_m else -INF
        kth = INF
        if use_k and chain == 1:
            kept_vals = np.sort(lp[alive])[::-1]
            kth = kept_vals[top_k - 1] if kept_vals.size >= top_k else -INF
        for i, mg, later in p_decisions:
            if "m" in later and lp[i] < thr_m - 1e-6:
                continue
            if "k" in later and lp[i] < kth - 1e-6:
                continue
            margins.append(mg)
    if alive.any():
        z = lp[alive] - lp[alive].max()
        z = z / temperature if chain == 0 else z / max(temperature, 1e-5)
        w = np.zeros(V)
        w[alive] = np.exp(z)
        margins.append(_draw_margin(w, u))
    return float(min(margins))


def sample_margins(logits_pen, params, u):
    """Per-row margins; params: the oracle's parameter records."""
    B = logits_pen.shape[0]
    out = np.empty(B)
    for b in range(B):
        p = params[b]
        out[b] = sample_margin(logits_pen[b], temperature=float(p["temperature"]), top_p=float(p["top_p"]),
                               top_k=int(p["top_k"]), min_p=float(p["min_p"]), chain=int(p["chain"]),
                               u=float(np.asarray(u).reshape(-1)[b]))
    return out


def verify_margin(target_lp, draft_lp, draft_tokens, u, temperature):
    """Margin of one verify entry.  target_lp [n+1, V], draft_lp [n, V]
    (float64 logprob rows), u [n+1]."""
    n = len(draft_tokens)
    margins = [INF]
    if not temperature > 0:
        for j in range(n + 1):
            s = np.sort(target_lp[j][np.isfinite(target_lp[j])])
            if s.size >= 2 and s[-1] != s[-2]:
                margins.append(s[-1] - s[-2])
        return min(margins)
    j = 0
    while j < n:
        t = int(draft_tokens[j])
        if not (0 <= t < target_lp.shape[1]):
            break
        g, d = target_lp[j, t], draft_lp[j, t]
        ratio = 1.0 if (np.isneginf(g) and np.isneginf(d)) else min(1.0, math.exp(g - d)) if np.isfinite(d) else 1.0
        margins.append(abs(float(u[j]) - ratio))
        if float(u[j]) > ratio:
            break
        j += 1
    if j == n:
        margins.append(_draw_margin(np.exp(target_lp[n]), u[n]))
    else:
        dlt = np.maximum(np.exp(target_lp[j]) - np.exp(draft_lp[j]), 0.0)
        margins.append(_draw_margin(dlt if dlt.sum() > 0 else np.exp(target_lp[j]), u[n]))
    return float(min(margins))
