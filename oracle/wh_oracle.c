/*
 * wh_oracle.c -- CPU oracle for Whallm's decode-time token selection.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product path links, loads or
 * calls this file: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker or the timed CPU baseline.
 *
 * Two restatements live here, both written in the reference's style (full
 * sorts, sequential scans), deliberately unlike the GPU's radix/threshold
 * kernels so that agreement between the two means something:
 *
 *  1. The CONTRACT oracle (who_sample_rows, who_verify_*): the exact
 *     arithmetic the HIP kernels must reproduce bit for bit.  Probability
 *     masses are fixed-point integers (44 fractional bits) of the contract
 *     exponential, so every sum is order independent and every cutoff and
 *     draw is an exact integer comparison.
 *
 *  2. The FAITHFUL oracle (who_sample_rows_faithful, who_verify_faithful):
 *     float32 arithmetic in the order mlx_lm / Whallm execute it
 *     (logsumexp, stable argsort, sequential cumsum).  It is used to report
 *     how often float rounding at a cumulative boundary changes a token, and
 *     it is the CPU baseline that bench.py times.
 *
 * Reference behaviour followed (paths relative to the reference root):
 *   runtime/deepseek_v4_ssd/generation.py:1279-1293  sampler + processors
 *   runtime/deepseek_v4_ssd/dspark.py:358-375        sampling_logprobs (chain B)
 *   runtime/deepseek_v4_ssd/dspark.py:857-898        _verify
 *   runtime/deepseek_v4_ssd/dspark.py:901-904        _sample
 *   runtime/deepseek_v4_ssd/qwen4_exp.py:946-958     penalties then chain B
 *   mlx_lm.sample_utils (third party, mlx-lm @ 5c10538, not vendored in the
 *   reference): make_sampler (chain A: top-k -> top-p -> min-p, then
 *   categorical(logprobs * (1/T))), apply_top_k/top_p/min_p,
 *   make_logits_processors (repetition -> presence -> frequency).  The
 *   third-party arithmetic is restated from its published source; the
 *   reference holds no golden vectors for it.
 *
 * Build: see oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define WHO_CHAIN_KPM 0 /* mlx_lm make_sampler: top_k -> top_p -> min_p, * (1/T) */
#define WHO_CHAIN_PMK 1 /* Whallm sampling_logprobs: top_p -> min_p -> top_k, / max(T,1e-5) */

#define WHO_OK 0
#define WHO_EINVAL -1
#define WHO_ENOMEM -2

typedef unsigned __int128 u128;

typedef struct {
  /* temperature, top_p and min_p are the caller's doubles (Python floats in
   * the reference); the float32 constants of the filters are derived from
   * them as MLX derives them: fp32(1 - top_p), fp32(1 / T), fp32(max(T, 1e-5)),
   * fp32(ln min_p). */
  double temperature;
  double top_p;
  double min_p;
  int32_t top_k;
  float repetition_penalty; /* 0 => processor absent */
  float presence_penalty;   /* 0 => processor absent */
  float frequency_penalty;  /* 0 => processor absent */
  int32_t repetition_context; /* 0 => whole history (Python tokens[-0:]) */
  int32_t presence_context;
  int32_t frequency_context;
  int32_t chain;
} who_params;

/* ------------------------------------------------------------------------ */
/* Contract exponential.                                                     */
/* ------------------------------------------------------------------------ */
/* Coefficients of p(f) ~ 2^f on [0,1], fitted by oracle/fit_exp2.py (Lawson
 * minimax on the relative error, float32 Horner error <= 0.55 ulp). */
static const float WHO_C1 = 0x1.62e42cp-1f;
static const float WHO_C2 = 0x1.ebfd58p-3f;
static const float WHO_C3 = 0x1.c68912p-5f;
static const float WHO_C4 = 0x1.3d0b92p-7f;
static const float WHO_C5 = 0x1.46d64cp-10f;
static const float WHO_C6 = 0x1.c5417ap-13f;
static const float WHO_LOG2E = 0x1.715476p+0f;

/* floor(2^44 * 2^t') with t' = fl(d * log2 e) split as n + f; an integer
 * approximation of exp(d) * 2^44 for d <= 0.  Arguments below -45 binades
 * (and -inf) give 0. */
uint64_t who_exp_fix44(float d) {
  float t = d * WHO_LOG2E;
  if (!(t > -45.0f)) return 0;
  if (t > 0.0f) t = 0.0f; /* d <= 0 by contract; clamp rounding of tiny positives */
  float n = floorf(t);
  float f = t - n;
  float p = WHO_C6;
  p = fmaf(p, f, WHO_C5);
  p = fmaf(p, f, WHO_C4);
  p = fmaf(p, f, WHO_C3);
  p = fmaf(p, f, WHO_C2);
  p = fmaf(p, f, WHO_C1);
  p = fmaf(p, f, 1.0f);
  uint32_t mant = (uint32_t)(p * 8388608.0f); /* exact: p in [1,2] */
  int sh = (int)n + 21;
  return sh >= 0 ? ((uint64_t)mant << sh) : (uint64_t)(mant >> (-sh));
}

/* The float value exp(d) the contract exponential represents (for tests). */
double who_exp_contract_value(float d) { return ldexp((double)who_exp_fix44(d), -44); }

/* A > theta * Z exactly, for integers A, Z and float32 theta in [0, 1).
 * For integer A, A > x  <=>  A > floor(x). */
static int who_gt_theta(uint64_t A, float theta, uint64_t Z) {
  if (!(theta > 0.0f)) return A > 0;
  int e;
  float fr = frexpf(theta, &e);                     /* theta = fr * 2^e */
  uint64_t M = (uint64_t)ldexpf(fr, 24);            /* theta = M * 2^(e-24) */
  int s = 24 - e;
  u128 prod = (u128)M * (u128)Z;
  u128 F = s >= 128 ? 0 : (prod >> s);
  return (u128)A > F;
}

/* Uniform in [0,1) -> 32-bit fixed point, clamped. */
static uint64_t who_u32(float u) {
  if (!(u > 0.0f)) return 0;
  if (u >= 1.0f) return 0xFFFFFFFFull;
  return (uint64_t)(u * 4294967296.0f); /* exact scaling, truncation */
}

/* Index of the first i with cumulative weight > (U * total) >> 32. */
static int who_locate(const uint64_t* w, const int* order, int n, uint64_t total, float u) {
  uint64_t tgt = (uint64_t)(((u128)who_u32(u) * (u128)total) >> 32);
  uint64_t c = 0;
  int last = -1;
  for (int j = 0; j < n; ++j) {
    int i = order ? order[j] : j;
    if (w[i] == 0) continue;
    c += w[i];
    last = i;
    if (c > tgt) return i;
  }
  return last; /* unreachable when total > 0 */
}

/* ------------------------------------------------------------------------ */
/* Penalties (mlx_lm make_logits_processors, applied in append order).       */
/* ------------------------------------------------------------------------ */
static int who_window(int ctx, int len) { return (ctx <= 0 || ctx > len) ? len : ctx; }

/* Repetition: once per unique id in its window, l<0 ? l*r : l/r.
 * Presence:   once per unique id in its window, l - p.
 * Frequency:  l - f*count, count = occurrences in its window.
 * Ids outside [0, V) are ignored.  All arithmetic is float32. */
static void who_penalize(float* l, int V, const int32_t* h, int len, const who_params* p,
                         int32_t* cnt /* V scratch, zeroed on entry and exit */) {
  if (p->repetition_penalty != 0.0f) {
    int w = who_window(p->repetition_context, len);
    for (int j = len - w; j < len; ++j) {
      int t = h[j];
      if (t < 0 || t >= V || cnt[t]) continue;
      cnt[t] = 1;
      float v = l[t];
      l[t] = v < 0.0f ? v * p->repetition_penalty : v / p->repetition_penalty;
    }
    for (int j = len - w; j < len; ++j) if (h[j] >= 0 && h[j] < V) cnt[h[j]] = 0;
  }
  if (p->presence_penalty != 0.0f) {
    int w = who_window(p->presence_context, len);
    for (int j = len - w; j < len; ++j) {
      int t = h[j];
      if (t < 0 || t >= V || cnt[t]) continue;
      cnt[t] = 1;
      l[t] = l[t] - p->presence_penalty;
    }
    for (int j = len - w; j < len; ++j) if (h[j] >= 0 && h[j] < V) cnt[h[j]] = 0;
  }
  if (p->frequency_penalty != 0.0f) {
    int w = who_window(p->frequency_context, len);
    for (int j = len - w; j < len; ++j) if (h[j] >= 0 && h[j] < V) cnt[h[j]]++;
    for (int j = len - w; j < len; ++j) {
      int t = h[j];
      if (t < 0 || t >= V || cnt[t] == 0) continue;
      l[t] = l[t] - p->frequency_penalty * (float)cnt[t];
      cnt[t] = 0;
    }
  }
}

void who_penalize_rows(float* logits, int B, int V, long ld, const int32_t* hist, long hist_ld,
                       const int32_t* hist_len, const who_params* params) {
  int32_t* cnt = (int32_t*)calloc((size_t)V, sizeof(int32_t));
  for (int b = 0; b < B; ++b)
    who_penalize(logits + (long)b * ld, V, hist ? hist + (long)b * hist_ld : NULL,
                 hist ? hist_len[b] : 0, &params[b], cnt);
  free(cnt);
}

/* ------------------------------------------------------------------------ */
/* Contract sampler.                                                         */
/* ------------------------------------------------------------------------ */
static __thread const float* g_sort_vals; /* per OpenMP thread */
/* (value desc, id asc); -0.0 == +0.0 as in float comparison. */
static int who_cmp_desc_idasc(const void* a, const void* b) {
  int i = *(const int*)a, j = *(const int*)b;
  float x = g_sort_vals[i], y = g_sort_vals[j];
  if (x > y) return -1;
  if (x < y) return 1;
  return (i > j) - (i < j);
}

typedef struct {
  int V;
  float* l;
  int* ord;      /* (value desc, id asc) */
  uint8_t* alive;
  uint64_t* w;   /* contract mass exp_fix44(l - m) */
  uint64_t* vw;  /* draw weights */
  int32_t* cnt;
} who_ws;

static int who_ws_init(who_ws* ws, int V) {
  ws->V = V;
  ws->l = (float*)malloc(sizeof(float) * V);
  ws->ord = (int*)malloc(sizeof(int) * V);
  ws->alive = (uint8_t*)malloc(V);
  ws->w = (uint64_t*)malloc(sizeof(uint64_t) * V);
  ws->vw = (uint64_t*)malloc(sizeof(uint64_t) * V);
  ws->cnt = (int32_t*)calloc(V, sizeof(int32_t));
  return (ws->l && ws->ord && ws->alive && ws->w && ws->vw && ws->cnt) ? 0 : -1;
}
static void who_ws_free(who_ws* ws) {
  free(ws->l); free(ws->ord); free(ws->alive); free(ws->w); free(ws->vw); free(ws->cnt);
}

static int who_argmax(const float* l, int V) {
  int best = 0;
  for (int i = 1; i < V; ++i) if (l[i] > l[best]) best = i;
  return best;
}

/* Sort indices by (value desc, id asc).  qsort is not stable but the
 * comparator is total, so the order is unique. */
static void who_sort_desc(const float* l, int* ord, int V) {
  for (int i = 0; i < V; ++i) ord[i] = i;
  g_sort_vals = l;
  qsort(ord, V, sizeof(int), who_cmp_desc_idasc);
}

/* top-k over alive entries in (value desc, id asc) order. */
static void who_top_k(who_ws* ws, int k) {
  int seen = 0;
  for (int j = 0; j < ws->V; ++j) {
    int i = ws->ord[j];
    if (!ws->alive[i]) continue;
    if (seen < k) seen++; else ws->alive[i] = 0;
  }
}

/* top-p: walk alive entries in (value desc, id desc) order -- the reverse of
 * an ascending stable argsort -- keeping i iff S - head_excl(i) > theta * Z,
 * where S is the alive mass and Z the mass of the full row (the row was
 * normalised before any filter).  Equal values form groups; inside a group
 * higher ids come first. */
static void who_top_p(who_ws* ws, float theta, uint64_t Z) {
  uint64_t S = 0;
  for (int i = 0; i < ws->V; ++i) if (ws->alive[i]) S += ws->w[i];
  uint64_t head = 0;
  int j = 0;
  while (j < ws->V) {
    int g = j;
    float v = ws->l[ws->ord[j]];
    while (g < ws->V && ws->l[ws->ord[g]] == v) g++;
    for (int q = g - 1; q >= j; --q) { /* id desc inside the group */
      int i = ws->ord[q];
      if (!ws->alive[i]) continue;
      int keep = who_gt_theta(S - head, theta, Z);
      head += ws->w[i];
      if (!keep) ws->alive[i] = 0;
    }
    j = g;
  }
}

/* min-p: keep alive i iff l_i >= fl(max_alive + fl32(ln min_p)). */
static void who_min_p(who_ws* ws, double min_p) {
  float mx = -INFINITY;
  for (int i = 0; i < ws->V; ++i) if (ws->alive[i] && ws->l[i] > mx) mx = ws->l[i];
  float c = (float)log(min_p);
  float thr = mx + c;
  for (int i = 0; i < ws->V; ++i) if (ws->alive[i] && !(ws->l[i] >= thr)) ws->alive[i] = 0;
}

/* The chain's float32 temperature scalings (reference: logits * (1/temp) in
 * make_sampler; logprobs / max(temperature, 1e-5) in sampling_logprobs). */
static float who_scale(int chain, float d, double temperature) {
  if (chain == WHO_CHAIN_KPM) return d * (float)(1.0 / temperature);
  return d / (float)fmax(temperature, 1e-5);
}

/* Validate the same ranges mlx_lm / Whallm reject. */
static int who_check(const who_params* p, int V) {
  if (p->chain != WHO_CHAIN_KPM && p->chain != WHO_CHAIN_PMK) return WHO_EINVAL;
  if (!(p->temperature >= 0.0)) return WHO_EINVAL;
  if (!(p->min_p >= 0.0 && p->min_p <= 1.0)) return WHO_EINVAL;
  if (p->repetition_penalty < 0.0f) return WHO_EINVAL;
  if (p->chain == WHO_CHAIN_KPM && p->temperature > 0.0 && p->top_k > 0 && p->top_k >= V) return WHO_EINVAL;
  if (p->top_k < 0) return WHO_EINVAL;
  return WHO_OK;
}

/* One row of the contract.  Returns the token; *kept gets |kept set|.
 * out_row (chain B only, nullable) receives the sampling_logprobs row. */
static int who_contract_row(who_ws* ws, const float* x, const int32_t* h, int hlen,
                            const who_params* p, float u, int32_t* kept_out, float* out_row) {
  int V = ws->V;
  float* l = ws->l;
  for (int i = 0; i < V; ++i) l[i] = x[i] + 0.0f; /* -0 -> +0 */
  who_penalize(l, V, h, hlen, p, ws->cnt);
  for (int i = 0; i < V; ++i) l[i] = l[i] + 0.0f;
  if (p->temperature == 0.0) {
    if (kept_out) *kept_out = 1;
    if (out_row) memcpy(out_row, l, sizeof(float) * V);
    return who_argmax(l, V);
  }
  float m = l[who_argmax(l, V)];
  uint64_t Z = 0;
  for (int i = 0; i < V; ++i) {
    ws->w[i] = (m == -INFINITY) ? 0 : who_exp_fix44(l[i] - m);
    Z += ws->w[i];
    ws->alive[i] = 1;
  }
  who_sort_desc(l, ws->ord, V);
  float theta = (float)(1.0 - p->top_p);
  int use_k = p->top_k > 0 && p->top_k < V;
  int use_p = p->top_p > 0.0 && p->top_p < 1.0;
  int use_m = p->min_p != 0.0;
  if (p->chain == WHO_CHAIN_KPM) {
    if (use_k) who_top_k(ws, p->top_k);
    if (use_p) who_top_p(ws, theta, Z);
    if (use_m) who_min_p(ws, p->min_p);
  } else {
    if (use_p) who_top_p(ws, theta, Z);
    if (use_m) who_min_p(ws, p->min_p);
    if (use_k) who_top_k(ws, p->top_k);
  }
  uint64_t ZV = 0;
  int nkept = 0;
  for (int i = 0; i < V; ++i) {
    ws->vw[i] = 0;
    if (!ws->alive[i]) continue;
    nkept++;
    ws->vw[i] = who_exp_fix44(who_scale(p->chain, l[i] - m, p->temperature));
    ZV += ws->vw[i];
  }
  if (kept_out) *kept_out = nkept;
  if (out_row) {
    double lz = log(ldexp((double)ZV, -44));
    for (int i = 0; i < V; ++i)
      out_row[i] = ws->alive[i] ? (float)((double)who_scale(p->chain, l[i] - m, p->temperature) - lz)
                                : -INFINITY;
  }
  if (nkept == 0 || ZV == 0) return 0; /* argmax of an all -inf row is index 0 */
  return who_locate(ws->vw, NULL, V, ZV, u);
}

/* Batched contract sampler.  logits: B rows of V float32 with row stride ld.
 * hist: B rows of token ids with stride hist_ld, lengths hist_len (hist may
 * be NULL).  params: B entries.  u: B uniforms.  tokens/kept: B outputs.
 * out_rows: nullable B x V (chain B logprob rows). */
int who_sample_rows(const float* logits, int B, int V, long ld, const int32_t* hist, long hist_ld,
                    const int32_t* hist_len, const who_params* params, const float* u,
                    int32_t* tokens, int32_t* kept, float* out_rows, int nthreads) {
  if (B < 0 || V <= 0 || V > (1 << 18)) return WHO_EINVAL;
  for (int b = 0; b < B; ++b) if (who_check(&params[b], V)) return WHO_EINVAL;
  int err = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
  {
    who_ws ws;
    if (who_ws_init(&ws, V)) {
#pragma omp atomic write
      err = WHO_ENOMEM;
    } else {
#pragma omp for schedule(dynamic, 1)
      for (int b = 0; b < B; ++b) {
        tokens[b] = who_contract_row(&ws, logits + (long)b * ld, hist ? hist + (long)b * hist_ld : NULL,
                                     hist ? hist_len[b] : 0, &params[b], u[b], kept ? &kept[b] : NULL,
                                     out_rows ? out_rows + (long)b * V : NULL);
      }
    }
    who_ws_free(&ws);
  }
  return err;
}

/* ------------------------------------------------------------------------ */
/* Contract verifier (dspark.py:857-898).                                    */
/* ------------------------------------------------------------------------ */
/* reject iff u > min(1, exp(g - d)): with r = exp_fix44(fl(g - d)) / 2^44.
 * g - d >= 0 (ratio 1) and NaN (both -inf) accept, as comparisons with the
 * reference's float ratio do. */
static int who_reject_lp(float u, float g, float d) {
  float diff = g - d;
  if (diff != diff) return 0;
  if (diff >= 0.0f) return 0;
  uint64_t R = who_exp_fix44(diff);
  return (double)u * 17592186044416.0 > (double)R; /* u * 2^44 is exact */
}

/* Draw from a logprob row with weights exp_fix44(r - max r). */
static int who_draw_lp_row(const float* r, int V, float u, uint64_t* w) {
  float m = r[who_argmax(r, V)];
  uint64_t Z = 0;
  for (int i = 0; i < V; ++i) { w[i] = m == -INFINITY ? 0 : who_exp_fix44(r[i] - m); Z += w[i]; }
  if (Z == 0) return 0;
  return who_locate(w, NULL, V, Z, u);
}

/* Verifier over logprob rows, the reference's own input form.
 * draft_lp: B x n x V, target_lp: B x (n+1) x V, draft_tok: B x n,
 * u: B x (n+1) (u[:, j<n] accept tests, u[:, n] the final draw).
 * Outputs accepted[B], token[B]; residual_rows (nullable, B x V) receives
 * the returned row (log(d/sum d), the target row, or the bonus row). */
int who_verify_logprobs(const float* draft_lp, const float* target_lp, const int32_t* draft_tok,
                        const float* u, int B, int n, int V, float temperature,
                        int32_t* accepted, int32_t* token, float* rows, int nthreads) {
  if (B < 0 || n < 0 || V <= 0 || V > (1 << 18)) return WHO_EINVAL;
  int err = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
  {
    uint64_t* w = (uint64_t*)malloc(sizeof(uint64_t) * V);
    if (!w) {
#pragma omp atomic write
      err = WHO_ENOMEM;
    } else {
#pragma omp for schedule(dynamic, 1)
      for (int b = 0; b < B; ++b) {
        const float* T = target_lp + (long)b * (n + 1) * V;
        const float* D = draft_lp + (long)b * n * V;
        const int32_t* t = draft_tok + (long)b * n;
        const float* ub = u + (long)b * (n + 1);
        float* row = rows ? rows + (long)b * V : NULL;
        int j = 0;
        if (temperature == 0.0f) {
          for (j = 0; j < n; ++j) if (t[j] != who_argmax(T + (long)j * V, V)) break;
          accepted[b] = j;
          token[b] = who_argmax(T + (long)j * V, V);
          if (row) memcpy(row, T + (long)j * V, sizeof(float) * V);
          continue;
        }
        for (j = 0; j < n; ++j) {
          int tok = t[j];
          if (tok < 0 || tok >= V) break; /* invalid draft id: reject */
          if (who_reject_lp(ub[j], T[(long)j * V + tok], D[(long)j * V + tok])) break;
        }
        accepted[b] = j;
        if (j == n) {
          token[b] = who_draw_lp_row(T + (long)n * V, V, ub[n], w);
          if (row) memcpy(row, T + (long)n * V, sizeof(float) * V);
          continue;
        }
        const float* g = T + (long)j * V;
        const float* d = D + (long)j * V;
        uint64_t S = 0;
        for (int i = 0; i < V; ++i) {
          uint64_t P = who_exp_fix44(g[i]), Q = who_exp_fix44(d[i]);
          w[i] = P > Q ? P - Q : 0;
          S += w[i];
        }
        if (S > 0) {
          token[b] = who_locate(w, NULL, V, S, ub[n]);
          if (row) {
            double ls = log((double)S);
            for (int i = 0; i < V; ++i) row[i] = w[i] ? (float)(log((double)w[i]) - ls) : -INFINITY;
          }
        } else {
          token[b] = who_draw_lp_row(g, V, ub[n], w);
          if (row) memcpy(row, g, sizeof(float) * V);
        }
      }
    }
    free(w);
  }
  return err;
}

/* floor(q * Z) exactly, q float32 >= 0, Z < 2^63. */
static uint64_t who_floor_qz(float q, uint64_t Z) {
  if (!(q > 0.0f)) return 0;
  if (q > 1.0f) q = 1.0f;
  int e;
  float fr = frexpf(q, &e);
  uint64_t M = (uint64_t)ldexpf(fr, 24);
  int s = 24 - e; /* q = M / 2^s */
  u128 prod = (u128)M * Z;
  if (s <= 0) { /* q >= 2^24: saturate */
    return ~0ull;
  }
  u128 F = s >= 128 ? 0 : (prod >> s);
  return F > (u128)(~0ull) ? ~0ull : (uint64_t)F;
}

/* reject iff u * q * Z > W, exactly (u, q float32, Z, W integers). */
static int who_reject_fused(float u, float q, uint64_t Z, uint64_t W) {
  if (!(u > 0.0f) || !(q > 0.0f)) return 0;
  if (q > 1.0f) q = 1.0f;
  int eu, eq;
  float fu = frexpf(u, &eu), fq = frexpf(q, &eq);
  uint64_t Mu = (uint64_t)ldexpf(fu, 24), Mq = (uint64_t)ldexpf(fq, 24);
  int s = 48 - eu - eq; /* u*q = Mu*Mq / 2^s, s >= 48 for u < 1, q <= 1 */
  u128 prod = (u128)(Mu * Mq) * (u128)Z; /* < 2^48 * 2^63 = 2^111 */
  /* compare prod / 2^s > W  <=>  prod > W * 2^s  (W < 2^46) */
  if (s >= 128) return 0;
  if (W == 0) return prod > 0;
  int wbits = 64 - __builtin_clzll(W);
  if (wbits + s > 127) return 0; /* W * 2^s >= 2^127 > prod */
  return prod > ((u128)W << s);
}

/* Fused verifier (configuration c3 form): target logits x (B x (n+1) x V)
 * tempered inside (p = softmax(x / T), the sampling_logprobs row with no
 * filter), draft probabilities q (B x n x V), draft ids, u (B x (n+1)).
 * Contract: W_i = exp_fix44(fl(fl(x_i - m) / Tc)), Z = sum W, p_i = W_i/Z;
 * reject iff u*q(t)*Z > W_t; residual D_i = max(W_i - floor(q_i Z), 0);
 * draw from D (or from W when sum D == 0) with u[:, n]; bonus draws from
 * W of position n. */
int who_verify_fused(const float* target_logits, const float* draft_q, const int32_t* draft_tok,
                     const float* u, int B, int n, int V, float temperature,
                     int32_t* accepted, int32_t* token, int nthreads) {
  if (B < 0 || n < 0 || V <= 0 || V > (1 << 18)) return WHO_EINVAL;
  int err = 0;
  float Tc = (float)fmax((double)temperature, 1e-5);
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
  {
    uint64_t* w = (uint64_t*)malloc(sizeof(uint64_t) * V);
    uint64_t* dd = (uint64_t*)malloc(sizeof(uint64_t) * V);
    if (!w || !dd) {
#pragma omp atomic write
      err = WHO_ENOMEM;
    } else {
#pragma omp for schedule(dynamic, 1)
      for (int b = 0; b < B; ++b) {
        const float* X = target_logits + (long)b * (n + 1) * V;
        const float* Q = draft_q + (long)b * n * V;
        const int32_t* t = draft_tok + (long)b * n;
        const float* ub = u + (long)b * (n + 1);
        int j;
        if (temperature == 0.0f) {
          for (j = 0; j < n; ++j) if (t[j] != who_argmax(X + (long)j * V, V)) break;
          accepted[b] = j;
          token[b] = who_argmax(X + (long)j * V, V);
          continue;
        }
        uint64_t Z = 0;
        for (j = 0; j < n; ++j) {
          const float* x = X + (long)j * V;
          int tok = t[j];
          if (tok < 0 || tok >= V) break;
          float m = x[who_argmax(x, V)];
          Z = 0;
          for (int i = 0; i < V; ++i) { w[i] = who_exp_fix44((x[i] - m) / Tc); Z += w[i]; }
          if (who_reject_fused(ub[j], Q[(long)j * V + tok], Z, w[tok])) break;
        }
        accepted[b] = j;
        const float* x = X + (long)j * V;
        float m = x[who_argmax(x, V)];
        Z = 0;
        for (int i = 0; i < V; ++i) { w[i] = m == -INFINITY ? 0 : who_exp_fix44((x[i] - m) / Tc); Z += w[i]; }
        if (j == n) {
          token[b] = Z ? who_locate(w, NULL, V, Z, ub[n]) : 0;
          continue;
        }
        const float* q = Q + (long)j * V;
        uint64_t S = 0;
        for (int i = 0; i < V; ++i) {
          uint64_t qz = who_floor_qz(q[i], Z);
          dd[i] = w[i] > qz ? w[i] - qz : 0;
          S += dd[i];
        }
        token[b] = S ? who_locate(dd, NULL, V, S, ub[n]) : (Z ? who_locate(w, NULL, V, Z, ub[n]) : 0);
      }
    }
    free(w);
    free(dd);
  }
  return err;
}

/* ------------------------------------------------------------------------ */
/* Faithful float32 restatement (mlx_lm / Whallm op order).                  */
/* ------------------------------------------------------------------------ */
static float who_lse_f32(const float* v, int V) {
  float m = -INFINITY;
  for (int i = 0; i < V; ++i) if (v[i] > m) m = v[i];
  if (m == -INFINITY) return -INFINITY;
  float s = 0.0f;
  for (int i = 0; i < V; ++i) s += expf(v[i] - m);
  return m + logf(s);
}

static __thread const float* g_asc_vals;
/* ascending value, stable (id asc) */
static int who_cmp_asc_stable(const void* a, const void* b) {
  int i = *(const int*)a, j = *(const int*)b;
  float x = g_asc_vals[i], y = g_asc_vals[j];
  if (x < y) return -1;
  if (x > y) return 1;
  return (i > j) - (i < j);
}
/* descending value, stable (id asc): argsort(-v) */
static int who_cmp_desc_stable(const void* a, const void* b) {
  int i = *(const int*)a, j = *(const int*)b;
  float x = g_asc_vals[i], y = g_asc_vals[j];
  if (x > y) return -1;
  if (x < y) return 1;
  return (i > j) - (i < j);
}

/* Inverse-CDF draw from a logprob-like row (entries -inf excluded).  The
 * reference draws by Gumbel-max (mx.random.categorical, dspark.py:329, 904),
 * which has no cumulative sum; a uniform-driven replay needs one, and it is
 * accumulated in float64 over the row's float32 weights expf(z - max) so the
 * draw adds no rounding of its own: a float32 sequential sum over a
 * 129,280-id residual row drifts by ~1e-5, far above the row's own float32
 * rounding. */
static int who_draw_f32(const float* z, int V, float u) {
  float m = -INFINITY;
  for (int i = 0; i < V; ++i) if (z[i] > m) m = z[i];
  if (m == -INFINITY) return 0;
  double tot = 0.0;
  for (int i = 0; i < V; ++i) tot += (double)expf(z[i] - m);
  double tgt = (double)u * tot, c = 0.0;
  int last = 0;
  for (int i = 0; i < V; ++i) {
    float w = expf(z[i] - m);
    if (w == 0.0f) continue;
    c += (double)w;
    last = i;
    if (c > tgt) return i;
  }
  return last;
}

typedef struct {
  float* l;
  float* lp;
  float* pr;
  int* idx;
  int32_t* cnt;
} who_fws;

static int who_faithful_row(who_fws* ws, int V, const float* x, const int32_t* h, int hlen,
                            const who_params* p, float u, int32_t* kept_out, float* out_row) {
  float* l = ws->l;
  float* lp = ws->lp;
  memcpy(l, x, sizeof(float) * V);
  who_penalize(l, V, h, hlen, p, ws->cnt);
  if (p->temperature == 0.0) {
    if (kept_out) *kept_out = 1;
    if (p->chain == WHO_CHAIN_PMK) {
      if (out_row) memcpy(out_row, l, sizeof(float) * V);
      return who_argmax(l, V);
    }
    float lse = who_lse_f32(l, V);
    for (int i = 0; i < V; ++i) lp[i] = l[i] - lse;
    return who_argmax(lp, V);
  }
  float lse = who_lse_f32(l, V);
  for (int i = 0; i < V; ++i) lp[i] = l[i] - lse;
  int use_k = p->top_k > 0 && p->top_k < V;
  int use_p = p->top_p > 0.0 && p->top_p < 1.0;
  int use_m = p->min_p != 0.0;
  float theta = (float)(1.0 - p->top_p);
  float cmin = (float)log(p->min_p);
  for (int s = 0; s < 3; ++s) {
    int step = p->chain == WHO_CHAIN_KPM ? s : (s + 1) % 3; /* KPM: k,p,m ; PMK: p,m,k */
    if (step == 0 && use_k) {
      for (int i = 0; i < V; ++i) ws->idx[i] = i;
      g_asc_vals = lp;
      qsort(ws->idx, V, sizeof(int), who_cmp_desc_stable);
      for (int j = p->top_k; j < V; ++j) lp[ws->idx[j]] = -INFINITY;
    } else if (step == 1 && use_p) {
      for (int i = 0; i < V; ++i) { ws->pr[i] = expf(lp[i]); ws->idx[i] = i; }
      g_asc_vals = lp;
      qsort(ws->idx, V, sizeof(int), who_cmp_asc_stable);
      float c = 0.0f;
      for (int j = 0; j < V; ++j) {
        int i = ws->idx[j];
        c += ws->pr[i];
        if (!(c > theta)) lp[i] = -INFINITY;
      }
    } else if (step == 2 && use_m) {
      for (int i = 0; i < V; ++i) ws->idx[i] = i;
      g_asc_vals = lp;
      qsort(ws->idx, V, sizeof(int), who_cmp_desc_stable);
      float thr = lp[ws->idx[0]] + cmin;
      for (int j = 1; j < V; ++j) if (lp[ws->idx[j]] < thr) lp[ws->idx[j]] = -INFINITY;
    }
  }
  int nk = 0;
  for (int i = 0; i < V; ++i) nk += lp[i] != -INFINITY;
  if (kept_out) *kept_out = nk;
  if (p->chain == WHO_CHAIN_KPM) {
    float inv = (float)(1.0 / p->temperature);
    for (int i = 0; i < V; ++i) lp[i] = lp[i] * inv;
    return who_draw_f32(lp, V, u);
  }
  float Tc = (float)fmax(p->temperature, 1e-5);
  for (int i = 0; i < V; ++i) lp[i] = lp[i] / Tc;
  float l2 = who_lse_f32(lp, V);
  for (int i = 0; i < V; ++i) lp[i] = lp[i] - l2;
  if (out_row) memcpy(out_row, lp, sizeof(float) * V);
  return who_draw_f32(lp, V, u);
}

int who_sample_rows_faithful(const float* logits, int B, int V, long ld, const int32_t* hist, long hist_ld,
                             const int32_t* hist_len, const who_params* params, const float* u,
                             int32_t* tokens, int32_t* kept, float* out_rows, int nthreads) {
  if (B < 0 || V <= 0) return WHO_EINVAL;
  for (int b = 0; b < B; ++b) if (who_check(&params[b], V)) return WHO_EINVAL;
  int err = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
  {
    who_fws ws;
    ws.l = (float*)malloc(sizeof(float) * V);
    ws.lp = (float*)malloc(sizeof(float) * V);
    ws.pr = (float*)malloc(sizeof(float) * V);
    ws.idx = (int*)malloc(sizeof(int) * V);
    ws.cnt = (int32_t*)calloc(V, sizeof(int32_t));
    if (!ws.l || !ws.lp || !ws.pr || !ws.idx || !ws.cnt) {
#pragma omp atomic write
      err = WHO_ENOMEM;
    } else {
#pragma omp for schedule(dynamic, 1)
      for (int b = 0; b < B; ++b)
        tokens[b] = who_faithful_row(&ws, V, logits + (long)b * ld, hist ? hist + (long)b * hist_ld : NULL,
                                     hist ? hist_len[b] : 0, &params[b], u[b], kept ? &kept[b] : NULL,
                                     out_rows ? out_rows + (long)b * V : NULL);
    }
    free(ws.l); free(ws.lp); free(ws.pr); free(ws.idx); free(ws.cnt);
  }
  return err;
}

/* Faithful verifier on logprob rows (dspark.py:857-898 in float32). */
int who_verify_faithful(const float* draft_lp, const float* target_lp, const int32_t* draft_tok,
                        const float* u, int B, int n, int V, float temperature,
                        int32_t* accepted, int32_t* token, int nthreads) {
  int err = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
  {
    float* c = (float*)malloc(sizeof(float) * V);
    if (!c) {
#pragma omp atomic write
      err = WHO_ENOMEM;
    } else {
#pragma omp for schedule(dynamic, 1)
      for (int b = 0; b < B; ++b) {
        const float* T = target_lp + (long)b * (n + 1) * V;
        const float* D = draft_lp + (long)b * n * V;
        const int32_t* t = draft_tok + (long)b * n;
        const float* ub = u + (long)b * (n + 1);
        int j;
        if (temperature == 0.0f) {
          for (j = 0; j < n; ++j) if (t[j] != who_argmax(T + (long)j * V, V)) break;
          accepted[b] = j;
          token[b] = who_argmax(T + (long)j * V, V);
          continue;
        }
        for (j = 0; j < n; ++j) {
          int tok = t[j];
          float pr = fminf(1.0f, expf(T[(long)j * V + tok] - D[(long)j * V + tok]));
          if (ub[j] > pr) break;
        }
        accepted[b] = j;
        if (j == n) { token[b] = who_draw_f32(T + (long)n * V, V, ub[n]); continue; }
        const float* g = T + (long)j * V;
        const float* d = D + (long)j * V;
        float tot = 0.0f;
        for (int i = 0; i < V; ++i) { c[i] = fmaxf(expf(g[i]) - expf(d[i]), 0.0f); tot += c[i]; }
        if (tot > 0.0f) {
          for (int i = 0; i < V; ++i) c[i] = logf(c[i] / tot);
          token[b] = who_draw_f32(c, V, ub[n]);
        } else {
          token[b] = who_draw_f32(g, V, ub[n]);
        }
      }
    }
    free(c);
  }
  return err;
}

/* Contract building blocks exported for tests. */
int who_gt_theta_export(uint64_t A, float theta, uint64_t Z) { return who_gt_theta(A, theta, Z); }
uint64_t who_floor_qz_export(float q, uint64_t Z) { return who_floor_qz(q, Z); }
int who_reject_fused_export(float u, float q, uint64_t Z, uint64_t W) { return who_reject_fused(u, q, Z, W); }
int who_reject_lp_export(float u, float g, float d) { return who_reject_lp(u, g, d); }

/* Batched contract exponential for tests. */
void who_exp_fix44_batch(const float* d, uint64_t* out, long n) {
  for (long i = 0; i < n; ++i) out[i] = who_exp_fix44(d[i]);
}
