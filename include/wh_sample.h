/*
 * wh_sample.h -- C ABI of the MI355X (gfx950) token-selection library
 * (libwh_sample.so).  Plain pointers and sizes only; every pointer named
 * "device" is HIP device memory; `stream` is a hipStream_t (NULL = the
 * default stream).  All entry points are asynchronous and stream ordered:
 * they validate host-side arguments, enqueue kernels and return; nothing
 * blocks on the device.  Status: 0 on success, a negative WH_E* code on
 * failure, with a message from wh_last_error() (thread local).
 *
 * The reference exposes this path as Python function objects over MLX arrays,
 * with no FFI; each entry point below replaces one of them:
 *
 *   wh_sample               mlx_lm make_sampler(temp, top_p, top_k, min_p)
 *                           + make_logits_processors(...), as called at
 *                           runtime/deepseek_v4_ssd/generation.py:1279-1293 and
 *                           driven per token by mlx_lm generate_step
 *                           (generation.py:1465-1475); chain WH_CHAIN_WHALLM is
 *                           sampling_logprobs + _sample
 *                           (runtime/deepseek_v4_ssd/dspark.py:358-375, 901-904),
 *                           with penalties first as in qwen4_exp.py:949-958.
 *   wh_apply_penalties      the processors returned by make_logits_processors
 *                           (generation.py:1286-1293), applied in place.
 *   wh_verify_logprobs      _verify(draft, target_logprobs, temperature)
 *                           (runtime/deepseek_v4_ssd/dspark.py:857-898).
 *   wh_verify_fused         _verify fused with the target rows'
 *                           sampling_logprobs(logits, T, top_p=1)
 *                           (dspark.py:663-670): target logits in, draft
 *                           probabilities q in.
 *   wh_markov_logits        one DSpark draft position's logits:
 *                           base_logits[:, position] + markov_head(previous)
 *                           (dspark.py:157-165, 319-324;
 *                           deepseek_v41/dspark.py:131-133), with `previous`
 *                           read from device memory.
 *   wh_top_logprobs         the n most likely entries of mlx_lm's per-step
 *                           logprobs = logits - logsumexp(logits)
 *                           (generation.py:1465-1475) and the chosen token's,
 *                           for the OpenAI `logprobs` / `top_logprobs` fields
 *                           that runtime/deepseek_v4_ssd/server.py:1110-1111
 *                           rejects today.
 *   wh_history_append       the per-step history extension the logits
 *                           processors read: mlx_lm generate_step's
 *                           `tokens = concat([tokens, y])` and the MTP loop's
 *                           sampling_tokens.append (qwen4_exp.py:1143-1149),
 *                           on a device buffer.
 *   wh_lmhead_logits        the LM head that produces the logits:
 *                           model.lm_head(hidden) (model.py:716,
 *                           dspark.py:313, qwen4_exp.py:960-961), bf16 MFMA.
 *   wh_lmhead_greedy        the LM head fused with greedy selection (argmax,
 *                           lowest index among equal maxima; make_sampler at
 *                           temp 0, dspark.py:326): the logits never reach
 *                           memory.
 *   wh_lmhead_sample        the LM head, then wh_sample on its logits; for
 *                           rows filtered by top-p alone or not at all (the
 *                           reference's defaults, generation.py:109-118),
 *                           the product's epilogue also emits the per-slice
 *                           maxima the sampler's first step would compute.
 *
 * Random numbers: the reference draws from MLX's global PRNG
 * (mx.random.categorical / uniform, dspark.py:329, 884, 904).  This library
 * has no RNG: callers pass one uniform in [0,1) per draw, and the draw is the
 * inverse CDF in vocabulary order over fixed-point weights.
 */
#ifndef WH_SAMPLE_H
#define WH_SAMPLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WH_OK 0
#define WH_EINVAL -1   /* invalid argument (the reference raises ValueError) */
#define WH_EHIP -2     /* a HIP runtime call failed */
#define WH_ELIMIT -3   /* a documented size limit was exceeded */

#define WH_DTYPE_F32 0
#define WH_DTYPE_BF16 1

/* Filter order.  MLX: mlx_lm make_sampler -- top_k -> top_p -> min_p on the
 * T=1 logprobs, then categorical(logprobs * (1/T)).  WHALLM: Whallm
 * sampling_logprobs -- top_p -> min_p -> top_k, then logprobs / max(T, 1e-5),
 * renormalised. */
#define WH_CHAIN_MLX 0
#define WH_CHAIN_WHALLM 1

#define WH_OUT_LOGPROBS 0
#define WH_OUT_MASKED 1

#define WH_MAX_VOCAB 262144      /* V <= 2^18 keeps fixed-point sums below 2^62 */
#define WH_MAX_WINDOW 4096       /* penalty window entries per row */
#define WH_MAX_TOP_LOGPROBS 64   /* n of wh_top_logprobs */
#define WH_LMHEAD_MAX_ROWS 64    /* M of the LM-head entry points */

typedef struct wh_sample_args {
  const void* logits;        /* device, B rows of V values (dtype), row stride in elements;
                                no NaN (entries may be -inf) */
  int32_t dtype;             /* WH_DTYPE_F32 or WH_DTYPE_BF16 (widened exactly to float32) */
  int32_t B;
  int32_t V;
  int32_t chain;             /* WH_CHAIN_MLX or WH_CHAIN_WHALLM */
  int64_t row_stride;

  const int32_t* history;    /* device, nullable: B rows of token ids, stride history_stride */
  int64_t history_stride;
  const int32_t* history_len;/* device, [B]; required with history */

  const float* uniforms;     /* device, [B] in [0,1); nullable only when tokens is NULL */

  /* Scalar parameters, overridden per row where the matching *_rows pointer
   * is non-NULL.  temperature, top_p and min_p are doubles: the reference's
   * callers pass Python floats, and the float32 constants the filters use are
   * derived from them as MLX derives them -- fp32(1 - top_p), fp32(1 / T),
   * fp32(max(T, 1e-5)), fp32(ln min_p) -- so a value such as top_p = 0.9
   * gives the same threshold (0.1f) as the reference, not fp32(1 - fp32(0.9)). */
  double temperature;
  double top_p;
  double min_p;
  int32_t top_k;
  int32_t history_share;     /* logits rows per history row: row b reads history row
                                b / history_share (0 and 1: one history row each).
                                MTP verification (qwen4_exp.py:1083-1092) penalises
                                position i of a batch entry over history + drafts[:i]:
                                its n+1 rows share one history row holding the
                                committed ids followed by the drafts, with
                                history_len = committed + i per row. */
  const double* temperature_rows; /* device, nullable */
  const double* top_p_rows;       /* device, nullable */
  const double* min_p_rows;       /* device, nullable */
  const int32_t* top_k_rows;      /* device, nullable; k >= V is a no-op */

  float repetition_penalty;  /* 0 = processor absent (1.0 is a no-op) */
  float presence_penalty;    /* 0 = absent */
  float frequency_penalty;   /* 0 = absent */
  int32_t repetition_context;/* window of the last N history ids; 0 = whole history */
  int32_t presence_context;
  int32_t frequency_context;

  int32_t* tokens;           /* device, [B] out; nullable when only logprobs_out is wanted */
  int32_t* kept_count;       /* device, [B] out, nullable: size of the kept set */
  float* logprobs_out;       /* device, [B, V] out, nullable; see out_mode */
  int32_t out_mode;          /* WH_OUT_LOGPROBS: sampling_logprobs row (WHALLM chain only);
                                WH_OUT_MASKED: the (penalised) input row with filtered-out
                                entries set to -inf, no temperature (mlx_lm apply_top_k /
                                apply_top_p / apply_min_p) */
  int32_t reserved;
  void* workspace;           /* device, wh_sample_workspace_bytes(B, V) bytes, contents need
                                no initialisation.  One workspace per stream: calls that
                                overlap on one workspace race.  NULL selects the slower
                                multi-pass engine, which needs none. */
  size_t workspace_bytes;
} wh_sample_args;

/* Workspace needed by wh_sample for B rows of V entries. */
size_t wh_sample_workspace_bytes(int32_t B, int32_t V);
int wh_sample(const wh_sample_args* args, void* stream);

/* wh_sample without a workspace and without any allocation.  No counterpart
 * in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The fast engine's scratch (slice headers and candidates) is a
 * library-owned device array of WH_NOALLOC_SCRATCH_BYTES on each GPU the
 * library runs on, resolved on the first call on that GPU and held until the
 * process ends; args->workspace and workspace_bytes are ignored.  Calls whose
 * wh_sample_workspace_bytes(B, V) exceeds the array are rejected with
 * WH_ELIMIT.  Every call on one GPU shares the array: calls that overlap on
 * one GPU (two streams, two threads) race, as two calls on one workspace do.
 * The stream's device must be the current device.  Results are those of
 * wh_sample. */
#define WH_NOALLOC_SCRATCH_BYTES (32u << 20)
int wh_sample_noalloc(const wh_sample_args* args, void* stream);

/* Penalty processors only, in place on float32 or bf16 logits (bf16 results
 * are rounded to nearest even).  Uses the history/penalty fields of args. */
int wh_apply_penalties(const wh_sample_args* args, void* stream);

typedef struct wh_verify_args {
  int32_t B;
  int32_t n;                 /* draft length; target has n+1 rows per batch entry */
  int32_t V;
  float temperature;
  const float* target;       /* device, [B, n+1, V]: logprob rows (wh_verify_logprobs)
                                or raw logits (wh_verify_fused) */
  const float* draft;        /* device, [B, n, V]: logprob rows (wh_verify_logprobs)
                                or probabilities q (wh_verify_fused) */
  const int32_t* draft_tokens; /* device, [B, n] */
  const float* uniforms;     /* device, [B, n+1]: [:, j<n] accept tests, [:, n] final draw */
  int32_t* accepted;         /* device, [B] out */
  int32_t* token;            /* device, [B] out */
  float* row_out;            /* device, [B, V] out, nullable (logprob form only) */
  void* workspace;           /* device, wh_verify_workspace_bytes(...) bytes */
  size_t workspace_bytes;
} wh_verify_args;

size_t wh_verify_workspace_bytes(int32_t B, int32_t n, int32_t V);
int wh_verify_logprobs(const wh_verify_args* args, void* stream);
int wh_verify_fused(const wh_verify_args* args, void* stream);

/* One DSpark draft position (dspark.py:319-324):
 *   logits_out = base + markov_w2 @ float32(markov_w1[*prev])
 * markov_w1 is the Markov head's embedding [V, rank] and markov_w2 its
 * output projection's weight [V, rank] (nn.Linear(rank, V)), both float32 or
 * bf16.  *prev is read on the device (clamped to [0, V)), so the previous
 * position's wh_sample token feeds the next position with no host sync.  The
 * float32 sum is formed in a fixed order (8-entry fused multiply-add chains,
 * then a 32-way butterfly), which the CPU oracle reproduces bit for bit; the
 * reference's order (an MLX matrix-vector product) is unspecified. */
typedef struct wh_markov_args {
  const float* base;         /* device, [V] float32: base_logits[0, position] */
  const void* embed;         /* device, [V, rank] markov_w1 weight, 16-byte aligned */
  const void* proj;          /* device, [V, rank] markov_w2 weight, 16-byte aligned */
  int32_t dtype;             /* WH_DTYPE_F32 or WH_DTYPE_BF16 (both weights) */
  int32_t V;
  int32_t rank;              /* a multiple of 8, at most 256 */
  int32_t reserved;
  const int32_t* prev;       /* device, [1]: the previous token */
  float* logits_out;         /* device, [V] float32 */
} wh_markov_args;
int wh_markov_logits(const wh_markov_args* args, void* stream);

/* Top-n logprobs of B logit rows: logprob = float32(double(l) - lse) with
 * lse = logsumexp(row) in float64; the n entries in order of value
 * descending, lower ids first among equal values; -inf entries rank last and
 * a row of all -inf gives -inf logprobs.  Pass the row the caller's logprobs
 * are defined on (mlx_lm: the logits after the logits processors, before
 * temperature).  With `token`, token_logprob[b] is row b's logprob of
 * token[b] (-inf for an id outside [0, V)).  Inputs must hold no NaN. */
typedef struct wh_top_logprobs_args {
  const void* logits;        /* device, B rows of V (row_stride apart) */
  int32_t dtype;             /* WH_DTYPE_F32 or WH_DTYPE_BF16 */
  int32_t B;
  int32_t V;                 /* 1 .. WH_MAX_VOCAB */
  int32_t n;                 /* 1 .. min(V, WH_MAX_TOP_LOGPROBS) */
  int64_t row_stride;        /* elements, >= V */
  const int32_t* token;      /* device, [B], nullable */
  int32_t* top_ids;          /* device, [B, n] */
  float* top_logprobs;       /* device, [B, n] */
  float* token_logprob;      /* device, [B], nullable (needs token) */
  void* workspace;           /* device, 16-byte aligned,
                                wh_top_logprobs_workspace_bytes(B, V, n) bytes */
  size_t workspace_bytes;
} wh_top_logprobs_args;
size_t wh_top_logprobs_workspace_bytes(int32_t B, int32_t V, int32_t n);
int wh_top_logprobs(const wh_top_logprobs_args* args, void* stream);

/* Append ids to B device-resident histories (the [B, capacity] buffer and
 * lengths wh_sample reads as history / history_len).  Row b receives
 * tokens[b, 0 .. counts[b]) (all m without counts), then tail[b] if tail is
 * given -- the MTP commit: accepted drafts, then the verifier's next token.
 * A row that would exceed capacity first keeps only its last `keep` ids,
 * moved to the front; keep must cover every penalty context in use (a
 * context of 0, the whole history, needs a capacity that never fills).
 * Requires keep + m (+1 with tail) <= capacity.  Lengths outside
 * [0, capacity] are clamped. */
typedef struct wh_history_args {
  int32_t* history;          /* device, [B, history_stride] */
  int64_t history_stride;    /* elements, >= capacity */
  int32_t* history_len;      /* device, [B], read and updated */
  int32_t B;
  int32_t capacity;
  int32_t keep;              /* 0 .. WH_MAX_WINDOW */
  int32_t m;                 /* ids per row in tokens */
  const int32_t* tokens;     /* device, [B, m] */
  const int32_t* counts;     /* device, [B], nullable: ids to take per row (clamped to [0, m]) */
  const int32_t* tail;       /* device, [B], nullable */
} wh_history_args;
int wh_history_append(const wh_history_args* args, void* stream);

/* LM head: logits[m, v] = sum_k x[m, k] * weight[v, k], bf16 inputs,
 * float32 accumulation (MFMA; the summation order is the kernel's, fixed
 * for given K).  x [M, K] and weight [V, K] are row-major bf16, 16-byte
 * aligned; K a multiple of 64; M <= WH_LMHEAD_MAX_ROWS.
 * wh_lmhead_logits writes logits_out [M, logits_stride] (float32).
 * wh_lmhead_greedy writes tokens [M]: per row the lowest index among the
 * largest logits -- the argmax of what wh_lmhead_logits writes -- without
 * writing the logits; it needs wh_lmhead_greedy_workspace_bytes(M, V) bytes
 * of workspace (8-byte aligned).  Inputs must hold no NaN. */
typedef struct wh_lmhead_args {
  const void* x;             /* device, [M, K] bf16 */
  const void* weight;        /* device, [V, K] bf16 */
  int32_t M;
  int32_t K;
  int32_t V;
  int32_t reserved;
  float* logits_out;         /* device, [M, logits_stride] (wh_lmhead_logits) */
  int64_t logits_stride;     /* elements, >= V */
  int32_t* tokens;           /* device, [M] (wh_lmhead_greedy) */
  void* workspace;           /* device (wh_lmhead_greedy) */
  size_t workspace_bytes;
} wh_lmhead_args;
int wh_lmhead_logits(const wh_lmhead_args* args, void* stream);
size_t wh_lmhead_greedy_workspace_bytes(int32_t M, int32_t V);
int wh_lmhead_greedy(const wh_lmhead_args* args, void* stream);
/* wh_lmhead_logits into args->logits_out, then wh_sample on those logits:
 * `sample` carries the sampling parameters and outputs (its logits, dtype,
 * B, V and row_stride are ignored: the logits are args'); results equal the
 * two calls made in turn.  Rows with a temperature above 0 whose only filter
 * is top-p (or none), without penalties or per-row temperatures, and a
 * workspace of wh_sample_workspace_bytes(M, V), take the fused form: the
 * product also merges each row's (value, index) maxima per sampler slice,
 * and the sampler starts after its max step. */
int wh_lmhead_sample(const wh_lmhead_args* args, const wh_sample_args* sample, void* stream);

/* Test hook: with on != 0, every entry of wh_verify_fused's sliced form
 * takes the exact per-row algorithm that entries the normaliser bounds leave
 * undecided take (same results, slower).  Process wide; returns the previous
 * setting. */
int wh_verify_force_exact(int on);

/* The contract exponential on device (floor(2^44 exp(d)) for d <= 0), for
 * bit-exactness tests against the CPU oracle. */
int wh_exp_fix44(const float* d, uint64_t* out, int64_t n, void* stream);

/* Message describing the last failure on this thread ("" if none). */
const char* wh_last_error(void);
/* Library version string. */
const char* wh_version(void);

#ifdef __cplusplus
}
#endif
#endif
