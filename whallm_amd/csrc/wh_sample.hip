// wh_sample.hip -- gfx950 decode-time token selection: penalties, temperature,
// top-k / top-p / min-p, and the categorical draw from a supplied uniform.
//
// Reference semantics (paths relative to the reference root):
//   runtime/deepseek_v4_ssd/generation.py:1279-1293  make_sampler + make_logits_processors
//   runtime/deepseek_v4_ssd/dspark.py:358-375        sampling_logprobs (p -> min-p -> k)
//   runtime/deepseek_v4_ssd/dspark.py:901-904        _sample
//   runtime/deepseek_v4_ssd/qwen4_exp.py:949-958     processors, then sampling_logprobs
//   third-party mlx_lm.sample_utils (make_sampler: k -> p -> min-p, * (1/T)).
//
// This file holds the per-row exact engine: one 1024-thread workgroup owns a
// row and makes several passes over it (the later passes hit L2 / the
// Infinity Cache).  Cutoffs are found by radix select over 50-bit
// (value, id) composites with LDS histograms -- counts for top-k, fixed-point
// probability mass for top-p -- and the draw is an inverse CDF over integer
// weights in vocabulary order, so results are bit-identical to the CPU
// oracle whatever the reduction order.
#include "wh_common.h"
#include "wh_internal.h"

#include <cmath>

namespace wh {

// ---------------------------------------------------------------------------
// Row context: the row's logits plus its penalised history tokens.
// ---------------------------------------------------------------------------
struct RowCtx {
  const float* xf;
  const uint16_t* xb;
  int V;
  // penalty table (LDS), empty when hmask < 0
  const int32_t* hkeys;
  const float* hval;
  const uint32_t* bitmap;
  int hmask;
  int hshift;

  __device__ __forceinline__ float raw(int i) const { return xf ? xf[i] : bf16_to_f32(xb[i]); }

  __device__ __forceinline__ float lookup(int i) const {
    uint32_t s = ((uint32_t)i * 2654435761u) >> hshift;
    while (hkeys[s] != i) s = (s + 1) & hmask;
    return hval[s];
  }
  // Effective (penalised) value, with -0 mapped to +0.
  __device__ __forceinline__ float val(int i) const {
    if (hmask >= 0 && ((bitmap[i >> 5] >> (i & 31)) & 1u)) return lookup(i);
    return raw(i) + 0.0f;
  }
};

// Filter state: an element is kept iff every active predicate holds.
struct Pred {
  int none;      // nothing kept
  int use_k;
  uint64_t ck;   // keep iff comp_a >= ck
  int use_p;
  uint64_t cp;   // keep iff comp_p >= cp
  int use_m;
  float thr;     // keep iff value >= thr
  __device__ __forceinline__ bool keep(int i, float l) const {
    if (none) return false;
    uint32_t k = fkey(l);
    if (use_k && comp_a(k, i) < ck) return false;
    if (use_p && comp_p(k, i) < cp) return false;
    if (use_m && !(l >= thr)) return false;
    return true;
  }
};

struct ExactSmem {
  uint64_t hist[1024];
  uint64_t scratch64[16];
  float scratchf[16];
  int scratchi[16];
  uint64_t bcast64[4];
  int bcasti[4];
};

// Penalty table setup in dynamic LDS.  Layout after ExactSmem:
//   hkeys[hcap] int32, hpos[hcap] int32 (reused as float values), hcnt[hcap] int32,
//   bitmap[(V+31)/32] uint32.
__device__ void build_penalties(const SampleKArgs& a, int b, RowCtx& rc, char* dyn) {
  const int tid = threadIdx.x, nt = blockDim.x;
  const int hcap = a.hcap;
  int32_t* hkeys = (int32_t*)dyn;
  int32_t* hpos = hkeys + hcap;
  int32_t* hcnt = hpos + hcap;
  uint32_t* bitmap = (uint32_t*)(hcnt + hcap);
  const int words = (a.V + 31) >> 5;
  rc.hkeys = hkeys;
  rc.hval = (const float*)hpos;
  rc.bitmap = bitmap;
  rc.hmask = hcap - 1;
  rc.hshift = 32 - a.hlog2;
  for (int s = tid; s < hcap; s += nt) { hkeys[s] = -1; hpos[s] = -1; hcnt[s] = 0; }
  for (int w = tid; w < words; w += nt) bitmap[w] = 0u;
  __syncthreads();
  int len = a.hist_len ? a.hist_len[b] : 0;
  if (len < 0) len = 0;
  if (len > a.hist_stride) len = (int)a.hist_stride;
  const bool on_r = a.rep != 0.0f, on_p = a.pres != 0.0f, on_f = a.freq != 0.0f;
  auto window = [len](int ctx) { return (ctx <= 0 || ctx > len) ? len : ctx; };
  const int wr = on_r ? window(a.rep_ctx) : 0;
  const int wp = on_p ? window(a.pres_ctx) : 0;
  const int wf = on_f ? window(a.freq_ctx) : 0;
  const int W = max(wr, max(wp, wf));
  const int32_t* h = a.hist + (long long)b * a.hist_stride;
  for (int j = len - W + tid; j < len; j += nt) {
    int t = h[j];
    if (t < 0 || t >= a.V) continue;
    uint32_t s = ((uint32_t)t * 2654435761u) >> rc.hshift;
    while (true) {
      int old = atomicCAS(&hkeys[s], -1, t);
      if (old == -1 || old == t) break;
      s = (s + 1) & rc.hmask;
    }
    atomicMax(&hpos[s], j);
    if (j >= len - wf) atomicAdd(&hcnt[s], 1);
    atomicOr(&bitmap[t >> 5], 1u << (t & 31));
  }
  __syncthreads();
  for (int s = tid; s < hcap; s += nt) {
    int t = hkeys[s];
    if (t < 0) continue;
    int lp = hpos[s];
    int c = hcnt[s];
    float v = rc.raw(t) + 0.0f;
    if (on_r && lp >= len - wr) v = v < 0.0f ? v * a.rep : v / a.rep;
    if (on_p && lp >= len - wp) v = v - a.pres;
    if (on_f && c > 0) v = v - a.freq * (float)c;
    ((float*)hpos)[s] = v + 0.0f;
  }
  __syncthreads();
}

// Radix select over 50-bit composites in descending order: returns the
// composite of the element at which the cumulative measure (count, or the
// fixed-point mass exp_fix44(l - m)) of kept elements first reaches
// `target` (> 0, <= total).  Five passes of 10-bit digits.
template <bool MASS, bool ORDER_P>
__device__ uint64_t radix_select(const RowCtx& rc, const Pred& pr, float m, uint64_t target, ExactSmem& sm) {
  const int tid = threadIdx.x, nt = blockDim.x;
  uint64_t prefix = 0;
  for (int pass = 0; pass < 5; ++pass) {
    const int shift = 40 - 10 * pass;
    for (int i = tid; i < 1024; i += nt) sm.hist[i] = 0;
    __syncthreads();
    for (int i = tid; i < rc.V; i += nt) {
      float l = rc.val(i);
      if (!pr.keep(i, l)) continue;
      uint32_t k = fkey(l);
      uint64_t c = ORDER_P ? comp_p(k, i) : comp_a(k, i);
      if ((c >> (shift + 10)) != prefix) continue;
      uint64_t meas = MASS ? exp_fix44(l - m) : 1ull;
      if (meas) atomicAdd((unsigned long long*)&sm.hist[(c >> shift) & 1023], (unsigned long long)meas);
    }
    __syncthreads();
    // suffix sums from the top bin: thread t owns bin 1023 - t
    const int bin = 1023 - tid;
    uint64_t hv = (tid < 1024) ? sm.hist[bin] : 0;
    uint64_t tot;
    uint64_t excl = block_exclusive_scan_u64(hv, sm.scratch64, &tot);
    if (tid < 1024 && excl < target && excl + hv >= target) {
      sm.bcast64[0] = (uint64_t)bin;
      sm.bcast64[1] = excl;
    }
    __syncthreads();
    prefix = (prefix << 10) | sm.bcast64[0];
    target -= sm.bcast64[1];
    __syncthreads();
  }
  return prefix;
}

__device__ __forceinline__ float chain_scale(int chain, float d, float invT, float Tc) {
  return chain == WH_CHAIN_MLX ? d * invT : d / Tc;
}

__global__ void __launch_bounds__(1024) sample_exact_kernel(SampleKArgs a) {
  extern __shared__ __align__(16) char dyn_smem[];
  __shared__ ExactSmem sm;
  const int b = blockIdx.x;
  const int tid = threadIdx.x, nt = blockDim.x;
  const int V = a.V;
  RowCtx rc;
  rc.V = V;
  rc.xf = a.dtype == WH_DTYPE_F32 ? (const float*)a.logits + b * a.row_stride : nullptr;
  rc.xb = a.dtype == WH_DTYPE_BF16 ? (const uint16_t*)a.logits + b * a.row_stride : nullptr;
  rc.hmask = -1;
  if (a.hcap > 0) build_penalties(a, b, rc, dyn_smem);

  const float T = a.T_rows ? a.T_rows[b] : a.T;
  const float top_p = a.top_p_rows ? a.top_p_rows[b] : a.top_p;
  const float min_p = a.min_p_rows ? a.min_p_rows[b] : a.min_p;
  const int top_k = a.top_k_rows ? a.top_k_rows[b] : a.top_k;
  float* out = a.out_rows ? a.out_rows + (long long)b * V : nullptr;

  if (!(T > 0.0f)) {
    // greedy: lowest index among the maxima (mx.argmax)
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int i = tid; i < V; i += nt) {
      float l = rc.val(i);
      if (bi == 0x7FFFFFFF || l > bv) { bv = l; bi = i; }
      if (out) out[i] = l;
    }
    float m = block_reduce(bv, sm.scratchf, OpMaxF(), -INFINITY);
    int cand = (bi != 0x7FFFFFFF && bv == m) ? bi : 0x7FFFFFFF;
    int tok = block_reduce(cand, sm.scratchi, OpMinI(), 0x7FFFFFFF);
    if (tid == 0) {
      if (a.tokens) a.tokens[b] = tok == 0x7FFFFFFF ? 0 : tok;
      if (a.kept) a.kept[b] = 1;
    }
    return;
  }

  float lmax = -INFINITY;
  for (int i = tid; i < V; i += nt) lmax = fmaxf(lmax, rc.val(i));
  const float m = block_reduce(lmax, sm.scratchf, OpMaxF(), -INFINITY);

  const bool use_k = top_k > 0 && top_k < V;
  const bool use_p = top_p > 0.0f && top_p < 1.0f;
  const bool use_m = min_p != 0.0f;
  const float theta = (float)(1.0 - (double)top_p);
  Pred pr = {0, 0, 0, 0, 0, 0, 0.0f};

  uint64_t Z = 0;
  if (use_p) {
    uint64_t z = 0;
    if (m != -INFINITY)
      for (int i = tid; i < V; i += nt) z += exp_fix44(rc.val(i) - m);
    Z = block_reduce(z, sm.scratch64, OpSumU64(), (uint64_t)0);
  }
  auto kept_mass = [&]() {
    uint64_t s = 0;
    if (m != -INFINITY)
      for (int i = tid; i < V; i += nt) {
        float l = rc.val(i);
        if (pr.keep(i, l)) s += exp_fix44(l - m);
      }
    return block_reduce(s, sm.scratch64, OpSumU64(), (uint64_t)0);
  };
  auto kept_count = [&]() {
    int c = 0;
    for (int i = tid; i < V; i += nt) c += pr.keep(i, rc.val(i)) ? 1 : 0;
    return block_reduce(c, sm.scratchi, OpSumI(), 0);
  };
  auto apply_p = [&](uint64_t S) {
    uint64_t F = floor_theta_z(theta, Z);
    if (S <= F) { pr.none = 1; return; }
    uint64_t cp = radix_select<true, true>(rc, pr, m, S - F, sm);
    pr.use_p = 1;
    pr.cp = cp;
  };
  auto apply_m = [&]() {
    const float c = a.min_p_rows ? (float)log((double)min_p) : a.min_p_log;
    pr.use_m = 1;
    pr.thr = m + c;
  };

  if (a.chain == WH_CHAIN_MLX) {
    if (use_k) {
      uint64_t ck = radix_select<false, false>(rc, pr, m, (uint64_t)top_k, sm);
      pr.use_k = 1;
      pr.ck = ck;
    }
    if (use_p) apply_p(use_k ? kept_mass() : Z);
    if (use_m && !pr.none) apply_m();
  } else {
    if (use_p) apply_p(Z);
    if (use_m && !pr.none) apply_m();
    if (use_k && !pr.none) {
      int n_alive = kept_count();
      if (n_alive > top_k) {
        uint64_t ck = radix_select<false, false>(rc, pr, m, (uint64_t)top_k, sm);
        pr.use_k = 1;
        pr.ck = ck;
      }
    }
  }

  // Draw: per-thread contiguous segments, integer inverse CDF in vocab order.
  const float invT = (float)(1.0 / (double)T);
  const float Tc = (float)fmax((double)T, 1e-5);
  const int seg = (V + nt - 1) / nt;
  const int lo = min(V, tid * seg), hi = min(V, lo + seg);
  uint64_t s = 0;
  int cnt = 0;
  for (int i = lo; i < hi; ++i) {
    float l = rc.val(i);
    if (!pr.keep(i, l)) continue;
    ++cnt;
    s += exp_fix44(chain_scale(a.chain, l - m, invT, Tc));
  }
  uint64_t ZV;
  uint64_t excl = block_exclusive_scan_u64(s, sm.scratch64, &ZV);
  const int nkept = block_reduce(cnt, sm.scratchi, OpSumI(), 0);
  if (a.tokens) {
    const uint64_t tgt = ZV ? draw_target(a.u[b], ZV) : 0;
    if (ZV == 0) {
      if (tid == 0) a.tokens[b] = 0;
    } else if (excl <= tgt && tgt < excl + s) {
      uint64_t c = excl;
      for (int i = lo; i < hi; ++i) {
        float l = rc.val(i);
        if (!pr.keep(i, l)) continue;
        c += exp_fix44(chain_scale(a.chain, l - m, invT, Tc));
        if (c > tgt) { a.tokens[b] = i; break; }
      }
    }
  }
  if (a.kept && tid == 0) a.kept[b] = nkept;
  if (out && a.out_mode == WH_OUT_MASKED) {
    for (int i = tid; i < V; i += nt) {
      float l = rc.val(i);
      out[i] = pr.keep(i, l) ? l : -INFINITY;
    }
  } else if (out) {
    const double lz = log(ldexp((double)ZV, -44));
    for (int i = tid; i < V; i += nt) {
      float l = rc.val(i);
      out[i] = pr.keep(i, l) ? (float)((double)chain_scale(a.chain, l - m, invT, Tc) - lz) : -INFINITY;
    }
  }
}

// In-place penalty processors (the unfused drop-in for make_logits_processors).
__global__ void __launch_bounds__(1024) penalties_kernel(SampleKArgs a) {
  extern __shared__ __align__(16) char dyn_smem[];
  const int b = blockIdx.x;
  RowCtx rc;
  rc.V = a.V;
  rc.xf = a.dtype == WH_DTYPE_F32 ? (const float*)a.logits + b * a.row_stride : nullptr;
  rc.xb = a.dtype == WH_DTYPE_BF16 ? (const uint16_t*)a.logits + b * a.row_stride : nullptr;
  build_penalties(a, b, rc, dyn_smem);
  for (int s = threadIdx.x; s < a.hcap; s += blockDim.x) {
    int t = rc.hkeys[s];
    if (t < 0) continue;
    float v = rc.hval[s];
    if (a.dtype == WH_DTYPE_F32) {
      ((float*)a.logits)[b * a.row_stride + t] = v;
    } else {
      // round to nearest even, as a float32 -> bfloat16 cast does
      uint32_t u = __float_as_uint(v);
      uint32_t r = u + 0x7FFFu + ((u >> 16) & 1u);
      if ((u & 0x7F800000u) == 0x7F800000u) r = u;  // inf / nan pass through
      ((uint16_t*)a.logits)[b * a.row_stride + t] = (uint16_t)(r >> 16);
    }
  }
}

__global__ void exp_fix44_kernel(const float* d, uint64_t* out, long long n) {
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = exp_fix44(d[i]);
}

}  // namespace wh

// ===========================================================================
// C ABI
// ===========================================================================
using namespace wh;

static thread_local char g_err[512];

extern "C" const char* wh_last_error(void) { return g_err; }
extern "C" const char* wh_version(void) { return "whallm_amd 0.1 (gfx950)"; }

int wh::fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}
void wh::clear_error() { g_err[0] = 0; }

static int window_bound(int32_t ctx, int64_t stride) { return (ctx <= 0 || ctx > stride) ? (int)stride : ctx; }

// Validate and translate the public struct into kernel arguments.
int wh::prepare_sample(const wh_sample_args* p, SampleKArgs* k, bool need_draw) {
  if (!p) return fail(WH_EINVAL, "args is NULL");
  if (p->dtype != WH_DTYPE_F32 && p->dtype != WH_DTYPE_BF16) return fail(WH_EINVAL, "dtype must be WH_DTYPE_F32 or WH_DTYPE_BF16");
  if (p->B < 0) return fail(WH_EINVAL, "B must be >= 0");
  if (p->V <= 0 || p->V > WH_MAX_VOCAB) return fail(WH_ELIMIT, "V must be in [1, %d], got %d", WH_MAX_VOCAB, p->V);
  if (p->row_stride < p->V) return fail(WH_EINVAL, "row_stride (%lld) < V (%d)", (long long)p->row_stride, p->V);
  if (!p->logits && p->B > 0) return fail(WH_EINVAL, "logits is NULL");
  if (p->chain != WH_CHAIN_MLX && p->chain != WH_CHAIN_WHALLM) return fail(WH_EINVAL, "chain must be WH_CHAIN_MLX or WH_CHAIN_WHALLM");
  if (!p->temperature_rows && !(p->temperature >= 0.0f)) return fail(WH_EINVAL, "temperature must be >= 0");
  if (!p->min_p_rows && !(p->min_p >= 0.0f && p->min_p <= 1.0f))
    return fail(WH_EINVAL, "`min_p` has to be a float in the [0, 1] interval, but is %g", (double)p->min_p);
  if (!p->top_k_rows && p->top_k < 0) return fail(WH_EINVAL, "top_k must be >= 0");
  if (p->chain == WH_CHAIN_MLX && !p->top_k_rows && !p->temperature_rows && p->temperature > 0.0f && p->top_k > 0 &&
      p->top_k >= p->V)
    return fail(WH_EINVAL, "`top_k` has to be an integer in the (0, %d] interval, but is %d.", p->V, p->top_k);
  if (p->repetition_penalty < 0.0f) return fail(WH_EINVAL, "penalty must be a non-negative float, got %g", (double)p->repetition_penalty);
  if (need_draw && p->tokens && !p->uniforms && p->B > 0) return fail(WH_EINVAL, "uniforms is NULL but tokens were requested");
  if (p->out_mode != WH_OUT_LOGPROBS && p->out_mode != WH_OUT_MASKED) return fail(WH_EINVAL, "out_mode must be WH_OUT_LOGPROBS or WH_OUT_MASKED");
  if (p->logprobs_out && p->out_mode == WH_OUT_LOGPROBS && p->chain != WH_CHAIN_WHALLM)
    return fail(WH_EINVAL, "the sampling_logprobs row (WH_OUT_LOGPROBS) is only defined for WH_CHAIN_WHALLM");
  memset(k, 0, sizeof(*k));
  k->logits = p->logits;
  k->dtype = p->dtype;
  k->B = p->B;
  k->V = p->V;
  k->chain = p->chain;
  k->row_stride = p->row_stride;
  k->hist = p->history;
  k->hist_stride = p->history_stride;
  k->hist_len = p->history_len;
  k->u = p->uniforms;
  k->T = p->temperature;
  k->top_p = p->top_p;
  k->min_p = p->min_p;
  k->min_p_log = (float)log((double)p->min_p);
  k->top_k = p->top_k;
  k->T_rows = p->temperature_rows;
  k->top_p_rows = p->top_p_rows;
  k->min_p_rows = p->min_p_rows;
  k->top_k_rows = p->top_k_rows;
  k->rep = p->repetition_penalty;
  k->pres = p->presence_penalty;
  k->freq = p->frequency_penalty;
  k->rep_ctx = p->repetition_context;
  k->pres_ctx = p->presence_context;
  k->freq_ctx = p->frequency_context;
  k->tokens = p->tokens;
  k->kept = p->kept_count;
  k->out_rows = p->logprobs_out;
  k->out_mode = p->out_mode;
  const bool pen = p->history && (p->repetition_penalty != 0.0f || p->presence_penalty != 0.0f || p->frequency_penalty != 0.0f);
  if (pen) {
    if (!p->history_len) return fail(WH_EINVAL, "history_len is NULL");
    if (p->history_stride <= 0) return fail(WH_EINVAL, "history_stride must be > 0");
    int w = 0;
    if (p->repetition_penalty != 0.0f) w = std::max(w, window_bound(p->repetition_context, p->history_stride));
    if (p->presence_penalty != 0.0f) w = std::max(w, window_bound(p->presence_context, p->history_stride));
    if (p->frequency_penalty != 0.0f) w = std::max(w, window_bound(p->frequency_context, p->history_stride));
    if (w > WH_MAX_WINDOW)
      return fail(WH_ELIMIT, "penalty window of %d ids exceeds WH_MAX_WINDOW (%d); pass a context size", w, WH_MAX_WINDOW);
    int cap = 64, lg = 6;
    while (cap < 2 * w) { cap <<= 1; ++lg; }
    k->hcap = cap;
    k->hlog2 = lg;
  }
  return WH_OK;
}

size_t wh::penalty_lds_bytes(const SampleKArgs& k) {
  if (k.hcap == 0) return 0;
  return (size_t)k.hcap * 12 + (size_t)((k.V + 31) / 32) * 4;
}

extern "C" size_t wh_sample_workspace_bytes(int32_t B, int32_t V) {
  (void)V;
  return wh::sample_workspace_bytes(B, V);
}

extern "C" int wh_sample(const wh_sample_args* args, void* stream) {
  clear_error();
  SampleKArgs k;
  int rc = prepare_sample(args, &k, true);
  if (rc) return rc;
  if (!args->tokens && !args->logprobs_out && !args->kept_count) return WH_OK;
  if (k.B == 0) return WH_OK;
  return wh::launch_sample(k, args, (hipStream_t)stream);
}

int wh::launch_sample_exact(const SampleKArgs& k, hipStream_t st) {
  size_t lds = penalty_lds_bytes(k);
  if (lds > 65536) hipFuncSetAttribute((const void*)sample_exact_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  hipLaunchKernelGGL(sample_exact_kernel, dim3(k.B), dim3(1024), lds, st, k);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "sample_exact_kernel launch failed: %s", hipGetErrorString(e));
  return WH_OK;
}

extern "C" int wh_apply_penalties(const wh_sample_args* args, void* stream) {
  clear_error();
  SampleKArgs k;
  int rc = prepare_sample(args, &k, false);
  if (rc) return rc;
  if (k.hcap == 0 || k.B == 0) return WH_OK;
  if (penalty_lds_bytes(k) > 65536)
    hipFuncSetAttribute((const void*)penalties_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)penalty_lds_bytes(k));
  hipLaunchKernelGGL(penalties_kernel, dim3(k.B), dim3(1024), penalty_lds_bytes(k), (hipStream_t)stream, k);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "penalties_kernel launch failed: %s", hipGetErrorString(e));
  return WH_OK;
}

extern "C" int wh_exp_fix44(const float* d, uint64_t* out, int64_t n, void* stream) {
  clear_error();
  if (n < 0 || (n > 0 && (!d || !out))) return fail(WH_EINVAL, "bad arguments");
  if (n == 0) return WH_OK;
  long long blocks = (n + 255) / 256;
  hipLaunchKernelGGL(exp_fix44_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, d, out, (long long)n);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "exp_fix44_kernel launch failed: %s", hipGetErrorString(e));
  return WH_OK;
}
