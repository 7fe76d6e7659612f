// wh_logprobs.hip -- top-n logprobs of a batch of logit rows on gfx950.
//
// What it serves: the OpenAI-style `logprobs` / `top_logprobs` response
// fields.  The reference server rejects them today
// (runtime/deepseek_v4_ssd/server.py:1110-1111, README.md:147); the value it
// would return is mlx_lm's per-step `logprobs = logits - logsumexp(logits)`
// (the row generate_step hands to the sampler, generation.py:1465-1475), of
// which a response carries the n most likely entries and the chosen token's.
//
// Order: value descending, id ascending among equal values (the composite
// key comp_a).  logprob = float32(double(l) - lse), lse = logsumexp in
// float64.  -inf entries rank last; a row of all -inf gives -inf logprobs.
//
// Two launches, no atomics in global memory:
//   1. tl_slice_kernel: one 256-thread workgroup per 4096-entry slice of a row
//      (one HBM pass over the logits, 16 entries per thread in registers).  It
//      writes the slice's top-n keys in order, its max and sum exp(l - max).
//   2. tl_merge_kernel: one workgroup per row merges the G slice summaries
//      (lse) and the G*n keys (top-n again), and writes the outputs.
// Top-n of a block's keys (block_topn): the n-th largest of the 256 per-thread
// maxima bounds the answer from below (n threads each hold an entry at least
// that large), so at most 16 n entries (those of the n leading threads) pass
// the bound; these are ranked by counting in LDS.
#include "wh_internal.h"
#include "wh_common.h"

namespace wh {

constexpr int TL_T = 256;              // threads per workgroup
constexpr int TL_E = 16;               // entries per thread
constexpr int TL_SL = TL_T * TL_E;     // slice length
constexpr int TL_CAND = TL_E * WH_MAX_TOP_LOGPROBS;

struct TlSlice {
  double s;  // sum over the slice of exp(l - m)
  float m;   // slice max (-inf when the slice is all -inf)
  int pad;
};

struct TopnSmem {
  uint64_t tk[TL_T];
  uint64_t cand[TL_CAND];
  uint64_t res[WH_MAX_TOP_LOGPROBS];
  double red[TL_T / 64];
  uint64_t tau;
  int cnt;
};

// Sorted top-n (largest first) of the block's keys into sm.res[0 .. n);
// key 0 marks an empty entry and fills res[] past the number of nonzero keys.
// Nonzero keys must be distinct.
template <int E>
__device__ void block_topn(const uint64_t (&k)[E], int n, TopnSmem& sm) {
  const int t = threadIdx.x;
  uint64_t km = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) km = k[e] > km ? k[e] : km;
  sm.tk[t] = km;
  if (t == 0) sm.cnt = 0;
  __syncthreads();
  int r = 0, nz = 0;
  for (int j = 0; j < TL_T; ++j) {
    const uint64_t o = sm.tk[j];
    r += o > km;
    nz += o != 0;
  }
  // nz is uniform; with fewer than n nonempty threads every nonzero key passes
  if (nz >= n) {
    if (km != 0 && r == n - 1) sm.tau = km;
  } else if (t == 0) {
    sm.tau = 1;
  }
  __syncthreads();
  const uint64_t tau = sm.tau;
  if (km >= tau) {
#pragma unroll
    for (int e = 0; e < E; ++e)
      if (k[e] >= tau) sm.cand[atomicAdd(&sm.cnt, 1)] = k[e];
  }
  __syncthreads();
  const int c = sm.cnt;
  for (int i = t; i < c; i += TL_T) {
    const uint64_t x = sm.cand[i];
    int rr = 0;
    for (int j = 0; j < c; ++j) rr += sm.cand[j] > x;
    if (rr < n) sm.res[rr] = x;
  }
  if (t >= c && t < n) sm.res[t] = 0;
  __syncthreads();
}

template <int DT>
__device__ __forceinline__ float tl_load(const void* row, int i) {
  if (DT) return bf16_to_f32(((const uint16_t*)row)[i]) + 0.0f;
  return ((const float*)row)[i] + 0.0f;  // -0 -> +0: equal values, equal keys
}

template <int DT>
__global__ void __launch_bounds__(TL_T) tl_slice_kernel(const void* __restrict__ logits, long long ld, int V, int G,
                                                         int n, TlSlice* __restrict__ summ, uint64_t* __restrict__ keys) {
  __shared__ TopnSmem sm;
  const int b = blockIdx.x / G, g = blockIdx.x - b * G;
  const char* row = (const char*)logits + (size_t)b * ld * (DT ? 2 : 4);
  const int base = g * TL_SL + threadIdx.x;
  float v[TL_E];
  uint64_t k[TL_E];
#pragma unroll
  for (int e = 0; e < TL_E; ++e) {
    const int i = base + e * TL_T;
    v[e] = i < V ? tl_load<DT>(row, i) : -INFINITY;
    k[e] = i < V ? comp_a(fkey(v[e]), i) : 0;
  }
  block_topn<TL_E>(k, n, sm);
  const uint64_t top = sm.res[0];  // the slice holds at least one entry
  const float m = key_to_float((uint32_t)(top >> 18));
  double s = 0.0;
  if (m != -INFINITY) {
#pragma unroll
    for (int e = 0; e < TL_E; ++e) s += (double)expf(v[e] - m);
  }
  s = block_reduce(s, sm.red, OpSumF64(), 0.0);
  const size_t slot = (size_t)b * G + g;
  if (threadIdx.x < n) keys[slot * n + threadIdx.x] = sm.res[threadIdx.x];
  if (threadIdx.x == 0) summ[slot] = TlSlice{s, m, 0};
}

template <int DT>
__global__ void __launch_bounds__(TL_T) tl_merge_kernel(const void* __restrict__ logits, long long ld, int V, int G,
                                                         int n, const TlSlice* __restrict__ summ,
                                                         const uint64_t* __restrict__ keys,
                                                         const int32_t* __restrict__ token, int32_t* __restrict__ ids,
                                                         float* __restrict__ lps, float* __restrict__ token_lp) {
  __shared__ TopnSmem sm;
  __shared__ double lse_s;
  const int b = blockIdx.x;
  const TlSlice* hs = summ + (size_t)b * G;
  if (threadIdx.x < 64) {
    // G <= 64 slices: one per lane
    const int l = threadIdx.x;
    const float mg = l < G ? hs[l].m : -INFINITY;
    const double sg = l < G ? hs[l].s : 0.0;
    float M = mg;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, WH_WAVE));
    const double part = (M == -INFINITY || mg == -INFINITY) ? 0.0 : sg * exp((double)mg - (double)M);
    const double S = wave_sum_f64(part);
    if (l == 0) lse_s = M == -INFINITY ? -INFINITY : (double)M + log(S);
  }
  const int total = G * n;
  const uint64_t* kr = keys + (size_t)b * total;
  uint64_t k[TL_E];
#pragma unroll
  for (int e = 0; e < TL_E; ++e) {
    const int i = threadIdx.x + e * TL_T;
    k[e] = i < total ? kr[i] : 0;
  }
  block_topn<TL_E>(k, n, sm);  // its barriers also publish lse_s
  const double lse = lse_s;
  if (threadIdx.x < n) {
    const uint64_t x = sm.res[threadIdx.x];
    const float val = key_to_float((uint32_t)(x >> 18));
    ids[(size_t)b * n + threadIdx.x] = 0x3FFFF - (int)(x & 0x3FFFF);
    lps[(size_t)b * n + threadIdx.x] = (lse == -INFINITY || val == -INFINITY) ? -INFINITY : (float)((double)val - lse);
  }
  if (token_lp && threadIdx.x == 0) {
    const int tk = token[b];
    float r = -INFINITY;
    if (tk >= 0 && tk < V && lse != -INFINITY) {
      const float x = tl_load<DT>((const char*)logits + (size_t)b * ld * (DT ? 2 : 4), tk);
      if (x != -INFINITY) r = (float)((double)x - lse);
    }
    token_lp[b] = r;
  }
}

static int tl_slices(int V) { return (V + TL_SL - 1) / TL_SL; }

static size_t tl_workspace(int B, int V, int n) {
  const size_t slots = (size_t)B * tl_slices(V);
  return slots * sizeof(TlSlice) + slots * n * sizeof(uint64_t);
}

}  // namespace wh

using namespace wh;

extern "C" size_t wh_top_logprobs_workspace_bytes(int32_t B, int32_t V, int32_t n) {
  if (B <= 0 || V <= 0 || n <= 0) return 0;
  return tl_workspace(B, V, n);
}

extern "C" int wh_top_logprobs(const wh_top_logprobs_args* a, void* stream) {
  clear_error();
  if (!a) return fail(WH_EINVAL, "args is NULL");
  if (a->dtype != WH_DTYPE_F32 && a->dtype != WH_DTYPE_BF16) return fail(WH_EINVAL, "dtype must be WH_DTYPE_F32 or WH_DTYPE_BF16");
  if (a->B < 0) return fail(WH_EINVAL, "B must be >= 0, got %d", a->B);
  if (a->V <= 0 || a->V > WH_MAX_VOCAB) return fail(WH_ELIMIT, "V must be in [1, %d], got %d", WH_MAX_VOCAB, a->V);
  if (a->n <= 0 || a->n > WH_MAX_TOP_LOGPROBS || a->n > a->V)
    return fail(WH_ELIMIT, "n must be in [1, min(V, %d)], got %d", WH_MAX_TOP_LOGPROBS, a->n);
  if (a->B == 0) return WH_OK;
  if (a->row_stride < a->V) return fail(WH_EINVAL, "row_stride (%lld) must be >= V (%d)", (long long)a->row_stride, a->V);
  if (!a->logits || !a->top_ids || !a->top_logprobs) return fail(WH_EINVAL, "logits, top_ids and top_logprobs are required");
  if (a->token_logprob && !a->token) return fail(WH_EINVAL, "token_logprob needs token");
  const size_t need = tl_workspace(a->B, a->V, a->n);
  if (!a->workspace || a->workspace_bytes < need)
    return fail(WH_EINVAL, "workspace must hold wh_top_logprobs_workspace_bytes(B, V, n) = %zu bytes", need);
  if ((uintptr_t)a->workspace % 16) return fail(WH_EINVAL, "workspace must be 16-byte aligned");
  const int G = tl_slices(a->V);
  const size_t slots = (size_t)a->B * G;
  if (slots > (size_t)0x7FFFFFFF) return fail(WH_ELIMIT, "B * slices exceeds the grid limit");
  TlSlice* summ = (TlSlice*)a->workspace;
  uint64_t* keys = (uint64_t*)((char*)a->workspace + slots * sizeof(TlSlice));
  hipStream_t st = (hipStream_t)stream;
  if (a->dtype == WH_DTYPE_BF16) {
    hipLaunchKernelGGL(tl_slice_kernel<1>, dim3((unsigned)slots), dim3(TL_T), 0, st, a->logits, (long long)a->row_stride,
                       a->V, G, a->n, summ, keys);
    hipLaunchKernelGGL(tl_merge_kernel<1>, dim3(a->B), dim3(TL_T), 0, st, a->logits, (long long)a->row_stride, a->V, G,
                       a->n, summ, keys, a->token, a->top_ids, a->top_logprobs, a->token_logprob);
  } else {
    hipLaunchKernelGGL(tl_slice_kernel<0>, dim3((unsigned)slots), dim3(TL_T), 0, st, a->logits, (long long)a->row_stride,
                       a->V, G, a->n, summ, keys);
    hipLaunchKernelGGL(tl_merge_kernel<0>, dim3(a->B), dim3(TL_T), 0, st, a->logits, (long long)a->row_stride, a->V, G,
                       a->n, summ, keys, a->token, a->top_ids, a->top_logprobs, a->token_logprob);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "top-logprob launch failed: %s", hipGetErrorString(e));
  return WH_OK;
}
