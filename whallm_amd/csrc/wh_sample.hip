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
#include <mutex>

#include "wh_rowops.h"

namespace wh {

__global__ void __launch_bounds__(1024) sample_exact_kernel(SampleKArgs a) {
  extern __shared__ __align__(16) char dyn_smem[];
  __shared__ ExactSmem sm;
  exact_row_impl(a, blockIdx.x, dyn_smem, sm);
}

// In-place penalty processors (the unfused drop-in for make_logits_processors).
__global__ void __launch_bounds__(1024) penalties_kernel(SampleKArgs a) {
  extern __shared__ __align__(16) char dyn_smem[];
  const int b = blockIdx.x;
  RowCtx rc;
  rc.V = a.V;
  rc.xf = a.dtype == WH_DTYPE_F32 ? (const float*)a.logits + b * a.row_stride : nullptr;
  rc.xb = a.dtype == WH_DTYPE_BF16 ? (const uint16_t*)a.logits + b * a.row_stride : nullptr;
  build_penalties(a, b, rc, dyn_smem, 0, a.V);
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
  if (!p->temperature_rows && !(p->temperature >= 0.0)) return fail(WH_EINVAL, "temperature must be >= 0");
  if (!p->min_p_rows && !(p->min_p >= 0.0 && p->min_p <= 1.0))
    return fail(WH_EINVAL, "`min_p` has to be a float in the [0, 1] interval, but is %g", (double)p->min_p);
  if (!p->top_k_rows && p->top_k < 0) return fail(WH_EINVAL, "top_k must be >= 0");
  if (p->chain == WH_CHAIN_MLX && !p->top_k_rows && !p->temperature_rows && p->temperature > 0.0 && p->top_k > 0 &&
      p->top_k >= p->V)
    return fail(WH_EINVAL, "`top_k` has to be an integer in the (0, %d] interval, but is %d.", p->V, p->top_k);
  if (p->history_share < 0) return fail(WH_EINVAL, "history_share must be >= 0");
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
  k->hshare = p->history_share > 1 ? p->history_share : 1;
  k->u = p->uniforms;
  k->T = p->temperature;
  k->top_p = p->top_p;
  k->min_p = p->min_p;
  k->min_p_log = (float)log(p->min_p);
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
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)sample_exact_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return fail(WH_EHIP, "hipFuncSetAttribute failed: %s", hipGetErrorString(e));
  }
  hipLaunchKernelGGL(sample_exact_kernel, dim3(k.B), dim3(1024), lds, st, k);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "sample_exact_kernel launch failed: %s", hipGetErrorString(e));
  return WH_OK;
}

// The no-allocation entry point's scratch: a file-scope device array (zero
// initialised in the code object, so it adds nothing to the file), one copy
// per GPU at its own address.  Host code never passes `scratch` itself -- its
// host-side name is not a device address -- only the address
// hipGetSymbolAddress returns for the current device, cached per device.
static __device__ __align__(256) char scratch[WH_NOALLOC_SCRATCH_BYTES];

constexpr int WH_SCRATCH_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[WH_SCRATCH_DEVICES];

static int scratch_for_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(WH_EHIP, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= WH_SCRATCH_DEVICES) return fail(WH_ELIMIT, "device %d beyond the %d the scratch table holds", dev, WH_SCRATCH_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return fail(WH_EHIP, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return WH_OK;
}

extern "C" int wh_sample_noalloc(const wh_sample_args* args, void* stream) {
  clear_error();
  SampleKArgs k;
  int rc = prepare_sample(args, &k, true);
  if (rc) return rc;
  if (!args->tokens && !args->logprobs_out && !args->kept_count) return WH_OK;
  if (k.B == 0) return WH_OK;
  const size_t need = wh::sample_workspace_bytes(k.B, k.V);
  if (need > WH_NOALLOC_SCRATCH_BYTES)
    return fail(WH_ELIMIT,
                "wh_sample_noalloc: %d rows of V=%d need %zu bytes of scratch, beyond its maximum of %u bytes "
                "(WH_NOALLOC_SCRATCH_BYTES); call wh_sample with a workspace instead",
                k.B, k.V, need, (unsigned)WH_NOALLOC_SCRATCH_BYTES);
  void* ptr = nullptr;
  rc = scratch_for_current_device(&ptr);
  if (rc) return rc;
  wh_sample_args a = *args;
  a.workspace = ptr;
  a.workspace_bytes = WH_NOALLOC_SCRATCH_BYTES;
  return wh::launch_sample(k, &a, (hipStream_t)stream);
}

extern "C" int wh_apply_penalties(const wh_sample_args* args, void* stream) {
  clear_error();
  SampleKArgs k;
  int rc = prepare_sample(args, &k, false);
  if (rc) return rc;
  if (k.hcap == 0 || k.B == 0) return WH_OK;
  if (penalty_lds_bytes(k) > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)penalties_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)penalty_lds_bytes(k));
    if (e != hipSuccess) return fail(WH_EHIP, "hipFuncSetAttribute failed: %s", hipGetErrorString(e));
  }
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
