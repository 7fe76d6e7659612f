// wh_verify.hip -- gfx950 speculative verification (DSpark / MTP accept-reject
// with residual resampling), runtime/deepseek_v4_ssd/dspark.py:857-898.
//
// Two input forms:
//  * logprob form (wh_verify_logprobs): the reference's own arguments --
//    target logprob rows [B, n+1, V] and draft logprob rows [B, n, V], both
//    already tempered/filtered by sampling_logprobs.  Ratio test
//    reject iff u > min(1, exp(g_t - d_t)), residual max(e^g - e^d, 0).
//  * fused form (wh_verify_fused): raw target logits plus T (the target rows
//    are sampling_logprobs(logits, T, top_p=1) = softmax(x / T), computed
//    here) and draft probabilities q.  Phase 1 runs one workgroup per
//    (batch, position) for the row max, the exact fixed-point normaliser and
//    the ratio test; phase 2 runs one workgroup per batch entry for the first
//    rejection's residual draw (or the bonus draw).
//
// All decisions are exact: masses are floor(2^44 exp(.)) integers, the
// ratio test u*q*Z > W is evaluated in 128-bit integers.
#include <cmath>

#include "wh_common.h"
#include "wh_internal.h"

namespace wh {

struct VerifyKArgs {
  int B, n, V;
  float T;     // temperature
  float Tc;    // fl32(max(T, 1e-5))
  const float* target;
  const float* draft;
  const int32_t* tok;
  const float* u;
  int32_t* accepted;
  int32_t* token;
  float* row_out;
  // fused-form workspace: per (b, j) reject flag, row max and normaliser
  int32_t* rej;
  float* rmax;
  unsigned long long* rz;
};

struct VSmem {
  uint64_t scratch64[16];
  float scratchf[16];
  int scratchi[16];
  int bcasti[4];
};

__device__ __forceinline__ bool reject_lp(float u, float g, float d) {
  float diff = g - d;
  if (diff != diff) return false;
  if (diff >= 0.0f) return false;
  uint64_t R = exp_fix44(diff);
  return (double)u * 17592186044416.0 > (double)R;
}

__device__ __forceinline__ uint64_t floor_qz(float q, uint64_t Z) {
  if (!(q > 0.0f)) return 0;
  if (q > 1.0f) q = 1.0f;
  int e;
  uint64_t M = mant24(q, &e);
  int s = 24 - e;
  u128 prod = (u128)M * Z;
  u128 F = s >= 128 ? (u128)0 : (prod >> s);
  return F > (u128)(~0ull) ? ~0ull : (uint64_t)F;
}

// reject iff u * q * Z > W (exact)
__device__ __forceinline__ bool reject_fused(float u, float q, uint64_t Z, uint64_t W) {
  if (!(u > 0.0f) || !(q > 0.0f)) return false;
  if (q > 1.0f) q = 1.0f;
  int eu, eq;
  uint64_t Mu = mant24(u, &eu), Mq = mant24(q, &eq);
  int s = 48 - eu - eq;
  u128 prod = (u128)(Mu * Mq) * (u128)Z;
  if (s >= 128) return false;
  if (W == 0) return prod > 0;
  int wbits = 64 - __clzll((long long)W);
  if (wbits + s > 127) return false;
  return prod > ((u128)W << s);
}

// Lowest index among the row's maxima.
__device__ int block_argmax(const float* x, int V, VSmem& sm) {
  float bv = -INFINITY;
  int bi = 0x7FFFFFFF;
  for (int i = threadIdx.x; i < V; i += blockDim.x) {
    float l = x[i];
    if (bi == 0x7FFFFFFF || l > bv) { bv = l; bi = i; }
  }
  float m = block_reduce(bv, sm.scratchf, OpMaxF(), -INFINITY);
  int cand = (bi != 0x7FFFFFFF && bv == m) ? bi : 0x7FFFFFFF;
  int t = block_reduce(cand, sm.scratchi, OpMinI(), 0x7FFFFFFF);
  return t == 0x7FFFFFFF ? 0 : t;
}

__device__ float block_max(const float* x, int V, VSmem& sm) {
  float m = -INFINITY;
  for (int i = threadIdx.x; i < V; i += blockDim.x) m = fmaxf(m, x[i]);
  return block_reduce(m, sm.scratchf, OpMaxF(), -INFINITY);
}

// Integer inverse-CDF draw over weights w(i) in vocabulary order with
// per-thread contiguous segments.  Returns the token (valid on all threads)
// and the total through *total.
template <typename WF>
__device__ int segment_draw(int V, float u, WF w, VSmem& sm, uint64_t* total) {
  const int tid = threadIdx.x, nt = blockDim.x;
  const int seg = (V + nt - 1) / nt;
  const int lo = min(V, tid * seg), hi = min(V, lo + seg);
  uint64_t s = 0;
  for (int i = lo; i < hi; ++i) s += w(i);
  uint64_t tot;
  uint64_t excl = block_exclusive_scan_u64(s, sm.scratch64, &tot);
  *total = tot;
  if (tid == 0) sm.bcasti[0] = 0;
  __syncthreads();
  if (tot) {
    const uint64_t tgt = draw_target(u, tot);
    if (excl <= tgt && tgt < excl + s) {
      uint64_t c = excl;
      for (int i = lo; i < hi; ++i) {
        c += w(i);
        if (c > tgt) { sm.bcasti[0] = i; break; }
      }
    }
  }
  __syncthreads();
  int t = sm.bcasti[0];
  __syncthreads();
  return t;
}

// Draw from a logprob row with weights exp_fix44(r - max r).
__device__ int draw_lp_row(const float* r, int V, float u, VSmem& sm) {
  float m = block_max(r, V, sm);
  uint64_t tot;
  if (m == -INFINITY) return 0;
  return segment_draw(V, u, [&](int i) { return exp_fix44(r[i] - m); }, sm, &tot);
}

__global__ void __launch_bounds__(1024) verify_lp_kernel(VerifyKArgs a) {
  __shared__ VSmem sm;
  const int b = blockIdx.x, tid = threadIdx.x;
  const int n = a.n, V = a.V;
  const float* T = a.target + (long long)b * (n + 1) * V;
  const float* D = a.draft + (long long)b * n * V;
  const int32_t* t = a.tok + (long long)b * n;
  const float* ub = a.u + (long long)b * (n + 1);
  float* row = a.row_out ? a.row_out + (long long)b * V : nullptr;
  if (!(a.T > 0.0f)) {
    int j = 0, am = 0;
    for (; j <= n; ++j) {
      am = block_argmax(T + (long long)j * V, V, sm);
      if (j == n || t[j] != am) break;
    }
    if (tid == 0) { a.accepted[b] = j; a.token[b] = am; }
    if (row) for (int i = tid; i < V; i += blockDim.x) row[i] = T[(long long)j * V + i];
    return;
  }
  if (tid == 0) {
    int j = 0;
    for (; j < n; ++j) {
      int tk = t[j];
      if (tk < 0 || tk >= V) break;
      if (reject_lp(ub[j], T[(long long)j * V + tk], D[(long long)j * V + tk])) break;
    }
    sm.bcasti[1] = j;
  }
  __syncthreads();
  const int j = sm.bcasti[1];
  const float* g = T + (long long)j * V;
  int tok;
  if (j == n) {
    tok = draw_lp_row(g, V, ub[n], sm);
    if (row) for (int i = tid; i < V; i += blockDim.x) row[i] = g[i];
  } else {
    const float* d = D + (long long)j * V;
    auto resid = [&](int i) {
      uint64_t P = exp_fix44(g[i]), Q = exp_fix44(d[i]);
      return P > Q ? P - Q : (uint64_t)0;
    };
    uint64_t S;
    tok = segment_draw(V, ub[n], resid, sm, &S);
    if (S == 0) {
      tok = draw_lp_row(g, V, ub[n], sm);
      if (row) for (int i = tid; i < V; i += blockDim.x) row[i] = g[i];
    } else if (row) {
      const double ls = log((double)S);
      for (int i = tid; i < V; i += blockDim.x) {
        uint64_t w = resid(i);
        row[i] = w ? (float)(log((double)w) - ls) : -INFINITY;
      }
    }
  }
  if (tid == 0) { a.accepted[b] = j; a.token[b] = tok; }
}

// Phase 1 of the fused form: one workgroup per (b, j), j < n.
__global__ void __launch_bounds__(1024) verify_fused_rows_kernel(VerifyKArgs a) {
  __shared__ VSmem sm;
  const int b = blockIdx.x / a.n, j = blockIdx.x % a.n, tid = threadIdx.x;
  const int V = a.V;
  const float* x = a.target + ((long long)b * (a.n + 1) + j) * V;
  const int tk = a.tok[(long long)b * a.n + j];
  const long long slot = (long long)b * a.n + j;
  if (!(a.T > 0.0f)) {
    int am = block_argmax(x, V, sm);
    if (tid == 0) a.rej[slot] = (tk != am);
    return;
  }
  const float m = block_max(x, V, sm);
  uint64_t z = 0;
  if (m != -INFINITY)
    for (int i = tid; i < V; i += blockDim.x) z += exp_fix44((x[i] - m) / a.Tc);
  const uint64_t Z = block_reduce(z, sm.scratch64, OpSumU64(), (uint64_t)0);
  if (tid == 0) {
    bool rj;
    if (tk < 0 || tk >= V) {
      rj = true;
    } else {
      uint64_t W = m == -INFINITY ? 0 : exp_fix44((x[tk] - m) / a.Tc);
      float q = a.draft[slot * V + tk];
      rj = reject_fused(a.u[(long long)b * (a.n + 1) + j], q, Z, W);
    }
    a.rej[slot] = rj ? 1 : 0;
    a.rmax[slot] = m;
    a.rz[slot] = Z;
  }
}

// Phase 2 of the fused form: one workgroup per batch entry.
__global__ void __launch_bounds__(1024) verify_fused_draw_kernel(VerifyKArgs a) {
  __shared__ VSmem sm;
  const int b = blockIdx.x, tid = threadIdx.x;
  const int n = a.n, V = a.V;
  int j = 0;
  while (j < n && !a.rej[(long long)b * n + j]) ++j;
  const float* x = a.target + ((long long)b * (n + 1) + j) * V;
  if (!(a.T > 0.0f)) {
    int am = block_argmax(x, V, sm);
    if (tid == 0) { a.accepted[b] = j; a.token[b] = am; }
    return;
  }
  const float u = a.u[(long long)b * (n + 1) + n];
  float m;
  uint64_t Z;
  if (j < n) {
    m = a.rmax[(long long)b * n + j];
    Z = a.rz[(long long)b * n + j];
  } else {
    m = block_max(x, V, sm);
    uint64_t z = 0;
    if (m != -INFINITY)
      for (int i = tid; i < V; i += blockDim.x) z += exp_fix44((x[i] - m) / a.Tc);
    Z = block_reduce(z, sm.scratch64, OpSumU64(), (uint64_t)0);
  }
  auto wt = [&](int i) { return m == -INFINITY ? (uint64_t)0 : exp_fix44((x[i] - m) / a.Tc); };
  int tok = 0;
  uint64_t tot;
  if (j == n) {
    tok = Z ? segment_draw(V, u, wt, sm, &tot) : 0;
  } else {
    const float* q = a.draft + ((long long)b * n + j) * V;
    auto resid = [&](int i) {
      uint64_t w = wt(i), qz = floor_qz(q[i], Z);
      return w > qz ? w - qz : (uint64_t)0;
    };
    uint64_t S;
    tok = segment_draw(V, u, resid, sm, &S);
    if (S == 0) tok = Z ? segment_draw(V, u, wt, sm, &tot) : 0;
  }
  if (tid == 0) { a.accepted[b] = j; a.token[b] = tok; }
}

static int check_verify(const wh_verify_args* p, bool fused) {
  if (!p) return fail(WH_EINVAL, "args is NULL");
  if (p->B < 0 || p->n < 0) return fail(WH_EINVAL, "B and n must be >= 0");
  if (p->V <= 0 || p->V > WH_MAX_VOCAB) return fail(WH_ELIMIT, "V must be in [1, %d]", WH_MAX_VOCAB);
  if (!(p->temperature >= 0.0f)) return fail(WH_EINVAL, "temperature must be >= 0");
  if (p->B > 0 && (!p->target || !p->accepted || !p->token)) return fail(WH_EINVAL, "target/accepted/token must be set");
  if (p->B > 0 && p->n > 0 && !p->draft_tokens) return fail(WH_EINVAL, "draft_tokens must be set");
  if (p->B > 0 && p->n > 0 && p->temperature > 0.0f && !p->draft) return fail(WH_EINVAL, "draft rows must be set when temperature > 0");
  if (p->B > 0 && p->temperature > 0.0f && !p->uniforms) return fail(WH_EINVAL, "uniforms must be set when temperature > 0");
  if (fused && p->row_out) return fail(WH_EINVAL, "row_out is only produced by wh_verify_logprobs");
  return WH_OK;
}

static VerifyKArgs to_kargs(const wh_verify_args* p) {
  VerifyKArgs k;
  memset(&k, 0, sizeof(k));
  k.B = p->B;
  k.n = p->n;
  k.V = p->V;
  k.T = p->temperature;
  k.Tc = (float)std::fmax((double)p->temperature, 1e-5);
  k.target = p->target;
  k.draft = p->draft;
  k.tok = p->draft_tokens;
  k.u = p->uniforms;
  k.accepted = p->accepted;
  k.token = p->token;
  k.row_out = p->row_out;
  return k;
}

}  // namespace wh

using namespace wh;

extern "C" size_t wh_verify_workspace_bytes(int32_t B, int32_t n, int32_t V) {
  (void)V;
  size_t slots = (size_t)(B > 0 ? B : 0) * (size_t)(n > 0 ? n : 0);
  return slots * 16 + 256;
}

extern "C" int wh_verify_logprobs(const wh_verify_args* args, void* stream) {
  clear_error();
  int rc = check_verify(args, false);
  if (rc) return rc;
  if (args->B == 0) return WH_OK;
  VerifyKArgs k = to_kargs(args);
  hipLaunchKernelGGL(verify_lp_kernel, dim3(k.B), dim3(1024), 0, (hipStream_t)stream, k);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "verify_lp_kernel launch failed: %s", hipGetErrorString(e));
  return WH_OK;
}

extern "C" int wh_verify_fused(const wh_verify_args* args, void* stream) {
  clear_error();
  int rc = check_verify(args, true);
  if (rc) return rc;
  if (args->B == 0) return WH_OK;
  size_t need = wh_verify_workspace_bytes(args->B, args->n, args->V);
  if (args->n > 0 && (!args->workspace || args->workspace_bytes < need))
    return fail(WH_EINVAL, "workspace too small: need %zu bytes", need);
  VerifyKArgs k = to_kargs(args);
  size_t slots = (size_t)args->B * args->n;
  char* ws = (char*)args->workspace;
  k.rz = (unsigned long long*)ws;
  k.rmax = (float*)(ws + slots * 8);
  k.rej = (int32_t*)(ws + slots * 12);
  hipStream_t st = (hipStream_t)stream;
  if (args->n > 0) {
    hipLaunchKernelGGL(verify_fused_rows_kernel, dim3((unsigned)slots), dim3(1024), 0, st, k);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(WH_EHIP, "verify_fused_rows_kernel launch failed: %s", hipGetErrorString(e));
  }
  hipLaunchKernelGGL(verify_fused_draw_kernel, dim3(k.B), dim3(1024), 0, st, k);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "verify_fused_draw_kernel launch failed: %s", hipGetErrorString(e));
  return WH_OK;
}
