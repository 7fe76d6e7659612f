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
#include <atomic>
#include <cmath>
#include <cstdlib>

#include "wh_common.h"
#include "wh_internal.h"

namespace wh {

struct VerifyKArgs {
  int B, n, V;
  float T;     // temperature
  float Tc;    // fl32(max(T, 1e-5))
  double rTc;  // 1 / (double)Tc: divisions by Tc as exact multiplies
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
  double scratchd[16];
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

// floor(q Z) for q clamped to [0, 1] (NaN and q <= 0 give 0), Z < 2^62, from
// q's bits: q <= 0, NaN or q < 2^-62 (then q Z < 1) give 0, q >= 1 gives Z;
// otherwise q = M 2^-s with the 24-bit significand M and s = 150 - E in
// [23, 85], and M Z = hi 2^32 + lo is shifted in two 64-bit pieces as in
// floor_theta_z.  Equal to floor_theta_z(q, Z) for every float q.
__device__ __forceinline__ uint64_t floor_qz(float q, uint64_t Z) {
  const uint32_t b = __float_as_uint(q);
  if ((int32_t)b <= 0 || b > 0x7F800000u) return 0;
  if (b >= 0x3F800000u) return Z;
  const int E = (int)(b >> 23);  // biased exponent, 1..126 here
  if (E < 65) return 0;
  const uint64_t M = (b & 0x7FFFFFu) | 0x800000u;
  const int s = 150 - E;  // 24..85: both shifts below stay in [0, 53]
  const uint64_t lo = M * (Z & 0xFFFFFFFFull), hi = M * (Z >> 32);
  return s <= 32 ? (hi << (32 - s)) + (lo >> s) : (hi + (lo >> 32)) >> (s - 32);
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
    for (int i = tid; i < V; i += blockDim.x) z += exp_fix44(div_by_recip(x[i] - m, a.rTc));
  const uint64_t Z = block_reduce(z, sm.scratch64, OpSumU64(), (uint64_t)0);
  if (tid == 0) {
    bool rj;
    if (tk < 0 || tk >= V) {
      rj = true;
    } else {
      uint64_t W = m == -INFINITY ? 0 : exp_fix44(div_by_recip(x[tk] - m, a.rTc));
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
      for (int i = tid; i < V; i += blockDim.x) z += exp_fix44(div_by_recip(x[i] - m, a.rTc));
    Z = block_reduce(z, sm.scratch64, OpSumU64(), (uint64_t)0);
  }
  auto wt = [&](int i) { return m == -INFINITY ? (uint64_t)0 : exp_fix44(div_by_recip(x[i] - m, a.rTc)); };
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

// ---------------------------------------------------------------------------
// Fused form, T > 0: sliced passes instead of one workgroup per row.
//   1. verify_sum_kernel, one 256-thread workgroup per slice of every target
//      row (about eight per CU): the slice's exact max and a float sum of
//      exp((x - max) / T), from loads that are all issued before any is used.
//      One HBM pass over the target rows.  The first slice's workgroup also
//      records the target logit and draft probability at the row's draft
//      token.
//   2. verify_prep_kernel, G2 workgroups per batch entry (slices of at most
//      4096 ids, about four workgroups per CU): each recomputes the
//      accept / reject decisions from the row summaries -- the normaliser Z
//      lies in [Zlo, Zhi] from the float sums, and u q Z > W is decided from
//      both ends (W exact, from the draft token's logit); the first
//      rejection j* is settled unless a test falls between them -- then sums
//      the exact fixed-point weights of its slice of row j*.
//   3. verify_resid_kernel: with the exact Z of row j*, the slice's residual
//      mass sum max(W_i - floor(q_i Z), 0).
//   4. verify_pick_kernel, one workgroup per batch entry: the slice holding
//      the draw target, then the element inside it.  A batch entry whose
//      decisions were not settled by the bounds runs the exact per-row
//      algorithm here instead (identical results, slower).
// ---------------------------------------------------------------------------
constexpr int VT1 = 256;       // threads, pass 1
constexpr int VL1 = 8;         // float4 loads per thread, pass 1
constexpr int VE1 = 4 * VL1 * VT1;  // elements per pass-1 slice, at most (8192)
constexpr int VBLK1 = 2048;    // pass-1 workgroups aimed for (eight per CU)
constexpr int VG1MAX = 64;     // pass-1 slices per row, at most (one wave lane each)
constexpr int VT2 = 256;       // threads, passes 2 and 3 (NQ float4 per thread, NQ = 2 or 4)
constexpr int VT3 = 1024;      // threads, pass 4
constexpr int VG2MAX = 64;     // slices of the selected row, at most (one wave lane each)
constexpr int VSEG4 = 1;       // float4 groups per thread in the final draw
constexpr int VE2 = 4 * VSEG4 * VT3;  // ids per slice of the selected row, at most (4096)
constexpr double VEPS = 2e-4;  // relative slack of the float normaliser
// a slice of the selected row fits the final draw's registers and the
// prep / residual passes' loads (4 float4 per thread at most)
static_assert(VE2 == 4 * 4 * VT2, "sliced verify: 4 float4 per thread cover a slice");
static_assert((WH_MAX_VOCAB + VE2 - 1) / VE2 <= VG2MAX, "slices of the selected row fit one wave's lanes");
static_assert((WH_MAX_VOCAB + VE1 - 1) / VE1 <= VG1MAX, "pass-1 slices of a row fit one wave's lanes");

struct VRowSum {
  float m;
  float pad;
  double zf;  // sum of exp((x - m) / T) over the slice (hardware exp)
};

// The target logit and draft probability at row j's draft token.
struct VTokRec {
  float xt, q;
};

struct VPlan {
  int G1, SL1, G2, SL2;
  int force_exact;  // test hook: every batch entry takes the exact per-row algorithm
  VRowSum* summ;  // [B, n+1, G1]
  VTokRec* trec;  // [B, n]
  int32_t* jst;   // [B, 4]: j*, undecided flag, bits of row j*'s max, unused
  unsigned long long* zpart;  // [B, G2] exact weights of row j*
  unsigned long long* rpart;  // [B, G2] residual mass of row j*
};

// (x - m) / Tc, exactly as the division rounds (rTc = 1 / (double)Tc)
__device__ __forceinline__ float vweight_arg(float x, float m, double rTc) { return div_by_recip(x - m, rTc); }

__global__ void __launch_bounds__(VT1) verify_sum_kernel(VerifyKArgs a, VPlan P) {
  __shared__ float s_m[VT1 / 64];
  __shared__ double s_z[VT1 / 64];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int rj = blockIdx.x / P.G1, s = blockIdx.x - rj * P.G1;
  const int V = a.V, n = a.n;
  const int v0 = s * P.SL1, v1 = min(V, v0 + P.SL1);
  const float* row = a.target + (long long)rj * V;
  // every load of the thread is issued before any is used; positions past
  // the slice (which may be empty) read the row's first float4 and are ignored
  float4 c[VL1];
#pragma unroll
  for (int k = 0; k < VL1; ++k) {
    const int i = v0 + (tid + k * VT1) * 4;
    c[k] = *(const float4*)(row + (i < v1 ? i : 0));
  }
  // the first slice's workgroup records the draft token's logit and draft
  // probability for the accept tests (rows j < n only)
  const int b = rj / (n + 1), j = rj - b * (n + 1);
  if (s == 0 && j < n && tid == 0) {
    const int tk = a.tok[(long long)b * n + j];
    if (tk >= 0 && tk < V) {
      VTokRec r;
      r.xt = row[tk];
      r.q = a.draft[((long long)b * n + j) * V + tk];
      P.trec[(long long)b * n + j] = r;
    }
  }
  float mt = -INFINITY;
#pragma unroll
  for (int k = 0; k < VL1; ++k) {
    const int i = v0 + (tid + k * VT1) * 4;
    if (i < v1) mt = fmaxf(mt, fmaxf(fmaxf(c[k].x, c[k].y), fmaxf(c[k].z, c[k].w)));
  }
  mt = wmax_f(mt);
  if (lane == 0) s_m[w] = mt;
  __syncthreads();
  float m = s_m[0];
#pragma unroll
  for (int k = 1; k < VT1 / 64; ++k) m = fmaxf(m, s_m[k]);
  // exp((x - m) / T) = 2^((x - m) log2(e) / T), hardware exp2; the float
  // sum of at most 32 terms per lane, then doubles
  float st = 0.0f;
  if (m != -INFINITY) {
    const float k2 = 1.44269504088896341f / a.Tc;
#pragma unroll
    for (int k = 0; k < VL1; ++k) {
      const int i = v0 + (tid + k * VT1) * 4;
      if (i < v1) {
        st += __builtin_amdgcn_exp2f((c[k].x - m) * k2) + __builtin_amdgcn_exp2f((c[k].y - m) * k2);
        st += __builtin_amdgcn_exp2f((c[k].z - m) * k2) + __builtin_amdgcn_exp2f((c[k].w - m) * k2);
      }
    }
  }
  const double zw = wsum_f64((double)st);
  if (lane == 0) s_z[w] = zw;
  __syncthreads();
  if (tid == 0) {
    double zs = 0.0;
#pragma unroll
    for (int k = 0; k < VT1 / 64; ++k) zs += s_z[k];
    VRowSum o;
    o.m = m;
    o.pad = 0.0f;
    o.zf = zs;
    P.summ[blockIdx.x] = o;
  }
}

// Row j's max and the proven interval of its fixed-point normaliser, from
// its slice summaries.  Every lane of a full wave calls it; lane l < G1
// passes slice l's summary (valid), and every lane gets the results.
__device__ __forceinline__ void vrow_bounds_w(const VRowSum& r, bool valid, float iT, int V, float* m_out,
                                              uint64_t* zlo, uint64_t* zhi) {
  const float m = wmax_f(valid ? r.m : -INFINITY);
  // the float rescale's relative error (a few ulp, with iT = fl(1 / T)) is
  // far inside VEPS
  const double t = (valid && m != -INFINITY && r.m != -INFINITY) ? r.zf * (double)__expf((r.m - m) * iT) : 0.0;
  const double zf = wsum_f64(t);
  const double SC = 17592186044416.0, LIM = 4.0e18;
  const double lo = zf * SC * (1.0 - VEPS) - (double)V, hi = zf * SC * (1.0 + VEPS) + (double)V;
  *m_out = m;
  *zlo = (m == -INFINITY || lo <= 0.0) ? 0ull : (uint64_t)lo;
  *zhi = m == -INFINITY ? 0ull : (hi >= LIM ? (1ull << 62) : (uint64_t)ceil(hi));
}

// The sum of cnt <= 64 per-slice partial sums: lane s reads one, so the
// reads are a single round trip, and a DPP reduction finishes them; every
// lane of the (full) wave gets the result.
__device__ __forceinline__ uint64_t vparts_sum_w(const unsigned long long* p, int cnt) {
  const int lane = threadIdx.x & 63;
  return wsum_u64(lane < cnt ? (uint64_t)p[lane] : 0ull);
}

template <int NQ>
__global__ void __launch_bounds__(VT2) verify_prep_kernel(VerifyKArgs a, VPlan P) {
  constexpr int NWV = VT2 / 64;              // waves
  constexpr int RPW = (64 + NWV - 1) / NWV;  // rows j <= n < 64 per wave
  __shared__ VSmem sm;
  __shared__ int s_state[64];
  __shared__ float s_m[64];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int b = blockIdx.x / P.G2, s = blockIdx.x - b * P.G2;
  const int n = a.n, V = a.V, G1 = P.G1;
  // One round trip: wave w reads the slice summaries of rows j = w + NWV q
  // (lane l: slice l), and its lane q the draft token, uniform and token
  // record of row w + NWV q.
  VRowSum r[RPW];
#pragma unroll
  for (int q = 0; q < RPW; ++q) {
    const int j = w + NWV * q;
    r[q].m = -INFINITY;
    r[q].zf = 0.0;
    if (j <= n && lane < G1) r[q] = P.summ[((long long)b * (n + 1) + j) * G1 + lane];
  }
  const int jl = w + NWV * lane;
  int tk = -1;
  float u = 0.0f;
  VTokRec tr;
  tr.xt = 0.0f;
  tr.q = 0.0f;
  if (lane < RPW && jl < n) {
    tk = a.tok[(long long)b * n + jl];
    u = a.u[(long long)b * (n + 1) + jl];
    tr = P.trec[(long long)b * n + jl];
  }
  // every row's max and bounds (wave-wide), and for rows j < n the accept
  // test by lane q: 0 accept, 1 reject, 2 undecided by the bounds
#pragma unroll
  for (int q = 0; q < RPW; ++q) {
    const int j = w + NWV * q;
    if (j <= n) {
      float m;
      uint64_t zlo, zhi;
      vrow_bounds_w(r[q], lane < G1, (float)a.rTc, V, &m, &zlo, &zhi);
      if (lane == q) {
        s_m[j] = m;
        if (j < n) {
          int st;
          if (tk < 0 || tk >= V) {
            st = 1;
          } else {
            const uint64_t W = m == -INFINITY ? 0ull : exp_fix44(vweight_arg(tr.xt, m, a.rTc));
            if (reject_fused(u, tr.q, zlo, W)) st = 1;
            else if (!reject_fused(u, tr.q, zhi, W)) st = 0;
            else st = 2;
          }
          s_state[j] = st;
        }
      }
    }
  }
  __syncthreads();
  // j*, the first position not accepted (n when all are)
  if (w == 0) {
    const int st = lane < n ? s_state[lane] : 0;
    const unsigned long long nz = __ballot(st != 0);
    const int j = nz ? (int)__ffsll((long long)nz) - 1 : n;
    const int und = ((nz && s_state[j] == 2) || P.force_exact) ? 1 : 0;
    if (lane == 0) {
      sm.bcasti[0] = j;
      sm.bcasti[1] = und;
      if (s == 0) *(int4*)(P.jst + 4 * b) = make_int4(j, und, __float_as_int(s_m[j]), 0);
    }
  }
  __syncthreads();
  const int js = sm.bcasti[0];
  if (sm.bcasti[1]) return;
  const float m = s_m[js];
  const float* x = a.target + ((long long)b * (n + 1) + js) * V;
  const int v0 = s * P.SL2, v1 = min(V, v0 + P.SL2);
  // the slice (at most NQ float4 per thread: SL2 <= 4 NQ VT2); positions
  // past the slice (the slice may be empty) read the row's first float4 and
  // are ignored
  float4 c[NQ];
#pragma unroll
  for (int k = 0; k < NQ; ++k) {
    const int i = v0 + (tid + k * VT2) * 4;
    c[k] = *(const float4*)(x + (i < v1 ? i : 0));
  }
  uint64_t z = 0;
#pragma unroll
  for (int k = 0; k < NQ; ++k) {
    const int i = v0 + (tid + k * VT2) * 4;
    if (m != -INFINITY && i < v1) {
      z += exp_fix44(vweight_arg(c[k].x, m, a.rTc)) + exp_fix44(vweight_arg(c[k].y, m, a.rTc));
      z += exp_fix44(vweight_arg(c[k].z, m, a.rTc)) + exp_fix44(vweight_arg(c[k].w, m, a.rTc));
    }
  }
  const uint64_t zt = block_reduce(z, sm.scratch64, OpSumU64(), (uint64_t)0);
  if (tid == 0) P.zpart[(long long)b * P.G2 + s] = zt;
}

template <int NQ>
__global__ void __launch_bounds__(VT2) verify_resid_kernel(VerifyKArgs a, VPlan P) {
  __shared__ VSmem sm;
  const int tid = threadIdx.x;
  const int b = blockIdx.x / P.G2, s = blockIdx.x - b * P.G2;
  const int n = a.n, V = a.V;
  const int4 jr = *(const int4*)(P.jst + 4 * b);
  const int js = jr.x;
  if (jr.y || js >= n) return;
  const float m = __int_as_float(jr.z);
  const float* x = a.target + ((long long)b * (n + 1) + js) * V;
  const float* q = a.draft + ((long long)b * n + js) * V;
  const int v0 = s * P.SL2, v1 = min(V, v0 + P.SL2);
  // the slice (at most NQ float4 of each row per thread) and the partial
  // sums are read in one round trip; positions past the slice read the row's
  // first float4 and are ignored
  float4 c[NQ], d[NQ];
#pragma unroll
  for (int k = 0; k < NQ; ++k) {
    const int i = v0 + (tid + k * VT2) * 4, ic = i < v1 ? i : 0;
    c[k] = *(const float4*)(x + ic);
    d[k] = *(const float4*)(q + ic);
  }
  const uint64_t Z = vparts_sum_w(P.zpart + (long long)b * P.G2, P.G2);
  uint64_t r = 0;
  auto res = [&](float xv, float qv) {
    const uint64_t w = m == -INFINITY ? 0ull : exp_fix44(vweight_arg(xv, m, a.rTc));
    const uint64_t qz = floor_qz(qv, Z);
    return w > qz ? w - qz : (uint64_t)0;
  };
#pragma unroll
  for (int k = 0; k < NQ; ++k) {
    const int i = v0 + (tid + k * VT2) * 4;
    if (i < v1) r += res(c[k].x, d[k].x) + res(c[k].y, d[k].y) + res(c[k].z, d[k].z) + res(c[k].w, d[k].w);
  }
  const uint64_t rt = block_reduce(r, sm.scratch64, OpSumU64(), (uint64_t)0);
  if (tid == 0) P.rpart[(long long)b * P.G2 + s] = rt;
}

// The first index in [lo, hi) whose inclusive weight sum exceeds rem (the
// weights there sum to more than rem).  Thread t owns the contiguous segment
// [lo + 4 SEG4 t, lo + 4 SEG4 (t + 1)); its weights are computed once, from
// float4 loads issued together, and kept in registers for both passes.
// Requires hi - lo <= 4 * SEG4 * blockDim.x and lo % 4 == hi % 4 == 0.
template <int SEG4, typename WF>
__device__ int segment_find(int lo, int hi, uint64_t rem, const float* x, const float* q, WF w, VSmem& sm) {
  const int tid = threadIdx.x;
  const int a0 = lo + tid * 4 * SEG4;
  float4 cx[SEG4], cq[SEG4];
#pragma unroll
  for (int k = 0; k < SEG4; ++k) {
    const int i = a0 + 4 * k;
    const int ic = i < hi ? i : lo;
    cx[k] = *(const float4*)(x + ic);
    cq[k] = q ? *(const float4*)(q + ic) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  uint64_t wv[4 * SEG4];
  uint64_t sum = 0;
#pragma unroll
  for (int e = 0; e < 4 * SEG4; ++e) wv[e] = 0ull;
  if (a0 < hi) {  // whole waves past the slice skip the weights
#pragma unroll
    for (int k = 0; k < SEG4; ++k) {
      const bool in = a0 + 4 * k < hi;
      wv[4 * k] = in ? w(cx[k].x, cq[k].x) : 0ull;
      wv[4 * k + 1] = in ? w(cx[k].y, cq[k].y) : 0ull;
      wv[4 * k + 2] = in ? w(cx[k].z, cq[k].z) : 0ull;
      wv[4 * k + 3] = in ? w(cx[k].w, cq[k].w) : 0ull;
      sum += wv[4 * k] + wv[4 * k + 1] + wv[4 * k + 2] + wv[4 * k + 3];
    }
  }
  uint64_t tot;
  const uint64_t excl = block_exclusive_scan_u64(sum, sm.scratch64, &tot);
  if (tid == 0) sm.bcasti[2] = lo;
  __syncthreads();
  if (excl <= rem && rem < excl + sum) {
    uint64_t c = excl;
    int hit = -1;
#pragma unroll
    for (int e = 0; e < 4 * SEG4; ++e) {
      c += wv[e];
      if (hit < 0 && c > rem) hit = e;
    }
    sm.bcasti[2] = a0 + hit;
  }
  __syncthreads();
  return sm.bcasti[2];
}

// The exact per-row algorithm for batch entry b by one workgroup: every
// row's max and normaliser by block reductions, the tests in order, then the
// residual (or bonus) draw over the whole row.
__device__ void verify_exact_entry(const VerifyKArgs& a, int b, VSmem& sm) {
  const int tid = threadIdx.x, n = a.n, V = a.V;
  int j = 0;
  float m = -INFINITY;
  uint64_t Z = 0;
  for (; j <= n; ++j) {
    const float* x = a.target + ((long long)b * (n + 1) + j) * V;
    m = block_max(x, V, sm);
    uint64_t z = 0;
    if (m != -INFINITY)
      for (int i = tid; i < V; i += blockDim.x) z += exp_fix44(vweight_arg(x[i], m, a.rTc));
    Z = block_reduce(z, sm.scratch64, OpSumU64(), (uint64_t)0);
    if (j == n) break;
    const int tk = a.tok[(long long)b * n + j];
    bool rj;
    if (tk < 0 || tk >= V) {
      rj = true;
    } else {
      const uint64_t W = m == -INFINITY ? 0ull : exp_fix44(vweight_arg(x[tk], m, a.rTc));
      rj = reject_fused(a.u[(long long)b * (n + 1) + j], a.draft[((long long)b * n + j) * V + tk], Z, W);
    }
    if (rj) break;
  }
  const float* x = a.target + ((long long)b * (n + 1) + j) * V;
  const float u = a.u[(long long)b * (n + 1) + n];
  auto wt = [&](int i) { return m == -INFINITY ? (uint64_t)0 : exp_fix44(vweight_arg(x[i], m, a.rTc)); };
  int tok = 0;
  uint64_t tot;
  if (j == n) {
    tok = Z ? segment_draw(V, u, wt, sm, &tot) : 0;
  } else {
    const float* q = a.draft + ((long long)b * n + j) * V;
    auto resid = [&](int i) {
      const uint64_t w = wt(i), qz = floor_qz(q[i], Z);
      return w > qz ? w - qz : (uint64_t)0;
    };
    uint64_t S;
    tok = segment_draw(V, u, resid, sm, &S);
    if (S == 0) tok = Z ? segment_draw(V, u, wt, sm, &tot) : 0;
  }
  if (tid == 0) {
    a.accepted[b] = j;
    a.token[b] = tok;
  }
}

__global__ void __launch_bounds__(VT3) verify_pick_kernel(VerifyKArgs a, VPlan P) {
  __shared__ VSmem sm;
  const int b = blockIdx.x, tid = threadIdx.x;
  const int n = a.n, V = a.V;
  // j*, its row max and lane t's partial sums of slice t in one round trip
  // (the residual sums exist only when j* < n); DPP sums and a scan over the
  // lanes pick the slice
  const int lane = tid & 63;
  const bool ls = lane < P.G2;
  const int4 jr = *(const int4*)(P.jst + 4 * b);
  const uint64_t zp = ls ? (uint64_t)P.zpart[(long long)b * P.G2 + lane] : 0ull;
  const uint64_t rraw = ls ? (uint64_t)P.rpart[(long long)b * P.G2 + lane] : 0ull;
  const float ub = a.u[(long long)b * (n + 1) + n];
  if (jr.y) {
    verify_exact_entry(a, b, sm);
    return;
  }
  const int js = jr.x;
  const float m = __int_as_float(jr.z);
  const uint64_t rp = js < n ? rraw : 0ull;
  const uint64_t Z = wsum_u64(zp), R = wsum_u64(rp);
  // residual mass when rejected and positive, else the row's own weights
  const bool use_r = js < n && R > 0;
  const uint64_t part = use_r ? rp : zp;
  const uint64_t total = use_r ? R : Z;
  const uint64_t incl = wscan_incl_u64(part);
  int tok = 0;
  if (total) {
    const uint64_t tgt = draw_target(ub, total);
    // the first slice whose inclusive sum exceeds the target (lane 63 holds
    // the total, which does)
    const int ss = (int)__ffsll((long long)__ballot(incl > tgt)) - 1;
    const uint64_t rem = tgt - (lane_u64(incl, ss) - lane_u64(part, ss));
    const float* x = a.target + ((long long)b * (n + 1) + js) * V;
    const int v0 = ss * P.SL2, v1 = min(V, v0 + P.SL2);
    auto wt = [&](float xv) { return m == -INFINITY ? (uint64_t)0 : exp_fix44(vweight_arg(xv, m, a.rTc)); };
    if (use_r) {
      const float* q = a.draft + ((long long)b * n + js) * V;
      tok = segment_find<VSEG4>(v0, v1, rem, x, q, [&](float xv, float qv) {
        const uint64_t w = wt(xv), qz = floor_qz(qv, Z);
        return w > qz ? w - qz : (uint64_t)0;
      }, sm);
    } else {
      tok = segment_find<VSEG4>(v0, v1, rem, x, nullptr, [&](float xv, float) { return wt(xv); }, sm);
    }
  }
  if (tid == 0) {
    a.accepted[b] = js;
    a.token[b] = tok;
  }
}

struct VHostPlan {
  int G1, SL1, G2, SL2;
  size_t summ, trec, jst, zpart, rpart, total;
};

// Workspace: the per-position slots of the one-workgroup-per-row form, then
// the sliced form's row summaries and per-entry sums.
static VHostPlan vplan(int B, int n, int V) {
  VHostPlan h;
  // enough pass-1 slices to fill the chip (at least 1024 ids each), and at
  // least enough that each fits one workgroup's loads
  const int rows = std::max(1, std::max(B, 0) * (std::max(n, 0) + 1));
  const int g_fill = std::min({VG1MAX, (VBLK1 + rows - 1) / rows, (V + 4 * VT1 - 1) / (4 * VT1)});
  h.G1 = std::max({1, (V + VE1 - 1) / VE1, g_fill});
  h.SL1 = ((V + h.G1 - 1) / h.G1 + 3) / 4 * 4;
  // slices of the selected row: about 1024 prep / residual workgroups (four
  // per CU) and small slices for the one-workgroup final draw, at least 1024
  // ids each; a slice must fit the final draw's register segments
  const int Bp = std::max(B, 1);
  h.G2 = std::max(1, std::min({VG2MAX, (1024 + Bp - 1) / Bp, (V + 1023) / 1024}));
  h.G2 = std::max(h.G2, (V + VE2 - 1) / VE2);
  h.SL2 = ((V + h.G2 - 1) / h.G2 + 3) / 4 * 4;
  const size_t slots = (size_t)std::max(B, 0) * (size_t)std::max(n, 0);
  size_t off = (slots * 16 + 255) / 256 * 256;
  h.summ = off;
  off += (size_t)std::max(B, 0) * (std::max(n, 0) + 1) * h.G1 * sizeof(VRowSum);
  h.trec = off;
  off += (size_t)std::max(B, 0) * std::max(n, 0) * sizeof(VTokRec);
  off = (off + 15) / 16 * 16;
  h.jst = off;
  off += (size_t)std::max(B, 0) * 16;
  off = (off + 15) / 16 * 16;
  h.zpart = off;
  off += (size_t)std::max(B, 0) * h.G2 * 8;
  h.rpart = off;
  off += (size_t)std::max(B, 0) * h.G2 * 8;
  h.total = off + 256;
  return h;
}

// Test hook (wh_verify_force_exact): route every batch entry of the sliced
// verifier through the exact per-row algorithm that entries undecided by the
// bounds take.  Off unless a test sets it.
static std::atomic<int> g_verify_force_exact{0};

extern "C" int wh_verify_force_exact(int on) { return g_verify_force_exact.exchange(on ? 1 : 0); }

static int launch_verify_sliced(const VerifyKArgs& k, const VHostPlan& h, char* ws, hipStream_t st) {
  VPlan P;
  P.force_exact = g_verify_force_exact.load(std::memory_order_relaxed);
  P.G1 = h.G1;
  P.SL1 = h.SL1;
  P.G2 = h.G2;
  P.SL2 = h.SL2;
  P.summ = (VRowSum*)(ws + h.summ);
  P.trec = (VTokRec*)(ws + h.trec);
  P.jst = (int32_t*)(ws + h.jst);
  P.zpart = (unsigned long long*)(ws + h.zpart);
  P.rpart = (unsigned long long*)(ws + h.rpart);
  hipLaunchKernelGGL(verify_sum_kernel, dim3(k.B * (k.n + 1) * h.G1), dim3(VT1), 0, st, k, P);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "verify_sum_kernel launch failed: %s", hipGetErrorString(e));
  // float4 loads per thread in the prep and residual passes
  const bool nq2 = h.SL2 <= 2 * 4 * VT2;
  if (nq2) hipLaunchKernelGGL(verify_prep_kernel<2>, dim3(k.B * h.G2), dim3(VT2), 0, st, k, P);
  else hipLaunchKernelGGL(verify_prep_kernel<4>, dim3(k.B * h.G2), dim3(VT2), 0, st, k, P);
  e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "verify_prep_kernel launch failed: %s", hipGetErrorString(e));
  if (nq2) hipLaunchKernelGGL(verify_resid_kernel<2>, dim3(k.B * h.G2), dim3(VT2), 0, st, k, P);
  else hipLaunchKernelGGL(verify_resid_kernel<4>, dim3(k.B * h.G2), dim3(VT2), 0, st, k, P);
  e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "verify_resid_kernel launch failed: %s", hipGetErrorString(e));
  hipLaunchKernelGGL(verify_pick_kernel, dim3(k.B), dim3(VT3), 0, st, k, P);
  e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "verify_pick_kernel launch failed: %s", hipGetErrorString(e));
  return WH_OK;
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
  k.rTc = 1.0 / (double)k.Tc;
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
  return vplan(B, n, V > 0 ? V : 1).total;
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
  hipStream_t st0 = (hipStream_t)stream;
  // the sliced passes need 16-byte aligned rows (float4 loads) and
  // workspace (16-byte records), and n < 64
  const VHostPlan vh = vplan(args->B, args->n, args->V);
  const bool sliced = args->temperature > 0.0f && args->n > 0 && args->n < 64 && args->V % 4 == 0 &&
                      (uintptr_t)args->target % 16 == 0 && (uintptr_t)args->draft % 16 == 0 && ws &&
                      (uintptr_t)ws % 16 == 0;
  if (sliced) return launch_verify_sliced(k, vh, ws, st0);
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
