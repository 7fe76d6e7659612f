// wh_rowops.h -- per-row building blocks shared by the exact engine and the
// sliced single-read engine: the penalised row view, filter predicates, radix
// select over (value, id) composites, and the complete exact per-row
// algorithm (exact_row), which the sliced engine also falls back to.
#pragma once
#include <cmath>

#include "wh_common.h"
#include "wh_internal.h"

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
  // The same from an already loaded raw(i).
  __device__ __forceinline__ float val_from(int i, float r) const {
    if (hmask >= 0 && ((bitmap[i >> 5] >> (i & 31)) & 1u)) return lookup(i);
    return r + 0.0f;
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
  float cov;     // keep iff value >= cov (restricts a search to a covered region)
  __device__ __forceinline__ bool keep(int i, float l) const {
    if (none) return false;
    if (!(l >= cov)) return false;
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
// Only history tokens in [lo, hi) are entered; the bitmap covers [lo, hi).
__device__ void build_penalties(const SampleKArgs& a, int b, RowCtx& rc, char* dyn, int lo, int hi) {
  const int tid = threadIdx.x, nt = blockDim.x;
  const int hcap = a.hcap;
  int32_t* hkeys = (int32_t*)dyn;
  int32_t* hpos = hkeys + hcap;
  int32_t* hcnt = hpos + hcap;
  uint32_t* bitmap = (uint32_t*)(hcnt + hcap);
  const int words = (hi - lo + 31) >> 5;
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
  const int32_t* h = a.hist + (long long)(b / a.hshare) * a.hist_stride;
  for (int j = len - W + tid; j < len; j += nt) {
    int t = h[j];
    if (t < lo || t >= hi || t >= a.V) continue;
    uint32_t s = ((uint32_t)t * 2654435761u) >> rc.hshift;
    while (true) {
      int old = atomicCAS(&hkeys[s], -1, t);
      if (old == -1 || old == t) break;
      s = (s + 1) & rc.hmask;
    }
    atomicMax(&hpos[s], j);
    if (j >= len - wf) atomicAdd(&hcnt[s], 1);
    atomicOr(&bitmap[(t - lo) >> 5], 1u << ((t - lo) & 31));
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

// Element sources for radix_select: the whole penalised row, or a list of
// (value, id) candidates held in LDS.
struct RowSource {
  const RowCtx* rc;
  template <typename F>
  __device__ __forceinline__ void each(F f) const {
    for (int i = threadIdx.x; i < rc->V; i += blockDim.x) f(i, rc->val(i));
  }
};
struct CandSource {
  const float* v;
  const int* id;
  int n;
  template <typename F>
  __device__ __forceinline__ void each(F f) const {
    for (int j = threadIdx.x; j < n; j += blockDim.x) f(id[j], v[j]);
  }
};

enum { ORD_A = 0, ORD_P = 1, ORD_ID = 2 };

template <int ORD>
__device__ __forceinline__ uint64_t composite(float l, int i) {
  if (ORD == ORD_ID) return (uint64_t)(0x3FFFF - i);  // vocabulary order
  uint32_t k = fkey(l);
  return ORD == ORD_P ? comp_p(k, i) : comp_a(k, i);
}

// Radix select in descending composite order (ORD_A: value desc, id asc;
// ORD_P: value desc, id desc; ORD_ID: id asc).  Returns the composite of
// the element at which the cumulative measure meas(i, l) over elements kept
// by `pr` first reaches `target` (0 < target <= total).  10-bit digits: five
// passes for the 50-bit value/id composites, two for ORD_ID.  With SKIP (for
// short candidate lists, whose composites often share their top bits), one
// min/max pass first drops the digits every kept composite shares, which
// would otherwise send every atomic of a pass to one bin.
template <int ORD, bool SKIP = false, typename Src, typename Meas>
__device__ uint64_t radix_select(const Src& src, const Pred& pr, Meas meas, uint64_t target, ExactSmem& sm) {
  const int tid = threadIdx.x;
  int PASSES = ORD == ORD_ID ? 2 : 5;
  uint64_t prefix = 0;
  if (SKIP) {
    uint64_t cmin = ~0ull, cmax = 0;
    src.each([&](int i, float l) {
      if (!pr.keep(i, l)) return;
      const uint64_t c = composite<ORD>(l, i);
      cmin = c < cmin ? c : cmin;
      cmax = c > cmax ? c : cmax;
    });
    cmin = block_reduce(cmin, sm.scratch64, OpMinU64(), (uint64_t)~0ull);
    cmax = block_reduce(cmax, sm.scratch64, OpMaxU64(), (uint64_t)0);
    if (cmax < cmin) return 0;
    const uint64_t diff = cmin ^ cmax;
    const int top = diff ? 64 - __clzll((long long)diff) : 1;
    PASSES = (top + 9) / 10;
    prefix = cmax >> (10 * PASSES);
  }
  for (int pass = 0; pass < PASSES; ++pass) {
    const int shift = 10 * (PASSES - 1 - pass);
    for (int i = tid; i < 1024; i += blockDim.x) sm.hist[i] = 0;
    __syncthreads();
    src.each([&](int i, float l) {
      if (!pr.keep(i, l)) return;
      uint64_t c = composite<ORD>(l, i);
      if ((c >> (shift + 10)) != prefix) return;
      uint64_t w = meas(i, l);
      if (w) atomicAdd((unsigned long long*)&sm.hist[(c >> shift) & 1023], (unsigned long long)w);
    });
    __syncthreads();
    // suffix sums from the top bin: thread t owns the 1024 / blockDim bins
    // 1023 - t * per .. 1024 - (t + 1) * per, in descending order
    const int per = 1024 / (int)blockDim.x;
    const int top = 1023 - tid * per;
    uint64_t ls = 0;
    for (int q = 0; q < per; ++q) ls += sm.hist[top - q];
    uint64_t tot;
    uint64_t c = block_exclusive_scan_u64(ls, sm.scratch64, &tot);
    if (c < target && c + ls >= target) {
      for (int q = 0; q < per; ++q) {
        const uint64_t hv = sm.hist[top - q];
        if (c < target && c + hv >= target) {
          sm.bcast64[0] = (uint64_t)(top - q);
          sm.bcast64[1] = c;
        }
        c += hv;
      }
    }
    __syncthreads();
    prefix = (prefix << 10) | sm.bcast64[0];
    target -= sm.bcast64[1];
    __syncthreads();
  }
  return prefix;
}

// The composite (order ORD) of the k-th largest kept element, the answer of
// radix_select<ORD> counting to target k (k >= 1), in *cut; false (no cut)
// when at most k elements are kept.  Below
// the bits every kept composite shares, 11-bit histogram passes (2048 32-bit
// bins, atomics in LDS) narrow the prefix only until the chosen bin holds at
// most 64 elements; those are gathered to an LDS list, and one wave ranks
// them (each lane counts the listed composites above its own from broadcast
// reads).  On continuous values one pass usually suffices, against the
// radix descent's pass per 10 bits until a bin of count one.
template <int ORD, typename Src>
__device__ bool block_kth_desc(const Src& src, const Pred& pr, uint64_t k, ExactSmem& sm, uint64_t* cut) {
  const int tid = threadIdx.x;
  uint64_t cmin = ~0ull, cmax = 0;
  int cnt = 0;
  src.each([&](int i, float l) {
    if (!pr.keep(i, l)) return;
    const uint64_t c = composite<ORD>(l, i);
    cmin = c < cmin ? c : cmin;
    cmax = c > cmax ? c : cmax;
    ++cnt;
  });
  cnt = block_reduce(cnt, sm.scratchi, OpSumI(), 0);
  if ((uint64_t)cnt <= k) return false;
  cmin = block_reduce(cmin, sm.scratch64, OpMinU64(), (uint64_t)~0ull);
  cmax = block_reduce(cmax, sm.scratch64, OpMaxU64(), (uint64_t)0);
  const uint64_t diff = cmin ^ cmax;
  int sh = diff ? 64 - __clzll((long long)diff) : 0;  // composites differ only below bit sh
  if (sh == 0) {
    *cut = cmax;
    return true;
  }
  uint64_t prefix = sh >= 64 ? 0ull : cmax >> sh;
  uint32_t* const h32 = (uint32_t*)sm.hist;  // 2048 bins
  uint64_t* const lst = sm.hist;             // the gathered list (bins are dead by then)
  uint64_t n_under = (uint64_t)cnt;          // kept elements under the prefix
  constexpr int NB = 2048;
  const int per = NB / (int)blockDim.x;      // bins per thread, descending from top
  const int top = NB - 1 - tid * per;
  while (sh > 0 && n_under > 64) {
    const int d = sh < 11 ? sh : 11;
    sh -= d;
    for (int i = tid; i < NB; i += blockDim.x) h32[i] = 0u;
    __syncthreads();
    src.each([&](int i, float l) {
      if (!pr.keep(i, l)) return;
      const uint64_t c = composite<ORD>(l, i);
      if ((sh + d >= 64 ? 0ull : c >> (sh + d)) != prefix) return;
      atomicAdd(&h32[(int)((c >> sh) & (uint64_t)((1 << d) - 1))], 1u);
    });
    __syncthreads();
    uint64_t ls = 0;
    for (int q = 0; q < per; ++q) ls += h32[top - q];
    uint64_t tot;
    uint64_t c = block_exclusive_scan_u64(ls, sm.scratch64, &tot);
    if (c < k && c + ls >= k) {
      for (int q = 0; q < per; ++q) {
        const uint64_t hv = h32[top - q];
        if (c < k && c + hv >= k) {
          sm.bcast64[0] = (uint64_t)(top - q);
          sm.bcast64[1] = c;
          sm.bcast64[2] = hv;
        }
        c += hv;
      }
    }
    __syncthreads();
    prefix = (prefix << d) | sm.bcast64[0];
    k -= sm.bcast64[1];
    n_under = sm.bcast64[2];
    __syncthreads();
  }
  if (sh == 0) {  // one composite is left: the prefix itself
    *cut = prefix;
    return true;
  }
  // at most 64 kept elements under the prefix: list them, then one wave ranks
  if (tid == 0) sm.bcasti[0] = 0;
  __syncthreads();
  src.each([&](int i, float l) {
    if (!pr.keep(i, l)) return;
    const uint64_t c = composite<ORD>(l, i);
    if ((c >> sh) == prefix) lst[atomicAdd(&sm.bcasti[0], 1)] = c;
  });
  __syncthreads();
  if (tid < 64) {
    const int n = sm.bcasti[0];
    const uint64_t mine = tid < n ? lst[tid] : 0ull;
    uint64_t above = 0;
    for (int j = 0; j < n; ++j) above += lst[j] > mine ? 1ull : 0ull;
    if (tid < n && above == k - 1) sm.bcast64[3] = mine;
  }
  __syncthreads();
  *cut = sm.bcast64[3];
  return true;
}

// The categorical draw over the kept elements in vocabulary order, with the
// normaliser and the kept count: returns the first id whose inclusive weight
// sum exceeds draw_target(u, ZV) (0 when ZV = 0 or want_tok is false), where
// ZV = the kept weights' sum.  One pass adds every kept weight into 1024
// bins of 256 ids; the scan's total is ZV, and the bin holding the target
// has at most 256 kept elements.  Those are listed in LDS, and each thread
// holding one sums the listed weights at or below its id: the answer is the
// element whose inclusive sum passes the remainder while its exclusive sum
// does not.  Ids must lie below 2^18.
template <typename Src, typename WF>
__device__ int block_draw_id(const Src& src, const Pred& pr, WF vw, float u, bool want_tok, ExactSmem& sm,
                             uint64_t* ZV_out, int* nk_out) {
  const int tid = threadIdx.x;
  constexpr int NB = 1024;
  const int per = NB / (int)blockDim.x;  // bins per thread, ascending from b0
  const int b0 = tid * per;
  for (int i = tid; i < NB; i += blockDim.x) sm.hist[i] = 0;
  __syncthreads();
  int nk = 0;
  src.each([&](int i, float l) {
    if (!pr.keep(i, l)) return;
    ++nk;
    const uint64_t w = vw(i, l);
    if (w) atomicAdd((unsigned long long*)&sm.hist[i >> 8], (unsigned long long)w);
  });
  __syncthreads();
  uint64_t ls = 0;
  for (int q = 0; q < per; ++q) ls += sm.hist[b0 + q];
  uint64_t ZV;
  uint64_t c = block_exclusive_scan_u64(ls, sm.scratch64, &ZV);
  *ZV_out = ZV;
  *nk_out = block_reduce(nk, sm.scratchi, OpSumI(), 0);
  if (!want_tok || ZV == 0) return 0;
  const uint64_t tgt = draw_target(u, ZV);  // < ZV
  if (c <= tgt && tgt < c + ls) {
    for (int q = 0; q < per; ++q) {
      const uint64_t hv = sm.hist[b0 + q];
      if (c <= tgt && tgt < c + hv) {
        sm.bcast64[0] = (uint64_t)(b0 + q);
        sm.bcast64[1] = c;
      }
      c += hv;
    }
  }
  __syncthreads();
  const int bin = (int)sm.bcast64[0];
  const uint64_t rem = tgt - sm.bcast64[1];  // inside the bin's weight
  if (tid == 0) sm.bcasti[0] = 0;
  __syncthreads();
  // the bin's kept elements (at most 256) as (weight, id) in the dead bins
  uint64_t* const lw = sm.hist;
  int* const lid = (int*)(sm.hist + 256);
  src.each([&](int i, float l) {
    if (!pr.keep(i, l) || (i >> 8) != bin) return;
    const int at = atomicAdd(&sm.bcasti[0], 1);
    lw[at] = vw(i, l);
    lid[at] = i;
  });
  __syncthreads();
  const int n = sm.bcasti[0];
  for (int t = tid; t < n; t += blockDim.x) {
    const int me = lid[t];
    uint64_t incl = 0;
    for (int j = 0; j < n; ++j) incl += lid[j] <= me ? lw[j] : 0ull;
    if (incl > rem && incl - lw[t] <= rem) sm.bcasti[1] = me;
  }
  __syncthreads();
  return sm.bcasti[1];
}

__device__ __forceinline__ float chain_scale(int chain, float d, float invT, double rTc) {
  return chain == WH_CHAIN_MLX ? d * invT : div_by_recip(d, rTc);
}

// The whole exact algorithm for row b by one workgroup (64..1024 threads, a
// power of two).  Inlined where it is the kernel's main path, so that its LDS
// pointers stay LDS pointers; exact_row below is the out-of-line copy for
// the kernels that reach it only as a fallback (there its LDS accesses are
// flat accesses through generic pointers).
__device__ __forceinline__ void exact_row_impl(const SampleKArgs& a, int b, char* dyn_smem, ExactSmem& sm) {
  const int tid = threadIdx.x, nt = blockDim.x;
  const int V = a.V;
  RowCtx rc;
  rc.V = V;
  rc.xf = a.dtype == WH_DTYPE_F32 ? (const float*)a.logits + b * a.row_stride : nullptr;
  rc.xb = a.dtype == WH_DTYPE_BF16 ? (const uint16_t*)a.logits + b * a.row_stride : nullptr;
  rc.hmask = -1;
  if (a.hcap > 0) build_penalties(a, b, rc, dyn_smem, 0, V);

  // the caller's doubles; the float32 constants below are derived from them
  // as MLX derives them from Python floats
  const double T = a.T_rows ? a.T_rows[b] : a.T;
  const double top_p = a.top_p_rows ? a.top_p_rows[b] : a.top_p;
  const double min_p = a.min_p_rows ? a.min_p_rows[b] : a.min_p;
  const int top_k = a.top_k_rows ? a.top_k_rows[b] : a.top_k;
  float* out = a.out_rows ? a.out_rows + (long long)b * V : nullptr;

  if (!(T > 0.0)) {
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
  const bool use_p = top_p > 0.0 && top_p < 1.0;
  const bool use_m = min_p != 0.0;
  const float theta = (float)(1.0 - top_p);
  Pred pr = {0, 0, 0, 0, 0, 0, 0.0f, -INFINITY};
  auto mass = [m](int, float l) { return exp_fix44(l - m); };
  auto one = [](int, float) { return (uint64_t)1; };

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
    uint64_t cp = radix_select<ORD_P>(RowSource{&rc}, pr, mass, S - F, sm);
    pr.use_p = 1;
    pr.cp = cp;
  };
  auto apply_m = [&]() {
    const float c = a.min_p_rows ? (float)log(min_p) : a.min_p_log;
    pr.use_m = 1;
    pr.thr = m + c;
  };

  if (a.chain == WH_CHAIN_MLX) {
    if (use_k) {
      uint64_t ck = radix_select<ORD_A>(RowSource{&rc}, pr, one, (uint64_t)top_k, sm);
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
        uint64_t ck = radix_select<ORD_A>(RowSource{&rc}, pr, one, (uint64_t)top_k, sm);
        pr.use_k = 1;
        pr.ck = ck;
      }
    }
  }

  // Draw: per-thread contiguous segments, integer inverse CDF in vocab order.
  const float invT = (float)(1.0 / T);
  const double rTc = 1.0 / (double)(float)fmax(T, 1e-5);
  const int seg = (V + nt - 1) / nt;
  const int lo = min(V, tid * seg), hi = min(V, lo + seg);
  uint64_t s = 0;
  int cnt = 0;
  for (int i = lo; i < hi; ++i) {
    float l = rc.val(i);
    if (!pr.keep(i, l)) continue;
    ++cnt;
    s += exp_fix44(chain_scale(a.chain, l - m, invT, rTc));
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
        c += exp_fix44(chain_scale(a.chain, l - m, invT, rTc));
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
      out[i] = pr.keep(i, l) ? (float)((double)chain_scale(a.chain, l - m, invT, rTc) - lz) : -INFINITY;
    }
  }
}

// A float sum of exp(l - m) over row b's penalised values with the hardware
// exponential, for normaliser bounds when the candidates' own bounds cannot
// settle a top-p cut.  Each thread sums fewer than 2^10 terms in float32 and
// the threads' sums are added in double, so the relative error stays far
// below the 2e-4 the bounds allow, for every term exp_fix44 does not flush
// to 0 (the same argument as the slice sums).  The row is read as 16-byte
// groups (the fast engine's rows are aligned and V a multiple of the group);
// the penalty table goes to dyn.  Every thread of the workgroup calls it.
template <int DT>
__device__ __forceinline__ double row_zsum_t(const SampleKArgs& a, int b, float m, char* dyn, ExactSmem& sm) {
  const int tid = threadIdx.x, nt = blockDim.x, V = a.V;
  constexpr int EPT = DT ? 8 : 4;
  RowCtx rc;
  rc.V = V;
  rc.xf = DT ? nullptr : (const float*)a.logits + b * a.row_stride;
  rc.xb = DT ? (const uint16_t*)a.logits + b * a.row_stride : nullptr;
  rc.hmask = -1;
  if (a.hcap > 0) build_penalties(a, b, rc, dyn, 0, V);
  const uint4* row = DT ? (const uint4*)rc.xb : (const uint4*)rc.xf;
  float z = 0.0f;
  if (m != -INFINITY) {
    for (int g = tid; g < V / EPT; g += nt) {
      const uint4 q = row[g];
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const uint32_t w = e / (EPT / 4) == 0 ? q.x : e / (EPT / 4) == 1 ? q.y : e / (EPT / 4) == 2 ? q.z : q.w;
        const float r = DT ? __uint_as_float((e & 1) ? (w & 0xFFFF0000u) : (w << 16)) : __uint_as_float(w);
        z += __expf(rc.val_from(g * EPT + e, r) - m);
      }
    }
  }
  return block_reduce((double)z, (double*)sm.scratch64, OpSumF64(), 0.0);
}

__device__ __noinline__ void exact_row(const SampleKArgs& a, int b, char* dyn_smem, ExactSmem& sm) {
  exact_row_impl(a, b, dyn_smem, sm);
}

}  // namespace wh
