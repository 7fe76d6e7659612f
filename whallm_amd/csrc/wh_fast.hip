// wh_fast.hip -- the sliced single-read sampler engine for gfx950.
//
// Two kernels per call.
//
// slice_kernel: a row of V logits is cut into G slices; each slice is owned
// by one 1024-thread workgroup that reads it from HBM exactly once (16-byte
// loads, all issued up front, held in VGPRs) and reduces it to a summary:
//   * the penalties for the slice's history tokens (LDS hash, values taken
//     from the registers that hold the logits -- no second read),
//   * the slice max m_s (and, for greedy rows, the lowest index attaining it),
//   * the candidates: every slice element at or above a threshold tau_s that
//     is provably below the row's kept set --
//       rule M (min-p active):   tau_s = fl(m_s + ln min_p)  <= the row's cut
//       rule K (top-k bounds the kept set): tau_s = the slice's k-th largest
//       rule P (top-p only):     tau_s = the slice's cap/2-th largest,
//   * bounds on the normaliser Z = sum_i exp_fix44(l_i - m): the exact
//     fixed-point mass of the elements within 8 nats of m_s (a lower bound,
//     with the count of the rest for an upper bound), plus a hardware-exp
//     float estimate when top-p may cut without min-p behind it.
// Workgroups never wait for each other: no fences, no atomics across them.
//
// merge_kernel: one workgroup per row.  Wave 0 merges the G summaries with
// wave-level primitives (no block barriers): global max, exact fixed-point
// masses of the candidates, top-k / top-p / min-p in the chain's order, and
// the inverse-CDF draw over integer weights in vocabulary order -- the same
// integer contract as the exact engine.  A top-p cut is taken only when it is
// the same at both ends of the proven [Zlo, Zhi] interval.  A row the
// candidates cannot settle (capacity overflow, an ambiguous cut, no filter at
// all) is finished by the whole workgroup with the exact engine.
#include "wh_rowops.h"

namespace wh {

constexpr int FT = 1024;          // slice-kernel threads per workgroup
constexpr int FAST_RMAX = 16;     // max 16-byte loads per thread per slice
constexpr float ZBAND = 8.0f;     // exact-mass band below the slice max, nats

enum { RULE_GREEDY = 0, RULE_M = 1, RULE_K = 2, RULE_P = 3, RULE_ALL = 4 };

struct SliceHdr {
  float m;       // slice max (penalised)
  float tau;     // every slice element >= tau is a candidate
  int n;         // candidates written (= elements >= tau unless flags)
  int flags;     // 1: overflow / rule ALL -- the row needs the exact engine
  float t[3];    // band floors t1 >= t2 >= t3, all <= tau
  int c[3];      // elements >= t1, >= t2, >= t3 (cumulative, include candidates)
  int nall;      // elements in the slice
  int best_i;    // greedy: lowest index attaining the max
  double zf;     // sum of exp(l - m) over the slice (hardware exp), < 0 if not computed
  int pad[2];
};
static_assert(sizeof(SliceHdr) == 64, "SliceHdr layout");

struct FastPlan {
  int G;          // slices per row
  int SL;         // slice length (multiple of the elements per 16-byte load)
  int cap;        // candidate capacity per slice
  int rule_cap;   // largest k (or top-p window) a slice may bound
  int* path;      // [B] 0: merged from candidates, 1: exact engine (overflow / no filter),
                  //     2: greedy, 3: exact engine (top-p cut not settled by the bounds)
  SliceHdr* hdr;  // [B * G]
  int2* cand;     // [B * G * cap] (value bits, id)
};

__device__ __forceinline__ int choose_rule(int chain, float T, bool use_k, bool use_p, bool use_m, int k, int rule_cap) {
  if (!(T > 0.0f)) return RULE_GREEDY;
  if (chain == WH_CHAIN_MLX && use_k && use_p) return k <= rule_cap ? RULE_K : RULE_ALL;
  if (use_m) return RULE_M;
  if (use_k) return k <= rule_cap ? RULE_K : RULE_ALL;
  if (use_p) return RULE_P;
  return RULE_ALL;
}

struct RowParams {
  float T, top_p, min_p;
  int top_k;
  bool use_k, use_p, use_m;
  int rule;
};

__device__ __forceinline__ RowParams row_params(const SampleKArgs& a, int b, int rule_cap) {
  RowParams r;
  r.T = a.T_rows ? a.T_rows[b] : a.T;
  r.top_p = a.top_p_rows ? a.top_p_rows[b] : a.top_p;
  r.min_p = a.min_p_rows ? a.min_p_rows[b] : a.min_p;
  r.top_k = a.top_k_rows ? a.top_k_rows[b] : a.top_k;
  r.use_k = r.top_k > 0 && r.top_k < a.V;
  r.use_p = r.top_p > 0.0f && r.top_p < 1.0f;
  r.use_m = r.min_p != 0.0f;
  r.rule = choose_rule(a.chain, r.T, r.use_k, r.use_p, r.use_m, r.top_k, rule_cap);
  return r;
}

__device__ __forceinline__ float min_p_log(const SampleKArgs& a, float min_p) {
  return a.min_p_rows ? (float)log((double)min_p) : a.min_p_log;
}

// Element e of a 16-byte group (DT 0: 4 x float32, DT 1: 8 x bfloat16), -0 -> +0.
__device__ __forceinline__ uint32_t comp(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}
__device__ __forceinline__ void set_comp(uint4& v, int i, uint32_t x) {
  if (i == 0) v.x = x; else if (i == 1) v.y = x; else if (i == 2) v.z = x; else v.w = x;
}
template <int DT>
__device__ __forceinline__ float grp_elem(const uint4& v, int e) {
  if (DT == 0) return __uint_as_float(comp(v, e)) + 0.0f;
  const uint32_t x = comp(v, e >> 1);
  return __uint_as_float((e & 1) ? (x & 0xFFFF0000u) : (x << 16)) + 0.0f;
}
// Write -inf into slot e of a 16-byte group.
template <int DT>
__device__ __forceinline__ void grp_kill(uint4& v, int e) {
  if (DT == 0) { set_comp(v, e, 0xFF800000u); return; }
  const uint32_t x = comp(v, e >> 1);
  set_comp(v, e >> 1, (e & 1) ? ((x & 0x0000FFFFu) | 0xFF800000u) : ((x & 0xFFFF0000u) | 0x0000FF80u));
}

// Dynamic LDS layout of the slice kernel:
//   [hkeys hcap][hpos/hval hcap][hcnt hcap][bitmap (SL+31)/32] | candidate buffer (cap int2)
__host__ __device__ __forceinline__ size_t cand_buf_offset(int hcap, int SL) {
  const size_t o = hcap > 0 ? (size_t)hcap * 12 + (size_t)((SL + 31) / 32) * 4 : 0;
  return (o + 15) / 16 * 16;
}

struct SliceSmem {
  uint64_t hist64[1024];   // slice_kth counters (as 2048 x u32)
  uint64_t s64[16];
  double sd[16];
  float sf[16];
  int si[16];
  uint64_t bc64[2];
  int cnt;
};

// The slice's k-th largest value (k >= 1) over register elements and the
// penalised hash entries; -inf when the slice holds fewer than k elements.
// 32-bit keys in three digit passes (11, 11, 10 bits), counts in LDS.
template <int DT, int R>
__device__ float slice_kth(const uint4 (&d)[R], int v0, int v1, const int* hk, const float* hv, int hcap,
                           int k, SliceSmem& sm) {
  const int tid = threadIdx.x;
  constexpr int EPT = DT ? 8 : 4;
  uint32_t* hist = (uint32_t*)sm.hist64;
  int cnt = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) cnt += (v0 + (r * FT + tid) * EPT < v1) ? EPT : 0;
  for (int j = tid; j < hcap; j += FT) cnt += hk[j] >= 0 ? 1 : 0;
  const int total = block_reduce(cnt, sm.si, OpSumI(), 0);
  if (total < k) return -INFINITY;
  uint32_t prefix = 0;
  uint32_t target = (uint32_t)k;
#pragma unroll
  for (int pass = 0; pass < 3; ++pass) {
    const int sh = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
    const int nb = pass == 2 ? 10 : 11;
    const uint32_t mask = (1u << nb) - 1u;
    for (int i = tid; i < 2048; i += FT) hist[i] = 0;
    __syncthreads();
    auto add = [&](float l) {
      const uint32_t key = fkey(l);
      if (pass > 0 && (key >> (sh + nb)) != prefix) return;
      atomicAdd(&hist[(key >> sh) & mask], 1u);
    };
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int g = v0 + (r * FT + tid) * EPT;
      if (g < v1) {
#pragma unroll
        for (int e = 0; e < EPT; ++e) add(grp_elem<DT>(d[r], e));
      }
    }
    for (int j = tid; j < hcap; j += FT)
      if (hk[j] >= 0) add(hv[j]);
    __syncthreads();
    const int nbins = 1 << nb;
    const int hi = nbins - 1 - 2 * tid, lo = hi - 1;
    const uint64_t h_hi = hi >= 0 ? hist[hi] : 0, h_lo = lo >= 0 ? hist[lo] : 0;
    uint64_t tot;
    const uint64_t excl = block_exclusive_scan_u64(h_hi + h_lo, sm.s64, &tot);
    if (hi >= 0 && excl < target && excl + h_hi >= target) {
      sm.bc64[0] = (uint64_t)hi;
      sm.bc64[1] = excl;
    } else if (lo >= 0 && excl + h_hi < target && excl + h_hi + h_lo >= target) {
      sm.bc64[0] = (uint64_t)lo;
      sm.bc64[1] = excl + h_hi;
    }
    __syncthreads();
    prefix = (prefix << nb) | (uint32_t)sm.bc64[0];
    target -= (uint32_t)sm.bc64[1];
    __syncthreads();
  }
  return key_to_float(prefix);
}

template <int DT, int R>
__global__ void __launch_bounds__(FT) slice_kernel(SampleKArgs a, FastPlan P) {
  extern __shared__ __align__(16) char dyn[];
  __shared__ SliceSmem sm;
  constexpr int EPT = DT ? 8 : 4;
  constexpr int ESZ = DT ? 2 : 4;
  const int tid = threadIdx.x;
  const int b = blockIdx.x / P.G, s = blockIdx.x % P.G;
  const int V = a.V;
  const int v0 = s * P.SL, v1 = min(V, v0 + P.SL);
  const RowParams rp = row_params(a, b, P.rule_cap);
  SliceHdr* hdr = P.hdr + (long long)b * P.G + s;
  if (rp.rule == RULE_ALL) {
    if (tid == 0) hdr->flags = 1;
    return;
  }
  float* out = a.out_rows ? a.out_rows + (long long)b * V : nullptr;

  // 1. the slice, straight into registers
  const char* rowp = (const char*)a.logits + (size_t)b * a.row_stride * ESZ;
  uint4 d[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int g = v0 + (r * FT + tid) * EPT;
    d[r] = make_uint4(0u, 0u, 0u, 0u);
    if (g < v1) d[r] = *(const uint4*)(rowp + (size_t)g * ESZ);
  }

  // 2. penalties: history window -> LDS hash of the slice's tokens; the owner
  //    of each penalised element computes its value from the register copy,
  //    stores it in the hash and writes -inf into the register slot.  The
  //    history row (up to 4 ids per thread) and its length are fetched with
  //    the logits, so their latency overlaps.
  const int hcap = a.hcap;
  int32_t* hkeys = (int32_t*)dyn;
  int32_t* hpos = hkeys + hcap;
  int32_t* hcnt = hpos + hcap;
  uint32_t* bm = (uint32_t*)(hcnt + hcap);
  float* hval = (float*)hpos;
  if (hcap > 0) {
    constexpr int HPF = 4;
    const int32_t* h = a.hist + (long long)b * a.hist_stride;
    const int hs = (int)a.hist_stride;
    const bool pf = hs <= HPF * FT;
    int hreg[HPF];
#pragma unroll
    for (int q = 0; q < HPF; ++q) {
      const int j = tid + q * FT;
      hreg[q] = (pf && j < hs) ? h[j] : -1;
    }
    int len = a.hist_len ? a.hist_len[b] : 0;
    const int words = (v1 - v0 + 31) >> 5;
    for (int t = tid; t < hcap; t += FT) { hkeys[t] = -1; hpos[t] = -1; hcnt[t] = 0; }
    for (int w = tid; w < words; w += FT) bm[w] = 0u;
    len = max(0, min(len, hs));
    const bool on_r = a.rep != 0.0f, on_p = a.pres != 0.0f, on_f = a.freq != 0.0f;
    auto window = [len](int ctx) { return (ctx <= 0 || ctx > len) ? len : ctx; };
    const int wr = on_r ? window(a.rep_ctx) : 0;
    const int wp = on_p ? window(a.pres_ctx) : 0;
    const int wf = on_f ? window(a.freq_ctx) : 0;
    const int W = max(wr, max(wp, wf));
    const int hshift = 32 - a.hlog2, hmask = hcap - 1;
    auto insert = [&](int j, int t) {
      if (t < v0 || t >= v1) return;
      uint32_t q = ((uint32_t)t * 2654435761u) >> hshift;
      while (true) {
        const int old = atomicCAS(&hkeys[q], -1, t);
        if (old == -1 || old == t) break;
        q = (q + 1) & hmask;
      }
      atomicMax(&hpos[q], j);
      if (j >= len - wf) atomicAdd(&hcnt[q], 1);
      atomicOr(&bm[(t - v0) >> 5], 1u << ((t - v0) & 31));
    };
    __syncthreads();
    if (pf) {
#pragma unroll
      for (int q = 0; q < HPF; ++q) {
        const int j = tid + q * FT;
        if (j >= len - W && j < len) insert(j, hreg[q]);
      }
    } else {
      for (int j = len - W + tid; j < len; j += FT) insert(j, h[j]);
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int g = v0 + (r * FT + tid) * EPT;
      if (g < v1) {
        const int o = g - v0;
        const uint32_t bits = (bm[o >> 5] >> (o & 31)) & ((1u << EPT) - 1u);
        if (bits) {
#pragma unroll
          for (int e = 0; e < EPT; ++e) {
            if (!((bits >> e) & 1u)) continue;
            const int t = g + e;
            uint32_t q = ((uint32_t)t * 2654435761u) >> hshift;
            while (hkeys[q] != t) q = (q + 1) & hmask;
            const int lp = hpos[q], c = hcnt[q];
            float v = grp_elem<DT>(d[r], e);
            if (on_r && lp >= len - wr) v = v < 0.0f ? v * a.rep : v / a.rep;
            if (on_p && lp >= len - wp) v = v - a.pres;
            if (on_f && c > 0) v = v - a.freq * (float)c;
            hval[q] = v + 0.0f;
            grp_kill<DT>(d[r], e);
          }
        }
      }
    }
    __syncthreads();
  }
  auto each_pen = [&](auto f) {
    for (int j = tid; j < hcap; j += FT) {
      const int i = hkeys[j];
      if (i >= 0) f(i, hval[j]);
    }
  };
  auto killed_bits = [&](int g) -> uint32_t {
    return hcap > 0 ? (bm[(g - v0) >> 5] >> ((g - v0) & 31)) & ((1u << EPT) - 1u) : 0u;
  };

  // 3. slice max and, for greedy rows, the lowest index attaining it
  const bool greedy = rp.rule == RULE_GREEDY;
  float mx = -INFINITY;
  int mi = 0x7FFFFFFF;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int g = v0 + (r * FT + tid) * EPT;
    if (g < v1) {
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const float l = grp_elem<DT>(d[r], e);
        if (greedy) {
          if (mi == 0x7FFFFFFF || l > mx) { mx = l; mi = g + e; }
        } else {
          mx = fmaxf(mx, l);
        }
      }
    }
  }
  each_pen([&](int i, float l) {
    if (greedy) {
      if (mi == 0x7FFFFFFF || l > mx || (l == mx && i < mi)) { mx = l; mi = i; }
    } else {
      mx = fmaxf(mx, l);
    }
  });
  const float ms = block_reduce(mx, sm.sf, OpMaxF(), -INFINITY);

  if (greedy) {
    const int cand = (mi != 0x7FFFFFFF && mx == ms) ? mi : 0x7FFFFFFF;
    const int bi = block_reduce(cand, sm.si, OpMinI(), 0x7FFFFFFF);
    if (out) {  // Whallm's sampling_logprobs returns the (penalised) logits at T == 0
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int g = v0 + (r * FT + tid) * EPT;
        if (g < v1) {
#pragma unroll
          for (int e = 0; e < EPT; ++e) out[g + e] = grp_elem<DT>(d[r], e);
        }
      }
      __syncthreads();
      each_pen([&](int i, float l) { out[i] = l; });
    }
    if (tid == 0) {
      hdr->m = ms;
      hdr->best_i = bi;
      hdr->flags = 0;
      hdr->n = 0;
    }
    return;
  }

  // 4. candidate threshold and the band thresholds below it
  float tau;
  if (rp.rule == RULE_M) tau = ms + min_p_log(a, rp.min_p);
  else tau = slice_kth<DT, R>(d, v0, v1, hkeys, hval, hcap, rp.rule == RULE_K ? rp.top_k : P.rule_cap, sm);
  const float t1 = fminf(tau, ms - 4.5f), t2 = fminf(t1, ms - 6.0f), t3 = fminf(t2, ms - 8.0f);
  const bool need_zf = rp.use_p && !rp.use_m;

  // 5. one pass: candidates (wave-aggregated appends to LDS), band counts
  //    (wave ballots), optional hardware-exp estimate of sum exp(l - ms)
  int2* buf = (int2*)(dyn + cand_buf_offset(hcap, P.SL));
  if (tid == 0) sm.cnt = 0;
  __syncthreads();
  const int lane = tid & 63;
  int c1 = 0, c2 = 0, c3 = 0, nall = 0;  // c*: wave-uniform ballot counts
  float zs = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int g = v0 + (r * FT + tid) * EPT;
    const bool in = g < v1;
    const uint32_t killed = in ? killed_bits(g) : 0xFFu;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const float l = grp_elem<DT>(d[r], e);
      const bool valid = in && !((killed >> e) & 1u);
      nall += valid ? 1 : 0;
      const uint64_t mk = __ballot(valid && l >= tau);
      if (mk) {
        int base = 0;
        if (lane == 0) base = atomicAdd(&sm.cnt, (int)__popcll(mk));
        base = __shfl(base, 0, 64);
        if (valid && l >= tau) {
          const int slot = base + (int)__popcll(mk & ((1ull << lane) - 1ull));
          if (slot < P.cap) buf[slot] = make_int2(__float_as_int(l), g + e);
        }
      }
      c1 += (int)__popcll(__ballot(valid && l >= t1));
      c2 += (int)__popcll(__ballot(valid && l >= t2));
      c3 += (int)__popcll(__ballot(valid && l >= t3));
      if (need_zf && valid) zs += __expf(l - ms);
    }
  }
  int p1 = 0, p2 = 0, p3 = 0;
  each_pen([&](int i, float l) {
    ++nall;
    if (l >= tau) {
      const int slot = atomicAdd(&sm.cnt, 1);
      if (slot < P.cap) buf[slot] = make_int2(__float_as_int(l), i);
    }
    p1 += l >= t1;
    p2 += l >= t2;
    p3 += l >= t3;
    if (need_zf) zs += __expf(l - ms);
  });
  // one combined block reduction
  const int wv = tid >> 6;
  int q1 = wave_sum_i(p1) + c1, q2 = wave_sum_i(p2) + c2, q3 = wave_sum_i(p3) + c3, qa = wave_sum_i(nall);
  const double qz = need_zf ? wave_sum_f64((double)zs) : 0.0;
  if (lane == 0) {
    sm.si[wv] = q1;
    ((int*)sm.s64)[wv] = q2;
    ((int*)sm.s64)[16 + wv] = q3;
    sm.sf[wv] = __int_as_float(qa);
    sm.sd[wv] = qz;
  }
  __syncthreads();
  const int n = sm.cnt;
  const int nw = min(n, P.cap);
  int2* gc = P.cand + ((long long)b * P.G + s) * P.cap;
  for (int j = tid; j < nw; j += FT) gc[j] = buf[j];
  if (out) {
    // non-candidates are never kept; the merge overwrites the kept ones
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int g = v0 + (r * FT + tid) * EPT;
      if (g < v1) {
#pragma unroll
        for (int e = 0; e < EPT; ++e) out[g + e] = -INFINITY;
      }
    }
  }
  if (tid == 0) {
    int s1 = 0, s2 = 0, s3 = 0, sa = 0;
    double sz = 0.0;
    const int nwv = FT / 64;
    for (int w = 0; w < nwv; ++w) {
      s1 += sm.si[w];
      s2 += ((int*)sm.s64)[w];
      s3 += ((int*)sm.s64)[16 + w];
      sa += __float_as_int(sm.sf[w]);
      sz += sm.sd[w];
    }
    hdr->m = ms;
    hdr->tau = tau;
    hdr->n = nw;
    hdr->flags = n > P.cap ? 1 : 0;
    hdr->t[0] = t1;
    hdr->t[1] = t2;
    hdr->t[2] = t3;
    hdr->c[0] = s1;
    hdr->c[1] = s2;
    hdr->c[2] = s3;
    hdr->nall = sa;
    hdr->zf = need_zf ? sz : -1.0;
  }
}

// ---------------------------------------------------------------------------
// Wave-level merge.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

struct MergeSmem {
  uint64_t hist[1024];
  uint64_t bc64[2];
};

struct WaveCands {
  const float* v;
  const int* id;
  int n;
  template <typename F>
  __device__ __forceinline__ void each(F f) const {
    for (int j = (int)(threadIdx.x & 63); j < n; j += 64) f(id[j], v[j]);
  }
};

// Wave-level radix select (same contract as radix_select): the composite of
// the element at which the cumulative measure over kept candidates first
// reaches target (0 < target <= total).
template <int ORD, typename Meas>
__device__ uint64_t wave_radix_select(const WaveCands& src, const Pred& pr, Meas meas, uint64_t target, MergeSmem& sm) {
  const int lane = threadIdx.x & 63;
  // Bits above the highest bit in which two kept composites differ are
  // common to all of them: start the 10-bit digits below it, so the first
  // pass spreads the candidates over the bins instead of piling them into
  // one (LDS atomics on one address serialise).
  uint64_t cmin = ~0ull, cmax = 0;
  src.each([&](int i, float l) {
    if (!pr.keep(i, l)) return;
    const uint64_t c = composite<ORD>(l, i);
    cmin = c < cmin ? c : cmin;
    cmax = c > cmax ? c : cmax;
  });
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t a = __shfl_xor(cmin, o, 64), b = __shfl_xor(cmax, o, 64);
    cmin = a < cmin ? a : cmin;
    cmax = b > cmax ? b : cmax;
  }
  if (cmax < cmin) return 0;  // nothing kept (callers never ask)
  const uint64_t diff = cmin ^ cmax;
  const int top = diff ? 64 - __clzll((long long)diff) : 1;  // bits that vary
  const int PASSES = (top + 9) / 10;
  uint64_t prefix = cmax >> (10 * PASSES);
  for (int pass = 0; pass < PASSES; ++pass) {
    const int shift = 10 * (PASSES - 1 - pass);
    for (int i = lane; i < 1024; i += 64) sm.hist[i] = 0;
    wave_sync();
    src.each([&](int i, float l) {
      if (!pr.keep(i, l)) return;
      const uint64_t c = composite<ORD>(l, i);
      if ((c >> (shift + 10)) != prefix) return;
      const uint64_t w = meas(i, l);
      if (w) atomicAdd((unsigned long long*)&sm.hist[(c >> shift) & 1023], (unsigned long long)w);
    });
    wave_sync();
    // lane owns bins 1023-16*lane .. 1008-16*lane (descending)
    uint64_t ls = 0;
#pragma unroll
    for (int q = 0; q < 16; ++q) ls += sm.hist[1023 - 16 * lane - q];
    uint64_t incl = ls;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t y = __shfl_up(incl, o, 64);
      if (lane >= o) incl += y;
    }
    uint64_t c = incl - ls;
    if (c < target && incl >= target) {
      for (int q = 0; q < 16; ++q) {
        const uint64_t hv = sm.hist[1023 - 16 * lane - q];
        if (c < target && c + hv >= target) {
          sm.bc64[0] = (uint64_t)(1023 - 16 * lane - q);
          sm.bc64[1] = c;
        }
        c += hv;
      }
    }
    wave_sync();
    prefix = (prefix << 10) | sm.bc64[0];
    target -= sm.bc64[1];
    wave_sync();
  }
  return prefix;
}

__global__ void __launch_bounds__(1024) merge_kernel(SampleKArgs a, FastPlan P) {
  extern __shared__ __align__(16) char dyn[];
  __shared__ ExactSmem esm;
  __shared__ MergeSmem sm;
  __shared__ int s_fallback;
  constexpr int SPEC = 64;  // candidates per slice fetched together with the headers
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int G = P.G;
  const RowParams rp = row_params(a, b, P.rule_cap);
  if (tid < 64) {
    const int lane = tid;
    const SliceHdr* H = P.hdr + (long long)b * G;
    // one round trip: headers (lane s < G), the row's uniform, and the first
    // SPEC candidates of every slice
    SliceHdr hd;
    if (lane < G) hd = H[lane];
    const float ub = (a.tokens && rp.rule != RULE_GREEDY) ? a.u[b] : 0.0f;
    float* cv = (float*)dyn;
    int* ci = (int*)(dyn + (size_t)G * P.cap * sizeof(float));
    int2 spec[4];
    const bool spec_ok = G <= 4 && rp.rule != RULE_GREEDY && rp.rule != RULE_ALL;
    if (spec_ok) {
#pragma unroll
      for (int s = 0; s < 4; ++s)
        if (s < G) spec[s] = P.cand[((long long)b * G + s) * P.cap + lane];
    }
    const float hm = lane < G ? hd.m : -INFINITY;
    const int hflag = lane < G ? hd.flags : 0;
    const float m = wave_max(hm);
    int fallback = (wave_sum_i(hflag) != 0 || rp.rule == RULE_ALL) ? 1 : 0;
    if (rp.rule == RULE_GREEDY) {
      const int cand = (lane < G && hm == m) ? hd.best_i : 0x7FFFFFFF;
      const int bi = wave_min_i(cand);
      if (lane == 0) {
        if (a.tokens) a.tokens[b] = bi;
        if (a.kept) a.kept[b] = 1;
        P.path[b] = 2;
      }
      fallback = 0;
    } else if (!fallback) {
      const int hn = lane < G ? hd.n : 0;
      float tcov = lane < G ? hd.tau : -INFINITY;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) tcov = fmaxf(tcov, __shfl_xor(tcov, o, 64));
      // candidate offsets (prefix over the first G lanes)
      int off = hn;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(off, o, 64);
        if (lane >= o) off += y;
      }
      const int N = __shfl(off, 63, 64);
      off -= hn;
      for (int s = 0; s < G; ++s) {
        const int ns = __shfl(hn, s, 64), os = __shfl(off, s, 64);
        const int2* src = P.cand + ((long long)b * G + s) * P.cap;
        int j0 = 0;
        if (spec_ok) {
          int2 c = spec[0];
          if (s == 1) c = spec[1];
          if (s == 2) c = spec[2];
          if (s == 3) c = spec[3];
          if (lane < ns) { cv[os + lane] = __int_as_float(c.x); ci[os + lane] = c.y; }
          j0 = SPEC;
        }
        for (int j = j0 + lane; j < ns; j += 64) {
          const int2 c = src[j];
          cv[os + j] = __int_as_float(c.x);
          ci[os + j] = c.y;
        }
      }
      wave_sync();
      const WaveCands src{cv, ci, N};
      Pred pr = {0, 0, 0, 0, 0, 0, 0.0f, -INFINITY};
      auto mass = [m](int, float l) { return exp_fix44(l - m); };
      auto one = [](int, float) { return (uint64_t)1; };
      auto count = [&](const Pred& p) {
        int c = 0;
        src.each([&](int i, float l) { c += p.keep(i, l) ? 1 : 0; });
        return wave_sum_i(c);
      };
      auto msum = [&](const Pred& p) {
        uint64_t z = 0;
        src.each([&](int i, float l) { if (p.keep(i, l)) z += exp_fix44(l - m); });
        return wave_sum_u64(z);
      };
      const float theta = (float)(1.0 - (double)rp.top_p);
      bool ambiguous = false;

      // Top-p with the normaliser Z = sum_i exp_fix44(l_i - m) known to lie in
      // [Zlo, Zhi].  S is the alive mass: exact when s_exact, else Z itself.
      auto apply_p = [&](bool s_exact) {
        // The candidates contribute their exact masses.  An element below the
        // candidate cut but at or above band floor t_j (counted by the slice)
        // has exp_fix44(l - m) >= floor(2^44 e^(t_j - m) (1 - eps)) - 1 and
        // <= 2^44 e^(t_(j-1) - m) (1 + eps) + 1 (t_0 = tau), with eps = 1e-4
        // well above exp_fix44's relative error (|t| + 2) 2^-23 for the
        // arguments that matter; below t3 only the upper bound counts.  With
        // a float estimate zf (hardware exp, error < 1e-5 including float
        // sums of < 2^7 terms) the upper bound is zf-based instead.
        const double SC = 17592186044416.0;
        const uint64_t Scand = msum(Pred{0, 0, 0, 0, 0, 0, 0.0f, -INFINITY});
        double lo = 0.0, hi = 0.0;
        if (lane < G && hd.m != -INFINITY) {
          const double fl[4] = {(double)hd.tau, (double)hd.t[0], (double)hd.t[1], (double)hd.t[2]};
          const int cum[4] = {hd.n, hd.c[0], hd.c[1], hd.c[2]};
          for (int j = 1; j < 4; ++j) {
            const double cnt = (double)(cum[j] - cum[j - 1]);
            if (cnt <= 0.0) continue;
            const double wl = floor(exp(fl[j] - (double)m) * SC * (1.0 - 1e-4)) - 1.0;
            lo += cnt * fmax(wl, 0.0);
            hi += cnt * (exp(fl[j - 1] - (double)m) * SC * (1.0 + 1e-4) + 1.0);
          }
          hi += (double)(hd.nall - hd.c[2]) * (exp(fl[3] - (double)m) * SC * (1.0 + 1e-4) + 1.0);
          if (hd.zf >= 0.0) hi = -1.0;  // replaced below
        }
        lo = wave_sum_f64(lo) + (double)Scand;
        bool use_zf = wave_sum_i(lane < G && hd.m != -INFINITY && hd.zf >= 0.0 ? 1 : 0) > 0;
        double zfh = 0.0;
        if (lane < G && hd.m != -INFINITY && hd.zf >= 0.0)
          zfh = hd.zf * exp((double)hd.m - (double)m) * (1.0 + 1e-4) * SC + (double)hd.nall + 1e-6 * SC;
        if (use_zf) hi = wave_sum_f64(zfh);
        else hi = wave_sum_f64(hi) + (double)Scand;
        const uint64_t Zlo = (uint64_t)lo;
        const uint64_t Zhi = hi >= 4.0e18 ? (1ull << 62) : (uint64_t)ceil(hi);
        long long Rlo, Rhi;
        if (s_exact) {
          const long long S = (long long)msum(pr);
          Rlo = S - (long long)floor_theta_z(theta, Zhi);
          Rhi = S - (long long)floor_theta_z(theta, Zlo);
        } else {
          Rlo = (long long)(Zlo - floor_theta_z(theta, Zlo));
          Rhi = (long long)(Zhi - floor_theta_z(theta, Zhi));
        }
        if (Rhi <= 0) { pr.none = 1; return; }
        if (Rlo <= 0) { ambiguous = true; return; }
        Pred pc = pr;
        pc.cov = tcov;
        const long long Scov = (long long)msum(pc);
        if (Rlo > Scov) {
          // every covered element survives; the kept set stays inside the
          // covered region only if a later filter confines it there (the
          // min-p cut is >= every slice threshold; the top-k set is covered)
          if (rp.rule == RULE_P) ambiguous = true;
          return;
        }
        if (Rhi > Scov) { ambiguous = true; return; }
        const uint64_t clo = wave_radix_select<ORD_P>(src, pc, mass, (uint64_t)Rlo, sm);
        const uint64_t chi = wave_radix_select<ORD_P>(src, pc, mass, (uint64_t)Rhi, sm);
        if (clo != chi) { ambiguous = true; return; }
        pr.use_p = 1;
        pr.cp = clo;
      };
      auto apply_m = [&]() {
        pr.use_m = 1;
        pr.thr = m + min_p_log(a, rp.min_p);
      };
      if (a.chain == WH_CHAIN_MLX && rp.rule == RULE_K) {
        // the candidates hold the whole top-k set (at least k of them)
        if (rp.use_k) {
          pr.ck = wave_radix_select<ORD_A>(src, pr, one, (uint64_t)rp.top_k, sm);
          pr.use_k = 1;
        }
        if (rp.use_p) apply_p(rp.use_k);
        if (!ambiguous && rp.use_m && !pr.none) apply_m();
      } else if (a.chain == WH_CHAIN_MLX) {
        // rule M or P: no top-p together with top-k here.  k -> min-p: the
        // min-p set is a value prefix held by the candidates; with more than k
        // members the row's first k (order A) are its first k, else top-k
        // keeps all of it.
        if (rp.use_p) apply_p(false);
        if (!ambiguous && rp.use_m && !pr.none) apply_m();
        if (!ambiguous && rp.use_k && !pr.none && count(pr) > rp.top_k) {
          pr.ck = wave_radix_select<ORD_A>(src, pr, one, (uint64_t)rp.top_k, sm);
          pr.use_k = 1;
        }
      } else {
        if (rp.use_p) apply_p(false);
        if (!ambiguous && rp.use_m && !pr.none) apply_m();
        if (!ambiguous && rp.use_k && !pr.none && count(pr) > rp.top_k) {
          pr.ck = wave_radix_select<ORD_A>(src, pr, one, (uint64_t)rp.top_k, sm);
          pr.use_k = 1;
        }
      }
      if (ambiguous) {
        fallback = 3;
      } else {
        // Draw: integer inverse CDF in vocabulary order over the kept candidates.
        const float invT = (float)(1.0 / (double)rp.T);
        const float Tc = (float)fmax((double)rp.T, 1e-5);
        auto vw = [&](int, float l) { return exp_fix44(chain_scale(a.chain, l - m, invT, Tc)); };
        uint64_t zv = 0;
        int nk = 0;
        src.each([&](int i, float l) {
          if (pr.keep(i, l)) { zv += vw(i, l); ++nk; }
        });
        const uint64_t ZV = wave_sum_u64(zv);
        const int nkept = wave_sum_i(nk);
        if (a.tokens) {
          int tok = 0;
          if (ZV) {
            const uint64_t tgt = draw_target(ub, ZV);
            tok = 0x3FFFF - (int)wave_radix_select<ORD_ID>(src, pr, vw, tgt + 1, sm);
          }
          if (lane == 0) a.tokens[b] = tok;
        }
        if (lane == 0) {
          if (a.kept) a.kept[b] = nkept;
          P.path[b] = 0;
        }
        float* out = a.out_rows ? a.out_rows + (long long)b * a.V : nullptr;
        if (out) {
          const double lz = log(ldexp((double)ZV, -44));
          src.each([&](int i, float l) {
            if (!pr.keep(i, l)) return;
            out[i] = a.out_mode == WH_OUT_MASKED ? l : (float)((double)chain_scale(a.chain, l - m, invT, Tc) - lz);
          });
        }
      }
    }
    if (lane == 0) s_fallback = fallback;
  }
  __syncthreads();
  if (s_fallback) {
    if (tid == 0) P.path[b] = s_fallback == 3 ? 3 : 1;
    exact_row(a, b, dyn, esm);
  }
}

// ---------------------------------------------------------------------------
// Host side: plan, workspace layout, dispatch.
// ---------------------------------------------------------------------------
struct HostPlan {
  int G, SL, R, cap, rule_cap, ept;
};

static HostPlan make_plan(int B, int V, int dtype) {
  HostPlan p;
  p.ept = dtype == WH_DTYPE_BF16 ? 8 : 4;
  const int slmax = FT * p.ept * FAST_RMAX;
  int g = std::max((256 + B - 1) / std::max(B, 1), (V + slmax - 1) / slmax);
  g = std::min(g, 32);
  p.G = g;
  int sl = (V + g - 1) / g;
  sl = (sl + p.ept - 1) / p.ept * p.ept;
  p.SL = sl;
  p.R = (sl + FT * p.ept - 1) / (FT * p.ept);
  p.cap = std::min(2048, 16384 / g);
  p.rule_cap = p.cap / 2;
  return p;
}

struct WsLayout {
  size_t path, hdr, cand, total;
};

// Workspace: [path B x int32][slice headers B*G][candidates B*G*cap]
static WsLayout ws_layout(int B, const HostPlan& p) {
  WsLayout w;
  w.path = 0;
  w.hdr = ((size_t)B * 4 + 255) / 256 * 256;
  w.cand = w.hdr + (size_t)B * p.G * sizeof(SliceHdr);
  w.total = w.cand + (size_t)B * p.G * p.cap * sizeof(int2);
  return w;
}

size_t sample_workspace_bytes(int B, int V) {
  if (B <= 0 || V <= 0) return 256;
  WsLayout a = ws_layout(B, make_plan(B, V, WH_DTYPE_F32));
  WsLayout b = ws_layout(B, make_plan(B, V, WH_DTYPE_BF16));
  return std::max(a.total, b.total);
}

static int set_lds(const void* fn, size_t lds) {
  if (lds <= 65536) return WH_OK;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return fail(WH_EHIP, "hipFuncSetAttribute(%zu bytes LDS) failed: %s", lds, hipGetErrorString(e));
  return WH_OK;
}

template <int DT, int R>
static int launch_slice_t(const SampleKArgs& k, const FastPlan& fp, size_t lds, hipStream_t st) {
  auto fn = slice_kernel<DT, R>;
  int rc = set_lds((const void*)fn, lds);
  if (rc) return rc;
  hipLaunchKernelGGL(fn, dim3(k.B * fp.G), dim3(FT), lds, st, k, fp);
  return WH_OK;
}

// R is rounded up to an instantiated register count.
template <int DT>
static int launch_slice_dt(int R, const SampleKArgs& k, const FastPlan& fp, size_t lds, hipStream_t st) {
  if (R <= 1) return launch_slice_t<DT, 1>(k, fp, lds, st);
  if (R <= 2) return launch_slice_t<DT, 2>(k, fp, lds, st);
  if (R <= 3) return launch_slice_t<DT, 3>(k, fp, lds, st);
  if (R <= 4) return launch_slice_t<DT, 4>(k, fp, lds, st);
  if (R <= 5) return launch_slice_t<DT, 5>(k, fp, lds, st);
  if (R <= 6) return launch_slice_t<DT, 6>(k, fp, lds, st);
  if (R <= 8) return launch_slice_t<DT, 8>(k, fp, lds, st);
  if (R <= 10) return launch_slice_t<DT, 10>(k, fp, lds, st);
  if (R <= 12) return launch_slice_t<DT, 12>(k, fp, lds, st);
  return launch_slice_t<DT, 16>(k, fp, lds, st);
}

int launch_sample(const SampleKArgs& k0, const wh_sample_args* p, hipStream_t st) {
  const int esz = k0.dtype == WH_DTYPE_BF16 ? 2 : 4;
  HostPlan hp = make_plan(k0.B, k0.V, k0.dtype);
  WsLayout wl = ws_layout(k0.B, hp);
  const bool aligned = ((uintptr_t)k0.logits % 16 == 0) && ((k0.row_stride * esz) % 16 == 0) && (k0.V % hp.ept == 0);
  if (!aligned || !p->workspace || p->workspace_bytes < wl.total) return launch_sample_exact(k0, st);
  SampleKArgs k = k0;
  FastPlan fp;
  fp.G = hp.G;
  fp.SL = hp.SL;
  fp.cap = hp.cap;
  fp.rule_cap = hp.rule_cap;
  char* ws = (char*)p->workspace;
  fp.path = (int*)(ws + wl.path);
  fp.hdr = (SliceHdr*)(ws + wl.hdr);
  fp.cand = (int2*)(ws + wl.cand);
  const size_t lds_slice = cand_buf_offset(k.hcap, hp.SL) + (size_t)hp.cap * sizeof(int2);
  const size_t lds_merge = std::max((size_t)hp.G * hp.cap * 8, penalty_lds_bytes(k));
  int rc = k.dtype == WH_DTYPE_BF16 ? launch_slice_dt<1>(hp.R, k, fp, lds_slice, st)
                                    : launch_slice_dt<0>(hp.R, k, fp, lds_slice, st);
  if (rc) return rc;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "slice_kernel launch failed: %s", hipGetErrorString(e));
  rc = set_lds((const void*)merge_kernel, lds_merge);
  if (rc) return rc;
  hipLaunchKernelGGL(merge_kernel, dim3(k.B), dim3(1024), lds_merge, st, k, fp);
  e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "merge_kernel launch failed: %s", hipGetErrorString(e));
  return WH_OK;
}

}  // namespace wh
