// wh_fast.hip -- the sliced single-read sampler engine for gfx950.
//
// A row of V logits is cut into G slices; each slice is owned by one
// 1024-thread workgroup that reads it from HBM exactly once (16-byte loads,
// all issued up front, held in VGPRs).  All G workgroups of a row are placed
// on the same XCD (workgroup ids are dealt to the 8 XCDs round robin), so the
// merge reads each other's results through one L2.
//
// Per slice: penalties for the slice's history tokens (LDS hash), the local
// max, a float estimate of sum exp(l - m_s) for top-p certification, and the
// candidates -- every slice element at or above a local threshold that is
// provably below the row's kept set:
//   rule M (min-p active):      tau_s = fl(m_s + ln min_p)  <= the row's min-p cut
//   rule K (top-k bounds the kept set): tau_s = the slice's k-th largest value
//   rule P (top-p only):        tau_s = the slice's (cap/2)-th largest value
// The last workgroup of the row to arrive merges the slices' candidates and
// decides with the exact integer contract (fixed-point masses exp_fix44);
// the normaliser Z, which needs every element, is known only to within a
// proven relative bound from the float estimates, so a top-p cut is taken
// only if it is the same at both ends of the bound.  Whenever the
// candidates cannot settle the row (capacity overflow, an ambiguous cut, no
// filter at all) the merging workgroup runs the exact engine on the row.
#include "wh_rowops.h"

namespace wh {

constexpr int FT = 1024;          // threads per workgroup
constexpr int FAST_RMAX = 8;      // max 16-byte loads per thread per slice

enum { RULE_GREEDY = 0, RULE_M = 1, RULE_K = 2, RULE_P = 3, RULE_ALL = 4 };

struct SliceHdr {
  float m;       // slice max (penalised)
  float tau;     // every slice element >= tau is a candidate
  int n;         // candidates written
  int flags;     // 1: overflow -- the slice could not bound the kept set
  double zf;     // sum over the slice of exp(l - m) (hardware exp)
  float best_v;  // greedy: slice maximum
  int best_i;    // greedy: lowest index attaining it
  int pad[8];
};
static_assert(sizeof(SliceHdr) == 64, "SliceHdr layout");

struct FastPlan {
  int G;          // slices per row
  int SL;         // slice length (multiple of the elements per 16-byte load)
  int cap;        // candidate capacity per slice
  int rule_cap;   // largest k (or top-p window) a slice may bound
  int* counters;  // [B] arrival counters (zero between calls)
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
template <int DT>
__device__ __forceinline__ void grp_kill(uint4& v, int e) {
  if (DT == 0) { set_comp(v, e, 0xFF800000u); return; }
  const uint32_t x = comp(v, e >> 1);
  set_comp(v, e >> 1, (e & 1) ? ((x & 0x0000FFFFu) | 0xFF800000u) : ((x & 0xFFFF0000u) | 0x0000FF80u));
}

// Byte offset of the slice-phase candidate buffer in dynamic LDS.
__host__ __device__ __forceinline__ size_t cand_buf_offset(int hcap, int SL) {
  const size_t o = hcap > 0 ? (size_t)hcap * 12 + (size_t)((SL + 31) / 32) * 4 : 0;
  return (o + 15) / 16 * 16;
}

// The slice's k-th largest value (k >= 1) over register elements and the
// penalised list; -inf when the slice holds fewer than k elements.
// 32-bit keys in three digit passes (11, 11, 10 bits), counts in LDS.
template <int DT, int R>
__device__ float slice_kth(const uint4 (&d)[R], int v0, int v1, const int* pl_id, const float* pl_v, int np,
                           int k, ExactSmem& sm) {
  const int tid = threadIdx.x;
  constexpr int EPT = DT ? 8 : 4;
  uint32_t* hist = (uint32_t*)sm.hist;  // 2048 counters
  int cnt = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) cnt += (v0 + (r * FT + tid) * EPT < v1) ? EPT : 0;
  for (int j = tid; j < np; j += FT) cnt++;
  const int total = block_reduce(cnt, sm.scratchi, OpSumI(), 0);
  if (total < k) return -INFINITY;
  uint32_t prefix = 0;
  uint32_t target = (uint32_t)k;
  const int shifts[3] = {21, 10, 0};
  const int bits[3] = {11, 11, 10};
  for (int pass = 0; pass < 3; ++pass) {
    const int sh = shifts[pass], nb = bits[pass];
    const uint32_t mask = (1u << nb) - 1u;
    for (int i = tid; i < 2048; i += FT) hist[i] = 0;
    __syncthreads();
    auto add = [&](float l) {
      uint32_t key = fkey(l);
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
    for (int j = tid; j < np; j += FT) add(pl_v[j]);
    __syncthreads();
    // descending scan: thread t owns bins 2047-2t (hi) and 2046-2t (lo) of the live range
    const int nbins = 1 << nb;
    const int hi = nbins - 1 - 2 * tid, lo = hi - 1;
    const uint64_t h_hi = hi >= 0 ? hist[hi] : 0, h_lo = lo >= 0 ? hist[lo] : 0;
    uint64_t tot;
    const uint64_t excl = block_exclusive_scan_u64(h_hi + h_lo, sm.scratch64, &tot);
    if (hi >= 0 && excl < target && excl + h_hi >= target) {
      sm.bcast64[0] = (uint64_t)hi;
      sm.bcast64[1] = excl;
    } else if (lo >= 0 && excl + h_hi < target && excl + h_hi + h_lo >= target) {
      sm.bcast64[0] = (uint64_t)lo;
      sm.bcast64[1] = excl + h_hi;
    }
    __syncthreads();
    prefix = (prefix << nb) | (uint32_t)sm.bcast64[0];
    target -= (uint32_t)sm.bcast64[1];
    __syncthreads();
  }
  return key_to_float(prefix);
}

// Merge of one row by the last-arriving workgroup.
__device__ void finalize_row(const SampleKArgs& a, const FastPlan& P, int b, int rule, float T, float top_p,
                             float min_p, int top_k, bool use_k, bool use_p, bool use_m, char* dyn, ExactSmem& sm) {
  const int tid = threadIdx.x;
  const int G = P.G;
  const SliceHdr* H = P.hdr + (long long)b * G;
  __shared__ float s_m[16], s_tau[16], s_bv[16];
  __shared__ int s_n[16], s_off[17], s_flag, s_bi[16];
  __shared__ double s_zf[16];
  if (tid < G) {
    s_m[tid] = H[tid].m;
    s_tau[tid] = H[tid].tau;
    s_n[tid] = H[tid].n;
    s_zf[tid] = H[tid].zf;
    s_bv[tid] = H[tid].best_v;
    s_bi[tid] = H[tid].best_i;
  }
  if (tid == 0) P.counters[b] = 0;  // all G slices have arrived: ready for the next call
  __syncthreads();
  if (tid == 0) {
    int f = 0, off = 0;
    for (int s = 0; s < G; ++s) {
      f |= H[s].flags;
      s_off[s] = off;
      off += s_n[s];
    }
    s_off[G] = off;
    s_flag = f;
  }
  __syncthreads();
  float* out = a.out_rows ? a.out_rows + (long long)b * a.V : nullptr;

  if (rule == RULE_GREEDY) {
    if (tid == 0) {
      float bv = s_bv[0];
      int bi = s_bi[0];
      for (int s = 1; s < G; ++s)
        if (s_bv[s] > bv || (s_bv[s] == bv && s_bi[s] < bi)) { bv = s_bv[s]; bi = s_bi[s]; }
      if (a.tokens) a.tokens[b] = bi;
      if (a.kept) a.kept[b] = 1;
    }
    return;
  }
  if (rule == RULE_ALL || s_flag) {
    exact_row(a, b, dyn, sm);
    return;
  }
  float m = -INFINITY, tcov = -INFINITY;
  for (int s = 0; s < G; ++s) { m = fmaxf(m, s_m[s]); tcov = fmaxf(tcov, s_tau[s]); }
  const int N = s_off[G];
  float* cv = (float*)dyn;
  int* ci = (int*)(dyn + (size_t)G * P.cap * sizeof(float));
  for (int s = 0; s < G; ++s) {
    const int2* src = P.cand + ((long long)b * G + s) * P.cap;
    for (int j = tid; j < s_n[s]; j += FT) {
      int2 c = src[j];
      cv[s_off[s] + j] = __int_as_float(c.x);
      ci[s_off[s] + j] = c.y;
    }
  }
  __syncthreads();
  CandSource src{cv, ci, N};
  Pred pr = {0, 0, 0, 0, 0, 0, 0.0f, -INFINITY};
  auto mass = [m](int, float l) { return exp_fix44(l - m); };
  auto one = [](int, float) { return (uint64_t)1; };
  auto count = [&](const Pred& p) {
    int c = 0;
    src.each([&](int i, float l) { c += p.keep(i, l) ? 1 : 0; });
    return block_reduce(c, sm.scratchi, OpSumI(), 0);
  };
  auto msum = [&](const Pred& p) {
    uint64_t z = 0;
    src.each([&](int i, float l) { if (p.keep(i, l)) z += exp_fix44(l - m); });
    return block_reduce(z, sm.scratch64, OpSumU64(), (uint64_t)0);
  };
  const float theta = (float)(1.0 - (double)top_p);
  bool ambiguous = false;

  // Top-p with the normaliser known to within [Zlo, Zhi] (fixed point, 44
  // fractional bits).  S is the alive mass (exact when `s_exact`, else Z).
  auto apply_p = [&](bool s_exact) {
    double zt = 0.0;
    for (int s = 0; s < G; ++s)
      if (s_m[s] != -INFINITY) zt += s_zf[s] * exp((double)s_m[s] - (double)m);
    // |Z/2^44 - zt| <= 1e-4 zt + 1e-6 (hardware-exp and float-sum error, with margin)
    const double sc = 17592186044416.0;
    const double zl = fmax(0.0, (zt * (1.0 - 1e-4) - 1e-6) * sc), zh = (zt * (1.0 + 1e-4) + 1e-6) * sc;
    const uint64_t Zlo = (uint64_t)zl, Zhi = (uint64_t)ceil(zh);
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
      // every covered element survives; the kept set stays inside the covered
      // region only if a later filter confines it there (min-p cut >= every
      // slice threshold, or the top-k set, all of which is covered)
      if (rule == RULE_P) ambiguous = true;
      return;
    }
    if (Rhi > Scov) { ambiguous = true; return; }
    const uint64_t clo = radix_select<ORD_P>(src, pc, mass, (uint64_t)Rlo, sm);
    const uint64_t chi = radix_select<ORD_P>(src, pc, mass, (uint64_t)Rhi, sm);
    if (clo != chi) { ambiguous = true; return; }
    pr.use_p = 1;
    pr.cp = clo;
  };
  auto apply_m = [&]() {
    const float c = a.min_p_rows ? (float)log((double)min_p) : a.min_p_log;
    pr.use_m = 1;
    pr.thr = m + c;
  };
  if (a.chain == WH_CHAIN_MLX && rule == RULE_K) {
    // the candidates hold the whole top-k set (at least k of them)
    if (use_k) {
      pr.ck = radix_select<ORD_A>(src, pr, one, (uint64_t)top_k, sm);
      pr.use_k = 1;
    }
    if (use_p) apply_p(use_k);
    if (!ambiguous && use_m && !pr.none) apply_m();
  } else if (a.chain == WH_CHAIN_MLX) {
    // rule M or P: no top-p together with top-k here.  k -> min-p: the min-p
    // set is a value prefix held by the candidates; if it has more than k
    // members the row's first k (order A) are its first k, else top-k keeps
    // all of it.
    if (use_p) apply_p(false);
    if (!ambiguous && use_m && !pr.none) apply_m();
    if (!ambiguous && use_k && !pr.none && count(pr) > top_k) {
      pr.ck = radix_select<ORD_A>(src, pr, one, (uint64_t)top_k, sm);
      pr.use_k = 1;
    }
  } else {
    if (use_p) apply_p(false);
    if (!ambiguous && use_m && !pr.none) apply_m();
    if (!ambiguous && use_k && !pr.none) {
      if (count(pr) > top_k) {
        pr.ck = radix_select<ORD_A>(src, pr, one, (uint64_t)top_k, sm);
        pr.use_k = 1;
      }
    }
  }
  if (ambiguous) {
    exact_row(a, b, dyn, sm);
    return;
  }
  // Draw: integer inverse CDF in vocabulary order over the kept candidates.
  const float invT = (float)(1.0 / (double)T);
  const float Tc = (float)fmax((double)T, 1e-5);
  auto vw = [&](int, float l) { return exp_fix44(chain_scale(a.chain, l - m, invT, Tc)); };
  uint64_t zv = 0;
  int nk = 0;
  src.each([&](int i, float l) {
    if (pr.keep(i, l)) { zv += vw(i, l); ++nk; }
  });
  const uint64_t ZV = block_reduce(zv, sm.scratch64, OpSumU64(), (uint64_t)0);
  const int nkept = block_reduce(nk, sm.scratchi, OpSumI(), 0);
  if (a.tokens) {
    int tok = 0;
    if (ZV) {
      const uint64_t tgt = draw_target(a.u[b], ZV);
      tok = 0x3FFFF - (int)radix_select<ORD_ID>(src, pr, vw, tgt + 1, sm);
    }
    if (tid == 0) a.tokens[b] = tok;
  }
  if (tid == 0 && a.kept) a.kept[b] = nkept;
  if (out) {
    const double lz = log(ldexp((double)ZV, -44));
    src.each([&](int i, float l) {
      if (!pr.keep(i, l)) return;
      out[i] = a.out_mode == WH_OUT_MASKED ? l : (float)((double)chain_scale(a.chain, l - m, invT, Tc) - lz);
    });
  }
}

template <int DT, int R>
__global__ void __launch_bounds__(FT) sample_fast_kernel(SampleKArgs a, FastPlan P) {
  extern __shared__ __align__(16) char dyn[];
  __shared__ ExactSmem sm;
  __shared__ int s_cnt, s_np, s_last;
  constexpr int EPT = DT ? 8 : 4;
  constexpr int ESZ = DT ? 2 : 4;
  const int tid = threadIdx.x;
  const int bid = blockIdx.x, xcd = bid & 7, q = bid >> 3;
  const int s = q % P.G, b = (q / P.G) * 8 + xcd;
  if (b >= a.B) return;
  const int V = a.V;
  const int v0 = s * P.SL, v1 = min(V, v0 + P.SL);

  const float T = a.T_rows ? a.T_rows[b] : a.T;
  const float top_p = a.top_p_rows ? a.top_p_rows[b] : a.top_p;
  const float min_p = a.min_p_rows ? a.min_p_rows[b] : a.min_p;
  const int top_k = a.top_k_rows ? a.top_k_rows[b] : a.top_k;
  const bool use_k = top_k > 0 && top_k < V;
  const bool use_p = top_p > 0.0f && top_p < 1.0f;
  const bool use_m = min_p != 0.0f;
  const int rule = choose_rule(a.chain, T, use_k, use_p, use_m, top_k, P.rule_cap);
  float* out = a.out_rows ? a.out_rows + (long long)b * V : nullptr;
  SliceHdr* hdr = P.hdr + (long long)b * P.G + s;

  if (rule != RULE_ALL) {
    // 1. the slice, straight into registers
    const char* rowp = (const char*)a.logits + (size_t)b * a.row_stride * ESZ;
    uint4 d[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int g = v0 + (r * FT + tid) * EPT;
      if (g < v1) d[r] = *(const uint4*)(rowp + (size_t)g * ESZ);
    }
    // 2. penalties for the slice's history tokens; the penalised values go to
    //    a list (ids pl_id, values pl_v) and their register copies become -inf
    int np = 0;
    const int* pl_id = nullptr;
    const float* pl_v = nullptr;
    if (a.hcap > 0) {
      RowCtx rc;
      rc.V = V;
      rc.xf = DT == 0 ? (const float*)rowp : nullptr;
      rc.xb = DT == 1 ? (const uint16_t*)rowp : nullptr;
      build_penalties(a, b, rc, dyn, v0, v1);
      int32_t* hkeys = (int32_t*)dyn;
      float* hval = (float*)(hkeys + a.hcap);
      int32_t* hcnt = hkeys + 2 * a.hcap;
      const uint32_t* bm = (const uint32_t*)(hkeys + 3 * a.hcap);
      // compact (key, value) pairs: read own slots, then write the list over
      // hcnt (ids) and hkeys (values)
      int kk[8];
      float vv[8];
      int nmine = 0;
      for (int t = tid; t < a.hcap; t += FT) {
        if (hkeys[t] >= 0) { kk[nmine] = hkeys[t]; vv[nmine] = hval[t]; ++nmine; }
      }
      if (tid == 0) s_np = 0;
      __syncthreads();
      for (int j = 0; j < nmine; ++j) {
        int slot = atomicAdd(&s_np, 1);
        hcnt[slot] = kk[j];
        ((float*)hkeys)[slot] = vv[j];
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int g = v0 + (r * FT + tid) * EPT;
        if (g < v1) {
          const int o = g - v0;
          const uint32_t bits = (bm[o >> 5] >> (o & 31)) & ((1u << EPT) - 1u);
          if (bits) {
#pragma unroll
            for (int e = 0; e < EPT; ++e)
              if ((bits >> e) & 1u) grp_kill<DT>(d[r], e);
          }
        }
      }
      __syncthreads();
      np = s_np;
      pl_id = hcnt;
      pl_v = (const float*)hkeys;
    }
    // 3. slice max and, for greedy rows, the lowest index attaining it
    float mx = -INFINITY;
    int mi = 0x7FFFFFFF;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int g = v0 + (r * FT + tid) * EPT;
      if (g < v1) {
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          const float l = grp_elem<DT>(d[r], e);
          if (mi == 0x7FFFFFFF || l > mx) { mx = l; mi = g + e; }
        }
      }
    }
    for (int j = tid; j < np; j += FT) {
      const float l = pl_v[j];
      const int i = pl_id[j];
      if (mi == 0x7FFFFFFF || l > mx || (l == mx && i < mi)) { mx = l; mi = i; }
    }
    const float ms = block_reduce(mx, sm.scratchf, OpMaxF(), -INFINITY);

    if (rule == RULE_GREEDY) {
      const int cand = (mi != 0x7FFFFFFF && mx == ms) ? mi : 0x7FFFFFFF;
      const int bi = block_reduce(cand, sm.scratchi, OpMinI(), 0x7FFFFFFF);
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
        for (int j = tid; j < np; j += FT) out[pl_id[j]] = pl_v[j];
      }
      if (tid == 0) {
        hdr->best_v = ms;
        hdr->best_i = bi;
        hdr->flags = 0;
        hdr->n = 0;
      }
    } else {
      // 4. candidate threshold
      float tau;
      if (rule == RULE_M) {
        const float c = a.min_p_rows ? (float)log((double)min_p) : a.min_p_log;
        tau = ms + c;
      } else {
        tau = slice_kth<DT, R>(d, v0, v1, pl_id, pl_v, np, rule == RULE_K ? top_k : P.rule_cap, sm);
      }
      // 5. compact the candidates into LDS, then to the workspace
      int2* buf = (int2*)(dyn + cand_buf_offset(a.hcap, P.SL));
      if (tid == 0) s_cnt = 0;
      __syncthreads();
      float zs = 0.0f;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int g = v0 + (r * FT + tid) * EPT;
        if (g < v1) {
#pragma unroll
          for (int e = 0; e < EPT; ++e) {
            const float l = grp_elem<DT>(d[r], e);
            if (l >= tau) {
              const int slot = atomicAdd(&s_cnt, 1);
              if (slot < P.cap) buf[slot] = make_int2(__float_as_int(l), g + e);
            }
            if (use_p && ms != -INFINITY) zs += __expf(l - ms);
          }
        }
      }
      for (int j = tid; j < np; j += FT) {
        const float l = pl_v[j];
        if (l >= tau) {
          const int slot = atomicAdd(&s_cnt, 1);
          if (slot < P.cap) buf[slot] = make_int2(__float_as_int(l), pl_id[j]);
        }
        if (use_p && ms != -INFINITY) zs += __expf(l - ms);
      }
      const double zf = use_p ? block_reduce((double)zs, (double*)sm.scratch64, OpSumF64(), 0.0) : 0.0;
      __syncthreads();
      const int n = s_cnt;
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
        hdr->m = ms;
        hdr->tau = tau;
        hdr->n = nw;
        hdr->flags = n > P.cap ? 1 : 0;
        hdr->zf = zf;
      }
    }
  }
  // 6. arrival: the last slice of the row merges
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = (atomicAdd(&P.counters[b], 1) == P.G - 1);
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  finalize_row(a, P, b, rule, T, top_p, min_p, top_k, use_k, use_p, use_m, dyn, sm);
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
  int g = std::max((512 + B - 1) / std::max(B, 1), (V + slmax - 1) / slmax);
  g = std::min(g, 8);
  p.G = g;
  int sl = (V + g - 1) / g;
  sl = (sl + p.ept - 1) / p.ept * p.ept;
  p.SL = sl;
  p.R = (sl + FT * p.ept - 1) / (FT * p.ept);
  p.cap = std::min(2048, 8192 / g);
  p.rule_cap = p.cap / 2;
  return p;
}

struct WsLayout {
  size_t counters, hdr, cand, total;
};

static WsLayout ws_layout(int B, const HostPlan& p) {
  WsLayout w;
  w.counters = 0;
  w.hdr = ((size_t)B * 4 + 255) / 256 * 256;
  w.cand = w.hdr + (size_t)B * p.G * sizeof(SliceHdr);
  w.total = w.cand + (size_t)B * p.G * p.cap * sizeof(int2);
  return w;
}

size_t sample_workspace_bytes(int B, int V) {
  if (B <= 0 || V <= 0) return 256;
  // the larger of the two element widths' plans
  WsLayout a = ws_layout(B, make_plan(B, V, WH_DTYPE_F32));
  WsLayout b = ws_layout(B, make_plan(B, V, WH_DTYPE_BF16));
  return std::max(a.total, b.total);
}

template <int DT, int R>
static void launch_fast_t(const SampleKArgs& k, const FastPlan& fp, int grid, size_t lds, hipStream_t st) {
  auto fn = sample_fast_kernel<DT, R>;
  if (lds > 65536) hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  hipLaunchKernelGGL(fn, dim3(grid), dim3(FT), lds, st, k, fp);
}

template <int DT>
static void launch_fast_dt(int R, const SampleKArgs& k, const FastPlan& fp, int grid, size_t lds, hipStream_t st) {
  switch (R) {
    case 1: launch_fast_t<DT, 1>(k, fp, grid, lds, st); break;
    case 2: launch_fast_t<DT, 2>(k, fp, grid, lds, st); break;
    case 3: launch_fast_t<DT, 3>(k, fp, grid, lds, st); break;
    case 4: launch_fast_t<DT, 4>(k, fp, grid, lds, st); break;
    case 5: launch_fast_t<DT, 5>(k, fp, grid, lds, st); break;
    case 6: launch_fast_t<DT, 6>(k, fp, grid, lds, st); break;
    case 7: launch_fast_t<DT, 7>(k, fp, grid, lds, st); break;
    default: launch_fast_t<DT, 8>(k, fp, grid, lds, st); break;
  }
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
  fp.counters = (int*)(ws + wl.counters);
  fp.hdr = (SliceHdr*)(ws + wl.hdr);
  fp.cand = (int2*)(ws + wl.cand);
  // dynamic LDS: slice phase (hash + slice bitmap + candidate buffer), merge
  // phase (G * cap candidates), exact fallback (hash + row bitmap)
  const size_t slice = cand_buf_offset(k.hcap, hp.SL) + (size_t)hp.cap * sizeof(int2);
  const size_t merge = (size_t)hp.G * hp.cap * 8;
  const size_t exact = penalty_lds_bytes(k);
  const size_t lds = std::max(slice, std::max(merge, exact));
  const int grid = (k.B + 7) / 8 * 8 * hp.G;
  if (k.dtype == WH_DTYPE_BF16) launch_fast_dt<1>(hp.R, k, fp, grid, lds, st);
  else launch_fast_dt<0>(hp.R, k, fp, grid, lds, st);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "sample_fast_kernel launch failed: %s", hipGetErrorString(e));
  return WH_OK;
}

}  // namespace wh
