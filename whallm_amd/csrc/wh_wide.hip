// wh_wide.hip -- the wide exact engine: rows whose only filter is top-p, or
// that have none, sampled by many workgroups per row.
//
// The fast engine bounds its candidates by the filters (top-k, min-p, or a
// top-p cut inside a few thousand candidates).  A nucleus larger than that,
// or no filter at all (every element kept), sent a row to the one-workgroup
// exact engine: 200-650 us for one row of 129,280.  Whallm's own defaults
// are exactly such rows (GenerationOptions: temperature 0.2, top_p 0.98, no
// top-k or min-p, runtime/deepseek_v4_ssd/generation.py:109-118; the Qwen
// package: 0.7 / 0.8), and so is an OpenAI request with top_p = 1.
//
// Same contract as exact_row (results identical), in slices of 256 * E
// entries (E = 4 for up to 8 rows, so one row spreads over more CUs; 16
// otherwise), one 256-thread workgroup each, every thread holding its E
// entries in registers (loads issued together):
//   1. max: each slice's max (and, for greedy rows, its lowest index at the
//      max); also clears the row's histogram.
//   2. hist (rows with top-p): each element's mass exp_fix44(l - m) is added
//      to a histogram of 2048 bins of 1/64 nat below the row max (bin
//      floor((m - l) * 64), clamped), u64 masses and counts, through LDS and
//      then global atomics.  The bin is monotone in the value, so bins are
//      ranges of the top-p order.
//   3. collect: every workgroup scans the row's histogram (identically) for
//      the bin where the cumulative mass reaches R = Z - floor(theta Z), and
//      appends that bin's elements to the row's list.
//   4. resolve (one workgroup per row): the listed element where the mass,
//      in (value desc, id desc) order, reaches R minus the bins above: the
//      cut.  Up to 1024 entries each thread ranks one against all the others
//      from LDS; longer lists take a radix select.  A list past its capacity
//      (a bin holding more than 8192 tied or near-tied entries) makes the row
//      run exact_row instead.  Greedy rows and rows with nothing kept finish
//      here.
//   5. drawsum: each slice's kept draw weights and count.
//   6. pick (one workgroup per row): the slice holding the draw target (a
//      block scan over the slice sums), then the element inside it (a block
//      scan over the slice, in id order).
//   7. rows (when logprob rows are requested): each slice writes its entries.
// Without top-p, steps 2-4 are skipped.  Penalties: every slice workgroup
// builds the penalty table of its own id range from the history window.
#include "wh_rowops.h"

namespace wh {

constexpr int WX_T = 256;       // threads per slice workgroup
constexpr int WX_BINS = 2048;   // mass bins, 1/64 nat each, below the row max
constexpr int WX_CAP = 8192;    // boundary-bin list capacity per row
constexpr int WX_RANK = 1024;   // sub-bin lists up to this long are ranked directly
constexpr int WX_DIRECT = 64;
constexpr int WX_HS = 4;        // slices per histogram workgroup   // boundary lists up to this long are ranked without sub-bins
constexpr int WX_MAXG = 256;    // slices per row, at most (V <= 2^18, 1024-entry slices)
constexpr int WX_DONE = 1;      // WxRec.flags: token, count and row already written
constexpr int WX_NONE = 2;      // WxRec.flags: nothing kept (set by the collect step)
constexpr int WX_PATH = 6;      // path code of rows this engine settles

struct WxRec {
  uint64_t cum_excl;  // mass of the bins above the boundary bin
  uint64_t R;         // cut target Z - floor(theta Z)
  uint64_t cstar;     // order-P composite of the last kept element
  uint64_t ZV;        // kept draw weights' sum
  int bstar;          // boundary bin
  int flags;
};

struct WxPtrs {
  int* path;          // [B]
  float* part_m;      // [B * G] slice maxima
  int* part_i;        // [B * G] lowest index at the slice max
  uint64_t* part_vw;  // [B * G] kept draw weights per slice
  int* part_n;        // [B * G] kept entries per slice
  uint64_t* hist_w;   // [B * WX_BINS]
  float* list_v;      // [B * WX_CAP]
  int* list_i;        // [B * WX_CAP]
  int* lcnt;          // [B]
  WxRec* rec;         // [B]
  // [B * G] (value key << 32 | ~index) maxima per slice, written by the LM
  // head's epilogue in place of the max step (nullptr otherwise)
  uint64_t* part_key;
  int G;              // slices per row
  int SL;             // entries per slice (256 * E)
};

struct WxRow {
  bool greedy, use_p;
  float theta, invT;
  double rTc;
};

__device__ __forceinline__ WxRow wx_row(const SampleKArgs& a, int b) {
  // the caller's doubles, and the float32 constants derived from them as
  // exact_row derives them
  const double T = a.T_rows ? a.T_rows[b] : a.T;
  const double top_p = a.top_p_rows ? a.top_p_rows[b] : a.top_p;
  WxRow r;
  r.greedy = !(T > 0.0);
  r.use_p = top_p > 0.0 && top_p < 1.0;
  r.theta = (float)(1.0 - top_p);
  r.invT = (float)(1.0 / T);
  r.rTc = 1.0 / (double)(float)fmax(T, 1e-5);
  return r;
}

// The row's view: its logits (penalties added by wx_pen).
__device__ __forceinline__ void wx_ptrs(const SampleKArgs& a, int b, RowCtx& rc) {
  rc.V = a.V;
  rc.xf = a.dtype == WH_DTYPE_F32 ? (const float*)a.logits + b * a.row_stride : nullptr;
  rc.xb = a.dtype == WH_DTYPE_BF16 ? (const uint16_t*)a.logits + b * a.row_stride : nullptr;
  rc.hmask = -1;
}

// The penalty table of the slice's id range [lo, hi) (lo is a multiple of
// 32, so the table's bitmap, which starts at lo, is addressed by absolute id
// after the offset below).
__device__ __forceinline__ void wx_pen_table(const SampleKArgs& a, int b, int lo, int hi, char* dyn, RowCtx& rc) {
  if (a.hcap > 0) {
    build_penalties(a, b, rc, dyn, lo, hi);
    rc.bitmap -= lo >> 5;
  }
}

// Id of a thread's entry j in the slice starting at lo.  Scalar layout:
// lo + tid + 256 j, one 2- or 4-byte load per entry.  Vector layout (V a
// multiple of 4, rows aligned to 4 entries): runs of four consecutive ids,
// lo + 4 (tid + 256 (j / 4)) + j % 4, one 8- or 16-byte load per run, so a
// wave's load instruction moves 512 or 1024 bytes instead of 128 or 256.
// Either way the ids grow with j.
// (The thread index within the slice's 256: a workgroup may cover several
// slices, 256 threads each.)
__device__ __forceinline__ int wx_t() { return (int)threadIdx.x & (WX_T - 1); }
template <bool VEC>
__device__ __forceinline__ int wx_id(int lo, int j) {
  return VEC ? lo + 4 * (wx_t() + WX_T * (j >> 2)) + (j & 3) : lo + wx_t() + WX_T * j;
}

// A thread's E raw entries of the slice (coalesced, in the layout above).
// Every load is unconditional, from an in-bounds address (entries past hi
// read entry lo and become 0), with the element type chosen once outside
// the loop: the loads then issue back to back and are waited for once.
// (Conditional loads had compiled to one branch and one full wait per
// entry, E dependent round trips per thread in every step of the engine.)
template <int E, bool VEC>
__device__ __forceinline__ void wx_raw(const RowCtx& rc, int lo, int hi, float (&v)[E]) {
  static_assert(!VEC || E % 4 == 0, "whole runs of four entries");
  if (VEC) {
    // a run lies wholly inside or outside [lo, hi): lo, hi and V are
    // multiples of 4
    constexpr int NQ = E / 4;
    if (rc.xf) {
      float4 q[NQ];
#pragma unroll
      for (int g = 0; g < NQ; ++g) {
        const int i0 = wx_id<true>(lo, 4 * g);
        q[g] = *(const float4*)(rc.xf + (i0 < hi ? i0 : lo));
      }
#pragma unroll
      for (int g = 0; g < NQ; ++g) {
        v[4 * g] = q[g].x;
        v[4 * g + 1] = q[g].y;
        v[4 * g + 2] = q[g].z;
        v[4 * g + 3] = q[g].w;
      }
    } else {
      uint2 q[NQ];
#pragma unroll
      for (int g = 0; g < NQ; ++g) {
        const int i0 = wx_id<true>(lo, 4 * g);
        q[g] = *(const uint2*)(rc.xb + (i0 < hi ? i0 : lo));
      }
#pragma unroll
      for (int g = 0; g < NQ; ++g) {
        v[4 * g] = bf16_to_f32((uint16_t)(q[g].x & 0xFFFFu));
        v[4 * g + 1] = bf16_to_f32((uint16_t)(q[g].x >> 16));
        v[4 * g + 2] = bf16_to_f32((uint16_t)(q[g].y & 0xFFFFu));
        v[4 * g + 3] = bf16_to_f32((uint16_t)(q[g].y >> 16));
      }
    }
  } else if (rc.xf) {
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const int i = wx_id<false>(lo, j);
      v[j] = rc.xf[i < hi ? i : lo];
    }
  } else {
    uint16_t h[E];
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const int i = wx_id<false>(lo, j);
      h[j] = rc.xb[i < hi ? i : lo];
    }
#pragma unroll
    for (int j = 0; j < E; ++j) v[j] = bf16_to_f32(h[j]);
  }
#pragma unroll
  for (int j = 0; j < E; ++j)
    if (wx_id<VEC>(lo, j) >= hi) v[j] = 0.0f;
}
// A thread's E consecutive raw entries s0 .. s0 + E - 1 (the pick step's
// layout), loaded the same way: unconditional, in bounds, back to back; in
// runs of four with the vector layout's alignment (a run past hi reads the
// slice's last run and becomes 0).
template <int E, bool VEC>
__device__ __forceinline__ void wx_raw_run(const RowCtx& rc, int s0, int hi, float (&v)[E]) {
  const int last = hi - 1;  // the slice is never empty
  if (VEC) {
    constexpr int NQ = E / 4;
    if (rc.xf) {
      float4 q[NQ];
#pragma unroll
      for (int g = 0; g < NQ; ++g) q[g] = *(const float4*)(rc.xf + min(s0 + 4 * g, hi - 4));
#pragma unroll
      for (int g = 0; g < NQ; ++g) {
        v[4 * g] = q[g].x;
        v[4 * g + 1] = q[g].y;
        v[4 * g + 2] = q[g].z;
        v[4 * g + 3] = q[g].w;
      }
    } else {
      uint2 q[NQ];
#pragma unroll
      for (int g = 0; g < NQ; ++g) q[g] = *(const uint2*)(rc.xb + min(s0 + 4 * g, hi - 4));
#pragma unroll
      for (int g = 0; g < NQ; ++g) {
        v[4 * g] = bf16_to_f32((uint16_t)(q[g].x & 0xFFFFu));
        v[4 * g + 1] = bf16_to_f32((uint16_t)(q[g].x >> 16));
        v[4 * g + 2] = bf16_to_f32((uint16_t)(q[g].y & 0xFFFFu));
        v[4 * g + 3] = bf16_to_f32((uint16_t)(q[g].y >> 16));
      }
    }
  } else if (rc.xf) {
#pragma unroll
    for (int j = 0; j < E; ++j) v[j] = rc.xf[min(s0 + j, last)];
  } else {
    uint16_t h[E];
#pragma unroll
    for (int j = 0; j < E; ++j) h[j] = rc.xb[min(s0 + j, last)];
#pragma unroll
    for (int j = 0; j < E; ++j) v[j] = bf16_to_f32(h[j]);
  }
#pragma unroll
  for (int j = 0; j < E; ++j)
    if (s0 + j >= hi) v[j] = 0.0f;
}
// Raw entries to effective (penalised, -0 as +0) values.
template <int E, bool VEC>
__device__ __forceinline__ void wx_pen(const RowCtx& rc, int lo, int hi, float (&v)[E]) {
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const int i = wx_id<VEC>(lo, j);
    v[j] = i < hi ? rc.val_from(i, v[j]) : 0.0f;
  }
}

// The slice's effective values: the logits loads issue first, then the
// penalty table is built while they are in flight.
template <int E, bool VEC>
__device__ __forceinline__ void wx_slice(const SampleKArgs& a, int b, int lo, int hi, char* dyn, RowCtx& rc,
                                         float (&v)[E]) {
  wx_ptrs(a, b, rc);
  wx_raw<E, VEC>(rc, lo, hi, v);
  wx_pen_table(a, b, lo, hi, dyn, rc);
  wx_pen<E, VEC>(rc, lo, hi, v);
}

// Row max from the slice maxima (every thread returns it).
__device__ __forceinline__ float wx_row_max(const WxPtrs& P, int b, float* scratch) {
  float m = -INFINITY;
  for (int g = threadIdx.x; g < P.G; g += blockDim.x) {
    if (P.part_key) {
      const uint64_t k = P.part_key[(size_t)b * P.G + g];
      m = fmaxf(m, k ? key_to_float((uint32_t)(k >> 32)) : -INFINITY);
    } else {
      m = fmaxf(m, P.part_m[(size_t)b * P.G + g]);
    }
  }
  return block_reduce(m, scratch, OpMaxF(), -INFINITY);
}

// Before an LM head that writes the slice maxima itself: clear them, the
// histograms and the list counters, and set the records (the max step's
// other duties).
__global__ void __launch_bounds__(WX_T) wx_init_kernel(WxPtrs P, int B) {
  const size_t i = (size_t)blockIdx.x * WX_T + threadIdx.x;
  if (i < (size_t)B * P.G) P.part_key[i] = 0;
  if (i < (size_t)B * WX_BINS) P.hist_w[i] = 0;
  if (i < (size_t)B) {
    P.lcnt[i] = 0;
    P.rec[i].flags = 0;
    P.path[i] = WX_PATH;
  }
}

__device__ __forceinline__ int wx_bin(float m, float l) {
  const float d = m - l;
  return d >= 32.0f ? WX_BINS - 1 : (int)(d * 64.0f);
}

template <int E, bool VEC>
__global__ void __launch_bounds__(WX_T) wx_max_kernel(SampleKArgs a, WxPtrs P) {
  extern __shared__ __align__(16) char dyn[];
  __shared__ float sf[16];
  __shared__ int si[16];
  const int b = blockIdx.y, g = blockIdx.x, tid = threadIdx.x;
  const int lo = g * P.SL, hi = min(a.V, lo + P.SL);
  RowCtx rc;
  float v[E];
  wx_slice<E, VEC>(a, b, lo, hi, dyn, rc, v);
  const WxRow rp = wx_row(a, b);
  float* out = (a.out_rows && rp.greedy) ? a.out_rows + (long long)b * a.V : nullptr;
  float bv = -INFINITY;
  int bi = 0x7FFFFFFF;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const int i = wx_id<VEC>(lo, j);
    if (i >= hi) break;
    if (bi == 0x7FFFFFFF || v[j] > bv) {
      bv = v[j];
      bi = i;
    }
    if (out) out[i] = v[j];  // sampling_logprobs returns the (penalised) logits at T == 0
  }
  const float m = block_reduce(bv, sf, OpMaxF(), -INFINITY);
  const int cand = (bi != 0x7FFFFFFF && bv == m) ? bi : 0x7FFFFFFF;
  const int is = block_reduce(cand, si, OpMinI(), 0x7FFFFFFF);
  if (tid == 0) {
    P.part_m[(size_t)b * P.G + g] = m;
    P.part_i[(size_t)b * P.G + g] = is;
  }
  for (int j = g * WX_T + tid; j < WX_BINS; j += P.G * WX_T) P.hist_w[(size_t)b * WX_BINS + j] = 0;
  if (g == 0 && tid == 0) {
    P.lcnt[b] = 0;
    // rows without top-p need no resolve step: their record is ready here
    // (the collect and resolve steps rewrite it for the others)
    P.rec[b].flags = 0;
    P.path[b] = WX_PATH;
  }
}

// The histogram step: one workgroup of 256 WX_HS threads per WX_HS
// consecutive slices (256 threads each), one LDS histogram for all of them,
// so each non-empty bin costs one global atomic per WX_HS slices.  (With one
// slice per workgroup the global atomics took half the step: 31 against
// 15.5 us at B = 64, V = 151,936.)  Slices past the row's last read the
// workgroup's first slice over an empty range: in bounds, nothing counted.
template <int E, bool VEC>
__global__ void __launch_bounds__(WX_T * WX_HS) wx_hist_kernel(SampleKArgs a, WxPtrs P) {
  extern __shared__ __align__(16) char dyn[];
  __shared__ float sf[16];
  __shared__ uint64_t hw[WX_BINS];
  const int b = blockIdx.y, tid = threadIdx.x;
  const WxRow rp = wx_row(a, b);
  if (rp.greedy || !rp.use_p) return;
  const int s0 = blockIdx.x * WX_HS, sl = s0 + (tid >> 8);
  const bool has = sl < P.G;
  const int lo = (has ? sl : s0) * P.SL, hi = has ? min(a.V, lo + P.SL) : lo;
  const int wlo = s0 * P.SL, whi = min(a.V, (s0 + WX_HS) * P.SL);  // the workgroup's id range
  RowCtx rc;
  float v[E];
  wx_ptrs(a, b, rc);
  wx_raw<E, VEC>(rc, lo, hi, v);  // in flight with the slice maxima
  const float m = wx_row_max(P, b, sf);
  if (m == -INFINITY) return;
  for (int j = tid; j < WX_BINS; j += WX_T * WX_HS) hw[j] = 0;
  __syncthreads();
  wx_pen_table(a, b, wlo, whi, dyn, rc);
  wx_pen<E, VEC>(rc, lo, hi, v);
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const float l = v[j];
    if (wx_id<VEC>(lo, j) >= hi || l != l) continue;
    const uint64_t w = exp_fix44(l - m);
    if (w) atomicAdd((unsigned long long*)&hw[wx_bin(m, l)], (unsigned long long)w);
  }
  __syncthreads();
  for (int j = tid; j < WX_BINS; j += WX_T * WX_HS)
    if (hw[j]) atomicAdd((unsigned long long*)&P.hist_w[(size_t)b * WX_BINS + j], (unsigned long long)hw[j]);
}

template <int E, bool VEC>
__global__ void __launch_bounds__(WX_T) wx_collect_kernel(SampleKArgs a, WxPtrs P) {
  extern __shared__ __align__(16) char dyn[];
  __shared__ float sf[16];
  __shared__ uint64_t s64[16];
  __shared__ uint64_t bc[1];
  __shared__ int bs[2];
  const int b = blockIdx.y, g = blockIdx.x, tid = threadIdx.x;
  const bool first = g == 0 && tid == 0;  // writes the row's record
  const WxRow rp = wx_row(a, b);
  if (rp.greedy || !rp.use_p) return;
  const int lo = g * P.SL, hi = min(a.V, lo + P.SL);
  RowCtx rc;
  float v[E];
  wx_ptrs(a, b, rc);
  wx_raw<E, VEC>(rc, lo, hi, v);  // in flight with the maxima and the histogram
  const float m = wx_row_max(P, b, sf);
  WxRec* rec = P.rec + b;
  if (m == -INFINITY) {  // nothing kept
    if (first) rec->flags = WX_NONE;
    return;
  }
  // the boundary bin, from the row's whole histogram (every workgroup alike)
  constexpr int PER = WX_BINS / WX_T;
  const uint64_t* hwr = P.hist_w + (size_t)b * WX_BINS + tid * PER;
  uint64_t hv[PER];
  uint64_t ls = 0;
#pragma unroll
  for (int q = 0; q < PER; ++q) hv[q] = hwr[q];
#pragma unroll
  for (int q = 0; q < PER; ++q) ls += hv[q];
  uint64_t Z;
  const uint64_t excl = block_exclusive_scan_u64(ls, s64, &Z);
  const uint64_t F = floor_theta_z(rp.theta, Z);
  if (Z <= F) {  // nothing kept
    if (first) rec->flags = WX_NONE;
    return;
  }
  const uint64_t R = Z - F;
  if (excl < R && R <= excl + ls) {
    uint64_t c = excl;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      if (c < R && c + hv[q] >= R) {
        bs[0] = tid * PER + q;
        bc[0] = c;
      }
      c += hv[q];
    }
  }
  __syncthreads();
  const int bstar = bs[0];
  if (first) {
    rec->cum_excl = bc[0];
    rec->R = R;
    rec->bstar = bstar;
    rec->flags = 0;
  }
  wx_pen_table(a, b, lo, hi, dyn, rc);
  wx_pen<E, VEC>(rc, lo, hi, v);
  // the slice's boundary-bin entries: one list reservation per workgroup
  uint32_t hit = 0;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const int i = wx_id<VEC>(lo, j);
    if (i < hi && v[j] == v[j] && wx_bin(m, v[j]) == bstar) hit |= 1u << j;
  }
  uint64_t nall;
  const uint64_t off = block_exclusive_scan_u64((uint64_t)__popc(hit), s64, &nall);
  if (nall == 0) return;
  if (tid == 0) bs[1] = atomicAdd(P.lcnt + b, (int)nall);
  __syncthreads();
  int slot = bs[1] + (int)off;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    if (!((hit >> j) & 1u)) continue;
    if (slot < WX_CAP) {
      P.list_v[(size_t)b * WX_CAP + slot] = v[j];
      P.list_i[(size_t)b * WX_CAP + slot] = wx_id<VEC>(lo, j);
    }
    ++slot;
  }
}

// Rows with nothing kept: token 0, count 0, every row entry -inf.
__device__ __forceinline__ void wx_none(const SampleKArgs& a, int b) {
  if (threadIdx.x == 0) {
    if (a.tokens) a.tokens[b] = 0;
    if (a.kept) a.kept[b] = 0;
  }
  if (a.out_rows)
    for (int i = threadIdx.x; i < a.V; i += blockDim.x) a.out_rows[(long long)b * a.V + i] = -INFINITY;
}

// The resolve kernel's arguments in place in the kernel-argument segment:
// the out-of-line exact_row reads them through this pointer, so the kernel
// need not copy its by-value arguments into private memory for it.
struct ResolveKernArgs {
  SampleKArgs a;
  WxPtrs P;
};
static_assert(offsetof(ResolveKernArgs, a) == 0, "resolve kernel argument layout");
__device__ __forceinline__ const ResolveKernArgs* resolve_kernargs() {
  return (const ResolveKernArgs*)__builtin_amdgcn_kernarg_segment_ptr();
}

__global__ void __launch_bounds__(1024) wx_resolve_kernel(SampleKArgs a, WxPtrs P) {
  extern __shared__ __align__(16) char dyn[];
  __shared__ ExactSmem esm;
  __shared__ float sf[16];
  __shared__ int si[16];
  const int b = blockIdx.x, tid = threadIdx.x;
  const WxRow rp = wx_row(a, b);
  WxRec* rec = P.rec + b;
  if (rp.greedy) {
    // lowest index among the row's maxima: the first slice at the max
    const float m = wx_row_max(P, b, sf);
    int cand = 0x7FFFFFFF;
    for (int g = tid; g < P.G; g += blockDim.x)
      if (P.part_m[(size_t)b * P.G + g] == m) cand = min(cand, P.part_i[(size_t)b * P.G + g]);
    const int tok = block_reduce(cand, si, OpMinI(), 0x7FFFFFFF);
    if (tid == 0) {
      if (a.tokens) a.tokens[b] = tok == 0x7FFFFFFF ? 0 : tok;
      if (a.kept) a.kept[b] = 1;
      rec->flags = WX_DONE;
      P.path[b] = 2;
    }
    return;
  }
  if (!rp.use_p) {
    if (tid == 0) {
      rec->flags = 0;
      P.path[b] = WX_PATH;
    }
    return;
  }
  const WxRec r = *rec;  // written by the collect step
  if (r.flags & WX_NONE) {
    wx_none(a, b);
    if (tid == 0) {
      rec->flags = WX_DONE;
      P.path[b] = WX_PATH;
    }
    return;
  }
  const int n = P.lcnt[b];
  if (n > WX_CAP) {
    // the boundary bin overflowed the list: the whole exact algorithm
    exact_row(resolve_kernargs()->a, b, dyn, esm);
    if (tid == 0) {
      rec->flags = WX_DONE;
      P.path[b] = 1;
    }
    return;
  }
  const float m = wx_row_max(P, b, sf);
  const uint64_t target = r.R - r.cum_excl;  // 0 < target <= the list's mass
  uint64_t cstar = 0;
  if (n <= WX_DIRECT) {
    // each listed element's inclusive mass in (value desc, id desc) order,
    // summed over every other from broadcast reads (composites unique)
    uint64_t* lc = (uint64_t*)dyn;
    uint64_t* lw = lc + WX_RANK;
    uint64_t myc = 0, myw = 0;
    if (tid < n) {
      const float l = P.list_v[(size_t)b * WX_CAP + tid];
      myc = comp_p(fkey(l), P.list_i[(size_t)b * WX_CAP + tid]);
      myw = exp_fix44(l - m);
      lc[tid] = myc;
      lw[tid] = myw;
    }
    __syncthreads();
    if (tid < n) {
      uint64_t incl = 0;
      for (int k = 0; k < n; ++k) incl += lc[k] >= myc ? lw[k] : 0;
      if (incl - myw < target && target <= incl) esm.bcast64[0] = myc;
    }
    __syncthreads();
    cstar = esm.bcast64[0];
  } else {
    // 256 sub-bins of the boundary bin (monotone in the value, equal values
    // alike): one pass of masses, a scan for the sub-bin where the target
    // falls, and the broadcast ranking over that sub-bin's entries (the
    // ranking costs n^2 broadcast reads: 13 us for a list of 1024); a
    // sub-bin of more than WX_RANK entries takes the radix select over the
    // whole list
    uint64_t* sub = (uint64_t*)dyn;
    uint64_t* lc = sub + 256;
    uint64_t* lw = lc + WX_RANK;
    __shared__ int s_cnt, s_star;
    __shared__ uint64_t s_rem;
    if (tid < 256) sub[tid] = 0;
    if (tid == 0) {
      s_cnt = 0;
      s_star = -1;
    }
    __syncthreads();
    constexpr int LPT = WX_CAP / 1024;  // entries per thread at most
    float lv[LPT];
    int li[LPT], sb[LPT];
#pragma unroll
    for (int q = 0; q < LPT; ++q) {
      const int j = tid + q * 1024;
      lv[q] = P.list_v[(size_t)b * WX_CAP + (j < n ? j : 0)];
      li[q] = P.list_i[(size_t)b * WX_CAP + (j < n ? j : 0)];
    }
#pragma unroll
    for (int q = 0; q < LPT; ++q) {
      const float d = (m - lv[q]) * 64.0f - (float)r.bstar;
      sb[q] = d >= 1.0f ? 255 : d <= 0.0f ? 0 : min((int)(d * 256.0f), 255);
      if (tid + q * 1024 < n) atomicAdd((unsigned long long*)&sub[sb[q]], (unsigned long long)exp_fix44(lv[q] - m));
    }
    __syncthreads();
    if (tid < 64) {
      // four sub-bins per lane, in order
      uint64_t w4[4], t = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        w4[q] = sub[tid * 4 + q];
        t += w4[q];
      }
      const uint64_t incl = wscan_incl_u64(t);
      uint64_t c = incl - t;
      if (c < target && target <= incl) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (c < target && target <= c + w4[q]) {
            s_star = tid * 4 + q;
            s_rem = target - c;
          }
          c += w4[q];
        }
      }
    }
    __syncthreads();
    const int star = s_star;
    const uint64_t t2 = s_rem;
#pragma unroll
    for (int q = 0; q < LPT; ++q) {
      if (tid + q * 1024 < n && sb[q] == star) {
        const int slot = atomicAdd(&s_cnt, 1);
        if (slot < WX_RANK) {
          lc[slot] = comp_p(fkey(lv[q]), li[q]);
          lw[slot] = exp_fix44(lv[q] - m);
        }
      }
    }
    __syncthreads();
    const int ns = s_cnt;
    // (the target lies within the list's mass, the sum of the same integer
    // masses, so some sub-bin holds it; should none, the select below
    // decides from the whole list)
    if (star >= 0 && ns <= WX_RANK) {
      if (tid < ns) {
        const uint64_t myc = lc[tid], myw = lw[tid];
        uint64_t incl = 0;
        for (int k = 0; k < ns; ++k) incl += lc[k] >= myc ? lw[k] : 0;
        if (incl - myw < t2 && t2 <= incl) esm.bcast64[0] = myc;
      }
      __syncthreads();
      cstar = esm.bcast64[0];
    } else {
      float* lvs = (float*)dyn;
      int* lis = (int*)(dyn + WX_CAP * sizeof(float));
      __syncthreads();
      for (int j = tid; j < n; j += blockDim.x) {
        lvs[j] = P.list_v[(size_t)b * WX_CAP + j];
        lis[j] = P.list_i[(size_t)b * WX_CAP + j];
      }
      __syncthreads();
      const Pred all = {0, 0, 0, 0, 0, 0, 0.0f, -INFINITY};
      auto mass = [m](int, float l) { return exp_fix44(l - m); };
      cstar = radix_select<ORD_P, true>(CandSource{lvs, lis, n}, all, mass, target, esm);
    }
  }
  if (tid == 0) {
    rec->cstar = cstar;
    rec->flags = 0;
    P.path[b] = WX_PATH;
  }
}

__device__ __forceinline__ bool wx_keep(const WxRow& rp, const WxRec& r, int i, float l) {
  return !rp.use_p || comp_p(fkey(l), i) >= r.cstar;
}

template <int E, bool VEC>
__global__ void __launch_bounds__(WX_T) wx_drawsum_kernel(SampleKArgs a, WxPtrs P) {
  extern __shared__ __align__(16) char dyn[];
  __shared__ float sf[16];
  __shared__ uint64_t s64[16];
  __shared__ int si[16];
  const int b = blockIdx.y, g = blockIdx.x, tid = threadIdx.x;
  const WxRow rp = wx_row(a, b);
  if (rp.greedy) return;
  const int lo = g * P.SL, hi = min(a.V, lo + P.SL);
  RowCtx rc;
  float v[E];
  wx_ptrs(a, b, rc);
  // the record and this slice's max first, then the logits: loads complete
  // in order, so the test below waits for the first two alone
  const WxRec r = P.rec[b];
  float smax;
  if (P.part_key) {
    const uint64_t k = P.part_key[(size_t)b * P.G + g];
    smax = k ? key_to_float((uint32_t)(k >> 32)) : -INFINITY;
  } else {
    smax = P.part_m[(size_t)b * P.G + g];
  }
  asm volatile("" ::: "memory");
  wx_raw<E, VEC>(rc, lo, hi, v);  // in flight with the maxima
  if (r.flags & WX_DONE) return;
  float* out = (a.out_rows && a.out_mode == WH_OUT_MASKED) ? a.out_rows + (long long)b * a.V : nullptr;
  // a slice whose largest (effective) value lies below the cut's value keeps
  // nothing: every composite there is below cstar.  On peaked rows that is
  // all slices but the nucleus's, whose passes this skips (not when the
  // masked row is written: its -inf entries are this pass's).
  if (rp.use_p && !out && fkey(smax + 0.0f) < (uint32_t)(r.cstar >> 18)) {
    if (tid == 0) {
      P.part_vw[(size_t)b * P.G + g] = 0;
      P.part_n[(size_t)b * P.G + g] = 0;
    }
    return;
  }
  const float m = wx_row_max(P, b, sf);
  wx_pen_table(a, b, lo, hi, dyn, rc);
  wx_pen<E, VEC>(rc, lo, hi, v);
  uint64_t s = 0;
  int cnt = 0;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const int i = wx_id<VEC>(lo, j);
    if (i >= hi) break;
    const bool k = wx_keep(rp, r, i, v[j]);
    if (k) {
      ++cnt;
      s += exp_fix44(chain_scale(a.chain, v[j] - m, rp.invT, rp.rTc));
    }
    if (out) out[i] = k ? v[j] : -INFINITY;
  }
  s = block_reduce(s, s64, OpSumU64(), (uint64_t)0);
  cnt = block_reduce(cnt, si, OpSumI(), 0);
  if (tid == 0) {
    P.part_vw[(size_t)b * P.G + g] = s;
    P.part_n[(size_t)b * P.G + g] = cnt;
  }
}

template <int E, bool VEC>
__global__ void __launch_bounds__(WX_T) wx_pick_kernel(SampleKArgs a, WxPtrs P) {
  extern __shared__ __align__(16) char dyn[];
  __shared__ float sf[16];
  __shared__ uint64_t s64[16];
  __shared__ int si[16];
  __shared__ uint64_t pick[2];
  const int b = blockIdx.x, tid = threadIdx.x;
  const WxRow rp = wx_row(a, b);
  if (rp.greedy) return;
  WxRec* rec = P.rec + b;
  // slice sums, one per thread (G <= 256), scanned in slice (= id) order;
  // loaded with the record
  const uint64_t w = tid < P.G ? P.part_vw[(size_t)b * P.G + tid] : 0;
  const int nk = tid < P.G ? P.part_n[(size_t)b * P.G + tid] : 0;
  const WxRec r = *rec;
  if (r.flags & WX_DONE) return;
  const float m = wx_row_max(P, b, sf);
  uint64_t ZV;
  const uint64_t excl = block_exclusive_scan_u64(w, s64, &ZV);
  const int nkept = block_reduce(nk, si, OpSumI(), 0);
  const bool draw = a.tokens && ZV;  // the uniforms exist only when a token is drawn
  const uint64_t tgt = draw ? draw_target(a.u[b], ZV) : 0;
  if (tid == 0) {
    rec->ZV = ZV;
    if (a.kept) a.kept[b] = nkept;
    if (a.tokens && !ZV) a.tokens[b] = 0;
  }
  if (draw && excl <= tgt && tgt < excl + w) {
    pick[0] = (uint64_t)tid;
    pick[1] = tgt - excl;
  }
  __syncthreads();
  if (!draw) return;
  const int g = (int)pick[0];
  const uint64_t t2 = pick[1];
  const int lo = g * P.SL, hi = min(a.V, lo + P.SL);
  RowCtx rc;
  wx_ptrs(a, b, rc);
  // E consecutive ids per thread, so the block scan runs in id order
  const int s0 = lo + tid * E;
  float v[E];
  wx_raw_run<E, VEC>(rc, s0, hi, v);
  wx_pen_table(a, b, lo, hi, dyn, rc);
#pragma unroll
  for (int j = 0; j < E; ++j) v[j] = s0 + j < hi ? rc.val_from(s0 + j, v[j]) : 0.0f;
  uint64_t wt[E];
  uint64_t s = 0;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    wt[j] = (s0 + j < hi && wx_keep(rp, r, s0 + j, v[j])) ? exp_fix44(chain_scale(a.chain, v[j] - m, rp.invT, rp.rTc))
                                                         : 0;
    s += wt[j];
  }
  uint64_t tot;
  const uint64_t ex = block_exclusive_scan_u64(s, s64, &tot);
  if (ex <= t2 && t2 < ex + s) {
    uint64_t c = ex;
#pragma unroll
    for (int j = 0; j < E; ++j) {
      c += wt[j];
      if (wt[j] && c > t2) {
        a.tokens[b] = s0 + j;
        break;
      }
    }
  }
}

template <int E, bool VEC>
__global__ void __launch_bounds__(WX_T) wx_rows_kernel(SampleKArgs a, WxPtrs P) {
  extern __shared__ __align__(16) char dyn[];
  __shared__ float sf[16];
  const int b = blockIdx.y, g = blockIdx.x, tid = threadIdx.x;
  const WxRow rp = wx_row(a, b);
  if (rp.greedy) return;
  const int lo = g * P.SL, hi = min(a.V, lo + P.SL);
  RowCtx rc;
  float v[E];
  wx_ptrs(a, b, rc);
  wx_raw<E, VEC>(rc, lo, hi, v);
  const WxRec r = P.rec[b];
  if (r.flags & WX_DONE) return;
  const float m = wx_row_max(P, b, sf);
  wx_pen_table(a, b, lo, hi, dyn, rc);
  wx_pen<E, VEC>(rc, lo, hi, v);
  const double lz = log(ldexp((double)r.ZV, -44));
  float* out = a.out_rows + (long long)b * a.V;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const int i = wx_id<VEC>(lo, j);
    if (i >= hi) break;
    out[i] = wx_keep(rp, r, i, v[j]) ? (float)((double)chain_scale(a.chain, v[j] - m, rp.invT, rp.rTc) - lz)
                                     : -INFINITY;
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
static int wx_entries(int B) { return B <= 8 ? 4 : 16; }
static int wx_slices(int V, int E) { return (V + WX_T * E - 1) / (WX_T * E); }

struct WxLayout {
  size_t path, part_m, part_i, part_vw, part_n, hist_w, list_v, list_i, lcnt, rec, part_key, total;
};

// Sized for the most slices any batch size uses (1024-entry slices).
static WxLayout wx_layout(int B, int V) {
  const size_t G = wx_slices(V, 4), Bz = (size_t)std::max(B, 1);
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  WxLayout l;
  size_t o = 0;
  l.path = o;    o = al(o + Bz * 4);
  l.part_m = o;  o = al(o + Bz * G * 4);
  l.part_i = o;  o = al(o + Bz * G * 4);
  l.part_vw = o; o = al(o + Bz * G * 8);
  l.part_n = o;  o = al(o + Bz * G * 4);
  l.hist_w = o;  o = al(o + Bz * WX_BINS * 8);
  l.list_v = o;  o = al(o + Bz * WX_CAP * 4);
  l.list_i = o;  o = al(o + Bz * WX_CAP * 4);
  l.lcnt = o;    o = al(o + Bz * 4);
  l.rec = o;     o = al(o + Bz * sizeof(WxRec));
  l.part_key = o; o = al(o + Bz * G * 8);
  l.total = o;
  return l;
}

size_t wide_workspace_bytes(int B, int V) { return wx_layout(B, V).total; }

// Rows the wide engine takes: no top-k and no min-p anywhere (top-p alone, or
// nothing), unless every row is greedy (the fast engine's greedy path).
bool wide_applicable(const SampleKArgs& k) {
  if (k.top_k_rows || k.min_p_rows) return false;
  if (k.top_k > 0 && k.top_k < k.V) return false;
  if (k.min_p != 0.0) return false;
  if (!k.T_rows && !(k.T > 0.0)) return false;
  return true;
}

static int wx_lds(const void* fn, size_t lds) {
  if (lds <= 65536) return WH_OK;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return fail(WH_EHIP, "hipFuncSetAttribute(%zu bytes LDS) failed: %s", lds, hipGetErrorString(e));
  return WH_OK;
}

template <int E, bool VEC>
static int wx_launch(const SampleKArgs& k, WxPtrs P, hipStream_t st, bool from_keys) {
  const bool any_p = k.top_p_rows || (k.top_p > 0.0 && k.top_p < 1.0);
  // slice workgroups: the penalty table of one slice's id range
  const size_t lds_s = k.hcap > 0 ? (size_t)k.hcap * 12 + (size_t)(WX_T * E / 32) * 4 : 0;
  const size_t lds_h = k.hcap > 0 ? (size_t)k.hcap * 12 + (size_t)(WX_T * E * WX_HS / 32) * 4 : 0;
  const size_t lds_r = std::max({penalty_lds_bytes(k), (size_t)WX_CAP * 8, (size_t)WX_RANK * 16});
  int rc;
  if ((rc = wx_lds((const void*)wx_max_kernel<E, VEC>, lds_s)) || (rc = wx_lds((const void*)wx_hist_kernel<E, VEC>, lds_h)) ||
      (rc = wx_lds((const void*)wx_collect_kernel<E, VEC>, lds_s)) || (rc = wx_lds((const void*)wx_resolve_kernel, lds_r)) ||
      (rc = wx_lds((const void*)wx_drawsum_kernel<E, VEC>, lds_s)) || (rc = wx_lds((const void*)wx_pick_kernel<E, VEC>, lds_s)) ||
      (rc = wx_lds((const void*)wx_rows_kernel<E, VEC>, lds_s)))
    return rc;
  const dim3 gs(P.G, k.B);
  if (!from_keys) hipLaunchKernelGGL((wx_max_kernel<E, VEC>), gs, dim3(WX_T), lds_s, st, k, P);
  if (any_p) {
    hipLaunchKernelGGL((wx_hist_kernel<E, VEC>), dim3((P.G + WX_HS - 1) / WX_HS, k.B), dim3(WX_T * WX_HS), lds_h, st,
                       k, P);
    hipLaunchKernelGGL((wx_collect_kernel<E, VEC>), gs, dim3(WX_T), lds_s, st, k, P);
  }
  // the resolve step settles rows with top-p and greedy rows; without
  // either (a scalar temperature above 0 and no top-p) the max step's
  // records stand
  if (any_p || k.T_rows) hipLaunchKernelGGL(wx_resolve_kernel, dim3(k.B), dim3(1024), lds_r, st, k, P);
  hipLaunchKernelGGL((wx_drawsum_kernel<E, VEC>), gs, dim3(WX_T), lds_s, st, k, P);
  hipLaunchKernelGGL((wx_pick_kernel<E, VEC>), dim3(k.B), dim3(WX_T), lds_s, st, k, P);
  if (k.out_rows && k.out_mode == WH_OUT_LOGPROBS)
    hipLaunchKernelGGL((wx_rows_kernel<E, VEC>), gs, dim3(WX_T), lds_s, st, k, P);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "wide engine launch failed: %s", hipGetErrorString(e));
  return WH_OK;
}

static WxPtrs wx_ptrs_of(const SampleKArgs& k, void* workspace) {
  const WxLayout L = wx_layout(k.B, k.V);
  char* ws = (char*)workspace;
  const int E = wx_entries(k.B);
  WxPtrs P;
  P.SL = WX_T * E;
  P.G = wx_slices(k.V, E);
  P.path = (int*)(ws + L.path);
  P.part_m = (float*)(ws + L.part_m);
  P.part_i = (int*)(ws + L.part_i);
  P.part_vw = (uint64_t*)(ws + L.part_vw);
  P.part_n = (int*)(ws + L.part_n);
  P.hist_w = (uint64_t*)(ws + L.hist_w);
  P.list_v = (float*)(ws + L.list_v);
  P.list_i = (int*)(ws + L.list_i);
  P.lcnt = (int*)(ws + L.lcnt);
  P.rec = (WxRec*)(ws + L.rec);
  P.part_key = nullptr;
  return P;
}

// Rows the vector layout can read: V a multiple of 4 (a run of four ids lies
// wholly inside or outside every slice), the logits and the row stride
// aligned to one run (8 bytes in bfloat16, 16 in float32).
static bool wx_vec(const SampleKArgs& k) {
  const size_t esz = k.dtype == WH_DTYPE_BF16 ? 2 : 4;
  return k.V % 4 == 0 && (uintptr_t)k.logits % (4 * esz) == 0 && ((size_t)k.row_stride * esz) % (4 * esz) == 0;
}

static int wx_dispatch(const SampleKArgs& k, WxPtrs P, hipStream_t st, bool from_keys) {
  const bool vec = wx_vec(k);
  if (P.SL == WX_T * 4)
    return vec ? wx_launch<4, true>(k, P, st, from_keys) : wx_launch<4, false>(k, P, st, from_keys);
  return vec ? wx_launch<16, true>(k, P, st, from_keys) : wx_launch<16, false>(k, P, st, from_keys);
}

int launch_sample_wide(const SampleKArgs& k, const wh_sample_args* p, hipStream_t st) {
  WxPtrs P = wx_ptrs_of(k, p->workspace);
  if (P.G > WX_MAXG) return fail(WH_ELIMIT, "too many slices for the wide engine");
  return wx_dispatch(k, P, st, false);
}

// The wide engine after an LM head that writes the slice maxima: the keys'
// array, slice count and length for the head, cleared on the stream first.
int wide_keys_prepare(const SampleKArgs& k, void* workspace, hipStream_t st, uint64_t** keys, int* G, int* SL) {
  WxPtrs P = wx_ptrs_of(k, workspace);
  if (P.G > WX_MAXG) return fail(WH_ELIMIT, "too many slices for the wide engine");
  P.part_key = (uint64_t*)((char*)workspace + wx_layout(k.B, k.V).part_key);
  const size_t n = std::max((size_t)k.B * WX_BINS, (size_t)k.B * P.G);
  hipLaunchKernelGGL(wx_init_kernel, dim3((unsigned)((n + WX_T - 1) / WX_T)), dim3(WX_T), 0, st, P, k.B);
  *keys = P.part_key;
  *G = P.G;
  *SL = P.SL;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "wide engine launch failed: %s", hipGetErrorString(e));
  return WH_OK;
}

int launch_sample_wide_from_keys(const SampleKArgs& k, const wh_sample_args* p, hipStream_t st) {
  WxPtrs P = wx_ptrs_of(k, p->workspace);
  P.part_key = (uint64_t*)((char*)p->workspace + wx_layout(k.B, k.V).part_key);
  return wx_dispatch(k, P, st, true);
}

}  // namespace wh
