// wh_fast.hip -- the sliced single-read sampler engine for gfx950.
//
// Two kernels per call and no synchronisation between workgroups.  On this
// part a kernel boundary costs about 2 us, while an agent-scope fence with a
// last-block merge costs 6-25 us, so the merge is a second kernel.
//
// slice_kernel: row b is cut into G slices.  One 1024-thread workgroup per
// slice reads its slice from HBM exactly once: 16-byte loads, all issued up
// front, held in VGPRs.  It reduces the slice to a 64-byte summary plus a
// short candidate list.  Every VALU op per element costs about a quarter of
// a microsecond over a full batch, so the per-element work is only the
// unpack and a max.  The rest is done per 16-byte group or per rare element:
//   * Penalties, worked from the history side (a few hundred ids per slice)
//     rather than the element side: sparse penalised elements spread over
//     every wave would make each wave run the penalty code.  The window
//     becomes a dense u16 code per slice element in LDS (count in the
//     frequency window, flags for the repetition and presence windows).  The
//     first thread to touch an element's code computes its penalised value
//     from a gathered raw logit and lists it.  The registers holding the
//     element turn it into a NaN with one OR per 4-byte word.
//   * The slice max m_s and the max of every 16-byte group.
//   * The candidate threshold tau_s.  No kept element of the row can fall
//     below it:
//       - min-p: fl(m_s + ln min_p);
//       - top-k: a threshold with at least k slice elements at or above it,
//         found by counting group maxima against a ladder of thresholds below
//         m_s;
//       - top-p alone: the lowest ladder rung whose count fits the buffer.
//   * The candidates, all elements >= tau_s.  They are appended from the rare
//     groups whose max reaches tau_s.
//   * Two band counts of groups whose max lies 1.5 / 3.5 nats below tau_s.
//     They give a lower bound on the normaliser's mass outside the
//     candidates.
//   * When the top-p cut needs the normaliser closely, a hardware-exp float
//     sum over the slice.
//
// merge_kernel: one workgroup per row.  Each of its eight waves loads the G
// summaries and QW of the row's first QSPEC 64-candidate chunks (chunk t / G
// of slice t % G) in one round trip, computes their exact masses and appends
// the candidates that can still be kept to one LDS list.  Wave 0 then keeps
// up to 16 of them per lane in registers and runs the integer contract:
//   * the proven interval [Zlo, Zhi] for the normaliser;
//   * top-k / top-p / min-p in the chain's order;
//   * the inverse-CDF draw, a 6-bit radix descent over the id.
// Cut points are found by bitwise searches over value/id composites, with
// ballot counts and DPP sums.  Larger candidate sets go through LDS with a
// radix select.  The exact engine finishes a row the candidates cannot
// settle: a buffer overflow, a top-p cut inside the uncertainty of Z, or no
// usable bound.  It uses the whole workgroup, and the results are identical,
// only slower.
#include "wh_rowops.h"

namespace wh {

constexpr int FT = 1024;          // slice-kernel threads per workgroup (four waves per SIMD)
constexpr int FNW = FT / 64;      // waves per slice workgroup
constexpr int FAST_NE = 48;       // logits per thread held in VGPRs, at most
constexpr int GPREF = 4;          // slices per row preferred for small batches
constexpr int GMAX = 6;           // slices per row the merge is compiled for
constexpr int FAST_CAP = 2048;    // candidate capacity per slice
constexpr int RUNGS = 8;          // thresholds per ladder round
constexpr int LADDER_ROUNDS = 2;  // ladder rounds at most (the first, then a far one or the top-p refinement)
constexpr int HB_BINS = 1024;     // top-k refinement: histogram bins over the ladder's bracket
constexpr int QM = 16;            // merge: candidate slots per lane, at most
constexpr int MW = 8;             // merge: waves per workgroup
constexpr int QW = 2;             // merge: candidate chunks each wave loads with the summaries
constexpr int QSPEC = MW * QW;    // merge: chunks loaded speculatively per row
constexpr int HDR_OVERFLOW = 1;   // SliceHdr.flags: the row needs the exact engine
constexpr float BAND1 = 1.5f;     // band floors below tau, nats
constexpr float BAND2 = 3.5f;

struct SliceHdr {
  float m;        // slice max (penalised)
  float tau;      // every slice element >= tau is a candidate
  int n;          // candidates written
  int flags;      // HDR_OVERFLOW: overflow or no usable bound (exact engine)
  float t1, t2;   // band floors t1 = tau - 1.5, t2 = tau - 3.5
  int g1, g2;     // groups (or penalised elements) whose max lies in [t1, tau) / [t2, t1)
  int nall;       // elements in the slice
  int best_i;     // greedy rows: lowest index attaining the max
  double zf;      // sum of exp(l - m) over the slice (hardware exp); < 0 when not computed
  int pad[4];
};
static_assert(sizeof(SliceHdr) == 64, "SliceHdr layout");

struct FastPlan {
  int G;           // slices per row
  int SL;          // slice length (a multiple of the elements per 16-byte load)
  int cap;         // candidate capacity per slice
  int rule_cap;    // largest k a slice may bound
  int pcap;        // capacity of the penalised-element list (with penalties)
  int codes_bytes; // LDS bytes of the penalty codes (0 without penalties)
  int zpass;       // the merge may take a row's float sum when its bounds leave a top-p cut open:
                   // bit 0 for the register merge, bit 1 for the block merge (LDS permitting)
  int* path;       // [B] 0: merged in registers, 4: merged through LDS, 1: exact engine
                   //     (overflow / no bound), 2: greedy, 3: exact engine (top-p cut unsettled),
                   //     7 / 8: merged in registers / through LDS after the row's float sum
  SliceHdr* hdr;   // [B * G]
  int2* cand;      // [B * G * cap] (value bits, id), in no particular order
};

struct RowParams {
  float theta;   // fl32(1 - top_p): the top-p threshold as MLX forms it from a double
  float cmin;    // fl32(ln min_p)
  float invT;    // fl32(1 / T): chain MLX scales the logprobs by it
  double rTc;    // 1 / fl32(max(T, 1e-5)): chain WHALLM divides by fl32(max(T, 1e-5))
  int top_k;
  bool use_k, use_p, use_m;
  bool greedy;
  bool tscale;   // T != 1: the draw weights differ from the masses
  bool tk;   // tau from the slice's k-th value
  bool tm;   // tau from min-p
  bool tp;   // tau from the candidate capacity (top-p is the only filter that bounds)
  bool all;  // nothing bounds the kept set: exact engine
};

// Both kernels take first the scalars and pointers their first loads need
// (leading scalar arguments are preloaded into SGPRs at wave launch, so
// those loads wait for no argument fetch), then (SampleKArgs, FastPlan).
// The structures mirror the argument segments.  Reading fields in place (a
// pointer, not a copy) keeps out-of-line callees and per-row parameter loads
// from forcing the arguments into private memory.
struct SliceKernArgs {
  const char* logits;
  const int32_t* hist;
  long long row_stride;  // elements
  int G, SL, V, hs;      // hs: history row stride
  int pen;               // penalties on
  int hshare;            // logits rows per history row
  SampleKArgs a;
  FastPlan p;
};
struct MergeKernArgs {
  const SliceHdr* hdr;
  const int2* cand;
  SampleKArgs a;
  FastPlan p;
};
static_assert(offsetof(SliceKernArgs, a) == 48, "slice kernel argument layout");
static_assert(offsetof(MergeKernArgs, a) == 16, "merge kernel argument layout");
__device__ __forceinline__ const SliceKernArgs* slice_kernargs() {
  return (const SliceKernArgs*)__builtin_amdgcn_kernarg_segment_ptr();
}
__device__ __forceinline__ const MergeKernArgs* merge_kernargs() {
  return (const MergeKernArgs*)__builtin_amdgcn_kernarg_segment_ptr();
}

// Which bounds the slices may use.  Chain MLX with top-k and top-p computes
// the top-p mass over the exact top-k set, so there the candidates must hold
// the whole top-k set and min-p may not raise the threshold.
// The row's raw parameters: one unconditional load each, from the per-row
// array or the scalar field (no branch join that waits for the load).
struct RowRaw {
  double T, top_p, min_p;
  int top_k;
};
// The loads go through the constant address space: the addresses are
// uniform and the data is read-only for the kernel's lifetime, so they are
// scalar loads, counted apart from the vector loads of the logits.
typedef __attribute__((address_space(4))) const double cdouble;
typedef __attribute__((address_space(4))) const int cint;
// ka is the kernel's own argument copy (in its argument segment).
__device__ __forceinline__ RowRaw row_raw(const SampleKArgs& a, const SampleKArgs& ka, int b) {
  RowRaw r;
  r.T = *(cdouble*)(a.T_rows ? a.T_rows + b : &ka.T);
  r.top_p = *(cdouble*)(a.top_p_rows ? a.top_p_rows + b : &ka.top_p);
  r.min_p = *(cdouble*)(a.min_p_rows ? a.min_p_rows + b : &ka.min_p);
  r.top_k = *(cint*)(a.top_k_rows ? a.top_k_rows + b : &ka.top_k);
  return r;
}
// The float32 constants of the filters, derived from the caller's doubles
// the way MLX derives them from Python floats (the scalar is rounded to the
// array's float32 type after the double arithmetic).  Unused ones are dead
// code in the kernels that do not need them.
__device__ __forceinline__ RowParams row_params(const SampleKArgs& a, const RowRaw& raw, int rule_cap) {
  RowParams r;
  r.top_k = raw.top_k;
  r.theta = (float)(1.0 - raw.top_p);
  r.cmin = a.min_p_rows ? (float)log(raw.min_p) : a.min_p_log;
  r.invT = (float)(1.0 / raw.T);
  r.rTc = 1.0 / (double)(float)fmax(raw.T, 1e-5);
  r.tscale = raw.T != 1.0;
  r.use_k = r.top_k > 0 && r.top_k < a.V;
  r.use_p = raw.top_p > 0.0 && raw.top_p < 1.0;
  r.use_m = raw.min_p != 0.0;
  r.greedy = !(raw.T > 0.0);
  const bool bk = r.use_k && r.top_k <= rule_cap;
  r.tk = r.tm = r.tp = false;
  if (!r.greedy) {
    if (a.chain == WH_CHAIN_MLX && r.use_k && r.use_p) {
      r.tk = bk;
    } else {
      r.tk = bk;
      r.tm = r.use_m;
      r.tp = !r.tk && !r.tm && r.use_p;
    }
  }
  r.all = !r.greedy && !r.tk && !r.tm && !r.tp;
  return r;
}


// Element e of a 16-byte group (DT 0: 4 x float32, DT 1: 8 x bfloat16).
__device__ __forceinline__ uint32_t comp(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}
template <int DT>
__device__ __forceinline__ float elem(const uint4& v, int e) {
  if (DT == 0) return __uint_as_float(comp(v, e));
  const uint32_t x = comp(v, e >> 1);
  return __uint_as_float((e & 1) ? (x & 0xFFFF0000u) : (x << 16));
}
// The element with -0 mapped to +0 (the value every order and key sees).
template <int DT>
__device__ __forceinline__ float elem_n(const uint4& v, int e) {
  return elem<DT>(v, e) + 0.0f;
}
template <int DT>
__device__ __forceinline__ float grp_max(const uint4& v) {
  if (DT == 0) {
    const float a = max3_raw(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z));
    return max3_raw(a, __uint_as_float(v.w), __uint_as_float(v.w));
  }
  float m = max3_raw(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xFFFF0000u), __uint_as_float(v.y << 16));
  m = max3_raw(m, __uint_as_float(v.y & 0xFFFF0000u), __uint_as_float(v.z << 16));
  m = max3_raw(m, __uint_as_float(v.z & 0xFFFF0000u), __uint_as_float(v.w << 16));
  return max3_raw(m, __uint_as_float(v.w & 0xFFFF0000u), __uint_as_float(v.w & 0xFFFF0000u));
}
// Penalty code bits: count in the frequency window (bits 0-12, at most 4096),
// in the repetition window (bit 13), in the presence window (bit 14).  A flag
// whose window equals the frequency window is read from the count instead.
constexpr uint32_t PEN_CNT = 0x1FFFu, PEN_R = 0x2000u, PEN_P = 0x4000u;

struct PenCtx {
  bool on_r, on_p, on_f, dr, dp;
  float rep, pres, freq;
  __device__ __forceinline__ float apply(float v, uint32_t code) const {
    const int c = (int)(code & PEN_CNT);
    const bool in_r = dr ? c > 0 : (code & PEN_R) != 0;
    const bool in_p = dp ? c > 0 : (code & PEN_P) != 0;
    if (on_r && in_r) v = v < 0.0f ? v * rep : v / rep;
    if (on_p && in_p) v = v - pres;
    if (on_f && c > 0) v = v - freq * (float)c;
    return v + 0.0f;
  }
};

struct SliceSmem {
  int cnt;                      // candidates appended
  int npatch;                   // penalised bf16 elements listed
  float redm[FNW];
  int redg[FNW];
  int lad[LADDER_ROUNDS][RUNGS];  // ladder totals per round (zeroed at kernel start)
  int hb[HB_BINS];                // top-k refinement histogram (zeroed at kernel start)
  int hwave[FNW];                 // its per-wave totals
  int hsel[2];                    // the chosen bins (two uses), -1 if none reaches k
  int redb[FNW][1];
  double redz[FNW];
};

// Ladder counts: for each rung x_j, the groups whose max is >= x_j plus the
// listed penalised elements >= x_j, over the whole slice.  Block-wide: wave
// sums by DPP, then one LDS atomic per wave and rung into round `buf`'s totals.
template <int R>
__device__ __forceinline__ void ladder_count(const float (&gm)[R], const int2* patch, int npatch, const float (&x)[RUNGS],
                                             int (&tot)[RUNGS], int buf, SliceSmem& sm) {
  const int tid = threadIdx.x, lane = tid & 63;
  int c[RUNGS];
#pragma unroll
  for (int j = 0; j < RUNGS; ++j) c[j] = 0;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < RUNGS; ++j) c[j] += gm[r] >= x[j] ? 1 : 0;
  for (int p = tid; p < npatch; p += FT) {
    const float v = __int_as_float(patch[p].x);
#pragma unroll
    for (int j = 0; j < RUNGS; ++j) c[j] += v >= x[j] ? 1 : 0;
  }
  // two rungs per reduction: a wave counts at most 64 * (R + 4) < 2^16
#pragma unroll
  for (int j = 0; j < RUNGS; j += 2) {
    const int w = wsum_i(c[j] | (c[j + 1] << 16));
    if (lane == 0 && w) {
      atomicAdd(&sm.lad[buf][j], w & 0xFFFF);
      atomicAdd(&sm.lad[buf][j + 1], w >> 16);
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < RUNGS; ++j) tot[j] = sm.lad[buf][j];
}

// Top-k cut over an interval: 1024 bins of w = (top - lo) / 1024 over the
// values v in [lo, top) ([lo, top] when incl); bin g takes the values with
// floor(fl(top - v) / w) = g that also reach its lower edge
// e(g) = fl(top - (g + 1) w) (a value the rounding puts one bin too high is
// not counted, which only lowers the counts).  chi values lie above the
// interval.  One LDS atomic per value in it, one block scan over the bins
// (one per thread); the result is the first bin whose cumulative count
// reaches k, or -1.  The edges do not increase with g, so at least k values
// are >= e(g*).  The histogram is left zeroed; `slot` picks the LDS word the
// chosen bin passes through (each use takes its own).
template <int R>
__device__ __forceinline__ int hist_cut(const float (&gm)[R], const int2* patch, int npatch, float lo, float top, bool incl,
                                        int chi, int k, int slot, SliceSmem& sm) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const float w = (top - lo) * (1.0f / (float)HB_BINS);
  const float iw = (float)HB_BINS / (top - lo);
  auto add = [&](float v) {
    if ((v < top || (incl && v == top)) && v >= lo) {
      const int g = max(0, min((int)((top - v) * iw), HB_BINS - 1));
      if (v >= top - (float)(g + 1) * w) atomicAdd(&sm.hb[g], 1);
    }
  };
#pragma unroll
  for (int r = 0; r < R; ++r) add(gm[r]);
  for (int p = tid; p < npatch; p += FT) add(__int_as_float(patch[p].x));
  __syncthreads();
  const uint32_t hc = (uint32_t)sm.hb[tid];
  sm.hb[tid] = 0;
  const uint32_t incl_sum = wscan_incl_u32(hc);
  if (lane == 63) sm.hwave[wv] = (int)incl_sum;
  __syncthreads();
  uint32_t before = (uint32_t)chi;
  for (int q = 0; q < wv; ++q) before += (uint32_t)sm.hwave[q];
  const uint32_t cum = before + incl_sum;
  if (cum >= (uint32_t)k && cum - hc < (uint32_t)k) sm.hsel[slot] = tid;
  __syncthreads();
  return sm.hsel[slot];
}

// Width of the interval below the slice max that a small top-k (k <= 64)
// first tries with one histogram, before the ladder.
constexpr float TOPK_NEAR = 8.0f;
constexpr int TOPK_NEAR_K = 64;

// Candidate threshold from the ladder (rungs from the slice max down to 1024
// nats below it) and, for top-k, one histogram over the bracketing interval.
//   k > 0 (top-k bound): a threshold with at least k slice elements at or
//     above it -- the highest rung whose group count reaches k (each counted
//     group holds at least one such element).  When that count exceeds
//     max(1.5 k, 64), the bracket between that rung and the one above it is
//     cut into 1024 bins and the threshold is the edge of the first bin whose
//     cumulative count reaches k.  When no rung reaches k (an outlier far
//     above the rest of the slice), a second round tries 2^11 .. 2^18 below
//     the max; -inf when that fails too.
//   k <= 0 (top-p alone): the lowest rung whose group count is at most half
//     the buffer, refined once towards the next rung.
template <int R>
__device__ __forceinline__ float ladder_tau(const float (&gm)[R], const int2* patch, int npatch, float ms, int k, int cap,
                                            SliceSmem& sm) {
  // Every rung array is indexed with compile-time indices only (unrolled
  // loops with selects), so it stays in registers.
  const float D0[RUNGS] = {0.0f, 0.5f, 1.0f, 2.0f, 4.0f, 16.0f, 128.0f, 1024.0f};
  const int half = cap / 2;
  if (k > 0 && k <= TOPK_NEAR_K) {
    // a small k is usually reached within a few nats of the max: one
    // histogram over [ms - 8, ms] settles it without the ladder
    const float lo = ms - TOPK_NEAR;
    if (lo < ms) {
      const int g = hist_cut<R>(gm, patch, npatch, lo, ms, true, 0, k, 0, sm);
      if (g >= 0) return ms - (float)(g + 1) * ((ms - lo) * (1.0f / (float)HB_BINS));
    }
  }
  float x[RUNGS];
  int c[RUNGS];
#pragma unroll
  for (int j = 0; j < RUNGS; ++j) x[j] = ms - D0[j];
  ladder_count<R>(gm, patch, npatch, x, c, 0, sm);
  if (k > 0) {
    // counts grow with j: hi = last rung with count < k, lo = first with >= k
    const int target = max(k + k / 2, 64);
    bool found = false;
    float lo = -INFINITY, hi = INFINITY;
    int clo = 0;
#pragma unroll
    for (int j = 0; j < RUNGS; ++j) {
      if (!found && c[j] >= k) {
        found = true;
        lo = x[j];
        clo = c[j];
      }
      if (!found) hi = x[j];
    }
    if (!found) {
      // fewer than k groups within 1024 of the max (an outlier far above the
      // rest): rungs 2^11 .. 2^18 below it
#pragma unroll
      for (int j = 0; j < RUNGS; ++j) x[j] = ms - (float)(2048 << j);
      ladder_count<R>(gm, patch, npatch, x, c, 1, sm);
#pragma unroll
      for (int j = 0; j < RUNGS; ++j) {
        if (!found && c[j] >= k) {
          found = true;
          lo = x[j];
          clo = c[j];
        }
        if (!found) hi = x[j];
      }
      if (!found) return -INFINITY;
    }
    if (clo > target && hi != INFINITY) {
      // one histogram over the bracket [lo, hi); the counts above hi are
      // known (fewer than k), and lo stands if no bin reaches k
      int chi = 0;
#pragma unroll
      for (int j = 0; j < RUNGS; ++j)
        if (x[j] == hi) chi = c[j];
      const int g = hist_cut<R>(gm, patch, npatch, lo, hi, false, chi, k, 1, sm);
      if (g >= 0) lo = hi - (float)(g + 1) * ((hi - lo) * (1.0f / (float)HB_BINS));
      return lo;
    }
    return lo;
  }
  // counts grow with j: the lowest rung with count <= half, then one refinement
  // towards the next rung down
  bool any = false;
  float sel = ms, nxt = ms;
#pragma unroll
  for (int j = 0; j < RUNGS; ++j) {
    if (c[j] <= half) {
      any = true;
      sel = x[j];
      nxt = j + 1 < RUNGS ? x[j + 1] : x[j];
    }
  }
  if (!any) return ms;
  if (nxt == sel) return sel;
  const float span = sel - nxt;
#pragma unroll
  for (int q = 0; q < RUNGS; ++q) x[q] = sel - span * ((float)(q + 1) / (float)(RUNGS + 1));
  ladder_count<R>(gm, patch, npatch, x, c, 1, sm);
  float best = sel;
#pragma unroll
  for (int q = 0; q < RUNGS; ++q)
    if (c[q] <= half) best = x[q];
  return best;
}

template <int DT, int R, bool XM>
__global__ void __launch_bounds__(FT) slice_kernel(const char* __restrict__ logits, const int32_t* __restrict__ hist,
                                                   long long row_stride, int G, int SL, int V, int hs, int pen,
                                                   int hshare,
                                                   SampleKArgs a, FastPlan P) {
  extern __shared__ __align__(16) char dyn[];
  __shared__ SliceSmem sm;
  constexpr int EPT = DT ? 8 : 4;
  constexpr int ESZ = DT ? 2 : 4;
  constexpr uint32_t NEG = DT ? 0xFF80FF80u : 0xFF800000u;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  // Workgroups go to the 8 XCDs in turn, in linear order (x fastest): the
  // workgroup at (x, y) to XCD (x + y gridDim.x) % 8.  XM (B a multiple of
  // 8): the grid is (8 G, B / 8) and (x, y) takes slice x / 8 of row
  // 8 y + x % 8, so a row's G slices share one XCD's L2, which fetches the
  // row's history and parameters from HBM once, and the merge's workgroup b
  // runs on XCD b % 8 as well (B = 64, V = 151,936 bf16 with 2,048-id
  // histories: -0.3 us per call; B = 128 with 4,096-id histories: -1.1 us;
  // B = 256, V = 129,280 f32: -0.4 us).  Otherwise the grid is (G, B), a
  // row's slices spread over the XCDs (a row count read in the kernel, to
  // bound the mapped rows, had cost B = 1 0.2-0.5 us).
  const int b = XM ? 8 * (int)blockIdx.y + ((int)blockIdx.x & 7) : (int)blockIdx.y;
  const int s = XM ? (int)blockIdx.x >> 3 : (int)blockIdx.x;
  const int v0 = s * SL, v1 = min(V, v0 + SL);

  // 1. loads, in the order they are needed: the history window (up to 4 ids
  //    per thread) and its length, then the slice straight into registers
  //    (padding groups read as -inf), then the row's parameters (scalar).
  //    Their addresses come from the preloaded leading arguments.  Vector
  //    loads complete in order, so waiting for the history leaves the logits
  //    in flight; the compiler barrier keeps every load issued before the
  //    first wait.
  constexpr int HPF = WH_MAX_WINDOW / FT;  // history positions per thread
  const bool pf = hs <= HPF * FT;  // the whole history row fits the prefetch
  int hreg[HPF];
  int len = 0, jbase = 0;
#pragma unroll
  for (int q = 0; q < HPF; ++q) hreg[q] = -1;
  // Every vector load is unconditional, from a clamped in-bounds address, so
  // the number of loads in flight is the same on every path and each wait is
  // for exactly the loads it needs.
  const int32_t* hrow = hist + (long long)(b / hshare) * hs;
  if (pen) {
    if (pf) {
      // the addresses do not need the length, which is read after the
      // logits loads have issued
#pragma unroll
      for (int q = 0; q < HPF; ++q)
        if (q * FT < hs) hreg[q] = hrow[min(tid + q * FT, hs - 1)];
    } else {
      // rows longer than the prefetch read the last HPF * FT positions
      // (every window is a suffix of at most WH_MAX_WINDOW ids)
      len = max(0, min(*(cint*)(a.hist_len + b), hs));
      jbase = max(0, len - HPF * FT);
#pragma unroll
      for (int q = 0; q < HPF; ++q) hreg[q] = hrow[min(jbase + tid + q * FT, hs - 1)];
    }
  }
  const char* rowp = logits + (size_t)b * row_stride * ESZ;
  uint4 d[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int g = v0 + (r * FT + tid) * EPT;
    d[r] = load_stream16(rowp + (size_t)(g < v1 ? g : v0) * ESZ);
  }
  asm volatile("" ::: "memory");
  if (pen && pf) len = max(0, min(*(cint*)(a.hist_len + b), hs));
  const RowRaw raw = row_raw(a, slice_kernargs()->a, b);
  const RowParams rp = row_params(a, raw, P.rule_cap);
  SliceHdr* hdr = P.hdr + (long long)b * G + s;
  if (rp.all) {
    if (tid == 0) hdr->flags = HDR_OVERFLOW;
    return;
  }
  float* out = a.out_rows ? a.out_rows + (long long)b * V : nullptr;
  if (tid < LADDER_ROUNDS * RUNGS) (&sm.lad[0][0])[tid] = 0;
  static_assert(HB_BINS == FT, "one histogram bin per thread");
  sm.hb[tid] = 0;
  if (tid == 0) {
    sm.cnt = 0;
    sm.npatch = 0;
    sm.hsel[0] = -1;
    sm.hsel[1] = -1;
  }

  // 2. penalties, from the history side, and 3. the group maxima.
  //    Each slice element has an element-sized code in LDS (u16 for bf16,
  //    u32 for float32): the count in the frequency window (bits 0-12) and
  //    the repetition / presence flags.  The in-window history ids of this
  //    slice enter it with LDS atomics; the thread whose atomic first touches
  //    an element owns it.  All of this needs only the history, so it runs
  //    while the logits are still in flight.  Owners then keep the final code,
  //    mark the element with all-ones and fetch its logit from memory (a
  //    2- or 4-byte gather that overlaps the groups landing).  As each 16-byte
  //    group lands, its holder ORs the codes into the registers: a penalised
  //    element becomes a NaN there, which every max and >= test ignores.  The
  //    owners apply the penalties to the fetched values and list the
  //    elements, which live on only in the list.
  char* codes = dyn;
  int2* patch = (int2*)(dyn + P.codes_bytes);
  float pmax = -INFINITY;
  PenCtx pc;
  uint32_t own = 0;
  uint32_t ocode[HPF], oraw[HPF];
  if (pen) {
    pc.rep = a.rep;
    pc.pres = a.pres;
    pc.freq = a.freq;
    pc.on_r = a.rep != 0.0f;
    pc.on_p = a.pres != 0.0f;
    pc.on_f = a.freq != 0.0f;
    auto window = [len](int ctx) { return (ctx <= 0 || ctx > len) ? len : ctx; };
    const int wr = pc.on_r ? window(a.rep_ctx) : 0;
    const int wp = pc.on_p ? window(a.pres_ctx) : 0;
    const int wf = pc.on_f ? window(a.freq_ctx) : 0;
    pc.dr = pc.on_r && pc.on_f && wr == wf;
    pc.dp = pc.on_p && pc.on_f && wp == wf;
    const int W = max(wr, max(wp, wf));
    const int words = P.codes_bytes / 16;
    for (int w = tid; w < words; w += FT) ((uint4*)codes)[w] = make_uint4(0u, 0u, 0u, 0u);
    bool inw[HPF];
#pragma unroll
    for (int q = 0; q < HPF; ++q) {
      const int j = jbase + tid + q * FT;
      const int t = hreg[q];
      inw[q] = j >= len - W && j < len && t >= v0 && t < v1;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < HPF; ++q) {
      if (!inw[q]) continue;
      const int j = jbase + tid + q * FT;
      const int ob = (hreg[q] - v0) * ESZ;  // byte offset of the element's code
      uint32_t* word = (uint32_t*)(codes + (ob & ~3));
      const int sh = (ob & 3) * 8;
      const uint32_t add = (pc.on_f && j >= len - wf) ? 1u : 0u;
      const uint32_t fl = ((pc.on_r && !pc.dr && j >= len - wr) ? PEN_R : 0u) | ((pc.on_p && !pc.dp && j >= len - wp) ? PEN_P : 0u);
      // the first read-modify-write of the element's code sees 0 (every
      // update leaves it non-zero): that thread owns the element
      uint32_t old = 0xFFFFFFFFu;
      if (add) old = atomicAdd(word, add << sh);
      if (fl) {
        const uint32_t o2 = atomicOr(word, fl << sh);
        if (!add) old = o2;
      }
      if (((old >> sh) & 0xFFFFu) == 0u) own |= 1u << q;
    }
  }
  // The owners' gathers, issued as soon as ownership is known so that their
  // latency overlaps the two barriers and the group loop below.  They are
  // issued on every path (other lanes, and every lane without penalties,
  // read the slice's first element: one shared line), so the waits for the
  // groups count the same loads on every path and never wait for a gather;
  // the values are first used at the apply.  A bfloat16 owner reads the
  // aligned word holding its element (V is even on this path).
#pragma unroll
  for (int q = 0; q < HPF; ++q) {
    const int t = ((own >> q) & 1u) ? hreg[q] : v0;
    oraw[q] = ((const uint32_t*)rowp)[DT ? (t >> 1) : t];
  }
  if (pen) {
    __syncthreads();
#pragma unroll
    for (int q = 0; q < HPF; ++q) {
      ocode[q] = 0;
      if (!((own >> q) & 1u)) continue;
      const int o = hreg[q] - v0;
      if (DT) {
        ocode[q] = ((uint16_t*)codes)[o];
        ((uint16_t*)codes)[o] = 0xFFFFu;
      } else {
        ocode[q] = ((uint32_t*)codes)[o];
        ((uint32_t*)codes)[o] = 0xFFFFFFFFu;
      }
    }
    __syncthreads();
  }
  // group maxima as the groups land (padding groups, duplicate loads, become
  // -inf); with penalties, the marked elements are swapped out first
  float gm[R];
  float mx = -INFINITY;
  if (pen) {
    // branch-free, so every group's code read issues back to back (a group
    // past the slice reads the first codes and is overwritten below)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int g = v0 + (r * FT + tid) * EPT;
      const uint4 cw = *(const uint4*)(codes + (size_t)(g < v1 ? g - v0 : 0) * ESZ);
      d[r].x |= cw.x;
      d[r].y |= cw.y;
      d[r].z |= cw.z;
      d[r].w |= cw.w;
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int g = v0 + (r * FT + tid) * EPT;
    if (g >= v1) d[r] = make_uint4(NEG, NEG, NEG, NEG);
    gm[r] = grp_max<DT>(d[r]);
    mx = max3_raw(mx, gm[r], gm[r]);
  }
  if (pen) {
#pragma unroll
    for (int q = 0; q < HPF; ++q) {
      if (!((own >> q) & 1u)) continue;
      const int t = hreg[q];
      // the empty asm redefines the gathered bits here, so their first use
      // (and the wait for them) cannot be hoisted above the group loop
      uint32_t raw = oraw[q];
      asm volatile("" : "+v"(raw));
      if (DT) raw = (t & 1) ? (raw & 0xFFFF0000u) : (raw << 16);
      const float v = pc.apply(__uint_as_float(raw) + 0.0f, ocode[q]);
      const int slot = atomicAdd(&sm.npatch, 1);
      if (slot < P.pcap) patch[slot] = make_int2(__float_as_int(v), t);
      pmax = max3_raw(pmax, v, v);
    }
  }
  mx = max3_raw(mx, pmax, pmax);
  mx = wmax_f(mx);
  if (lane == 0) sm.redm[wv] = mx;
  __syncthreads();
  float ms = sm.redm[0];
#pragma unroll
  for (int w = 1; w + 1 < FNW; w += 2) ms = max3_raw(ms, sm.redm[w], sm.redm[w + 1]);
  if (FNW % 2 == 0) ms = max3_raw(ms, sm.redm[FNW - 1], sm.redm[FNW - 1]);
  const int npatch_raw = sm.npatch;
  const int npatch = min(npatch_raw, P.pcap);

  if (rp.greedy) {
    int bi = 0x7FFFFFFF;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int g = v0 + (r * FT + tid) * EPT;
      if (gm[r] == ms && bi == 0x7FFFFFFF) {
#pragma unroll
        for (int e = 0; e < EPT; ++e)
          if (bi == 0x7FFFFFFF && g + e < v1 && elem<DT>(d[r], e) == ms) bi = g + e;
      }
    }
    for (int p = tid; p < npatch; p += FT)
      if (__int_as_float(patch[p].x) == ms) bi = min(bi, patch[p].y);
    bi = wmin_i(bi);
    if (lane == 0) sm.redg[wv] = bi;
    if (out) {  // Whallm's sampling_logprobs returns the (penalised) logits at T == 0
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int g = v0 + (r * FT + tid) * EPT;
        if (g < v1) {
#pragma unroll
          for (int e = 0; e < EPT; ++e) out[g + e] = elem_n<DT>(d[r], e);
        }
      }
    }
    __syncthreads();
    if (out)
      for (int p = tid; p < npatch; p += FT) out[patch[p].y] = __int_as_float(patch[p].x);
    if (wv == 0) {
      const int best = wmin_i(lane < FNW ? sm.redg[lane & (FNW - 1)] : 0x7FFFFFFF);
      if (lane == 0) {
        hdr->m = ms;
        hdr->best_i = best;
        hdr->flags = npatch_raw > P.pcap ? HDR_OVERFLOW : 0;
        hdr->n = 0;
      }
    }
    return;
  }

  // 4. candidate threshold
  float tau = -INFINITY;
  if (rp.tm) tau = ms + rp.cmin;
  if (rp.tk || rp.tp) {
    const float tl = ladder_tau<R>(gm, patch, npatch, ms, rp.tk ? rp.top_k : 0, P.cap, sm);
    tau = rp.tm ? fmaxf(tau, tl) : tl;
  }
  const float t1 = tau - BAND1, t2 = tau - BAND2;
  const bool need_zf = rp.use_p && !rp.tm;

  // 5. candidates from the groups whose max reaches tau, written straight to
  //    the workspace; group band counts; optional hardware-exp sum
  int2* gc = P.cand + ((long long)b * G + s) * P.cap;
  // groups (and listed penalised elements) at or above tau, t1 and t2; the
  // band counts are the differences (a NaN group max counts nowhere)
  int c0 = 0, c1 = 0, c2 = 0;
  float zs = 0.0f;
  // element masks of the candidate groups, 8 bits per group
  uint32_t mk[(R + 3) / 4];
#pragma unroll
  for (int q = 0; q < (R + 3) / 4; ++q) mk[q] = 0u;
  int tcnt = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float x = gm[r];
    c0 += x >= tau ? 1 : 0;
    c1 += x >= t1 ? 1 : 0;
    c2 += x >= t2 ? 1 : 0;
    const int g = v0 + (r * FT + tid) * EPT;
    const bool cg = x >= tau && g < v1;
    if (__ballot(cg)) {
      // penalised elements are NaN here and fail the test; a group lies
      // wholly inside or outside the slice
      uint32_t msk = 0;
#pragma unroll
      for (int e = 0; e < EPT; ++e) msk |= (elem<DT>(d[r], e) >= tau) ? (1u << e) : 0u;
      msk = cg ? msk : 0u;
      mk[r >> 2] |= msk << (8 * (r & 3));
      tcnt += __popc(msk);
    }
    if (need_zf) {
#pragma unroll
      for (int e = 0; e < EPT; ++e) zs += __expf(fmaxf(elem<DT>(d[r], e), -INFINITY) - ms);  // NaN (penalised) -> 0
    }
  }
  if (__ballot(tcnt > 0)) {
    // The wave reserves its slots with one LDS atomic: an inclusive scan of
    // the per-lane counts gives each lane its offset.
    const uint32_t incl = wscan_incl_u32((uint32_t)tcnt);
    int base = 0;
    if (lane == 63) base = atomicAdd(&sm.cnt, (int)incl);
    int slot = (int)lane_u32((uint32_t)base, 63) + (int)incl - tcnt;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      uint32_t msk = (mk[r >> 2] >> (8 * (r & 3))) & 0xFFu;
      if (__ballot(msk != 0u)) {
        const int g = v0 + (r * FT + tid) * EPT;
        while (msk) {
          const int e = __ffs(msk) - 1;
          msk &= msk - 1u;
          if (slot < P.cap) gc[slot] = make_int2(__float_as_int(elem_n<DT>(d[r], e)), g + e);
          ++slot;
        }
      }
    }
  }
  for (int p = tid; p < npatch; p += FT) {
    const float v = __int_as_float(patch[p].x);
    c0 += v >= tau ? 1 : 0;
    c1 += v >= t1 ? 1 : 0;
    c2 += v >= t2 ? 1 : 0;
    if (v >= tau) {
      const int slot = atomicAdd(&sm.cnt, 1);
      if (slot < P.cap) gc[slot] = make_int2(patch[p].x, patch[p].y);
    }
    if (need_zf) zs += __expf(v - ms);
  }
  // n1 | n2 << 16 in one reduction (at most 7 per thread, 7168 per slice)
  const int pk = wsum_i((c1 - c0) | ((c2 - c1) << 16));
  const double zw = need_zf ? wsum_f64((double)zs) : 0.0;
  if (lane == 0) {
    sm.redb[wv][0] = pk;
    sm.redz[wv] = zw;
  }
  __syncthreads();
  const int n = sm.cnt;
  const int nw = min(n, P.cap);
  if (out) {
    // non-candidates are never kept; the merge writes the kept ones
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int g = v0 + (r * FT + tid) * EPT;
      if (g < v1) {
#pragma unroll
        for (int e = 0; e < EPT; ++e) out[g + e] = -INFINITY;
      }
    }
  }
  if (wv == 0) {
    // lanes 0..15 read one wave's partials each; DPP sums finish them
    const bool lw = lane < FNW;
    const int s12 = wsum_i(lw ? sm.redb[lane & (FNW - 1)][0] : 0);
    const int s1 = s12 & 0xFFFF, s2 = s12 >> 16;
    const double sz = need_zf ? wsum_f64(lw ? sm.redz[lane & (FNW - 1)] : 0.0) : 0.0;
    if (lane == 0) {
    hdr->m = ms;
    hdr->tau = tau;
    hdr->n = nw;
    hdr->flags = (n > P.cap || npatch_raw > P.pcap) ? HDR_OVERFLOW : 0;
    hdr->t1 = t1;
    hdr->t2 = t2;
    hdr->g1 = s1;
    hdr->g2 = s2;
    hdr->nall = v1 - v0;
    hdr->best_i = 0;
    hdr->zf = need_zf ? sz : -1.0;
    }
  }
}

// ---------------------------------------------------------------------------
// Merge.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

struct ZBounds {
  uint64_t lo, hi;
};

// [Zlo, Zhi] for Z = sum_i exp_fix44(l_i - m) over the row, from the slice
// summaries and the exact candidate mass Scand.
//  * Lower bound: the candidates' exact masses, plus for every group counted
//    in a band [t_j, t_(j-1)) at least one element of mass
//    >= floor(2^44 e^(t_j - m) (1 - eps)) - 1.
//  * Upper bound: every non-candidate is below tau.  (A row whose
//    candidates hold most but not all of the mass can leave a top-p cut
//    open this way; rescue_row then takes a float sum over the row.)
//  * When every slice carries its float sum zf (hardware exp, relative error
//    far below eps = 2e-4 for every term that exp_fix44 does not flush to 0),
//    both bounds are also taken from zf.
// The summaries' share (ZParts, summed over the slices in slice order) does
// not depend on the candidates, so it is computed beside them.
struct ZParts {
  double lo, hi, zl, zh;
  int nz;  // slices without a float sum
};

__device__ __forceinline__ ZParts z_slice(const SliceHdr& h, float m) {
  const double SC = 17592186044416.0, EPS = 2e-4;
  ZParts p{0.0, 0.0, 0.0, 0.0, 0};
  if (h.m == -INFINITY) return p;
  // float exponentials: their error (a few ulp, arguments <= 0) is far inside
  // EPS
  auto wlo = [&](float t) {
    return t == -INFINITY ? 0.0 : fmax(floor((double)expf(t - m) * SC * (1.0 - EPS)) - 1.0, 0.0);
  };
  p.lo = (double)h.g1 * wlo(h.t1) + (double)h.g2 * wlo(h.t2);
  p.hi = (double)(h.nall - h.n) * ((double)expf(h.tau - m) * SC * (1.0 + EPS) + 1.0);
  if (h.zf >= 0.0) {
    const double sc = (double)expf(h.m - m) * SC;
    p.zl = h.zf * sc * (1.0 - EPS) - (double)h.nall;
    p.zh = h.zf * sc * (1.0 + EPS) + (double)h.nall;
  } else {
    p.nz = 1;
  }
  return p;
}

// Lanes 0..G-1 hold the slices: each takes its own share, and the G shares
// are read across the lanes.
template <int G>
__device__ __forceinline__ ZParts z_parts(const SliceHdr& hd, bool own, float m) {
  const ZParts q = own ? z_slice(hd, m) : ZParts{0.0, 0.0, 0.0, 0.0, 0};
  auto lane_f64 = [](double v, int l) {
    return __longlong_as_double((long long)lane_u64((uint64_t)__double_as_longlong(v), l));
  };
  ZParts s{0.0, 0.0, 0.0, 0.0, 0};
#pragma unroll
  for (int l = 0; l < G; ++l) {
    s.lo += lane_f64(q.lo, l);
    s.hi += lane_f64(q.hi, l);
    s.zl += lane_f64(q.zl, l);
    s.zh += lane_f64(q.zh, l);
    s.nz += (int)lane_u32((uint32_t)q.nz, l);
  }
  return s;
}

__device__ __forceinline__ ZBounds z_finish(const ZParts& s, uint64_t Scand) {
  const double LIM = 4.0e18;
  ZBounds z;
  z.lo = Scand + (uint64_t)fmax(s.lo, 0.0);
  z.hi = (s.hi >= LIM) ? (1ull << 62) : Scand + (uint64_t)ceil(s.hi);
  if (s.nz == 0) {
    const uint64_t a = s.zl <= 0.0 ? 0ull : (uint64_t)s.zl;
    const uint64_t c = s.zh >= LIM ? (1ull << 62) : (uint64_t)ceil(s.zh);
    z.lo = a > z.lo ? a : z.lo;
    z.hi = c < z.hi ? c : z.hi;
  }
  if (z.hi > (1ull << 62)) z.hi = 1ull << 62;
  return z;
}

// Candidates in registers: NS slots per lane (a compile-time count, so every
// loop over the slots is straight-line code), alive bits in `al`.
template <int NS>
struct RegStore {
  float cl[NS];
  int ci[NS];
  uint64_t w[NS];  // exp_fix44(l - m) (replaced by the draw weights at the end)
  uint32_t al;
  uint64_t* bkt;  // 64 LDS buckets for the radix descents
  ulonglong2* lp;  // 64 LDS (composite, mass) pairs for the small top-p cut
  // masses of the alive set (all / covered) while no filter has changed it
  bool cached;
  uint64_t m_all, m_cov;

  __device__ __forceinline__ bool on(int t) const { return (al >> t) & 1u; }
  template <typename F>
  __device__ __forceinline__ int count_if(F f) const {
    int c = 0;
#pragma unroll
    for (int t = 0; t < NS; ++t) c += ballot_count(on(t) && f(t));
    return c;
  }
  template <typename F>
  __device__ __forceinline__ uint64_t mass_if(F f) const {
    uint64_t z = 0;
#pragma unroll
    for (int t = 0; t < NS; ++t) z += (on(t) && f(t)) ? w[t] : 0ull;
    return wsum_u64(z);
  }
  template <typename F>
  __device__ __forceinline__ void keep_if(F f) {
    uint32_t m = 0;
#pragma unroll
    for (int t = 0; t < NS; ++t) m |= (on(t) && f(t)) ? (1u << t) : 0u;
    al = m;
    cached = false;
  }
  __device__ __forceinline__ int count() const { return count_if([](int) { return true; }); }
  __device__ __forceinline__ uint64_t mass(bool cov_only, float tcov) const {
    if (cached) return cov_only ? m_cov : m_all;
    return mass_if([&](int t) { return !cov_only || cl[t] >= tcov; });
  }
  __device__ __forceinline__ void none() {
    al = 0;
    cached = false;
  }
  __device__ __forceinline__ void keep_min(float thr) {
    keep_if([&](int t) { return cl[t] >= thr; });
  }
  // The composite (order ORD) of the element at which the cumulative measure
  // (count, or mass when MASS) over the alive slots where f holds first
  // reaches target (0 < target <= total), in descending composite order.  A
  // radix descent, 6 bits per level below the bits every such composite
  // shares: each level adds the measures of the slots under the current
  // prefix into 64 LDS buckets (bucket d at lane 63 - d, so lane order is
  // descending), scans the lanes and takes the first bucket whose inclusive
  // sum reaches the remaining target.
  template <int ORD, bool MASS, typename F>
  __device__ __forceinline__ uint64_t select_desc(F f, uint64_t target, uint64_t* bucket) const {
    const int lane = threadIdx.x & 63;
    uint64_t c[NS];
    uint64_t cmin = ~0ull, cmax = 0ull;
#pragma unroll
    for (int t = 0; t < NS; ++t) {
      const uint32_t k = fkey(cl[t]);
      c[t] = ORD == ORD_P ? comp_p(k, ci[t]) : comp_a(k, ci[t]);
      const bool p = on(t) && f(t);
      cmin = p && c[t] < cmin ? c[t] : cmin;
      cmax = p && c[t] > cmax ? c[t] : cmax;
    }
    cmin = dpp_reduce_u64(cmin, [](uint64_t x, uint64_t y) { return x < y ? x : y; });
    cmax = dpp_reduce_u64(cmax, [](uint64_t x, uint64_t y) { return x > y ? x : y; });
    const uint64_t diff = cmin ^ cmax;
    const int top = diff ? 64 - __clzll((long long)diff) : 1;
    const int L = (top + 5) / 6;
    uint64_t prefix = cmax >> (6 * L);
    for (int lev = 0; lev < L; ++lev) {
      const int sh = 6 * (L - 1 - lev);
      uint64_t bsel;  // the chosen bucket's measure
      if constexpr (MASS) {
        bucket[lane] = 0;
        wave_sync();
#pragma unroll
        for (int t = 0; t < NS; ++t) {
          if (on(t) && f(t) && (c[t] >> (sh + 6)) == prefix)
            atomicAdd((unsigned long long*)&bucket[63 - (int)((c[t] >> sh) & 63)], (unsigned long long)w[t]);
        }
        wave_sync();
        const uint64_t bv = bucket[lane];
        const uint64_t incl = wscan_incl_u64(bv);
        const int sel = (int)__ffsll((long long)__ballot(incl >= target)) - 1;
        target -= lane_u64(incl, sel) - lane_u64(bv, sel);
        prefix = (prefix << 6) | (uint64_t)(63 - sel);
        bsel = lane_u64(bv, sel);
      } else {
        // counts fit 32 bits: 32-bit buckets, atomics and scan
        uint32_t* b32 = (uint32_t*)bucket;
        b32[lane] = 0u;
        wave_sync();
#pragma unroll
        for (int t = 0; t < NS; ++t) {
          if (on(t) && f(t) && (c[t] >> (sh + 6)) == prefix) atomicAdd(&b32[63 - (int)((c[t] >> sh) & 63)], 1u);
        }
        wave_sync();
        const uint32_t bv = b32[lane];
        const uint32_t incl = wscan_incl_u32(bv);
        const int sel = (int)__ffsll((long long)__ballot((uint64_t)incl >= target)) - 1;
        target -= (uint64_t)(lane_u32(incl, sel) - lane_u32(bv, sel));
        prefix = (prefix << 6) | (uint64_t)(63 - sel);
        bsel = lane_u32(bv, sel);
      }
      wave_sync();
      // counting, a chosen bucket of count one is the answer: the target lies
      // inside that bucket's measure
      if (!MASS && sh > 0 && bsel == 1ull) {
        uint64_t only = 0;
#pragma unroll
        for (int t = 0; t < NS; ++t) only |= (on(t) && f(t) && (c[t] >> sh) == prefix) ? c[t] : 0ull;
        return dpp_reduce_u64(only, [](uint64_t x, uint64_t y) { return x | y; });
      }
    }
    return prefix;
  }
  // Top-k in order A (value desc, id asc) over the alive slots; the caller
  // has checked that more than k are alive.
  __device__ __forceinline__ void keep_topk(int k) {
    const uint64_t ck = select_desc<ORD_A, false>([](int) { return true; }, (uint64_t)k, bkt);
    keep_if([&](int t) { return comp_a(fkey(cl[t]), ci[t]) >= ck; });
  }
  __device__ __forceinline__ void topk_filter(int k) {
    if (count() > k) keep_topk(k);
  }
  // Top-p cut over the alive covered slots: both ends of [Rlo, Rhi] must
  // select the same element (order P).
  __device__ __forceinline__ bool keep_pcut(uint64_t Rlo, uint64_t Rhi, float tcov) {
    auto cov = [&](int t) { return cl[t] >= tcov; };
    uint64_t clo, chi;
    if (count_if(cov) <= 64) {
      // At most one slot per lane (after a small top-k): the slots go to LDS
      // as (composite, mass) pairs, zero-padded, and each lane sums the
      // masses of the composites at or above its own from broadcast reads,
      // eight pairs per step.  Those inclusive sums grow in descending
      // order, so the element where the sum first reaches R is the largest
      // composite whose sum reaches R.
      const int lane = threadIdx.x & 63;
      lp[lane] = make_ulonglong2(0ull, 0ull);
      int n = 0;
#pragma unroll
      for (int t = 0; t < NS; ++t) {
        const bool p = on(t) && cov(t);
        const uint64_t bal = __ballot(p);
        if (p) {
          const int i = n + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
          lp[i] = make_ulonglong2(comp_p(fkey(cl[t]), ci[t]), w[t]);
        }
        n += (int)__popcll(bal);
      }
      wave_sync();
      const uint64_t mine = lane < n ? lp[lane].x : 0ull;
      uint64_t incl = 0;
      for (int j0 = 0; j0 < n; j0 += 8) {  // j0 <= 56: every read is inside the 64 pairs
        ulonglong2 e[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) e[q] = lp[j0 + q];
#pragma unroll
        for (int q = 0; q < 8; ++q) incl += e[q].x >= mine ? e[q].y : 0ull;
      }
      auto umax = [](uint64_t x, uint64_t y) { return x > y ? x : y; };
      clo = dpp_reduce_u64(lane < n && incl >= Rlo ? mine : 0ull, umax);
      chi = dpp_reduce_u64(lane < n && incl >= Rhi ? mine : 0ull, umax);
      wave_sync();
    } else {
      clo = select_desc<ORD_P, true>(cov, Rlo, bkt);
      chi = select_desc<ORD_P, true>(cov, Rhi, bkt);
    }
    if (clo != chi) return false;
    keep_if([&](int t) { return comp_p(fkey(cl[t]), ci[t]) >= clo; });
    return true;
  }
};

// Register merge scratch.
struct MergeSmem {
  uint64_t bucket[3][64];  // draw buckets, one array per radix level
  // per lane, added by every listing wave: [0] hot mass, [1] hot mass at or
  // above tcov, [2] cold mass; [3] level-0 draw buckets (4096 ids each) over
  // every hot candidate
  alignas(16) uint64_t acc[4][64];
  ZParts zp;  // the summaries' share of the normaliser bounds
  int n;      // hot candidates listed
  int tok;    // wave 1's draw over the whole list
  uint64_t sv[5];  // [3], [4]: the normaliser bounds of a row whose top-p cut they left open
};

// Candidates in LDS (any number), filtered by the whole workgroup: masses are
// block reductions, the top-k cut a histogram-then-rank select, the top-p cut
// block radix selects.  Every method is called by every thread.
struct BlockStore {
  CandSource src;
  Pred pr;
  float m;
  ExactSmem* sm;

  __device__ __forceinline__ int count() const {
    int c = 0;
    src.each([&](int i, float l) { c += pr.keep(i, l) ? 1 : 0; });
    return block_reduce(c, sm->scratchi, OpSumI(), 0);
  }
  __device__ __forceinline__ uint64_t mass(bool cov_only, float tcov) const {
    Pred p = pr;
    if (cov_only) p.cov = tcov;
    uint64_t z = 0;
    const float mm = m;
    src.each([&](int i, float l) { if (p.keep(i, l)) z += exp_fix44(l - mm); });
    return block_reduce(z, sm->scratch64, OpSumU64(), (uint64_t)0);
  }
  __device__ __forceinline__ void none() { pr.none = 1; }
  __device__ __forceinline__ void keep_min(float thr) {
    pr.use_m = 1;
    pr.thr = thr;
  }
  // top-k when more than k are kept (the count comes from the select's
  // first pass)
  __device__ __forceinline__ void topk_filter(int k) {
    uint64_t ck;
    if (block_kth_desc<ORD_A>(src, pr, (uint64_t)k, *sm, &ck)) {
      pr.use_k = 1;
      pr.ck = ck;
    }
  }
  __device__ __forceinline__ bool keep_pcut(uint64_t Rlo, uint64_t Rhi, float tcov) {
    Pred pc = pr;
    pc.cov = tcov;
    const float mm = m;
    auto mass_fn = [mm](int, float l) { return exp_fix44(l - mm); };
    const uint64_t clo = radix_select<ORD_P, true>(src, pc, mass_fn, Rlo, *sm);
    const uint64_t chi = radix_select<ORD_P, true>(src, pc, mass_fn, Rhi, *sm);
    if (clo != chi) return false;
    pr.use_p = 1;
    pr.cp = clo;
    return true;
  }
};

// The filters in the chain's order over a candidate store.  Returns false when
// the top-p cut is not settled by [Zlo, Zhi] (the row goes to the exact engine).
template <typename St>
__device__ __forceinline__ bool run_filters(St& st, const SampleKArgs& a, const RowParams& rp, float m, float tcov, ZBounds zb) {
  const float theta = rp.theta;
  bool none = false;
  // Top-p keeps i iff S - head_excl(i) > floor(theta Z).  With Z only known
  // to lie in [Zlo, Zhi] the cut is taken when both ends agree.  S is the
  // alive mass: exact when s_exact (after an exact top-k), else Z itself.
  auto apply_p = [&](bool s_exact) -> bool {
    if (zb.lo > zb.hi) return false;
    long long Rlo, Rhi;
    if (s_exact) {
      const long long S = (long long)st.mass(false, tcov);
      Rlo = S - (long long)floor_theta_z(theta, zb.hi);
      Rhi = S - (long long)floor_theta_z(theta, zb.lo);
    } else {
      Rlo = (long long)(zb.lo - floor_theta_z(theta, zb.lo));
      Rhi = (long long)(zb.hi - floor_theta_z(theta, zb.hi));
    }
    if (Rhi <= 0) {
      st.none();
      none = true;
      return true;
    }
    if (Rlo <= 0) return false;
    // Candidates at or above tcov (the largest slice threshold) have every
    // element ranked above them among the candidates.
    const long long Scov = (long long)st.mass(true, tcov);
    if (Rlo > Scov) {
      // every covered element survives; the kept set stays inside the
      // covered region only when a later filter or the top-k set confines it
      return !rp.tp;
    }
    if (Rhi > Scov) return false;
    return st.keep_pcut((uint64_t)Rlo, (uint64_t)Rhi, tcov);
  };
  const float thr = m + rp.cmin;
  if (a.chain == WH_CHAIN_MLX && rp.use_k && rp.use_p) {
    // k -> p -> min-p; the candidates hold the whole top-k set
    st.topk_filter(rp.top_k);
    if (!apply_p(true)) return false;
    if (!none && rp.use_m) st.keep_min(thr);
  } else {
    // p -> min-p -> k (Whallm), or mlx_lm without top-p and top-k together:
    // k -> min-p keeps the first k of the min-p set, which is a value prefix
    if (rp.use_p && !apply_p(false)) return false;
    if (!none && rp.use_m) st.keep_min(thr);
    if (!none && rp.use_k) st.topk_filter(rp.top_k);
  }
  return true;
}

// LDS list of the hot candidates (those that can still be kept): entry i is
// cand[i] = (logit bits, id), mass[i] = exp_fix44(logit - m) and, when T != 1,
// dw[i] = the draw weight exp_fix44(scaled logit).
struct HotList {
  int2* cand;
  uint64_t* mass;
  uint64_t* dw;
};
__device__ __forceinline__ HotList hot_list(char* dyn) {
  HotList h;
  h.cand = (int2*)dyn;
  h.mass = (uint64_t*)(dyn + (size_t)QSPEC * 64 * sizeof(int2));
  h.dw = h.mass + QSPEC * 64;
  return h;
}
constexpr int DRAW_MEMBERS = 16;  // draw: bucket members resolved directly, at most
constexpr size_t HOT_LIST_BYTES = (size_t)QSPEC * 64 * (sizeof(int2) + 2 * sizeof(uint64_t));

// The draw is the smallest id whose inclusive kept weight, in vocabulary
// order, exceeds the target draw_target(u, ZV).  The candidates are in no
// order.  Level 0 sums the kept weights of each block of 4096 ids (bucket d
// at lane d), scans the lanes and takes the first bucket whose inclusive sum
// exceeds the target; its scan total is the normaliser ZV.  Inside the
// chosen block, a handful of members is resolved directly: each member's
// inclusive weight over the members at or below its id, then the smallest
// id above the remaining target.  More members go through two more 6-bit
// radix levels (LDS buckets 1 and 2).
//
// Level 0: the chosen block, and rem reduced to the remainder inside it
// (incl0 / bv0: the lane's inclusive scan and bucket; ZV > 0).
__device__ __forceinline__ int draw_level0(uint64_t incl0, uint64_t bv0, uint64_t ZV, float u, uint64_t& rem) {
  rem = draw_target(u, ZV);
  // a bucket exists: rem is below the total
  const int p0 = (int)__ffsll((long long)__ballot(incl0 > rem)) - 1;
  rem -= lane_u64(incl0, p0) - lane_u64(bv0, p0);
  return p0;
}
// Inside block p0, over the slots in `on` (ids ci, weights w).
template <int NS>
__device__ __forceinline__ int draw_in_block(const int (&ci)[NS], const uint64_t (&w)[NS], uint32_t on, int p0, uint64_t rem,
                                             MergeSmem& sm) {
  const int lane = threadIdx.x & 63;
  auto member = [&](int t) { return ((on >> t) & 1u) && ((uint32_t)ci[t] >> 12) == (uint32_t)p0; };
  int nmem = 0;
#pragma unroll
  for (int t = 0; t < NS; ++t) nmem += ballot_count(member(t));
  if (nmem <= DRAW_MEMBERS) {
    uint64_t cum[NS];
#pragma unroll
    for (int t = 0; t < NS; ++t) cum[t] = 0;
#pragma unroll
    for (int t = 0; t < NS; ++t) {
      uint64_t bits = __ballot(member(t));
      while (bits) {
        const int k = (int)__builtin_ctzll(bits);
        bits &= bits - 1;
        const uint32_t idk = lane_u32((uint32_t)ci[t], k);
        const uint64_t wk = lane_u64(w[t], k);
#pragma unroll
        for (int q = 0; q < NS; ++q) cum[q] += (uint32_t)ci[q] >= idk ? wk : 0ull;
      }
    }
    uint32_t best = 0xFFFFFFFFu;
#pragma unroll
    for (int t = 0; t < NS; ++t)
      if (member(t) && cum[t] > rem) best = min(best, (uint32_t)ci[t]);
    return (int)wmin_u32(best);
  }
  uint32_t prefix = (uint32_t)p0;
  sm.bucket[1][lane] = 0;
  sm.bucket[2][lane] = 0;
  wave_sync();
  for (int lev = 1; lev < 3; ++lev) {
    const int sh = 12 - 6 * lev;
#pragma unroll
    for (int t = 0; t < NS; ++t) {
      if (((on >> t) & 1u) && ((uint32_t)ci[t] >> (sh + 6)) == prefix)
        atomicAdd((unsigned long long*)&sm.bucket[lev][((uint32_t)ci[t] >> sh) & 63u], (unsigned long long)w[t]);
    }
    wave_sync();
    const uint64_t bv = sm.bucket[lev][lane];
    const uint64_t incl = wscan_incl_u64(bv);
    const int bsel = (int)__ffsll((long long)__ballot(incl > rem)) - 1;
    rem -= lane_u64(incl, bsel) - lane_u64(bv, bsel);
    prefix = (prefix << 6) | (uint32_t)bsel;
  }
  return (int)prefix;
}

// The draw of row b over every listed hot candidate, by wave 1 while wave 0
// runs the filters: it is the row's draw whenever the filters keep the whole
// list (level 0 is then the listing waves' buckets).  Lane 0 leaves the
// token in sm.tok.
template <int NS>
__device__ __forceinline__ void spec_draw(bool tscale, float ub, const HotList& hl, int N, MergeSmem& sm) {
  const int lane = threadIdx.x & 63;
  int ci[NS];
  uint64_t w[NS];
  uint32_t on = 0;
#pragma unroll
  for (int t = 0; t < NS; ++t) {
    const bool valid = t * 64 + lane < N;
    const int i = valid ? t * 64 + lane : 0;
    const int id = hl.cand[i].y;
    const uint64_t x = tscale ? hl.dw[i] : hl.mass[i];
    ci[t] = valid ? id : -1;
    w[t] = valid ? x : 0ull;
    on |= valid ? (1u << t) : 0u;
  }
  const uint64_t bv0 = sm.acc[3][lane];
  const uint64_t incl0 = wscan_incl_u64(bv0);
  const uint64_t ZV = lane_u64(incl0, 63);
  int tok = 0;
  if (ZV) {
    uint64_t rem;
    const int p0 = draw_level0(incl0, bv0, ZV, ub, rem);
    tok = draw_in_block<NS>(ci, w, on, p0, rem, sm);
  }
  if (lane == 0) sm.tok = tok;
}

// Totals of the four 64-entry per-lane sums in LDS: lanes 16k..16k+15 add
// four entries of array k each, the four DPP steps inside a row of 16
// (dpp_reduce_u64's first four) finish each row, and lane 16k holds array
// k's total.
__device__ __forceinline__ void totals4(const uint64_t (*acc)[64], uint64_t (&t)[4]) {
  const int lane = threadIdx.x & 63;
  const uint64_t* p = &acc[lane >> 4][(lane & 15) * 4];
  uint64_t x = (p[0] + p[1]) + (p[2] + p[3]);
#define WH_ROW_STEP(C)                                                                          \
  {                                                                                             \
    const uint64_t y_ = ((uint64_t)dpp32<C>((uint32_t)(x >> 32)) << 32) | dpp32<C>((uint32_t)x); \
    x += y_;                                                                                    \
  }
  WH_ROW_STEP(0xB1)
  WH_ROW_STEP(0x4E)
  WH_ROW_STEP(0x141)
  WH_ROW_STEP(0x140)
#undef WH_ROW_STEP
#pragma unroll
  for (int k = 0; k < 4; ++k) t[k] = lane_u64(x, 16 * k);
}

// The filters' outcome from the totals alone, for chains where min-p is the
// last filter on the listed candidates and there is no top-k: the listed
// candidates all reach thr, so min-p keeps them all, and top-p (the same
// steps as run_filters) either keeps every listed candidate (0), sends the
// row to the exact engine (3), or needs the candidates themselves (-1: a cut
// inside the list, or nothing kept).
__device__ __forceinline__ int quick_filters(const RowParams& rp, ZBounds zb, uint64_t m_cov) {
  if (!rp.use_p) return 0;
  if (zb.lo > zb.hi) return 3;
  const float theta = rp.theta;
  const long long Rlo = (long long)(zb.lo - floor_theta_z(theta, zb.lo));
  const long long Rhi = (long long)(zb.hi - floor_theta_z(theta, zb.hi));
  if (Rhi <= 0) return -1;
  if (Rlo <= 0) return 3;
  const long long Scov = (long long)m_cov;
  if (Rlo > Scov) return rp.tp ? 3 : 0;
  if (Rhi > Scov) return 3;
  return -1;
}

// Register merge of row b by wave 0.  The row's N hot candidates sit in the
// LDS list in no particular order (every step below is order independent);
// slot t of lane l holds entry 64 t + l, so NS is ceil(N / 64) rounded up to
// a compiled slot count.  The listing waves' per-lane partial sums are in
// m_all / m_cov are the list's exact mass and its mass at or above tcov, ZV
// its total draw weight, zb the row's normaliser bounds.  Between the
// filters and the draw it takes part in one workgroup barrier (every other
// wave takes part in it too), after which wave 1's speculative token is in
// sm.tok.  Returns the path code (0 done, 3 exact engine).
template <int NS>
__device__ __forceinline__ int merge_regs(const SampleKArgs& a, int b, const RowParams& rp, float m, float tcov, float ub,
                                          const HotList& hl, int N, uint64_t m_all, uint64_t m_cov, uint64_t ZV_all,
                                          ZBounds zb, MergeSmem& sm) {
  const int lane = threadIdx.x & 63;
  const bool tscale = rp.tscale;
  RegStore<NS> st;
  uint64_t wd[NS];
  st.al = 0;
  st.bkt = sm.bucket[0];
  // the listing's per-lane sums are consumed by the totals before the filters
  st.lp = (ulonglong2*)&sm.acc[0][0];
#pragma unroll
  for (int t = 0; t < NS; ++t) {
    const bool valid = t * 64 + lane < N;
    const int i = valid ? t * 64 + lane : 0;
    const int2 c = hl.cand[i];
    const uint64_t w = hl.mass[i];
    wd[t] = tscale ? hl.dw[i] : 0ull;
    st.cl[t] = valid ? __int_as_float(c.x) : -INFINITY;
    st.ci[t] = valid ? c.y : -1;
    st.w[t] = valid ? w : 0ull;
    st.al |= valid ? (1u << t) : 0u;
  }
  st.m_all = m_all;
  st.m_cov = m_cov;
  st.cached = true;
  const uint32_t al0 = st.al;
  const bool ok = run_filters(st, a, rp, m, tcov, zb);
  const bool all_kept = __ballot(st.al != al0) == 0ull;
  __syncthreads();  // wave 1's speculative token is in sm.tok
  if (!ok) return 3;

  // Draw: integer inverse CDF in vocabulary order over the kept slots.
  const float invT = rp.invT;
  const double rTc = rp.rTc;
  uint64_t ZV;
  int tok = 0;
  if (all_kept) {
    ZV = ZV_all;
    tok = sm.tok;
  } else {
    if (tscale) {
#pragma unroll
      for (int t = 0; t < NS; ++t) st.w[t] = st.on(t) ? wd[t] : 0ull;
    }
    sm.bucket[0][lane] = 0;
    wave_sync();
#pragma unroll
    for (int t = 0; t < NS; ++t)
      if (st.on(t)) atomicAdd((unsigned long long*)&sm.bucket[0][(uint32_t)st.ci[t] >> 12], (unsigned long long)st.w[t]);
    wave_sync();
    const uint64_t bv0 = sm.bucket[0][lane];
    const uint64_t incl0 = wscan_incl_u64(bv0);
    ZV = lane_u64(incl0, 63);
    if (a.tokens && ZV) {
      uint64_t rem;
      const int p0 = draw_level0(incl0, bv0, ZV, ub, rem);
      tok = draw_in_block<NS>(st.ci, st.w, st.al, p0, rem, sm);
    }
  }
  if (a.tokens && lane == 0) a.tokens[b] = ZV ? tok : 0;
  if (a.kept) {
    const int nkept = st.count();
    if (lane == 0) a.kept[b] = nkept;
  }
  float* out = a.out_rows ? a.out_rows + (long long)b * a.V : nullptr;
  if (out) {
    const double lz = log(ldexp((double)ZV, -44));
#pragma unroll
    for (int t = 0; t < NS; ++t)
      if (st.on(t))
        out[st.ci[t]] = a.out_mode == WH_OUT_MASKED ? st.cl[t]
                                                    : (float)((double)chain_scale(a.chain, st.cl[t] - m, invT, rTc) - lz);
  }
  return 0;
}

// Normaliser bounds narrowed by a float sum zs of exp(l - m) over a row of V
// values (relative error far below EPS, each term's floor costs under 1).
__device__ __forceinline__ void tighten_z(ZBounds& zb, double zs, int V) {
  const double SC = 17592186044416.0, EPS = 2e-4, LIM = 4.0e18;
  const double zl = zs * SC * (1.0 - EPS) - (double)V, zh = zs * SC * (1.0 + EPS) + (double)V;
  const uint64_t lo = zl <= 0.0 ? 0ull : (uint64_t)zl;
  const uint64_t hi = zh >= LIM ? (1ull << 62) : (uint64_t)ceil(zh);
  zb.lo = lo > zb.lo ? lo : zb.lo;
  zb.hi = hi < zb.hi ? hi : zb.hi;
}

// The filters and the draw of a listed row by wave 0 (path 0, or 3 for the
// exact engine): the quick decision from the totals when min-p is the last
// filter and there is no top-k, else the register merge.  Either way wave 0
// takes part in exactly one workgroup barrier, after which wave 1's
// speculative token is in sm.tok.
__device__ __forceinline__ int merge_filters(const SampleKArgs& a, int b, const RowParams& rp, float m, float tcov, float ub,
                                             const HotList& hl, int N, uint64_t m_all, uint64_t m_cov, uint64_t ZV,
                                             ZBounds zb, MergeSmem& sm) {
  const int lane = threadIdx.x & 63;
  // with min-p last and no top-k the totals settle most rows: then the
  // candidates need not be loaded at all
  const int quick = (rp.use_m && !rp.use_k && !a.out_rows) ? quick_filters(rp, zb, m_cov) : -1;
  if (quick >= 0) {
    __syncthreads();  // wave 1's speculative token is in sm.tok
    if (quick == 0 && lane == 0) {
      if (a.tokens) a.tokens[b] = ZV ? sm.tok : 0;
      if (a.kept) a.kept[b] = N;
    }
    return quick;
  }
  if (N <= 64) return merge_regs<1>(a, b, rp, m, tcov, ub, hl, N, m_all, m_cov, ZV, zb, sm);
  if (N <= 128) return merge_regs<2>(a, b, rp, m, tcov, ub, hl, N, m_all, m_cov, ZV, zb, sm);
  if (N <= 256) return merge_regs<4>(a, b, rp, m, tcov, ub, hl, N, m_all, m_cov, ZV, zb, sm);
  if (N <= 512) return merge_regs<8>(a, b, rp, m, tcov, ub, hl, N, m_all, m_cov, ZV, zb, sm);
  return merge_regs<QM>(a, b, rp, m, tcov, ub, hl, N, m_all, m_cov, ZV, zb, sm);
}

// The filters and the draw over candidates in LDS (src), run by every thread
// of the workgroup: path 4 done, 3 when the bounds zb leave a top-p cut open.
__device__ __forceinline__ int block_finish(const SampleKArgs& a, int b, const RowParams& rp, float m, float tcov, float ub,
                                            const CandSource& src0, ZBounds zb, ExactSmem& sm) {
  const int tid = threadIdx.x;
  BlockStore st{src0, Pred{0, 0, 0, 0, 0, 0, 0.0f, -INFINITY}, m, &sm};
  if (!run_filters(st, a, rp, m, tcov, zb)) return 3;
  const float invT = rp.invT;
  const double rTc = rp.rTc;
  const Pred pr = st.pr;
  const CandSource src = st.src;
  auto vw = [&](int, float l) { return exp_fix44(chain_scale(a.chain, l - m, invT, rTc)); };
  // the draw weights' sum, the kept count and the draw in one pass plus the
  // target's bin
  uint64_t ZV;
  int nkept;
  const int tok = block_draw_id(src, pr, vw, ub, a.tokens != nullptr, sm, &ZV, &nkept);
  if (tid == 0 && a.tokens) a.tokens[b] = tok;
  if (tid == 0 && a.kept) a.kept[b] = nkept;
  float* out = a.out_rows ? a.out_rows + (long long)b * a.V : nullptr;
  if (out) {
    const double lz = log(ldexp((double)ZV, -44));
    src.each([&](int i, float l) {
      if (!pr.keep(i, l)) return;
      out[i] = a.out_mode == WH_OUT_MASKED ? l : (float)((double)chain_scale(a.chain, l - m, invT, rTc) - lz);
    });
  }
  return 4;
}

// Block merge of row b (any number of candidates), run by every thread of
// the workgroup.  Returns the path code (4 done, 3 exact engine).  The
// arguments are read in place from the kernel-argument segment (a pointer,
// not a copy).  It is inlined: out of line, its LDS pointers arrive as
// generic pointers and every LDS access becomes a flat access (B = 256,
// V = 129,280 f32 rows with per-row top-k up to 1024 took 84.4 us per call
// that way, 79.2 us inlined).  hdl is the kernel's
// register copy of the summaries (lane s < G holds slice s): the counts and
// the normaliser bounds come from it, and the candidates are loaded U per
// thread before any is stored, so a row costs one round trip per U * 512
// candidates.
template <int G>
__device__ __forceinline__ int merge_block(const SampleKArgs* ap, const FastPlan* pp, int b, RowParams rp, const SliceHdr& hdl,
                                           float m, float tcov, float ub, char* dyn, ExactSmem* smp, MergeSmem* msp) {
  const SampleKArgs& a = *ap;
  const FastPlan& P = *pp;
  ExactSmem& sm = *smp;
  const int tid = threadIdx.x, nt = blockDim.x;
  float* cv = (float*)dyn;
  int* ci = (int*)(dyn + (size_t)G * P.cap * sizeof(float));
  // slice s's candidates go to [off[s], off[s + 1])
  int off[G + 1];
  off[0] = 0;
#pragma unroll
  for (int s = 0; s < G; ++s) off[s + 1] = off[s] + min((int)lane_u32((uint32_t)hdl.n, s), P.cap);
  const int N = off[G];
  const int2* row = P.cand + (long long)b * G * P.cap;
  constexpr int U = 8;
  for (int i0 = 0; i0 < N; i0 += U * nt) {
    int2 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * nt + tid;
      int s = 0, os = 0;
#pragma unroll
      for (int q = 1; q < G; ++q)
        if (i >= off[q]) {
          s = q;
          os = off[q];
        }
      v[u] = row[i < N ? (long long)s * P.cap + (i - os) : 0];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * nt + tid;
      if (i < N) {
        cv[i] = __int_as_float(v[u].x);
        ci[i] = v[u].y;
      }
    }
  }
  __syncthreads();
  // the normaliser bounds serve the top-p cut alone (rp.use_p is uniform
  // over the workgroup, so the block reductions inside run on every thread)
  const CandSource src{cv, ci, N};
  ZBounds zb{0ull, 0ull};
  if (rp.use_p) {
    BlockStore st{src, Pred{0, 0, 0, 0, 0, 0, 0.0f, -INFINITY}, m, &sm};
    zb = z_finish(z_parts<G>(hdl, (threadIdx.x & 63) < G, m), st.mass(false, 0.0f));
  }
  const int path = block_finish(a, b, rp, m, tcov, ub, src, zb, sm);
  if (path == 3 && tid == 0) {
    // for the second bounds pass (rescue_row)
    msp->n = N;
    msp->sv[3] = zb.lo;
    msp->sv[4] = zb.hi;
  }
  return path;
}

// A second bounds pass for a row whose bounds left the top-p cut open
// (typically a row whose candidates hold most but not all of the mass, with
// min-p setting the slices' thresholds, so the slices took no float sums):
// one float sum of exp(l - m) over the row bounds Z to 2e-4, and the filters
// run again, through the block merge, on the candidates still in LDS -- the
// register merge's hot list (from_list; moved into value / id arrays
// first) or the block merge's arrays.  The penalty table goes after them.
// Returns 7 or 8 (settled after the register or the block merge) or 3 (the
// exact engine).  Out of line and called at the end of the merge kernel,
// where nothing of the caller's is live: inlined or called earlier it cost
// the common path registers (2-5 us per call); its LDS accesses are flat
// accesses.  Every thread of the workgroup calls it.
__device__ __noinline__ int rescue_row(const SampleKArgs* ap, const FastPlan* pp, int b, float m, float tcov, float ub,
                                       char* dyn, ExactSmem* esm, MergeSmem* msm, int G, int from_list) {
  const SampleKArgs& a = *ap;
  const FastPlan& P = *pp;
  const int tid = threadIdx.x, nt = blockDim.x;
  const RowParams rp = row_params(a, row_raw(a, a, b), P.rule_cap);
  const int N = msm->n;
  float* cv = (float*)dyn;
  int* ci;
  char* pen;
  if (from_list) {
    // the hot list (at most QSPEC * 64 entries) into value / id arrays in
    // place: every entry is read before any is written
    constexpr int LPT = (QSPEC * 64) / (MW * 64);
    const HotList hl = hot_list(dyn);
    int2 e[LPT];
#pragma unroll
    for (int q = 0; q < LPT; ++q) e[q] = hl.cand[min(tid + q * nt, N > 0 ? N - 1 : 0)];
    __syncthreads();
    ci = (int*)(dyn + (size_t)QSPEC * 64 * sizeof(float));
#pragma unroll
    for (int q = 0; q < LPT; ++q)
      if (tid + q * nt < N) {
        cv[tid + q * nt] = __int_as_float(e[q].x);
        ci[tid + q * nt] = e[q].y;
      }
    pen = dyn + (size_t)QSPEC * 64 * 8;
  } else {
    ci = (int*)(dyn + (size_t)G * P.cap * sizeof(float));
    pen = dyn + (size_t)G * P.cap * 8;
  }
  ZBounds zb{msm->sv[3], msm->sv[4]};
  tighten_z(zb, a.dtype == WH_DTYPE_BF16 ? row_zsum_t<1>(a, b, m, pen, *esm) : row_zsum_t<0>(a, b, m, pen, *esm), a.V);
  const int path = block_finish(a, b, rp, m, tcov, ub, CandSource{cv, ci, N}, zb, *esm);
  return path == 3 ? 3 : (from_list ? 7 : 8);
}

template <int G>
__global__ void __launch_bounds__(MW * 64) merge_kernel(const SliceHdr* __restrict__ hdr, const int2* __restrict__ cand,
                                                         SampleKArgs a, FastPlan P) {
  extern __shared__ __align__(16) char dyn[];
  __shared__ ExactSmem esm;
  __shared__ MergeSmem sm;
  __shared__ int s_path;
  const int b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  // One round trip per wave, issued first (its pointers are preloaded
  // arguments): the summaries (lane s < G) and the wave's QW candidate
  // chunks (slot t = QW wv + j: chunk t / G of slice t % G).  Every load is
  // unconditional from an in-bounds address (lanes >= G read a duplicate
  // summary, chunks past a slice's count stale entries, both ignored), so no
  // branch join waits for a load to land.
  const SliceHdr hd = hdr[(long long)b * G + min(lane, G - 1)];
  int2 spec[QW];
#pragma unroll
  for (int j = 0; j < QW; ++j) {
    const int t = wv * QW + j;
    spec[j] = cand[((long long)b * G + t % G) * FAST_CAP + (t / G) * 64 + lane];
  }
  asm volatile("" ::: "memory");
  const RowRaw raw = row_raw(a, merge_kernargs()->a, b);
  const RowParams rp = row_params(a, raw, P.rule_cap);
  const float ub = (a.tokens && !rp.greedy) ? a.u[b] : 0.0f;
  // the list counter and the per-lane sums are zero before any wave adds to
  // them (the barrier waits for none of the loads above)
  if (tid == 0) sm.n = 0;
  if (tid < 4 * 64) (&sm.acc[0][0])[tid] = 0ull;
  __syncthreads();
  // the G summaries sit in lanes 0..G-1: aggregate them with readlanes
  float m = -INFINITY, tcov = -INFINITY;
  int fl = 0, nmax = 0;
#pragma unroll
  for (int l = 0; l < G; ++l) {
    m = fmaxf(m, __uint_as_float(lane_u32(__float_as_uint(hd.m), l)));
    tcov = fmaxf(tcov, __uint_as_float(lane_u32(__float_as_uint(hd.tau), l)));
    fl |= (int)lane_u32((uint32_t)hd.flags, l);
    nmax = max(nmax, (int)lane_u32((uint32_t)hd.n, l));
  }
  const int flagged = fl & HDR_OVERFLOW;
  // the path is the same in every wave: 0 register merge, 1 exact engine,
  // 2 greedy, 5 block merge (too many candidates for the loaded chunks)
  int path;
  int from_list = 1;  // a path 3 row came from the register merge (0: the block merge)
  if (rp.greedy) path = flagged ? 1 : 2;
  else if (flagged || rp.all) path = 1;
  else path = G * ((nmax + 63) / 64) <= QSPEC ? 0 : 5;
  if (path == 2) {
    if (wv == 0) {
      const int bi = wmin_i((lane < G && hd.m == m) ? hd.best_i : 0x7FFFFFFF);
      if (lane == 0) {
        if (a.tokens) a.tokens[b] = bi == 0x7FFFFFFF ? 0 : bi;
        if (a.kept) a.kept[b] = 1;
        P.path[b] = 2;
      }
    }
    return;
  }
  if (path == 0) {
    // Every wave lists the candidates of its chunks.  Chunk t holds lanes
    // [0, cnt_t) (a slice's candidates are a prefix of its list).  When
    // min-p is the chain's last filter on the candidates (every chain but
    // mlx_lm's top-k + top-p), a candidate below thr = m + ln min_p can never
    // be kept: only its exact mass matters (to the normaliser), so it is
    // summed and left out of the list.  Elsewhere thr is -inf and every
    // candidate is listed.  Each lane adds its three masses to its own LDS
    // sums, and every listed candidate its draw weight to the level-0 draw
    // bucket of its id; wave 0 scans both.
    const HotList hl = hot_list(dyn);
    const bool split = rp.use_m && !(a.chain == WH_CHAIN_MLX && rp.use_k && rp.use_p);
    const float thr = split ? m + rp.cmin : -INFINITY;
    const bool tscale = rp.tscale;
    const float invT = rp.invT;
    const double rTc = rp.rTc;
    const int hn = lane < G ? hd.n : 0;
    uint64_t mv[3] = {0ull, 0ull, 0ull};  // hot mass, covered hot mass, cold mass
    uint64_t e[QW], bh[QW];
    int H = 0;
    bool any = false;
#pragma unroll
    for (int j = 0; j < QW; ++j) {
      const int t = wv * QW + j;
      // cnt is wave uniform: an empty chunk is skipped by a scalar branch
      const int cnt = min(max((int)lane_u32((uint32_t)hn, t % G) - (t / G) * 64, 0), 64);
      e[j] = 0ull;
      bh[j] = 0ull;
      if (cnt > 0) {
        any = true;
        const float l = __int_as_float(spec[j].x);
        const bool v = lane < cnt;
        const bool hot = v && l >= thr;
        const uint64_t ej = exp_fix44(l - m);
        mv[0] += hot ? ej : 0ull;
        mv[1] += (hot && l >= tcov) ? ej : 0ull;
        mv[2] += (v && !hot) ? ej : 0ull;
        e[j] = ej;
        bh[j] = __ballot(hot);
        H += (int)__popcll(bh[j]);
      }
    }
    int base = 0;
    if (H > 0) {
      int r = 0;
      if (lane == 0) r = atomicAdd(&sm.n, H);
      base = __builtin_amdgcn_readfirstlane(r);
    }
#pragma unroll
    for (int j = 0; j < QW; ++j) {
      if ((bh[j] >> lane) & 1ull) {
        const int i = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bh[j] >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bh[j], 0u));
        uint64_t dw = e[j];
        if (tscale) {
          dw = exp_fix44(chain_scale(a.chain, __int_as_float(spec[j].x) - m, invT, rTc));
          hl.dw[i] = dw;
        }
        hl.cand[i] = spec[j];
        hl.mass[i] = e[j];
        atomicAdd((unsigned long long*)&sm.acc[3][(uint32_t)spec[j].y >> 12], (unsigned long long)dw);
      }
      base += (int)__popcll(bh[j]);
    }
    if (any) {
#pragma unroll
      for (int k = 0; k < 3; ++k) atomicAdd((unsigned long long*)&sm.acc[k][lane], (unsigned long long)mv[k]);
    }
    // the summaries' share of the normaliser bounds, beside the list (the
    // last wave's chunks are the ones most often empty)
    if (wv == MW - 1) {
      const ZParts zp = z_parts<G>(hd, lane < G, m);
      if (lane == 0) sm.zp = zp;
    }
    __syncthreads();
    const int N = sm.n;
    if (wv != 0) {
      // wave 1 draws over the whole list meanwhile; every wave then meets
      // wave 0 at the barrier between its filters and its draw
      if (wv == 1 && a.tokens) {
        if (N <= 64) spec_draw<1>(tscale, ub, hl, N, sm);
        else if (N <= 128) spec_draw<2>(tscale, ub, hl, N, sm);
        else if (N <= 256) spec_draw<4>(tscale, ub, hl, N, sm);
        else if (N <= 512) spec_draw<8>(tscale, ub, hl, N, sm);
        else spec_draw<QM>(tscale, ub, hl, N, sm);
      }
      __syncthreads();
    } else {
      // the exact masses and the normaliser of the whole list
      uint64_t tot[4];
      totals4(sm.acc, tot);
      const uint64_t m_all = tot[0], m_cov = tot[1], ZV = tot[3];
      const ZBounds zb = z_finish(sm.zp, m_all + tot[2]);
      path = merge_filters(a, b, rp, m, tcov, ub, hl, N, m_all, m_cov, ZV, zb, sm);
      if (lane == 0) {
        if (path == 3) {
          // for the second bounds pass (rescue_row)
          sm.sv[3] = zb.lo;
          sm.sv[4] = zb.hi;
        }
        s_path = path;
        P.path[b] = path;
      }
    }
    __syncthreads();
    path = s_path;
  } else if (path == 5) {
    from_list = 0;
    path = merge_block<G>(&merge_kernargs()->a, &merge_kernargs()->p, b, rp, hd, m, tcov, ub, dyn, &esm, &sm);
    if (tid == 0) P.path[b] = path;
    __syncthreads();
  } else if (tid == 0) {
    P.path[b] = path;
  }
  if (path == 3 && rp.use_p && (P.zpass & (from_list ? 1 : 2))) {
    path = rescue_row(&merge_kernargs()->a, &merge_kernargs()->p, b, m, tcov, ub, dyn, &esm, &sm, G, from_list);
    if (tid == 0) P.path[b] = path;
    __syncthreads();
  }
  if (path == 1 || path == 3) exact_row(merge_kernargs()->a, b, dyn, esm);
}

// ---------------------------------------------------------------------------
// Host side: plan, workspace layout, dispatch.
// ---------------------------------------------------------------------------
struct HostPlan {
  int G, SL, R, cap, rule_cap, ept, pcap, codes_bytes;
  size_t lds;
};

// Dynamic LDS of the merge kernel at most (its static LDS is under 13 KB).
constexpr size_t MERGE_LDS_MAX = 160 * 1024 - 16 * 1024;
// Dynamic LDS of the slice kernel at most (its static LDS is under 5 KB).
constexpr size_t SLICE_LDS_MAX = 160 * 1024 - 6 * 1024;

static HostPlan make_plan(int B, int V, int dtype, int hcap) {
  HostPlan p;
  p.ept = dtype == WH_DTYPE_BF16 ? 8 : 4;
  const int esz = dtype == WH_DTYPE_BF16 ? 2 : 4;
  const int slmax = FT * FAST_NE;
  const int bb = std::max(B, 1);
  int g = std::max(std::min((256 + bb - 1) / bb, GPREF), (V + slmax - 1) / slmax);
  g = std::max(g, 1);
  // more slices until the penalty codes (one per element) and the listed
  // penalised elements fit in LDS
  for (;; ++g) {
    int sl = (V + g - 1) / g;
    sl = (sl + p.ept - 1) / p.ept * p.ept;
    // rounding the slice length up can leave trailing slices empty (bf16
    // V = 40 over 4 slices of 16); drop them, so every slice starts inside
    // the row and its clamped load addresses stay in bounds
    p.G = (V + sl - 1) / sl;
    p.SL = sl;
    p.codes_bytes = hcap > 0 ? (sl * esz + 15) / 16 * 16 : 0;
    p.pcap = hcap > 0 ? std::min(hcap / 2, sl) : 0;
    p.lds = (size_t)p.codes_bytes + (size_t)p.pcap * 8;
    if (p.lds <= SLICE_LDS_MAX) break;
  }
  p.R = (p.SL + FT * p.ept - 1) / (FT * p.ept);
  p.cap = FAST_CAP;
  p.rule_cap = FAST_CAP / 2;
  return p;
}

struct WsLayout {
  size_t path, hdr, cand, total;
};

// Workspace: [path B x int32][slice summaries B*G][candidates B*G*cap]
static WsLayout ws_layout(int B, const HostPlan& p) {
  WsLayout w;
  w.path = 0;
  w.hdr = ((size_t)B * 4 + 255) / 256 * 256;
  w.cand = w.hdr + (size_t)B * p.G * sizeof(SliceHdr);
  w.total = w.cand + (size_t)B * p.G * p.cap * sizeof(int2);
  return w;
}

// The largest layout over both element types, with and without penalties
// (penalties can take more slices for the codes to fit in LDS).
size_t sample_workspace_bytes(int B, int V) {
  if (B <= 0 || V <= 0) return 256;
  size_t t = wide_workspace_bytes(B, V);
  for (int dt : {WH_DTYPE_F32, WH_DTYPE_BF16})
    for (int hc : {0, 2 * WH_MAX_WINDOW}) t = std::max(t, ws_layout(B, make_plan(B, V, dt, hc)).total);
  return t;
}

static int set_lds(const void* fn, size_t lds) {
  if (lds <= 65536) return WH_OK;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return fail(WH_EHIP, "hipFuncSetAttribute(%zu bytes LDS) failed: %s", lds, hipGetErrorString(e));
  return WH_OK;
}

template <int DT, int R>
static int launch_slice_t(const SampleKArgs& k, const FastPlan& fp, size_t lds, hipStream_t st) {
  const bool xm = k.B % 8 == 0;
  auto fn = xm ? slice_kernel<DT, R, true> : slice_kernel<DT, R, false>;
  int rc = set_lds((const void*)fn, lds);
  if (rc) return rc;
  const dim3 grid = xm ? dim3(8 * fp.G, k.B / 8) : dim3(fp.G, k.B);
  hipLaunchKernelGGL(fn, grid, dim3(FT), lds, st, (const char*)k.logits, k.hist,
                     (long long)k.row_stride, fp.G, fp.SL, k.V, (int)k.hist_stride, k.hcap > 0 ? 1 : 0, k.hshare, k, fp);
  return WH_OK;
}

// R (16-byte loads per thread) is rounded up to an instantiated value.
static int launch_slice(int dtype, int R, const SampleKArgs& k, const FastPlan& fp, size_t lds, hipStream_t st) {
  if (dtype == WH_DTYPE_BF16) {
    switch (R) {
      case 1: return launch_slice_t<1, 1>(k, fp, lds, st);
      case 2: return launch_slice_t<1, 2>(k, fp, lds, st);
      case 3: return launch_slice_t<1, 3>(k, fp, lds, st);
      case 4: return launch_slice_t<1, 4>(k, fp, lds, st);
      case 5: return launch_slice_t<1, 5>(k, fp, lds, st);
      default: return launch_slice_t<1, 6>(k, fp, lds, st);
    }
  }
  if (R <= 1) return launch_slice_t<0, 1>(k, fp, lds, st);
  if (R <= 2) return launch_slice_t<0, 2>(k, fp, lds, st);
  if (R <= 3) return launch_slice_t<0, 3>(k, fp, lds, st);
  if (R <= 4) return launch_slice_t<0, 4>(k, fp, lds, st);
  if (R <= 6) return launch_slice_t<0, 6>(k, fp, lds, st);
  if (R <= 8) return launch_slice_t<0, 8>(k, fp, lds, st);
  if (R <= 10) return launch_slice_t<0, 10>(k, fp, lds, st);
  return launch_slice_t<0, 12>(k, fp, lds, st);
}

template <int G>
static int launch_merge_t(const SampleKArgs& k, const FastPlan& fp, size_t lds, hipStream_t st) {
  auto fn = merge_kernel<G>;
  int rc = set_lds((const void*)fn, lds);
  if (rc) return rc;
  hipLaunchKernelGGL(fn, dim3(k.B), dim3(MW * 64), lds, st, (const SliceHdr*)fp.hdr, (const int2*)fp.cand, k, fp);
  return WH_OK;
}

// The merge is compiled per slice count (slot -> slice / chunk maps are then
// constants); plans use 1..6 slices.
static int launch_merge(const SampleKArgs& k, const FastPlan& fp, size_t lds, hipStream_t st) {
  switch (fp.G) {
    case 1: return launch_merge_t<1>(k, fp, lds, st);
    case 2: return launch_merge_t<2>(k, fp, lds, st);
    case 3: return launch_merge_t<3>(k, fp, lds, st);
    case 4: return launch_merge_t<4>(k, fp, lds, st);
    case 5: return launch_merge_t<5>(k, fp, lds, st);
    case 6: return launch_merge_t<6>(k, fp, lds, st);
    default: return fail(WH_EINVAL, "no merge kernel for %d slices", fp.G);
  }
}

int launch_sample(const SampleKArgs& k0, const wh_sample_args* p, hipStream_t st) {
  // top-p alone, or no filter: candidates cannot bound the kept set, so the
  // wide exact engine (many workgroups per row) takes the rows
  if (wide_applicable(k0) && p->workspace && p->workspace_bytes >= wide_workspace_bytes(k0.B, k0.V))
    return launch_sample_wide(k0, p, st);
  const int esz = k0.dtype == WH_DTYPE_BF16 ? 2 : 4;
  HostPlan hp = make_plan(k0.B, k0.V, k0.dtype, k0.hcap);
  WsLayout wl = ws_layout(k0.B, hp);
  const bool aligned = ((uintptr_t)k0.logits % 16 == 0) && ((k0.row_stride * esz) % 16 == 0) && (k0.V % hp.ept == 0);
  if (!aligned || !p->workspace || p->workspace_bytes < wl.total || hp.G > GMAX) return launch_sample_exact(k0, st);
  SampleKArgs k = k0;
  FastPlan fp;
  fp.G = hp.G;
  fp.SL = hp.SL;
  fp.cap = hp.cap;
  fp.rule_cap = hp.rule_cap;
  fp.pcap = hp.pcap;
  fp.codes_bytes = hp.codes_bytes;
  char* ws = (char*)p->workspace;
  fp.path = (int*)(ws + wl.path);
  fp.hdr = (SliceHdr*)(ws + wl.hdr);
  fp.cand = (int2*)(ws + wl.cand);
  // the list stays in place under the penalty table of a second bounds pass,
  // when both fit the LDS next to the merge kernel's static arrays
  const size_t pen = penalty_lds_bytes(k), blk = (size_t)hp.G * hp.cap * 8;
  const size_t lst = (size_t)QSPEC * 64 * 8;  // the hot list as value / id arrays
  fp.zpass = (lst + pen <= MERGE_LDS_MAX ? 1 : 0) | (blk + pen <= MERGE_LDS_MAX ? 2 : 0);
  const size_t lds_merge =
      std::max({blk, pen, HOT_LIST_BYTES, (fp.zpass & 1) ? lst + pen : 0, (fp.zpass & 2) ? blk + pen : 0});
  int rc = launch_slice(k.dtype, hp.R, k, fp, hp.lds, st);
  if (rc) return rc;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "slice_kernel launch failed: %s", hipGetErrorString(e));
  rc = launch_merge(k, fp, lds_merge, st);
  if (rc) return rc;
  e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "merge_kernel launch failed: %s", hipGetErrorString(e));
  return WH_OK;
}

}  // namespace wh
