// wh_common.h -- device helpers shared by the gfx950 token-selection kernels.
//
// Everything here is written for CDNA4 wave64: reductions use 64-lane
// cross-lane shuffles and one LDS slot per wave.  Arithmetic that decides a
// token is either IEEE float32 in a fixed operation order (compiled with
// -ffp-contract=off, so no multiply-add is fused behind our back), or
// integer fixed point (sums are associative, so any parallel order gives the
// same bits as the CPU oracle).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define WH_WAVE 64

namespace wh {

typedef unsigned __int128 u128;

// --------------------------------------------------------------------------
// Contract exponential: floor(2^44 * 2^f * 2^n) with t = fl(d * log2 e) = n+f.
// p(f) ~ 2^f on [0,1] is a degree-6 minimax polynomial (coefficients fitted
// for this library; float32 Horner error <= 0.55 ulp).  Inputs d <= 0;
// t <= -45 and -inf give 0.
// --------------------------------------------------------------------------
// Written without branches (the flushed case computes on t = 0 and is
// selected away), so wave code over many slots stays straight-line.
__device__ __forceinline__ uint64_t exp_fix44(float d) {
  const float L = 0x1.715476p+0f;
  float t = d * L;
  const bool flush = !(t > -45.0f);
  t = (flush || t > 0.0f) ? 0.0f : t;
  float n = floorf(t);
  float f = t - n;
  float p = 0x1.c5417ap-13f;
  p = fmaf(p, f, 0x1.46d64cp-10f);
  p = fmaf(p, f, 0x1.3d0b92p-7f);
  p = fmaf(p, f, 0x1.c68912p-5f);
  p = fmaf(p, f, 0x1.ebfd58p-3f);
  p = fmaf(p, f, 0x1.62e42cp-1f);
  p = fmaf(p, f, 1.0f);
  uint32_t mant = (uint32_t)(p * 8388608.0f);
  int sh = (int)n + 21;
  const uint64_t r = sh >= 0 ? ((uint64_t)mant << sh) : (uint64_t)(mant >> (-sh));
  return flush ? 0ull : r;
}

// 16-byte load of a once-read stream (logits), marked non-temporal: the
// stream then does not displace what the caches hold for the next kernel
// (its code and the workspace lines it reads).
__device__ __forceinline__ uint4 load_stream16(const void* p) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// d / t in float32, correctly rounded, from r = 1.0 / (double)t (rounded to
// double): the double product is within 2^-52 (relative) of d / t, while a
// quotient of two 24-bit significands is never a midpoint between floats and
// lies at least about 2^-49 (relative) from every one, so the product rounds
// to the same float -- a multiply in place of the division sequence.  The
// same holds for zeros, infinities, NaNs and subnormal results.
__device__ __forceinline__ float div_by_recip(float d, double r) { return (float)((double)d * r); }

// float32 mantissa/exponent split: x = M * 2^(e - 24), M a 24-bit integer.
__device__ __forceinline__ uint64_t mant24(float x, int* e) {
  float fr = frexpf(x, e);
  return (uint64_t)ldexpf(fr, 24);
}

// floor(theta * Z) for float32 theta in [0,1] (NaN and negatives give 0,
// larger values clamp to 1), Z < 2^62 (exact).  theta =
// M 2^-s with a 24-bit M and s >= 23, so with Z = Zh 2^32 + Zl the product
// M Z = hi 2^32 + lo (hi = M Zh < 2^54, lo = M Zl < 2^56) is shifted in two
// 64-bit pieces: for s <= 32, hi 2^(32-s) is whole and only lo loses bits;
// beyond, (M Z) >> 32 = hi + (lo >> 32).
__device__ __forceinline__ uint64_t floor_theta_z(float theta, uint64_t Z) {
  if (!(theta > 0.0f)) return 0;
  if (theta > 1.0f) theta = 1.0f;
  int e;
  const uint64_t M = mant24(theta, &e);
  const int s = 24 - e;
  const uint64_t lo = M * (Z & 0xFFFFFFFFull), hi = M * (Z >> 32);
  if (s <= 32) return (hi << (32 - s)) + (lo >> s);
  const uint64_t t = hi + (lo >> 32);
  return s - 32 >= 64 ? 0 : t >> (s - 32);
}

// u in [0,1) -> floor(u * 2^32), clamped; NaN and negatives give 0.
__device__ __forceinline__ uint64_t u32_fix(float u) {
  if (!(u > 0.0f)) return 0;
  if (u >= 1.0f) return 0xFFFFFFFFull;
  return (uint64_t)(u * 4294967296.0f);
}

// Draw target inside a total weight: floor(U * total / 2^32), total < 2^62,
// as U Th + ((U Tl) >> 32) with total = Th 2^32 + Tl (exact: U Th is whole).
__device__ __forceinline__ uint64_t draw_target(float u, uint64_t total) {
  const uint64_t U = u32_fix(u);
  return U * (total >> 32) + ((U * (total & 0xFFFFFFFFull)) >> 32);
}

// Monotone 32-bit key of a float (larger value -> larger key); callers map
// -0 to +0 first so equal floats have equal keys.
__device__ __forceinline__ uint32_t fkey(float v) {
  uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_to_float(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __uint_as_float(u);
}

// Composite orders over (value, id), larger = earlier:
//   order A (top-k): value desc, id asc;  order P (top-p): value desc, id desc.
__device__ __forceinline__ uint64_t comp_a(uint32_t key, int id) {
  return ((uint64_t)key << 18) | (uint64_t)(0x3FFFF - id);
}
__device__ __forceinline__ uint64_t comp_p(uint32_t key, int id) {
  return ((uint64_t)key << 18) | (uint64_t)id;
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// max(a, b, c) as one v_max3_f32, for reductions over loaded logits.
// Written as fmaxf, IEEE mode makes the compiler quiet every operand first
// (one extra v_max_f32 x, x, x each) because bits loaded from memory could
// be signalling NaNs, and keeps the two-operand form.  Logits are never
// signalling NaNs here; the penalty marks are quiet NaNs, which the
// instruction ignores (returning the max of the other operands) exactly as
// fmaxf does.
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// --------------------------------------------------------------------------
// Wave / block reductions (blockDim.x a multiple of 64, <= 1024).
// --------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WH_WAVE));
  return v;
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WH_WAVE);
  return v;
}
__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, WH_WAVE));
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WH_WAVE);
  return v;
}
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WH_WAVE);
  return v;
}

// --------------------------------------------------------------------------
// DPP wave reductions.  All 64 lanes must be active.  Four steps combine each
// lane with a partner inside its row of 16 (quad_perm [1,0,3,2], quad_perm
// [2,3,0,1], row_half_mirror, row_mirror), leaving every lane of a row with
// the row's result; the four row results are read with v_readlane and
// combined, so the value returned is wave uniform.  VALU latency only, no LDS.
// --------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ uint32_t dpp32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t lane_u32(uint32_t x, int l) { return (uint32_t)__builtin_amdgcn_readlane((int)x, l); }
__device__ __forceinline__ uint64_t lane_u64(uint64_t x, int l) {
  return ((uint64_t)lane_u32((uint32_t)(x >> 32), l) << 32) | lane_u32((uint32_t)x, l);
}
template <typename Op>
__device__ __forceinline__ uint32_t dpp_reduce_u32(uint32_t x, Op op) {
  x = op(x, dpp32<0xB1>(x));
  x = op(x, dpp32<0x4E>(x));
  x = op(x, dpp32<0x141>(x));
  x = op(x, dpp32<0x140>(x));
  return op(op(lane_u32(x, 0), lane_u32(x, 16)), op(lane_u32(x, 32), lane_u32(x, 48)));
}
#define WH_DPP64_STEP(C)                                                                        \
  {                                                                                             \
    const uint64_t y_ = ((uint64_t)dpp32<C>((uint32_t)(x >> 32)) << 32) | dpp32<C>((uint32_t)x); \
    x = op(x, y_);                                                                              \
  }
template <typename Op>
__device__ __forceinline__ uint64_t dpp_reduce_u64(uint64_t x, Op op) {
  WH_DPP64_STEP(0xB1)
  WH_DPP64_STEP(0x4E)
  WH_DPP64_STEP(0x141)
  WH_DPP64_STEP(0x140)
  return op(op(lane_u64(x, 0), lane_u64(x, 16)), op(lane_u64(x, 32), lane_u64(x, 48)));
}
#undef WH_DPP64_STEP
__device__ __forceinline__ int wsum_i(int v) {
  return (int)dpp_reduce_u32((uint32_t)v, [](uint32_t a, uint32_t b) { return a + b; });
}
__device__ __forceinline__ uint64_t wsum_u64(uint64_t v) {
  return dpp_reduce_u64(v, [](uint64_t a, uint64_t b) { return a + b; });
}
__device__ __forceinline__ float wmax_f(float v) {
  return __uint_as_float(dpp_reduce_u32(__float_as_uint(v), [](uint32_t a, uint32_t b) {
    return __float_as_uint(max3_raw(__uint_as_float(a), __uint_as_float(b), __uint_as_float(b)));
  }));
}
__device__ __forceinline__ int wmin_i(int v) {
  return (int)dpp_reduce_u32((uint32_t)v, [](uint32_t a, uint32_t b) { return (uint32_t)min((int)a, (int)b); });
}
__device__ __forceinline__ int wmax_i(int v) {
  return (int)dpp_reduce_u32((uint32_t)v, [](uint32_t a, uint32_t b) { return (uint32_t)max((int)a, (int)b); });
}
__device__ __forceinline__ uint32_t wmin_u32(uint32_t v) {
  return dpp_reduce_u32(v, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}
__device__ __forceinline__ uint32_t wmax_u32(uint32_t v) {
  return dpp_reduce_u32(v, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}
__device__ __forceinline__ double wsum_f64(double v) {
  return __longlong_as_double((long long)dpp_reduce_u64((uint64_t)__double_as_longlong(v), [](uint64_t a, uint64_t b) {
    return (uint64_t)__double_as_longlong(__longlong_as_double((long long)a) + __longlong_as_double((long long)b));
  }));
}
// K independent u64 sums reduced together: the DPP steps of the K chains
// interleave, so their latencies overlap.
template <int K>
__device__ __forceinline__ void wsum_u64_k(uint64_t (&v)[K]) {
#define WH_DPPK_STEP(C)                                                                              \
  _Pragma("unroll") for (int k_ = 0; k_ < K; ++k_) {                                                 \
    const uint64_t y_ = ((uint64_t)dpp32<C>((uint32_t)(v[k_] >> 32)) << 32) | dpp32<C>((uint32_t)v[k_]); \
    v[k_] += y_;                                                                                     \
  }
  WH_DPPK_STEP(0xB1)
  WH_DPPK_STEP(0x4E)
  WH_DPPK_STEP(0x141)
  WH_DPPK_STEP(0x140)
#undef WH_DPPK_STEP
#pragma unroll
  for (int k = 0; k < K; ++k) v[k] = (lane_u64(v[k], 0) + lane_u64(v[k], 16)) + (lane_u64(v[k], 32) + lane_u64(v[k], 48));
}

// Inclusive prefix sum over the 64 lanes (lane order), all lanes active.
// Hillis-Steele inside each row of 16 (row_shr 1, 2, 4, 8), then
// row_bcast:15 carries row 0 into row 1 and row 2 into row 3, and
// row_bcast:31 carries rows 0-1 into rows 2-3.  Lanes a step does not
// write (no source lane, or a row outside its row mask) add 0.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp32z(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROWS, 0xF, true);
}
__device__ __forceinline__ uint64_t wscan_incl_u64(uint64_t x) {
#define WH_SCAN_STEP(C, ROWS)                                                                                \
  {                                                                                                           \
    const uint64_t y_ = ((uint64_t)dpp32z<C, ROWS>((uint32_t)(x >> 32)) << 32) | dpp32z<C, ROWS>((uint32_t)x); \
    x += y_;                                                                                                  \
  }
  WH_SCAN_STEP(0x111, 0xF)
  WH_SCAN_STEP(0x112, 0xF)
  WH_SCAN_STEP(0x114, 0xF)
  WH_SCAN_STEP(0x118, 0xF)
  WH_SCAN_STEP(0x142, 0xA)
  WH_SCAN_STEP(0x143, 0xC)
#undef WH_SCAN_STEP
  return x;
}

__device__ __forceinline__ uint32_t wscan_incl_u32(uint32_t x) {
  x += dpp32z<0x111, 0xF>(x);
  x += dpp32z<0x112, 0xF>(x);
  x += dpp32z<0x114, 0xF>(x);
  x += dpp32z<0x118, 0xF>(x);
  x += dpp32z<0x142, 0xA>(x);
  x += dpp32z<0x143, 0xC>(x);
  return x;
}

// Number of lanes (of the active ones) where p holds; wave uniform.
__device__ __forceinline__ int ballot_count(bool p) { return (int)__popcll(__ballot(p)); }

// Reductions across the block through a 16-slot LDS scratch (one per wave).
template <typename T, typename Op>
__device__ __forceinline__ T block_reduce(T v, T* scratch, Op op, T ident) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = op(v, __shfl_xor(v, o, WH_WAVE));
  __syncthreads();
  if (lane == 0) scratch[w] = v;
  __syncthreads();
  T r = ident;
  for (int i = 0; i < nw; ++i) r = op(r, scratch[i]);
  return r;
}

struct OpMaxF { __device__ float operator()(float a, float b) const { return fmaxf(a, b); } };
struct OpMinI { __device__ int operator()(int a, int b) const { return min(a, b); } };
struct OpSumI { __device__ int operator()(int a, int b) const { return a + b; } };
struct OpSumU64 { __device__ uint64_t operator()(uint64_t a, uint64_t b) const { return a + b; } };
struct OpSumF64 { __device__ double operator()(double a, double b) const { return a + b; } };
struct OpMaxU32 { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; } };
struct OpMinU64 { __device__ uint64_t operator()(uint64_t a, uint64_t b) const { return a < b ? a : b; } };
struct OpMaxU64 { __device__ uint64_t operator()(uint64_t a, uint64_t b) const { return a > b ? a : b; } };

// Exclusive prefix sum of u64 across the block (thread order); returns the
// exclusive prefix and writes the block total.
__device__ __forceinline__ uint64_t block_exclusive_scan_u64(uint64_t v, uint64_t* scratch, uint64_t* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  uint64_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    uint64_t y = __shfl_up(x, o, WH_WAVE);
    if (lane >= o) x += y;
  }
  __syncthreads();
  if (lane == 63) scratch[w] = x;
  __syncthreads();
  uint64_t before = 0, tot = 0;
  for (int i = 0; i < nw; ++i) {
    uint64_t s = scratch[i];
    if (i < w) before += s;
    tot += s;
  }
  *total = tot;
  return before + x - v;
}

}  // namespace wh
