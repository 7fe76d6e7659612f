// wh_lmhead.hip -- the LM head (logits = x @ W^T) on gfx950 MFMA, with a
// greedy token-selection epilogue.
//
// Reference: the logits the token selection consumes come from the LM head,
// runtime/deepseek_v4_ssd/model.py:716 (`model.lm_head(output)`),
// dspark.py:313 (`main_model.lm_head(self.norm(head_hidden))`) and
// qwen4_exp.py:960-961; with temperature 0 the selection is
// argmax (mlx: lowest index among equal maxima, dspark.py:326,
// generation.py's make_sampler(temp=0)).
//
// Shapes: x [M, K] bf16 (M <= 64 decode rows), W [V, K] bf16 (the nn.Linear
// weight, row v is vocabulary entry v), K a multiple of 64.  At decode sizes
// the product is bound by the one pass over W (V*K*2 bytes: 778 MB for
// V = 151,936, K = 2560), so the kernel is built to stream W:
//   * a workgroup of NWV waves owns 32 * NWV vocabulary rows; per step it
//     reads a 64-k slab of them with coalesced 16-byte loads (consecutive
//     lanes on consecutive bytes of a row) and stages it, with the same k of
//     x, through LDS; the next slab is in registers while this one computes;
//   * each wave multiplies its 32 rows by every x row (one or two 32-row
//     blocks) with v_mfma_f32_32x32x16_bf16, float32 accumulation; the
//     fragments come from LDS, so every W byte crosses HBM once;
//   * x is re-read from L2 by every workgroup, so with two x row blocks the
//     workgroup is 8 waves (256 rows: half the x traffic of 4 waves); with
//     one block, 8 waves when that grid spreads evenly over the CUs, else 4
//     (more workgroups, better balance).
// (Loading MFMA fragments straight from memory -- 32 rows per load
// instruction -- ran at 1.1-2.1 TB/s; the staged form at 3.4-6.5 TB/s.)
// Epilogues: (a) the float32 logits, (b) greedy: per row the largest
// (value, lowest index) key of the workgroup's 128 or 256 columns, written to a
// partials buffer; wh_lmhead_greedy's second kernel reduces them per row.
// The logits never reach HBM on the greedy path, and the two epilogues see
// identical accumulator values, so the fused tokens equal the argmax of the
// unfused logits.
#include <atomic>

#include "wh_internal.h"
#include "wh_common.h"

namespace wh {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int LM_KS = 64;          // k per pipeline step
constexpr int LM_MIN_COLS = 128;   // vocabulary rows per workgroup, at least (4 waves)

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& q) {
  bf16x8 r;
  __builtin_memcpy(&r, &q, 16);
  return r;
}

// LDS tiles of one pipeline step: KS k of the workgroup's 32 * NWV W rows
// and of the 32 * MB x rows, rows padded by 16 bytes (fragment reads of 32
// rows at one k then fall on distinct bank groups).
template <int MB, int KS, int NWV>
struct LmSmem {
  static constexpr int RS = KS * 2 + 16;
  char w[32 * NWV * RS];
  char x[32 * MB * RS];
};

// Accumulate x[rows] . W[cols] over K for the wave's 32 columns
// (row0 + 32 * wave ..) and all 32 * MB x rows.  Per step the workgroup
// loads KS k of its 32 * NWV W rows with coalesced 16-byte loads (KS * 2 / 16
// lanes per row, consecutive lanes on consecutive bytes) and the same k of
// x, stores both to LDS, and each wave reads its MFMA fragments from there.
// The next step's loads are in registers while the current step computes.
// Two accumulators per row block (the two 16-k halves of every 32 k) keep
// consecutive MFMAs independent; the result is their sum.
template <int MB, int KS, int NWV>
__device__ __forceinline__ void lm_tile(const char* __restrict__ x, const char* __restrict__ w, int M, int K, int V,
                                        int row0, LmSmem<MB, KS, NWV>& sm, f32x16 (&res)[MB]) {
  constexpr int RS = LmSmem<MB, KS, NWV>::RS;
  constexpr int LPR = KS * 2 / 16;          // lanes per row
  constexpr int WR = 64 * NWV / LPR;        // rows per load round
  constexpr int NW = 32 * NWV / WR;         // W load rounds
  constexpr int XR = 32 * MB;
  constexpr int NX = (XR + WR - 1) / WR;    // x load rounds
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6, h = lane >> 5, r = lane & 31;
  const int lr = t / LPR, ch = t % LPR;
  f32x16 acc[MB], acc2[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[mb][i] = acc2[mb][i] = 0.0f;
  uint4 sw[NW], sx[NX];
  // columns past V load the last row and x rows past M the last x row;
  // neither is stored
  auto load = [&](int s) {
#pragma unroll
    for (int j = 0; j < NW; ++j)
      sw[j] = load_stream16(w + ((size_t)min(row0 + j * WR + lr, V - 1) * K + (size_t)s * KS) * 2 + ch * 16);
#pragma unroll
    for (int j = 0; j < NX; ++j)
      sx[j] = *(const uint4*)(x + ((size_t)min(j * WR + lr, M - 1) * K + (size_t)s * KS) * 2 + ch * 16);
  };
  auto store = [&]() {
#pragma unroll
    for (int j = 0; j < NW; ++j) *(uint4*)(sm.w + (j * WR + lr) * RS + ch * 16) = sw[j];
#pragma unroll
    for (int j = 0; j < NX; ++j)
      if (j * WR + lr < XR) *(uint4*)(sm.x + (j * WR + lr) * RS + ch * 16) = sx[j];
  };
  const int ns = K / KS;
  load(0);
  store();
  __syncthreads();
  for (int s = 0; s < ns; ++s) {
    if (s + 1 < ns) load(s + 1);
    const char* lw = sm.w + (32 * wv + r) * RS;
#pragma unroll
    for (int q = 0; q < KS / 32; ++q) {
      const uint4 wa = *(const uint4*)(lw + (32 * q + 8 * h) * 2);
      const uint4 wb = *(const uint4*)(lw + (32 * q + 16 + 8 * h) * 2);
      uint4 xa[MB], xb[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const char* lx = sm.x + (32 * mb + r) * RS + (32 * q + 8 * h) * 2;
        xa[mb] = *(const uint4*)lx;
        xb[mb] = *(const uint4*)(lx + 32);
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(xa[mb]), as_bf16x8(wa), acc[mb], 0, 0, 0);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        acc2[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(xb[mb]), as_bf16x8(wb), acc2[mb], 0, 0, 0);
    }
    __syncthreads();
    if (s + 1 < ns) store();
    __syncthreads();
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) res[mb] = acc[mb] + acc2[mb];
}

// Accumulator element i of lane l is row 8 (i / 4) + 4 (l / 32) + i % 4 of
// the 32-row block, column l % 32.
__device__ __forceinline__ int acc_row(int i, int lane) { return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3); }

template <int MB, int KS, int NWV>
__global__ void __launch_bounds__(64 * NWV) lmhead_logits_kernel(const char* __restrict__ x, const char* __restrict__ w,
                                                                 float* __restrict__ out, long long ldo, int M, int K,
                                                                 int V) {
  __shared__ __align__(16) LmSmem<MB, KS, NWV> sm;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int col0 = blockIdx.x * 32 * NWV + wv * 32;
  f32x16 acc[MB];
  lm_tile<MB, KS, NWV>(x, w, M, K, V, blockIdx.x * 32 * NWV, sm, acc);
  const int col = col0 + (lane & 31);
  if (col >= V) return;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = 32 * mb + acc_row(i, lane);
      if (row < M) out[(size_t)row * ldo + col] = acc[mb][i];
    }
}

// Greedy key: larger value first, then lower index; 0 is below every key.
__device__ __forceinline__ uint64_t greedy_key(float v, int col) {
  return ((uint64_t)fkey(v + 0.0f) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)col);
}

// Per row, the largest key of the workgroup's columns into red[wave][row]:
// each wave writes its 32 x 32 block of each row block to its own LDS region
// (the tile loop's buffers, free after its final barrier; rows 33 floats
// apart), then lane r < 32 scans row r.  (Reducing 64-bit keys across lanes
// with shuffles cost more than the logits' store.)
template <int MB, int KS, int NWV>
__device__ __forceinline__ void lm_row_keys(const f32x16 (&acc)[MB], LmSmem<MB, KS, NWV>& sm, uint64_t (*red)[64],
                                            int col0, int V) {
  static_assert(sizeof(sm.w) >= NWV * 32 * 33 * sizeof(float), "key transpose region");
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  float* reg = (float*)sm.w + wv * (32 * 33);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
    for (int i = 0; i < 16; ++i) reg[acc_row(i, lane) * 33 + (lane & 31)] = acc[mb][i];
    __syncthreads();
    if (lane < 32) {
      uint64_t k = 0;
#pragma unroll 8
      for (int c = 0; c < 32; ++c) {
        const uint64_t y = col0 + c < V ? greedy_key(reg[lane * 33 + c], col0 + c) : 0;
        k = y > k ? y : k;
      }
      red[wv][32 * mb + lane] = k;
    }
    __syncthreads();
  }
}

template <int MB, int KS, int NWV>
__global__ void __launch_bounds__(64 * NWV) lmhead_greedy_kernel(const char* __restrict__ x, const char* __restrict__ w,
                                                                 uint64_t* __restrict__ part, int M, int K, int V) {
  __shared__ __align__(16) LmSmem<MB, KS, NWV> sm;
  __shared__ uint64_t red[NWV][64];
  const int wv = threadIdx.x >> 6;
  f32x16 acc[MB];
  lm_tile<MB, KS, NWV>(x, w, M, K, V, blockIdx.x * 32 * NWV, sm, acc);
  lm_row_keys<MB, KS, NWV>(acc, sm, red, blockIdx.x * 32 * NWV + wv * 32, V);
  if (threadIdx.x < 32 * MB) {
    const int row = threadIdx.x;
    uint64_t k = red[0][row];
#pragma unroll
    for (int q = 1; q < NWV; ++q) k = red[q][row] > k ? red[q][row] : k;
    if (row < M) part[(size_t)row * gridDim.x + blockIdx.x] = k;
  }
}

// The logits, plus each row's largest key over the workgroup's columns
// merged (atomic max) into keys[row * G + slice] of the wide sampler, whose
// slices (SL entries, a multiple of 32 * NWV) each hold whole workgroups.
template <int MB, int KS, int NWV>
__global__ void __launch_bounds__(64 * NWV) lmhead_slicemax_kernel(const char* __restrict__ x,
                                                                   const char* __restrict__ w,
                                                                   float* __restrict__ out, long long ldo, int M,
                                                                   int K, int V, uint64_t* __restrict__ keys, int G,
                                                                   int SL) {
  __shared__ __align__(16) LmSmem<MB, KS, NWV> sm;
  __shared__ uint64_t red[NWV][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int col0 = blockIdx.x * 32 * NWV + wv * 32;
  f32x16 acc[MB];
  lm_tile<MB, KS, NWV>(x, w, M, K, V, blockIdx.x * 32 * NWV, sm, acc);
  const int col = col0 + (lane & 31);
  if (col < V) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = 32 * mb + acc_row(i, lane);
        if (row < M) out[(size_t)row * ldo + col] = acc[mb][i];
      }
  }
  lm_row_keys<MB, KS, NWV>(acc, sm, red, col0, V);
  if (threadIdx.x < 32 * MB) {
    const int row = threadIdx.x;
    uint64_t k = red[0][row];
#pragma unroll
    for (int q = 1; q < NWV; ++q) k = red[q][row] > k ? red[q][row] : k;
    if (row < M && k) atomicMax((unsigned long long*)&keys[(size_t)row * G + blockIdx.x * 32 * NWV / SL],
                                (unsigned long long)k);
  }
}

// One workgroup per row: the largest key over the row's partials.
__global__ void __launch_bounds__(256) lmhead_greedy_final(const uint64_t* __restrict__ part, int nwg,
                                                           int32_t* __restrict__ tokens) {
  __shared__ uint64_t red[4];
  const int row = blockIdx.x;
  uint64_t k = 0;
  for (int i = threadIdx.x; i < nwg; i += 256) {
    const uint64_t y = part[(size_t)row * nwg + i];
    k = y > k ? y : k;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint64_t y = __shfl_xor(k, o, 64);
    k = y > k ? y : k;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = k;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t best = red[0];
    for (int q = 1; q < 4; ++q) best = red[q] > best ? red[q] : best;
    tokens[row] = (int32_t)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFu));
  }
}

static int lm_check(const wh_lmhead_args* a) {
  if (!a) return fail(WH_EINVAL, "args is NULL");
  if (a->M < 0 || a->M > WH_LMHEAD_MAX_ROWS) return fail(WH_ELIMIT, "M must be in [0, %d], got %d", WH_LMHEAD_MAX_ROWS, a->M);
  if (a->V <= 0 || a->V > WH_MAX_VOCAB) return fail(WH_ELIMIT, "V must be in [1, %d], got %d", WH_MAX_VOCAB, a->V);
  if (a->K <= 0 || a->K % 64 != 0) return fail(WH_EINVAL, "K must be a positive multiple of 64, got %d", a->K);
  if (!a->x || !a->weight) return fail(WH_EINVAL, "x and weight are required");
  if ((uintptr_t)a->x % 16 || (uintptr_t)a->weight % 16) return fail(WH_EINVAL, "x and weight must be 16-byte aligned");
  return WH_OK;
}

// Workgroups of a launch (vocabulary rows per workgroup: 32 * NWV); the
// greedy partials are sized for the narrowest workgroup.
static int lm_blocks(int V, int cols) { return (V + cols - 1) / cols; }

// Compute units of the current device, read once per device.
static int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Waves per workgroup with one x row block (M <= 32).  The grid is a few
// workgroups per CU, all streaming W at once; a workgroup count that leaves
// the last round on the CUs part-filled lets some CUs run on alone.  Eight
// waves (256 vocabulary rows, half the x re-reads per W byte of four) when
// their grid fills at least 95 % of its rounds, else four (twice as many,
// finer workgroups).  Measured on 256 CUs at K = 2560-7168: V = 129,280
// (505 workgroups of 8 waves: 99 % of two rounds) runs 4-13 % faster on 8
// waves; V = 151,936 (594: 77 % of three) 7-15 % slower, so it keeps 4
// (1,187: 93 % of five).
static int lm_waves_one_block(int V) {
  const int cu = device_cus();
  const int n = lm_blocks(V, 256);
  const int rounds = (n + cu - 1) / cu;
  return (double)n >= 0.95 * rounds * cu ? 8 : 4;
}

}  // namespace wh

using namespace wh;

extern "C" int wh_lmhead_logits(const wh_lmhead_args* a, void* stream) {
  clear_error();
  int rc = lm_check(a);
  if (rc) return rc;
  if (a->M == 0) return WH_OK;
  if (!a->logits_out) return fail(WH_EINVAL, "logits_out is required");
  if (a->logits_stride < a->V) return fail(WH_EINVAL, "logits_stride (%lld) must be >= V (%d)", (long long)a->logits_stride, a->V);
  hipStream_t st = (hipStream_t)stream;
  const char *x = (const char*)a->x, *w = (const char*)a->weight;
  const long long ldo = a->logits_stride;
  // one x row block: 4 or 8 waves (128 or 256 rows); two: 8 waves
  if (a->M <= 32 && lm_waves_one_block(a->V) == 8)
    hipLaunchKernelGGL((lmhead_logits_kernel<1, LM_KS, 8>), dim3(lm_blocks(a->V, 256)), dim3(512), 0, st, x, w,
                       a->logits_out, ldo, a->M, a->K, a->V);
  else if (a->M <= 32)
    hipLaunchKernelGGL((lmhead_logits_kernel<1, LM_KS, 4>), dim3(lm_blocks(a->V, 128)), dim3(256), 0, st, x, w,
                       a->logits_out, ldo, a->M, a->K, a->V);
  else
    hipLaunchKernelGGL((lmhead_logits_kernel<2, LM_KS, 8>), dim3(lm_blocks(a->V, 256)), dim3(512), 0, st, x, w,
                       a->logits_out, ldo, a->M, a->K, a->V);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "lmhead_logits_kernel launch failed: %s", hipGetErrorString(e));
  return WH_OK;
}

extern "C" size_t wh_lmhead_greedy_workspace_bytes(int32_t M, int32_t V) {
  if (M <= 0 || V <= 0) return 0;
  return (size_t)M * lm_blocks(V, LM_MIN_COLS) * sizeof(uint64_t);
}

extern "C" int wh_lmhead_greedy(const wh_lmhead_args* a, void* stream) {
  clear_error();
  int rc = lm_check(a);
  if (rc) return rc;
  if (a->M == 0) return WH_OK;
  if (!a->tokens) return fail(WH_EINVAL, "tokens is required");
  const size_t need = (size_t)a->M * lm_blocks(a->V, LM_MIN_COLS) * sizeof(uint64_t);
  if (!a->workspace || a->workspace_bytes < need)
    return fail(WH_EINVAL, "workspace must hold wh_lmhead_greedy_workspace_bytes(M, V) = %zu bytes", need);
  if ((uintptr_t)a->workspace % 8) return fail(WH_EINVAL, "workspace must be 8-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  uint64_t* part = (uint64_t*)a->workspace;
  const char *x = (const char*)a->x, *w = (const char*)a->weight;
  int nwg;
  if (a->M <= 32 && lm_waves_one_block(a->V) == 8) {
    nwg = lm_blocks(a->V, 256);
    hipLaunchKernelGGL((lmhead_greedy_kernel<1, LM_KS, 8>), dim3(nwg), dim3(512), 0, st, x, w, part, a->M, a->K, a->V);
  } else if (a->M <= 32) {
    nwg = lm_blocks(a->V, 128);
    hipLaunchKernelGGL((lmhead_greedy_kernel<1, LM_KS, 4>), dim3(nwg), dim3(256), 0, st, x, w, part, a->M, a->K, a->V);
  } else {
    nwg = lm_blocks(a->V, 256);
    hipLaunchKernelGGL((lmhead_greedy_kernel<2, LM_KS, 8>), dim3(nwg), dim3(512), 0, st, x, w, part, a->M, a->K, a->V);
  }
  hipLaunchKernelGGL(lmhead_greedy_final, dim3(a->M), dim3(256), 0, st, (const uint64_t*)part, nwg, a->tokens);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "lmhead greedy launch failed: %s", hipGetErrorString(e));
  return WH_OK;
}

extern "C" int wh_lmhead_sample(const wh_lmhead_args* lm, const wh_sample_args* sp, void* stream) {
  clear_error();
  int rc = lm_check(lm);
  if (rc) return rc;
  if (!sp) return fail(WH_EINVAL, "sample args is NULL");
  if (lm->M == 0) return WH_OK;
  if (!lm->logits_out) return fail(WH_EINVAL, "logits_out is required (the sampler reads the logits)");
  if (lm->logits_stride < lm->V)
    return fail(WH_EINVAL, "logits_stride (%lld) must be >= V (%d)", (long long)lm->logits_stride, lm->V);
  wh_sample_args s = *sp;
  s.logits = lm->logits_out;
  s.dtype = WH_DTYPE_F32;
  s.B = lm->M;
  s.V = lm->V;
  s.row_stride = lm->logits_stride;
  SampleKArgs k;
  rc = prepare_sample(&s, &k, true);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  // rows the wide sampler takes, without penalties (the epilogue sees the
  // raw logits) and with one temperature: the product writes their slice
  // maxima, and the sampler starts from its histogram step
  const bool fuse = wide_applicable(k) && k.hcap == 0 && !k.T_rows && s.workspace &&
                    s.workspace_bytes >= wide_workspace_bytes(k.B, k.V);
  if (!fuse) {
    rc = wh_lmhead_logits(lm, stream);
    if (rc) return rc;
    if (!s.tokens && !s.logprobs_out && !s.kept_count) return WH_OK;
    return launch_sample(k, &s, st);
  }
  uint64_t* keys = nullptr;
  int G = 0, SL = 0;
  rc = wide_keys_prepare(k, s.workspace, st, &keys, &G, &SL);
  if (rc) return rc;
  const char *x = (const char*)lm->x, *w = (const char*)lm->weight;
  const long long ldo = lm->logits_stride;
  if (lm->M <= 32 && lm_waves_one_block(lm->V) == 8)
    hipLaunchKernelGGL((lmhead_slicemax_kernel<1, LM_KS, 8>), dim3(lm_blocks(lm->V, 256)), dim3(512), 0, st, x, w,
                       lm->logits_out, ldo, lm->M, lm->K, lm->V, keys, G, SL);
  else if (lm->M <= 32)
    hipLaunchKernelGGL((lmhead_slicemax_kernel<1, LM_KS, 4>), dim3(lm_blocks(lm->V, 128)), dim3(256), 0, st, x, w,
                       lm->logits_out, ldo, lm->M, lm->K, lm->V, keys, G, SL);
  else
    hipLaunchKernelGGL((lmhead_slicemax_kernel<2, LM_KS, 8>), dim3(lm_blocks(lm->V, 256)), dim3(512), 0, st, x, w,
                       lm->logits_out, ldo, lm->M, lm->K, lm->V, keys, G, SL);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "lmhead_slicemax_kernel launch failed: %s", hipGetErrorString(e));
  return launch_sample_wide_from_keys(k, &s, st);
}
