// wh_draft.hip -- the DSpark draft step's Markov bias on gfx950.
//
// Reference: runtime/deepseek_v4_ssd/dspark.py:157-165 (_MarkovHead) and
// dspark.py:319-330 / deepseek_v41/dspark.py:128-137 (the draft loop):
//   embedding = markov_w1(previous)                       # [rank] row gather
//   bias      = markov_w2(embedding.astype(float32))      # [V] = W2 @ e
//   logits    = base_logits[:, position] + bias
// followed by sampling_logprobs and the draw, which are wh_sample's chain
// WH_CHAIN_WHALLM.  The previous token is read from device memory (the
// previous position's wh_sample output), so a whole draft block runs with no
// host round trip.
//
// The product W2 @ e is a GEMV over V x rank weights (66 MB in bf16 at
// V = 129,280, rank 256): HBM-bound, one pass over W2.  Each half-wave owns
// one row: lane c holds the 8 rank entries 8c .. 8c+7 (one 16-byte bf16
// load, two for float32), forms their partial sum with a chain of fused
// multiply-adds, and a 5-step butterfly over the 32 lanes sums the row.
// That fixed order is the contract the CPU oracle follows, so the logits are
// bit-identical to it.
#include "wh_internal.h"
#include "wh_common.h"

namespace wh {

constexpr int MK_T = 256;       // threads per workgroup
constexpr int MK_PAIRS = 8;     // row pairs per wave (all loads issued first)

template <int DT>
__global__ void __launch_bounds__(MK_T) markov_kernel(const float* __restrict__ base, const void* __restrict__ embed,
                                                      const void* __restrict__ proj, const int32_t* __restrict__ prev,
                                                      float* __restrict__ out, int V, int rank) {
  constexpr int ESZ = DT ? 2 : 4;
  constexpr int NLD = DT ? 1 : 2;  // 16-byte loads per 8 entries
  const int lane = threadIdx.x & 63, half = lane >> 5, c = lane & 31;
  const int wave = (blockIdx.x * MK_T + threadIdx.x) >> 6;
  const bool active = c < rank / 8;
  const int p0 = min(max(*prev, 0), V - 1);
  // the lane's 8 embedding entries, widened exactly to float32
  float e[8];
  {
    const char* er = (const char*)embed + ((size_t)p0 * rank + 8 * (active ? c : 0)) * ESZ;
    uint4 q[NLD];
#pragma unroll
    for (int k = 0; k < NLD; ++k) q[k] = *(const uint4*)(er + 16 * k);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (DT) {
        const uint32_t w = i < 2 ? q[0].x : i < 4 ? q[0].y : i < 6 ? q[0].z : q[0].w;
        e[i] = __uint_as_float((i & 1) ? (w & 0xFFFF0000u) : (w << 16));
      } else {
        const uint4& v = q[i >> 2];
        const int j = i & 3;
        e[i] = __uint_as_float(j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w);
      }
      if (!active) e[i] = 0.0f;
    }
  }
  // every weight load first (rows past V read row 0 and are not written)
  uint4 w[MK_PAIRS][NLD];
  int rows[MK_PAIRS];
#pragma unroll
  for (int t = 0; t < MK_PAIRS; ++t) {
    const int v = 2 * (wave * MK_PAIRS + t) + half;
    rows[t] = v;
    const int vr = v < V ? v : 0;
    const char* wr = (const char*)proj + ((size_t)vr * rank + 8 * (active ? c : 0)) * ESZ;
#pragma unroll
    for (int k = 0; k < NLD; ++k) w[t][k] = load_stream16(wr + 16 * k);
  }
#pragma unroll
  for (int t = 0; t < MK_PAIRS; ++t) {
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float wi;
      if (DT) {
        const uint32_t x = i < 2 ? w[t][0].x : i < 4 ? w[t][0].y : i < 6 ? w[t][0].z : w[t][0].w;
        wi = __uint_as_float((i & 1) ? (x & 0xFFFF0000u) : (x << 16));
      } else {
        const uint4& v = w[t][i >> 2];
        const int j = i & 3;
        wi = __uint_as_float(j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w);
      }
      p = __builtin_fmaf(wi, e[i], p);
    }
    if (!active) p = 0.0f;
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) p = p + __shfl_xor(p, off, 64);
    const int v = rows[t];
    if (c == 0 && v < V) out[v] = base[v] + p;
  }
}

}  // namespace wh

using namespace wh;

extern "C" int wh_markov_logits(const wh_markov_args* a, void* stream) {
  clear_error();
  if (!a) return fail(WH_EINVAL, "args is NULL");
  if (a->dtype != WH_DTYPE_F32 && a->dtype != WH_DTYPE_BF16) return fail(WH_EINVAL, "dtype must be WH_DTYPE_F32 or WH_DTYPE_BF16");
  if (a->V <= 0 || a->V > WH_MAX_VOCAB) return fail(WH_ELIMIT, "V must be in [1, %d], got %d", WH_MAX_VOCAB, a->V);
  if (a->rank <= 0 || a->rank > 256 || a->rank % 8 != 0)
    return fail(WH_EINVAL, "rank must be a positive multiple of 8, at most 256, got %d", a->rank);
  if (!a->base || !a->embed || !a->proj || !a->prev || !a->logits_out) return fail(WH_EINVAL, "a pointer is NULL");
  if ((uintptr_t)a->embed % 16 || (uintptr_t)a->proj % 16) return fail(WH_EINVAL, "weights must be 16-byte aligned");
  const int pairs = (a->V + 1) / 2;
  const int waves = (pairs + MK_PAIRS - 1) / MK_PAIRS;
  const int blocks = (waves * 64 + MK_T - 1) / MK_T;
  hipStream_t st = (hipStream_t)stream;
  if (a->dtype == WH_DTYPE_BF16)
    hipLaunchKernelGGL(markov_kernel<1>, dim3(blocks), dim3(MK_T), 0, st, a->base, a->embed, a->proj, a->prev,
                       a->logits_out, a->V, a->rank);
  else
    hipLaunchKernelGGL(markov_kernel<0>, dim3(blocks), dim3(MK_T), 0, st, a->base, a->embed, a->proj, a->prev,
                       a->logits_out, a->V, a->rank);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "markov_kernel launch failed: %s", hipGetErrorString(e));
  return WH_OK;
}
