// wh_history.hip -- device-resident token history for the penalty window.
//
// Reference: mlx_lm generate_step keeps every sequence's token history and
// extends it each step before the logits processors read it
// (`tokens = concat([tokens, y])`, driven by stream_generate at
// runtime/deepseek_v4_ssd/generation.py:1465-1475); the MTP loop keeps its own
// list (qwen4_exp.py:947, appended at 1032, 1046, 1143, 1149: the accepted
// drafts, then the next token).  Here the history is an int32 [B, capacity]
// device buffer with per-row lengths, the form wh_sample reads, so a decode
// loop never moves it to the host.
//
// The processors read only the last `context` ids of the history, so a row
// that would overflow its capacity first keeps only its last `keep` ids
// (keep >= every context in use), moved to the front of the row.  The copy
// goes through registers with a barrier between the loads and the stores
// (source and destination overlap).  Amortised cost per appended id is
// keep / (capacity - keep) moved ids.
#include "wh_internal.h"
#include "wh_common.h"

namespace wh {

constexpr int HA_T = 256;
constexpr int HA_E = WH_MAX_WINDOW / HA_T;  // keep <= WH_MAX_WINDOW

__global__ void __launch_bounds__(HA_T) history_append_kernel(int32_t* __restrict__ hist, long long hs,
                                                              int32_t* __restrict__ hist_len, int cap, int keep,
                                                              const int32_t* __restrict__ tokens, int m,
                                                              const int32_t* __restrict__ counts,
                                                              const int32_t* __restrict__ tail) {
  const int b = blockIdx.x, t = threadIdx.x;
  int32_t* row = hist + (size_t)b * hs;
  const int len0 = min(max(hist_len[b], 0), cap);
  const int c = counts ? min(max(counts[b], 0), m) : m;
  const int add = c + (tail ? 1 : 0);
  int len = len0;
  if (len0 + add > cap) {
    // keep + m + 1 <= cap (checked on the host), so the kept ids and the
    // appended ones fit
    const int kk = min(len0, keep);
    int32_t r[HA_E];
#pragma unroll
    for (int j = 0; j < HA_E; ++j) {
      const int i = t + j * HA_T;
      r[j] = i < kk ? row[len0 - kk + i] : 0;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < HA_E; ++j) {
      const int i = t + j * HA_T;
      if (i < kk) row[i] = r[j];
    }
    len = kk;
  }
  for (int i = t; i < c; i += HA_T) row[len + i] = tokens[(size_t)b * m + i];
  if (t == 0) {
    if (tail) row[len + c] = tail[b];
    hist_len[b] = len + add;
  }
}

}  // namespace wh

using namespace wh;

extern "C" int wh_history_append(const wh_history_args* a, void* stream) {
  clear_error();
  if (!a) return fail(WH_EINVAL, "args is NULL");
  if (a->B < 0) return fail(WH_EINVAL, "B must be >= 0, got %d", a->B);
  if (a->m < 0) return fail(WH_EINVAL, "m must be >= 0, got %d", a->m);
  if (a->capacity <= 0) return fail(WH_EINVAL, "capacity must be positive, got %d", a->capacity);
  if (a->history_stride < a->capacity)
    return fail(WH_EINVAL, "history_stride (%lld) must be >= capacity (%d)", (long long)a->history_stride, a->capacity);
  if (a->keep < 0 || a->keep > WH_MAX_WINDOW) return fail(WH_ELIMIT, "keep must be in [0, %d], got %d", WH_MAX_WINDOW, a->keep);
  const long long need = (long long)a->keep + a->m + (a->tail ? 1 : 0);
  if (need > a->capacity)
    return fail(WH_EINVAL, "keep + m%s (%lld) must not exceed capacity (%d)", a->tail ? " + 1" : "", need, a->capacity);
  if (a->B == 0) return WH_OK;
  if (!a->history || !a->history_len) return fail(WH_EINVAL, "history and history_len are required");
  if (a->m > 0 && !a->tokens) return fail(WH_EINVAL, "tokens is NULL with m > 0");
  hipLaunchKernelGGL(history_append_kernel, dim3(a->B), dim3(HA_T), 0, (hipStream_t)stream, a->history,
                     (long long)a->history_stride, a->history_len, a->capacity, a->keep, a->tokens, a->m, a->counts,
                     a->tail);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WH_EHIP, "history_append_kernel launch failed: %s", hipGetErrorString(e));
  return WH_OK;
}
