// wh_internal.h -- host/device structures shared by the library's sources.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "wh_sample.h"

namespace wh {

// Kernel-side view of wh_sample_args (passed by value).
struct SampleKArgs {
  const void* logits;
  int dtype, B, V, chain;
  long long row_stride;
  const int32_t* hist;
  long long hist_stride;
  const int32_t* hist_len;
  int hshare;  // logits rows per history row (>= 1)
  const float* u;
  double T, top_p, min_p;
  int top_k;
  float min_p_log;  // fl32(ln(min_p)) computed on the host for the scalar min_p
  const double* T_rows;
  const double* top_p_rows;
  const double* min_p_rows;
  const int32_t* top_k_rows;
  float rep, pres, freq;
  int rep_ctx, pres_ctx, freq_ctx;
  int32_t* tokens;
  int32_t* kept;
  float* out_rows;
  int out_mode;
  int hcap;   // penalty hash capacity (power of two), 0 = no penalties
  int hlog2;
  void* ws;   // workspace
  size_t ws_bytes;
};

int fail(int code, const char* fmt, ...);
void clear_error();
int prepare_sample(const wh_sample_args* p, SampleKArgs* k, bool need_draw);
size_t penalty_lds_bytes(const SampleKArgs& k);
size_t sample_workspace_bytes(int B, int V);
int launch_sample(const SampleKArgs& k, const wh_sample_args* p, hipStream_t st);
int launch_sample_exact(const SampleKArgs& k, hipStream_t st);
bool wide_applicable(const SampleKArgs& k);
size_t wide_workspace_bytes(int B, int V);
int launch_sample_wide(const SampleKArgs& k, const wh_sample_args* p, hipStream_t st);
int wide_keys_prepare(const SampleKArgs& k, void* workspace, hipStream_t st, uint64_t** keys, int* G, int* SL);
int launch_sample_wide_from_keys(const SampleKArgs& k, const wh_sample_args* p, hipStream_t st);

}  // namespace wh
