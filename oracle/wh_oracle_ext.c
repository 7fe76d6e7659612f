/*
 * wh_oracle_ext.c -- CPU oracle for the steps around the token selection:
 * the DSpark draft step's Markov bias and the top-n logprob output.
 *
 * TEST INFRASTRUCTURE ONLY: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, as the checker.
 *
 * Reference behaviour followed (paths relative to the reference root):
 *   runtime/deepseek_v4_ssd/dspark.py:157-165   _MarkovHead: embedding =
 *       markov_w1(token); bias = markov_w2(embedding.astype(float32))
 *   runtime/deepseek_v4_ssd/dspark.py:319-330   per position: logits =
 *       base_logits[:, position] + bias, then sampling_logprobs and the draw
 *   runtime/deepseek_v4_ssd/deepseek_v41/dspark.py:128-137  the same loop
 *   runtime/deepseek_v4_ssd/server.py:1110-1111 logprobs are rejected today;
 *       the top-n output is the build's own API (its definition below).
 *
 * The bias's float32 summation order is unspecified in the reference (an MLX
 * matrix-vector product); the contract fixes one, which the GPU kernel
 * reproduces bit for bit:
 *   chunk c (8 consecutive rank entries 8c .. 8c+7):  p_c = fma chain
 *       p = fma(w_{8c+i}, e_{8c+i}, p), i = 0..7, from p = 0;
 *   chunks beyond rank/8 up to 32 are 0;
 *   then a butterfly over the 32 chunks: for off = 16, 8, 4, 2, 1:
 *       p_c = p_c + p_(c xor off);  bias = p_0;
 *   logits[v] = base[v] + bias[v] (one float32 rounding).
 * Weights are float32 or bfloat16 (widened exactly).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static float who_w(const void* w, int dtype, long i) {
  if (dtype == 0) return ((const float*)w)[i];
  uint32_t b = (uint32_t)((const uint16_t*)w)[i] << 16;
  float f;
  memcpy(&f, &b, 4);
  return f;
}

/* out[v] = base[v] + markov_w2[v, :] . float32(markov_w1[prev, :]) */
int who_markov_logits(const float* base, const void* w1, const void* w2, int dtype, int V, int rank, int prev,
                      float* out) {
  if (V <= 0 || rank <= 0 || rank > 256 || rank % 8 != 0 || prev < 0 || prev >= V) return -1;
  float e[256];
  for (int r = 0; r < rank; ++r) e[r] = who_w(w1, dtype, (long)prev * rank + r);
  for (int v = 0; v < V; ++v) {
    float p[32];
    for (int c = 0; c < 32; ++c) {
      float s = 0.0f;
      if (c < rank / 8)
        for (int i = 0; i < 8; ++i) s = fmaf(who_w(w2, dtype, (long)v * rank + 8 * c + i), e[8 * c + i], s);
      p[c] = s;
    }
    for (int off = 16; off >= 1; off >>= 1) {
      float q[32];
      for (int c = 0; c < 32; ++c) q[c] = p[c] + p[c ^ off];
      memcpy(p, q, sizeof(p));
    }
    out[v] = base[v] + p[0];
  }
  return 0;
}

/* Top-n logprobs of a float32 row: the n largest entries in (value desc, id
 * asc) order -- lower ids first among equal values -- with logprob
 * l - logsumexp(l) computed in float64 and rounded to float32.  Entries of
 * -inf are ranked last (logprob -inf); n <= V. */
static __thread const float* g_tl_vals;
static int who_cmp_tl(const void* a, const void* b) {
  int i = *(const int*)a, j = *(const int*)b;
  float x = g_tl_vals[i], y = g_tl_vals[j];
  if (x > y) return -1;
  if (x < y) return 1;
  return (i > j) - (i < j);
}

int who_top_logprobs(const float* logits, int B, int V, long ld, int n, int32_t* ids, float* lps) {
  if (B < 0 || V <= 0 || n <= 0 || n > V) return -1;
  int* idx = (int*)malloc(sizeof(int) * V);
  if (!idx) return -2;
  for (int b = 0; b < B; ++b) {
    const float* l = logits + (long)b * ld;
    double m = -INFINITY;
    for (int i = 0; i < V; ++i) if (l[i] > m) m = l[i];
    double s = 0.0;
    if (m != -INFINITY)
      for (int i = 0; i < V; ++i) s += exp((double)l[i] - m);
    const double lse = m + log(s);
    for (int i = 0; i < V; ++i) idx[i] = i;
    g_tl_vals = l;
    qsort(idx, V, sizeof(int), who_cmp_tl);
    for (int k = 0; k < n; ++k) {
      ids[(long)b * n + k] = idx[k];
      lps[(long)b * n + k] = m == -INFINITY ? -INFINITY : (float)((double)l[idx[k]] - lse);
    }
  }
  free(idx);
  return 0;
}
