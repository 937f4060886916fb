/*
 * CPU baseline GEMV/GEMM (dequant-on-the-fly, f32 accumulate) -- TEST
 * INFRASTRUCTURE ONLY: timed by bench.py's cpu_baseline leg as a "port" of the
 * reference's CPU path (MLX CPU quantized_matmul reached from quant.rs:56-65).
 * Compiled separately from oracle.c so the compiler may vectorize and fuse
 * multiply-adds here (this function is a timing baseline, not a bit-exact
 * checker).
 */
#include "oracle.h"

#include <stdlib.h>

static int check_qargs(int64_t rows, int64_t cols, int group_size, int bits) {
  if (bits != 4 && bits != 8) return 3;
  if (group_size != 32 && group_size != 64 && group_size != 128) return 3;
  if (rows < 0 || cols <= 0 || cols % group_size) return 2;
  return 0;
}

static float bf16f(uint16_t b) {
  union { uint32_t u; float f; } v;
  v.u = (uint32_t)b << 16;
  return v.f;
}

int orc_qmatmul_f32(const uint16_t* x, int64_t M, const uint32_t* wq,
                    const uint16_t* scales, const uint16_t* biases,
                    int64_t N, int64_t K, int group_size, int bits,
                    float* y, int threads) {
  int rc = check_qargs(N, K, group_size, bits);
  if (rc) return rc;
  int64_t wpr = K * bits / 32, gpr = K / group_size;
  int per_word = 32 / bits;
  uint32_t mask = (1u << bits) - 1u;
  /* activations to f32 and per-group sums once (dequant-on-the-fly GEMV in
   * the factored form sum_g s*(x.q) + b*sum(x)). */
  float* xf = (float*)malloc(sizeof(float) * (size_t)(M * K));
  float* xs = (float*)malloc(sizeof(float) * (size_t)(M * gpr));
  if (!xf || !xs) { free(xf); free(xs); return 4; }
  for (int64_t i = 0; i < M * K; i++) xf[i] = bf16f(x[i]);
  for (int64_t m = 0; m < M; m++)
    for (int64_t g = 0; g < gpr; g++) {
      float s = 0.f;
      for (int j = 0; j < group_size; j++) s += xf[m * K + g * group_size + j];
      xs[m * gpr + g] = s;
    }
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
#endif
  for (int64_t n = 0; n < N; n++) {
    const uint32_t* row = wq + n * wpr;
    float qf[128];
    for (int64_t g = 0; g < gpr; g++) {
      for (int j = 0; j < group_size; j++) {
        int64_t k = g * group_size + j;
        qf[j] = (float)((row[k / per_word] >> ((k % per_word) * bits)) & mask);
      }
      float s = bf16f(scales[n * gpr + g]);
      float b = bf16f(biases[n * gpr + g]);
      for (int64_t m = 0; m < M; m++) {
        const float* xr = xf + m * K + g * group_size;
        float dot = 0.f;
        for (int j = 0; j < group_size; j++) dot += xr[j] * qf[j];
        float prev = g ? y[m * N + n] : 0.f;
        y[m * N + n] = prev + s * dot + b * xs[m * gpr + g];
      }
    }
  }
  (void)threads;
  free(xf);
  free(xs);
  return 0;
}
