/* Exact-order fp32 restatement of the reference's matmul kernel
 * (reference src/wxx/shaders/matmul.wgsl:56-147), TEST INFRASTRUCTURE ONLY.
 *
 * Every output element of the reference is one accumulator updated with
 * fma(a, b, acc) for k = 0, 1, ..., K-1 in ascending order (the K loop runs
 * over 16-wide tiles in order, and over k inside a tile in order), starting
 * from 0.0, followed by one separate add of the bias value
 * (matmul.wgsl:103-120 and :129-146).  This file computes exactly that with
 * C99 fmaf, so its result is the reference's result under a fused fma.
 *
 * Layouts as in the reference host code (src/wxx/functional/utils.py:389-433):
 * A is (M, K) row-major or (K, M) when transA; B is (K, N) or (N, K) when
 * transB; batch strides are sA / sB (0 = unbatched); bias mode 0 none,
 * 1 (N,), 2 (M, N), 3 (batch, M, N).  Rows [row0, row1) of every batch are
 * computed (a bounded sample for timing), the rest of C is left untouched.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

void oracle_gemm_fma(const float *A, const float *B, const float *bias, float *C,
                     int64_t M, int64_t N, int64_t K, int64_t batch, int64_t sA,
                     int64_t sB, int bias_mode, int transA, int transB, int64_t row0,
                     int64_t row1) {
  if (row1 > M) row1 = M;
  for (int64_t b = 0; b < batch; ++b) {
    const float *Ab = A + b * sA;
    const float *Bb = B + b * sB;
    float *Cb = C + b * M * N;
#pragma omp parallel for schedule(static)
    for (int64_t i = row0; i < row1; ++i) {
      float *acc = (float *)calloc((size_t)N, sizeof(float));
      if (!transB) {
        for (int64_t k = 0; k < K; ++k) {
          const float a = transA ? Ab[k * M + i] : Ab[i * K + k];
          const float *brow = Bb + k * N;
          for (int64_t j = 0; j < N; ++j) acc[j] = fmaf(a, brow[j], acc[j]);
        }
      } else {
        for (int64_t j = 0; j < N; ++j) {
          float s = 0.0f;
          const float *bcol = Bb + j * K;
          for (int64_t k = 0; k < K; ++k) {
            const float a = transA ? Ab[k * M + i] : Ab[i * K + k];
            s = fmaf(a, bcol[k], s);
          }
          acc[j] = s;
        }
      }
      for (int64_t j = 0; j < N; ++j) {
        float bv = 0.0f;
        if (bias_mode == 1) bv = bias[j];
        else if (bias_mode == 2) bv = bias[i * N + j];
        else if (bias_mode == 3) bv = bias[b * M * N + i * N + j];
        Cb[i * N + j] = acc[j] + bv;
      }
      free(acc);
    }
  }
}
