/*
 * CPU oracle — dense fp32 products (TEST INFRASTRUCTURE ONLY, see oracle.h).
 *
 * Stands in for Apple Accelerate's cblas_sgemm / cblas_sgemv, which the
 * reference calls at src/kernels/matmul.cc:119,140,212,218,
 * src/kernels/fused_matmul_add_gelu.cc:68 and src/kernels/attention.cc:71,95,131.
 * Accelerate's accumulation order is closed; this file uses one fixed order:
 * every C[i,j] is the k-ascending sum of A[i,k]*B[k,j] in fp32, then
 * C = alpha*sum + beta*C. Compiled with FMA contraction allowed (speed of the
 * timed CPU baseline); parity with the GPU is by tolerance.
 *
 * Pinned by: tests/test_oracle.py (kernels_test.cc:65-104 known answers,
 * amx_gemm_test.cc:21-38 sin/cos fixture vs a float64 numpy product,
 * kernels_test.cc:111-159 GEMV == sgemm).
 */
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define ORC_MB 32
#define ORC_NB 256
#define ORC_KB 256

/* Contiguous copy of op(X) with shape [rows, cols]. */
static float* materialize(int trans, int64_t rows, int64_t cols, const float* X,
                          int64_t ld) {
  float* t = (float*)malloc(sizeof(float) * (size_t)(rows * cols));
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c)
      t[r * cols + c] = trans ? X[c * ld + r] : X[r * ld + c];
  return t;
}

void orc_sgemm(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
               float alpha, const float* A, int64_t lda, const float* B,
               int64_t ldb, float beta, float* C, int64_t ldc) {
  if (M <= 0 || N <= 0) return;
  float* at = NULL;
  float* bt = NULL;
  if (trans_a) { at = materialize(1, M, K, A, lda); A = at; lda = K; }
  if (trans_b) { bt = materialize(1, K, N, B, ldb); B = bt; ldb = N; }
  const int64_t mt = (M + ORC_MB - 1) / ORC_MB;
  const int64_t nt = (N + ORC_NB - 1) / ORC_NB;
#pragma omp parallel for schedule(static)
  for (int64_t task = 0; task < mt * nt; ++task) {
    const int64_t i0 = (task / nt) * ORC_MB, j0 = (task % nt) * ORC_NB;
    const int64_t mb = (M - i0 < ORC_MB) ? M - i0 : ORC_MB;
    const int64_t nb = (N - j0 < ORC_NB) ? N - j0 : ORC_NB;
    float acc[ORC_MB][ORC_NB];
    for (int64_t i = 0; i < mb; ++i)
      for (int64_t j = 0; j < nb; ++j) acc[i][j] = 0.0f;
    for (int64_t k0 = 0; k0 < K; k0 += ORC_KB) {
      const int64_t k1 = (K - k0 < ORC_KB) ? K : k0 + ORC_KB;
      for (int64_t i = 0; i < mb; ++i) {
        float* ar = acc[i];
        for (int64_t k = k0; k < k1; ++k) {
          const float a = A[(i0 + i) * lda + k];
          const float* br = B + k * ldb + j0;
          for (int64_t j = 0; j < nb; ++j) ar[j] += a * br[j];
        }
      }
    }
    for (int64_t i = 0; i < mb; ++i) {
      float* cr = C + (i0 + i) * ldc + j0;
      if (beta == 0.0f) {
        for (int64_t j = 0; j < nb; ++j) cr[j] = alpha * acc[i][j];
      } else {
        for (int64_t j = 0; j < nb; ++j) cr[j] = alpha * acc[i][j] + beta * cr[j];
      }
    }
  }
  free(at);
  free(bt);
}

/* fp32 GEMV with the 4-accumulator pattern of the reference's decode floor
 * (bench/amx/decode_floor.cc:54-67): y[r] = sum_k W[r,k] x[k]. */
void orc_sgemv_rows(int64_t N, int64_t K, const float* W, const float* x,
                    float* y) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < N; ++r) {
    const float* w = W + r * K;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    int64_t k = 0;
    for (; k + 4 <= K; k += 4) {
      a0 += w[k] * x[k];
      a1 += w[k + 1] * x[k + 1];
      a2 += w[k + 2] * x[k + 2];
      a3 += w[k + 3] * x[k + 3];
    }
    for (; k < K; ++k) a0 += w[k] * x[k];
    y[r] = (a0 + a1) + (a2 + a3);
  }
}

/* fp32-accumulated int4 GEMV, the timed CPU baseline for the int4 path
 * (formula of bench/amx/decode_floor.cc:88-106, per-row scale applied after
 * the row sum: y = s_r * sum_k (nib-8) x_k). */
void orc_int4_gemv_f32acc(const uint8_t* W, const float* scales,
                          const float* x, float* y, int64_t N, int64_t K,
                          int64_t B) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < N; ++r) {
    const uint8_t* w = W + r * (K / 2);
    for (int64_t b = 0; b < B; ++b) {
      const float* xb = x + b * K;
      float a0 = 0.f, a1 = 0.f;
      for (int64_t k = 0; k < K; k += 2) {
        const uint8_t byte = w[k / 2];
        a0 += (float)((int)(byte & 0xf) - 8) * xb[k];
        a1 += (float)((int)(byte >> 4) - 8) * xb[k + 1];
      }
      y[b * N + r] = scales[r] * (a0 + a1);
    }
  }
}
