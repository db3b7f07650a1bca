/*
 * CPU oracle for the inferc runtime hot path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the arithmetic of inferc's CPU runtime kernels
 * (the .cc files under src/kernels in the reference) and of the int4 per-row GEMV of
 * bench/amx/int4_gemv_amx.cc. Only the test-suite, the smoke check and the
 * CPU-baseline leg of the benchmark may load it; the shipped library never
 * links it and never falls back to it.
 *
 * Vendor calls are replaced by textbook loops:
 *   cblas_sgemm / cblas_sgemv  -> a blocked fp32 sgemm / row-dot GEMV
 *   vDSP / vForce              -> straight loops over libm expf/erff/tanhf
 *   GCD dispatch_apply         -> OpenMP static schedule
 * Accumulation order of Apple Accelerate is closed and cannot be reproduced,
 * so parity with the shipped library is by tolerance for fp32 sums and exact
 * for integer/byte work (int4 unpack, argmax, gather, split/concat).
 *
 * Pinning status of each function is listed at its definition in oracle.c.
 */
#ifndef INFERC_ORACLE_H_
#define INFERC_ORACLE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Activation codes shared with the product library's epilogues. */
enum { ORC_ACT_NONE = 0, ORC_ACT_GELU_ERF = 1, ORC_ACT_GELU_TANH = 2, ORC_ACT_RELU = 3 };

/* bias kinds for orc_gemm (C operand of ONNX Gemm). */
enum { ORC_C_NONE = 0, ORC_C_ROW = 1, ORC_C_FULL = 2, ORC_C_SCALAR = 3 };

int orc_num_threads(void);
void orc_set_num_threads(int n);
/* par::ParallelFor's partition of [0, n) (src/util/parallel.cc:49-72):
 * blocks = min(max_threads, max(1, ceil(n / grain))) (grain <= 0: max_threads
 * blocks), chunk = ceil(n / blocks), block b = [b*chunk, min(n, b*chunk +
 * chunk)), empty blocks skipped. Writes the non-empty blocks' bounds (room
 * for max(1, max_threads) entries) and returns their count; n <= 0 gives 0. */
int64_t orc_parallel_blocks(int64_t n, int64_t grain, int64_t max_threads,
                            int64_t* begin, int64_t* end);

/* C[M,N] = alpha*op(A)*op(B) + beta*C (row-major, leading dims in elements). */
void orc_sgemm(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
               float alpha, const float* A, int64_t lda, const float* B,
               int64_t ldb, float beta, float* C, int64_t ldc);

/* numpy-style batched MatMul with per-operand batch strides (0 = broadcast). */
void orc_matmul(int64_t batch, int64_t M, int64_t N, int64_t K,
                const float* A, int64_t stride_a, const float* B,
                int64_t stride_b, float* Y);

/* ONNX Gemm: Y = alpha*op(A)op(B) + beta*C (C pre-filled, broadcast). */
void orc_gemm(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
              float alpha, const float* A, const float* B, float beta,
              const float* C, int c_kind, float* Y);

/* Y = GELU_erf(X*W + b). */
void orc_fused_matmul_add_gelu(int64_t M, int64_t N, int64_t K, const float* X,
                               const float* W, const float* b, float* Y);

/* Q,K,V = X*Wi + bi. */
void orc_fused_qkv(int64_t M, int64_t K, int64_t N, const float* X,
                   const float* wq, const float* bq, const float* wk,
                   const float* bk, const float* wv, const float* bv,
                   float* q, float* k, float* v);

/* Fused multi-head attention over [B,S,H]; mask (nullable) indexed with
 * element strides ms[4] against [B,nH,S,S]. */
void orc_fused_attention(int64_t B, int64_t S, int64_t H, int64_t head_dim,
                         const float* q, const float* k, const float* v,
                         const uint8_t* mask, const int64_t* ms, float fill,
                         float* out);

void orc_layernorm(int64_t rows, int64_t feat, const float* x,
                   const float* gamma, const float* beta, float eps, float* y);
void orc_gelu(int64_t n, const float* x, float* y);
void orc_gelu_tanh(int64_t n, const float* x, float* y);
void orc_relu(int64_t n, const float* x, float* y);
void orc_softmax(int64_t outer, int64_t axis_dim, int64_t inner,
                 const float* x, float* y);

/* y = a + b with b broadcast by repeating it every b_n elements
 * (b_n == n: elementwise; b_n == row: row-bias; b_n == 1: scalar). */
void orc_add_bcast(int64_t n, const float* a, const float* b, int64_t b_n,
                   float* y);

/* Gather rows (axis 0) of table [rows, row_len]; returns 0 or -1 on a bad index. */
int orc_gather_rows(int64_t rows, int64_t row_len, const float* table,
                    const int64_t* idx, int64_t n_idx, float* out);

/* Split along an axis given outer/axis/inner sizes; Concat is its inverse. */
void orc_split(int64_t outer, int64_t axis_full, int64_t inner,
               int64_t n_parts, const int64_t* sizes, const float* x,
               float* const* outs);
void orc_concat(int64_t outer, int64_t inner, int64_t n_parts,
                const int64_t* sizes, const float* const* parts, float* out);

/* first index of the maximum (strict '>' scan). */
int64_t orc_argmax(int64_t n, const float* x);

/* int4 per-row GEMV (double accumulation). W [N,K/2] bytes, low nibble = even k. */
void orc_int4_gemv_per_row(const uint8_t* W, const float* scales,
                           const float* x, float* y, int64_t N, int64_t K);
/* batched: x [B,K], y [B,N]. */
void orc_int4_gemv_per_row_batched(const uint8_t* W, const float* scales,
                                   const float* x, float* y, int64_t N,
                                   int64_t K, int64_t B);
/* per-tensor scale variant. */
void orc_int4_gemv_per_tensor(const uint8_t* W, float scale, const float* x,
                              float* y, int64_t N, int64_t K);
/* dequantise: out[r,k] = scales[r] * (float)(nib - 8). */
void orc_int4_unpack(const uint8_t* W, const float* scales, int64_t N,
                     int64_t K, float* out);
/* fp32 accumulation variant used for the timed CPU baseline. */
void orc_int4_gemv_f32acc(const uint8_t* W, const float* scales,
                          const float* x, float* y, int64_t N, int64_t K,
                          int64_t B);

/* fp32 GEMV, W row-major [N,K]: y = W x (4 accumulators). */
void orc_sgemv_rows(int64_t N, int64_t K, const float* W, const float* x,
                    float* y);

/* ---- model-level restatements ---- */

/* DistilBERT-shape encoder (post-optimize fused graph), weight blob layout
 * documented in oracle.c. logits [B, n_classes]. */
typedef struct {
  int64_t layers, hidden, heads, ffn, vocab, max_pos, n_classes;
  float eps;
} orc_encoder_cfg;

int orc_encoder_forward(const orc_encoder_cfg* cfg, const float* const* w,
                        int64_t B, int64_t S, const int64_t* ids,
                        const int64_t* attn_mask, float* logits);

typedef struct {
  int64_t layers, hidden, heads, ffn, vocab, max_pos;
  float eps;
} orc_gpt2_cfg;

/* GPT-2 greedy decode: prefill over the prompt, then max_tokens-1 cached
 * steps. tokens_out[max_tokens]. Optional last_logits[vocab] of the final step
 * and per-step top-2 margin (margins[max_tokens], may be NULL). */
int orc_gpt2_generate(const orc_gpt2_cfg* cfg, const float* const* w,
                      const int64_t* prompt, int64_t n_prompt,
                      int64_t max_tokens, int64_t* tokens_out,
                      float* last_logits, float* margins);
/* orc_gpt2_generate that also writes each decode step's wall time in ms
 * (step_ms[max_tokens-1], nullable): the step's forward and LM head, not
 * the argmax or the prefill, as the reference's step timer
 * (src/cli/main.cpp:863-872). */
int orc_gpt2_generate_timed(const orc_gpt2_cfg* cfg, const float* const* w,
                            const int64_t* prompt, int64_t n_prompt,
                            int64_t max_tokens, int64_t* tokens_out,
                            float* last_logits, float* margins, double* step_ms);

/* full-sequence GPT-2 forward logits for every position: logits [n, vocab]. */
int orc_gpt2_forward(const orc_gpt2_cfg* cfg, const float* const* w,
                     const int64_t* ids, int64_t n, float* logits);

#ifdef __cplusplus
}
#endif
#endif
