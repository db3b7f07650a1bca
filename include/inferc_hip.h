/*
 * inferc_hip.h — C-ABI of the MI355X (gfx950) backend for inferc's runtime
 * hot path. Every entry point takes plain device pointers and sizes; no C++
 * or torch types cross this boundary. All citations are path:line into the
 * inferc repository, naming the reference function each entry point replaces.
 *
 * Conventions
 *  - Every function returns an inferc_status; on failure a thread-local
 *    message is available from inferc_hip_last_error(). No exception crosses
 *    the ABI. (The reference throws std::runtime_error from its kernels, e.g.
 *    src/kernels/attention.cc:35-39; a C++ caller rethrows on non-zero.)
 *  - A context owns one device and one HIP stream. Kernel entry points are
 *    asynchronous on that stream; h2d/d2h/sync synchronise it. A context is
 *    single-threaded: one host thread at a time.
 *  - Device pointers are caller-owned unless a function says otherwise.
 *    Inputs are read-only; outputs must not alias inputs unless stated.
 *  - Matrices are row-major with leading dimensions counted in elements.
 */
#ifndef INFERC_HIP_H_
#define INFERC_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define INFERC_HIP_ABI_VERSION 1

typedef enum {
  INFERC_OK = 0,
  INFERC_ERR_ARG = 1,         /* null pointer, bad enum, negative size      */
  INFERC_ERR_SHAPE = 2,       /* inconsistent dimensions                    */
  INFERC_ERR_HIP = 3,         /* HIP runtime error                          */
  INFERC_ERR_OOM = 4,         /* device allocation failed                   */
  INFERC_ERR_UNSUPPORTED = 5, /* op / dtype / configuration not supported   */
  INFERC_ERR_STATE = 6        /* call out of order (e.g. missing input)     */
} inferc_status;

/* Epilogue activations. */
typedef enum {
  INFERC_ACT_NONE = 0,
  INFERC_ACT_GELU_ERF = 1,  /* v*0.5*(1+erf(v*0.70710678)) */
  INFERC_ACT_GELU_TANH = 2, /* 0.5*v*(1+tanh(0.79788456*(v+0.044715 v^3))) */
  INFERC_ACT_RELU = 3
} inferc_act;

/* Kind of the C operand of a Gemm (the reference pre-fills the output with C,
 * src/kernels/matmul.cc:174-193). */
typedef enum {
  INFERC_C_NONE = 0,
  INFERC_C_ROW = 1,    /* C[N] broadcast over rows   */
  INFERC_C_FULL = 2,   /* C[M,N] with leading dim ldc */
  INFERC_C_SCALAR = 3  /* C[1]                        */
} inferc_c_kind;

/* Tensor element types, as ONNX TensorProto.DataType codes (the reference
 * maps its IR DType to these with DTypeToOnnx, src/ir/graph.h:27-28). */
typedef enum {
  INFERC_DT_F32 = 1,
  INFERC_DT_U8 = 2,
  INFERC_DT_I32 = 6,
  INFERC_DT_I64 = 7,
  INFERC_DT_BOOL = 9
} inferc_dtype;

typedef struct inferc_hip_ctx inferc_hip_ctx;

/* ---------------- errors, context, memory ---------------- */

const char* inferc_hip_last_error(void);
int inferc_hip_abi_version(void);
int inferc_hip_device_count(int* count);

/* One device + one stream (replaces the process-wide state of
 * src/util/parallel.cc:16-47 and the toggles of src/kernels/matmul.cc:56-61). */
int inferc_hip_create(int device, inferc_hip_ctx** out);
int inferc_hip_destroy(inferc_hip_ctx* ctx);
/* Reserve at least `bytes` of context workspace (split-K partials, argmax
 * partials, int4 x preparation). Ops grow it on demand outside graph capture.
 * The context also keeps up to 32 grouped-GEMV descriptor tables on the
 * device, keyed by their bytes, and frees them all when a launch needs room. */
int inferc_hip_reserve_workspace(inferc_hip_ctx* ctx, size_t bytes);
/* One-row products whose B is transposed ([N,K] rows) take the batch-1 GEMV
 * route: on by default, off as the ablation baseline of `inferc decode
 * --no-gemv`. Replaces rt::SetGemvDecodeEnabled / GemvDecodeEnabled
 * (src/kernels/matmul.cc:56-61,207-216; main.cpp:718,727), per context
 * instead of process-wide. Executors' captured graphs are recorded again
 * after a change. */
int inferc_hip_set_gemv_decode(inferc_hip_ctx* ctx, int enabled);
int inferc_hip_gemv_decode_enabled(inferc_hip_ctx* ctx, int* enabled);

int inferc_hip_malloc(inferc_hip_ctx* ctx, size_t bytes, void** dptr);
int inferc_hip_free(inferc_hip_ctx* ctx, void* dptr);
int inferc_hip_h2d(inferc_hip_ctx* ctx, void* dst, const void* src, size_t bytes);
int inferc_hip_d2h(inferc_hip_ctx* ctx, void* dst, const void* src, size_t bytes);
int inferc_hip_d2d(inferc_hip_ctx* ctx, void* dst, const void* src, size_t bytes);
int inferc_hip_sync(inferc_hip_ctx* ctx);
/* HIP-event timing on the context stream (the per-op wall clock of
 * src/profiler/profiler.h:40-85, taken on the device). */
int inferc_hip_timer_start(inferc_hip_ctx* ctx);
int inferc_hip_timer_stop(inferc_hip_ctx* ctx, float* ms);

/* Record the kernels of any sequence of entry points on the context stream
 * into a HIP graph, then replay it with one launch (the reference re-walks
 * its graph per call; a replay issues the whole sequence at once). Entry
 * points that would allocate or upload during capture fail with
 * INFERC_ERR_STATE, so run the sequence once before capturing it. A replay
 * fails with INFERC_ERR_STATE if the context workspace was reallocated, or
 * its cached descriptor tables freed, after the capture. */
typedef struct inferc_hip_capture inferc_hip_capture;
int inferc_hip_capture_begin(inferc_hip_ctx* ctx);
int inferc_hip_capture_end(inferc_hip_ctx* ctx, inferc_hip_capture** out);
int inferc_hip_capture_replay(inferc_hip_capture* cap);
int inferc_hip_capture_destroy(inferc_hip_capture* cap);

/* ---------------- dense products ---------------- */

/* ONNX Gemm: Y = act(alpha*op(A)*op(B) + beta*C (+ R)).
 * Replaces rt::Gemm, src/kernels/matmul.cc:161-228 (incl. the M==1 sgemv
 * route of :207-216), and — with c_kind/R/act — the MatMul->Add(b)->Add(res)
 * and FusedMatMulAddGELU epilogues. op(A) is [M,K], op(B) is [K,N].
 * R (nullable) is a residual [M,N] with leading dim ldr, added after C.
 * Y may alias R (in-place residual update) but not A, B or C. */
int inferc_hip_gemm_f32(inferc_hip_ctx* ctx, int trans_a, int trans_b,
                        int64_t M, int64_t N, int64_t K, float alpha,
                        const float* A, int64_t lda, const float* B,
                        int64_t ldb, float beta, const float* C, int c_kind,
                        int64_t ldc, const float* R, int64_t ldr, int act,
                        float* Y, int64_t ldy);
/* inferc_hip_gemm_f32 that allocates nothing: no counterpart in the
 * reference. It is for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc). The
 * split-K partial sums that inferc_hip_gemm_f32 keeps in the context
 * workspace (growing it when needed) live here in a fixed 16 MiB static
 * device array, one per device, held until the process ends. A product whose
 * partial sums need more fails with INFERC_ERR_SHAPE before launching. Every
 * call on one device shares that array: calls that overlap on one device
 * (other streams, other threads) race. */
int inferc_hip_gemm_f32_noalloc(inferc_hip_ctx* ctx, int trans_a, int trans_b,
                                int64_t M, int64_t N, int64_t K, float alpha,
                                const float* A, int64_t lda, const float* B,
                                int64_t ldb, float beta, const float* C,
                                int c_kind, int64_t ldc, const float* R,
                                int64_t ldr, int act, float* Y, int64_t ldy);

/* numpy MatMul over a flattened batch: Y[b] = A[b*stride_a] * B[b*stride_b],
 * a stride of 0 broadcasts. Replaces rt::MatMul, src/kernels/matmul.cc:63-159. */
int inferc_hip_matmul_f32(inferc_hip_ctx* ctx, int64_t batch, int64_t M,
                          int64_t N, int64_t K, const float* A,
                          int64_t stride_a, const float* B, int64_t stride_b,
                          float* Y);

/* Y[M,N] = GELU_erf(X[M,K]*W[K,N] + b[N]).
 * Replaces rt::FusedMatMulAddGELU, src/kernels/fused_matmul_add_gelu.cc:13-80. */
int inferc_hip_fused_matmul_add_gelu_f32(inferc_hip_ctx* ctx, int64_t M,
                                         int64_t N, int64_t K, const float* X,
                                         const float* W, const float* bias,
                                         float* Y);

/* Q,K,V[M,N] = X[M,K]*Wi[K,N] + bi[N], one launch for the three projections.
 * Replaces rt::FusedQKVProjection, src/kernels/attention.cc:102-141. */
int inferc_hip_fused_qkv_f32(inferc_hip_ctx* ctx, int64_t M, int64_t K,
                             int64_t N, const float* X, const float* wq,
                             const float* bq, const float* wk, const float* bk,
                             const float* wv, const float* bv, float* q,
                             float* k, float* v);

/* ---------------- attention ---------------- */

/* Multi-head attention over [B,S,H] (head h = columns [h*hd,(h+1)*hd)):
 * O = softmax(mask(scale*Q_h K_h^T)) V_h with scale = 1/sqrtf(head_dim);
 * masked scores take the value `fill`. `mask` (nullable, one byte per
 * element, non-zero = masked) is read at
 * b*ms[0] + h*ms[1] + i*ms[2] + j*ms[3]; `mask_strides` is a HOST array of 4.
 * Replaces rt::FusedAttention, src/kernels/attention.cc:32-100
 * (MaskStrides :17-29). */
int inferc_hip_fused_attention_f32(inferc_hip_ctx* ctx, int64_t B, int64_t S,
                                   int64_t H, int64_t head_dim, const float* q,
                                   const float* k, const float* v,
                                   const uint8_t* mask,
                                   const int64_t* mask_strides, float fill,
                                   float* out);

/* ---------------- normalisation and pointwise ---------------- */

/* y = LN(x (+ residual)) over the last `feat` elements of each row:
 * mean, d = x-mean, var = mean(d^2), y = d*(1/sqrtf(var+eps))*gamma + beta.
 * residual is nullable. Replaces rt::LayerNorm, src/kernels/activation.cc:103-150
 * (dispatch of FusedLayerNorm at src/runtime/executor.cc:213-217). */
int inferc_hip_layernorm_f32(inferc_hip_ctx* ctx, int64_t rows, int64_t feat,
                             const float* x, const float* residual,
                             const float* gamma, const float* beta, float eps,
                             float* y);

/* Pointwise activations; act is an inferc_act. Replaces rt::Gelu and
 * rt::GeluTanh (src/kernels/activation.cc:15-50) and Relu
 * (src/kernels/elementwise.cc). y may alias x. */
int inferc_hip_activation_f32(inferc_hip_ctx* ctx, int64_t n, const float* x,
                              int act, float* y);

/* Softmax along an axis viewed as [outer, axis_dim, inner].
 * Replaces rt::Softmax, src/kernels/activation.cc:52-101. */
int inferc_hip_softmax_f32(inferc_hip_ctx* ctx, int64_t outer,
                           int64_t axis_dim, int64_t inner, const float* x,
                           float* y);

/* y[i] = a[i] + b[i % b_n] (elementwise, row-bias or scalar broadcast).
 * Replaces the hot-path forms of rt::Add, src/kernels/elementwise.cc:225. */
int inferc_hip_add_f32(inferc_hip_ctx* ctx, int64_t n, const float* a,
                       const float* b, int64_t b_n, float* y);

/* out[k,:] = table[idx[k],:] for int64 device indices (negative wraps).
 * Out-of-range indices write zeros and set *err_flag (device int32,
 * nullable) to 1. Replaces rt::Gather axis 0, src/kernels/embedding.cc:9-72. */
int inferc_hip_gather_f32(inferc_hip_ctx* ctx, int64_t rows, int64_t row_len,
                          const float* table, const int64_t* idx,
                          int64_t n_idx, float* out, int32_t* err_flag);

/* Split / Concat of an [outer, axis, inner] view (QKV split, KV concat).
 * parts / outs are HOST arrays of device pointers. Replace rt::Split and
 * rt::Concat, src/kernels/movement.cc:391-431 and :142-189. */
int inferc_hip_split_f32(inferc_hip_ctx* ctx, int64_t outer,
                         int64_t axis_full, int64_t inner, int64_t n_parts,
                         const int64_t* sizes, const float* x,
                         float* const* outs);
int inferc_hip_concat_f32(inferc_hip_ctx* ctx, int64_t outer, int64_t inner,
                          int64_t n_parts, const int64_t* sizes,
                          const float* const* parts, float* out);

/* First index of the maximum of x[n] into *out_idx (device int64).
 * Replaces the greedy argmax of src/cli/main.cpp:820-828,875-879. */
int inferc_hip_argmax_f32(inferc_hip_ctx* ctx, int64_t n, const float* x,
                          int64_t* out_idx);

/* ---------------- batch-1 decode products ---------------- */

/* y[N] = act(W[N,K] x (+ bias) (+ residual)); if ln_gamma is non-null the
 * input is first normalised, x' = LN(x; ln_gamma, ln_beta, ln_eps), inside
 * the kernel. W is the transB=1 layout (src/kernels/matmul.cc:207-216 routes
 * exactly this form to cblas_sgemv); y may alias residual. */
int inferc_hip_gemv_f32(inferc_hip_ctx* ctx, int64_t N, int64_t K,
                        const float* W, const float* x, const float* ln_gamma,
                        const float* ln_beta, float ln_eps, const float* bias,
                        const float* residual, int act, float* y);

/* int4 per-row-scale weights, reference layout: byte W[r*K/2 + k/2], low
 * nibble = even k, q = nib - 8 (bench/amx/int4_gemv_amx.cc:258-271).
 * unpack: out[r,k] = scales[r] * (float)q, bit-exact fp32 products. */
int inferc_hip_int4_unpack(inferc_hip_ctx* ctx, int64_t N, int64_t K,
                           const uint8_t* W, const float* scales, float* out);
/* y[b,r] = sum_k (scales[r]*q[r,k]) * x[b,k] for b < batch (1..8).
 * Replaces scalar_int4_gemv_perRow / amx_int4_gemv_b4_perRow,
 * bench/amx/int4_gemv_amx.cc:258-356. K must be even. */
int inferc_hip_int4_gemv(inferc_hip_ctx* ctx, int64_t N, int64_t K,
                         const uint8_t* W, const float* scales,
                         int64_t batch, const float* x, float* y);
/* Host-side symmetric per-row quantisation of w [N,K] (fp32) into the
 * layout above: s_r = max_k |w[r,k]| / 7, q = clamp(rint(w[r,k] / s_r),
 * -8, 7) (0 for an all-zero row), packed [N, K/2] with nibble q + 8;
 * deq (nullable) receives s_r * q. The reference's int4 benchmark draws q
 * at random (int4_gemv_amx.cc:520-535); this is the quantiser for real
 * weights. No GPU is used. */
int inferc_int4_quantize_rows(int64_t N, int64_t K, const float* w,
                              uint8_t* packed, float* scales, float* deq);
/* One launch over n_mats independent int4 GEMVs (all of a model's matrices).
 * Ns, Ks and the pointer arrays are HOST arrays of length n_mats holding
 * device pointers. x[i] is [batch, Ks[i]], y[i] is [batch, Ns[i]]. */
int inferc_hip_int4_gemv_grouped(inferc_hip_ctx* ctx, int64_t n_mats,
                                 const int64_t* Ns, const int64_t* Ks,
                                 const uint8_t* const* W,
                                 const float* const* scales, int64_t batch,
                                 const float* const* x, float* const* y);

/* Append one token's K/V (k_new/v_new [n_heads*head_dim]) at position *pos
 * (device int64) of the caches [n_heads, max_t, head_dim], then attend:
 * out = softmax((q.k_j)/sqrtf(head_dim), j <= pos) V. Replaces the
 * with-past graph's Concat(past,new) -> MatMul -> Div -> Softmax -> MatMul
 * (src/kernels/movement.cc:142-189 and the decode loop of
 * src/cli/main.cpp:854-889). */
int inferc_hip_kv_append_attend_f32(inferc_hip_ctx* ctx, int64_t n_heads,
                                    int64_t head_dim, int64_t max_t,
                                    const int64_t* pos, const float* q,
                                    const float* k_new, const float* v_new,
                                    float* k_cache, float* v_cache, float* out);

/* ---------------- executor (rt::Executor) ---------------- */

/* A host-side graph of (fused) nodes as the reference's passes leave it
 * (src/ir/graph.h:45-97). Attributes are "name=value" pairs joined by ';'
 * (ints, floats, comma-separated int lists). */
typedef struct inferc_graph inferc_graph;
int inferc_graph_create(inferc_graph** out);
int inferc_graph_destroy(inferc_graph* g);
int inferc_graph_add_initializer(inferc_graph* g, const char* name, int dtype,
                                 int rank, const int64_t* shape,
                                 const void* host_data);
int inferc_graph_add_node(inferc_graph* g, const char* op_type,
                          const char* name, int n_inputs,
                          const char* const* inputs, int n_outputs,
                          const char* const* outputs, const char* attrs);
int inferc_graph_add_output(inferc_graph* g, const char* name);
/* A declared graph input (Graph::inputs, src/ir/graph.h:80): dtype and
 * shape, -1 for a symbolic dim (onnx_to_ir.cc:10-23). */
int inferc_graph_add_input(inferc_graph* g, const char* name, int dtype,
                           int rank, const int64_t* shape);
/* A tensor-valued attribute (AttributeProto TENSOR, e.g. Constant's
 * "value", graph.h:69-72) on the most recently added node. */
int inferc_graph_add_tensor_attr(inferc_graph* g, const char* attr, int dtype,
                                 int rank, const int64_t* shape,
                                 const void* host_data);
/* The graph as JSON: name, inputs, outputs, initializers (name, dtype, shape,
 * bytes) and nodes (op, name, domain, inputs, outputs, attrs as text,
 * tensor_attrs). *len is the length without the NUL; buf == NULL queries it.
 * No counterpart in the reference (its IR is inspected in C++ directly). */
int inferc_graph_to_json(const inferc_graph* g, char* buf, size_t capacity,
                         size_t* len);
/* Copies an initializer's dtype, shape (room for 8 dims) and, when host_dst is
 * not NULL, its bytes (Graph::GetTensor, graph.h:90-92). */
int inferc_graph_get_initializer(const inferc_graph* g, const char* name,
                                 int* dtype, int* rank, int64_t* shape,
                                 void* host_dst, size_t capacity_bytes);

/* ---------------- ONNX reader and fusion passes ---------------- */

/* LoadOnnx + ConvertOnnxToIR (src/frontend/onnx_loader.cc:107-111,
 * onnx_to_ir.cc:87-144) without libprotobuf: the ModelProto subset inferc
 * reads (opset imports, graph name, nodes with INT/FLOAT/STRING/TENSOR/
 * INTS/FLOATS/STRINGS attributes, initializers from raw_data or typed
 * fields, inputs/outputs with dtype and shape). A malformed or truncated
 * file fails with INFERC_ERR_ARG; external tensor data and graph-valued
 * attributes with INFERC_ERR_UNSUPPORTED. The result feeds
 * inferc_graph_optimize and inferc_executor_create. */
int inferc_onnx_load(const char* path, inferc_graph** out);
int inferc_onnx_load_bytes(const void* data, size_t n, inferc_graph** out);
/* SummarizeModel as JSON (as_text = 0) or PrintSummary's text (as_text = 1)
 * (onnx_loader.cc:113-210); buffer protocol as inferc_graph_to_json. */
int inferc_onnx_summary(const void* data, size_t n, int as_text, char* buf,
                        size_t capacity, size_t* len);
/* OnnxElementBytes (onnx_loader.cc:69-86): 0 for variable-width types. */
int inferc_onnx_element_bytes(int onnx_dtype, int64_t* bytes);
/* One pass by name: "fold_constant_transpose" (constant_fold.cc:12-54),
 * "recognize_attention" (recognize_attention.cc:49-165),
 * "recognize_attention_additive" (no reference counterpart: the same block
 * with an additive float mask), "fuse_qkv_projection"
 * (recognize_attention.cc:167-237), "recognize_layernorm"
 * (recognize_layernorm.cc:46-187), "recognize_gelu" (recognize_gelu.cc:
 * 57-163), "recognize_gelu_tanh" (:165-296), "fuse_matmul_add_gelu"
 * (fuse_matmul_add_gelu.cc:20-122). *count = patterns folded. */
int inferc_graph_run_pass(inferc_graph* g, const char* pass, int* count);
/* All eight in the order of `inferc optimize` (src/cli/main.cpp:265-271),
 * the additive attention form right after the reference's; counts (nullable)
 * receives the eight match counts in that order. */
int inferc_graph_optimize(inferc_graph* g, int* counts);

/* Executor: uploads every initializer once (src/runtime/executor.cc:89-96);
 * run() walks the nodes in order and dispatches each op to a kernel
 * (executor.cc:98-366). Unsupported ops fail with INFERC_ERR_UNSUPPORTED
 * (executor.cc:340-343). After the first run for a given input shape the
 * launch sequence is captured in a HIP graph and replayed. */
typedef struct inferc_executor inferc_executor;
int inferc_executor_create(inferc_hip_ctx* ctx, const inferc_graph* g,
                           inferc_executor** out);
int inferc_executor_destroy(inferc_executor* ex);
/* Device-free executor for planning: run() performs the node walk with shape
 * inference, host shape plumbing and peephole fusion but launches nothing
 * (the role of InferShapes, src/ir/shape_inference.cc:577-633, for the fused
 * graph); output_info() then reports every output's shape. */
int inferc_executor_create_dry(const inferc_graph* g, inferc_executor** out);
/* Number of nodes after peephole fusion. */
int inferc_executor_node_count(inferc_executor* ex, int* count);
/* Bind an input from host memory (copied to the device) or a device pointer
 * (borrowed until the next set_input of that name). */
int inferc_executor_set_input(inferc_executor* ex, const char* name, int dtype,
                              int rank, const int64_t* shape,
                              const void* host_data);
int inferc_executor_set_input_device(inferc_executor* ex, const char* name,
                                     int dtype, int rank, const int64_t* shape,
                                     const void* dev_data);
/* Enqueue one forward pass on the context stream. A Gather whose indices
 * are on the device (e.g. input_ids) cannot check them before the pass runs:
 * an out-of-range index sets a flag that the next call waiting for the
 * stream (get_output, output_argmax, output_device, run_profiled) reports as
 * INFERC_ERR_ARG "Gather: index out of range" (src/kernels/embedding.cc:63),
 * clearing it. */
int inferc_executor_run(inferc_executor* ex);
/* Shape and dtype of a graph output after run(); shape has room for 8 dims. */
int inferc_executor_output_info(inferc_executor* ex, const char* name,
                                int* dtype, int* rank, int64_t* shape);
/* Copy an output to host memory (synchronises the stream). A dry-run
 * executor returns outputs whose values are known on the host (constants and
 * shape arithmetic folded while planning) and fails for the rest. */
int inferc_executor_get_output(inferc_executor* ex, const char* name,
                               void* host_dst, size_t capacity_bytes);
/* 0 = eager dispatch every run, 1 = capture/replay HIP graphs (default). */
int inferc_executor_set_graph_mode(inferc_executor* ex, int enabled);
/* Device KV cache for decode over an exported with-past graph: the
 * FusedAttentionPast nodes (GPT-2's attention over Concat(past, new), made
 * by the additive-attention pass) keep K/V in a persistent [B, nH, max_t, dh]
 * cache. Each run appends the new rows at the past length P (the past
 * input's dim 2); a past input set with data seeds rows [0, P), one set by
 * inferc_executor_set_input_shape means the cache already holds them. The
 * present.* outputs are views of the cache, copied out by get_output. This
 * replaces the reference's present -> past renaming through host tensors
 * (src/cli/main.cpp:831-836, 883-888). max_t = 0 unbinds. */
int inferc_executor_bind_kv_cache(inferc_executor* ex, int64_t max_t);
/* Decode mode for a with-past graph bound to a KV cache (no counterpart in
 * the reference, which re-plans every step of main.cpp:854-889): the caches
 * hold `len` positions (each FusedAttentionPast cache must hold at least
 * that many), a count kept on the device. Each run is then one decode step:
 * the caller gives the past inputs by shape with length 0 and the attention
 * mask (mask_input, nullable) for the new positions alone, all ones (as
 * `inferc decode` feeds, main.cpp:792-799); the attention nodes take the
 * past length from the device and ignore the mask, the position-embedding
 * gathers start at it, and the step advances it. Consecutive steps thus walk
 * the same graph: the second records a HIP graph, the rest replay it. Fails
 * with INFERC_ERR_UNSUPPORTED when a value derived from the past length
 * reaches anything else. len < 0 leaves decode mode. */
int inferc_executor_set_decode_position(inferc_executor* ex, int64_t len,
                                        const char* mask_input);
/* Positions the caches hold in decode mode (-1 outside it). */
int inferc_executor_decode_position(inferc_executor* ex, int64_t* len);
/* Decode feedback, in decode mode: each run ends with the greedy token of
 * `inferc decode` (first maximum of the last row of output `logits`,
 * main.cpp:875-879), which becomes the value of input `ids` (bound by this
 * call to a device [1,1] int64 holding first_token) for the next run and is
 * recorded on the device at its sequence position; so steps run back to back
 * with no host copy between them (the reference copies the token through
 * host tensors each step, main.cpp:880-889). logits = NULL turns it off;
 * leaving decode mode turns it off too. */
int inferc_executor_set_decode_feedback(inferc_executor* ex, const char* logits,
                                        const char* ids, int64_t first_token);
/* `steps` runs of the executor back to back; with step_ms (steps floats) it
 * waits for them and returns each run's device time from HIP events between
 * the runs, as main.cpp:863-872 times each step; without, it returns once
 * they are enqueued. */
int inferc_executor_run_steps(inferc_executor* ex, int64_t steps, float* step_ms);
/* The fed-back tokens at sequence positions first_pos .. first_pos + n - 1
 * (the first is first_token's position). Synchronises the stream. */
int inferc_executor_decode_tokens(inferc_executor* ex, int64_t first_pos, int64_t n,
                                  int64_t* tokens);
/* An input that carries only a shape (no data): a past the KV cache holds.
 * A node that needs its data fails with INFERC_ERR_STATE. */
int inferc_executor_set_input_shape(inferc_executor* ex, const char* name,
                                    int dtype, int rank, const int64_t* shape);
/* Device address of an output computed on the device (valid until the next
 * run of this executor), e.g. to hand a prefill's present.* to a with-past
 * executor through inferc_executor_set_input_device without a host copy.
 * No counterpart in the reference, whose tensors live on the host. */
int inferc_executor_output_device(inferc_executor* ex, const char* name,
                                  const void** ptr);
/* Index of the first maximum of the last row (last dim) of a float32
 * output, computed on the device: the greedy token of `inferc decode`
 * (main.cpp:875-879). Synchronises the stream. */
int inferc_executor_output_argmax(inferc_executor* ex, const char* name,
                                  int64_t* index);
/* Device bytes the executor holds: the uploaded initializers, the
 * transposed [N,K] copies of [K,N] weight initializers that one-row
 * products read on the GEMV route (made on the first run of a signature
 * that needs them, kept with the initializers), and the activation arena.
 * No counterpart in the reference, whose tensors live on the host. Any
 * pointer may be null. */
int inferc_executor_device_bytes(inferc_executor* ex, int64_t* initializers,
                                 int64_t* transposed_copies, int64_t* arena);

/* ---------------- Profiler (src/profiler/profiler.h:40-89) ---------------- */

/* prof::Profiler: per-op records over a sequence of inference passes
 * ("iterations") and the JSON report of profiler.cc:138-176. The host-clock
 * calls mirror BeginIteration/EndIteration/BeginOp/EndOp
 * (profiler.h:42-47): BeginOp while an op is in flight and EndOp without
 * BeginOp fail with INFERC_ERR_STATE (profiler.cc:68-90). Records made by
 * inferc_executor_run_profiled and inferc_gpt2_generate_profiled carry
 * device times instead. */
typedef struct inferc_profiler inferc_profiler;
int inferc_profiler_create(inferc_profiler** out);
int inferc_profiler_destroy(inferc_profiler* p);
int inferc_profiler_begin_iteration(inferc_profiler* p);
int inferc_profiler_end_iteration(inferc_profiler* p);
int inferc_profiler_begin_op(inferc_profiler* p, const char* op_type,
                             const char* node_name);
int inferc_profiler_end_op(inferc_profiler* p, int64_t activation_bytes_after);
/* Records a finished op whose time the caller measured itself (no
 * counterpart in the reference, whose ops are always timed by the host clock
 * between BeginOp and EndOp); fails while an op is in flight. */
int inferc_profiler_record_op(inferc_profiler* p, const char* op_type,
                              const char* node_name, double ms,
                              int64_t activation_bytes_after);
/* SetTrackActivationBytes (profiler.h:53): with 0, profiled executor runs
 * record 0 activation bytes and skip the O(tape) sum per node. Default 1. */
int inferc_profiler_set_track_activation_bytes(inferc_profiler* p, int on);
/* SnapshotPeakRss (profiler.h:57): the process's peak resident set. */
int inferc_profiler_snapshot_peak_rss(inferc_profiler* p);
int inferc_profiler_iteration_count(inferc_profiler* p, int64_t* n);
/* TotalStats (profiler.h:64): out5 = {mean, p50, p95, min, max} in ms. */
int inferc_profiler_total_stats(inferc_profiler* p, double* out5);
/* ToJson (profiler.h:75-76). *len receives the length without the NUL;
 * buf == NULL only queries it; capacity must be at least *len + 1. */
int inferc_profiler_to_json(inferc_profiler* p, const char* backend,
                            const char* model, char* buf, size_t capacity,
                            size_t* len);
/* Percentile (profiler.h:87): linear interpolation between closest ranks
 * (numpy's default); 0 for an empty sample. */
int inferc_profile_percentile(const double* v, int64_t n, double p, double* out);
/* StatsFrom (profiler.h:88): out5 = {mean, p50, p95, min, max}. */
int inferc_profile_stats(const double* v, int64_t n, double* out5);
/* Executor::Run(inputs, profiler) (src/runtime/executor.cc:98-125,349-354):
 * one eager pass recorded as one iteration, one op record per node. An op's
 * time is the device time between HIP events recorded on the stream around
 * the node; the iteration total is the host wall clock from the first
 * node's enqueue until the stream drains. Synchronises the stream. */
int inferc_executor_run_profiled(inferc_executor* ex, inferc_profiler* p);

/* ---------------- GPT-2 greedy decode (inferc decode) ---------------- */

typedef struct {
  int64_t layers, hidden, heads, ffn, vocab, max_pos;
  float eps;
} inferc_gpt2_config;

/* Weights are host pointers in this order (fp32, [K,N] = ONNX Gemm layout):
 *   0 wte [V,H]  1 wpe [P,H]
 *   per layer l, base 2+12l: +0 ln1_g +1 ln1_b +2 attn_w [H,3H] +3 attn_b
 *     +4 proj_w [H,H] +5 proj_b +6 ln2_g +7 ln2_b +8 fc_w [H,F] +9 fc_b
 *     +10 fcproj_w [F,H] +11 fcproj_b
 *   tail, base 2+12L: +0 lnf_g +1 lnf_b
 * Uploaded once; the LM head is the tied wte. max_t bounds prompt+generated. */
typedef struct inferc_gpt2 inferc_gpt2;
int inferc_gpt2_create(inferc_hip_ctx* ctx, const inferc_gpt2_config* cfg,
                       const float* const* host_weights, int64_t max_t,
                       inferc_gpt2** out);
int inferc_gpt2_destroy(inferc_gpt2* m);
/* The decode loop of src/cli/main.cpp:786-896: prefill over the prompt,
 * argmax, then max_tokens-1 cached steps (one replayed HIP graph each).
 * tokens_out[max_tokens] (host). step_ms (host, nullable) receives the
 * device time of each post-prefill step; last_logits (host, nullable, [V])
 * the final step's logits. */
int inferc_gpt2_generate(inferc_gpt2* m, const int64_t* prompt,
                         int64_t n_prompt, int64_t max_tokens,
                         int64_t* tokens_out, float* step_ms,
                         float* last_logits);
/* generate() with per-op profiling of the decode steps (main.cpp:846-872,
 * 914-934): each of the max_tokens-1 steps is enqueued eagerly and recorded
 * as one iteration whose ops are the step's fused launch groups
 * ("LayerNorm+QKV", "AttentionDecode", "MatMul+Bias+Residual",
 * "LayerNorm+MatMulAddGELU" per layer, then "LayerNorm+LMHead+ArgMax"),
 * each timed between HIP events. Tokens equal generate()'s. */
int inferc_gpt2_generate_profiled(inferc_gpt2* m, const int64_t* prompt,
                                  int64_t n_prompt, int64_t max_tokens,
                                  int64_t* tokens_out, inferc_profiler* p);
/* Full-sequence forward logits [n, V] (host) for every position. */
int inferc_gpt2_forward(inferc_gpt2* m, const int64_t* ids, int64_t n,
                        float* logits);
/* Switches the model to int4 weight-only decode, irreversibly: every
 * projection and the tied LM head are quantised per output row with
 * inferc_int4_quantize_rows (the int4 format of
 * bench/amx/int4_gemv_amx.cc:249-250,264-267), the fp32 weights are replaced
 * by their dequantised values (so prefill, embedding lookup and
 * inferc_gpt2_forward run the same quantised model), and each decode step
 * streams the packed weights through the int4 GEMV. The reference measures
 * that GEMV only standalone; it never runs its decode loop on int4. Needs
 * hidden 768 and ffn 3072. */
int inferc_gpt2_use_int4(inferc_gpt2* m);

#ifdef __cplusplus
}
#endif
#endif /* INFERC_HIP_H_ */
