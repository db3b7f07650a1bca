// Shared internals of the gfx950 backend: error plumbing, the context, and
// small device helpers. Not part of the C-ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/inferc_hip.h"

namespace ih {

// Internal error carried to the ABI edge, where it becomes a status code plus
// the thread-local message.
struct Error {
  int code;
  std::string msg;
};

void set_last_error(const std::string& msg);

[[noreturn]] inline void fail(int code, const std::string& msg) {
  throw Error{code, msg};
}

#define IH_HIP(expr)                                                        \
  do {                                                                      \
    hipError_t ih_e_ = (expr);                                              \
    if (ih_e_ != hipSuccess)                                                \
      ::ih::fail(ih_e_ == hipErrorOutOfMemory ? INFERC_ERR_OOM              \
                                              : INFERC_ERR_HIP,             \
                 std::string(#expr) + ": " + hipGetErrorString(ih_e_));     \
  } while (0)

#define IH_REQUIRE(cond, code, msg)          \
  do {                                       \
    if (!(cond)) ::ih::fail((code), (msg));  \
  } while (0)

// Runs `f`, converting every failure into a status code (no exception crosses
// the C-ABI).
template <class F>
int guard(F&& f) {
  try {
    f();
    return INFERC_OK;
  } catch (const Error& e) {
    set_last_error(e.msg);
    return e.code;
  } catch (const std::bad_alloc&) {
    set_last_error("host allocation failed");
    return INFERC_ERR_OOM;
  } catch (const std::exception& e) {
    set_last_error(e.what());
    return INFERC_ERR_HIP;
  } catch (...) {
    set_last_error("unknown error");
    return INFERC_ERR_HIP;
  }
}

// Throws if the last launch failed (bad configuration, missing code object).
inline void check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(INFERC_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace ih

// One device, one stream, one growable workspace.
struct inferc_hip_ctx {
  int device = 0;
  int num_cus = 256;
  hipStream_t stream = nullptr;
  hipEvent_t ev_start = nullptr, ev_stop = nullptr;
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
  // Bumped whenever device memory that a captured HIP graph may have baked in
  // is freed (the workspace on regrowth, the descriptor tables on eviction):
  // such a graph must be captured again.
  uint64_t ws_generation = 0;
  bool capturing = false;  // set while a HIP graph is being recorded
  // One-row products with a transposed B take the GEMV route (the
  // reference's g_gemv_decode_enabled, src/kernels/matmul.cc:56-61,207-216).
  bool gemv_decode = true;
  uint64_t route_generation = 0;  // bumped when gemv_decode changes
  // Arrival counters of the small-M GEMM's tiles when K is split over blocks
  // (zeroed once here; each launch leaves them zero). Launches on the
  // context's one stream run in order, so they never share a counter.
  static constexpr int64_t kKsCounters = 8192;
  unsigned* ks_count = nullptr;

  // Device copies of small launch descriptor tables, keyed by their bytes,
  // so repeated launches over the same operands skip the upload.
  struct Table {
    std::string key;
    void* dev = nullptr;
  };
  static constexpr size_t kMaxTables = 32;
  std::vector<Table> tables;

  // Returns a workspace of at least `bytes`; grows it outside capture only.
  void* ws(size_t bytes);
  // Makes room for `n` tables not yet cached, so that every table one launch
  // uploads is still alive when it runs: when the cache cannot take them all,
  // it waits for the stream and frees every cached table first (outside
  // capture only). Call it before the first table() of a launch.
  void reserve_tables(size_t n);
  // The device copy of `bytes` (len bytes), uploaded on a miss. A miss needs
  // a slot reserved by reserve_tables() and is refused during capture.
  const void* table(const void* bytes, size_t len);
  void free_tables();
  void make_current() const;
};

namespace ih {

inferc_hip_ctx* check_ctx(inferc_hip_ctx* ctx);

// ---------------- device helpers ----------------

__device__ __forceinline__ float gelu_erf_f(float v) {
  // src/kernels/fused_matmul_add_gelu.cc:56,73-75: multiply by 1/sqrt(2).
  return v * 0.5f * (1.0f + erff(v * 0.70710678118654752440f));
}

__device__ __forceinline__ float gelu_tanh_f(float v) {
  // src/kernels/activation.cc:42-47.
  const float inner = 0.7978845608028654f * (v + 0.044715f * v * v * v);
  return 0.5f * v * (1.0f + tanhf(inner));
}

__device__ __forceinline__ float apply_act(float v, int act) {
  switch (act) {
    case INFERC_ACT_GELU_ERF: return gelu_erf_f(v);
    case INFERC_ACT_GELU_TANH: return gelu_tanh_f(v);
    case INFERC_ACT_RELU: return v > 0.0f ? v : 0.0f;
    default: return v;
  }
}

// Wave64 butterfly reductions (all lanes receive the result).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Wave64 reductions without LDS: DPP rotations within each 16-lane row
// (every lane then holds its row's result), then the four rows' values read
// as scalars; all 64 lanes must be active. dpp_pair_swap exchanges lanes
// 2i and 2i+1 through a DPP quad permutation.
template <int R>
__device__ __forceinline__ float dpp_row_ror(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x120 + R, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_pair_swap(float v) {  // quad_perm [1,0,3,2]
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_lane(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_row_ror<8>(v));
  v = fmaxf(v, dpp_row_ror<4>(v));
  v = fmaxf(v, dpp_row_ror<2>(v));
  v = fmaxf(v, dpp_row_ror<1>(v));
  return fmaxf(fmaxf(row_lane(v, 0), row_lane(v, 16)), fmaxf(row_lane(v, 32), row_lane(v, 48)));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_row_ror<8>(v);
  v += dpp_row_ror<4>(v);
  v += dpp_row_ror<2>(v);
  v += dpp_row_ror<1>(v);
  return (row_lane(v, 0) + row_lane(v, 16)) + (row_lane(v, 32) + row_lane(v, 48));
}

// LayerNorm of one row by one wave64: the reference's two passes (mean, then
// the centred second moment; activation.cc:103-150), with y = (d * inv) *
// gamma + beta. x (+ res when given) is read once when the row fits 64*VPL
// values, else re-read per pass.
template <int VPL>
__device__ __forceinline__ void ln_row(int lane, const float* __restrict__ xr,
                                       const float* __restrict__ rr, const float* __restrict__ g,
                                       const float* __restrict__ b, int64_t feat, float eps,
                                       float* __restrict__ yr) {
  const float inv_n = 1.0f / float(feat);
  if (feat <= 64 * VPL) {
    // gamma and beta are loaded with x, so the row costs one memory round
    // trip before the reductions instead of a second one after them.
    float v[VPL], gv[VPL], bv[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int64_t c = lane + 64 * i;
      const bool in = c < feat;
      v[i] = in ? (rr ? xr[c] + rr[c] : xr[c]) : 0.0f;
      gv[i] = in ? g[c] : 0.0f;
      bv[i] = in ? b[c] : 0.0f;
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) s += v[i];
    const float mean = wave_sum_dpp(s) * inv_n;
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int64_t c = lane + 64 * i;
      const float d = (c < feat) ? v[i] - mean : 0.0f;
      v[i] = d;
      q += d * d;
    }
    const float var = wave_sum_dpp(q) * inv_n;
    const float inv = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int64_t c = lane + 64 * i;
      if (c < feat) yr[c] = (v[i] * inv) * gv[i] + bv[i];
    }
    return;
  }
  float s = 0.0f;
  for (int64_t c = lane; c < feat; c += 64) s += rr ? xr[c] + rr[c] : xr[c];
  const float mean = wave_sum_dpp(s) * inv_n;
  float q = 0.0f;
  for (int64_t c = lane; c < feat; c += 64) {
    const float d = (rr ? xr[c] + rr[c] : xr[c]) - mean;
    q += d * d;
  }
  const float inv = 1.0f / sqrtf(wave_sum_dpp(q) * inv_n + eps);
  for (int64_t c = lane; c < feat; c += 64) {
    const float d = (rr ? xr[c] + rr[c] : xr[c]) - mean;
    yr[c] = (d * inv) * g[c] + b[c];
  }
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

}  // namespace ih

// Internal launchers shared between translation units (all enqueue on
// ctx->stream and throw ih::Error on bad arguments).
namespace ih {

// LayerNorm of a GEMM operand's rows, applied as the operand is read:
// x' = (x - mean) * rstd * gamma + beta over the row's D <= 1024 features,
// with mean and rstd combined from per-16-column partials [rows][D/16][2] =
// (mean, M2 = sum of squared deviations) that the GEMM producing the rows
// wrote (GemmArgs::stats_out). Only the small-M GEMM path reads rows this
// way. For A the caller folds gamma into B (B'_kn = gamma_k B_kn) and beta
// into the bias (C_n + sum_k beta_k B_kn) and passes colsum_n = sum_k B'_kn
// per slice; the product is then rstd * (sum_k x_k B'_kn - mean * colsum_n),
// applied in the epilogue. For R, gamma and beta are applied as read.
struct RowNorm {
  const float* stats = nullptr;
  const float* gamma = nullptr;              // R
  const float* beta = nullptr;               // R
  const float* colsum[3] = {nullptr, nullptr, nullptr};  // A, per slice
  float eps = 1e-5f;
};

struct GemmArgs {
  int trans_a = 0, trans_b = 0;
  int64_t M = 0, N = 0, K = 0;
  float alpha = 1.0f, beta = 0.0f;
  const float* A = nullptr;
  int64_t lda = 0;
  const float* B = nullptr;
  int64_t ldb = 0;
  const float* C = nullptr;
  int c_kind = INFERC_C_NONE;
  int64_t ldc = 0;
  const float* R = nullptr;
  int64_t ldr = 0;
  int act = INFERC_ACT_NONE;
  float* Y = nullptr;
  int64_t ldy = 0;
  // batching: blockIdx.z selects slice b; strides in elements (0 broadcasts)
  int64_t batch = 1, stride_a = 0, stride_b = 0, stride_y = 0, stride_r = 0;
  // small-M path only: A's rows (over K) and R's rows (over N) normalized
  // as read, and Y's per-16-column (mean, M2) written to stats_out
  // [M][N/16][2] for a later GEMM that reads Y through a RowNorm
  RowNorm norm_a, norm_r;
  float* stats_out = nullptr;
  // one-row GEMV route only (gemm_gemv_route): LayerNorm of the A row first
  const float* gemv_ln_g = nullptr;
  const float* gemv_ln_b = nullptr;
  float gemv_ln_eps = 1e-5f;
  // Split-K partial sums go to this caller-given device buffer of
  // partial_bytes instead of the context workspace (a product that needs
  // more fails); null: the workspace.
  void* partial_buf = nullptr;
  size_t partial_bytes = 0;
};

// Looks up, once per device, the device address of the allocation-free
// GEMM's static scratch array; `device` must be current. Called when a
// context is created.
void init_gemm_scratch(int device);

// Whether gemm() sends `a` to the batch-1 GEMV (one row of A times a [N,K]
// B^T), the route that can apply a LayerNorm to the A row (gemv_ln_*).
bool gemm_gemv_route(const inferc_hip_ctx* ctx, const GemmArgs& a);

void gemm(inferc_hip_ctx* ctx, const GemmArgs& a);

// Three projections that share X in one launch: Y_i = X*W_i + b_i (X's rows
// normalized as read when norm_a is given).
void gemm_qkv(inferc_hip_ctx* ctx, int64_t M, int64_t K, int64_t N, const float* X,
              const float* const w[3], const float* const b[3], float* const y[3],
              int64_t ldy, const RowNorm* norm_a = nullptr);

// Whether an unbatched, untransposed product with 16-byte aligned operands
// (M x K times K x N, `slices` such products sharing A) takes the small-M
// path, the one that supports RowNorm operands and stats_out.
bool gemm_small_m_path(const inferc_hip_ctx* ctx, int64_t M, int64_t N, int64_t K,
                       int64_t slices);

struct AttnArgs {
  int64_t B = 0, S = 0, H = 0, head_dim = 0;
  const float* q = nullptr;
  const float* k = nullptr;
  const float* v = nullptr;
  int64_t ldq = 0, ldk = 0, ldv = 0, ldo = 0;  // row strides (elements)
  const uint8_t* mask = nullptr;
  int64_t ms[4] = {0, 0, 0, 0};
  float fill = -3.0e38f;
  int causal = 0;  // mask j > i with `fill` (GPT-2 prefill)
  float* out = nullptr;
};

void attention(inferc_hip_ctx* ctx, const AttnArgs& a);

void layernorm(inferc_hip_ctx* ctx, int64_t rows, int64_t feat, const float* x,
               const float* residual, const float* gamma, const float* beta, float eps,
               float* y);
// An elementwise compare that rides along with a LayerNorm launch, on
// operands independent of it: out[i] = (a[i] == b[i % b_n]) for i < n, with
// n % b_n == 0 (an Equal on graph inputs, e.g. an encoder's padding mask).
// n == 0: none.
struct EqSide {
  const int64_t* a = nullptr;
  const int64_t* b = nullptr;
  int64_t n = 0, b_n = 1;
  uint8_t* out = nullptr;
};
// As layernorm_res_period, with row r of x being row ids[r] of table
// [vocab, feat] (an embedding Gather folded in; an out-of-range id sets
// *err, which may be null).
void layernorm_gather(inferc_hip_ctx* ctx, int64_t rows, int64_t feat, const float* table,
                      int64_t vocab, const int64_t* ids, int32_t* err, const float* residual,
                      int64_t res_rows, const float* gamma, const float* beta, float eps,
                      float* y, const EqSide& side = EqSide{});
// As layernorm, with row r adding residual row r % res_rows.
void layernorm_res_period(inferc_hip_ctx* ctx, int64_t rows, int64_t feat, const float* x,
                          const float* residual, int64_t res_rows, const float* gamma,
                          const float* beta, float eps, float* y,
                          const EqSide& side = EqSide{});
void activation(inferc_hip_ctx* ctx, int64_t n, const float* x, int act, float* y);
void add_bcast(inferc_hip_ctx* ctx, int64_t n, const float* a, const float* b, int64_t b_n,
               float* y);
void gather_rows(inferc_hip_ctx* ctx, int64_t rows, int64_t row_len, const float* table,
                 const int64_t* idx, int64_t n_idx, float* out, int32_t* err_flag);
void gather_axis(inferc_hip_ctx* ctx, int64_t outer, int64_t rows, int64_t row_len,
                 const float* table, const int64_t* idx, int64_t n_idx, float* out,
                 int32_t* err_flag);
// `partial` (nullable) is caller-owned scratch of kArgmaxScratchBytes; when
// null the context workspace is used.
constexpr size_t kArgmaxScratchBytes = 256 * 16;
void argmax(inferc_hip_ctx* ctx, int64_t n, const float* x, int64_t* out_idx,
            void* partial = nullptr);
void copy2d(inferc_hip_ctx* ctx, float* dst, int64_t dpitch, const float* src, int64_t spitch,
            int64_t width, int64_t height);
void equal_i64(inferc_hip_ctx* ctx, int64_t n, const int64_t* a, const int64_t* b, int64_t b_n,
               uint8_t* out);
void kv_append_attend(inferc_hip_ctx* ctx, int64_t nH, int64_t D, int64_t T,
                      const int64_t* pos, const float* q, const float* k_new,
                      const float* v_new, float* kc, float* vc, float* out);

void gemv(inferc_hip_ctx* ctx, int64_t N, int64_t K, const float* W, const float* x,
          const float* ln_g, const float* ln_b, float ln_eps, const float* bias,
          const float* residual, int act, float* y);

// ---- batch-1 decode building blocks ----

// (value, index) partial of an argmax.
struct ValIdxPart {
  float v;
  int64_t i;
};
constexpr int kDecChunk = 32;  // keys per chunk of the decode attention

// y = act(W x' + bias + residual) with W [N, K], where x' is x or LN(x).
// When amax is non-null each block also writes the (max, first index) of
// its outputs.
// Returns the number of blocks launched (the size amax needs).
struct Gemv2Args {
  int64_t N = 0, K = 0;
  const float* W = nullptr;
  const float* x = nullptr;
  const float* ln_g = nullptr;
  const float* ln_b = nullptr;
  float ln_eps = 0.0f;
  const float* bias = nullptr;
  const float* res = nullptr;
  int act = INFERC_ACT_NONE;
  float* y = nullptr;
  ValIdxPart* amax = nullptr;
};
bool gemv2_supported(int64_t K);
// Batch-1 int4 GEMV for the decode step (K = 768 or 3072): optional
// LayerNorm of x (K = 768), y = act(s_r*acc + bias + res), or with amax set
// one first-max (value, row) partial per wave instead of y.
int64_t int4_dec_waves(int64_t N, int64_t K);
void int4_gemv_dec(inferc_hip_ctx* ctx, int64_t N, int64_t K, const uint8_t* W,
                   const float* scales, const float* x, const float* ln_g, const float* ln_b,
                   float ln_eps, const float* bias, const float* res, int act, float* y,
                   ValIdxPart* amax);
// Symmetric per-row int4 quantisation of an [N, K] fp32 matrix (host):
// s_r = max|w_r| / 7, q = clamp(rint(w / s_r), -8, 7), packed nibble q + 8
// (low nibble = even k); deq (optional) receives s_r * q.
void int4_quantize_rows(int64_t N, int64_t K, const float* w, uint8_t* packed, float* scales,
                        float* deq);
int64_t gemv2_blocks(inferc_hip_ctx* ctx, int64_t N, int64_t K, bool argmax);
void gemv2(inferc_hip_ctx* ctx, const Gemv2Args& a);

}  // namespace ih
