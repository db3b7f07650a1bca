// Generic tensor ops (elementwise.hip): numpy-broadcast binary ops, Where,
// unary math, Cast, Expand, Transpose, Slice, ReduceMean and a typed
// Gather. Each runs on the device when `ctx` is non-null and as a host loop
// over host memory when `ctx` is null. Not part of the C-ABI.
#pragma once

#include <cstdint>
#include <vector>

#include "common.h"

namespace ih {

constexpr int kEwMaxRank = 8;

// Binary ops: arithmetic keeps the input type; kEwEqual and later give bool.
enum EwBinary : int {
  kEwAdd = 1, kEwSub, kEwMul, kEwDiv, kEwPow, kEwMax, kEwMin,
  kEwEqual = 16, kEwLess, kEwLessOrEqual, kEwGreater, kEwGreaterOrEqual, kEwAnd, kEwOr, kEwXor,
};

enum EwUnary : int {
  kEwSqrt = 1, kEwErf, kEwTanh, kEwNeg, kEwAbs, kEwExp, kEwLog, kEwReciprocal, kEwSigmoid,
  kEwFloor, kEwCeil, kEwRelu, kEwNot,
};

std::vector<int64_t> ew_broadcast_shape(const std::vector<std::vector<int64_t>>& shapes);
int ew_binary_out_dtype(int op, int dtype);
void ew_binary(inferc_hip_ctx* ctx, int op, int dtype, const std::vector<int64_t>& out,
               const void* a, const std::vector<int64_t>& ash, const void* b,
               const std::vector<int64_t>& bsh, void* y);
void ew_where(inferc_hip_ctx* ctx, int dtype, const std::vector<int64_t>& out, const void* c,
              const std::vector<int64_t>& csh, const void* a, const std::vector<int64_t>& ash,
              const void* b, const std::vector<int64_t>& bsh, void* y);
void ew_unary(inferc_hip_ctx* ctx, int op, int dtype, int64_t n, const void* x, void* y);
void ew_cast(inferc_hip_ctx* ctx, int from, int to, int64_t n, const void* x, void* y);
void ew_expand(inferc_hip_ctx* ctx, int dtype, const std::vector<int64_t>& out, const void* x,
               const std::vector<int64_t>& xsh, void* y);
void ew_transpose(inferc_hip_ctx* ctx, int dtype, const std::vector<int64_t>& in,
                  const std::vector<int64_t>& perm, const void* x, void* y);
// y = x[start + i * step] per dim; `out` is the result shape.
void ew_slice(inferc_hip_ctx* ctx, int dtype, const std::vector<int64_t>& in,
              const std::vector<int64_t>& start, const std::vector<int64_t>& step,
              const std::vector<int64_t>& out, const void* x, void* y);
void ew_reduce_mean(inferc_hip_ctx* ctx, const std::vector<int64_t>& in,
                    const std::vector<bool>& reduce, const float* x, float* y);
// Gather along one axis of x viewed as [outer, rows, inner]. The device form
// writes 0 for an out-of-range index and sets *err (when err is not null) to
// 1; the host form fails.
void ew_gather(inferc_hip_ctx* ctx, int dtype, int64_t outer, int64_t rows, int64_t inner,
               const void* x, const int64_t* idx, int64_t n_idx, void* y,
               int32_t* err = nullptr);

std::string shape_str(const std::vector<int64_t>& s);

// Attention of S query rows ([B, S, nH*dh], row stride ldq) over T keys of a
// head-major cache [B, nH, max_t, dh] (attention_cache.hip).
struct CacheAttnArgs {
  int64_t B = 0, S = 0, nH = 0, dh = 0;
  int64_t T = 0, max_t = 0;
  // Past length on the device (decode mode; null: T - S): the S new rows sit
  // at *pos .. *pos + S - 1 and T is taken as *pos + S in the kernel.
  const int64_t* pos = nullptr;
  // New K/V rows [B, S, nH*dh] (row stride ldn), appended to the cache by
  // the attention kernel itself (null: already in the cache).
  const float* kn = nullptr;
  const float* vn = nullptr;
  int64_t ldn = 0;
  const float* q = nullptr;
  int64_t ldq = 0;
  const float* kc = nullptr;
  const float* vc = nullptr;
  const uint8_t* mask = nullptr;
  int64_t ms[4] = {0, 0, 0, 0};  // strides over [B, nH, S, T]; 0 on broadcast dims
  float fill = -3.0e38f;
  float* out = nullptr;
  int64_t ldo = 0;
};
void cache_attention(inferc_hip_ctx* ctx, const CacheAttnArgs& a);
// cache[b, h, t0 + s, :] = src[b, s, h*dh : (h+1)*dh] for s < S, with t0
// offset by *pos when pos (device) is given.
void cache_write_tokens(inferc_hip_ctx* ctx, int64_t B, int64_t S, int64_t nH, int64_t dh,
                        int64_t max_t, int64_t t0, const float* src, int64_t ld, float* cache,
                        const int64_t* pos = nullptr);
// out[i, :] = a[ids[i], :] + b[*pos + i, :] for i < n (ids on the device; one
// out of range sets *err when err is given and reads zeros).
void embed_add_at(inferc_hip_ctx* ctx, const float* a, int64_t a_rows, const int64_t* ids,
                  const float* b, int64_t b_rows, const int64_t* pos, int64_t n, int64_t row_len,
                  float* out, int32_t* err);
// out[i, :] = table[*pos + i, :] for i < n (rows clamped to the table): the
// position-embedding rows of a decode step whose past length is on the device.
void gather_rows_at(inferc_hip_ctx* ctx, int64_t rows, int64_t row_len, const float* table,
                    const int64_t* pos, int64_t n, float* out);
// *pos += step (one thread): a decode step's advance, recorded with the step.
void advance_position(inferc_hip_ctx* ctx, int64_t* pos, int64_t step);
// *pos advances by step after hist[*pos + step] = ids[0] = *tok (the decode
// step's arg-max fed back as the next step's token; hist holds a position's
// token at its index, so it needs the cache's max_t + 1 entries).
void decode_feedback(inferc_hip_ctx* ctx, int64_t* pos, int64_t step, const int64_t* tok,
                     int64_t* ids, int64_t* hist);
// The same with the token reduced from n (max, first index) partials of an
// arg-max GEMV (first maximum wins).
void decode_feedback_parts(inferc_hip_ctx* ctx, const ValIdxPart* parts, int64_t n, int64_t* pos,
                           int64_t step, int64_t* ids, int64_t* hist);

}  // namespace ih
