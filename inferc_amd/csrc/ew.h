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
// writes 0 for an out-of-range index (callers validate host-known indices);
// the host form fails.
void ew_gather(inferc_hip_ctx* ctx, int dtype, int64_t outer, int64_t rows, int64_t inner,
               const void* x, const int64_t* idx, int64_t n_idx, void* y);

std::string shape_str(const std::vector<int64_t>& s);

}  // namespace ih
