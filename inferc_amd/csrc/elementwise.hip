// Generic tensor ops for graphs the fusion passes leave partly unfused
// (the reference executor's elementwise / movement / reduction cases,
// src/runtime/executor.cc:226-339; src/kernels/elementwise.cc,
// movement.cc): numpy-broadcast binary arithmetic, comparisons and logic,
// Where, unary math, Cast, Expand, Transpose, Slice, ReduceMean and a
// typed Gather.
//
// Every op has one element-level definition used twice: by a device kernel
// (grid-stride loop, 256 threads) for tensors on the GPU, and by a host loop
// for small tensors whose values are known on the host (shape plumbing and
// masks built from shapes: constant folding of values that do not depend on
// any graph input's data). Shapes are up to rank 8; a broadcast input reads
// with stride 0 along its broadcast dims. Element types: float32, int32,
// int64, uint8/bool.
#include <cmath>
#include <cstring>
#include <string>
#include <type_traits>
#include <vector>

#include "common.h"
#include "ew.h"

namespace ih {
namespace {

constexpr int kEwBlock = 256;

unsigned ew_grid(int64_t n) {
  const int64_t b = (n + kEwBlock - 1) / kEwBlock;
  return unsigned(b < 1 ? 1 : (b > 16384 ? 16384 : b));
}

// Output dims and per-input strides (0 on broadcast dims), right-aligned.
struct BView {
  int rank = 0;
  int64_t dims[kEwMaxRank] = {};
  int64_t st[3][kEwMaxRank] = {};
  int64_t n = 1;
};

BView make_view(const std::vector<int64_t>& out, const std::vector<int64_t>* ins[3], int n_in) {
  BView v;
  IH_REQUIRE(out.size() <= size_t(kEwMaxRank), INFERC_ERR_UNSUPPORTED, "rank above 8");
  v.rank = int(out.size());
  for (int d = 0; d < v.rank; ++d) {
    v.dims[d] = out[size_t(d)];
    v.n *= out[size_t(d)];
  }
  for (int k = 0; k < n_in; ++k) {
    const std::vector<int64_t>& s = *ins[k];
    IH_REQUIRE(s.size() <= out.size(), INFERC_ERR_SHAPE, "broadcast: input rank above output");
    int64_t stride = 1;
    for (int d = v.rank - 1, j = int(s.size()) - 1; d >= 0; --d, --j) {
      if (j < 0) {
        v.st[k][d] = 0;
        continue;
      }
      const int64_t sd = s[size_t(j)];
      IH_REQUIRE(sd == v.dims[d] || sd == 1, INFERC_ERR_SHAPE, "broadcast: incompatible dims");
      v.st[k][d] = sd == 1 ? 0 : stride;
      stride *= sd;
    }
  }
  return v;
}

__host__ __device__ inline void offsets(const BView& v, int64_t e, int n_in, int64_t* off) {
  for (int k = 0; k < n_in; ++k) off[k] = 0;
  for (int d = v.rank - 1; d >= 0; --d) {
    const int64_t i = e % v.dims[d];
    e /= v.dims[d];
    for (int k = 0; k < n_in; ++k) off[k] += i * v.st[k][d];
  }
}

// ---------------------------------------------------------------- binary

template <class T>
__host__ __device__ inline T arith(int op, T a, T b) {
  switch (op) {
    case kEwAdd: return a + b;
    case kEwSub: return a - b;
    case kEwMul: return a * b;
    case kEwDiv: return b == T(0) && !std::is_floating_point<T>::value ? T(0) : a / b;
    case kEwMax: return a > b ? a : b;
    case kEwMin: return a < b ? a : b;
    default: return a;
  }
}

__host__ __device__ inline float arith_f(int op, float a, float b) {
  return op == kEwPow ? powf(a, b) : arith<float>(op, a, b);
}

template <class T>
__host__ __device__ inline bool compare(int op, T a, T b) {
  switch (op) {
    case kEwEqual: return a == b;
    case kEwLess: return a < b;
    case kEwLessOrEqual: return a <= b;
    case kEwGreater: return a > b;
    case kEwGreaterOrEqual: return a >= b;
    case kEwAnd: return (a != T(0)) && (b != T(0));
    case kEwOr: return (a != T(0)) || (b != T(0));
    case kEwXor: return (a != T(0)) != (b != T(0));
    default: return false;
  }
}

template <class T>
__host__ __device__ inline void binary_at(const BView& v, int op, const T* a, const T* b, void* y,
                                          int64_t e) {
  int64_t off[2];
  offsets(v, e, 2, off);
  if (op >= kEwEqual) {
    static_cast<uint8_t*>(y)[e] = compare<T>(op, a[off[0]], b[off[1]]) ? 1 : 0;
  } else if constexpr (std::is_same<T, float>::value) {
    static_cast<float*>(y)[e] = arith_f(op, a[off[0]], b[off[1]]);
  } else {
    static_cast<T*>(y)[e] = arith<T>(op, a[off[0]], b[off[1]]);
  }
}

template <class T>
__global__ __launch_bounds__(kEwBlock) void binary_kernel(BView v, int op,
                                                          const T* __restrict__ a,
                                                          const T* __restrict__ b, void* y) {
  for (int64_t e = int64_t(blockIdx.x) * kEwBlock + threadIdx.x; e < v.n;
       e += int64_t(gridDim.x) * kEwBlock)
    binary_at<T>(v, op, a, b, y, e);
}

// ---------------------------------------------------------------- where / copy

template <class T>
__host__ __device__ inline void where_at(const BView& v, const uint8_t* c, const T* a, const T* b,
                                         T* y, int64_t e) {
  int64_t off[3];
  offsets(v, e, 3, off);
  y[e] = c[off[0]] ? a[off[1]] : b[off[2]];
}

template <class T>
__global__ __launch_bounds__(kEwBlock) void where_kernel(BView v, const uint8_t* __restrict__ c,
                                                         const T* __restrict__ a,
                                                         const T* __restrict__ b,
                                                         T* __restrict__ y) {
  for (int64_t e = int64_t(blockIdx.x) * kEwBlock + threadIdx.x; e < v.n;
       e += int64_t(gridDim.x) * kEwBlock)
    where_at<T>(v, c, a, b, y, e);
}

// y[e] = x[offset of e under the view's input 0 strides]: Expand, Transpose
// and Slice are all this gather with different strides and a base offset.
template <class T>
__host__ __device__ inline void strided_at(const BView& v, int64_t base, const T* x, T* y,
                                           int64_t e) {
  int64_t off[1];
  offsets(v, e, 1, off);
  y[e] = x[base + off[0]];
}

template <class T>
__global__ __launch_bounds__(kEwBlock) void strided_kernel(BView v, int64_t base,
                                                           const T* __restrict__ x,
                                                           T* __restrict__ y) {
  for (int64_t e = int64_t(blockIdx.x) * kEwBlock + threadIdx.x; e < v.n;
       e += int64_t(gridDim.x) * kEwBlock)
    strided_at<T>(v, base, x, y, e);
}

// ---------------------------------------------------------------- unary / cast

__host__ __device__ inline float unary_f(int op, float x) {
  switch (op) {
    case kEwSqrt: return sqrtf(x);
    case kEwErf: return erff(x);
    case kEwTanh: return tanhf(x);
    case kEwNeg: return -x;
    case kEwAbs: return fabsf(x);
    case kEwExp: return expf(x);
    case kEwLog: return logf(x);
    case kEwReciprocal: return 1.0f / x;
    case kEwSigmoid: return 1.0f / (1.0f + expf(-x));
    case kEwFloor: return floorf(x);
    case kEwCeil: return ceilf(x);
    case kEwRelu: return x > 0.0f ? x : 0.0f;
    default: return x;
  }
}

template <class T>
__host__ __device__ inline void unary_at(int op, const T* x, T* y, int64_t e) {
  if constexpr (std::is_same<T, float>::value) {
    y[e] = unary_f(op, x[e]);
  } else if constexpr (std::is_same<T, uint8_t>::value) {
    y[e] = op == kEwNot ? uint8_t(x[e] ? 0 : 1) : x[e];
  } else {
    y[e] = op == kEwNeg ? T(-x[e]) : op == kEwAbs ? (x[e] < 0 ? T(-x[e]) : x[e]) : x[e];
  }
}

template <class T>
__global__ __launch_bounds__(kEwBlock) void unary_kernel(int64_t n, int op, const T* __restrict__ x,
                                                         T* __restrict__ y) {
  for (int64_t e = int64_t(blockIdx.x) * kEwBlock + threadIdx.x; e < n;
       e += int64_t(gridDim.x) * kEwBlock)
    unary_at<T>(op, x, y, e);
}

template <class S, class D>
__host__ __device__ inline D cast_one(S v) {
  if constexpr (std::is_same<D, uint8_t>::value) {
    return v != S(0) ? 1 : 0;  // bool and uint8 destinations: nonzero -> 1 for bool
  } else {
    return static_cast<D>(v);
  }
}

template <class S, class D>
__global__ __launch_bounds__(kEwBlock) void cast_kernel(int64_t n, const S* __restrict__ x,
                                                        D* __restrict__ y, int to_bool) {
  for (int64_t e = int64_t(blockIdx.x) * kEwBlock + threadIdx.x; e < n;
       e += int64_t(gridDim.x) * kEwBlock) {
    if constexpr (std::is_same<D, uint8_t>::value)
      y[e] = to_bool ? cast_one<S, D>(x[e]) : static_cast<D>(x[e]);
    else
      y[e] = cast_one<S, D>(x[e]);
  }
}

// ---------------------------------------------------------------- reduce / gather

// y[o] = mean over the reduced positions; `v` enumerates the kept dims of
// the output (strides into x), `r` the reduced dims.
__host__ __device__ inline void mean_at(const BView& v, const BView& r, const float* x, float* y,
                                        int64_t o) {
  int64_t base[1];
  offsets(v, o, 1, base);
  float s = 0.0f;
  for (int64_t k = 0; k < r.n; ++k) {
    int64_t off[1];
    offsets(r, k, 1, off);
    s += x[base[0] + off[0]];
  }
  y[o] = s / float(r.n);
}

__global__ __launch_bounds__(kEwBlock) void mean_kernel(BView v, BView r, const float* __restrict__ x,
                                                        float* __restrict__ y) {
  for (int64_t o = int64_t(blockIdx.x) * kEwBlock + threadIdx.x; o < v.n;
       o += int64_t(gridDim.x) * kEwBlock)
    mean_at(v, r, x, y, o);
}

template <class T>
__global__ __launch_bounds__(kEwBlock) void gather_t_kernel(int64_t outer, int64_t rows,
                                                            int64_t inner,
                                                            const T* __restrict__ x,
                                                            const int64_t* __restrict__ idx,
                                                            int64_t n_idx, T* __restrict__ y,
                                                            int32_t* err) {
  const int64_t total = outer * n_idx * inner;
  for (int64_t e = int64_t(blockIdx.x) * kEwBlock + threadIdx.x; e < total;
       e += int64_t(gridDim.x) * kEwBlock) {
    const int64_t c = e % inner, k = (e / inner) % n_idx, o = e / (inner * n_idx);
    int64_t i = idx[k];
    if (i < 0) i += rows;
    if (i < 0 || i >= rows) {
      y[e] = T(0);
      if (err) *err = 1;
    } else {
      y[e] = x[(o * rows + i) * inner + c];
    }
  }
}

template <class F>
void by_dtype(int dt, F&& f) {
  switch (dt) {
    case INFERC_DT_F32: f(float{}); break;
    case INFERC_DT_I64: f(int64_t{}); break;
    case INFERC_DT_I32: f(int32_t{}); break;
    case INFERC_DT_U8: case INFERC_DT_BOOL: f(uint8_t{}); break;
    default: fail(INFERC_ERR_UNSUPPORTED, "unsupported element type " + std::to_string(dt));
  }
}

}  // namespace

std::string shape_str(const std::vector<int64_t>& s) {
  std::string o = "[";
  for (size_t i = 0; i < s.size(); ++i) o += (i ? "," : "") + std::to_string(s[i]);
  return o + "]";
}

std::vector<int64_t> ew_broadcast_shape(const std::vector<std::vector<int64_t>>& shapes) {
  size_t r = 0;
  for (const auto& s : shapes) r = s.size() > r ? s.size() : r;
  std::vector<int64_t> out(r, 1);
  for (const auto& s : shapes)
    for (size_t i = 0; i < s.size(); ++i) {
      int64_t& o = out[r - s.size() + i];
      const int64_t d = s[i];
      IH_REQUIRE(d == o || d == 1 || o == 1, INFERC_ERR_SHAPE,
                 "incompatible broadcast: " + shape_str(s));
      if (o == 1) o = d;
    }
  return out;
}

int ew_binary_out_dtype(int op, int dtype) { return op >= kEwEqual ? INFERC_DT_BOOL : dtype; }

void ew_binary(inferc_hip_ctx* ctx, int op, int dtype, const std::vector<int64_t>& out,
               const void* a, const std::vector<int64_t>& ash, const void* b,
               const std::vector<int64_t>& bsh, void* y) {
  IH_REQUIRE(op != kEwPow || dtype == INFERC_DT_F32, INFERC_ERR_UNSUPPORTED,
             "Pow: float32 only");
  const std::vector<int64_t>* ins[3] = {&ash, &bsh, nullptr};
  const BView v = make_view(out, ins, 2);
  if (v.n == 0) return;
  by_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    const T* ap = static_cast<const T*>(a);
    const T* bp = static_cast<const T*>(b);
    if (ctx == nullptr) {
      for (int64_t e = 0; e < v.n; ++e) binary_at<T>(v, op, ap, bp, y, e);
    } else {
      hipLaunchKernelGGL(binary_kernel<T>, dim3(ew_grid(v.n)), dim3(kEwBlock), 0, ctx->stream, v,
                         op, ap, bp, y);
      check_launch("elementwise binary");
    }
  });
}

void ew_where(inferc_hip_ctx* ctx, int dtype, const std::vector<int64_t>& out, const void* c,
              const std::vector<int64_t>& csh, const void* a, const std::vector<int64_t>& ash,
              const void* b, const std::vector<int64_t>& bsh, void* y) {
  const std::vector<int64_t>* ins[3] = {&csh, &ash, &bsh};
  const BView v = make_view(out, ins, 3);
  if (v.n == 0) return;
  by_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    const uint8_t* cp = static_cast<const uint8_t*>(c);
    if (ctx == nullptr) {
      for (int64_t e = 0; e < v.n; ++e)
        where_at<T>(v, cp, static_cast<const T*>(a), static_cast<const T*>(b), static_cast<T*>(y), e);
    } else {
      hipLaunchKernelGGL(where_kernel<T>, dim3(ew_grid(v.n)), dim3(kEwBlock), 0, ctx->stream, v,
                         cp, static_cast<const T*>(a), static_cast<const T*>(b),
                         static_cast<T*>(y));
      check_launch("where");
    }
  });
}

namespace {

void strided_copy(inferc_hip_ctx* ctx, int dtype, const BView& v, int64_t base, const void* x,
                  void* y) {
  if (v.n == 0) return;
  by_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    if (ctx == nullptr) {
      for (int64_t e = 0; e < v.n; ++e)
        strided_at<T>(v, base, static_cast<const T*>(x), static_cast<T*>(y), e);
    } else {
      hipLaunchKernelGGL(strided_kernel<T>, dim3(ew_grid(v.n)), dim3(kEwBlock), 0, ctx->stream,
                         v, base, static_cast<const T*>(x), static_cast<T*>(y));
      check_launch("strided copy");
    }
  });
}

std::vector<int64_t> strides_of(const std::vector<int64_t>& s) {
  std::vector<int64_t> st(s.size(), 1);
  for (int i = int(s.size()) - 2; i >= 0; --i) st[size_t(i)] = st[size_t(i + 1)] * s[size_t(i + 1)];
  return st;
}

}  // namespace

void ew_expand(inferc_hip_ctx* ctx, int dtype, const std::vector<int64_t>& out, const void* x,
               const std::vector<int64_t>& xsh, void* y) {
  const std::vector<int64_t>* ins[3] = {&xsh, nullptr, nullptr};
  strided_copy(ctx, dtype, make_view(out, ins, 1), 0, x, y);
}

void ew_transpose(inferc_hip_ctx* ctx, int dtype, const std::vector<int64_t>& in,
                  const std::vector<int64_t>& perm, const void* x, void* y) {
  const int r = int(in.size());
  IH_REQUIRE(int(perm.size()) == r && r <= kEwMaxRank, INFERC_ERR_SHAPE,
             "Transpose: perm does not match the input rank");
  const std::vector<int64_t> st = strides_of(in);
  BView v;
  v.rank = r;
  for (int d = 0; d < r; ++d) {
    const int64_t p = perm[size_t(d)];
    IH_REQUIRE(p >= 0 && p < r, INFERC_ERR_SHAPE, "Transpose: perm out of range");
    v.dims[d] = in[size_t(p)];
    v.st[0][d] = st[size_t(p)];
    v.n *= v.dims[d];
  }
  strided_copy(ctx, dtype, v, 0, x, y);
}

void ew_slice(inferc_hip_ctx* ctx, int dtype, const std::vector<int64_t>& in,
              const std::vector<int64_t>& start, const std::vector<int64_t>& step,
              const std::vector<int64_t>& out, const void* x, void* y) {
  const int r = int(in.size());
  IH_REQUIRE(r <= kEwMaxRank, INFERC_ERR_UNSUPPORTED, "Slice: rank above 8");
  const std::vector<int64_t> st = strides_of(in);
  BView v;
  v.rank = r;
  int64_t base = 0;
  for (int d = 0; d < r; ++d) {
    v.dims[d] = out[size_t(d)];
    v.st[0][d] = st[size_t(d)] * step[size_t(d)];
    v.n *= v.dims[d];
    base += start[size_t(d)] * st[size_t(d)];
  }
  strided_copy(ctx, dtype, v, base, x, y);
}

void ew_unary(inferc_hip_ctx* ctx, int op, int dtype, int64_t n, const void* x, void* y) {
  if (n == 0) return;
  IH_REQUIRE(dtype == INFERC_DT_F32 || op == kEwNeg || op == kEwAbs || op == kEwNot,
             INFERC_ERR_UNSUPPORTED, "unary op: float32 only for this op");
  IH_REQUIRE(op != kEwNot || dtype == INFERC_DT_BOOL, INFERC_ERR_UNSUPPORTED,
             "Not: bool input only");
  by_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    if (ctx == nullptr) {
      for (int64_t e = 0; e < n; ++e) unary_at<T>(op, static_cast<const T*>(x), static_cast<T*>(y), e);
    } else {
      hipLaunchKernelGGL(unary_kernel<T>, dim3(ew_grid(n)), dim3(kEwBlock), 0, ctx->stream, n, op,
                         static_cast<const T*>(x), static_cast<T*>(y));
      check_launch("elementwise unary");
    }
  });
}

void ew_cast(inferc_hip_ctx* ctx, int from, int to, int64_t n, const void* x, void* y) {
  if (n == 0) return;
  const int to_bool = to == INFERC_DT_BOOL;
  by_dtype(from, [&](auto stag) {
    using S = decltype(stag);
    by_dtype(to, [&](auto dtag) {
      using D = decltype(dtag);
      const S* xp = static_cast<const S*>(x);
      D* yp = static_cast<D*>(y);
      if (ctx == nullptr) {
        for (int64_t e = 0; e < n; ++e) {
          if constexpr (std::is_same<D, uint8_t>::value)
            yp[e] = to_bool ? cast_one<S, D>(xp[e]) : static_cast<D>(xp[e]);
          else
            yp[e] = cast_one<S, D>(xp[e]);
        }
      } else {
        hipLaunchKernelGGL((cast_kernel<S, D>), dim3(ew_grid(n)), dim3(kEwBlock), 0, ctx->stream,
                           n, xp, yp, to_bool);
        check_launch("cast");
      }
    });
  });
}

void ew_reduce_mean(inferc_hip_ctx* ctx, const std::vector<int64_t>& in,
                    const std::vector<bool>& reduce, const float* x, float* y) {
  const int r = int(in.size());
  IH_REQUIRE(r <= kEwMaxRank, INFERC_ERR_UNSUPPORTED, "ReduceMean: rank above 8");
  const std::vector<int64_t> st = strides_of(in);
  BView kept, red;
  for (int d = 0; d < r; ++d) {
    BView& v = reduce[size_t(d)] ? red : kept;
    v.dims[v.rank] = in[size_t(d)];
    v.st[0][v.rank] = st[size_t(d)];
    v.n *= in[size_t(d)];
    ++v.rank;
  }
  if (kept.n == 0) return;
  IH_REQUIRE(red.n > 0, INFERC_ERR_SHAPE, "ReduceMean over an empty axis");
  if (ctx == nullptr) {
    for (int64_t o = 0; o < kept.n; ++o) mean_at(kept, red, x, y, o);
  } else {
    hipLaunchKernelGGL(mean_kernel, dim3(ew_grid(kept.n)), dim3(kEwBlock), 0, ctx->stream, kept,
                       red, x, y);
    check_launch("reduce mean");
  }
}

void ew_gather(inferc_hip_ctx* ctx, int dtype, int64_t outer, int64_t rows, int64_t inner,
               const void* x, const int64_t* idx, int64_t n_idx, void* y, int32_t* err) {
  const int64_t total = outer * n_idx * inner;
  if (total == 0) return;
  by_dtype(dtype, [&](auto tag) {
    using T = decltype(tag);
    const T* xp = static_cast<const T*>(x);
    T* yp = static_cast<T*>(y);
    if (ctx == nullptr) {
      for (int64_t e = 0; e < total; ++e) {
        const int64_t c = e % inner, k = (e / inner) % n_idx, o = e / (inner * n_idx);
        int64_t i = idx[k];
        if (i < 0) i += rows;
        IH_REQUIRE(i >= 0 && i < rows, INFERC_ERR_ARG, "Gather: index out of range");
        yp[e] = xp[(o * rows + i) * inner + c];
      }
    } else {
      hipLaunchKernelGGL(gather_t_kernel<T>, dim3(ew_grid(total)), dim3(kEwBlock), 0, ctx->stream,
                         outer, rows, inner, xp, idx, n_idx, yp, err);
      check_launch("gather");
    }
  });
}

}  // namespace ih
