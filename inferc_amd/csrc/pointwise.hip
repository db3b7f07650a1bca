// Row-wise and pointwise kernels: LayerNorm, GELU/ReLU, Softmax, broadcast
// Add, Gather, Split/Concat copies and argmax.
//
// Reference semantics:
//   rt::LayerNorm   src/kernels/activation.cc:103-150
//   rt::Gelu / GeluTanh / Softmax  src/kernels/activation.cc:15-101
//   rt::Add         src/kernels/elementwise.cc:69-189,225
//   rt::Gather      src/kernels/embedding.cc:9-72
//   rt::Split / Concat  src/kernels/movement.cc:391-431, :142-189
//   greedy argmax   src/cli/main.cpp:820-828,875-879
#include "common.h"

namespace ih {
namespace {

constexpr int kBlock = 256;

// One wave64 per row (ln_row): rows up to 64*VPL features stay in registers
// for the two passes (mean, then the centred second moment, as the
// reference's vDSP_meanv / vDSP_measqv sequence); wider rows are re-read.
// Row r adds residual row r % res_rows (a residual repeated over leading
// dims, as a suffix-broadcast Add would).
//
// ids set: row r of x is row ids[r] of a [vocab, feat] table (an embedding
// Gather folded in, embedding.cc:9-72): negative ids wrap, and an id out of
// range raises the error flag (the table's first row stands in).
typedef float lnf4 __attribute__((ext_vector_type(4)));

// ln_row with float4 access (feat % 4 == 0, feat <= 256 * V4, every row and
// gamma/beta 16-byte aligned): lane holds features 4(lane + 64j) .. +3, so
// each load moves 1 KB per wave instead of 256 bytes. Loads are unconditional
// (a lane past the row reads chunk 0 and drops it).
template <int V4>
__device__ __forceinline__ void ln_row4(int lane, const float* __restrict__ xr,
                                        const float* __restrict__ rr, const float* __restrict__ g,
                                        const float* __restrict__ b, int64_t feat, float eps,
                                        float* __restrict__ yr) {
  const float inv_n = 1.0f / float(feat);
  const int64_t n4 = feat / 4;
  const lnf4* x4 = reinterpret_cast<const lnf4*>(xr);
  const lnf4* r4 = reinterpret_cast<const lnf4*>(rr);
  const lnf4* g4 = reinterpret_cast<const lnf4*>(g);
  const lnf4* b4 = reinterpret_cast<const lnf4*>(b);
  lnf4 v[V4], gv[V4], bv[V4], rv[V4];
#pragma unroll
  for (int j = 0; j < V4; ++j) {
    const int64_t c = lane + 64 * j;
    const int64_t cc = c < n4 ? c : 0;
    v[j] = x4[cc];
    rv[j] = rr ? r4[cc] : lnf4{0.f, 0.f, 0.f, 0.f};
    gv[j] = g4[cc];
    bv[j] = b4[cc];
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < V4; ++j) {
    const bool in = lane + 64 * j < n4;
    if (rr) v[j] = v[j] + rv[j];
    v[j] = in ? v[j] : lnf4{0.f, 0.f, 0.f, 0.f};
    s += (v[j][0] + v[j][1]) + (v[j][2] + v[j][3]);
  }
  const float mean = wave_sum_dpp(s) * inv_n;
  float q = 0.0f;
#pragma unroll
  for (int j = 0; j < V4; ++j) {
    const bool in = lane + 64 * j < n4;
    lnf4 d = v[j] - mean;
    d = in ? d : lnf4{0.f, 0.f, 0.f, 0.f};
    v[j] = d;
    q += (d[0] * d[0] + d[1] * d[1]) + (d[2] * d[2] + d[3] * d[3]);
  }
  const float inv = 1.0f / sqrtf(wave_sum_dpp(q) * inv_n + eps);
  lnf4* y4 = reinterpret_cast<lnf4*>(yr);
#pragma unroll
  for (int j = 0; j < V4; ++j) {
    const int64_t c = lane + 64 * j;
    if (c < n4) y4[c] = (v[j] * inv) * gv[j] + bv[j];
  }
}

// VPL: values per lane of the scalar row routine; V4 > 0: the float4 routine
// with V4 chunks per lane.
template <int VPL, int V4>
__global__ __launch_bounds__(kBlock) void layernorm_kernel(int64_t rows, int64_t feat,
                                                           const float* __restrict__ x,
                                                           const float* __restrict__ res,
                                                           const float* __restrict__ g,
                                                           const float* __restrict__ b,
                                                           float eps, float* __restrict__ y,
                                                           int64_t res_rows,
                                                           const int64_t* __restrict__ ids,
                                                           int64_t vocab, int32_t* err,
                                                           EqSide side) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
  // the compare riding along (independent of the rows)
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < side.n;
       i += int64_t(gridDim.x) * kBlock)
    side.out[i] = side.a[i] == side.b[side.b_n == side.n ? i : i % side.b_n] ? 1 : 0;
  if (row >= rows) return;
  int64_t xr = row;
  if (ids) {
    xr = ids[row];
    if (xr < 0) xr += vocab;
    if (xr < 0 || xr >= vocab) {
      if (lane == 0 && err) *err = 1;
      xr = 0;
    }
  }
  if constexpr (V4 > 0)
    ln_row4<V4>(lane, x + xr * feat, res ? res + (row % res_rows) * feat : nullptr, g, b, feat,
                eps, y + row * feat);
  else
    ln_row<VPL>(lane, x + xr * feat, res ? res + (row % res_rows) * feat : nullptr, g, b, feat,
                eps, y + row * feat);
}

__global__ __launch_bounds__(kBlock) void activation_kernel(int64_t n, const float* __restrict__ x,
                                                            int act, float* __restrict__ y) {
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * kBlock)
    y[i] = apply_act(x[i], act);
}

// One wave per softmax row of the [outer, axis, inner] view: max, exp(x-max)
// with the sum, then multiply by 1/sum.
__global__ __launch_bounds__(kBlock) void softmax_kernel(int64_t outer, int64_t axis_dim,
                                                         int64_t inner, const float* __restrict__ x,
                                                         float* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
  if (r >= outer * inner) return;
  const int64_t o = r / inner, in = r % inner;
  const float* xr = x + o * axis_dim * inner + in;
  float* yr = y + o * axis_dim * inner + in;
  float m = -INFINITY;
  for (int64_t k = lane; k < axis_dim; k += 64) m = fmaxf(m, xr[k * inner]);
  m = wave_max(m);
  float s = 0.0f;
  for (int64_t k = lane; k < axis_dim; k += 64) {
    const float e = expf(xr[k * inner] - m);
    yr[k * inner] = e;
    s += e;
  }
  const float inv = 1.0f / wave_sum(s);
  for (int64_t k = lane; k < axis_dim; k += 64) yr[k * inner] *= inv;
}

__global__ __launch_bounds__(kBlock) void add_kernel(int64_t n, const float* __restrict__ a,
                                                     const float* __restrict__ b, int64_t b_n,
                                                     float* __restrict__ y) {
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * kBlock)
    y[i] = a[i] + b[b_n == n ? i : i % b_n];
}

// out[o, k, c] = table[o, idx[k], c] over the [outer, rows, row_len] view
// (Gather along any axis); negative indices wrap, out-of-range ones write 0
// and raise the error flag.
__global__ __launch_bounds__(kBlock) void gather_kernel(int64_t outer, int64_t rows,
                                                        int64_t row_len,
                                                        const float* __restrict__ table,
                                                        const int64_t* __restrict__ idx,
                                                        int64_t n_idx, float* __restrict__ out,
                                                        int32_t* err) {
  const int64_t total = outer * n_idx * row_len;
  for (int64_t e = int64_t(blockIdx.x) * kBlock + threadIdx.x; e < total;
       e += int64_t(gridDim.x) * kBlock) {
    const int64_t c = e % row_len, k = (e / row_len) % n_idx, o = e / (row_len * n_idx);
    int64_t i = idx[k];
    if (i < 0) i += rows;
    if (i < 0 || i >= rows) {
      out[e] = 0.0f;
      if (err) *err = 1;
    } else {
      out[e] = table[(o * rows + i) * row_len + c];
    }
  }
}

// dst[h, 0:width] = src[h, 0:width] for strided rows (elements).
__global__ __launch_bounds__(kBlock) void copy2d_kernel(float* __restrict__ dst, int64_t dpitch,
                                                        const float* __restrict__ src,
                                                        int64_t spitch, int64_t width,
                                                        int64_t height) {
  const int64_t total = width * height;
  for (int64_t e = int64_t(blockIdx.x) * kBlock + threadIdx.x; e < total;
       e += int64_t(gridDim.x) * kBlock) {
    const int64_t h = e / width, w = e % width;
    dst[h * dpitch + w] = src[h * spitch + w];
  }
}

// out[i] = (a[i] == b[i % b_n]) for int64 operands (ONNX Equal, the
// attention-mask predicate of the encoder graph).
__global__ __launch_bounds__(kBlock) void equal_i64_kernel(int64_t n, const int64_t* __restrict__ a,
                                                           const int64_t* __restrict__ b,
                                                           int64_t b_n, uint8_t* __restrict__ out) {
  for (int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * kBlock)
    out[i] = a[i] == b[b_n == n ? i : i % b_n] ? 1 : 0;
}

struct ValIdx {
  float v;
  int64_t i;
};

// (v, i) wins over (w, j) when v > w, or v == w and i < j: the first maximum
// of a left-to-right strict '>' scan.
__device__ __forceinline__ void vi_merge(float& v, int64_t& i, float w, int64_t j) {
  if (w > v || (w == v && j < i)) {
    v = w;
    i = j;
  }
}

__device__ __forceinline__ void block_argmax(float& v, int64_t& i) {
  __shared__ float sv[kBlock / 64];
  __shared__ int64_t si[kBlock / 64];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float w = __shfl_xor(v, o, 64);
    const int64_t j = __shfl_xor(i, o, 64);
    vi_merge(v, i, w, j);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = v;
    si[wave] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kBlock / 64; ++w) vi_merge(v, i, sv[w], si[w]);
  }
}

__global__ __launch_bounds__(kBlock) void argmax_partial(int64_t n, const float* __restrict__ x,
                                                         ValIdx* __restrict__ part) {
  float v = -INFINITY;
  int64_t i = INT64_MAX;
  for (int64_t e = int64_t(blockIdx.x) * kBlock + threadIdx.x; e < n;
       e += int64_t(gridDim.x) * kBlock)
    vi_merge(v, i, x[e], e);
  block_argmax(v, i);
  if (threadIdx.x == 0) part[blockIdx.x] = ValIdx{v, i};
}

__global__ __launch_bounds__(kBlock) void argmax_final(int nparts, const ValIdx* __restrict__ part,
                                                       int64_t* __restrict__ out) {
  float v = -INFINITY;
  int64_t i = INT64_MAX;
  for (int e = threadIdx.x; e < nparts; e += kBlock) vi_merge(v, i, part[e].v, part[e].i);
  block_argmax(v, i);
  // All elements -inf/NaN: the reference scan keeps index 0.
  if (threadIdx.x == 0) *out = (i == INT64_MAX) ? 0 : i;
}

unsigned grid_for(int64_t n, int64_t per_block = kBlock, int64_t cap = 8192) {
  int64_t g = ceil_div(n, per_block);
  if (g < 1) g = 1;
  return unsigned(g < cap ? g : cap);
}

}  // namespace

void layernorm(inferc_hip_ctx* ctx, int64_t rows, int64_t feat, const float* x,
               const float* residual, const float* gamma, const float* beta, float eps,
               float* y) {
  layernorm_res_period(ctx, rows, feat, x, residual, rows, gamma, beta, eps, y);
}

namespace {
void launch_layernorm(inferc_hip_ctx* ctx, int64_t rows, int64_t feat, const float* x,
                      const float* residual, int64_t res_rows, const float* gamma,
                      const float* beta, float eps, float* y, const int64_t* ids, int64_t vocab,
                      int32_t* err, const EqSide& side) {
  IH_REQUIRE(rows >= 0 && feat > 0, INFERC_ERR_SHAPE, "layernorm: bad shape");
  IH_REQUIRE(residual == nullptr || (res_rows > 0 && rows % res_rows == 0), INFERC_ERR_SHAPE,
             "layernorm: residual rows must divide the rows");
  IH_REQUIRE(side.n >= 0 && side.b_n > 0 && (side.n == 0 || side.n % side.b_n == 0),
             INFERC_ERR_SHAPE, "equal: broadcast size must divide the output size");
  IH_REQUIRE(side.n == 0 || (side.a && side.b && side.out), INFERC_ERR_ARG,
             "equal: null pointer");
  if (rows == 0) {
    if (side.n > 0) equal_i64(ctx, side.n, side.a, side.b, side.b_n, side.out);
    return;
  }
  IH_REQUIRE(x && gamma && beta && y, INFERC_ERR_ARG, "layernorm: null pointer");
  const unsigned blocks = unsigned(ceil_div(rows, kBlock / 64));
  const int64_t rr = residual ? res_rows : int64_t(1);
  const bool vec4 = feat % 4 == 0 && feat <= 256 * 4 && aligned16(x) && aligned16(gamma) &&
                    aligned16(beta) && aligned16(y) && (residual == nullptr || aligned16(residual));
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(kBlock), 0, ctx->stream, rows, feat, x, residual,
                       gamma, beta, eps, y, rr, ids, vocab, err, side);
  };
  if (vec4 && feat <= 256 * 3) go(layernorm_kernel<16, 3>);
  else if (vec4) go(layernorm_kernel<16, 4>);
  else if (feat <= 64 * 4) go(layernorm_kernel<4, 0>);
  else go(layernorm_kernel<16, 0>);
  check_launch("layernorm");
}
}  // namespace

void layernorm_res_period(inferc_hip_ctx* ctx, int64_t rows, int64_t feat, const float* x,
                          const float* residual, int64_t res_rows, const float* gamma,
                          const float* beta, float eps, float* y, const EqSide& side) {
  launch_layernorm(ctx, rows, feat, x, residual, res_rows, gamma, beta, eps, y, nullptr, 0,
                   nullptr, side);
}

void layernorm_gather(inferc_hip_ctx* ctx, int64_t rows, int64_t feat, const float* table,
                      int64_t vocab, const int64_t* ids, int32_t* err, const float* residual,
                      int64_t res_rows, const float* gamma, const float* beta, float eps,
                      float* y, const EqSide& side) {
  IH_REQUIRE(vocab > 0 && ids != nullptr, INFERC_ERR_ARG, "layernorm: gather without rows");
  launch_layernorm(ctx, rows, feat, table, residual, res_rows, gamma, beta, eps, y, ids, vocab,
                   err, side);
}

void activation(inferc_hip_ctx* ctx, int64_t n, const float* x, int act, float* y) {
  IH_REQUIRE(n >= 0, INFERC_ERR_SHAPE, "activation: negative size");
  IH_REQUIRE(act >= INFERC_ACT_NONE && act <= INFERC_ACT_RELU, INFERC_ERR_ARG,
             "activation: unknown activation");
  if (n == 0) return;
  IH_REQUIRE(x && y, INFERC_ERR_ARG, "activation: null pointer");
  hipLaunchKernelGGL(activation_kernel, dim3(grid_for(n)), dim3(kBlock), 0, ctx->stream, n, x,
                     act, y);
  check_launch("activation");
}

void add_bcast(inferc_hip_ctx* ctx, int64_t n, const float* a, const float* b, int64_t b_n,
               float* y) {
  IH_REQUIRE(n >= 0 && b_n > 0 && (n == 0 || n % b_n == 0), INFERC_ERR_SHAPE,
             "add: broadcast size must divide the output size");
  if (n == 0) return;
  IH_REQUIRE(a && b && y, INFERC_ERR_ARG, "add: null pointer");
  hipLaunchKernelGGL(add_kernel, dim3(grid_for(n)), dim3(kBlock), 0, ctx->stream, n, a, b, b_n,
                     y);
  check_launch("add");
}

void gather_axis(inferc_hip_ctx* ctx, int64_t outer, int64_t rows, int64_t row_len,
                 const float* table, const int64_t* idx, int64_t n_idx, float* out,
                 int32_t* err_flag) {
  IH_REQUIRE(outer >= 0 && rows > 0 && row_len >= 0 && n_idx >= 0, INFERC_ERR_SHAPE,
             "gather: bad shape");
  if (outer == 0 || n_idx == 0 || row_len == 0) return;
  IH_REQUIRE(table && idx && out, INFERC_ERR_ARG, "gather: null pointer");
  hipLaunchKernelGGL(gather_kernel, dim3(grid_for(outer * n_idx * row_len)), dim3(kBlock), 0,
                     ctx->stream, outer, rows, row_len, table, idx, n_idx, out, err_flag);
  check_launch("gather");
}

void gather_rows(inferc_hip_ctx* ctx, int64_t rows, int64_t row_len, const float* table,
                 const int64_t* idx, int64_t n_idx, float* out, int32_t* err_flag) {
  gather_axis(ctx, 1, rows, row_len, table, idx, n_idx, out, err_flag);
}

void argmax(inferc_hip_ctx* ctx, int64_t n, const float* x, int64_t* out_idx, void* partial) {
  IH_REQUIRE(n > 0, INFERC_ERR_SHAPE, "argmax: empty input");
  IH_REQUIRE(x && out_idx, INFERC_ERR_ARG, "argmax: null pointer");
  const unsigned parts = grid_for(n, kBlock * 8, 256);
  static_assert(sizeof(ValIdx) * 256 <= kArgmaxScratchBytes, "argmax scratch too small");
  auto* part = static_cast<ValIdx*>(partial ? partial : ctx->ws(sizeof(ValIdx) * parts));
  hipLaunchKernelGGL(argmax_partial, dim3(parts), dim3(kBlock), 0, ctx->stream, n, x, part);
  hipLaunchKernelGGL(argmax_final, dim3(1), dim3(kBlock), 0, ctx->stream, int(parts), part,
                     out_idx);
  check_launch("argmax");
}

void equal_i64(inferc_hip_ctx* ctx, int64_t n, const int64_t* a, const int64_t* b, int64_t b_n,
               uint8_t* out) {
  IH_REQUIRE(n >= 0 && b_n > 0 && (n == 0 || n % b_n == 0), INFERC_ERR_SHAPE,
             "equal: broadcast size must divide the output size");
  if (n == 0) return;
  IH_REQUIRE(a && b && out, INFERC_ERR_ARG, "equal: null pointer");
  hipLaunchKernelGGL(equal_i64_kernel, dim3(grid_for(n)), dim3(kBlock), 0, ctx->stream, n, a, b,
                     b_n, out);
  check_launch("equal");
}

void copy2d(inferc_hip_ctx* ctx, float* dst, int64_t dpitch, const float* src, int64_t spitch,
            int64_t width, int64_t height) {
  if (width <= 0 || height <= 0) return;
  hipLaunchKernelGGL(copy2d_kernel, dim3(grid_for(width * height)), dim3(kBlock), 0, ctx->stream,
                     dst, dpitch, src, spitch, width, height);
  check_launch("copy2d");
}

}  // namespace ih

extern "C" {

int inferc_hip_layernorm_f32(inferc_hip_ctx* ctx, int64_t rows, int64_t feat, const float* x,
                             const float* residual, const float* gamma, const float* beta,
                             float eps, float* y) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    ih::layernorm(ctx, rows, feat, x, residual, gamma, beta, eps, y);
  });
}

int inferc_hip_activation_f32(inferc_hip_ctx* ctx, int64_t n, const float* x, int act, float* y) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    ih::activation(ctx, n, x, act, y);
  });
}

int inferc_hip_softmax_f32(inferc_hip_ctx* ctx, int64_t outer, int64_t axis_dim, int64_t inner,
                           const float* x, float* y) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    IH_REQUIRE(outer >= 0 && axis_dim > 0 && inner > 0, INFERC_ERR_SHAPE, "softmax: bad shape");
    if (outer == 0) return;
    IH_REQUIRE(x && y, INFERC_ERR_ARG, "softmax: null pointer");
    const unsigned blocks = unsigned(ih::ceil_div(outer * inner, ih::kBlock / 64));
    hipLaunchKernelGGL(ih::softmax_kernel, dim3(blocks), dim3(ih::kBlock), 0, ctx->stream, outer,
                       axis_dim, inner, x, y);
    ih::check_launch("softmax");
  });
}

int inferc_hip_add_f32(inferc_hip_ctx* ctx, int64_t n, const float* a, const float* b,
                       int64_t b_n, float* y) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    ih::add_bcast(ctx, n, a, b, b_n, y);
  });
}

int inferc_hip_gather_f32(inferc_hip_ctx* ctx, int64_t rows, int64_t row_len, const float* table,
                          const int64_t* idx, int64_t n_idx, float* out, int32_t* err_flag) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    ih::gather_rows(ctx, rows, row_len, table, idx, n_idx, out, err_flag);
  });
}

int inferc_hip_split_f32(inferc_hip_ctx* ctx, int64_t outer, int64_t axis_full, int64_t inner,
                         int64_t n_parts, const int64_t* sizes, const float* x,
                         float* const* outs) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    IH_REQUIRE(outer >= 0 && axis_full >= 0 && inner >= 0 && n_parts >= 0, INFERC_ERR_SHAPE,
               "split: negative size");
    IH_REQUIRE(n_parts == 0 || (sizes && outs), INFERC_ERR_ARG, "split: null array");
    int64_t total = 0;
    for (int64_t p = 0; p < n_parts; ++p) {
      IH_REQUIRE(sizes[p] >= 0, INFERC_ERR_SHAPE, "split: negative part size");
      total += sizes[p];
    }
    IH_REQUIRE(total == axis_full, INFERC_ERR_SHAPE, "split: sum(split_sizes) != axis size");
    int64_t off = 0;
    for (int64_t p = 0; p < n_parts; ++p) {
      if (sizes[p] > 0 && outer > 0 && inner > 0) {
        IH_REQUIRE(x && outs[p], INFERC_ERR_ARG, "split: null pointer");
        ih::copy2d(ctx, outs[p], sizes[p] * inner, x + off * inner, axis_full * inner,
                   sizes[p] * inner, outer);
      }
      off += sizes[p];
    }
  });
}

int inferc_hip_concat_f32(inferc_hip_ctx* ctx, int64_t outer, int64_t inner, int64_t n_parts,
                          const int64_t* sizes, const float* const* parts, float* out) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    IH_REQUIRE(outer >= 0 && inner >= 0 && n_parts > 0, INFERC_ERR_SHAPE, "concat: bad shape");
    IH_REQUIRE(sizes && parts, INFERC_ERR_ARG, "concat: null array");
    int64_t total = 0;
    for (int64_t p = 0; p < n_parts; ++p) {
      IH_REQUIRE(sizes[p] >= 0, INFERC_ERR_SHAPE, "concat: negative part size");
      total += sizes[p];
    }
    int64_t pos = 0;
    for (int64_t p = 0; p < n_parts; ++p) {
      if (sizes[p] > 0 && outer > 0 && inner > 0) {
        IH_REQUIRE(out && parts[p], INFERC_ERR_ARG, "concat: null pointer");
        ih::copy2d(ctx, out + pos * inner, total * inner, parts[p], sizes[p] * inner,
                   sizes[p] * inner, outer);
      }
      pos += sizes[p];
    }
  });
}

int inferc_hip_argmax_f32(inferc_hip_ctx* ctx, int64_t n, const float* x, int64_t* out_idx) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    ih::argmax(ctx, n, x, out_idx);
  });
}

}  // extern "C"
