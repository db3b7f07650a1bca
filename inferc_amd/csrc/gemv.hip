// Batch-1 decode products: fp32 GEMV and the int4 per-row-scale GEMV.
//
// Reference semantics:
//   Gemm M==1 -> cblas_sgemv             src/kernels/matmul.cc:207-216
//   fp32 GEMV floor                       bench/amx/decode_floor.cc:54-67
//   scalar_int4_gemv_perRow (ground truth) bench/amx/int4_gemv_amx.cc:258-271
//   amx_int4_gemv_b4_perRow (optimised)    bench/amx/int4_gemv_amx.cc:280-356
//
// Both kernels are HBM-streaming: every weight byte is read exactly once per
// call with 16-byte loads, the activation vector stays on chip, and the
// row reductions are done in a fixed order (run-to-run deterministic).
#include <cstring>
#include <vector>

#include "common.h"

namespace ih {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;

// ---------------------------------------------------------------- fp32 GEMV

struct GemvP {
  int64_t N, K;
  const float* W;  // [N, K]
  const float* x;  // [K]
  const float* ln_g;
  const float* ln_b;
  float ln_eps;
  const float* bias;
  const float* res;
  int act;
  float* y;
};

__device__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();  // red may still be read by a previous reduction
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float s = 0.0f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) s += red[w];
  return s;
}

// x (optionally LayerNorm-ed with the same formula as the LayerNorm kernel)
// is staged in LDS; each wave then streams R rows of W at a time, lanes
// striding K in float4, and reduces each row with a butterfly.
template <int R, bool VEC>
__global__ __launch_bounds__(kBlock) void gemv_f32_kernel(GemvP p) {
  extern __shared__ __attribute__((aligned(16))) float xs[];
  __shared__ float red[kWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t K = p.K;
  for (int64_t k = tid; k < K; k += kBlock) xs[k] = p.x[k];
  __syncthreads();
  if (p.ln_g) {
    float s = 0.0f;
    for (int64_t k = tid; k < K; k += kBlock) s += xs[k];
    const float mean = block_sum(s, red) / float(K);
    float q = 0.0f;
    for (int64_t k = tid; k < K; k += kBlock) {
      const float d = xs[k] - mean;
      q += d * d;
    }
    const float var = block_sum(q, red) / float(K);
    const float inv = 1.0f / sqrtf(var + p.ln_eps);
    for (int64_t k = tid; k < K; k += kBlock) xs[k] = ((xs[k] - mean) * inv) * p.ln_g[k] + p.ln_b[k];
    __syncthreads();
  }
  const int64_t row_stride = int64_t(gridDim.x) * kWaves * R;
  for (int64_t r0 = (int64_t(blockIdx.x) * kWaves + wave) * R; r0 < p.N; r0 += row_stride) {
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = 0.0f;
    if (VEC) {
      for (int64_t k = 4 * lane; k < K; k += 256) {
        const float4 xv = *reinterpret_cast<const float4*>(xs + k);
        float4 wv[R];
#pragma unroll
        for (int i = 0; i < R; ++i) {
          wv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
          if (r0 + i < p.N) wv[i] = *reinterpret_cast<const float4*>(p.W + (r0 + i) * K + k);
        }
#pragma unroll
        for (int i = 0; i < R; ++i)
          acc[i] += wv[i].x * xv.x + wv[i].y * xv.y + wv[i].z * xv.z + wv[i].w * xv.w;
      }
    } else {
      for (int64_t k = lane; k < K; k += 64) {
        const float xv = xs[k];
#pragma unroll
        for (int i = 0; i < R; ++i)
          if (r0 + i < p.N) acc[i] += p.W[(r0 + i) * K + k] * xv;
      }
    }
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = wave_sum(acc[i]);
    if (lane < R && r0 + lane < p.N) {
      float v = acc[0];
#pragma unroll
      for (int i = 1; i < R; ++i)
        if (lane == i) v = acc[i];
      const int64_t r = r0 + lane;
      if (p.bias) v = v + p.bias[r];
      if (p.res) v = v + p.res[r];
      p.y[r] = apply_act(v, p.act);
    }
  }
}

// ------------------------------------------------- fp32 GEMV, short-chain form
//
// For K = 256*KV a wave owns R consecutive rows. Lane l's part of every row
// is the KV float4 at k = 4l + 256j, and it needs x at exactly those k, so x
// lives in registers, not LDS. The kernel's latency chain is one global load
// round trip: the weight loads are issued first (they depend on nothing), x
// is fetched (from L2) and, for XSRC_LN, normalised with wave-wide shuffles
// while they are in flight. There is no LDS and no block barrier.
//
// ARGMAX: each block also leaves (max logit, first index) of its rows for the
// decode step's final kernel.
enum { XSRC_PLAIN = 0, XSRC_LN = 1 };

struct Gemv2P {
  int64_t N;
  const float* W;
  const float* x;
  const float* ln_g;
  const float* ln_b;
  float ln_eps;
  const float* bias;
  const float* res;
  int act;
  float* y;
  // ARGMAX
  ValIdxPart* amax;      // [gridDim.x]
};

template <int KV, int XSRC>
__device__ __forceinline__ void gemv2_x(const Gemv2P& p, int lane, float4 (&xv)[KV]) {
  constexpr int K = 256 * KV;
#pragma unroll
  for (int j = 0; j < KV; ++j) xv[j] = *reinterpret_cast<const float4*>(p.x + 4 * lane + 256 * j);
  if (XSRC == XSRC_LN) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < KV; ++j) s += (xv[j].x + xv[j].y) + (xv[j].z + xv[j].w);
    const float mean = wave_sum(s) / float(K);
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < KV; ++j) {
      xv[j].x -= mean; xv[j].y -= mean; xv[j].z -= mean; xv[j].w -= mean;
      q += (xv[j].x * xv[j].x + xv[j].y * xv[j].y) + (xv[j].z * xv[j].z + xv[j].w * xv[j].w);
    }
    const float var = wave_sum(q) / float(K);
    const float inv = 1.0f / sqrtf(var + p.ln_eps);
#pragma unroll
    for (int j = 0; j < KV; ++j) {
      const float4 g = *reinterpret_cast<const float4*>(p.ln_g + 4 * lane + 256 * j);
      const float4 b = *reinterpret_cast<const float4*>(p.ln_b + 4 * lane + 256 * j);
      xv[j].x = (xv[j].x * inv) * g.x + b.x;
      xv[j].y = (xv[j].y * inv) * g.y + b.y;
      xv[j].z = (xv[j].z * inv) * g.z + b.z;
      xv[j].w = (xv[j].w * inv) * g.w + b.w;
    }
  }
}

template <int R, int KV, int XSRC, bool ARGMAX>
__global__ __launch_bounds__(kBlock) void gemv2_kernel(Gemv2P p) {
  constexpr int K = 256 * KV;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = (int64_t(blockIdx.x) * kWaves + wave) * R;
  float4 w[R][KV];
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int j = 0; j < KV; ++j)
      w[i][j] = (r0 + i < p.N)
                    ? *reinterpret_cast<const float4*>(p.W + (r0 + i) * K + 4 * lane + 256 * j)
                    : make_float4(0.f, 0.f, 0.f, 0.f);
  float4 xv[KV];
  gemv2_x<KV, XSRC>(p, lane, xv);
  float acc[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < KV; ++j)
      a += w[i][j].x * xv[j].x + w[i][j].y * xv[j].y + w[i][j].z * xv[j].z + w[i][j].w * xv[j].w;
    acc[i] = wave_sum(a);
  }
  float bv = -INFINITY;
  int64_t bi = INT64_MAX;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t r = r0 + i;
    if (r < p.N) {
      float v = acc[i];
      if (p.bias) v = v + p.bias[r];
      if (p.res) v = v + p.res[r];
      v = apply_act(v, p.act);
      if (lane == i) p.y[r] = v;
      if (ARGMAX && v > bv) {  // rows ascend: strict '>' keeps the first max
        bv = v;
        bi = r;
      }
    }
  }
  if (ARGMAX) {
    __shared__ float sv[kWaves];
    __shared__ int64_t si[kWaves];
    if (lane == 0) {
      sv[wave] = bv;
      si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int w2 = 1; w2 < kWaves; ++w2)
        if (sv[w2] > bv || (sv[w2] == bv && si[w2] < bi)) {
          bv = sv[w2];
          bi = si[w2];
        }
      p.amax[blockIdx.x] = ValIdxPart{bv, bi};
    }
  }
}

// ---------------------------------------------------------------- int4 GEMV

// One matrix of a (grouped) int4 GEMV launch.
struct Int4Mat {
  const uint8_t* W;  // [N, K/2], byte k/2 of row r: low nibble k even, high k odd
  const float* s;    // [N] per-row scales
  const float* x;    // [batch, K]
  float* y;          // [batch, N]
  int64_t N, K;
  int64_t block_begin;  // first block of this matrix in the launch
  int cpr;              // 16-byte chunks (32 weights) per row
  int groups;           // row groups per block pass = 256 / cpr
};

constexpr int kMaxBatch = 8;
constexpr int kRowsPerThread = 4;

// Byte N of v as a float; the backend selects v_cvt_f32_ubyteN for this form.
template <int N>
__device__ __forceinline__ float ubyte(uint32_t v) {
  return float((v >> (8 * N)) & 0xFFu);
}

// Layout of the work: thread t of a block owns chunk c = t % cpr of rows
// r0 + t/cpr + groups*j (j < 4), so its 32 x values (fp32) are loaded once and
// reused for 4 rows. Nibbles become floats with v_cvt_f32_ubyteN, and the
// -8 offset is folded: sum (nib-8) x = sum nib*x - 8*sum x. Per-(row, chunk)
// partials are reduced through LDS in chunk order, then scaled by s_r.
__global__ __launch_bounds__(kBlock) void int4_gemv_kernel(const Int4Mat* __restrict__ mats,
                                                           int n_mats, int batch) {
  __shared__ float part[kMaxBatch * kRowsPerThread * kBlock];
  // Locate this block's matrix (the table is sorted by block_begin).
  int lo = 0, hi = n_mats - 1;
  const int64_t bid = blockIdx.x;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (mats[mid].block_begin <= bid) lo = mid;
    else hi = mid - 1;
  }
  const Int4Mat m = mats[lo];
  const int tid = threadIdx.x;
  const int cpr = m.cpr, groups = m.groups;
  const int c = tid % cpr, g = tid / cpr;
  const int64_t rows_per_block = int64_t(groups) * kRowsPerThread;
  const int64_t rbase = (bid - m.block_begin) * rows_per_block;
  const bool active = g < groups;
  const int64_t rb = m.K / 2;

  // Load the weight chunks of this thread's rows (16 bytes each).
  uint4 w[kRowsPerThread];
#pragma unroll
  for (int j = 0; j < kRowsPerThread; ++j) {
    const int64_t r = rbase + g + int64_t(groups) * j;
    w[j] = make_uint4(0u, 0u, 0u, 0u);
    if (active && r < m.N) w[j] = *reinterpret_cast<const uint4*>(m.W + r * rb + c * 16);
  }
  for (int b = 0; b < batch; ++b) {
    float acc[kRowsPerThread];
#pragma unroll
    for (int j = 0; j < kRowsPerThread; ++j) acc[j] = 0.0f;
    float xsum = 0.0f;
    if (active) {
      const float4* xp = reinterpret_cast<const float4*>(m.x + b * m.K + c * 32);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // 8 consecutive k values: word q of the chunk holds k = 8q .. 8q+7.
        const float4 xa = xp[2 * q], xb = xp[2 * q + 1];
        xsum += (xa.x + xa.y) + (xa.z + xa.w) + (xb.x + xb.y) + (xb.z + xb.w);
#pragma unroll
        for (int j = 0; j < kRowsPerThread; ++j) {
          const uint32_t word = (q == 0) ? w[j].x : (q == 1) ? w[j].y : (q == 2) ? w[j].z : w[j].w;
          const uint32_t ev = word & 0x0F0F0F0Fu;         // nibbles of k = 8q + 0,2,4,6
          const uint32_t od = (word >> 4) & 0x0F0F0F0Fu;  // nibbles of k = 8q + 1,3,5,7
          float a = acc[j];
          a += ubyte<0>(ev) * xa.x;
          a += ubyte<0>(od) * xa.y;
          a += ubyte<1>(ev) * xa.z;
          a += ubyte<1>(od) * xa.w;
          a += ubyte<2>(ev) * xb.x;
          a += ubyte<2>(od) * xb.y;
          a += ubyte<3>(ev) * xb.z;
          a += ubyte<3>(od) * xb.w;
          acc[j] = a;
        }
      }
    }
    // part[b][j][g][c] laid out so each row's chunks are contiguous.
#pragma unroll
    for (int j = 0; j < kRowsPerThread; ++j)
      if (active) part[((b * kRowsPerThread + j) * groups + g) * cpr + c] = acc[j] - 8.0f * xsum;
  }
  __syncthreads();
  // One thread per (b, row): sum the row's chunk partials in chunk order.
  const int outs = batch * kRowsPerThread * groups;
  for (int o = tid; o < outs; o += kBlock) {
    const int b = o / (kRowsPerThread * groups);
    const int jg = o % (kRowsPerThread * groups);  // = j*groups + g
    const int j = jg / groups, gg = jg % groups;
    const int64_t r = rbase + gg + int64_t(groups) * j;
    if (r >= m.N) continue;
    const float* pp = part + (b * kRowsPerThread * groups + jg) * cpr;
    float s = 0.0f;
    for (int q = 0; q < cpr; ++q) s += pp[q];
    m.y[b * m.N + r] = m.s[r] * s;
  }
}

// Fallback for K not a multiple of 32: one thread per (b, row), exact formula.
__global__ __launch_bounds__(kBlock) void int4_gemv_generic(const uint8_t* __restrict__ W,
                                                            const float* __restrict__ s,
                                                            const float* __restrict__ x,
                                                            float* __restrict__ y, int64_t N,
                                                            int64_t K, int64_t batch) {
  const int64_t t = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (t >= N * batch) return;
  const int64_t r = t % N, b = t / N;
  float acc = 0.0f;
  for (int64_t k = 0; k < K; ++k) {
    const uint8_t byte = W[r * (K / 2) + k / 2];
    const int nib = (k & 1) ? (byte >> 4) : (byte & 0xF);
    acc += (s[r] * float(nib - 8)) * x[b * K + k];
  }
  y[b * N + r] = acc;
}

__global__ __launch_bounds__(kBlock) void int4_unpack_kernel(const uint8_t* __restrict__ W,
                                                             const float* __restrict__ s,
                                                             int64_t N, int64_t K,
                                                             float* __restrict__ out) {
  const int64_t nbytes = N * (K / 2);
  for (int64_t e = int64_t(blockIdx.x) * kBlock + threadIdx.x; e < nbytes;
       e += int64_t(gridDim.x) * kBlock) {
    const int64_t r = e / (K / 2), cb = e % (K / 2);
    const uint8_t byte = W[e];
    const float sr = s[r];
    // One IEEE round-to-nearest product each, as s_r * float(nib - 8).
    out[r * K + 2 * cb] = __fmul_rn(sr, float(int(byte & 0xF) - 8));
    out[r * K + 2 * cb + 1] = __fmul_rn(sr, float(int(byte >> 4) - 8));
  }
}

}  // namespace

bool gemv2_supported(int64_t K) { return K == 768 || K == 3072; }

namespace {

// Rows per wave: enough waves to keep ~8 per CU streaming, within the
// register budget (the K=3072 form holds 12 float4 of x per lane).
int gemv2_rows(inferc_hip_ctx* ctx, int64_t N, int64_t K) {
  if (K == 3072) return 1;
  const int64_t cus = ctx->num_cus;
  return N >= 32 * cus ? 4 : N >= 16 * cus ? 2 : 1;
}

template <int R, int KV>
void gemv2_launch_r(const Gemv2P& p, unsigned blocks, int xsrc, bool argmax, hipStream_t s) {
  const dim3 g(blocks), b(kBlock);
  if (argmax) {
    if (xsrc == XSRC_LN) hipLaunchKernelGGL((gemv2_kernel<R, KV, XSRC_LN, true>), g, b, 0, s, p);
    else hipLaunchKernelGGL((gemv2_kernel<R, KV, XSRC_PLAIN, true>), g, b, 0, s, p);
    return;
  }
  if (xsrc == XSRC_LN) hipLaunchKernelGGL((gemv2_kernel<R, KV, XSRC_LN, false>), g, b, 0, s, p);
  else hipLaunchKernelGGL((gemv2_kernel<R, KV, XSRC_PLAIN, false>), g, b, 0, s, p);
}

}  // namespace

int64_t gemv2_blocks(inferc_hip_ctx* ctx, int64_t N, int64_t K, bool /*argmax*/) {
  return ceil_div(ceil_div(N, gemv2_rows(ctx, N, K)), kWaves);
}

void gemv2(inferc_hip_ctx* ctx, const Gemv2Args& a) {
  IH_REQUIRE(gemv2_supported(a.K), INFERC_ERR_UNSUPPORTED, "gemv2: K must be 768 or 3072");
  IH_REQUIRE(a.N > 0 && a.W && a.y, INFERC_ERR_ARG, "gemv2: bad arguments");
  const int xsrc = a.ln_g ? XSRC_LN : XSRC_PLAIN;
  IH_REQUIRE(a.x, INFERC_ERR_ARG, "gemv2: null x");
  Gemv2P p{};
  p.N = a.N; p.W = a.W; p.x = a.x; p.ln_g = a.ln_g; p.ln_b = a.ln_b; p.ln_eps = a.ln_eps;
  p.bias = a.bias; p.res = a.res; p.act = a.act; p.y = a.y;
  p.amax = a.amax;
  const int R = gemv2_rows(ctx, a.N, a.K);
  const int64_t blocks = ceil_div(ceil_div(a.N, R), kWaves);
  IH_REQUIRE(blocks < (int64_t(1) << 31), INFERC_ERR_SHAPE, "gemv2: too many rows");
  const unsigned nb = unsigned(blocks);
  const bool am = a.amax != nullptr;
  if (a.K == 768) {
    if (R == 4) gemv2_launch_r<4, 3>(p, nb, xsrc, am, ctx->stream);
    else if (R == 2) gemv2_launch_r<2, 3>(p, nb, xsrc, am, ctx->stream);
    else gemv2_launch_r<1, 3>(p, nb, xsrc, am, ctx->stream);
  } else {
    gemv2_launch_r<1, 12>(p, nb, xsrc, am, ctx->stream);
  }
  check_launch("gemv2");
}

void gemv(inferc_hip_ctx* ctx, int64_t N, int64_t K, const float* W, const float* x,
          const float* ln_g, const float* ln_b, float ln_eps, const float* bias,
          const float* residual, int act, float* y) {
  IH_REQUIRE(N >= 0 && K >= 0, INFERC_ERR_SHAPE, "gemv: negative dimension");
  IH_REQUIRE(act >= INFERC_ACT_NONE && act <= INFERC_ACT_RELU, INFERC_ERR_ARG,
             "gemv: unknown activation");
  if (N == 0) return;
  IH_REQUIRE(y && (K == 0 || (W && x)), INFERC_ERR_ARG, "gemv: null pointer");
  IH_REQUIRE((ln_g == nullptr) == (ln_b == nullptr), INFERC_ERR_ARG,
             "gemv: LayerNorm needs both gamma and beta");
  IH_REQUIRE(!ln_g || K > 0, INFERC_ERR_SHAPE, "gemv: LayerNorm over an empty vector");
  IH_REQUIRE(K * sizeof(float) <= 64 * 1024, INFERC_ERR_UNSUPPORTED,
             "gemv: K > 16384 does not fit the on-chip activation buffer");
  if (gemv2_supported(K) && aligned16(W) && aligned16(x) && (!ln_g || (aligned16(ln_g) &&
                                                                      aligned16(ln_b)))) {
    Gemv2Args a;
    a.N = N; a.K = K; a.W = W; a.x = x; a.ln_g = ln_g; a.ln_b = ln_b; a.ln_eps = ln_eps;
    a.bias = bias; a.res = residual; a.act = act; a.y = y;
    gemv2(ctx, a);
    return;
  }
  GemvP p{N, K, W, x, ln_g, ln_b, ln_eps, bias, residual, act, y};
  const bool vec = aligned16(W) && K % 4 == 0;
  const size_t lds = size_t(K > 0 ? K : 1) * sizeof(float);
  // Enough waves to cover the rows with ~4 rows each on large outputs, one
  // row per wave on small ones (more CUs streaming).
  const bool big = N >= 16 * int64_t(ctx->num_cus);
  const int R = big ? 4 : 1;
  int64_t blocks = ceil_div(ceil_div(N, R), kWaves);
  if (blocks > 16 * int64_t(ctx->num_cus)) blocks = 16 * int64_t(ctx->num_cus);
  const dim3 grid(static_cast<unsigned>(blocks));
  if (big) {
    if (vec) hipLaunchKernelGGL((gemv_f32_kernel<4, true>), grid, dim3(kBlock), lds, ctx->stream, p);
    else hipLaunchKernelGGL((gemv_f32_kernel<4, false>), grid, dim3(kBlock), lds, ctx->stream, p);
  } else {
    if (vec) hipLaunchKernelGGL((gemv_f32_kernel<1, true>), grid, dim3(kBlock), lds, ctx->stream, p);
    else hipLaunchKernelGGL((gemv_f32_kernel<1, false>), grid, dim3(kBlock), lds, ctx->stream, p);
  }
  check_launch("gemv_f32");
}

namespace {

// Device copies of recently used grouped-GEMV descriptor tables, keyed by
// their bytes, so repeated calls with the same matrices skip the upload.
struct TableCache {
  struct Entry {
    std::vector<Int4Mat> key;
    Int4Mat* dev = nullptr;
  };
  std::vector<Entry> entries;
};

TableCache& table_cache(inferc_hip_ctx* ctx) {
  static thread_local std::vector<std::pair<inferc_hip_ctx*, TableCache>> caches;
  for (auto& c : caches)
    if (c.first == ctx) return c.second;
  caches.emplace_back(ctx, TableCache{});
  return caches.back().second;
}

const Int4Mat* upload_table(inferc_hip_ctx* ctx, const std::vector<Int4Mat>& mats) {
  TableCache& tc = table_cache(ctx);
  for (auto& e : tc.entries)
    if (e.key.size() == mats.size() &&
        std::memcmp(e.key.data(), mats.data(), mats.size() * sizeof(Int4Mat)) == 0)
      return e.dev;
  IH_REQUIRE(!ctx->capturing, INFERC_ERR_STATE,
             "int4 grouped GEMV: descriptor table must be uploaded before graph capture");
  if (tc.entries.size() >= 32) {
    IH_HIP(hipStreamSynchronize(ctx->stream));
    for (auto& e : tc.entries) (void)hipFree(e.dev);
    tc.entries.clear();
  }
  TableCache::Entry e;
  e.key = mats;
  IH_HIP(hipMalloc(&e.dev, mats.size() * sizeof(Int4Mat)));
  IH_HIP(hipMemcpy(e.dev, mats.data(), mats.size() * sizeof(Int4Mat), hipMemcpyHostToDevice));
  tc.entries.push_back(std::move(e));
  return tc.entries.back().dev;
}

void int4_grouped(inferc_hip_ctx* ctx, int64_t n_mats, const int64_t* Ns, const int64_t* Ks,
                  const uint8_t* const* W, const float* const* scales, int64_t batch,
                  const float* const* x, float* const* y) {
  IH_REQUIRE(n_mats >= 0, INFERC_ERR_SHAPE, "int4 gemv: negative matrix count");
  IH_REQUIRE(batch >= 1 && batch <= kMaxBatch, INFERC_ERR_UNSUPPORTED,
             "int4 gemv: batch must be in [1, 8]");
  if (n_mats == 0) return;
  IH_REQUIRE(Ns && Ks && W && scales && x && y, INFERC_ERR_ARG, "int4 gemv: null array");
  std::vector<Int4Mat> mats;
  int64_t blocks = 0;
  for (int64_t i = 0; i < n_mats; ++i) {
    const int64_t N = Ns[i], K = Ks[i];
    IH_REQUIRE(N >= 0 && K >= 0 && K % 2 == 0, INFERC_ERR_SHAPE, "int4 gemv: K must be even");
    if (N == 0) continue;
    IH_REQUIRE(y[i] && (K == 0 || (W[i] && scales[i] && x[i])), INFERC_ERR_ARG,
               "int4 gemv: null pointer");
    const bool fast = K > 0 && K % 32 == 0 && K / 32 <= kBlock && aligned16(W[i]) &&
                      aligned16(x[i]);
    if (!fast) {
      // Odd shapes run alone through the exact per-row kernel.
      const int64_t t = N * batch;
      hipLaunchKernelGGL(int4_gemv_generic, dim3(unsigned(ceil_div(t, kBlock))), dim3(kBlock), 0,
                         ctx->stream, W[i], scales[i], x[i], y[i], N, K, batch);
      check_launch("int4_gemv_generic");
      continue;
    }
    Int4Mat m{};
    m.W = W[i]; m.s = scales[i]; m.x = x[i]; m.y = y[i];
    m.N = N; m.K = K;
    m.cpr = int(K / 32);
    m.groups = kBlock / m.cpr;
    m.block_begin = blocks;
    blocks += ceil_div(N, int64_t(m.groups) * kRowsPerThread);
    mats.push_back(m);
  }
  if (mats.empty()) return;
  IH_REQUIRE(blocks < (int64_t(1) << 31), INFERC_ERR_SHAPE, "int4 gemv: launch too large");
  const Int4Mat* dev = upload_table(ctx, mats);
  hipLaunchKernelGGL(int4_gemv_kernel, dim3(unsigned(blocks)), dim3(kBlock), 0, ctx->stream, dev,
                     int(mats.size()), int(batch));
  check_launch("int4_gemv");
}

}  // namespace
}  // namespace ih

extern "C" {

int inferc_hip_gemv_f32(inferc_hip_ctx* ctx, int64_t N, int64_t K, const float* W,
                        const float* x, const float* ln_gamma, const float* ln_beta,
                        float ln_eps, const float* bias, const float* residual, int act,
                        float* y) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    ih::gemv(ctx, N, K, W, x, ln_gamma, ln_beta, ln_eps, bias, residual, act, y);
  });
}

int inferc_hip_int4_unpack(inferc_hip_ctx* ctx, int64_t N, int64_t K, const uint8_t* W,
                           const float* scales, float* out) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    IH_REQUIRE(N >= 0 && K >= 0 && K % 2 == 0, INFERC_ERR_SHAPE, "int4 unpack: K must be even");
    if (N == 0 || K == 0) return;
    IH_REQUIRE(W && scales && out, INFERC_ERR_ARG, "int4 unpack: null pointer");
    int64_t blocks = ih::ceil_div(N * (K / 2), ih::kBlock);
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(ih::int4_unpack_kernel, dim3(unsigned(blocks)), dim3(ih::kBlock), 0,
                       ctx->stream, W, scales, N, K, out);
    ih::check_launch("int4_unpack");
  });
}

int inferc_hip_int4_gemv(inferc_hip_ctx* ctx, int64_t N, int64_t K, const uint8_t* W,
                         const float* scales, int64_t batch, const float* x, float* y) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    ih::int4_grouped(ctx, 1, &N, &K, &W, &scales, batch, &x, &y);
  });
}

int inferc_hip_int4_gemv_grouped(inferc_hip_ctx* ctx, int64_t n_mats, const int64_t* Ns,
                                 const int64_t* Ks, const uint8_t* const* W,
                                 const float* const* scales, int64_t batch,
                                 const float* const* x, float* const* y) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    ih::int4_grouped(ctx, n_mats, Ns, Ks, W, scales, batch, x, y);
  });
}

}  // extern "C"
