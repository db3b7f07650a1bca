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
#include <algorithm>
#include <cmath>
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

// x (and LayerNorm's gamma and beta) for the lane's columns; the loads go
// out before any of them is used.
template <int KV, int XSRC>
__device__ __forceinline__ void gemv2_x_load(const float* ln_g, const float* ln_b, const float* x,
                                             int lane, float4 (&xv)[KV], float4 (&lg)[KV],
                                             float4 (&lb)[KV]) {
#pragma unroll
  for (int j = 0; j < KV; ++j) xv[j] = *reinterpret_cast<const float4*>(x + 4 * lane + 256 * j);
  if (XSRC == XSRC_LN) {
#pragma unroll
    for (int j = 0; j < KV; ++j) {
      lg[j] = *reinterpret_cast<const float4*>(ln_g + 4 * lane + 256 * j);
      lb[j] = *reinterpret_cast<const float4*>(ln_b + 4 * lane + 256 * j);
    }
  }
}

// x through the optional LayerNorm prologue
template <int KV, int XSRC>
__device__ __forceinline__ void gemv2_x(const Gemv2P& p, int lane, float4 (&xv)[KV],
                                        const float4 (&lg)[KV], const float4 (&lb)[KV]) {
  constexpr int K = 256 * KV;
  if (XSRC == XSRC_LN) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < KV; ++j) s += (xv[j].x + xv[j].y) + (xv[j].z + xv[j].w);
    const float mean = wave_sum_dpp(s) / float(K);
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < KV; ++j) {
      xv[j].x -= mean; xv[j].y -= mean; xv[j].z -= mean; xv[j].w -= mean;
      q += (xv[j].x * xv[j].x + xv[j].y * xv[j].y) + (xv[j].z * xv[j].z + xv[j].w * xv[j].w);
    }
    const float var = wave_sum_dpp(q) / float(K);
    const float inv = 1.0f / sqrtf(var + p.ln_eps);
#pragma unroll
    for (int j = 0; j < KV; ++j) {
      const float4 g = lg[j], b = lb[j];
      xv[j].x = (xv[j].x * inv) * g.x + b.x;
      xv[j].y = (xv[j].y * inv) * g.y + b.y;
      xv[j].z = (xv[j].z * inv) * g.z + b.z;
      xv[j].w = (xv[j].w * inv) * g.w + b.w;
    }
  }
}

// A weight chunk, streamed once per call: a nontemporal load (the `nt`
// cache policy) that does not displace reusable lines.
__device__ __forceinline__ float4 w_load_nt(const float* p) {
  typedef float v4 __attribute__((ext_vector_type(4)));
  const v4 v = __builtin_nontemporal_load(
      reinterpret_cast<const __attribute__((address_space(1))) v4*>(reinterpret_cast<uintptr_t>(p)));
  return make_float4(v.x, v.y, v.z, v.w);
}

template <int R, int KV, int XSRC, bool ARGMAX>
// W, x and N lead the arguments, then the LayerNorm terms, bias, residual
// and output: none of the kernel's loads waits on a scalar load of the
// argument block (leading arguments arrive in SGPRs). Only the epsilon, the
// activation and the arg-max partials come in p.
__global__ __launch_bounds__(kBlock) void gemv2_kernel(const float* __restrict__ W,
                                                      const float* __restrict__ x, int64_t N,
                                                      const float* __restrict__ ln_g,
                                                      const float* __restrict__ ln_b,
                                                      const float* __restrict__ bias,
                                                      const float* __restrict__ res, float* y,
                                                      Gemv2P p) {
  constexpr int K = 256 * KV;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = (int64_t(blockIdx.x) * kWaves + wave) * R;
  float4 w[R][KV];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t rc = r0 + i < N ? r0 + i : N - 1;  // rows past N: clamped, never stored
#pragma unroll
    for (int j = 0; j < KV; ++j)
      w[i][j] = w_load_nt(W + rc * K + 4 * lane + 256 * j);
  }
  float4 xv[KV], lg[KV], lb[KV];
  gemv2_x_load<KV, XSRC>(ln_g, ln_b, x, lane, xv, lg, lb);
  // the epilogue's bias and residual of the wave's rows (an absent operand
  // reads W instead)
  float bb[R], rr[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t rc = r0 + i < N ? r0 + i : N - 1;
    bb[i] = (bias ? bias : W)[bias ? rc : 0];
    rr[i] = (res ? res : W)[res ? rc : 0];
  }
  gemv2_x<KV, XSRC>(p, lane, xv, lg, lb);
  float acc[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < KV; ++j)
      a += w[i][j].x * xv[j].x + w[i][j].y * xv[j].y + w[i][j].z * xv[j].z + w[i][j].w * xv[j].w;
    acc[i] = wave_sum_dpp(a);
  }
  float bv = -INFINITY;
  int64_t bi = INT64_MAX;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t r = r0 + i;
    if (r < N) {
      float v = acc[i];
      if (bias) v = v + bb[i];
      if (res) v = v + rr[i];
      v = apply_act(v, p.act);
      if (lane == i) y[r] = v;
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

// Pointers read from a descriptor table are generic to the compiler, which
// then emits flat accesses that wait on both memory counters and serialise.
// They all point into device global memory, so access them as such.
// (The integer round trip makes the cast stick; a direct pointer cast is
// folded back to a generic access. Native vector types, not HIP's vector
// classes, can be read through an address-space-qualified pointer.)
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 gload_u4(const uint4* p) {
  const u32x4_t v = *reinterpret_cast<const __attribute__((address_space(1))) u32x4_t*>(
      reinterpret_cast<uintptr_t>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 gload_f4(const float4* p) {
  const f32x4_t v = *reinterpret_cast<const __attribute__((address_space(1))) f32x4_t*>(
      reinterpret_cast<uintptr_t>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ int64_t gload_i64(const int64_t* p) {
  return *reinterpret_cast<const __attribute__((address_space(1))) int64_t*>(
      reinterpret_cast<uintptr_t>(p));
}
// Streamed-once weights: nontemporal loads (the `nt` cache policy) keep them
// from displacing reusable lines and measure 7-14% faster for pure streaming
// reads on gfx950.
__device__ __forceinline__ uint4 gload_u4_nt(const uint4* p) {
  const u32x4_t v = __builtin_nontemporal_load(
      reinterpret_cast<const __attribute__((address_space(1))) u32x4_t*>(
          reinterpret_cast<uintptr_t>(p)));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t gload_u32_nt(const uint32_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const __attribute__((address_space(1))) uint32_t*>(
      reinterpret_cast<uintptr_t>(p)));
}
__device__ __forceinline__ float gload_f(const float* p) {
  return *reinterpret_cast<const __attribute__((address_space(1))) float*>(
      reinterpret_cast<uintptr_t>(p));
}
__device__ __forceinline__ void gstore_f(float* p, float v) {
  *reinterpret_cast<__attribute__((address_space(1))) float*>(reinterpret_cast<uintptr_t>(p)) = v;
}

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

// v & 0x0F0F0F0F with the result's known bits hidden from the optimiser: if
// it sees that the high nibble of every byte is zero, it rewrites each
// ubyte<N> of the result as a 4-bit field extract plus ubyte<0> (two
// instructions where v_cvt_f32_ubyteN alone suffices). For VALU consumers
// only: the compiler does not insert the wait states between a VALU write
// and a matrix-core read of the same register around inline assembly, and
// an MFMA fed by this value read stale operands in some schedules.
__device__ __forceinline__ uint32_t low_nibbles(uint32_t v) {
  uint32_t r;
  asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(r) : "v"(v));
  return r;
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
    if (active && r < m.N) w[j] = gload_u4_nt(reinterpret_cast<const uint4*>(m.W + r * rb + c * 16));
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
        const float4 xa = gload_f4(xp + 2 * q), xb = gload_f4(xp + 2 * q + 1);
        xsum += (xa.x + xa.y) + (xa.z + xa.w) + (xb.x + xb.y) + (xb.z + xb.w);
#pragma unroll
        for (int j = 0; j < kRowsPerThread; ++j) {
          const uint32_t word = (q == 0) ? w[j].x : (q == 1) ? w[j].y : (q == 2) ? w[j].z : w[j].w;
          const uint32_t ev = low_nibbles(word);       // nibbles of k = 8q + 0,2,4,6
          const uint32_t od = low_nibbles(word >> 4);  // nibbles of k = 8q + 1,3,5,7
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
    gstore_f(m.y + b * m.N + r, gload_f(m.s + r) * s);
  }
}

// Workgroup barrier for LDS data only: unlike __syncthreads it does not make
// the wave wait for its global loads still in flight.
__device__ __forceinline__ void lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Batch-1 int4 GEMV on the vector ALUs (the streaming form of the fp32
// GEMV). Rows are contiguous in memory and L lanes share a row (L a power of
// two, L * DW dwords = K/8): lane s owns dwords [DW*s, DW*s + DW) of every
// row it visits, i.e. 8*DW consecutive weights, so one load instruction
// covers 64/L whole consecutive rows. A chunk is kI4Passes passes of 64/L
// rows. Each wave streams a run of consecutive chunks of one matrix: it
// prepares its 8*DW x values once, then software-pipelines the run, issuing
// the loads of chunk c+2 before it computes chunk c+1 (a ring of two
// register buffers), so its memory requests stay in flight while it
// computes.
//
// The transformer row lengths (K = 768: DW 3, L 32; K = 3072: DW 6, L 64)
// run fully unrolled in int4_gemv_b1_kernel. Its blocks each cover one
// matrix, and their four waves stage that matrix's x in LDS once (a quarter
// each) instead of each wave fetching its slice from L2. Run lengths per
// wave are 18 KB at K = 3072, 15 KB for K = 768 matrices over kI4BigRows
// rows and 12 KB for the other K = 768 matrices, longest runs first in the
// launch: with 4 waves per SIMD (the register budget) the whole GPT-2 set
// is ~4300 waves, about one residency round, and the short runs last fill
// its tail. Other row lengths take int4_gemv_valu_kernel (run-time L,
// looped runs of about kI4RunKB).
//
// Arithmetic per dword w (8 nibbles, low nibble = even k): with
// e = w & 0x0F0F0F0F (even nibbles) and b_i = byte i of w = e_i + 16 o_i,
//   sum_i e_i x[2i] + o_i x[2i+1] = sum_i e_i (x[2i] - x[2i+1]/16)
//                                 + sum_i b_i (x[2i+1]/16),
// i.e. one mask, eight v_cvt_f32_ubyteN and eight FMAs per 8 weights (the
// x terms are prepared once per wave; x/16 is an exact power-of-two
// scaling for normal x). The -8 offset is
// folded: sum (nib-8) x = sum nib*x - 8*sum x.
//
// Reduction over the L lanes of a row, in a fixed order (deterministic).
// For a compile-time L >= 4 it is a reduce-scatter: two exchanges spread
// the chunk's 4 rows over the lanes (lane s ends up with row s / (L/4)),
// then log2(L/4) DPP steps finish the sums; lane s keeps chunk s % (L/4)
// of its run, so every result is stored once, after the loop (a store
// inside the pipelined loop would tie up registers the next loads need).
// Other L reduce all 4 rows over all L lanes and lane s keeps chunk s.
// The descriptors live in a device table; one launch serves every matrix
// of the unrolled forms (the wave's matrix picks the form, wave-uniformly),
// so matrices of both row lengths overlap instead of running back to back.
constexpr int kI4Passes = 4;
constexpr int kI4RunKB = 12;  // weights per wave of the unrolled run
constexpr int kI4Ring = 2;    // chunks in flight per wave

struct Int4VaDesc {
  const uint8_t* W;
  const float* s;
  const float* x;
  float* y;
  int64_t N, K;
  int64_t task_begin;  // first wave of this matrix in the launch
  int64_t dw;          // dwords per lane for this matrix
  int64_t chunks;      // chunks of this matrix
  int64_t per_wave;    // chunks per wave (the last wave may get fewer)
};

// Partner value across lane distance O (lane ^ O), for O < 16 by DPP. For
// O = 4 and 8 the DPP mirrors stand in for the exchange, which is exact
// only when the value is already uniform within groups of O lanes (true in
// the reductions below, which go from the smallest distance up).
template <int O>
__device__ __forceinline__ float lane_partner(float v) {
  if constexpr (O == 1 || O == 2) {
    constexpr int ctrl = O == 1 ? 0xB1 : 0x4E;  // quad_perm [1,0,3,2] / [2,3,0,1]
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, false));
  } else if constexpr (O == 4 || O == 8) {
    constexpr int ctrl = O == 4 ? 0x141 : 0x140;  // row_half_mirror / row_mirror
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, false));
  } else {
    return __shfl_xor(v, O, 64);
  }
}

template <int G, int O = 1>
__device__ __forceinline__ float group_sum(float v) {  // sum over lane groups of G
  if constexpr (O >= G) {
    return v;
  } else {
    return group_sum<G, 2 * O>(v + lane_partner<O>(v));
  }
}

template <int DW>
struct I4Chunk {
  uint32_t w[kI4Passes][DW];
  float sc;                // compile-time L: scale of the row this lane reports
  float sc4[kI4Passes];    // run-time L: scales of the chunk's 4 passes
};

// Loads one chunk. With keep = 0 (a chunk past the run's end) every lane
// reads the matrix's first dwords instead: one cache line per instruction,
// and the load stays unconditional so the wait counts stay exact (a branch
// around it would make the compiler wait for every load at the join).
template <int DW, int LT>
__device__ __forceinline__ void i4_load_chunk(I4Chunk<DW>& b, const Int4VaDesc& d, int64_t chunk,
                                              uint32_t keep, int rpp, int rg, int s) {
  // rows fit in 32 bits (the host checks N < 2^31); clamped to the last row
  const uint32_t rb = uint32_t(d.K / 2), last = uint32_t(d.N - 1);
  const uint32_t r0 = uint32_t(chunk) * (kI4Passes * rpp) + rg;
  const uint8_t* wl = d.W + ((4 * DW * s) & keep);
#pragma unroll
  for (int p = 0; p < kI4Passes; ++p) {
    const uint32_t r = min(r0 + uint32_t(p * rpp), last) & keep;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(wl + uint64_t(r) * rb);
#pragma unroll
    for (int q = 0; q < DW; ++q) b.w[p][q] = gload_u32_nt(src + q);
  }
  if constexpr (LT >= 4) {
    const int p = s / (LT / 4);
    b.sc = gload_f(d.s + (min(r0 + uint32_t(p * rpp), last) & keep));
  } else {
#pragma unroll
    for (int p = 0; p < kI4Passes; ++p)
      b.sc4[p] = gload_f(d.s + (min(r0 + uint32_t(p * rpp), last) & keep));
  }
}

template <int DW, int LT>
__device__ __forceinline__ void i4_chunk_rows(const I4Chunk<DW>& b, const float (&xe)[4 * DW],
                                              const float (&xo)[4 * DW], float xsum8, int L, int s,
                                              int j, float& res, float (&res4)[kI4Passes]) {
  float acc[kI4Passes];
#pragma unroll
  for (int p = 0; p < kI4Passes; ++p) {
    float t = -xsum8;
#pragma unroll
    for (int q = 0; q < DW; ++q) {
      const uint32_t w = b.w[p][q], e = low_nibbles(w);
      t += ubyte<0>(e) * xe[4 * q + 0];
      t += ubyte<0>(w) * xo[4 * q + 0];
      t += ubyte<1>(e) * xe[4 * q + 1];
      t += ubyte<1>(w) * xo[4 * q + 1];
      t += ubyte<2>(e) * xe[4 * q + 2];
      t += ubyte<2>(w) * xo[4 * q + 2];
      t += ubyte<3>(e) * xe[4 * q + 3];
      t += ubyte<3>(w) * xo[4 * q + 3];
    }
    acc[p] = t;
  }
  if constexpr (LT >= 4) {
    // reduce-scatter: distance L/2 splits rows {0,1} / {2,3}, L/4 splits again
    const bool h1 = s & (LT / 2), h2 = s & (LT / 4);
    float k0 = h1 ? acc[2] : acc[0], k1 = h1 ? acc[3] : acc[1];
    const float g0 = h1 ? acc[0] : acc[2], g1 = h1 ? acc[1] : acc[3];
    k0 += __shfl_xor(g0, LT / 2, 64);
    k1 += __shfl_xor(g1, LT / 2, 64);
    float k = h2 ? k1 : k0;
    k += __shfl_xor(h2 ? k0 : k1, LT / 4, 64);
    k = group_sum<LT / 4>(k);  // row s / (L/4) of this chunk, summed over its L lanes
    res = s % (LT / 4) == j ? b.sc * k : res;
  } else {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      if (o < L) {
#pragma unroll
        for (int p = 0; p < kI4Passes; ++p) acc[p] += __shfl_xor(acc[p], o, 64);
      }
    }
#pragma unroll
    for (int p = 0; p < kI4Passes; ++p) res4[p] = s == j ? b.sc4[p] * acc[p] : res4[p];
  }
}

template <int DW, int LT>
__device__ __forceinline__ void int4_valu_run(const Int4VaDesc& d, int64_t wid, int lane) {
  const int L = LT ? LT : int((d.K / 8) / DW), rpp = 64 / L;
  const int s = lane & (L - 1), rg = lane / L;
  const int64_t c0 = (wid - d.task_begin) * d.per_wave;
  const int64_t c1 = c0 + d.per_wave < d.chunks ? c0 + d.per_wave : d.chunks;
  const int n = int(c1 - c0);  // chunks in this run (the host bounds it by the lanes that keep results)

  auto keep = [&](int j) { return j < n ? ~0u : 0u; };
  I4Chunk<DW> A, B;
  i4_load_chunk<DW, LT>(A, d, c0, ~0u, rpp, rg, s);
  i4_load_chunk<DW, LT>(B, d, c0 + 1, keep(1), rpp, rg, s);
  float4 xv[2 * DW];
  const float4* xp = reinterpret_cast<const float4*>(d.x + 8 * DW * s);
#pragma unroll
  for (int q = 0; q < 2 * DW; ++q) xv[q] = gload_f4(xp + q);
  float xsum = 0.0f, xe[4 * DW], xo[4 * DW];
#pragma unroll
  for (int q = 0; q < 2 * DW; ++q) {
    xsum += (xv[q].x + xv[q].y) + (xv[q].z + xv[q].w);
    xo[2 * q] = xv[q].y * 0.0625f;
    xo[2 * q + 1] = xv[q].w * 0.0625f;
    xe[2 * q] = xv[q].x - xo[2 * q];
    xe[2 * q + 1] = xv[q].z - xo[2 * q + 1];
  }
  const float xsum8 = 8.0f * xsum;
  // Two chunks are in flight when the loop starts; each half-step computes
  // the older one and refills its buffer with the chunk two ahead, so one
  // chunk's loads are always outstanding while the other is computed.
  float res = 0.0f, res4[kI4Passes] = {};
  for (int j = 0; j < n; j += 2) {
    i4_chunk_rows<DW, LT>(A, xe, xo, xsum8, L, s, j, res, res4);
    if (j + 1 >= n) break;
    __builtin_amdgcn_sched_barrier(0);
    i4_load_chunk<DW, LT>(A, d, c0 + j + 2, keep(j + 2), rpp, rg, s);
    __builtin_amdgcn_sched_barrier(0);
    i4_chunk_rows<DW, LT>(B, xe, xo, xsum8, L, s, j + 1, res, res4);
    __builtin_amdgcn_sched_barrier(0);
    i4_load_chunk<DW, LT>(B, d, c0 + j + 3, keep(j + 3), rpp, rg, s);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (s < n) {
#pragma unroll
    for (int p = 0; p < kI4Passes; ++p) {
      const int64_t r = ((c0 + s) * kI4Passes + p) * rpp + rg;
      if (r < d.N) gstore_f(d.y + r, res4[p]);
    }
  }
}

// The run with a compile-time lane count L (>= 4) and NC chunks per wave,
// fully unrolled: straight-line code lets the compiler count every wait
// exactly (in a loop, copies of registers whose loads are still in flight
// make it wait for all of them). A matrix's last runs may hold fewer than NC
// chunks, or none (the waves that round a matrix up to whole blocks); the
// missing ones load the broadcast line and are not stored. x comes through
// xs: each of the block's kWaves waves loads a quarter of the matrix's x,
// and one LDS barrier (which leaves the weight loads in flight) publishes it.
template <int DW, int LT, int NC>
__device__ __forceinline__ void int4_valu_fixed(const Int4VaDesc& d, int64_t wid, int lane,
                                                float* xs) {
  static_assert(LT >= 4 && NC <= LT / 4, "a lane keeps one chunk's row");
  constexpr int rpp = 64 / LT, K = 8 * DW * LT;
  constexpr int F4 = K / 4 / kWaves, PER = (F4 + 63) / 64;  // x float4s per wave, per lane
  const int s = lane & (LT - 1), rg = lane / LT;
  const int wave = threadIdx.x >> 6;
  const int64_t c0 = (wid - d.task_begin) * NC;
  const int n = int(d.chunks - c0 < NC ? d.chunks - c0 : NC);  // <= 0: a rounding wave
  auto keep = [&](int j) { return j < n ? ~0u : 0u; };
  // x first: it is waited for (to be staged) while both chunks' loads,
  // issued after it, stay in flight
  float4 xl[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    xl[i] = gload_f4(reinterpret_cast<const float4*>(d.x) + wave * F4 + (e < F4 ? e : 0));
  }
  __builtin_amdgcn_sched_barrier(0);
  constexpr int R = NC < kI4Ring ? NC : kI4Ring;
  I4Chunk<DW> buf[R];
#pragma unroll
  for (int j = 0; j < R; ++j) i4_load_chunk<DW, LT>(buf[j], d, c0 + j, keep(j), rpp, rg, s);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    if (e < F4) reinterpret_cast<float4*>(xs)[wave * F4 + e] = xl[i];
  }
  lds_sync();
  float4 xv[2 * DW];
#pragma unroll
  for (int q = 0; q < 2 * DW; ++q) xv[q] = reinterpret_cast<const float4*>(xs + 8 * DW * s)[q];
  float xsum = 0.0f, xe[4 * DW], xo[4 * DW];
#pragma unroll
  for (int q = 0; q < 2 * DW; ++q) {
    xsum += (xv[q].x + xv[q].y) + (xv[q].z + xv[q].w);
    xo[2 * q] = xv[q].y * 0.0625f;
    xo[2 * q + 1] = xv[q].w * 0.0625f;
    xe[2 * q] = xv[q].x - xo[2 * q];
    xe[2 * q + 1] = xv[q].z - xo[2 * q + 1];
  }
  const float xsum8 = 8.0f * xsum;
  float res = 0.0f, res4[kI4Passes];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    __builtin_amdgcn_sched_barrier(0);
    i4_chunk_rows<DW, LT>(buf[j % R], xe, xo, xsum8, LT, s, j, res, res4);
    __builtin_amdgcn_sched_barrier(0);
    if (j + R < NC) i4_load_chunk<DW, LT>(buf[j % R], d, c0 + j + R, keep(j + R), rpp, rg, s);
  }
  const int j = s % (LT / 4), p = s / (LT / 4);
  const int64_t r = ((c0 + j) * kI4Passes + p) * rpp + rg;
  if (j < n && r < d.N) gstore_f(d.y + r, res);
}

// Run lengths of int4_gemv_b1_kernel in chunks per wave (a sweep of run
// lengths on the 49-matrix GPT-2 set, measured on the box).
constexpr int kI4NcK3072 = 3;            // 18 KB
constexpr int kI4NcK768 = 4;             // 12 KB
constexpr int kI4NcK768Big = 5;          // 15 KB
constexpr int64_t kI4BigRows = 8192;     // "big": more rows than this
static_assert(kI4NcK768 != kI4NcK768Big, "the run length tells the K = 768 forms apart");

// Index of the descriptor whose waves hold wave `wid` (task_begin ascends):
// one ballot per 64 entries.
__device__ __forceinline__ int i4_find_desc(const Int4VaDesc* tab, int n, int64_t wid, int lane) {
  int cnt = 0;
  for (int base = 0; base < n; base += 64) {
    const int j = base + lane;
    const int c = __popcll(__ballot(j < n && gload_i64(&tab[j].task_begin) <= wid));
    cnt += c;
    if (c < 64) break;
  }
  return __builtin_amdgcn_readfirstlane(cnt - 1);
}

// The unrolled forms (K = 768 and 3072) in one launch; each matrix's waves
// are rounded up to whole blocks, so the grid is exactly the waves.
__global__ __launch_bounds__(kBlock) void int4_gemv_b1_kernel(const Int4VaDesc* __restrict__ tab,
                                                              int n) {
  __shared__ __attribute__((aligned(16))) float xs[3072];
  const int lane = threadIdx.x & 63;
  const int64_t wid = int64_t(blockIdx.x) * kWaves +
                      __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const Int4VaDesc d = tab[i4_find_desc(tab, n, wid, lane)];
  if (d.dw == 6)
    int4_valu_fixed<6, 64, kI4NcK3072>(d, wid, lane, xs);
  else if (d.per_wave == kI4NcK768Big)
    int4_valu_fixed<3, 32, kI4NcK768Big>(d, wid, lane, xs);
  else
    int4_valu_fixed<3, 32, kI4NcK768>(d, wid, lane, xs);
}

// Other row lengths: DW dwords per lane, L from K at run time, looped runs.
template <int DW>
__global__ __launch_bounds__(kBlock) void int4_gemv_valu_kernel(const Int4VaDesc* __restrict__ tab,
                                                               int n, int64_t n_waves) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = int64_t(blockIdx.x) * kWaves +
                      __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  if (wid >= n_waves) return;
  int4_valu_run<DW, 0>(tab[i4_find_desc(tab, n, wid, lane)], wid, lane);
}

// Batch-1 int4 GEMV of one matrix for the decode step: the unrolled run of
// int4_valu_fixed with the step's fusions around it.
//   - LayerNorm prologue (ln_g set; the K = 768 form): every wave reduces
//     the whole x row (mean, then the centred second moment, as LayerNorm)
//     and normalises its own slice before the weight arithmetic.
//   - Epilogue per row, in the fp32 GEMV's order: v = s_r*acc + bias +
//     residual, then the activation; y may alias the residual (each row is
//     read and written by the same lane).
//   - amax set (the LM head): each wave also stores the first maximum
//     (value, row) of its rows, for the step's finishing kernel (y may be
//     null then).
// The pointers and sizes the first loads need lead the kernel's arguments,
// which then arrive in SGPRs; the rest come in Int4DecP.
struct Int4DecP {
  float* y;
  ValIdxPart* amax;
  float ln_eps;
  int act;
};

// One wave per block: a decode-step matrix (1.7 to 2.4 MB of int4) is a few
// hundred waves, which then land on as many CUs.
constexpr int kI4DecBlock = 64;

template <int DW, int LT, int NC>
__global__ __launch_bounds__(kI4DecBlock) void int4_gemv_dec_kernel(
    const uint8_t* __restrict__ W, const float* __restrict__ sc, const float* __restrict__ x,
    const float* __restrict__ ln_g, const float* __restrict__ ln_b,
    const float* __restrict__ bias, const float* resid, int32_t N, int32_t chunks, Int4DecP p) {
  static_assert(LT >= 4 && NC <= LT / 4, "a lane keeps one chunk's row");
  constexpr int K = 8 * DW * LT, rpp = 64 / LT;
  const int lane = threadIdx.x & 63;
  const int64_t wid = blockIdx.x;  // the grid is exactly the matrix's waves
  const Int4VaDesc d{W, sc, x, p.y, N, K, 0, DW, chunks, NC};
  const int s = lane & (LT - 1), rg = lane / LT;
  const int64_t c0 = wid * NC;
  const int n = int(d.chunks - c0 < NC ? d.chunks - c0 : NC);
  auto keep = [&](int j) { return j < n ? ~0u : 0u; };

  float4 xv[2 * DW];
  const float4* xp = reinterpret_cast<const float4*>(d.x + 8 * DW * s);
#pragma unroll
  for (int q = 0; q < 2 * DW; ++q) xv[q] = gload_f4(xp + q);
  constexpr int PL = K / 64;  // x values per lane for the row statistics
  float xs[PL];
  if (ln_g) {
#pragma unroll
    for (int i = 0; i < PL; ++i) xs[i] = gload_f(d.x + lane + 64 * i);
  }
  __builtin_amdgcn_sched_barrier(0);
  I4Chunk<DW> buf[2];
  i4_load_chunk<DW, LT>(buf[0], d, c0, ~0u, rpp, rg, s);
  if constexpr (NC > 1) i4_load_chunk<DW, LT>(buf[1], d, c0 + 1, keep(1), rpp, rg, s);
  __builtin_amdgcn_sched_barrier(0);
  // the row this lane reports, and its bias and residual, fetched behind the
  // weights so the epilogue waits on no memory (unconditional: an absent
  // operand reads the scales instead)
  const int jr = s % (LT / 4), pr = s / (LT / 4);
  const int64_t r = ((c0 + jr) * kI4Passes + pr) * rpp + rg;
  const int64_t rc = r < d.N ? r : d.N - 1;
  const float bpre = gload_f((bias ? bias : d.s) + (bias ? rc : 0));
  const float rpre = gload_f((resid ? resid : d.s) + (resid ? rc : 0));
  __builtin_amdgcn_sched_barrier(0);
  if (ln_g) {
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < PL; ++i) sum += xs[i];
    const float mean = wave_sum_dpp(sum) / float(K);
    float q2 = 0.0f;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const float dd = xs[i] - mean;
      q2 += dd * dd;
    }
    const float inv = 1.0f / sqrtf(wave_sum_dpp(q2) / float(K) + p.ln_eps);
    const float4* gp = reinterpret_cast<const float4*>(ln_g + 8 * DW * s);
    const float4* bp = reinterpret_cast<const float4*>(ln_b + 8 * DW * s);
#pragma unroll
    for (int q = 0; q < 2 * DW; ++q) {
      const float4 g = gload_f4(gp + q), b = gload_f4(bp + q);
      xv[q].x = ((xv[q].x - mean) * inv) * g.x + b.x;
      xv[q].y = ((xv[q].y - mean) * inv) * g.y + b.y;
      xv[q].z = ((xv[q].z - mean) * inv) * g.z + b.z;
      xv[q].w = ((xv[q].w - mean) * inv) * g.w + b.w;
    }
  }
  float xsum = 0.0f, xe[4 * DW], xo[4 * DW];
#pragma unroll
  for (int q = 0; q < 2 * DW; ++q) {
    xsum += (xv[q].x + xv[q].y) + (xv[q].z + xv[q].w);
    xo[2 * q] = xv[q].y * 0.0625f;
    xo[2 * q + 1] = xv[q].w * 0.0625f;
    xe[2 * q] = xv[q].x - xo[2 * q];
    xe[2 * q + 1] = xv[q].z - xo[2 * q + 1];
  }
  const float xsum8 = 8.0f * xsum;
  float res = 0.0f, res4[kI4Passes];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    __builtin_amdgcn_sched_barrier(0);
    i4_chunk_rows<DW, LT>(buf[j & 1], xe, xo, xsum8, LT, s, j, res, res4);
    __builtin_amdgcn_sched_barrier(0);
    if (j + 2 < NC) i4_load_chunk<DW, LT>(buf[j & 1], d, c0 + j + 2, keep(j + 2), rpp, rg, s);
  }
  const bool valid = jr < n && r < d.N;
  float v = res;
  if (valid) {
    if (bias) v += bpre;
    if (resid) v += rpre;
    v = apply_act(v, p.act);
  }
  if (valid && d.y) gstore_f(d.y + r, v);
  if (p.amax == nullptr) return;
  // first maximum of the wave's rows (a NaN never wins, as in the fp32 head)
  float bv = valid ? v : -INFINITY;
  int64_t bi = valid ? r : INT64_MAX;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float w = __shfl_xor(bv, o, 64);
    const int64_t wi = __shfl_xor(bi, o, 64);
    if (w > bv || (w == bv && wi < bi)) {
      bv = w;
      bi = wi;
    }
  }
  if (lane == 0) p.amax[wid] = ValIdxPart{bv, bi};
}

// int4 GEMV on the int8 matrix cores, exact in integer arithmetic.
//
// The dequantised product is y[b][r] = s_r * sum_k (nib - 8) x[b][k]. The
// kernel computes sum_k nib * x - 8 * sum_k x exactly:
//   - nibbles (0..15) are int8 operands as they sit in memory, after one
//     mask (even k) or shift+mask (odd k) per dword;
//   - x[b] becomes a fixed-point integer X = rint(x * 2^F), with F chosen from
//     max|x[b]| so that |X| < 2^30, split into four signed int8 limbs
//     X = d0 + 2^8 d1 + 2^16 d2 + 2^24 d3;
//   - v_mfma_i32_16x16x64_i8 multiplies 16 rows of nibbles with 16 columns of
//     limbs (4 limbs x up to 4 batches) and accumulates exactly in int32;
//   - each limb's integer sum (below 2^24) converts exactly to fp32 and is
//     scaled by an exact power of two; y = s_r * (sum of the 4 limb terms).
// The approximations are x's rounding to 2^-F (about 2^-30 of max|x[b]|) and
// the last few fp32 roundings: the long sum over k itself is exact, closer
// to the reference's double accumulation (int4_gemv_amx.cc:258-271) than an
// fp32 dot product.
//
// Layout. A "unit" is 16 rows of one matrix. In step t (128 k) lane (r, g)
// (r = lane%16, g = lane/16) loads the 16 bytes of row r at byte 64t + 16g:
// 32 nibbles, 16 even-k and 16 odd-k, the A operands of two MFMAs. The MFMA
// pairs A byte j of lane group g with B byte j of lane group g; B byte j of
// lane (c, g) is limb c%4 of x[c/4][128t + 32g + 2j] (+1 for the odd MFMA).
// The B operands depend only on x, so a block writes them to LDS once per
// matrix and reuses them for every unit it streams.
//
// Scheduling. One launch per K (= 128*STEPS, so registers are sized
// exactly). A block owns a few units and issues all of their weight loads
// first; the x preparation then overlaps those loads. For long rows two
// waves share a unit, each taking half of K, and add their exact partial
// sums through LDS. The matrix descriptors live in a device table (uploaded
// once, cached): a multi-kilobyte kernel argument would be copied by a blit
// before every launch of a captured graph.
constexpr int kI4MaxK = 3072;      // B operands in LDS: K * 16 bytes
constexpr int kI4Batch = 4;        // batches per pass: 4 limbs x 4 = 16 columns

typedef int i32x4_t __attribute__((ext_vector_type(4)));

struct Int4MfDesc {
  const uint8_t* W;
  const float* s;
  const float* x;  // [nb, K] (this pass's batches)
  float* y;        // [nb, N]
  int64_t N;
  int64_t block_begin;  // first block of this matrix in the launch
};

// Work split for K = 128*STEPS. KS waves share a unit (16 rows), each taking
// STEPS/KS of the steps, so long rows still give enough blocks; a wave group
// owns RBW units. Rows per block = (4/KS) * RBW * 16.
__host__ __device__ constexpr int i4_ks(int steps) { return steps >= 16 ? 2 : 1; }
__host__ __device__ constexpr int i4_rbw(int steps) { return steps >= 6 ? 1 : steps >= 4 ? 2 : 4; }
__host__ __device__ constexpr int i4_rows_per_block(int steps) {
  return (kBlock / 64 / i4_ks(steps)) * i4_rbw(steps) * 16;
}
__host__ __device__ constexpr bool i4_steps_ok(int steps) {
  return steps == 2 || steps == 4 || steps == 6 || steps == 8 || steps == 12 || steps == 16 ||
         steps == 24;
}

struct I4Shared {
  uint32_t bop[kI4MaxK * 4];  // B operands: [step][even/odd][lane][4 dwords]
  float smax[kBlock / 64][kI4Batch];
  i32x4_t part[kBlock / 64][64];  // K-split partial sums (one unit per wave)
};

// Quad-lane exchange (lanes 4i..4i+3) without LDS: DPP quad permutes.
template <int XOR>
__device__ __forceinline__ float quad_xor_f(float v) {
  constexpr int ctrl = XOR == 1 ? 0xB1 : 0x4E;  // quad_perm [1,0,3,2] / [2,3,0,1]
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, false));
}

template <int STEPS>
__global__ __launch_bounds__(kBlock) void int4_gemv_mfma_kernel(const Int4MfDesc* __restrict__ tab,
                                                               int n, int nb) {
  constexpr int KS = i4_ks(STEPS), RBW = i4_rbw(STEPS), SPW = STEPS / KS;
  constexpr int K = 128 * STEPS, KPT = K / kBlock;  // x values per thread per batch
  static_assert(K % kBlock == 0, "K must split evenly over the block");
  __shared__ __attribute__((aligned(16))) I4Shared sh;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave / KS, part = wave % KS;
  const int r = lane & 15, g = lane >> 4;
  const int64_t bid = blockIdx.x;
  // This block's matrix: how many table entries start at or before bid
  // (block_begin ascends), one ballot per 64 entries.
  int cnt = 0;
  for (int base = 0; base < n; base += 64) {
    const int j = base + lane;
    const int c = __popcll(__ballot(j < n && gload_i64(&tab[j].block_begin) <= bid));
    cnt += c;
    if (c < 64) break;
  }
  const Int4MfDesc d = tab[__builtin_amdgcn_readfirstlane(cnt - 1)];
  const int64_t N = d.N;
  const int64_t r0 = (bid - d.block_begin) * i4_rows_per_block(STEPS) + int64_t(grp) * RBW * 16;

  // 1. every weight this wave needs, its rows' scales, this thread's x
  uint4 w[RBW][SPW];
#pragma unroll
  for (int rb = 0; rb < RBW; ++rb) {
    const int64_t row = r0 + rb * 16 + r;
    const uint8_t* rp = d.W + (row < N ? row : N - 1) * int64_t(K / 2);
#pragma unroll
    for (int t = 0; t < SPW; ++t)
      w[rb][t] = gload_u4_nt(reinterpret_cast<const uint4*>(rp + 64 * (part * SPW + t) + 16 * g));
  }
  float scv[RBW][4];
#pragma unroll
  for (int rb = 0; rb < RBW; ++rb)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t row = r0 + rb * 16 + 4 * g + v;
      scv[rb][v] = gload_f(d.s + (row < N ? row : N - 1));
    }
  float xr[kI4Batch][KPT];
#pragma unroll
  for (int b = 0; b < kI4Batch; ++b)
#pragma unroll
    for (int i = 0; i < KPT; ++i)
      xr[b][i] = b < nb ? gload_f(d.x + int64_t(b) * K + tid + kBlock * i) : 0.0f;

  // 2. x -> fixed-point limbs in the B-operand layout (overlaps the weights)
  for (int i = tid; i < K; i += kBlock)  // unused columns stay zero
    *reinterpret_cast<uint4*>(sh.bop + 4 * i) = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
  for (int b = 0; b < kI4Batch; ++b) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      // fmaxf would drop a NaN, so a non-finite |x| enters the maximum as inf
      const float ax = fabsf(xr[b][i]);
      m = ax <= 3.4028235e38f ? fmaxf(m, ax) : INFINITY;
    }
    m = wave_max(m);
    if (lane == 0) sh.smax[wave][b] = m;
  }
  __syncthreads();
  int F[kI4Batch];
  bool finite[kI4Batch];
#pragma unroll
  for (int b = 0; b < kI4Batch; ++b) {
    float m = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < kBlock / 64; ++w2) m = fmaxf(m, sh.smax[w2][b]);
    finite[b] = m <= 3.4028235e38f;
    if (!finite[b]) m = 0.0f;
    int e = 0;
    (void)frexpf(m, &e);  // m < 2^e
    F[b] = m > 0.0f ? 30 - e : 0;
  }
  uint8_t* bb = reinterpret_cast<uint8_t*>(sh.bop);
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int k = tid + kBlock * i;
    const int st = k >> 7, kk = k & 127, gg = kk >> 5, q = kk & 31;
    const int eo = q & 1, j = q >> 1;
#pragma unroll
    for (int b = 0; b < kI4Batch; ++b) {
      if (b >= nb) break;
      int X = finite[b] ? int(rintf(ldexpf(xr[b][i], F[b]))) : 0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int dg = c < 3 ? ((X + 128) & 255) - 128 : X;  // balanced digit; top in [-64, 64]
        X = (X - dg) >> 8;
        bb[(((2 * st + eo) * 64 + (4 * b + c) + 16 * gg) * 16) + j] = uint8_t(int8_t(dg));
      }
    }
  }
  __syncthreads();

  // 3. the fold term sum_k X per column: an MFMA with an all-ones A
  const i32x4_t ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
  i32x4_t fold = {0, 0, 0, 0};
#pragma unroll
  for (int t = 0; t < STEPS; ++t) {
    const i32x4_t be = *reinterpret_cast<const i32x4_t*>(sh.bop + ((2 * t) * 64 + lane) * 4);
    const i32x4_t bo = *reinterpret_cast<const i32x4_t*>(sh.bop + ((2 * t + 1) * 64 + lane) * 4);
    fold = __builtin_amdgcn_mfma_i32_16x16x64_i8(ones, be, fold, 0, 0, 0);
    fold = __builtin_amdgcn_mfma_i32_16x16x64_i8(ones, bo, fold, 0, 0, 0);
  }

  // 4. this wave's steps of each of its units
  i32x4_t acc[RBW];
#pragma unroll
  for (int rb = 0; rb < RBW; ++rb) {
    acc[rb] = i32x4_t{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < SPW; ++t) {
      const int st = part * SPW + t;
      const uint4 q = w[rb][t];
      const i32x4_t ev = {int(q.x & 0x0F0F0F0Fu), int(q.y & 0x0F0F0F0Fu), int(q.z & 0x0F0F0F0Fu),
                          int(q.w & 0x0F0F0F0Fu)};
      const i32x4_t od = {int((q.x >> 4) & 0x0F0F0F0Fu), int((q.y >> 4) & 0x0F0F0F0Fu),
                          int((q.z >> 4) & 0x0F0F0F0Fu), int((q.w >> 4) & 0x0F0F0F0Fu)};
      const i32x4_t be = *reinterpret_cast<const i32x4_t*>(sh.bop + ((2 * st) * 64 + lane) * 4);
      const i32x4_t bo = *reinterpret_cast<const i32x4_t*>(sh.bop + ((2 * st + 1) * 64 + lane) * 4);
      acc[rb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ev, be, acc[rb], 0, 0, 0);
      acc[rb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(od, bo, acc[rb], 0, 0, 0);
    }
  }
  if constexpr (KS > 1) {
    static_assert(RBW == 1, "a K-split wave owns one unit");
    // the other K parts hand their exact partial sums to part 0
    if (part != 0) sh.part[wave][lane] = acc[0];
    __syncthreads();
    if (part != 0) return;
#pragma unroll
    for (int p2 = 1; p2 < KS; ++p2) acc[0] += sh.part[wave + p2][lane];
  }

  // 5. acc[rb][v]: row 4g+v of unit rb, column col = (batch cb, limb cl). Each
  //    limb term acc - 8*fold is below 2^24 in magnitude, so it and its
  //    power-of-two scaling are exact in fp32; a batch's 4 terms (a lane
  //    quad) are summed in fp32.
  const int col = lane & 15, cb = col >> 2, cl = col & 3;
  int Fc = 0;
  bool okc = true;
#pragma unroll
  for (int b = 0; b < kI4Batch; ++b) {
    Fc = b == cb ? F[b] : Fc;
    okc = b == cb ? finite[b] : okc;
  }
  const int sh_exp = 8 * cl - Fc;
#pragma unroll
  for (int rb = 0; rb < RBW; ++rb)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float t = ldexpf(float(acc[rb][v] - 8 * fold[v]), sh_exp);
      t += quad_xor_f<1>(t);
      t += quad_xor_f<2>(t);
      const int64_t row = r0 + rb * 16 + 4 * g + v;
      if (cl == 0 && cb < nb && row < N)
        // a non-finite x makes the whole output non-finite, as in the reference
        gstore_f(d.y + int64_t(cb) * N + row, okc ? scv[rb][v] * t : __int_as_float(0x7fc00000));
    }
}

constexpr int kI4SlabK = 768;                 // k per slab: one fixed-point scale
constexpr int kI4SlabSteps = kI4SlabK / 128;  // 128 k (64 bytes of a row) per MFMA step

// int4 GEMV for batches 2-8 with K = 768 * S (S = 1, 2 or 4): the exact
// integer arithmetic of int4_gemv_mfma_kernel (x to fixed point per 768-k
// slab, 4 balanced int8 limbs, v_mfma_i32_16x16x64_i8, the -8 offset through
// each column's limb sum), one launch for every matrix of the call, one
// long-lived block per CU:
// - A block owns T tiles of 16 rows per wave group of one matrix. Its NW
//   waves split into NW / S groups of S waves; wave w streams slab w % S of
//   its group's tiles, so every wave reads 384-byte row pieces whatever K.
// - At its start the block turns x into the B operands of every (slab,
//   column group) in LDS (S x G x 12 KB), wave by (batch, slab): three
//   coalesced 1 KB loads, the slab's largest |x| and the columns' limb sums
//   by DPP within the wave, the digit records written as 16-bit pieces. The
//   first R tiles' weights are already in flight meanwhile.
// - Each wave then runs its T tiles through a ring of R in flight: a tile's
//   MFMAs, the next load into its slot, its epilogue. A slab's limb terms
//   acc - 8 fold (below 2^24, exact in fp32) are scaled by 2^(8 limb - F);
//   with S > 1 the group's S waves meet in LDS and add their terms in slab
//   order, then a batch's 4 limbs (a lane quad) add and the row's scale
//   applies. The outputs collect in LDS ([batch][row of the block]).
// - At its end the block stores its rows of every batch, 256 consecutive
//   bytes per store instruction (measured: 16.3 -> 15.8 us on the 49-matrix
//   GPT-2 set at batch 8, against 16-row pieces stored after each tile).
// Each block reads its own descriptor (one scalar load): at a launch's start
// every dependent load is a full memory round trip.
struct I4B8Block {
  const uint8_t* W;
  const float* s;
  const float* x;  // [batch][K]
  float* y;        // [batch][N]
  int32_t N;
  int32_t S;     // slabs per row
  int32_t rblk;  // this block's row block of the matrix
  int32_t unused;
};

// Wave-wide reductions through DPP within rows of 16 lanes, then the four
// rows' lanes 0, 16, 32 and 48 (every lane must be active).
__device__ __forceinline__ int wave_max_bits(int v) {
  v = max(v, __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false));   // quad [1,0,3,2]
  v = max(v, __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false));   // quad [2,3,0,1]
  v = max(v, __builtin_amdgcn_mov_dpp(v, 0x124, 0xF, 0xF, false));  // row_ror:4
  v = max(v, __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, false));  // row_ror:8
  return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ int wave_sum_int(int v) {
  v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
  v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);
  v += __builtin_amdgcn_mov_dpp(v, 0x124, 0xF, 0xF, false);
  v += __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, false);
  return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
         (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}

template <int G, int NW, int ROWS>
struct I4B8Smem {
  // B operands: [slab][step][parity][group][lane][16 bytes]
  __attribute__((aligned(16))) uint32_t bop[4 * kI4SlabSteps * 2 * G * 64 * 4];
  int sfold[4][G][16];  // per slab and column: the sum of its limbs
  int sF[4][4 * G];     // per slab and batch: x scaled by 2^F before rounding
  int sfin[4][4 * G];   // per slab and batch: 0 if x holds a NaN or inf
  // the block's outputs, [batch][row of the block], stored at its end
  __attribute__((aligned(16))) float yblk[4 * G][ROWS];
};

// One block of int4_gemv_b8_kernel for rows of S slabs: each wave runs U
// units (16-row tile, slab), the slabs of a tile in order, through a ring of
// R; RE of them go out before the x preparation.
//
// Every vector memory instruction in the loop is issued unconditionally. On
// this GPU loads and stores return in issue order under one counter, and the
// compiler cannot count an instruction behind a branch: the wait for the next
// unit would then also wait for as many later loads as such stores issued,
// draining the ring. So S is a template parameter (no branch around a tile's
// epilogue), and the outputs collect in LDS and leave at the block's end, as
// whole rows of each batch.
template <int G, int S, int U, int R, int RE, int NW, int ROWS>
__device__ __forceinline__ void int4_b8_block(I4B8Smem<G, NW, ROWS>& sm, const I4B8Block& d,
                                              int batch) {
  constexpr int ST = kI4SlabSteps;  // 6 MFMA steps of 128 k per slab
  constexpr int NB = 4 * G;         // batch columns
  constexpr int SMAX = 4;
  constexpr int TASKS = (NB * SMAX + NW - 1) / NW;  // (batch, slab) preparations per wave
  constexpr int SLAB = ST * 2 * G * 64 * 4;         // dwords of one slab's B operands
  auto& bop = sm.bop;
  auto& sfold = sm.sfold;
  auto& sF = sm.sF;
  auto& sfin = sm.sfin;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int ls = S == 4 ? 2 : S == 2 ? 1 : 0;  // log2 of the slabs per row
  static_assert(U % S == 0, "whole tiles per wave");
  const int64_t N = d.N, K = int64_t(kI4SlabK) * S, rb = K / 2;
  const int64_t tile0 = d.rblk * (U >> ls);  // this block's first tile per wave
  const int r = lane & 15, g = lane >> 4, col = lane & 15, cl = col & 3;
  // unit u: tile (tile0 + u / S) * NW + wave, slab u % S
  auto tile_of = [&](int u) { return (tile0 + (u >> ls)) * NW + wave; };
  // the block's rows: [row0, row0 + BROWS), tiles tile0 * NW .. (tile0 + U/S) * NW - 1
  constexpr int BROWS = (U / S) * NW * 16;
  static_assert(BROWS <= ROWS, "the block's outputs must fit its LDS stage");
  const int64_t row0 = tile0 * NW * 16;

  // 1. x loads of this wave's (batch, slab) tasks: lane l of piece j holds
  //    positions 256 j + 4 l + e (e < 4) of the slab. Idle tasks load the
  //    first piece of x and drop it: a load under a branch would make the
  //    wave wait for it.
  float4 xv[TASKS][3];
#pragma unroll
  for (int k = 0; k < TASKS; ++k) {
    const int task = wave + NW * k, tb = task % NB, tq = task / NB;
    const bool on = tq < S && tb < batch;
    const float4* xs = reinterpret_cast<const float4*>(
        d.x + (on ? int64_t(tb) * K + kI4SlabK * tq : 0));
#pragma unroll
    for (int j = 0; j < 3; ++j) xv[k][j] = gload_f4(xs + 64 * j + lane);
  }
  __builtin_amdgcn_sched_barrier(0);
  // Every wave's x requests go out before any weight request of the block:
  // a CU serves its waves' loads in issue order, and x queued behind the
  // other waves' first units held up the preparation. A bare s_barrier
  // leaves the loads in flight.
  asm volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  // the ring: slot j holds a unit's 6 steps (lane (r, g): row 16 i + r,
  // bytes [384 q + 64 t + 16 g, +16)) and, with the slab-0 unit of a tile,
  // the scale of row 16 i + r; rows past N are clamped and never stored
  uint4 wb[R][ST];
  float sb[R];
  auto load_unit = [&](int slot, int u) {
    int64_t row = tile_of(u) * 16 + r;
    row = row < N ? row : N - 1;
    const int q = u & (S - 1);
    const uint8_t* rp = d.W + row * rb + kI4SlabK / 2 * q + 16 * g;
#pragma unroll
    for (int t = 0; t < ST; ++t) wb[slot][t] = gload_u4(reinterpret_cast<const uint4*>(rp + 64 * t));
    if (q == 0) sb[slot] = gload_f(d.s + row);
  };
  constexpr int R0 = R < U ? R : U, E0 = RE < R0 ? RE : R0;
#pragma unroll
  for (int j = 0; j < E0; ++j) load_unit(j, j);
  __builtin_amdgcn_sched_barrier(0);

  // 2. the B operands
#pragma unroll
  for (int k = 0; k < TASKS; ++k) {
    const int task = wave + NW * k, b = task % NB, tq = task / NB;
    if (tq >= S) break;  // wave-uniform
    const bool on = b < batch;
    const int gr = b / 4, bb = b % 4;
    // the slab's largest |x| as the largest bits of |x| (non-negative floats
    // order as their bits; NaN and inf lie above every finite value), and F
    int mb = 0;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      mb = max(mb, __float_as_int(xv[k][j].x) & 0x7fffffff);
      mb = max(mb, __float_as_int(xv[k][j].y) & 0x7fffffff);
      mb = max(mb, __float_as_int(xv[k][j].z) & 0x7fffffff);
      mb = max(mb, __float_as_int(xv[k][j].w) & 0x7fffffff);
    }
    mb = on ? wave_max_bits(mb) : 0;
    const bool fin = mb < 0x7f800000;
    const float mm = fin ? __int_as_float(mb) : 0.0f;
    int e = 0;
    (void)frexpf(mm, &e);  // mm < 2^e, so |x * 2^(30-e)| < 2^30
    const int F = mm > 0.0f ? 30 - e : 0;
    // Balanced base-256 digits of X = rint(x 2^F) (three in [-128, 127],
    // the top one in [-64, 64]): with Y = X + 0x808080 the low three are
    // Y's bytes minus 128 and the top one is Y >> 24, so the digits' bytes
    // are exactly the bytes of Z = Y ^ 0x808080 (byte - 128 = byte ^ 0x80
    // modulo 256). A batch past the call's or with a non-finite x gets
    // digits that no output uses.
    // Record (t, eo, gr, lane' = 4 bb + c + 16 kg) of the slab holds in byte
    // jj limb c of x[b][128 t + 32 kg + 2 jj + eo]. Lane l of piece j holds
    // e = 0..3 at t = 2 j + l / 32, kg = (l % 32) / 8, jj = 2 (l % 8) +
    // e / 2, eo = e % 2: per parity, the 16-bit piece at byte 2 (l % 8) of
    // limb c's record is [limb c of e = eo, limb c of e = eo + 2].
    int fsum[4] = {0, 0, 0, 0};
    uint8_t* recs = reinterpret_cast<uint8_t*>(bop) + tq * (ST * 2 * G * 64 * 16);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const float vals[4] = {xv[k][j].x, xv[k][j].y, xv[k][j].z, xv[k][j].w};
      uint32_t Z[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        Z[u] = uint32_t(int(rintf(ldexpf(vals[u], F))) + 0x808080) ^ 0x808080u;
      const int t = 2 * j + lane / 32, kg = (lane % 32) / 8;
#pragma unroll
      for (int eo = 0; eo < 2; ++eo) {
        // [Z_eo.b0, Z_eo+2.b0, Z_eo.b1, Z_eo+2.b1] and the same for bytes 2, 3
        const uint32_t p01 = __builtin_amdgcn_perm(Z[eo + 2], Z[eo], 0x05010400u);
        const uint32_t p23 = __builtin_amdgcn_perm(Z[eo + 2], Z[eo], 0x07030602u);
        fsum[0] = __builtin_amdgcn_sdot4(int(p01), 0x00000101, fsum[0], false);
        fsum[1] = __builtin_amdgcn_sdot4(int(p01), 0x01010000, fsum[1], false);
        fsum[2] = __builtin_amdgcn_sdot4(int(p23), 0x00000101, fsum[2], false);
        fsum[3] = __builtin_amdgcn_sdot4(int(p23), 0x01010000, fsum[3], false);
        uint8_t* rec = recs + (((t * 2 + eo) * G + gr) * 64 + 4 * bb + 16 * kg) * 16 + 2 * (lane % 8);
        *reinterpret_cast<uint16_t*>(rec + 0 * 16) = uint16_t(p01);
        *reinterpret_cast<uint16_t*>(rec + 1 * 16) = uint16_t(p01 >> 16);
        *reinterpret_cast<uint16_t*>(rec + 2 * 16) = uint16_t(p23);
        *reinterpret_cast<uint16_t*>(rec + 3 * 16) = uint16_t(p23 >> 16);
      }
    }
    // the columns' limb sums over the slab: exact integers
#pragma unroll
    for (int c = 0; c < 4; ++c) fsum[c] = wave_sum_int(fsum[c]);
    if (lane == 0) {
#pragma unroll
      for (int c = 0; c < 4; ++c) sfold[tq][gr][4 * bb + c] = fsum[c];
      sF[tq][b] = F;
      sfin[tq][b] = on ? int(fin) : 1;
    }
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = E0; j < R0; ++j) load_unit(j, j);
  __builtin_amdgcn_sched_barrier(0);
  lds_sync();

  // 3. the units through the ring; a tile's slab terms add in slab order in
  //    registers, then its epilogue
  const __amdgpu_buffer_rsrc_t ybuf =
      __builtin_amdgcn_make_buffer_rsrc(d.y, 0, int(batch * N * int64_t(sizeof(float))), 0x00020000);
  f32x4_t tv[G];
  float scale = 0.0f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int slot = u % R, q = u & (S - 1);
    const uint32_t* bq = bop + q * SLAB;
    i32x4_t acc[G];
#pragma unroll
    for (int gr = 0; gr < G; ++gr) acc[gr] = i32x4_t{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < ST; ++t) {
      const uint4 w = wb[slot][t];
      // plain masks, not low_nibbles: these feed the matrix cores
      const i32x4_t ev = {int(w.x & 0x0F0F0F0Fu), int(w.y & 0x0F0F0F0Fu), int(w.z & 0x0F0F0F0Fu),
                          int(w.w & 0x0F0F0F0Fu)};
      const i32x4_t od = {int((w.x >> 4) & 0x0F0F0F0Fu), int((w.y >> 4) & 0x0F0F0F0Fu),
                          int((w.z >> 4) & 0x0F0F0F0Fu), int((w.w >> 4) & 0x0F0F0F0Fu)};
#pragma unroll
      for (int gr = 0; gr < G; ++gr) {
        const u32x4_t e4 = *reinterpret_cast<const u32x4_t*>(bq + (((t * 2 + 0) * G + gr) * 64 + lane) * 4);
        const u32x4_t o4 = *reinterpret_cast<const u32x4_t*>(bq + (((t * 2 + 1) * G + gr) * 64 + lane) * 4);
        acc[gr] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
            ev, i32x4_t{int(e4.x), int(e4.y), int(e4.z), int(e4.w)}, acc[gr], 0, 0, 0);
        acc[gr] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
            od, i32x4_t{int(o4.x), int(o4.y), int(o4.z), int(o4.w)}, acc[gr], 0, 0, 0);
      }
    }
    if (q == 0) scale = sb[slot];
    __builtin_amdgcn_sched_barrier(0);
    if (u + R < U) load_unit(slot, u + R);
    __builtin_amdgcn_sched_barrier(0);
    // acc[gr][v]: row 16 i + 4 g + v, column (batch 4 gr + col / 4, limb
    // cl). A limb term acc - 8 fold is below 2^24, so it and its power-of-two
    // scaling are exact in fp32; a slab whose x is not finite gives NaN, so
    // the whole output row is non-finite, as in the reference.
#pragma unroll
    for (int gr = 0; gr < G; ++gr) {
      const int b = 4 * gr + (col >> 2);
      const int fold = sfold[q][gr][col], ex = 8 * cl - sF[q][b];
      const bool fin = sfin[q][b] != 0;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float term = fin ? ldexpf(float(acc[gr][v] - 8 * fold), ex) : __int_as_float(0x7fc00000);
        tv[gr][v] = q == 0 ? term : tv[gr][v] + term;
      }
    }
    if (q == S - 1) {
      // a batch's 4 limb terms (a lane quad) add in fp32, times the rows'
      // scales (from lanes 4 g + v); lane (4 bb, g) then holds rows 4 g ..
      // 4 g + 3 of batch 4 gr + bb, kept in LDS until the block's end
      const int lrow = int(tile_of(u) * 16 - row0);
      float sc[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) sc[v] = __shfl(scale, 4 * g + v, 64);
#pragma unroll
      for (int gr = 0; gr < G; ++gr) {
        const int b = 4 * gr + (col >> 2);
        f32x4_t o;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float t2 = tv[gr][v];
          t2 += quad_xor_f<1>(t2);
          t2 += quad_xor_f<2>(t2);
          o[v] = sc[v] * t2;
        }
        if (cl == 0) *reinterpret_cast<f32x4_t*>(&sm.yblk[b][lrow + 4 * g]) = o;
      }
    }
  }
  // The block's rows of every batch, 256 consecutive bytes per store
  // instruction; nontemporal (streaming) stores, and offsets past the buffer
  // for rows past N and batches past the call's, which the hardware drops.
  __syncthreads();
#pragma unroll
  for (int k = 0; k < (4 * G * BROWS + 64 * NW - 1) / (64 * NW); ++k) {
    const int e = tid + 64 * NW * k;
    const int b = e / BROWS, r = e % BROWS;
    const int64_t row = row0 + r;
    const bool on = e < 4 * G * BROWS && b < batch && row < N;
    const float v = sm.yblk[on ? b : 0][on ? r : 0];
    const int off = on ? int((int64_t(b) * N + row) * int64_t(sizeof(float))) : int(0x80000000u);
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), ybuf, off, 0, 2 /* nt */);
  }
}
// U1 units per wave for K = 768 and 1536, U4 for K = 3072 (whose blocks
// prepare four slabs of x and so stream fewer units).
template <int G, int U1, int U4, int R, int RE, int NW>
__global__ __launch_bounds__(64 * NW) void int4_gemv_b8_kernel(const I4B8Block* __restrict__ tab,
                                                               int batch) {
  constexpr int ROWS = U1 * NW * 16;  // the most rows a block covers (K = 768)
  __shared__ I4B8Smem<G, NW, ROWS> sm;
  const I4B8Block d = tab[blockIdx.x];
  if (d.S == 4)
    int4_b8_block<G, 4, U4, R, RE, NW, ROWS>(sm, d, batch);
  else if (d.S == 2)
    int4_b8_block<G, 2, U1, R, RE, NW, ROWS>(sm, d, batch);
  else
    int4_b8_block<G, 1, U1, R, RE, NW, ROWS>(sm, d, batch);
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
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, g, b, 0, s, p.W, p.x, p.N, p.ln_g, p.ln_b, p.bias, p.res, p.y, p);
  };
  if (argmax) {
    if (xsrc == XSRC_LN) go(gemv2_kernel<R, KV, XSRC_LN, true>);
    else go(gemv2_kernel<R, KV, XSRC_PLAIN, true>);
    return;
  }
  if (xsrc == XSRC_LN) go(gemv2_kernel<R, KV, XSRC_LN, false>);
  else go(gemv2_kernel<R, KV, XSRC_PLAIN, false>);
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

// The context's device copy of a launch's descriptor table. The launch calls
// ctx->reserve_tables() with its table count before the first upload.
template <class T>
const T* upload_table(inferc_hip_ctx* ctx, const std::vector<T>& mats) {
  return static_cast<const T*>(ctx->table(mats.data(), mats.size() * sizeof(T)));
}

struct Int4MfMat {
  const uint8_t* W;
  const float* s;
  const float* x;
  float* y;
  int64_t N, K;
};

// Shapes the int8-MFMA kernel takes: K = 128*STEPS for a supported STEPS,
// 16-byte aligned rows.
bool int4_mfma_ok(int64_t K, const uint8_t* W) {
  return K > 0 && K % 128 == 0 && K <= kI4MaxK && i4_steps_ok(int(K / 128)) && aligned16(W);
}

template <int STEPS>
void launch_int4_mfma_k(inferc_hip_ctx* ctx, const std::vector<Int4MfMat>& mats, int64_t batch) {
  if (mats.empty()) return;
  for (int64_t b0 = 0; b0 < batch; b0 += kI4Batch) {
    const int nb = int(std::min<int64_t>(kI4Batch, batch - b0));
    std::vector<Int4MfDesc> tab;
    int64_t blocks = 0;
    for (const Int4MfMat& m : mats) {
      Int4MfDesc dsc{};
      dsc.W = m.W; dsc.s = m.s;
      dsc.x = m.x + b0 * m.K;
      dsc.y = m.y + b0 * m.N;
      dsc.N = m.N;
      dsc.block_begin = blocks;
      blocks += ceil_div(m.N, int64_t(i4_rows_per_block(STEPS)));
      tab.push_back(dsc);
    }
    IH_REQUIRE(blocks < (int64_t(1) << 31) && tab.size() < (size_t(1) << 20), INFERC_ERR_SHAPE,
               "int4 gemv: launch too large");
    ctx->reserve_tables(1);
    const Int4MfDesc* dev = upload_table(ctx, tab);
    hipLaunchKernelGGL(int4_gemv_mfma_kernel<STEPS>, dim3(unsigned(blocks)), dim3(kBlock), 0,
                       ctx->stream, dev, int(tab.size()), nb);
    check_launch("int4_gemv_mfma");
  }
}

// Groups the matrices by K and launches each group.
void launch_int4_mfma(inferc_hip_ctx* ctx, const std::vector<Int4MfMat>& mats, int64_t batch) {
  std::vector<Int4MfMat> by_k[kI4MaxK / 128 + 1];
  for (const Int4MfMat& m : mats) by_k[m.K / 128].push_back(m);
  launch_int4_mfma_k<2>(ctx, by_k[2], batch);
  launch_int4_mfma_k<4>(ctx, by_k[4], batch);
  launch_int4_mfma_k<6>(ctx, by_k[6], batch);
  launch_int4_mfma_k<8>(ctx, by_k[8], batch);
  launch_int4_mfma_k<12>(ctx, by_k[12], batch);
  launch_int4_mfma_k<16>(ctx, by_k[16], batch);
  launch_int4_mfma_k<24>(ctx, by_k[24], batch);
}

// Shapes of the streaming MFMA kernel: K = 768 * S with S = 1, 2 or 4 and
// 16-byte aligned rows (x must be 16-byte aligned too).
bool int4_stream_ok(int64_t K, const uint8_t* W) {
  const int64_t S = K / kI4SlabK;
  return K > 0 && K % kI4SlabK == 0 && (S == 1 || S == 2 || S == 4) && aligned16(W);
}

constexpr int kI4B8Units = 6;   // (tile, slab) units per wave, K = 768 and 1536
constexpr int kI4B8Units4 = 4;  // and K = 3072
constexpr int kI4B8Ring = 2;    // units in flight per wave
constexpr int kI4B8Early = 1;   // of which issued before the x preparation
constexpr int kI4B8Waves = 8;   // waves per block
static_assert(kI4B8Units % 2 == 0 && kI4B8Units4 % 4 == 0, "whole tiles per wave");

// One int4_gemv_b8_kernel launch over every matrix; a block covers
// 16 x (units / S) x kI4B8Waves rows of one matrix.
template <int G>
void launch_int4_b8(inferc_hip_ctx* ctx, const std::vector<Int4MfMat>& mats, int batch) {
  std::vector<I4B8Block> tab;
  for (const Int4MfMat& m : mats) {
    const int64_t S = m.K / kI4SlabK;
    // buffer-store offsets of the output are 31-bit byte counts (int4_grouped
    // sends larger outputs to the int8-MFMA kernel)
    IH_REQUIRE(m.N * batch * int64_t(sizeof(float)) < (int64_t(1) << 31), INFERC_ERR_SHAPE,
               "int4 gemv: output too large for the batched kernel");
    const int64_t tiles = (S == 4 ? kI4B8Units4 : kI4B8Units) / S;
    const int64_t rblocks = ceil_div(m.N, 16 * tiles * kI4B8Waves);
    for (int64_t rbk = 0; rbk < rblocks; ++rbk)
      tab.push_back(I4B8Block{m.W, m.s, m.x, m.y, int32_t(m.N), int32_t(S), int32_t(rbk), 0});
  }
  IH_REQUIRE(tab.size() < (size_t(1) << 31), INFERC_ERR_SHAPE, "int4 gemv: launch too large");
  ctx->reserve_tables(1);
  const I4B8Block* dev = upload_table(ctx, tab);
  hipLaunchKernelGGL((int4_gemv_b8_kernel<G, kI4B8Units, kI4B8Units4, kI4B8Ring, kI4B8Early,
                                          kI4B8Waves>),
                     dim3(unsigned(tab.size())), dim3(64 * kI4B8Waves), 0, ctx->stream, dev, batch);
  check_launch("int4_gemv_b8");
}

void launch_int4_stream(inferc_hip_ctx* ctx, const std::vector<Int4MfMat>& mats, int64_t batch) {
  if (mats.empty()) return;
  if (batch <= 4)
    launch_int4_b8<1>(ctx, mats, int(batch));
  else
    launch_int4_b8<2>(ctx, mats, int(batch));
}

// Dwords per lane for the VALU kernel: L = (K/8)/DW lanes per row must be a
// power of two no larger than 64. 0 if none fits.
int int4_valu_dw(int64_t K) {
  if (K <= 0 || K % 8) return 0;
  const int64_t dwords = K / 8;
  for (int dw : {3, 6, 2, 4}) {
    if (dwords % dw) continue;
    const int64_t l = dwords / dw;
    if (l >= 1 && l <= 64 && (l & (l - 1)) == 0) return dw;
  }
  return 0;
}

// Lanes per row of the VALU kernel for a given K and DW.
int64_t int4_valu_lanes(int64_t K, int dw) { return (K / 8) / dw; }

// One int4_gemv_b1_kernel launch over the K = 768 and K = 3072 matrices,
// longest runs first (K = 3072, then the big K = 768 matrices, then the
// rest); each matrix's waves are rounded up to whole blocks.
void launch_int4_b1(inferc_hip_ctx* ctx, const std::vector<Int4MfMat>& k3072,
                    const std::vector<Int4MfMat>& k768) {
  if (k3072.empty() && k768.empty()) return;
  std::vector<Int4VaDesc> tab;
  int64_t waves = 0;
  auto add = [&](const Int4MfMat& m, int dw, int nc) {
    const int64_t L = int4_valu_lanes(m.K, dw);
    const int64_t chunks = ceil_div(m.N, int64_t(kI4Passes) * (64 / L));
    tab.push_back(Int4VaDesc{m.W, m.s, m.x, m.y, m.N, m.K, waves, dw, chunks, nc});
    waves += ceil_div(ceil_div(chunks, nc), kWaves) * kWaves;
  };
  for (const Int4MfMat& m : k3072) add(m, 6, kI4NcK3072);
  for (const Int4MfMat& m : k768)
    if (m.N > kI4BigRows) add(m, 3, kI4NcK768Big);
  for (const Int4MfMat& m : k768)
    if (m.N <= kI4BigRows) add(m, 3, kI4NcK768);
  IH_REQUIRE(waves / kWaves < (int64_t(1) << 31), INFERC_ERR_SHAPE, "int4 gemv: launch too large");
  ctx->reserve_tables(1);
  const Int4VaDesc* dev = upload_table(ctx, tab);
  hipLaunchKernelGGL(int4_gemv_b1_kernel, dim3(unsigned(waves / kWaves)), dim3(kBlock), 0,
                     ctx->stream, dev, int(tab.size()));
  check_launch("int4_gemv_b1");
}

// One int4_gemv_valu_kernel<DW> launch (run-time lane count): every wave
// streams about kI4RunKB of weights, bounded by the lanes that keep a run's
// results.
template <int DW>
void launch_int4_valu_generic(inferc_hip_ctx* ctx, const std::vector<Int4MfMat>& mats) {
  if (mats.empty()) return;
  std::vector<Int4VaDesc> tab;
  int64_t waves = 0;
  for (const Int4MfMat& m : mats) {
    const int64_t L = int4_valu_lanes(m.K, DW);
    const int64_t chunks = ceil_div(m.N, int64_t(kI4Passes) * (64 / L));
    const int64_t chunk_bytes = int64_t(kI4Passes) * 64 * DW * 4;
    const int64_t per_wave =
        std::min<int64_t>(L, std::max<int64_t>(1, kI4RunKB * 1024 / chunk_bytes));
    tab.push_back(Int4VaDesc{m.W, m.s, m.x, m.y, m.N, m.K, waves, DW, chunks, per_wave});
    waves += ceil_div(chunks, per_wave);
  }
  IH_REQUIRE(ceil_div(waves, kWaves) < (int64_t(1) << 31), INFERC_ERR_SHAPE,
             "int4 gemv: launch too large");
  ctx->reserve_tables(1);
  const Int4VaDesc* dev = upload_table(ctx, tab);
  hipLaunchKernelGGL(int4_gemv_valu_kernel<DW>, dim3(unsigned(ceil_div(waves, kWaves))),
                     dim3(kBlock), 0, ctx->stream, dev, int(tab.size()), waves);
  check_launch("int4_gemv_valu");
}

void launch_int4_valu(inferc_hip_ctx* ctx, const std::vector<Int4MfMat>& mats) {
  // the transformer forms (K = 768: DW 3, L 32; K = 3072: DW 6, L 64) share
  // one unrolled launch; the rest run per DW with a run-time lane count
  std::vector<Int4MfMat> k768, k3072, by_dw[7];
  for (const Int4MfMat& m : mats) {
    const int dw = int4_valu_dw(m.K);
    if (dw == 3 && int4_valu_lanes(m.K, 3) == 32)
      k768.push_back(m);
    else if (dw == 6 && int4_valu_lanes(m.K, 6) == 64)
      k3072.push_back(m);
    else
      by_dw[dw].push_back(m);
  }
  launch_int4_b1(ctx, k3072, k768);
  launch_int4_valu_generic<2>(ctx, by_dw[2]);
  launch_int4_valu_generic<3>(ctx, by_dw[3]);
  launch_int4_valu_generic<4>(ctx, by_dw[4]);
  launch_int4_valu_generic<6>(ctx, by_dw[6]);
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
  std::vector<Int4MfMat> mf;  // int8-MFMA form
  std::vector<Int4MfMat> va;  // batch-1 VALU streaming form
  std::vector<Int4MfMat> st;  // streaming int8-MFMA form (K = 768, 1536, 3072)
  int64_t blocks = 0;
  for (int64_t i = 0; i < n_mats; ++i) {
    const int64_t N = Ns[i], K = Ks[i];
    IH_REQUIRE(N >= 0 && K >= 0 && K % 2 == 0, INFERC_ERR_SHAPE, "int4 gemv: K must be even");
    if (N == 0) continue;
    IH_REQUIRE(y[i] && (K == 0 || (W[i] && scales[i] && x[i])), INFERC_ERR_ARG,
               "int4 gemv: null pointer");
    const bool fast = K > 0 && K % 32 == 0 && K / 32 <= kBlock && aligned16(W[i]) &&
                      aligned16(x[i]);
    // batch 1: the VALU streaming kernel (read the fewest bytes per output);
    // several batches: the int8 matrix-core kernel (VALU work would grow with
    // the batch, matrix-core work barely does)
    if (batch == 1 && int4_valu_dw(K) > 0 && N < (int64_t(1) << 31) && aligned16(x[i]) &&
        (reinterpret_cast<uintptr_t>(W[i]) & 3) == 0) {
      va.push_back(Int4MfMat{W[i], scales[i], x[i], y[i], N, K});
      continue;
    }
    // (its output is addressed with 31-bit buffer offsets)
    if (int4_stream_ok(K, W[i]) && aligned16(x[i]) &&
        N * batch * int64_t(sizeof(float)) < (int64_t(1) << 31)) {
      st.push_back(Int4MfMat{W[i], scales[i], x[i], y[i], N, K});
      continue;
    }
    if (int4_mfma_ok(K, W[i])) {
      mf.push_back(Int4MfMat{W[i], scales[i], x[i], y[i], N, K});
      continue;
    }
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
  launch_int4_valu(ctx, va);
  launch_int4_stream(ctx, st, batch);
  launch_int4_mfma(ctx, mf, batch);
  if (mats.empty()) return;
  IH_REQUIRE(blocks < (int64_t(1) << 31), INFERC_ERR_SHAPE, "int4 gemv: launch too large");
  ctx->reserve_tables(1);
  const Int4Mat* dev = upload_table(ctx, mats);
  hipLaunchKernelGGL(int4_gemv_kernel, dim3(unsigned(blocks)), dim3(kBlock), 0, ctx->stream, dev,
                     int(mats.size()), int(batch));
  check_launch("int4_gemv");
}

}  // namespace

// Chunks per wave of the decode-step int4 GEMV: one (the least latency) for
// the layers' matrices, a 12 KB run for the LM head (a 19 MB stream).
int int4_dec_chunks(int64_t N, int64_t K) {
  return N * K / 2 > (int64_t(8) << 20) ? kI4RunKB / (K == 768 ? 3 : 6) : 1;
}

// Waves of the decode-step int4 GEMV for an [N, K] matrix (also the number
// of argmax partials it writes); 0 when K is not a supported row length.
int64_t int4_dec_waves(int64_t N, int64_t K) {
  if (K != 768 && K != 3072) return 0;
  const int64_t rows_per_chunk = int64_t(kI4Passes) * (K == 768 ? 2 : 1);
  return ceil_div(ceil_div(N, rows_per_chunk), int4_dec_chunks(N, K));
}

void int4_quantize_rows(int64_t N, int64_t K, const float* w, uint8_t* packed, float* scales,
                        float* deq) {
  IH_REQUIRE(N >= 0 && K >= 0 && K % 2 == 0, INFERC_ERR_SHAPE, "int4 quantize: K must be even");
  IH_REQUIRE(N == 0 || K == 0 || (w && packed && scales), INFERC_ERR_ARG,
             "int4 quantize: null pointer");
  for (int64_t r = 0; r < N; ++r) {
    const float* wr = w + r * K;
    float m = 0.0f;
    for (int64_t k = 0; k < K; ++k) m = std::max(m, std::fabs(wr[k]));
    const float sc = m / 7.0f;
    scales[r] = sc;
    for (int64_t k = 0; k < K; k += 2) {
      int q[2];
      for (int e = 0; e < 2; ++e) {
        const float t = sc > 0.0f ? std::nearbyint(wr[k + e] / sc) : 0.0f;
        q[e] = int(std::min(7.0f, std::max(-8.0f, t)));
        if (deq) deq[r * K + k + e] = sc * float(q[e]);
      }
      packed[r * (K / 2) + k / 2] = uint8_t((q[0] + 8) | ((q[1] + 8) << 4));
    }
  }
}

void int4_gemv_dec(inferc_hip_ctx* ctx, int64_t N, int64_t K, const uint8_t* W,
                   const float* scales, const float* x, const float* ln_g, const float* ln_b,
                   float ln_eps, const float* bias, const float* res, int act, float* y,
                   ValIdxPart* amax) {
  IH_REQUIRE(int4_dec_waves(N, K) > 0 && N > 0 && N < (int64_t(1) << 31), INFERC_ERR_UNSUPPORTED,
             "int4 decode GEMV: K must be 768 or 3072");
  IH_REQUIRE(W && scales && x && (y || amax), INFERC_ERR_ARG, "int4 decode GEMV: null pointer");
  IH_REQUIRE((reinterpret_cast<uintptr_t>(W) & 3) == 0 && aligned16(x), INFERC_ERR_ARG,
             "int4 decode GEMV: W must be 4-byte and x 16-byte aligned");
  IH_REQUIRE(!ln_g || (K == 768 && ln_b && aligned16(ln_g) && aligned16(ln_b)), INFERC_ERR_ARG,
             "int4 decode GEMV: LayerNorm needs K = 768 and aligned gamma/beta");
  const int dw = K == 768 ? 3 : 6, nc = int4_dec_chunks(N, K);
  const int64_t L = K / 8 / dw, chunks = ceil_div(N, int64_t(kI4Passes) * (64 / L));
  const int64_t waves = int4_dec_waves(N, K);
  const Int4DecP p{y, amax, ln_eps, act};
  const int32_t n32 = int32_t(N), c32 = int32_t(chunks);
  const dim3 grid{unsigned(waves)}, block{unsigned(kI4DecBlock)};
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, block, 0, ctx->stream, W, scales, x, ln_g, ln_b, bias, res, n32,
                       c32, p);
  };
  if (dw == 3 && nc == 1)
    go(int4_gemv_dec_kernel<3, 32, 1>);
  else if (dw == 3)
    go(int4_gemv_dec_kernel<3, 32, kI4RunKB / 3>);
  else if (nc == 1)
    go(int4_gemv_dec_kernel<6, 64, 1>);
  else
    go(int4_gemv_dec_kernel<6, 64, kI4RunKB / 6>);
  check_launch("int4_gemv_dec");
}


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

int inferc_int4_quantize_rows(int64_t N, int64_t K, const float* w, uint8_t* packed,
                              float* scales, float* deq) {
  return ih::guard([&] { ih::int4_quantize_rows(N, K, w, packed, scales, deq); });
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
