// Attention over a key/value cache: the FusedAttentionPast node that the
// additive-attention pass makes of GPT-2's with-past decoder block
// (present = Concat(past, new); softmax(q K^T * scale + mask) V; the
// reference runs this block unfused and renames present.* to past.* between
// decode steps, src/cli/main.cpp:831-888).
//
// Cache layout: head-major [B, nH, max_t, dh] floats, the layout of the
// GPT-2 decoder's device cache. S new query rows attend over T = P + S keys
// (P cached before the call).
//
// cache_attention: one 64-lane wave per (batch, head, query row), four rows
// per 256-thread block. Keys are taken 64 at a time: each lane scores one key
// (dot product over dh with the query row held in LDS), a first sweep finds
// the row maximum, a second recomputes the scores, turns them into
// exp(s - max) and accumulates sum_j e_j V[j] with lanes over dh (coalesced
// rows of V), and the result is scaled by 1/sum at the end. Masked scores
// take `fill` as in FusedAttention (src/kernels/attention.cc:77-91).
// head_dim 64 (GPT-2) takes cache_attn_d64_kernel below.
#include "common.h"
#include "ew.h"

namespace ih {

namespace {

constexpr int kCaWaves = 4;
constexpr int kCaMaxDh = 256;

__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__global__ __launch_bounds__(64 * kCaWaves) void cache_attn_kernel(CacheAttnArgs p, float scale) {
  __shared__ float qs[kCaWaves][kCaMaxDh];
  __shared__ float es[kCaWaves][64];
  const int wave = int(threadIdx.x) / 64, lane = int(threadIdx.x) % 64;
  const int64_t rows = p.B * p.nH * p.S;
  const int64_t row = int64_t(blockIdx.x) * kCaWaves + wave;
  const bool live = row < rows;
  const int64_t r = live ? row : 0;
  const int64_t i = r % p.S, h = (r / p.S) % p.nH, b = r / (p.S * p.nH);
  const int dh = int(p.dh);
  const float* qrow = p.q + (b * p.S + i) * p.ldq + h * p.dh;
  for (int d = lane; d < dh; d += 64) qs[wave][d] = live ? qrow[d] : 0.0f;
  __syncthreads();
  const float* kbase = p.kc + (b * p.nH + h) * p.max_t * p.dh;
  const float* vbase = p.vc + (b * p.nH + h) * p.max_t * p.dh;
  const uint8_t* mrow = p.mask ? p.mask + b * p.ms[0] + h * p.ms[1] + i * p.ms[2] : nullptr;
  const int64_t T = p.pos ? *p.pos + p.S : p.T;
  auto score = [&](int64_t j) {
    const float* kr = kbase + j * p.dh;
    float s = 0.0f;
    for (int d = 0; d < dh; ++d) s += qs[wave][d] * kr[d];
    s *= scale;
    if (mrow && mrow[j * p.ms[3]]) s = p.fill;
    return s;
  };
  float mx = -INFINITY;
  for (int64_t j0 = 0; j0 < T; j0 += 64) {
    const int64_t j = j0 + lane;
    if (live && j < T) mx = fmaxf(mx, score(j));
  }
  mx = wave_max(mx);
  float part = 0.0f;
  float acc[kCaMaxDh / 64] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int64_t j0 = 0; j0 < T; j0 += 64) {
    const int64_t j = j0 + lane;
    const float e = (live && j < T) ? expf(score(j) - mx) : 0.0f;
    part += e;
    es[wave][lane] = e;
    __syncthreads();
    const int n = int(T - j0 < 64 ? T - j0 : 64);
    if (live) {
      for (int k = 0; k < n; ++k) {
        const float ek = es[wave][k];
        const float* vr = vbase + (j0 + k) * p.dh;
#pragma unroll
        for (int c = 0; c < kCaMaxDh / 64; ++c) {
          const int d = lane + 64 * c;
          if (d < dh) acc[c] += ek * vr[d];
        }
      }
    }
    __syncthreads();
  }
  const float inv = 1.0f / wave_sum(part);
  if (!live) return;
  float* orow = p.out + (b * p.S + i) * p.ldo + h * p.dh;
#pragma unroll
  for (int c = 0; c < kCaMaxDh / 64; ++c) {
    const int d = lane + 64 * c;
    if (d < dh) orow[d] = acc[c] * inv;
  }
}

// The same attention for head_dim 64: one block of 8 waves per (batch,
// head, query row). Wave w takes key chunks w, w+8, ... of 32 keys; in a
// chunk lane pair (2c, 2c+1) holds key c, each lane half of its 64 dims as
// eight float4, so a key row is one coalesced 256-byte read and a chunk's
// K and V loads (indices past the last key clamped to it, their weights
// zero) all go out before any is used. Per chunk: the scores (a masked key
// scores `fill`), their maximum m, e_j = exp(s_j - m), l = sum e_j and
// O = sum e_j v_j over the wave's 64 dims, merged online within the wave and
// across the eight waves through LDS in wave order; out = O / L.
// With kn/vn given, the new rows (keys P .. T-1) are read from there, and
// wave 0 of the block of query row i appends row P + i of its head to the
// cache (no read of the cache depends on that write).
constexpr int kCa64Waves = 8;
constexpr int kCa64Chunk = 32;

__global__ __launch_bounds__(64 * kCa64Waves) void cache_attn_d64_kernel(CacheAttnArgs p,
                                                                        float scale) {
  constexpr int D = 64;
  __shared__ float sm[kCa64Waves], sl[kCa64Waves];
  __shared__ float so[kCa64Waves][D];
  __shared__ __align__(16) float se[kCa64Waves][kCa64Chunk];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r = blockIdx.x;  // (b, h, i), i fastest
  const int64_t i = r % p.S, h = (r / p.S) % p.nH, b = r / (p.S * p.nH);
  const int64_t P = p.pos ? *p.pos : p.T - p.S, T = P + p.S;
  float* kcache = const_cast<float*>(p.kc) + (b * p.nH + h) * p.max_t * D;
  float* vcache = const_cast<float*>(p.vc) + (b * p.nH + h) * p.max_t * D;
  const float* kbase = kcache;
  const float* vbase = vcache;
  // new rows: key j >= P is row j - P of kn / vn (their head's 64 columns)
  const float* knb = p.kn ? p.kn + b * p.S * p.ldn + h * D : nullptr;
  const float* vnb = p.vn ? p.vn + b * p.S * p.ldn + h * D : nullptr;
  if (p.kn && wave == 0) {
    kcache[(P + i) * D + lane] = knb[i * p.ldn + lane];
    vcache[(P + i) * D + lane] = vnb[i * p.ldn + lane];
  }
  const uint8_t* mrow = p.mask ? p.mask + b * p.ms[0] + h * p.ms[1] + i * p.ms[2] : nullptr;
  const int dh = (lane & 1) * 32;
  const float* qrow = p.q + (b * p.S + i) * p.ldq + h * D;
  float4 qv[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) qv[k] = *reinterpret_cast<const float4*>(qrow + dh + 4 * k);
  float M = -INFINITY, L = 0.0f, O = 0.0f;
  for (int64_t j0 = int64_t(wave) * kCa64Chunk; j0 < T; j0 += kCa64Waves * kCa64Chunk) {
    const int64_t jl = j0 + (lane >> 1);
    const int64_t jc = jl < T ? jl : T - 1;
    const float* kr = knb && jc >= P ? knb + (jc - P) * p.ldn : kbase + jc * D;
    float4 kv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) kv[k] = *reinterpret_cast<const float4*>(kr + dh + 4 * k);
    float vv[kCa64Chunk];
#pragma unroll
    for (int k = 0; k < kCa64Chunk; ++k) {
      const int64_t jv = j0 + k < T ? j0 + k : T - 1;
      vv[k] = vnb && jv >= P ? vnb[(jv - P) * p.ldn + lane] : vbase[jv * D + lane];
    }
    const bool masked = mrow != nullptr && mrow[jc * p.ms[3]] != 0;
    float dot = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      dot += qv[k].x * kv[k].x + qv[k].y * kv[k].y + qv[k].z * kv[k].z + qv[k].w * kv[k].w;
    dot += dpp_pair_swap(dot);
    const float s = jl < T ? (masked ? p.fill : dot * scale) : -INFINITY;
    const float m = wave_max_dpp(s);
    const float e = jl < T ? expf(s - m) : 0.0f;
    const float l = wave_sum_dpp((lane & 1) ? 0.0f : e);
    // e_k of the chunk's keys through the wave's own LDS slot (one write,
    // eight broadcast reads); the wave-scope fences order the slot's reuse
    if (!(lane & 1)) se[wave][lane >> 1] = e;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float o = 0.0f;
#pragma unroll
    for (int k4 = 0; k4 < kCa64Chunk / 4; ++k4) {
      const float4 e4 = *reinterpret_cast<const float4*>(&se[wave][4 * k4]);
      o += e4.x * vv[4 * k4];
      o += e4.y * vv[4 * k4 + 1];
      o += e4.z * vv[4 * k4 + 2];
      o += e4.w * vv[4 * k4 + 3];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // a chunk whose every score is -inf (fill = -inf) leaves the state as
    // it was (its e are NaN, wave-uniformly)
    if (m != -INFINITY) {
      const float Mn = fmaxf(M, m);
      const float a = expf(M - Mn), c = expf(m - Mn);
      L = L * a + l * c;
      O = O * a + o * c;
      M = Mn;
    }
  }
  if (lane == 0) {
    sm[wave] = M;
    sl[wave] = L;
  }
  so[wave][lane] = O;
  __syncthreads();
  if (wave == 0) {
    float Mx = sm[0];
    for (int w = 1; w < kCa64Waves; ++w) Mx = fmaxf(Mx, sm[w]);
    float Lt = 0.0f, Ot = 0.0f;
    for (int w = 0; w < kCa64Waves; ++w) {
      const float c = expf(sm[w] - Mx);  // a wave without keys: sm = -inf, weight 0
      Lt += c * sl[w];
      Ot += c * so[w][lane];
    }
    p.out[(b * p.S + i) * p.ldo + h * D + lane] = Ot / Lt;
  }
}

// cache[b, h, t0 + s, :] = src[b, s, h*dh : (h+1)*dh] (token-major rows).
__global__ __launch_bounds__(256) void cache_write_tokens_kernel(int64_t B, int64_t S, int64_t nH,
                                                                 int64_t dh, int64_t max_t,
                                                                 int64_t t0,
                                                                 const float* __restrict__ src,
                                                                 int64_t ld,
                                                                 float* __restrict__ cache,
                                                                 const int64_t* pos) {
  if (pos) t0 += *pos;
  const int64_t total = B * S * nH * dh;
  for (int64_t e = int64_t(blockIdx.x) * 256 + threadIdx.x; e < total;
       e += int64_t(gridDim.x) * 256) {
    const int64_t d = e % dh, h = (e / dh) % nH, s = (e / (dh * nH)) % S, b = e / (dh * nH * S);
    cache[((b * nH + h) * max_t + t0 + s) * dh + d] = src[(b * S + s) * ld + h * dh + d];
  }
}

// out[i, :] = table[min(*pos + i, rows - 1), :]
__global__ __launch_bounds__(256) void gather_rows_at_kernel(int64_t rows, int64_t row_len,
                                                             const float* __restrict__ table,
                                                             const int64_t* __restrict__ pos,
                                                             int64_t n, float* __restrict__ out) {
  const int64_t p0 = *pos;
  for (int64_t e = int64_t(blockIdx.x) * 256 + threadIdx.x; e < n * row_len;
       e += int64_t(gridDim.x) * 256) {
    const int64_t i = e / row_len, c = e % row_len;
    int64_t rw = p0 + i;
    rw = rw < 0 ? 0 : rw < rows ? rw : rows - 1;
    out[e] = table[rw * row_len + c];
  }
}

// out[i, :] = a[ids[i], :] + b[min(*pos + i, b_rows - 1), :]: a token
// embedding row (negative ids wrap; an id out of range reads zeros and sets
// *err, as gather_kernel does) plus the position embedding row at the device
// position.
__global__ __launch_bounds__(256) void embed_add_at_kernel(
    const float* __restrict__ a, int64_t a_rows, const int64_t* __restrict__ ids,
    const float* __restrict__ b, int64_t b_rows, const int64_t* __restrict__ pos, int64_t n,
    int64_t row_len, float* __restrict__ out, int32_t* err) {
  const int64_t p0 = *pos;
  for (int64_t e = int64_t(blockIdx.x) * 256 + threadIdx.x; e < n * row_len;
       e += int64_t(gridDim.x) * 256) {
    const int64_t i = e / row_len, c = e % row_len;
    int64_t t = ids[i];
    if (t < 0) t += a_rows;
    const bool ok = t >= 0 && t < a_rows;
    if (!ok && err) *err = 1;
    int64_t rw = p0 + i;
    rw = rw < 0 ? 0 : rw < b_rows ? rw : b_rows - 1;
    out[e] = (ok ? a[t * row_len + c] : 0.0f) + b[rw * row_len + c];
  }
}

__global__ void advance_position_kernel(int64_t* pos, int64_t step) {
  if (threadIdx.x == 0) *pos += step;
}

// Decode feedback: the step's arg-max token becomes the next step's input
// (ids[0]) and is recorded at its position in the history (hist[pos + step]);
// then the position advances.
__global__ void decode_feedback_kernel(int64_t* pos, int64_t step, const int64_t* tok,
                                       int64_t* ids, int64_t* hist) {
  if (threadIdx.x == 0) {
    const int64_t p = *pos + step, t = *tok;
    ids[0] = t;
    hist[p] = t;
    *pos = p;
  }
}

}  // namespace

void gather_rows_at(inferc_hip_ctx* ctx, int64_t rows, int64_t row_len, const float* table,
                    const int64_t* pos, int64_t n, float* out) {
  IH_REQUIRE(rows > 0 && row_len >= 0 && n >= 0, INFERC_ERR_SHAPE, "gather: bad shape");
  if (n == 0 || row_len == 0) return;
  IH_REQUIRE(table && pos && out, INFERC_ERR_ARG, "gather: null pointer");
  const int64_t blocks = ceil_div(n * row_len, 256);
  hipLaunchKernelGGL(gather_rows_at_kernel, dim3(unsigned(blocks > 1024 ? 1024 : blocks)),
                     dim3(256), 0, ctx->stream, rows, row_len, table, pos, n, out);
  check_launch("gather at position");
}

void embed_add_at(inferc_hip_ctx* ctx, const float* a, int64_t a_rows, const int64_t* ids,
                  const float* b, int64_t b_rows, const int64_t* pos, int64_t n, int64_t row_len,
                  float* out, int32_t* err) {
  IH_REQUIRE(a_rows > 0 && b_rows > 0 && row_len >= 0 && n >= 0, INFERC_ERR_SHAPE,
             "embedding add: bad shape");
  if (n == 0 || row_len == 0) return;
  IH_REQUIRE(a && ids && b && pos && out, INFERC_ERR_ARG, "embedding add: null pointer");
  const int64_t blocks = ceil_div(n * row_len, 256);
  hipLaunchKernelGGL(embed_add_at_kernel, dim3(unsigned(blocks > 1024 ? 1024 : blocks)),
                     dim3(256), 0, ctx->stream, a, a_rows, ids, b, b_rows, pos, n, row_len, out,
                     err);
  check_launch("embedding add");
}

void advance_position(inferc_hip_ctx* ctx, int64_t* pos, int64_t step) {
  IH_REQUIRE(pos != nullptr, INFERC_ERR_ARG, "advance: null position");
  hipLaunchKernelGGL(advance_position_kernel, dim3(1), dim3(64), 0, ctx->stream, pos, step);
  check_launch("advance position");
}

// The same after reducing the LM head's per-block (max, first index) partials
// to the greedy token (first maximum wins; with no finite maximum, token 0).
// Each thread loads kFbPer partials, and the position, before it compares any
// of them: one memory round trip per 8192 partials instead of one per partial.
constexpr int kFbThreads = 1024;
constexpr int kFbPer = 8;

__global__ __launch_bounds__(kFbThreads) void decode_feedback_parts_kernel(
    const ValIdxPart* __restrict__ parts, int64_t n, int64_t* pos, int64_t step,
    int64_t* ids, int64_t* hist) {
  __shared__ float sv[kFbThreads / 64];
  __shared__ int64_t si[kFbThreads / 64];
  // read by every thread before thread 0 rewrites it behind the barrier
  const int64_t p0 = *pos;
  float v = -INFINITY;
  int64_t i = INT64_MAX;
  for (int64_t base = 0; base < n; base += int64_t(kFbThreads) * kFbPer) {
    ValIdxPart q[kFbPer];
#pragma unroll
    for (int k = 0; k < kFbPer; ++k) {
      const int64_t e = base + threadIdx.x + int64_t(k) * kFbThreads;
      q[k] = e < n ? parts[e] : ValIdxPart{-INFINITY, INT64_MAX};
    }
#pragma unroll
    for (int k = 0; k < kFbPer; ++k)
      if (q[k].v > v || (q[k].v == v && q[k].i < i)) {
        v = q[k].v;
        i = q[k].i;
      }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float w = __shfl_xor(v, o, 64);
    const int64_t j = __shfl_xor(i, o, 64);
    if (w > v || (w == v && j < i)) {
      v = w;
      i = j;
    }
  }
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = v;
    si[threadIdx.x >> 6] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kFbThreads / 64; ++w)
      if (sv[w] > v || (sv[w] == v && si[w] < i)) {
        v = sv[w];
        i = si[w];
      }
    const int64_t t = i == INT64_MAX ? 0 : i, p = p0 + step;
    ids[0] = t;
    hist[p] = t;
    *pos = p;
  }
}

void decode_feedback_parts(inferc_hip_ctx* ctx, const ValIdxPart* parts, int64_t n, int64_t* pos,
                           int64_t step, int64_t* ids, int64_t* hist) {
  IH_REQUIRE(parts && n > 0 && pos && ids && hist, INFERC_ERR_ARG,
             "decode feedback: bad partials");
  hipLaunchKernelGGL(decode_feedback_parts_kernel, dim3(1), dim3(kFbThreads), 0, ctx->stream,
                     parts, n, pos, step, ids, hist);
  check_launch("decode feedback");
}

void decode_feedback(inferc_hip_ctx* ctx, int64_t* pos, int64_t step, const int64_t* tok,
                     int64_t* ids, int64_t* hist) {
  IH_REQUIRE(pos && tok && ids && hist, INFERC_ERR_ARG, "decode feedback: null pointer");
  hipLaunchKernelGGL(decode_feedback_kernel, dim3(1), dim3(64), 0, ctx->stream, pos, step, tok,
                     ids, hist);
  check_launch("decode feedback");
}

void cache_attention(inferc_hip_ctx* ctx, const CacheAttnArgs& a) {
  IH_REQUIRE(a.dh > 0 && a.dh <= kCaMaxDh, INFERC_ERR_UNSUPPORTED,
             "attention over a cache: head_dim must be in [1, 256]");
  // (with the past length on the device, the caller checks T against max_t)
  IH_REQUIRE(a.S >= 1 && (a.pos != nullptr || (a.T >= a.S && a.T <= a.max_t)), INFERC_ERR_SHAPE,
             "attention over a cache: bad lengths");
  IH_REQUIRE(a.ldq >= a.nH * a.dh && a.ldo >= a.nH * a.dh, INFERC_ERR_SHAPE,
             "attention over a cache: row stride smaller than the hidden size");
  const int64_t rows = a.B * a.nH * a.S;
  if (rows == 0) return;
  const float scale = 1.0f / sqrtf(float(a.dh));
  auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  if (a.dh == 64 && a.ldq % 4 == 0 && al16(a.q) && al16(a.kc) && al16(a.vc) &&
      (a.kn == nullptr || (a.ldn % 4 == 0 && al16(a.kn) && al16(a.vn))) &&
      rows < (int64_t(1) << 31)) {
    hipLaunchKernelGGL(cache_attn_d64_kernel, dim3(unsigned(rows)), dim3(64 * kCa64Waves), 0,
                       ctx->stream, a, scale);
    check_launch("cache attention");
    return;
  }
  CacheAttnArgs g = a;
  if (a.kn) {
    // the general kernel reads every key from the cache: append first
    const int64_t t0 = a.pos ? 0 : a.T - a.S;
    cache_write_tokens(ctx, a.B, a.S, a.nH, a.dh, a.max_t, t0, a.kn, a.ldn,
                       const_cast<float*>(a.kc), a.pos);
    cache_write_tokens(ctx, a.B, a.S, a.nH, a.dh, a.max_t, t0, a.vn, a.ldn,
                       const_cast<float*>(a.vc), a.pos);
    g.kn = g.vn = nullptr;
  }
  hipLaunchKernelGGL(cache_attn_kernel, dim3(unsigned(ceil_div(rows, kCaWaves))),
                     dim3(64 * kCaWaves), 0, ctx->stream, g, scale);
  check_launch("cache attention");
}

void cache_write_tokens(inferc_hip_ctx* ctx, int64_t B, int64_t S, int64_t nH, int64_t dh,
                        int64_t max_t, int64_t t0, const float* src, int64_t ld, float* cache,
                        const int64_t* pos) {
  // (with an offset on the device, the caller checks it against max_t)
  IH_REQUIRE(t0 >= 0 && (pos != nullptr || t0 + S <= max_t), INFERC_ERR_SHAPE,
             "KV cache: append past max_t");
  const int64_t total = B * S * nH * dh;
  if (total == 0) return;
  const int64_t blocks = ceil_div(total, 256);
  hipLaunchKernelGGL(cache_write_tokens_kernel, dim3(unsigned(blocks > 8192 ? 8192 : blocks)),
                     dim3(256), 0, ctx->stream, B, S, nH, dh, max_t, t0, src, ld, cache, pos);
  check_launch("cache write");
}

}  // namespace ih
