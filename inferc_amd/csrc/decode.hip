// GPT-2 greedy decode on one GPU: device-resident weights, a preallocated
// device KV cache, and a decode step that is captured once as a HIP graph and
// replayed per token. The step's kernels read the position and the current
// token from a small device state block that the step itself advances, so the
// host only launches the graph.
//
// Reference: `inferc decode` (src/cli/main.cpp:700-936) running the GPT-2
// with-past graph through rt::Executor. Per layer the graph computes
//   LN -> Gemm(c_attn) -> Split -> Concat(past, new) -> QK^T -> Div(8) ->
//   Where(causal) -> Softmax -> PV -> Gemm(c_proj) -> Add(residual) -> LN ->
//   Gemm(c_fc) -> GeluTanh -> Gemm(c_proj) -> Add(residual)
// then final LN and logits = h * wte^T (folded transpose,
// src/ir/passes/constant_fold.cc:12-54), and the host takes the first argmax
// (main.cpp:875-879). Here each Gemm at M=1 is one HBM-streaming GEMV with the
// preceding LayerNorm fused into its prologue and bias / residual / GELU in
// its epilogue; Concat+attention is one kernel over the device cache.
#include <cstring>
#include <string>
#include <vector>

#include "common.h"
#include "profiler.h"

namespace ih {
namespace {

constexpr int kBlock = 256;

struct KvP {
  int64_t nH, D, T;
  const int64_t* pos;
  const float* q;
  const float* k_new;
  const float* v_new;
  float* kc;  // [nH, T, D]
  float* vc;
  float* out;  // [nH*D]
};

// One block per head. Appends the token's K/V at *pos, then computes
// softmax((q.k_j)/sqrt(D)) over j <= pos and the weighted sum of V rows.
__global__ __launch_bounds__(kBlock) void kv_append_attend_kernel(KvP p) {
  extern __shared__ float sc[];  // [T] scores / probabilities
  __shared__ float qs[256];
  __shared__ float red[kBlock / 64];
  __shared__ float opart[kBlock];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t h = blockIdx.x, D = p.D, T = p.T;
  const int64_t pos = *p.pos;
  if (pos < 0 || pos >= T) return;  // host guarantees the range
  const int64_t t = pos + 1;
  float* kc = p.kc + h * T * D;
  float* vc = p.vc + h * T * D;
  const float* kn = p.k_new + h * D;
  const float* vn = p.v_new + h * D;
  for (int64_t d = tid; d < D; d += kBlock) {
    kc[pos * D + d] = kn[d];
    vc[pos * D + d] = vn[d];
    qs[d] = p.q[h * D + d];
  }
  __syncthreads();
  // Scores: D/4 lanes per key, each lane a float4 slice of the row.
  const int lpk = int(D / 4), kpw = 64 / lpk;
  const float rs = sqrtf(float(D));
  for (int64_t base = int64_t(wave) * kpw; base < t; base += int64_t(kBlock / 64) * kpw) {
    const int64_t j = base + lane / lpk;
    const int dl = (lane % lpk) * 4;
    float dot = 0.0f;
    if (j < t && lane < kpw * lpk) {
      // The new row is read from the input vector, not back from the cache.
      const float* kr = (j == pos) ? kn : kc + j * D;
      const float4 kv = *reinterpret_cast<const float4*>(kr + dl);
      dot = qs[dl] * kv.x + qs[dl + 1] * kv.y + qs[dl + 2] * kv.z + qs[dl + 3] * kv.w;
    }
    for (int o = lpk / 2; o > 0; o >>= 1) dot += __shfl_xor(dot, o, 64);
    if (j < t && (lane % lpk) == 0 && lane < kpw * lpk) sc[j] = dot / rs;
  }
  __syncthreads();
  float m = -INFINITY;
  for (int64_t j = tid; j < t; j += kBlock) m = fmaxf(m, sc[j]);
  m = wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = red[0];
  for (int w = 1; w < kBlock / 64; ++w) m = fmaxf(m, red[w]);
  __syncthreads();
  float s = 0.0f;
  for (int64_t j = tid; j < t; j += kBlock) {
    const float e = expf(sc[j] - m);
    sc[j] = e;
    s += e;
  }
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  s = 0.0f;
  for (int w = 0; w < kBlock / 64; ++w) s += red[w];
  const float inv = 1.0f / s;
  // out[d] = sum_j p_j v[j][d]: thread (d, g) sums keys j = g (mod groups).
  const int groups = int(kBlock / D);
  const int d = tid % int(D), g = tid / int(D);
  float acc = 0.0f;
  if (g < groups) {
    for (int64_t j = g; j < t; j += groups) {
      const float* vr = (j == pos) ? vn : vc + j * D;
      acc += (sc[j] * inv) * vr[d];
    }
  }
  opart[tid] = acc;
  __syncthreads();
  if (tid < D) {
    float o = 0.0f;
    for (int gg = 0; gg < groups; ++gg) o += opart[gg * D + tid];
    p.out[h * D + tid] = o;
  }
}

// Decode attention for head_dim 64, one block (8 waves) per head. The block
// appends the token's K/V at *pos, then wave w walks key chunks w, w+8, ...
// of 32 keys. For a chunk every K and V load is issued before any is used
// (indices past the last key are clamped to it and weighted by 0), so a
// chunk costs one memory round trip. Per chunk: s_j = (q . k_j) / sqrt(64)
// (the with-past graph's MatMul -> Div), m = max s_j, e_j = exp(s_j - m),
// l = sum e_j, O = sum e_j v_j (e_j shared across the wave through LDS);
// chunks are merged online within a wave and the eight waves through LDS in
// wave order; out = O / L.
struct AttnDecP {
  int64_t T;
  const int64_t* pos;
  const float* q;
  const float* k_new;
  const float* v_new;
  float* kc;
  float* vc;
  float* out;
};

constexpr int kDecWaves = 8;

// The operands are scalar arguments (not an AttnDecP by value): the leading
// ones arrive preloaded in SGPRs, so the position and row loads wait on no
// load of the argument block.
__global__ __launch_bounds__(64 * kDecWaves) void attn_decode_d64(
    const int64_t* __restrict__ pos_p, const float* __restrict__ q_all,
    const float* __restrict__ k_new, const float* __restrict__ v_new, float* kc_all,
    float* vc_all, float* out, int64_t T) {
  constexpr int D = 64;
  __shared__ float sm[kDecWaves], sl[kDecWaves];
  __shared__ float so[kDecWaves][D];
  __shared__ __align__(16) float se[kDecWaves][kDecChunk];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t h = blockIdx.x;
  const int64_t pos = *pos_p;
  if (pos < 0 || pos >= T) return;  // uniform: the host keeps pos < T
  const int64_t t = pos + 1;
  float* kc = kc_all + h * T * D;
  float* vc = vc_all + h * T * D;
  const float* kn = k_new + h * D;
  const float* vn = v_new + h * D;
  if (wave == 0) {
    // Rows of position pos are read from kn/vn below, never from the cache,
    // so this append needs no barrier.
    kc[pos * D + lane] = kn[lane];
    vc[pos * D + lane] = vn[lane];
  }
  const int dh = (lane & 1) * 32;
  float4 qv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) qv[i] = *reinterpret_cast<const float4*>(q_all + h * D + dh + 4 * i);
  const float rs = sqrtf(float(D));
  float M = -INFINITY, L = 0.0f, O = 0.0f;
  for (int64_t j0 = int64_t(wave) * kDecChunk; j0 < t; j0 += kDecWaves * kDecChunk) {
    const int64_t jl = j0 + (lane >> 1);
    const int64_t jc = jl < t ? jl : t - 1;
    const float* kr = (jc == pos) ? kn : kc + jc * D;
    float4 kv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) kv[i] = *reinterpret_cast<const float4*>(kr + dh + 4 * i);
    float vv[kDecChunk];
#pragma unroll
    for (int k = 0; k < kDecChunk; ++k) {
      const int64_t jv = (j0 + k < t) ? j0 + k : t - 1;
      vv[k] = ((jv == pos) ? vn : vc + jv * D)[lane];
    }
    float dot = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      dot += qv[i].x * kv[i].x + qv[i].y * kv[i].y + qv[i].z * kv[i].z + qv[i].w * kv[i].w;
    dot += dpp_pair_swap(dot);
    const float s = (jl < t) ? dot / rs : -INFINITY;
    const float m = wave_max_dpp(s);
    const float e = (jl < t) ? expf(s - m) : 0.0f;
    const float l = wave_sum_dpp((lane & 1) ? 0.0f : e);
    // e_k of the chunk's 32 keys through the wave's own LDS slot: one write,
    // then eight broadcast reads (an indexed shuffle per key would be 32
    // dependent LDS trips). The slot is private to the wave, whose LDS
    // operations execute in program order; the wave-scope fences keep the
    // compiler from moving the reads above the write, or the next chunk's
    // write above these reads.
    if (!(lane & 1)) se[wave][lane >> 1] = e;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float o = 0.0f;
#pragma unroll
    for (int k4 = 0; k4 < kDecChunk / 4; ++k4) {
      const float4 e4 = *reinterpret_cast<const float4*>(&se[wave][4 * k4]);
      o += e4.x * vv[4 * k4];
      o += e4.y * vv[4 * k4 + 1];
      o += e4.z * vv[4 * k4 + 2];
      o += e4.w * vv[4 * k4 + 3];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float Mn = fmaxf(M, m);
    const float a = expf(M - Mn), b = expf(m - Mn);
    L = L * a + l * b;
    O = O * a + o * b;
    M = Mn;
  }
  if (lane == 0) {
    sm[wave] = M;
    sl[wave] = L;
  }
  so[wave][lane] = O;
  __syncthreads();
  if (wave == 0) {
    float Mx = sm[0];
    for (int w = 1; w < kDecWaves; ++w) Mx = fmaxf(Mx, sm[w]);
    float Lt = 0.0f, Ot = 0.0f;
    for (int w = 0; w < kDecWaves; ++w) {
      const float c = expf(sm[w] - Mx);
      Lt += c * sl[w];
      Ot += c * so[w][lane];
    }
    out[h * D + lane] = Ot / Lt;
  }
}

void launch_attn_decode(const AttnDecP& p, int64_t heads, hipStream_t s) {
  hipLaunchKernelGGL(attn_decode_d64, dim3(unsigned(heads)), dim3(64 * kDecWaves), 0, s, p.pos,
                     p.q, p.k_new, p.v_new, p.kc, p.vc, p.out, p.T);
}

// The decode step's tail, one block of 1024 threads: merges the LM-head
// blocks' (max logit, first index) partials (the strict '>' rule of
// main.cpp:875-879), records tokens[pos+1], advances state = {pos+1, tok,
// tok}, and writes the next step's input h = wte[tok] + wpe[pos+1]. Each
// thread loads all of its partials, pos and its first wpe value before
// merging them (one memory round trip instead of one per partial; only the
// wte row waits for the merged token).
constexpr int kFinishThreads = 1024;
constexpr int kFinishPerThread = 8;  // up to 8192 partials

__global__ __launch_bounds__(kFinishThreads) void decode_finish_kernel(
    const ValIdxPart* __restrict__ parts, int n, int64_t* __restrict__ state,
    int64_t* __restrict__ tokens, const float* __restrict__ wte, const float* __restrict__ wpe,
    float* __restrict__ h, int64_t H, int64_t max_pos) {
  __shared__ float sv[kFinishThreads / 64];
  __shared__ int64_t si[kFinishThreads / 64];
  __shared__ int64_t s_tok;
  ValIdxPart q[kFinishPerThread];
#pragma unroll
  for (int k = 0; k < kFinishPerThread; ++k) {
    const int e = threadIdx.x + k * kFinishThreads;
    q[k] = e < n ? parts[e] : ValIdxPart{-INFINITY, INT64_MAX};
  }
  // state[0] is read by every thread here, before thread 0 rewrites it
  // behind the first barrier
  const int64_t pos0 = state[0];
  const bool emb = pos0 + 1 < max_pos;
  const float wp0 = emb && threadIdx.x < H ? wpe[(pos0 + 1) * H + threadIdx.x] : 0.0f;
  float v = -INFINITY;
  int64_t i = INT64_MAX;
#pragma unroll
  for (int k = 0; k < kFinishPerThread; ++k)
    if (q[k].v > v || (q[k].v == v && q[k].i < i)) {
      v = q[k].v;
      i = q[k].i;
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
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = v;
    si[wave] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kFinishThreads / 64; ++w)
      if (sv[w] > v || (sv[w] == v && si[w] < i)) {
        v = sv[w];
        i = si[w];
      }
    const int64_t tok = (i == INT64_MAX) ? 0 : i;
    tokens[pos0 + 1] = tok;
    state[2] = tok;
    state[1] = tok;
    state[0] = pos0 + 1;
    s_tok = tok;
  }
  __syncthreads();
  if (emb) {
    const int64_t tok = s_tok, p1 = pos0 + 1;
    if (threadIdx.x < H) h[threadIdx.x] = wte[tok * H + threadIdx.x] + wp0;
    for (int64_t c = threadIdx.x + kFinishThreads; c < H; c += kFinishThreads)
      h[c] = wte[tok * H + c] + wpe[p1 * H + c];
  }
}

// h[c] = wte[tok][c] + wpe[pos][c] with (pos, tok) = (state[0], state[1]).
__global__ __launch_bounds__(kBlock) void embed_step_kernel(const float* __restrict__ wte,
                                                            const float* __restrict__ wpe,
                                                            const int64_t* __restrict__ state,
                                                            int64_t H, float* __restrict__ h) {
  const int64_t pos = state[0], tok = state[1];
  for (int64_t c = int64_t(blockIdx.x) * kBlock + threadIdx.x; c < H;
       c += int64_t(gridDim.x) * kBlock)
    h[c] = wte[tok * H + c] + wpe[pos * H + c];
}

// Prefill embedding: rows i < n, ids validated on the host.
__global__ __launch_bounds__(kBlock) void embed_rows_kernel(const float* __restrict__ wte,
                                                            const float* __restrict__ wpe,
                                                            const int64_t* __restrict__ ids,
                                                            int64_t n, int64_t H,
                                                            float* __restrict__ h) {
  for (int64_t e = int64_t(blockIdx.x) * kBlock + threadIdx.x; e < n * H;
       e += int64_t(gridDim.x) * kBlock) {
    const int64_t i = e / H, c = e % H;
    h[e] = wte[ids[i] * H + c] + wpe[i * H + c];
  }
}

// Scatter the K and V columns of qkv rows [n, 3H] into the caches at
// positions pos0 .. pos0+n-1 ([nH, T, D] per tensor).
__global__ __launch_bounds__(kBlock) void kv_scatter_kernel(const float* __restrict__ qkv,
                                                            int64_t n, int64_t pos0, int64_t nH,
                                                            int64_t D, int64_t T,
                                                            float* __restrict__ kc,
                                                            float* __restrict__ vc) {
  const int64_t H = nH * D;
  for (int64_t e = int64_t(blockIdx.x) * kBlock + threadIdx.x; e < n * H;
       e += int64_t(gridDim.x) * kBlock) {
    const int64_t i = e / H, c = e % H, hh = c / D, d = c % D;
    kc[(hh * T + pos0 + i) * D + d] = qkv[i * 3 * H + H + c];
    vc[(hh * T + pos0 + i) * D + d] = qkv[i * 3 * H + 2 * H + c];
  }
}

// After the argmax of a step whose input sat at state[0]: record the token at
// sequence position state[0]+1 and advance the state.
__global__ void advance_state_kernel(int64_t* __restrict__ state, int64_t* __restrict__ tokens) {
  if (threadIdx.x == 0) {
    const int64_t pos = state[0], tok = state[2];
    tokens[pos + 1] = tok;
    state[1] = tok;
    state[0] = pos + 1;
  }
}

}  // namespace

void kv_append_attend(inferc_hip_ctx* ctx, int64_t nH, int64_t D, int64_t T,
                      const int64_t* pos, const float* q, const float* k_new,
                      const float* v_new, float* kc, float* vc, float* out) {
  IH_REQUIRE(nH > 0 && D > 0 && T > 0, INFERC_ERR_SHAPE, "kv_append_attend: bad shape");
  IH_REQUIRE(D % 4 == 0 && D <= 256 && 64 % (D / 4) == 0, INFERC_ERR_UNSUPPORTED,
             "kv_append_attend: head_dim must be a multiple of 4 dividing 256");
  IH_REQUIRE(T <= 16384, INFERC_ERR_UNSUPPORTED, "kv_append_attend: max_t > 16384");
  IH_REQUIRE(pos && q && k_new && v_new && kc && vc && out, INFERC_ERR_ARG,
             "kv_append_attend: null pointer");
  IH_REQUIRE(aligned16(q) && aligned16(k_new) && aligned16(kc) && aligned16(vc),
             INFERC_ERR_ARG, "kv_append_attend: pointers must be 16-byte aligned");
  if (D == 64) {
    launch_attn_decode(AttnDecP{T, pos, q, k_new, v_new, kc, vc, out}, nH, ctx->stream);
    check_launch("attn_decode");
    return;
  }
  KvP p{nH, D, T, pos, q, k_new, v_new, kc, vc, out};
  hipLaunchKernelGGL(kv_append_attend_kernel, dim3(unsigned(nH)), dim3(kBlock),
                     size_t(T) * sizeof(float), ctx->stream, p);
  check_launch("kv_append_attend");
}

}  // namespace ih

// ---------------------------------------------------------------- GPT-2 model

// Op types of a profiled decode step's launch groups. Each group is one
// fused launch standing for a run of the reference's with-past graph ops:
// LayerNorm -> MatMul -> Add (qkv), the attention over past + new K/V,
// MatMul -> Add -> Add (projection, bias, residual), LayerNorm -> MatMul ->
// Add -> GELU (MLP up), and the final LayerNorm -> LM-head MatMul -> argmax.
namespace {
constexpr const char* kOpEmbed = "Embedding";
constexpr const char* kOpLnQkv = "LayerNorm+QKV";
constexpr const char* kOpAttn = "AttentionDecode";
constexpr const char* kOpProjRes = "MatMul+Bias+Residual";
constexpr const char* kOpLnFcGelu = "LayerNorm+MatMulAddGELU";
constexpr const char* kOpHead = "LayerNorm+LMHead+ArgMax";
}  // namespace

struct inferc_gpt2 {
  inferc_hip_ctx* ctx = nullptr;
  inferc_gpt2_config cfg{};
  int64_t max_t = 0;
  std::vector<void*> allocs;
  float* wte = nullptr;  // [V, H]: tied LM head, already the [N, K] GEMV layout
  float* wpe = nullptr;
  struct Layer {
    float *ln1_g, *ln1_b, *attn_w, *attn_b, *proj_w, *proj_b;
    float *ln2_g, *ln2_b, *fc_w, *fc_b, *fcproj_w, *fcproj_b;  // *_w are [N, K]
    // int4 weight-only mode: packed [N, K/2] nibbles and per-row scales
    uint8_t *attn_q = nullptr, *proj_q = nullptr, *fc_q = nullptr, *fcproj_q = nullptr;
    float *attn_s = nullptr, *proj_s = nullptr, *fc_s = nullptr, *fcproj_s = nullptr;
  };
  std::vector<Layer> layers;
  float *lnf_g = nullptr, *lnf_b = nullptr;
  float *kc = nullptr, *vc = nullptr;  // [L, nH, max_t, D]
  float *h = nullptr, *qkv = nullptr, *att = nullptr, *f = nullptr, *logits = nullptr;
  int64_t* state = nullptr;   // [0] pos of the next input token, [1] that token, [2] argmax
  int64_t* tokens = nullptr;  // [max_t + 1]
  void* argmax_ws = nullptr;  // model-owned, so the captured step never uses ctx->ws
  ih::ValIdxPart* amax = nullptr;  // LM-head block partials of the argmax
  int64_t amax_n = 0;
  // int4 weight-only decode: every projection and the tied LM head are
  // quantised per row; the fp32 copies hold the dequantised values (used by
  // the prefill and the embedding lookup, so the whole model is the
  // quantised one).
  bool int4 = false;
  uint8_t* wte_q = nullptr;
  float* wte_s = nullptr;
  ih::ValIdxPart* amax4 = nullptr;  // one partial per wave of the int4 LM head
  int64_t amax4_n = 0;
  int64_t* ids = nullptr;     // [max_t]
  float *ph = nullptr, *pa = nullptr, *pqkv = nullptr, *patt = nullptr, *pf = nullptr;
  hipGraphExec_t step_exec = nullptr;
  hipGraph_t step_graph = nullptr;
  std::vector<hipEvent_t> events;
  // Profiled steps run eagerly: mark() records an event on the stream before
  // each launch group and remembers the op type and name that group starts.
  bool profiling = false;
  std::vector<hipEvent_t> pev;
  std::vector<std::pair<const char*, std::string>> pops;

  template <class T>
  T* alloc(size_t n) {
    void* p = nullptr;
    IH_HIP(hipMalloc(&p, n * sizeof(T)));
    allocs.push_back(p);
    return static_cast<T*>(p);
  }
  void release() {
    if (step_exec) (void)hipGraphExecDestroy(step_exec);
    if (step_graph) (void)hipGraphDestroy(step_graph);
    for (auto e : events) (void)hipEventDestroy(e);
    for (auto e : pev) (void)hipEventDestroy(e);
    for (void* p : allocs) (void)hipFree(p);
    allocs.clear();
    events.clear();
    pev.clear();
    step_exec = nullptr;
    step_graph = nullptr;
  }

  float* upload(const float* src, size_t n) {
    float* d = alloc<float>(n);
    IH_HIP(hipMemcpy(d, src, n * sizeof(float), hipMemcpyHostToDevice));
    return d;
  }
  // ONNX Gemm weights are [K, N]; the GEMV streams rows of [N, K].
  float* upload_transposed(const float* src, int64_t K, int64_t N) {
    std::vector<float> t(size_t(K) * size_t(N));
    for (int64_t k = 0; k < K; ++k)
      for (int64_t n = 0; n < N; ++n) t[size_t(n) * K + k] = src[size_t(k) * N + n];
    return upload(t.data(), t.size());
  }

  int64_t H() const { return cfg.hidden; }
  int64_t D() const { return cfg.hidden / cfg.heads; }
  float* kc_l(int64_t l) const { return kc + l * cfg.heads * max_t * D(); }
  float* vc_l(int64_t l) const { return vc + l * cfg.heads * max_t * D(); }

  // GPT-2-small dimensions take the short-chain kernels (register-resident
  // x, split-KV attention, argmax fused into the LM head); other shapes use
  // the general GEMV / attention kernels.
  bool fast() const {
    return D() == 64 && H() == 768 && ih::gemv2_supported(cfg.ffn);
  }

  // Records the start of a launch group when profiling; `op` == nullptr
  // records the end of the last group.
  void mark(const char* op, int64_t layer = -1, const char* part = "") {
    if (!profiling) return;
    if (pev.size() < pops.size() + 1) {
      hipEvent_t e;
      IH_HIP(hipEventCreate(&e));
      pev.push_back(e);
    }
    IH_HIP(hipEventRecord(pev[pops.size()], ctx->stream));
    if (op) pops.emplace_back(op, layer >= 0 ? "h." + std::to_string(layer) + part : part);
  }

  // One decode step for the token in state[1] at position state[0]. On the
  // fast path the step's input embedding h was written by the previous
  // step's LM-head tail (or the prefill's), so the step starts with layer 0.
  void enqueue_step() {
    hipStream_t s = ctx->stream;
    const int64_t Hh = H(), F = cfg.ffn;
    if (!fast()) {
      mark(kOpEmbed, -1, "embed");
      hipLaunchKernelGGL(ih::embed_step_kernel, dim3(unsigned(ih::ceil_div(Hh, ih::kBlock))),
                         dim3(ih::kBlock), 0, s, wte, wpe, state, Hh, h);
      ih::check_launch("embed_step");
    }
    if (int4) {
      // the same five launches per layer, weights streamed as int4
      for (int64_t l = 0; l < cfg.layers; ++l) {
        const Layer& L = layers[size_t(l)];
        mark(kOpLnQkv, l, ".attn.qkv");
        ih::int4_gemv_dec(ctx, 3 * Hh, Hh, L.attn_q, L.attn_s, h, L.ln1_g, L.ln1_b, cfg.eps,
                          L.attn_b, nullptr, INFERC_ACT_NONE, qkv, nullptr);
        mark(kOpAttn, l, ".attn");
        ih::launch_attn_decode(
            ih::AttnDecP{max_t, state, qkv, qkv + Hh, qkv + 2 * Hh, kc_l(l), vc_l(l), att},
            cfg.heads, s);
        ih::check_launch("attn_decode");
        mark(kOpProjRes, l, ".attn.proj");
        ih::int4_gemv_dec(ctx, Hh, Hh, L.proj_q, L.proj_s, att, nullptr, nullptr, 0.0f, L.proj_b,
                          h, INFERC_ACT_NONE, h, nullptr);
        mark(kOpLnFcGelu, l, ".mlp.fc");
        ih::int4_gemv_dec(ctx, F, Hh, L.fc_q, L.fc_s, h, L.ln2_g, L.ln2_b, cfg.eps, L.fc_b,
                          nullptr, INFERC_ACT_GELU_TANH, f, nullptr);
        mark(kOpProjRes, l, ".mlp.proj");
        ih::int4_gemv_dec(ctx, Hh, F, L.fcproj_q, L.fcproj_s, f, nullptr, nullptr, 0.0f,
                          L.fcproj_b, h, INFERC_ACT_NONE, h, nullptr);
      }
      lm_head_finish(h);
      return;
    }
    for (int64_t l = 0; l < cfg.layers; ++l) {
      const Layer& L = layers[size_t(l)];
      mark(kOpLnQkv, l, ".attn.qkv");
      ih::gemv(ctx, 3 * Hh, Hh, L.attn_w, h, L.ln1_g, L.ln1_b, cfg.eps, L.attn_b, nullptr,
               INFERC_ACT_NONE, qkv);
      mark(kOpAttn, l, ".attn");
      if (fast()) {
        ih::launch_attn_decode(
            ih::AttnDecP{max_t, state, qkv, qkv + Hh, qkv + 2 * Hh, kc_l(l), vc_l(l), att},
            cfg.heads, s);
        ih::check_launch("attn_decode");
      } else {
        ih::kv_append_attend(ctx, cfg.heads, D(), max_t, state, qkv, qkv + Hh, qkv + 2 * Hh,
                             kc_l(l), vc_l(l), att);
      }
      mark(kOpProjRes, l, ".attn.proj");
      ih::gemv(ctx, Hh, Hh, L.proj_w, att, nullptr, nullptr, 0.0f, L.proj_b, h, INFERC_ACT_NONE,
               h);
      mark(kOpLnFcGelu, l, ".mlp.fc");
      ih::gemv(ctx, F, Hh, L.fc_w, h, L.ln2_g, L.ln2_b, cfg.eps, L.fc_b, nullptr,
               INFERC_ACT_GELU_TANH, f);
      mark(kOpProjRes, l, ".mlp.proj");
      ih::gemv(ctx, Hh, F, L.fcproj_w, f, nullptr, nullptr, 0.0f, L.fcproj_b, h, INFERC_ACT_NONE,
               h);
    }
    lm_head_finish(h);
  }

  // Final LN + LM head on one hidden row, then the greedy token:
  // tokens[state[0]+1] = argmax (first max), state advanced by one position.
  void lm_head_finish(const float* hrow) {
    const int64_t Hh = H(), V = cfg.vocab;
    mark(kOpHead, -1, "lm_head");
    if (int4) {
      ih::int4_gemv_dec(ctx, V, Hh, wte_q, wte_s, hrow, lnf_g, lnf_b, cfg.eps, nullptr, nullptr,
                        INFERC_ACT_NONE, logits, amax4);
      hipLaunchKernelGGL(ih::decode_finish_kernel, dim3(1), dim3(ih::kFinishThreads), 0,
                         ctx->stream, amax4, int(amax4_n), state, tokens, wte, wpe, h, Hh,
                         cfg.max_pos);
      ih::check_launch("decode_finish");
      return;
    }
    if (fast()) {
      ih::Gemv2Args a;
      a.N = V; a.K = Hh; a.W = wte; a.x = hrow; a.ln_g = lnf_g; a.ln_b = lnf_b;
      a.ln_eps = cfg.eps; a.y = logits; a.amax = amax;
      ih::gemv2(ctx, a);
      hipLaunchKernelGGL(ih::decode_finish_kernel, dim3(1), dim3(ih::kFinishThreads), 0,
                         ctx->stream, amax, int(amax_n), state, tokens, wte, wpe, h, Hh,
                         cfg.max_pos);
      ih::check_launch("decode_finish");
      return;
    }
    ih::gemv(ctx, V, Hh, wte, hrow, lnf_g, lnf_b, cfg.eps, nullptr, nullptr, INFERC_ACT_NONE,
             logits);
    ih::argmax(ctx, V, logits, state + 2, argmax_ws);
    hipLaunchKernelGGL(ih::advance_state_kernel, dim3(1), dim3(64), 0, ctx->stream, state,
                       tokens);
    ih::check_launch("advance_state");
  }

  // Prefill over n prompt tokens (ids already on the device): fills the
  // cache at positions [0, n) and leaves the final-LN-free hidden rows in ph.
  void enqueue_prefill_blocks(int64_t n) {
    hipStream_t s = ctx->stream;
    const int64_t Hh = H(), F = cfg.ffn;
    {
      int64_t blocks = ih::ceil_div(n * Hh, ih::kBlock);
      hipLaunchKernelGGL(ih::embed_rows_kernel, dim3(unsigned(blocks < 8192 ? blocks : 8192)),
                         dim3(ih::kBlock), 0, s, wte, wpe, ids, n, Hh, ph);
      ih::check_launch("embed_rows");
    }
    for (int64_t l = 0; l < cfg.layers; ++l) {
      const Layer& L = layers[size_t(l)];
      ih::layernorm(ctx, n, Hh, ph, nullptr, L.ln1_g, L.ln1_b, cfg.eps, pa);
      ih::GemmArgs g;
      g.trans_b = 1; g.M = n; g.N = 3 * Hh; g.K = Hh;
      g.A = pa; g.lda = Hh; g.B = L.attn_w; g.ldb = Hh;
      g.beta = 1.0f; g.C = L.attn_b; g.c_kind = INFERC_C_ROW;
      g.Y = pqkv; g.ldy = 3 * Hh;
      ih::gemm(ctx, g);
      int64_t blocks = ih::ceil_div(n * Hh, ih::kBlock);
      hipLaunchKernelGGL(ih::kv_scatter_kernel, dim3(unsigned(blocks < 8192 ? blocks : 8192)),
                         dim3(ih::kBlock), 0, s, pqkv, n, int64_t(0), cfg.heads, D(), max_t,
                         kc_l(l), vc_l(l));
      ih::check_launch("kv_scatter");
      ih::AttnArgs a;
      a.B = 1; a.S = n; a.H = Hh; a.head_dim = D();
      a.q = pqkv; a.k = pqkv + Hh; a.v = pqkv + 2 * Hh;
      a.ldq = a.ldk = a.ldv = 3 * Hh; a.ldo = Hh;
      a.causal = 1;
      a.fill = -3.4028234663852886e38f;  // torch.finfo(float32).min of the export
      a.out = patt;
      ih::attention(ctx, a);
      ih::GemmArgs g2;
      g2.trans_b = 1; g2.M = n; g2.N = Hh; g2.K = Hh;
      g2.A = patt; g2.lda = Hh; g2.B = L.proj_w; g2.ldb = Hh;
      g2.beta = 1.0f; g2.C = L.proj_b; g2.c_kind = INFERC_C_ROW;
      g2.R = ph; g2.ldr = Hh; g2.Y = ph; g2.ldy = Hh;
      ih::gemm(ctx, g2);
      ih::layernorm(ctx, n, Hh, ph, nullptr, L.ln2_g, L.ln2_b, cfg.eps, pa);
      ih::GemmArgs g3;
      g3.trans_b = 1; g3.M = n; g3.N = F; g3.K = Hh;
      g3.A = pa; g3.lda = Hh; g3.B = L.fc_w; g3.ldb = Hh;
      g3.beta = 1.0f; g3.C = L.fc_b; g3.c_kind = INFERC_C_ROW;
      g3.act = INFERC_ACT_GELU_TANH; g3.Y = pf; g3.ldy = F;
      ih::gemm(ctx, g3);
      ih::GemmArgs g4;
      g4.trans_b = 1; g4.M = n; g4.N = Hh; g4.K = F;
      g4.A = pf; g4.lda = F; g4.B = L.fcproj_w; g4.ldb = F;
      g4.beta = 1.0f; g4.C = L.fcproj_b; g4.c_kind = INFERC_C_ROW;
      g4.R = ph; g4.ldr = Hh; g4.Y = ph; g4.ldy = Hh;
      ih::gemm(ctx, g4);
    }
  }

  // Quantises the [N, K] matrix at dev (host round trip: read, quantise per
  // row, write back the dequantised values) into packed nibbles and scales.
  void quantize_matrix(float* dev, int64_t N, int64_t K, uint8_t** q, float** sc) {
    const size_t nk = static_cast<size_t>(N * K);
    std::vector<float> w(nk), deq(nk), s(static_cast<size_t>(N));
    std::vector<uint8_t> packed(nk / 2);
    IH_HIP(hipMemcpy(w.data(), dev, w.size() * sizeof(float), hipMemcpyDeviceToHost));
    ih::int4_quantize_rows(N, K, w.data(), packed.data(), s.data(), deq.data());
    *q = alloc<uint8_t>(packed.size());
    *sc = alloc<float>(s.size());
    IH_HIP(hipMemcpy(*q, packed.data(), packed.size(), hipMemcpyHostToDevice));
    IH_HIP(hipMemcpy(*sc, s.data(), s.size() * sizeof(float), hipMemcpyHostToDevice));
    IH_HIP(hipMemcpy(dev, deq.data(), deq.size() * sizeof(float), hipMemcpyHostToDevice));
  }

  void enable_int4() {
    if (int4) return;
    const int64_t Hh = H(), F = cfg.ffn, V = cfg.vocab;
    IH_REQUIRE(fast() && Hh == 768 && F == 3072, INFERC_ERR_UNSUPPORTED,
               "int4 decode: needs the GPT-2-small row lengths (hidden 768, ffn 3072)");
    IH_HIP(hipStreamSynchronize(ctx->stream));
    for (Layer& L : layers) {
      quantize_matrix(L.attn_w, 3 * Hh, Hh, &L.attn_q, &L.attn_s);
      quantize_matrix(L.proj_w, Hh, Hh, &L.proj_q, &L.proj_s);
      quantize_matrix(L.fc_w, F, Hh, &L.fc_q, &L.fc_s);
      quantize_matrix(L.fcproj_w, Hh, F, &L.fcproj_q, &L.fcproj_s);
    }
    quantize_matrix(wte, V, Hh, &wte_q, &wte_s);
    amax4_n = ih::int4_dec_waves(V, Hh);
    IH_REQUIRE(amax4_n <= ih::kFinishThreads * ih::kFinishPerThread, INFERC_ERR_UNSUPPORTED,
               "int4 decode: vocabulary too large for the argmax tail");
    amax4 = alloc<ih::ValIdxPart>(size_t(amax4_n));
    // the captured step used the fp32 kernels: capture it again
    if (step_exec) (void)hipGraphExecDestroy(step_exec);
    if (step_graph) (void)hipGraphDestroy(step_graph);
    step_exec = nullptr;
    step_graph = nullptr;
    int4 = true;
  }

  void capture_step() {
    if (step_exec) return;
    IH_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
    try {
      enqueue_step();
    } catch (...) {
      ctx->capturing = false;
      hipGraph_t g = nullptr;
      (void)hipStreamEndCapture(ctx->stream, &g);
      if (g) (void)hipGraphDestroy(g);
      throw;
    }
    ctx->capturing = false;
    IH_HIP(hipStreamEndCapture(ctx->stream, &step_graph));
    IH_HIP(hipGraphInstantiate(&step_exec, step_graph, nullptr, nullptr, 0));
  }
};

namespace {

void check_model(inferc_gpt2* m) {
  IH_REQUIRE(m != nullptr && m->ctx != nullptr, INFERC_ERR_ARG, "null GPT-2 model");
  m->ctx->make_current();
}

void upload_ids(inferc_gpt2* m, const int64_t* ids, int64_t n) {
  IH_REQUIRE(ids != nullptr, INFERC_ERR_ARG, "null token ids");
  for (int64_t i = 0; i < n; ++i)
    IH_REQUIRE(ids[i] >= 0 && ids[i] < m->cfg.vocab, INFERC_ERR_ARG,
               "token id " + std::to_string(ids[i]) + " out of range");
  IH_HIP(hipMemcpyAsync(m->ids, ids, size_t(n) * sizeof(int64_t), hipMemcpyHostToDevice,
                        m->ctx->stream));
}

// Checks the request, then enqueues the prefill and the first greedy token:
// state = {pos = n_prompt - 1} lets the prefill's last row play the role of
// a step input, so the LM-head tail records the first generated token at
// position n_prompt and leaves the state at the first decode step
// (main.cpp:820-828).
void start_generation(inferc_gpt2* m, const int64_t* prompt, int64_t n_prompt,
                      int64_t max_tokens, const int64_t* tokens_out) {
  check_model(m);
  IH_REQUIRE(n_prompt > 0, INFERC_ERR_ARG, "inferc decode: empty prompt");
  IH_REQUIRE(max_tokens > 0, INFERC_ERR_ARG, "inferc decode: max_tokens must be > 0");
  IH_REQUIRE(tokens_out != nullptr, INFERC_ERR_ARG, "null tokens_out");
  IH_REQUIRE(n_prompt + max_tokens - 1 <= m->max_t, INFERC_ERR_SHAPE,
             "prompt + generated tokens exceed the KV cache (max_t)");
  const int64_t init[4] = {n_prompt - 1, 0, 0, 0};
  IH_HIP(hipMemcpyAsync(m->state, init, sizeof(init), hipMemcpyHostToDevice, m->ctx->stream));
  upload_ids(m, prompt, n_prompt);
  m->enqueue_prefill_blocks(n_prompt);
  m->lm_head_finish(m->ph + (n_prompt - 1) * m->H());
}

}  // namespace

extern "C" {

int inferc_hip_kv_append_attend_f32(inferc_hip_ctx* ctx, int64_t n_heads, int64_t head_dim,
                                    int64_t max_t, const int64_t* pos, const float* q,
                                    const float* k_new, const float* v_new, float* k_cache,
                                    float* v_cache, float* out) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    ih::kv_append_attend(ctx, n_heads, head_dim, max_t, pos, q, k_new, v_new, k_cache, v_cache,
                         out);
  });
}

int inferc_gpt2_create(inferc_hip_ctx* ctx, const inferc_gpt2_config* cfg,
                       const float* const* w, int64_t max_t, inferc_gpt2** out) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    IH_REQUIRE(cfg && w && out, INFERC_ERR_ARG, "gpt2_create: null argument");
    *out = nullptr;
    IH_REQUIRE(cfg->layers > 0 && cfg->hidden > 0 && cfg->heads > 0 && cfg->ffn > 0 &&
                   cfg->vocab > 0 && cfg->max_pos > 0,
               INFERC_ERR_SHAPE, "gpt2_create: bad config");
    IH_REQUIRE(cfg->hidden % cfg->heads == 0, INFERC_ERR_SHAPE,
               "gpt2_create: hidden not divisible by heads");
    IH_REQUIRE(max_t > 0 && max_t <= cfg->max_pos, INFERC_ERR_SHAPE,
               "gpt2_create: max_t must be in [1, max_pos]");
    const int64_t H = cfg->hidden, F = cfg->ffn, V = cfg->vocab, L = cfg->layers;
    for (int64_t i = 0; i < 2 + 12 * L + 2; ++i)
      IH_REQUIRE(w[i] != nullptr, INFERC_ERR_ARG, "gpt2_create: null weight pointer");
    auto* m = new inferc_gpt2();
    m->ctx = ctx;
    m->cfg = *cfg;
    m->max_t = max_t;
    try {
      m->wte = m->upload(w[0], size_t(V * H));
      m->wpe = m->upload(w[1], size_t(cfg->max_pos * H));
      for (int64_t l = 0; l < L; ++l) {
        const float* const* lw = w + 2 + 12 * l;
        inferc_gpt2::Layer Ly{};
        Ly.ln1_g = m->upload(lw[0], size_t(H));
        Ly.ln1_b = m->upload(lw[1], size_t(H));
        Ly.attn_w = m->upload_transposed(lw[2], H, 3 * H);
        Ly.attn_b = m->upload(lw[3], size_t(3 * H));
        Ly.proj_w = m->upload_transposed(lw[4], H, H);
        Ly.proj_b = m->upload(lw[5], size_t(H));
        Ly.ln2_g = m->upload(lw[6], size_t(H));
        Ly.ln2_b = m->upload(lw[7], size_t(H));
        Ly.fc_w = m->upload_transposed(lw[8], H, F);
        Ly.fc_b = m->upload(lw[9], size_t(F));
        Ly.fcproj_w = m->upload_transposed(lw[10], F, H);
        Ly.fcproj_b = m->upload(lw[11], size_t(H));
        m->layers.push_back(Ly);
      }
      m->lnf_g = m->upload(w[2 + 12 * L], size_t(H));
      m->lnf_b = m->upload(w[2 + 12 * L + 1], size_t(H));
      const size_t cache = size_t(L * cfg->heads * max_t * (H / cfg->heads));
      m->kc = m->alloc<float>(cache);
      m->vc = m->alloc<float>(cache);
      m->h = m->alloc<float>(size_t(H));
      m->qkv = m->alloc<float>(size_t(3 * H));
      m->att = m->alloc<float>(size_t(H));
      m->f = m->alloc<float>(size_t(F));
      m->logits = m->alloc<float>(size_t(V));
      m->state = m->alloc<int64_t>(4);
      m->tokens = m->alloc<int64_t>(size_t(max_t + 1));
      m->argmax_ws = m->alloc<uint8_t>(ih::kArgmaxScratchBytes);
      m->amax_n = ih::gemv2_blocks(ctx, V, H, true);
      m->amax = m->alloc<ih::ValIdxPart>(size_t(m->amax_n));
      IH_REQUIRE(m->amax_n <= ih::kFinishThreads * ih::kFinishPerThread, INFERC_ERR_UNSUPPORTED,
                 "gpt2_create: vocabulary too large for the argmax tail");
      m->ids = m->alloc<int64_t>(size_t(max_t));
      m->ph = m->alloc<float>(size_t(max_t * H));
      m->pa = m->alloc<float>(size_t(max_t * H));
      m->pqkv = m->alloc<float>(size_t(max_t * 3 * H));
      m->patt = m->alloc<float>(size_t(max_t * H));
      m->pf = m->alloc<float>(size_t(max_t * F));
      IH_HIP(hipMemset(m->kc, 0, cache * sizeof(float)));
      IH_HIP(hipMemset(m->vc, 0, cache * sizeof(float)));
      IH_HIP(hipDeviceSynchronize());
    } catch (...) {
      m->release();
      delete m;
      throw;
    }
    *out = m;
  });
}

int inferc_gpt2_use_int4(inferc_gpt2* m) {
  return ih::guard([&] {
    check_model(m);
    m->enable_int4();
  });
}

int inferc_gpt2_destroy(inferc_gpt2* m) {
  return ih::guard([&] {
    if (!m) return;
    if (m->ctx) {
      m->ctx->make_current();
      (void)hipStreamSynchronize(m->ctx->stream);
    }
    m->release();
    delete m;
  });
}

int inferc_gpt2_generate(inferc_gpt2* m, const int64_t* prompt, int64_t n_prompt,
                         int64_t max_tokens, int64_t* tokens_out, float* step_ms,
                         float* last_logits) {
  return ih::guard([&] {
    start_generation(m, prompt, n_prompt, max_tokens, tokens_out);
    inferc_hip_ctx* ctx = m->ctx;
    hipStream_t s = ctx->stream;
    const int64_t V = m->cfg.vocab;
    m->capture_step();
    const int64_t steps = max_tokens - 1;
    if (step_ms && steps > 0) {
      while (int64_t(m->events.size()) < steps + 1) {
        hipEvent_t e;
        IH_HIP(hipEventCreate(&e));
        m->events.push_back(e);
      }
      IH_HIP(hipEventRecord(m->events[0], s));
    }
    for (int64_t i = 0; i < steps; ++i) {
      IH_HIP(hipGraphLaunch(m->step_exec, s));
      if (step_ms) IH_HIP(hipEventRecord(m->events[size_t(i + 1)], s));
    }
    IH_HIP(hipStreamSynchronize(s));
    IH_HIP(hipMemcpy(tokens_out, m->tokens + n_prompt, size_t(max_tokens) * sizeof(int64_t),
                     hipMemcpyDeviceToHost));
    if (step_ms)
      for (int64_t i = 0; i < steps; ++i)
        IH_HIP(hipEventElapsedTime(&step_ms[i], m->events[size_t(i)], m->events[size_t(i + 1)]));
    if (last_logits)
      IH_HIP(hipMemcpy(last_logits, m->logits, size_t(V) * sizeof(float),
                       hipMemcpyDeviceToHost));
  });
}

// generate() with each decode step recorded as one profiler iteration
// (main.cpp:849-872): the step is enqueued eagerly rather than replayed from
// its graph, an event opens each launch group, and an op's time is the device
// time to the next event. The iteration total is the host wall clock of the
// step from enqueue until the stream has drained. Activation bytes are not
// tracked (main.cpp:850).
int inferc_gpt2_generate_profiled(inferc_gpt2* m, const int64_t* prompt, int64_t n_prompt,
                                  int64_t max_tokens, int64_t* tokens_out,
                                  inferc_profiler* p) {
  return ih::guard([&] {
    IH_REQUIRE(p != nullptr, INFERC_ERR_ARG, "null profiler");
    start_generation(m, prompt, n_prompt, max_tokens, tokens_out);
    hipStream_t s = m->ctx->stream;
    struct Off {
      inferc_gpt2* m;
      ~Off() { m->profiling = false; }
    } off{m};
    for (int64_t i = 0; i + 1 < max_tokens; ++i) {
      IH_HIP(hipStreamSynchronize(s));
      m->pops.clear();
      m->profiling = true;
      p->begin_iteration();
      m->enqueue_step();
      m->mark(nullptr);
      m->profiling = false;
      const size_t n_ops = m->pops.size();
      IH_HIP(hipEventSynchronize(m->pev[n_ops]));
      std::vector<float> ms(n_ops, 0.0f);
      for (size_t k = 0; k < n_ops; ++k)
        IH_HIP(hipEventElapsedTime(&ms[k], m->pev[k], m->pev[k + 1]));
      const double total = std::chrono::duration<double, std::milli>(
                               inferc_profiler::clock::now() - p->iter_t0).count();
      for (size_t k = 0; k < n_ops; ++k)
        p->add_op(m->pops[k].first, m->pops[k].second, double(ms[k]), 0);
      p->end_iteration(total);
    }
    IH_HIP(hipStreamSynchronize(s));
    IH_HIP(hipMemcpy(tokens_out, m->tokens + n_prompt, size_t(max_tokens) * sizeof(int64_t),
                     hipMemcpyDeviceToHost));
  });
}

int inferc_gpt2_forward(inferc_gpt2* m, const int64_t* ids, int64_t n, float* logits) {
  return ih::guard([&] {
    check_model(m);
    IH_REQUIRE(n > 0 && n <= m->max_t, INFERC_ERR_SHAPE, "gpt2_forward: n out of range");
    IH_REQUIRE(logits != nullptr, INFERC_ERR_ARG, "null logits");
    inferc_hip_ctx* ctx = m->ctx;
    const int64_t H = m->H(), V = m->cfg.vocab;
    upload_ids(m, ids, n);
    m->enqueue_prefill_blocks(n);
    ih::layernorm(ctx, n, H, m->ph, nullptr, m->lnf_g, m->lnf_b, m->cfg.eps, m->pa);
    float* dl = nullptr;
    IH_HIP(hipMalloc(&dl, size_t(n * V) * sizeof(float)));
    try {
      ih::GemmArgs g;
      g.trans_b = 1; g.M = n; g.N = V; g.K = H;
      g.A = m->pa; g.lda = H; g.B = m->wte; g.ldb = H;
      g.Y = dl; g.ldy = V;
      ih::gemm(ctx, g);
      IH_HIP(hipStreamSynchronize(ctx->stream));
      IH_HIP(hipMemcpy(logits, dl, size_t(n * V) * sizeof(float), hipMemcpyDeviceToHost));
    } catch (...) {
      (void)hipStreamSynchronize(ctx->stream);
      (void)hipFree(dl);
      throw;
    }
    IH_HIP(hipFree(dl));
  });
}

}  // extern "C"
