// Fused multi-head attention (prefill / encoder) on CDNA4 matrix cores.
//
// Reference: rt::FusedAttention, src/kernels/attention.cc:32-100. Per
// (batch, head): scores = (1/sqrt(d)) * Q_h K_h^T, masked entries set to
// `fill`, softmax with max subtraction, context = P V_h, written in place into
// the [B,S,H] output at column offset h*d.
//
// Design (head_dim 64): a wave owns 32 queries and walks the keys in tiles of
// 32 that the block stages through LDS (double-buffered). Scores are computed
// transposed, S^T = K Q^T, with v_mfma_f32_32x32x2_f32: in that layout every
// lane holds 16 scores of ONE query (column lane%32), so
//   - the online-softmax max/sum need one cross-half shuffle per tile,
//   - the rescale of the running output is a per-lane scalar, and
//   - the probabilities are already in the B-operand layout of the next MFMA,
//     O^T += V^T P^T, once the key index of the V operand is permuted to match
//     (the summation index of an MFMA is a dummy index).
// Softmax is online (running max and sum, output rescaled per tile); the
// reference's two-pass softmax is reproduced to fp32 rounding. Key tiles past
// the last unmasked key of a query-independent mask, and tiles above the
// causal diagonal, are skipped; that is exact because exp(fill - max) is 0 in
// fp32 once one unmasked key has been seen.
#include "common.h"

namespace ih {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kD = 64;     // head_dim of the MFMA kernel
constexpr int kKT = 32;    // keys per tile
constexpr int kKS = kD + 4;  // LDS row stride of K (float4 rows; 16 rows span all banks)
constexpr int kVS = kD + 4;  // LDS row stride of V (float4-aligned rows)

struct AttnP {
  int64_t B, S, nH;
  const float* q;
  const float* k;
  const float* v;
  int64_t ldq, ldk, ldv, ldo;
  const uint8_t* mask;
  int64_t ms0, ms1, ms2, ms3;
  float fill, scale;
  int causal;
  float* out;
};

// Orders a wave's LDS writes before its later LDS reads by other lanes of
// the same wave (no cross-wave synchronisation).
__device__ __forceinline__ void wave_lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The head dim that S^T = K Q^T pairs with MFMA step s (of kD/2) in lane half
// `half`: 8*(s/4) + 4*half + s%4. Any pairing gives the same dot product up to
// summation order (the MFMA summation index is a dummy index); this one gives
// each lane its 32 Q values as 8 runs of 4 consecutive dims, one float4 each.
__device__ __forceinline__ int qk_dim(int s, int half) { return 8 * (s >> 2) + 4 * half + (s & 3); }

constexpr int kQS = kD + 4;  // LDS row stride of the Q and O staging (float4 rows)

// A wave's 32 query rows q0.. read whole: each load covers 4 rows of 256 bytes
// (rows past S are clamped; their outputs are not written). Loading the
// operand layout directly costs a load per 16 bytes of 32 rows instead.
__device__ __forceinline__ void q_rows_load(const float* qbase, int64_t ldq, int64_t q0,
                                            int64_t S, int lane, floatx4 (&qr)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int idx = lane + 64 * i;
    const int64_t row = q0 + idx / 16;
    const int64_t rc = row < S ? row : S - 1;
    qr[i] = *reinterpret_cast<const floatx4*>(qbase + rc * ldq + (idx % 16) * 4);
  }
}

// The rows of q_rows_load through the wave's LDS slice qs (32 rows of kQS)
// into the B operand of S^T = K Q^T: qf[s] = Q[query l32][qk_dim(s, half)].
__device__ __forceinline__ void q_rows_to_operand(float* qs, const floatx4 (&qr)[8], int lane,
                                                  float (&qf)[kD / 2]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int idx = lane + 64 * i;
    *reinterpret_cast<floatx4*>(qs + (idx / 16) * kQS + (idx % 16) * 4) = qr[i];
  }
  wave_lds_barrier();
  const int half = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const floatx4 t = *reinterpret_cast<const floatx4*>(qs + l32 * kQS + 8 * j + 4 * half);
    qf[4 * j] = t[0]; qf[4 * j + 1] = t[1]; qf[4 * j + 2] = t[2]; qf[4 * j + 3] = t[3];
  }
}

// One 32-key tile for a wave's 32 queries: S^T = K Q^T on the matrix cores,
// scale, mask, online-softmax update, then O^T += V^T P^T. BITS: the mask
// comes as mbits (bit v: score register v's key is masked, loaded ahead by
// the caller; KEYBITS: bit o: key k0 + o is masked); otherwise it is read
// here from mbase.
template <bool BITS = false, bool KEYBITS = false>
__device__ __forceinline__ void attn_tile(const AttnP& p, const float* __restrict__ ks,
                                          const float* __restrict__ vs, int64_t k0, int64_t qi,
                                          const uint8_t* mbase, const float (&qf)[kD / 2],
                                          floatx16 (&oacc)[2], float& m_run, float& l_run,
                                          int half, int l32, uint32_t mbits = 0) {
  const int64_t S = p.S;
  floatx16 sacc;
#pragma unroll
  for (int v = 0; v < 16; ++v) sacc[v] = 0.0f;
  // steps 4j..4j+3 take dims qk_dim(4j + e, half) = 8j + 4 half + e: one
  // float4 of the lane's key row per four steps
#pragma unroll
  for (int j = 0; j < kD / 8; ++j) {
    const floatx4 a = *reinterpret_cast<const floatx4*>(ks + l32 * kKS + 8 * j + 4 * half);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], qf[4 * j + e], sacc, 0, 0, 0);
  }
  // sacc[v]: key k0 + 8*(v/4) + 4*half + v%4, query qi.
  float sv[16];
  float tmax = -INFINITY;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int64_t j = k0 + 8 * (v >> 2) + 4 * half + (v & 3);
    float s = p.scale * sacc[v];
    if (j >= S) {
      s = -INFINITY;  // key does not exist
    } else if (p.causal) {
      if (j > qi) s = p.fill;
    } else if (BITS) {
      const int bit = KEYBITS ? 8 * (v >> 2) + 4 * half + (v & 3) : v;
      if ((mbits >> bit) & 1u) s = p.fill;
    } else if (mbase && qi < S) {
      if (mbase[qi * p.ms2 + j * p.ms3]) s = p.fill;
    }
    sv[v] = s;
    tmax = fmaxf(tmax, s);
  }
  tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
  const float m_new = fmaxf(m_run, tmax);
  // A fill of -inf can leave a tile with no finite score; keep the state.
  const bool none = m_new == -INFINITY;
  const float corr = none ? 1.0f : __expf(m_run - m_new);
  float lsum = 0.0f;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    sv[v] = none ? 0.0f : __expf(sv[v] - m_new);
    lsum += sv[v];
  }
  lsum += __shfl_xor(lsum, 32, 64);
  l_run = l_run * corr + lsum;
  m_run = m_new;
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int v = 0; v < 16; ++v) oacc[d][v] *= corr;
  // O^T[dim][query] += V^T[dim][key] P^T[key][query]; step s pairs key
  // 8*(s/4) + 4*kidx + s%4 with the MFMA summation index kidx.
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    const int key = 8 * (s >> 2) + 4 * half + (s & 3);
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const float a = vs[key * kVS + d * 32 + l32];
      oacc[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, sv[s], oacc[d], 0, 0, 0);
    }
  }
}

// Writes query qi's 64 outputs: oacc[d][v] holds dim d*32 + 8*(v/4) +
// 4*half + v%4, scaled by inv = 1/l.
__device__ __forceinline__ void attn_store(const AttnP& p, int64_t b, int64_t h, int64_t qi,
                                           const floatx16 (&oacc)[2], float inv, int half) {
  float* orow = p.out + (b * p.S + qi) * p.ldo + h * kD;
  const bool vec = (p.ldo % 4 == 0) && ((reinterpret_cast<uintptr_t>(p.out) & 15) == 0);
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float* dst = orow + d * 32 + 8 * g + 4 * half;
      const float4 o = make_float4(oacc[d][4 * g] * inv, oacc[d][4 * g + 1] * inv,
                                   oacc[d][4 * g + 2] * inv, oacc[d][4 * g + 3] * inv);
      if (vec) {
        *reinterpret_cast<float4*>(dst) = o;
      } else {
        dst[0] = o.x; dst[1] = o.y; dst[2] = o.z; dst[3] = o.w;
      }
    }
}

// attn_store for 16-byte aligned rows: the wave's 32 output rows q0.. go
// through its LDS slice os (32 rows of kQS) and out whole, 4 rows of 256
// bytes per store. (Stored straight from the accumulator layout, each store
// would write 32 bytes into each of 32 rows.)
__device__ __forceinline__ void o_rows_store(const AttnP& p, int64_t b, int64_t h, int64_t q0,
                                             float* os, const floatx16 (&oacc)[2], float inv,
                                             int lane) {
  const int half = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      floatx4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = oacc[d][4 * g + e] * inv;
      *reinterpret_cast<floatx4*>(os + l32 * kQS + d * 32 + 8 * g + 4 * half) = o;
    }
  wave_lds_barrier();
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int idx = lane + 64 * i;
    const int64_t row = q0 + idx / 16;
    const floatx4 o = *reinterpret_cast<const floatx4*>(os + (idx / 16) * kQS + (idx % 16) * 4);
    if (row < p.S)
      *reinterpret_cast<floatx4*>(p.out + (b * p.S + row) * p.ldo + h * kD + (idx % 16) * 4) = o;
  }
}

// Large grids: WAVES waves of 32 queries share each K/V tile, staged through
// LDS (double-buffered). The loads of tile t+1, the lane's mask bytes
// included, are issued before tile t's matrix-core work and are unconditional
// (keys clamped into the sequence; a clamped key's score is -inf and its V
// row weighs 0), so the waits before the LDS writes count them exactly.
// VEC: 16-byte aligned rows (float4 loads). MASKED: a mask that is neither
// absent nor replaced by the causal rule. MROW: a masked row that is the same
// for every query (ms2 == 0): a tile's 32 mask bytes are one load per lane
// (key k0 + lane % 32), shared by a ballot, instead of 16 per lane.
template <int WAVES, bool VEC, bool MASKED, bool MROW = false>
__global__ __launch_bounds__(64 * WAVES, 12 / WAVES) void attn_fwd_d64(AttnP p) {
  static_assert(MASKED || !MROW, "MROW is a kind of mask");
  constexpr int NT = 64 * WAVES;
  // K and V tiles (double-buffered). With VEC the same LDS also holds each
  // wave's Q rows before the first tile and its output rows after the last.
  constexpr int kKVF = 2 * kKT * kKS + 2 * kKT * kVS, kQF = WAVES * 32 * kQS;
  __shared__ __attribute__((aligned(16))) float lds[kKVF > kQF ? kKVF : kQF];
  float(*Ks)[kKT * kKS] = reinterpret_cast<float(*)[kKT * kKS]>(lds);
  float(*Vs)[kKT * kVS] = reinterpret_cast<float(*)[kKT * kVS]>(lds + 2 * kKT * kKS);
  __shared__ int s_last_valid;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, l32 = lane & 31;
  const int64_t b = blockIdx.z, h = blockIdx.y;
  const int64_t qb0 = int64_t(blockIdx.x) * (32 * WAVES);
  const int64_t q0 = qb0 + 32 * wave;
  const int64_t qi = q0 + l32;  // this lane's query
  const int64_t S = p.S;
  const int64_t qc = qi < S ? qi : S - 1;

  const float* qbase = p.q + b * S * p.ldq + h * kD;
  const float* kbase = p.k + b * S * p.ldk + h * kD;
  const float* vbase = p.v + b * S * p.ldv + h * kD;
  const uint8_t* mbase = p.mask ? p.mask + b * p.ms0 + h * p.ms1 : nullptr;

  // Key range of this block.
  int64_t key_end = S;
  if (p.causal) {
    const int64_t qlast = qb0 + 32 * WAVES;
    key_end = qlast < S ? qlast : S;
  } else if (MASKED && p.ms2 == 0) {
    // Query-independent mask: stop after the last unmasked key. If every key
    // is masked, keep all of them (softmax over `fill` values, as the
    // reference computes it).
    if (tid == 0) s_last_valid = -1;
    __syncthreads();
    int last = -1;
    for (int64_t j = tid; j < S; j += NT)
      if (!mbase[j * p.ms3]) last = int(j);
    if (last >= 0) atomicMax(&s_last_valid, last);
    __syncthreads();
    if (s_last_valid >= 0) key_end = s_last_valid + 1;
  }
  // key_end >= 1 (S >= 1; a masked row keeps at least key 0), so ntiles >= 1
  const int64_t ntiles = (key_end + kKT - 1) / kKT;

  // Q^T operand: lane supplies Q[qi][qk_dim(s, half)] for step s (a lane
  // past the sequence reads the last query; its output is not written).
  float qf[kD / 2];
  floatx4 qr[8];
  if constexpr (VEC) {
    q_rows_load(qbase, p.ldq, q0, S, lane, qr);
  } else {
#pragma unroll
    for (int s = 0; s < kD / 2; ++s) qf[s] = qbase[qc * p.ldq + qk_dim(s, half)];
  }

  floatx16 oacc[2];
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int v = 0; v < 16; ++v) oacc[d][v] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  // Cooperative K/V tile staging: 32 keys x 64 dims = 512 float4 per tensor.
  static_assert((kKT * kD / 4) % NT == 0, "tile must split into float4 per thread");
  constexpr int NV = kKT * kD / 4 / NT;
  // native vectors: a whole-value copy of HIP's float4 struct becomes a
  // private-memory copy
  floatx4 kr[NV], vr[NV];
  uint32_t mnext = 0;  // the next tile's mask bits (bit v: score register v)
  uint8_t mown = 0;    // MROW: the next tile's mask byte of key k0 + lane % 32
  const uint8_t* mrow = MASKED ? mbase + qc * p.ms2 : nullptr;
  auto load_tile = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int idx = tid + NT * i;
      const int key = idx / (kD / 4), dq = (idx % (kD / 4)) * 4;
      const int64_t kc = k0 + key < S ? k0 + key : S - 1;
      const float* kp = kbase + kc * p.ldk + dq;
      const float* vp = vbase + kc * p.ldv + dq;
      if (VEC) {
        kr[i] = *reinterpret_cast<const floatx4*>(kp);
        vr[i] = *reinterpret_cast<const floatx4*>(vp);
      } else {
        kr[i] = floatx4{kp[0], kp[1], kp[2], kp[3]};
        vr[i] = floatx4{vp[0], vp[1], vp[2], vp[3]};
      }
    }
    if (MROW) {
      const int64_t j = k0 + l32;
      mown = mrow[(j < S ? j : S - 1) * p.ms3];
    } else if (MASKED) {
      mnext = 0;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t j = k0 + 8 * (v >> 2) + 4 * half + (v & 3);
        mnext |= uint32_t(mrow[(j < S ? j : S - 1) * p.ms3] != 0) << v;
      }
    }
  };
  // the loaded tile's mask bits (MROW: bit o for key k0 + o, from lanes 0..31)
  auto tile_bits = [&]() -> uint32_t {
    if constexpr (MROW) return uint32_t(__ballot(mown != 0));
    else return mnext;
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int idx = tid + NT * i;
      const int key = idx / (kD / 4), dq = (idx % (kD / 4)) * 4;
      *reinterpret_cast<floatx4*>(&Ks[buf][key * kKS + dq]) = kr[i];
      *reinterpret_cast<floatx4*>(&Vs[buf][key * kVS + dq]) = vr[i];
    }
  };

  load_tile(0);
  if constexpr (VEC) {
    q_rows_to_operand(lds + wave * 32 * kQS, qr, lane, qf);
    __syncthreads();  // every wave has its Q before tile 0 overwrites the slices
  }
  store_tile(0);
  uint32_t mbits = tile_bits();
  __syncthreads();

  for (int64_t t = 0; t < ntiles; ++t) {
    const int cur = int(t & 1);
    const int64_t k0 = t * kKT;
    // the next tile's loads (the last tile repeats itself past the end)
    load_tile(t + 1 < ntiles ? k0 + kKT : k0);

    // A wave whose 32 queries all lie above this tile's keys skips it
    // (causal), as does a wave past the end of the sequence.
    const bool skip = (q0 >= S) || (p.causal && k0 > q0 + 31);
    if (!skip)
      attn_tile<MASKED, MROW>(p, Ks[cur], Vs[cur], k0, qi, nullptr, qf, oacc, m_run, l_run, half,
                              l32, mbits);
    store_tile(cur ^ 1);
    mbits = tile_bits();
    __syncthreads();
  }
  // (the loop's last barrier: no wave reads the K/V tiles any more)
  if constexpr (VEC) o_rows_store(p, b, h, q0, lds + wave * 32 * kQS, oacc, 1.0f / l_run, lane);
  else if (qi < S) attn_store(p, b, h, qi, oacc, 1.0f / l_run, half);
}

// Short sequences (S <= 32*MAXT keys) on large grids: the block stages the
// whole K and V of its (batch, head), and the mask row of a query-independent
// mask, in LDS at once, so every global load of the block goes out in one
// round trip and the tile loop runs without further loads or barriers. (The
// tiled kernel above waits for each tile's loads and a barrier per tile; at
// S = 128 that latency, not the matrix cores, sets its time.) Mask handling
// as the tiled kernel: keys past the last unmasked key are skipped, and if
// every key is masked all are kept. WAVES waves of 32 queries per block;
// VEC: 16-byte aligned rows. MASK_ROW: a query-independent mask (ms2 == 0).
template <int WAVES, int MAXT, bool VEC, bool MASK_ROW>
__global__ __launch_bounds__(64 * WAVES, 2) void attn_fwd_d64_full(AttnP p) {
  constexpr int NT = 64 * WAVES;
  __shared__ __attribute__((aligned(16))) float Ks[MAXT][kKT * kKS];
  __shared__ __attribute__((aligned(16))) float Vs[MAXT][kKT * kVS];
  __shared__ uint8_t s_mask[MAXT * kKT];
  __shared__ int s_last_valid;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, l32 = lane & 31;
  const int64_t b = blockIdx.z, h = blockIdx.y;
  const int64_t qb0 = int64_t(blockIdx.x) * (32 * WAVES);
  const int64_t q0 = qb0 + 32 * wave;
  const int64_t qi = q0 + l32;
  const int64_t S = p.S;  // 1 <= S <= MAXT * kKT (host-checked)
  const int64_t qc = qi < S ? qi : S - 1;
  const float* qbase = p.q + b * S * p.ldq + h * kD;
  const float* kbase = p.k + b * S * p.ldk + h * kD;
  const float* vbase = p.v + b * S * p.ldv + h * kD;
  const uint8_t* mbase = MASK_ROW ? p.mask + b * p.ms0 + h * p.ms1 : nullptr;

  // Every load first: Q, all K/V tiles, the mask row (keys clamped into the
  // sequence; a clamped key's score is -inf, so its V row weighs 0). With VEC
  // the Q rows, and at the end the output rows, pass through Vs.
  static_assert(WAVES * 32 * kQS <= MAXT * kKT * kVS, "Q/O staging must fit in Vs");
  float qf[kD / 2];
  floatx4 qr[8];
  if constexpr (VEC) {
    q_rows_load(qbase, p.ldq, q0, S, lane, qr);
  } else {
#pragma unroll
    for (int s = 0; s < kD / 2; ++s) qf[s] = qbase[qc * p.ldq + qk_dim(s, half)];
  }
  static_assert((kKT * kD / 4) % NT == 0, "tile must split into float4 per thread");
  constexpr int NV = kKT * kD / 4 / NT;
  floatx4 kr[MAXT][NV], vr[MAXT][NV];
#pragma unroll
  for (int t = 0; t < MAXT; ++t)
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int idx = tid + NT * i;
      const int key = t * kKT + idx / (kD / 4), dq = (idx % (kD / 4)) * 4;
      const int64_t kc = key < S ? key : S - 1;
      const float* kp = kbase + kc * p.ldk + dq;
      const float* vp = vbase + kc * p.ldv + dq;
      if (VEC) {
        kr[t][i] = *reinterpret_cast<const floatx4*>(kp);
        vr[t][i] = *reinterpret_cast<const floatx4*>(vp);
      } else {
        kr[t][i] = floatx4{kp[0], kp[1], kp[2], kp[3]};
        vr[t][i] = floatx4{vp[0], vp[1], vp[2], vp[3]};
      }
    }
  uint8_t mrow[(MAXT * kKT + NT - 1) / NT];
  if (MASK_ROW) {
#pragma unroll
    for (int i = 0; i < (MAXT * kKT + NT - 1) / NT; ++i) {
      const int j = tid + NT * i;
      mrow[i] = mbase[(j < S ? j : S - 1) * p.ms3];
    }
  }
  if constexpr (VEC) {
    q_rows_to_operand(&Vs[0][0] + wave * 32 * kQS, qr, lane, qf);
    __syncthreads();  // every wave has its Q before the tiles overwrite Vs
  }
#pragma unroll
  for (int t = 0; t < MAXT; ++t)
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int idx = tid + NT * i;
      const int key = idx / (kD / 4), dq = (idx % (kD / 4)) * 4;
      *reinterpret_cast<floatx4*>(&Ks[t][key * kKS + dq]) = kr[t][i];
      *reinterpret_cast<floatx4*>(&Vs[t][key * kVS + dq]) = vr[t][i];
    }
  int64_t key_end = S;
  if (MASK_ROW) {
    if (tid == 0) s_last_valid = -1;
    int last = -1;
#pragma unroll
    for (int i = 0; i < (MAXT * kKT + NT - 1) / NT; ++i) {
      const int j = tid + NT * i;
      if (j < MAXT * kKT) s_mask[j] = mrow[i];
      if (j < S && !mrow[i]) last = j;
    }
    __syncthreads();
    if (last >= 0) atomicMax(&s_last_valid, last);
    __syncthreads();
    if (s_last_valid >= 0) key_end = s_last_valid + 1;
  } else {
    __syncthreads();
    if (p.causal) {
      const int64_t qlast = qb0 + 32 * WAVES;
      key_end = qlast < S ? qlast : S;
    }
  }
  const int ntiles = int((key_end + kKT - 1) / kKT);

  floatx16 oacc[2];
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int v = 0; v < 16; ++v) oacc[d][v] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;
  if (q0 < S) {
    for (int t = 0; t < ntiles; ++t) {
      const int64_t k0 = int64_t(t) * kKT;
      if (p.causal && k0 > q0 + 31) break;  // later tiles are masked for all 32 queries
      // bit o: key k0 + o is masked (one LDS byte per lane, shared by a ballot)
      const uint32_t mbits = MASK_ROW ? uint32_t(__ballot(s_mask[k0 + l32] != 0)) : 0u;
      attn_tile<MASK_ROW, true>(p, Ks[t], Vs[t], k0, qi, nullptr, qf, oacc, m_run, l_run, half,
                                l32, mbits);
    }
  }
  if constexpr (VEC) {
    __syncthreads();  // every wave is done with the tiles in Vs
    o_rows_store(p, b, h, q0, &Vs[0][0] + wave * 32 * kQS, oacc, 1.0f / l_run, lane);
  } else if (qi < S) {
    attn_store(p, b, h, qi, oacc, 1.0f / l_run, half);
  }
}

// Small grids (b=1): the KW waves of a block share the same 32 queries and
// split the key tiles (wave w takes tiles w, w+KW, ...), each staging its
// tiles in its own LDS slice, so a block finishes after ceil(tiles/KW) tile
// steps instead of all of them. The KW partial states (m, l, O) are merged
// through LDS: M = max_w m_w, O = sum_w exp(m_w - M) O_w, l likewise.
template <int KW>
__global__ __launch_bounds__(64 * KW) void attn_fwd_d64_ks(AttnP p) {
  constexpr int NT = 64 * KW;
  __shared__ __attribute__((aligned(16))) float Ks[KW][kKT * kKS];
  __shared__ __attribute__((aligned(16))) float Vs[KW][kKT * kVS];
  __shared__ int s_last_valid;
  __shared__ float sm[KW][32], sl[KW][32];
  static_assert(KW * 32 * kD <= KW * kKT * kKS, "O merge buffer must fit in Ks");

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, l32 = lane & 31;
  const int64_t b = blockIdx.z, h = blockIdx.y;
  const int64_t q0 = int64_t(blockIdx.x) * 32;
  const int64_t qi = q0 + l32;
  const int64_t S = p.S;
  const float* qbase = p.q + b * S * p.ldq + h * kD;
  const float* kbase = p.k + b * S * p.ldk + h * kD;
  const float* vbase = p.v + b * S * p.ldv + h * kD;
  const uint8_t* mbase = p.mask ? p.mask + b * p.ms0 + h * p.ms1 : nullptr;

  int64_t key_end = S;
  if (p.causal) {
    key_end = (q0 + 32) < S ? q0 + 32 : S;
  } else if (mbase && p.ms2 == 0) {
    if (tid == 0) s_last_valid = -1;
    __syncthreads();
    int last = -1;
    for (int64_t j = tid; j < S; j += NT)
      if (!mbase[j * p.ms3]) last = int(j);
    if (last >= 0) atomicMax(&s_last_valid, last);
    __syncthreads();
    if (s_last_valid >= 0) key_end = s_last_valid + 1;
  }
  const int64_t ntiles = (key_end + kKT - 1) / kKT;

  float qf[kD / 2];
#pragma unroll
  for (int s = 0; s < kD / 2; ++s) qf[s] = (qi < S) ? qbase[qi * p.ldq + qk_dim(s, half)] : 0.0f;
  floatx16 oacc[2];
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int v = 0; v < 16; ++v) oacc[d][v] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  float* ks = Ks[wave];
  float* vs = Vs[wave];
  for (int64_t t = wave; t < ntiles; t += KW) {
    const int64_t k0 = t * kKT;
    // wave-private staging of 32 keys x 64 dims of K and V (8 float4 per lane)
    float4 kr[8], vr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int idx = lane + 64 * i;
      const int key = idx / (kD / 4), dq = (idx % (kD / 4)) * 4;
      kr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      vr[i] = kr[i];
      if (k0 + key < S) {
        const float* kp = kbase + (k0 + key) * p.ldk + dq;
        const float* vp = vbase + (k0 + key) * p.ldv + dq;
        kr[i] = make_float4(kp[0], kp[1], kp[2], kp[3]);
        vr[i] = make_float4(vp[0], vp[1], vp[2], vp[3]);
      }
    }
    wave_lds_barrier();  // the previous tile's LDS reads are done
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int idx = lane + 64 * i;
      const int key = idx / (kD / 4), dq = (idx % (kD / 4)) * 4;
      *reinterpret_cast<float4*>(ks + key * kKS + dq) = kr[i];
      *reinterpret_cast<float4*>(vs + key * kVS + dq) = vr[i];
    }
    wave_lds_barrier();  // this tile is visible to every lane of the wave
    if (!(q0 >= S || (p.causal && k0 > q0 + 31)))
      attn_tile(p, ks, vs, k0, qi, mbase, qf, oacc, m_run, l_run, half, l32);
  }

  __syncthreads();  // every wave is done with its K/V slice: reuse Ks for O
  float* obuf = &Ks[0][0];  // [KW][32 queries][64 dims]
  if (half == 0) {
    sm[wave][l32] = m_run;
    sl[wave][l32] = l_run;
  }
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int v = 0; v < 16; ++v)
      obuf[(wave * 32 + l32) * kD + d * 32 + 8 * (v >> 2) + 4 * half + (v & 3)] = oacc[d][v];
  __syncthreads();
  if (wave != 0 || qi >= S) return;
  float M = sm[0][l32];
  for (int w = 1; w < KW; ++w) M = fmaxf(M, sm[w][l32]);
  float L = 0.0f, cw[KW];
#pragma unroll
  for (int w = 0; w < KW; ++w) {
    cw[w] = __expf(sm[w][l32] - M);
    L += cw[w] * sl[w][l32];
  }
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      float o = 0.0f;
#pragma unroll
      for (int w = 0; w < KW; ++w)
        o += cw[w] * obuf[(w * 32 + l32) * kD + d * 32 + 8 * (v >> 2) + 4 * half + (v & 3)];
      oacc[d][v] = o;
    }
  attn_store(p, b, h, qi, oacc, 1.0f / L, half);
}

// Small grids with 16-byte aligned rows (the b=1 encoder, GPT-2 prefill): 16
// queries per block on v_mfma_f32_16x16x4f32, so twice as many blocks as the
// 32-query kernels and half the matrix-core chain per wave. The KW waves
// split the 32-key tiles (wave w takes tiles w, w+KW, ...) and load their
// operands straight into registers, mask bytes included; nothing waits on a
// block-wide scan. Lane l (r = l%16, g = l/16):
//   S^T = K Q^T:  step s pairs MFMA k-index g with head dim 16g + s, so the
//                 lane's Q row (query q0+r) and K rows (keys k0+16kb+r) are
//                 four float4 loads of dims [16g, 16g+16) each;
//                 score register v of key block kb: key k0+16kb+4g+v, query r.
//   O^T += V^T P^T: step (kb, v) pairs k-index g with key k0+16kb+4g+v, which
//                 is exactly the probability the lane already holds. Output
//                 row i of dim block db is dim 4i + db, so the V^T operands
//                 of the lane's four blocks are one float4, V[that key][4r..
//                 4r+3], and accumulator register v of block db holds dim
//                 16g + 4v + db of query r.
// MROW: a query-independent mask (ms2 == 0, not causal): each wave loads the
// tile's 32 mask bytes once, one per lane, and shares them by a ballot.
// The KW partial states (m, l, O) are merged through LDS, wave w merging dim
// block w for all 16 queries.

template <int KW, bool MROW>
// The operands of the first loads lead the arguments as scalars (preloaded
// in SGPRs); the rest of the launch's parameters come in p.
__global__ __launch_bounds__(64 * KW) void attn_fwd_d64_q16(const float* __restrict__ q_,
                                                            const float* __restrict__ k_,
                                                            const float* __restrict__ v_,
                                                            int64_t S_, int64_t ldq, int64_t ldk,
                                                            int64_t ldv, AttnP p) {
  __shared__ __attribute__((aligned(16))) float obuf[KW][16][kD + 4];
  __shared__ float sm[KW][16], sl[KW][16];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int64_t b = blockIdx.z, h = blockIdx.y, S = S_;
  const int64_t q0 = int64_t(blockIdx.x) * 16;
  const int64_t qi = q0 + r;
  const int64_t qc = qi < S ? qi : S - 1;
  const float* qbase = q_ + b * S * ldq + h * kD;
  const float* kbase = k_ + b * S * ldk + h * kD;
  const float* vbase = v_ + b * S * ldv + h * kD;
  const uint8_t* mbase = p.mask ? p.mask + b * p.ms0 + h * p.ms1 : nullptr;

  float4 qv[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    qv[c] = *reinterpret_cast<const float4*>(qbase + qc * ldq + 16 * g + 4 * c);

  floatx4 oacc[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) oacc[d] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;

  const int64_t ntiles = (S + kKT - 1) / kKT;
  for (int64_t t = wave; t < ntiles; t += KW) {
    const int64_t k0 = t * kKT;
    if (p.causal && k0 > q0 + 15) break;  // later tiles are masked for every query here
    // Operands of this tile, all loads issued before any use.
    float4 kv[2][4];
    floatx4 vv[2][4];  // [kb][v]: component db is the V^T operand of dim block db
    uint8_t mk[2][4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int64_t kr = k0 + 16 * kb + r;
      const float* kp = kbase + (kr < S ? kr : S - 1) * ldk + 16 * g;
#pragma unroll
      for (int c = 0; c < 4; ++c) kv[kb][c] = *reinterpret_cast<const float4*>(kp + 4 * c);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t key = k0 + 16 * kb + 4 * g + v;
        const int64_t kc = key < S ? key : S - 1;
        vv[kb][v] = *reinterpret_cast<const floatx4*>(vbase + kc * ldv + 4 * r);
        if (!MROW)
          mk[kb][v] = (mbase && !p.causal && qi < S) ? mbase[qi * p.ms2 + kc * p.ms3] : uint8_t(0);
      }
    }
    uint8_t mown = 0;  // MROW: the mask byte of key k0 + lane % 32
    if (MROW) {
      const int64_t j = k0 + (lane & 31);
      mown = mbase[(j < S ? j : S - 1) * p.ms3];
    }
    floatx4 sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sacc[kb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const float4 kq = kv[kb][s >> 2], qq = qv[s >> 2];
        const int e = s & 3;
        const float a = e == 0 ? kq.x : e == 1 ? kq.y : e == 2 ? kq.z : kq.w;
        const float bq = e == 0 ? qq.x : e == 1 ? qq.y : e == 2 ? qq.z : qq.w;
        sacc[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, bq, sacc[kb], 0, 0, 0);
      }
    }
    float sv[2][4];
    float tmax = -INFINITY;
    // bit o: key k0 + o is masked (lanes 32..63 repeat lanes 0..31)
    const uint64_t mbits = MROW ? __ballot(mown != 0) : 0;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t j = k0 + 16 * kb + 4 * g + v;
        const bool masked = MROW ? ((mbits >> (16 * kb + 4 * g + v)) & 1u) != 0 : mk[kb][v] != 0;
        float s = p.scale * sacc[kb][v];
        if (j >= S) s = -INFINITY;  // key does not exist
        else if (p.causal ? (j > qi) : masked) s = p.fill;
        sv[kb][v] = s;
        tmax = fmaxf(tmax, s);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    // A fill of -inf can leave a tile with no finite score; keep the state.
    const bool none = m_new == -INFINITY;
    const float corr = none ? 1.0f : __expf(m_run - m_new);
    float lsum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        sv[kb][v] = none ? 0.0f : __expf(sv[kb][v] - m_new);
        lsum += sv[kb][v];
      }
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    l_run = l_run * corr + lsum;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < 4; ++db) oacc[db] *= corr;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int db = 0; db < 4; ++db)
          oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[kb][v][db], sv[kb][v], oacc[db], 0,
                                                          0, 0);
  }

  // oacc[db] register v: dim 16g + 4v + db of query r.
#pragma unroll
  for (int v = 0; v < 4; ++v)
    *reinterpret_cast<floatx4*>(&obuf[wave][r][16 * g + 4 * v]) =
        floatx4{oacc[0][v], oacc[1][v], oacc[2][v], oacc[3][v]};
  if (g == 0) {
    sm[wave][r] = m_run;
    sl[wave][r] = l_run;
  }
  __syncthreads();
  if (qi >= S) return;
  float M = sm[0][r];
#pragma unroll
  for (int w = 1; w < KW; ++w) M = fmaxf(M, sm[w][r]);
  float cw[KW], L = 0.0f;
#pragma unroll
  for (int w = 0; w < KW; ++w) {
    cw[w] = __expf(sm[w][r] - M);  // 0 for a wave that saw no tile (m = -inf)
    L += cw[w] * sl[w][r];
  }
  const float inv = 1.0f / L;
  float* orow = p.out + (b * S + qi) * p.ldo + h * kD;
  for (int db = wave; db < 4; db += KW) {
    float o[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float acc = 0.0f;
#pragma unroll
      for (int w = 0; w < KW; ++w) acc += cw[w] * obuf[w][r][16 * db + 4 * g + v];
      o[v] = acc * inv;
    }
    *reinterpret_cast<float4*>(orow + 16 * db + 4 * g) = make_float4(o[0], o[1], o[2], o[3]);
  }
}

// Any head_dim up to 256: one thread per (b, h, query) with an online softmax
// over the keys. Used for shapes the MFMA kernel does not cover.
constexpr int kMaxGenericD = 256;

__global__ __launch_bounds__(128) void attn_fwd_generic(AttnP p, int64_t D) {
  const int64_t total = p.B * p.nH * p.S;
  const int64_t t = int64_t(blockIdx.x) * 128 + threadIdx.x;
  if (t >= total) return;
  const int64_t i = t % p.S, h = (t / p.S) % p.nH, b = t / (p.S * p.nH);
  const float* qr = p.q + (b * p.S + i) * p.ldq + h * D;
  const uint8_t* mb = p.mask ? p.mask + b * p.ms0 + h * p.ms1 + i * p.ms2 : nullptr;
  float o[kMaxGenericD];
  for (int64_t d = 0; d < D; ++d) o[d] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  for (int64_t j = 0; j < p.S; ++j) {
    const float* kr = p.k + (b * p.S + j) * p.ldk + h * D;
    float acc = 0.0f;
    for (int64_t d = 0; d < D; ++d) acc += qr[d] * kr[d];
    float s = p.scale * acc;
    if (p.causal ? (j > i) : (mb && mb[j * p.ms3])) s = p.fill;
    const float m_new = fmaxf(m, s);
    const float corr = expf(m - m_new);
    const float e = expf(s - m_new);
    l = l * corr + e;
    const float* vr = p.v + (b * p.S + j) * p.ldv + h * D;
    for (int64_t d = 0; d < D; ++d) o[d] = o[d] * corr + e * vr[d];
    m = m_new;
  }
  float* orow = p.out + (b * p.S + i) * p.ldo + h * D;
  const float inv = 1.0f / l;
  for (int64_t d = 0; d < D; ++d) orow[d] = o[d] * inv;
}

}  // namespace

void attention(inferc_hip_ctx* ctx, const AttnArgs& a) {
  IH_REQUIRE(a.B >= 0 && a.S >= 0 && a.H > 0 && a.head_dim > 0, INFERC_ERR_SHAPE,
             "attention: bad shape");
  IH_REQUIRE(a.H % a.head_dim == 0, INFERC_ERR_SHAPE,
             "FusedAttention: H not divisible by head_dim");
  if (a.B == 0 || a.S == 0) return;
  IH_REQUIRE(a.q && a.k && a.v && a.out, INFERC_ERR_ARG, "attention: null pointer");
  IH_REQUIRE(a.ldq >= a.H && a.ldk >= a.H && a.ldv >= a.H && a.ldo >= a.H, INFERC_ERR_SHAPE,
             "attention: row stride smaller than H");
  AttnP p{};
  p.B = a.B; p.S = a.S; p.nH = a.H / a.head_dim;
  p.q = a.q; p.k = a.k; p.v = a.v;
  p.ldq = a.ldq; p.ldk = a.ldk; p.ldv = a.ldv; p.ldo = a.ldo;
  p.mask = a.mask;
  p.ms0 = a.ms[0]; p.ms1 = a.ms[1]; p.ms2 = a.ms[2]; p.ms3 = a.ms[3];
  p.fill = a.fill;
  p.scale = 1.0f / sqrtf(float(a.head_dim));
  p.causal = a.causal;
  p.out = a.out;
  if (a.head_dim == kD) {
    IH_REQUIRE(a.B < 65536 && p.nH < 65536, INFERC_ERR_SHAPE, "attention: grid too large");
    const int64_t blocks4 = ceil_div(a.S, 128) * p.nH * a.B;
    const bool vec = a.ldq % 4 == 0 && a.ldk % 4 == 0 && a.ldv % 4 == 0 && a.ldo % 4 == 0 &&
                     aligned16(a.q) && aligned16(a.k) && aligned16(a.v) && aligned16(a.out);
    if (blocks4 < ctx->num_cus && vec) {
      // few blocks: 16 queries per block, four waves splitting the key tiles
      dim3 grid(unsigned(ceil_div(a.S, 16)), unsigned(p.nH), unsigned(a.B));
      if (p.mask != nullptr && !p.causal && p.ms2 == 0)
        hipLaunchKernelGGL((attn_fwd_d64_q16<4, true>), grid, dim3(256), 0, ctx->stream, p.q, p.k,
                           p.v, p.S, p.ldq, p.ldk, p.ldv, p);
      else
        hipLaunchKernelGGL((attn_fwd_d64_q16<4, false>), grid, dim3(256), 0, ctx->stream, p.q,
                           p.k, p.v, p.S, p.ldq, p.ldk, p.ldv, p);
    } else if (blocks4 >= ctx->num_cus && a.S <= 4 * kKT &&
               (p.mask == nullptr || p.causal || p.ms2 == 0)) {
      // short sequences: the whole K/V of a (batch, head) staged at once
      const bool mrow = p.mask != nullptr && !p.causal;
      dim3 grid(unsigned(ceil_div(a.S, 128)), unsigned(p.nH), unsigned(a.B));
      auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(256), 0, ctx->stream, p); };
      if (vec) {
        if (mrow) go(attn_fwd_d64_full<4, 4, true, true>);
        else go(attn_fwd_d64_full<4, 4, true, false>);
      } else {
        if (mrow) go(attn_fwd_d64_full<4, 4, false, true>);
        else go(attn_fwd_d64_full<4, 4, false, false>);
      }
    } else if (blocks4 >= ctx->num_cus) {
      const bool masked = p.mask != nullptr && !p.causal;
      dim3 grid(unsigned(ceil_div(a.S, 128)), unsigned(p.nH), unsigned(a.B));
      auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(256), 0, ctx->stream, p); };
      const bool mrow = masked && p.ms2 == 0;
      if (vec) {
        if (mrow) go(attn_fwd_d64<4, true, true, true>);
        else if (masked) go(attn_fwd_d64<4, true, true>);
        else go(attn_fwd_d64<4, true, false>);
      } else {
        if (mrow) go(attn_fwd_d64<4, false, true, true>);
        else if (masked) go(attn_fwd_d64<4, false, true>);
        else go(attn_fwd_d64<4, false, false>);
      }
    } else {
      // few blocks: four waves per 32 queries, splitting the key tiles
      dim3 grid(unsigned(ceil_div(a.S, 32)), unsigned(p.nH), unsigned(a.B));
      hipLaunchKernelGGL(attn_fwd_d64_ks<4>, grid, dim3(256), 0, ctx->stream, p);
    }
    check_launch("attn_fwd_d64");
    return;
  }
  IH_REQUIRE(a.head_dim <= kMaxGenericD, INFERC_ERR_UNSUPPORTED,
             "attention: head_dim > 256 is not supported");
  const int64_t total = a.B * p.nH * a.S;
  hipLaunchKernelGGL(attn_fwd_generic, dim3(unsigned(ceil_div(total, 128))), dim3(128), 0,
                     ctx->stream, p, a.head_dim);
  check_launch("attn_fwd_generic");
}

}  // namespace ih

extern "C" int inferc_hip_fused_attention_f32(inferc_hip_ctx* ctx, int64_t B, int64_t S,
                                              int64_t H, int64_t head_dim, const float* q,
                                              const float* k, const float* v,
                                              const uint8_t* mask, const int64_t* mask_strides,
                                              float fill, float* out) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    ih::AttnArgs a;
    a.B = B; a.S = S; a.H = H; a.head_dim = head_dim;
    a.q = q; a.k = k; a.v = v;
    a.ldq = a.ldk = a.ldv = a.ldo = H;
    a.mask = mask;
    if (mask) {
      IH_REQUIRE(mask_strides != nullptr, INFERC_ERR_ARG, "attention: mask without strides");
      for (int i = 0; i < 4; ++i) a.ms[i] = mask_strides[i];
    }
    a.fill = fill;
    a.out = out;
    ih::attention(ctx, a);
  });
}
