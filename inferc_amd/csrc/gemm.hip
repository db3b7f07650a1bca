// fp32 GEMM on CDNA4 matrix cores (v_mfma_f32_32x32x2_f32), with the fused
// epilogues of inferc's fused ops.
//
// Reference semantics:
//   rt::MatMul / rt::Gemm            src/kernels/matmul.cc:63-228
//   rt::FusedMatMulAddGELU           src/kernels/fused_matmul_add_gelu.cc:13-80
//   rt::FusedQKVProjection           src/kernels/attention.cc:102-141
// Epilogue order: v = alpha*acc; v = v + beta*C; v = v + R; y = act(v), which
// is (acc + b) + residual for MatMul->Add(b)->Add(res) and GELU(acc + b) for
// the fused FFN, as the reference computes them.
//
// Design: 256-thread blocks (4 wave64s in a 2x2 or 4x1 grid). Each wave owns
// a sub-tile made of 32x32 MFMA tiles. K advances in BK-deep panels staged
// through LDS, double-buffered, with the global loads two panels ahead: those
// of panel t+2 are in flight while panel t feeds the matrix cores. Both
// operands sit in LDS k-major ([BK][outer]) so every MFMA operand read is 32
// consecutive floats per half-wave.
//
// Shapes with too few 128x128 tiles to fill the 256 CUs go to one of two
// other paths. Small M with float4-aligned row-major A (the b=1 encoder, GPT-2
// prefill) goes to gemm_f32_ksplit: K is split between the waves of a block,
// and the partial tiles are summed through LDS in the same launch. Other
// shapes run the 64x64 kernel with K split over blocks; partial sums land in
// the context workspace, and a second kernel reduces them in fixed order
// (deterministic) and applies the epilogue.
#include <mutex>
#include <type_traits>
#include <string>
#include <vector>

#include "common.h"

namespace ih {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kMaxSlices = 3;

struct GemmParams {
  int64_t M, N, K;
  const float* A;
  int64_t lda, sa;
  const float* B;
  int64_t ldb, sb;
  float alpha, beta;
  const float* C;
  int c_kind;
  int64_t ldc;
  const float* R;
  int64_t ldr, sr;
  int act;
  float* Y;
  int64_t ldy, sy;
  // Optional per-slice pointer tables (fused QKV); when use_table is set the
  // slice index selects B/C/Y from these instead of the strides above.
  int use_table;
  const float* Bt[kMaxSlices];
  const float* Ct[kMaxSlices];
  float* Yt[kMaxSlices];
  int splits;
  int64_t k_per_split;
  float* partial;  // [slices][splits][M][N] when splits > 1
  // small-M path: LayerNorm of A's rows (over K) and R's rows (over N) as
  // read, from producer partials; Y's per-16-column (mean, M2) out
  const float* na_stats;
  const float* na_c[kMaxSlices];  // per slice: column sums of the gamma-scaled B
  float na_eps;
  const float* nr_stats;
  const float* nr_g;
  const float* nr_b;
  float nr_eps;
  float* st_out;
};

// Merges the (count, mean, M2) summary b into a (Chan et al.'s pairwise
// update); an empty side leaves the other unchanged. The counts are small
// integers, so a hardware reciprocal stands in for the divisions.
__device__ __forceinline__ void merge_moments(float& na, float& ma, float& sa, float nb, float mb,
                                              float sb) {
  const float n = na + nb;
  const float inv = n > 0.0f ? __builtin_amdgcn_rcpf(n) : 0.0f;
  const float d = mb - ma;
  ma = fmaf(d, nb * inv, ma);
  sa = sa + sb + d * d * (na * nb * inv);
  na = n;
}

// Value of the lane R places further on within its row of 16 lanes (DPP
// row_ror).
template <int R>
__device__ __forceinline__ float row_ror(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x120 + R, 0xF, 0xF, false));
}

// LayerNorm row statistics from per-16-column partials st[row][c] =
// (mean_c, M2_c), c < nc <= 64 (D = 16 * nc <= 1024 features): a group of 16
// lanes per row, lane l of the group holding columns l, l + 16, ... The
// loads come first (row_stats_load), so the merge (row_stats_merge) can run
// while later loads are still in flight.
struct RowStatLoads {
  float2 v[4];
};

// Unconditional loads from columns clamped into the row (nc >= 1); the
// merge masks the columns past nc, so the wait for these loads counts them
// exactly.
__device__ __forceinline__ void row_stats_load(RowStatLoads& r, const float* __restrict__ st,
                                               int64_t row, int64_t nc, int lane) {
  const float2* p = reinterpret_cast<const float2*>(st) + row * nc;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t c = (lane & 15) + 16 * u;
    r.v[u] = p[c < nc ? c : nc - 1];
  }
}

// (mean, 1/sqrt(var + eps)) of the group's row: the lane's columns, then
// rotations by 8, 4, 2 and 1 within the 16 lanes, after which every lane has
// merged all 16 (in its own order; lane 0 of the group gives the row's
// values). var = M2 / D, the biased variance LayerNorm uses.
template <int R>
__device__ __forceinline__ void merge_rotated(float& n, float& mean, float& m2) {
  const float nb = row_ror<R>(n), mb = row_ror<R>(mean), sb = row_ror<R>(m2);
  merge_moments(n, mean, m2, nb, mb, sb);
}

__device__ __forceinline__ float2 row_stats_merge(const RowStatLoads& r, int64_t nc, float eps,
                                                  int lane) {
  float n = 0.0f, mean = 0.0f, m2 = 0.0f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const bool in = (lane & 15) + 16 * u < nc;
    merge_moments(n, mean, m2, in ? 16.0f : 0.0f, r.v[u].x, in ? r.v[u].y : 0.0f);
  }
  merge_rotated<8>(n, mean, m2);
  merge_rotated<4>(n, mean, m2);
  merge_rotated<2>(n, mean, m2);
  merge_rotated<1>(n, mean, m2);
  return make_float2(mean, 1.0f / sqrtf(m2 / n + eps));  // as the LayerNorm kernel
}

// Workgroup barrier for LDS data only: unlike __syncthreads it does not make
// the wave wait for its global loads still in flight.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// alpha * acc + beta * C: the epilogue up to the residual
__device__ __forceinline__ float epilogue_pre(const GemmParams& p, const float* C, float acc,
                                              int64_t row, int64_t col) {
  float v = p.alpha * acc;
  if (C != nullptr && p.beta != 0.0f) {
    float c = 0.0f;
    if (p.c_kind == INFERC_C_ROW) c = C[col];
    else if (p.c_kind == INFERC_C_FULL) c = C[row * p.ldc + col];
    else if (p.c_kind == INFERC_C_SCALAR) c = C[0];
    v = v + p.beta * c;
  }
  return v;
}

__device__ __forceinline__ float epilogue(const GemmParams& p, const float* C,
                                          const float* R, float acc,
                                          int64_t row, int64_t col) {
  float v = epilogue_pre(p, C, acc, row, col);
  if (R != nullptr) v = v + R[row * p.ldr + col];
  return apply_act(v, p.act);
}

// Stages one operand panel (OUTER rows of the output dimension x BK of K)
// from global memory into registers, then into LDS laid out [BK][STRIDE].
// KCONTIG: element (o,k) lives at P[o*ld + k] (K contiguous); otherwise at
// P[k*ld + o] (the output dimension contiguous).
//
// PanelAddr holds a thread's element offsets, computed once (32-bit: the
// host keeps each operand below 2^31 elements); PanelRegs loads one panel
// at depth k0 from them. Every load is issued, from coordinates clamped
// into the matrix: a load under a branch would make the compiler wait for
// all loads in flight at the join, not just for the panel being written.
// Rows and columns past M and N only reach outputs that are never written;
// k past the last panel's valid depth is masked when that panel is read.
template <int OUTER, int BK, bool KCONTIG, bool VEC>
struct PanelAddr {
  static_assert((OUTER * BK) % (4 * kThreads) == 0, "panel must split into float4 per thread");
  static constexpr int NV = OUTER * BK / (4 * kThreads);
  int off[NV];  // the thread's float4 i at k0 = 0 (o clamped into the matrix)
  int lim[NV];  // largest k0 whose load stays inside the matrix
  int d[NV][4];  // !KCONTIG && !VEC: column j's offset, clamped
  int ld;

  // k_end: the matrix's K (the loads' bound; a split's own end is kn's)
  __device__ __forceinline__ void init(int64_t ld_, int64_t o0, int64_t o_lim, int64_t k_end,
                                       int tid) {
    ld = int(ld_);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int idx = tid + kThreads * i;
      if (KCONTIG) {
        const int64_t o = o0 + idx / (BK / 4);
        const int kq = (idx % (BK / 4)) * 4;
        const int oc = int(o < o_lim ? o : o_lim - 1);
        off[i] = oc * ld + kq;
        // VEC: the float4 at k0 + kq must end by k_end (k_end % 4 == 0)
        lim[i] = int(k_end - (VEC ? 4 : 1) - kq);
      } else {
        const int kl = idx / (OUTER / 4);
        const int64_t o = o0 + (idx % (OUTER / 4)) * 4;
        // VEC: o_lim % 4 == 0, so a float4 starting in range stays in range
        const int oc = int(VEC ? (o < o_lim ? o : o_lim - 4) : o);
        off[i] = kl * ld + oc;
        lim[i] = int(k_end - 1 - kl);
        if (!VEC) {
#pragma unroll
          for (int j = 0; j < 4; ++j) d[i][j] = int((o + j < o_lim ? o + j : o_lim - 1) - o);
        }
      }
    }
  }
};

template <int OUTER, int BK, int STRIDE, bool KCONTIG, bool VEC>
struct PanelRegs {
  using Addr = PanelAddr<OUTER, BK, KCONTIG, VEC>;
  static constexpr int NV = Addr::NV;
  floatx4 r[NV];  // a native vector: whole-value copies stay in registers

  __device__ __forceinline__ void load(const float* __restrict__ P, const Addr& a, int k0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (KCONTIG) {
        if (VEC) {
          r[i] = *reinterpret_cast<const floatx4*>(P + (a.off[i] + (k0 < a.lim[i] ? k0 : a.lim[i])));
        } else {
          float e[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) e[j] = P[a.off[i] + (k0 + j < a.lim[i] ? k0 + j : a.lim[i])];
          r[i] = floatx4{e[0], e[1], e[2], e[3]};
        }
      } else {
        const int row = a.off[i] + (k0 < a.lim[i] ? k0 : a.lim[i]) * a.ld;
        if (VEC) {
          r[i] = *reinterpret_cast<const floatx4*>(P + row);
        } else {
          r[i] = floatx4{P[row + a.d[i][0]], P[row + a.d[i][1]], P[row + a.d[i][2]],
                         P[row + a.d[i][3]]};
        }
      }
    }
  }

  __device__ __forceinline__ void store(float* __restrict__ S, int tid) const {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int idx = tid + kThreads * i;
      if (KCONTIG) {
        const int ol = idx / (BK / 4), kq = (idx % (BK / 4)) * 4;
        S[(kq + 0) * STRIDE + ol] = r[i][0];
        S[(kq + 1) * STRIDE + ol] = r[i][1];
        S[(kq + 2) * STRIDE + ol] = r[i][2];
        S[(kq + 3) * STRIDE + ol] = r[i][3];
      } else {
        const int kl = idx / (OUTER / 4), oq = (idx % (OUTER / 4)) * 4;
        *reinterpret_cast<floatx4*>(S + kl * STRIDE + oq) = r[i];
      }
    }
  }
};

// Four waves in a WGM x WGN grid, each owning a (BM/WGM) x (BN/WGN) sub-tile of
// 32x32 MFMA tiles. Two register sets stage the panels, so the loads of panel
// t+2 are issued before panel t's MFMAs and panel t+1, loaded during panel
// t-1, is written to LDS after them: a panel's global latency is hidden
// behind two panels of MFMAs instead of one. Every load is unconditional (a
// panel index past the end repeats the last panel, whose copy is never
// read), so the wait before each LDS write counts exactly the loads it needs.
template <int BM, int BN, int BK, int WGM, int WGN, bool TA, bool TB, bool VEC>
__global__ __launch_bounds__(kThreads, 2) void gemm_f32_mfma(GemmParams p) {
  static_assert(WGM * WGN * 64 == kThreads, "four waves");
  // LDS row padding: 4 floats where rows are written as float4 (keeps
  // 16-byte alignment); where rows are written element-wise (the
  // transposing stores of a row-major A) the padding makes a half-wave's 32
  // stores hit 32 banks: lanes (a, b) = (lane % (BK/4), lane / (BK/4)) write
  // bank 4*SA*a + b (mod 32), distinct when SA = 2 (mod 8) for BK = 16 and
  // SA = 1 (mod 8) for BK = 32.
  constexpr int SA = BM + (TA ? 4 : BK == 32 ? 1 : 2);
  constexpr int SB = BN + (TB ? 2 : 4);
  constexpr int WTM = BM / WGM, WTN = BN / WGN, TM = WTM / 32, TN = WTN / 32;
  static_assert(TM * 32 == WTM && TN * 32 == WTN, "wave tiles of whole 32x32 MFMA tiles");
  __shared__ __attribute__((aligned(16))) float As[2][BK * SA];
  __shared__ __attribute__((aligned(16))) float Bs[2][BK * SB];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = (wave / WGN) * WTM, wn = (wave % WGN) * WTN;
  const int half = lane >> 5, l32 = lane & 31;

  const int64_t m0 = int64_t(blockIdx.y) * BM, n0 = int64_t(blockIdx.x) * BN;
  const int z = blockIdx.z;
  const int slice = z / p.splits, split = z % p.splits;

  const float* A = p.A + slice * p.sa;
  const float* B = p.use_table ? p.Bt[slice] : p.B + slice * p.sb;
  const int64_t kb = split * p.k_per_split;
  const int64_t ke = (kb + p.k_per_split < p.K) ? kb + p.k_per_split : p.K;
  const int64_t nt = (ke > kb) ? (ke - kb + BK - 1) / BK : 0;

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  auto compute = [&](const float* as, const float* bs) {
#pragma unroll
    for (int kk = 0; kk < BK; kk += 2) {
      float a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = as[(kk + half) * SA + wm + i * 32 + l32];
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j] = bs[(kk + half) * SB + wn + j * 32 + l32];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  };
  // the last panel, of valid depth kn <= BK: LDS rows at or past kn hold
  // stale or clamped values, so both operands of those k are taken as 0
  auto compute_last = [&](const float* as, const float* bs, int kn) {
#pragma unroll
    for (int kk = 0; kk < BK; kk += 2) {
      if (kk >= kn) break;
      const bool in = kk + half < kn;
      float a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = in ? as[(kk + half) * SA + wm + i * 32 + l32] : 0.0f;
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j] = in ? bs[(kk + half) * SB + wn + j * 32 + l32] : 0.0f;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  };

  if (nt > 0) {
    PanelAddr<BM, BK, !TA, VEC> aa;
    PanelAddr<BN, BK, TB, VEC> ab;
    aa.init(p.lda, m0, p.M, p.K, tid);
    ab.init(p.ldb, n0, p.N, p.K, tid);
    PanelRegs<BM, BK, SA, !TA, VEC> la0, la1;
    PanelRegs<BN, BK, SB, TB, VEC> lb0, lb1;
    // depth of panel t, and the last panel's valid depth (BK but for a
    // partial last panel)
    const int kb32 = int(kb), ntm1 = int(nt - 1);
    const int kn_last = int(ke - (kb + int64_t(ntm1) * BK));
#define IH_K_OF(t) (kb32 + (t) * BK)
    la0.load(A, aa, IH_K_OF(0));
    lb0.load(B, ab, IH_K_OF(0));
    la1.load(A, aa, IH_K_OF(ntm1 > 0 ? 1 : 0));
    lb1.load(B, ab, IH_K_OF(ntm1 > 0 ? 1 : 0));
    la0.store(As[0], tid);
    lb0.store(Bs[0], tid);
    lds_barrier();
    // Panels in pairs while two more follow the pair (both halves
    // unconditional, so the two register sets stay two sets of registers);
    // then the last one or two, without further loads.
    int t = 0;
    for (; t + 2 <= ntm1; t += 2) {
      la0.load(A, aa, IH_K_OF(t + 2));
      lb0.load(B, ab, IH_K_OF(t + 2));
      __builtin_amdgcn_sched_barrier(0);  // the loads go out before the MFMAs
      compute(As[0], Bs[0]);
      la1.store(As[1], tid);
      lb1.store(Bs[1], tid);
      lds_barrier();
      la1.load(A, aa, IH_K_OF(t + 3 <= ntm1 ? t + 3 : ntm1));
      lb1.load(B, ab, IH_K_OF(t + 3 <= ntm1 ? t + 3 : ntm1));
      __builtin_amdgcn_sched_barrier(0);
      compute(As[1], Bs[1]);
      la0.store(As[0], tid);
      lb0.store(Bs[0], tid);
      lds_barrier();
    }
    if (t + 1 == ntm1) {  // panels t (in LDS) and t + 1 (in la1/lb1) remain
      compute(As[0], Bs[0]);
      la1.store(As[1], tid);
      lb1.store(Bs[1], tid);
      lds_barrier();
      compute_last(As[1], Bs[1], kn_last);
    } else {  // panel t is the last
      compute_last(As[0], Bs[0], kn_last);
    }
#undef IH_K_OF
  }

  // Accumulator layout of a 32x32 MFMA tile: register v of lane l holds
  // row 8*(v/4) + 4*(l/32) + (v%4), column l%32.
  if (p.splits > 1) {
    float* part = p.partial + (int64_t(slice) * p.splits + split) * p.M * p.N;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t row = m0 + wm + i * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
          const int64_t col = n0 + wn + j * 32 + l32;
          if (row < p.M && col < p.N) part[row * p.N + col] = acc[i][j][v];
        }
    return;
  }
  const float* C = p.use_table ? p.Ct[slice] : p.C;
  const float* R = p.R ? p.R + slice * p.sr : nullptr;
  float* Y = p.use_table ? p.Yt[slice] : p.Y + slice * p.sy;
  // One row of 32x32 MFMA tiles at a time: every operand load of the row
  // first, then the arithmetic (epilogue()'s order) and the stores. Loads
  // under a per-element bounds branch would cost one memory round trip per
  // element, so a tile at the matrix's edge (EDGE) loads from rows and
  // columns clamped into the matrix and bounds-checks only its stores. The
  // activation is a template argument of the store loop (one straight run of
  // stores per activation instead of a switch per element), and the uniform
  // tests sit outside the load loops, so each loop is one block of loads.
  const int64_t M = p.M, N = p.N;
  const bool full = m0 + BM <= M && n0 + BN <= N;
  const bool has_c = C != nullptr && p.beta != 0.0f;
  const int kind = has_c ? p.c_kind : INFERC_C_NONE;
  float cr[TN];
  const float c0 = kind == INFERC_C_SCALAR ? C[0] : 0.0f;
  if (kind == INFERC_C_ROW) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t col = n0 + wn + j * 32 + l32;
      cr[j] = C[col < N ? col : N - 1];
    }
  }
  // element (v, j) of the lane sits at row r0 + 8*(v/4) + v%4, column cb + 32j
  const int64_t r0 = m0 + wm + 4 * half, cb = n0 + wn + l32;
  auto finish = [&](auto act_tag, auto edge_tag) {
    constexpr int ACT = decltype(act_tag)::value;
    constexpr bool EDGE = decltype(edge_tag)::value;
    // a whole row of tiles per batch of loads; an edge tile one 32-column
    // block at a time (its clamped addresses cost registers)
    constexpr int JB = EDGE ? 1 : TN;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int64_t ri = r0 + i * 32;
#pragma unroll
      for (int j0 = 0; j0 < TN; j0 += JB) {
        float cx[JB][16], rx[JB][16];
        auto gather = [&](const float* X, int64_t ld, float (&dst)[JB][16]) {
          const float* xb = X + ri * ld + cb;
#pragma unroll
          for (int jj = 0; jj < JB; ++jj)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              if (EDGE) {
                const int64_t row = ri + 8 * (v >> 2) + (v & 3), col = cb + 32 * (j0 + jj);
                dst[jj][v] = X[(row < M ? row : M - 1) * ld + (col < N ? col : N - 1)];
              } else {
                dst[jj][v] = xb[(8 * (v >> 2) + (v & 3)) * ld + 32 * (j0 + jj)];
              }
            }
        };
        if (kind == INFERC_C_FULL) gather(C, p.ldc, cx);
        if (R != nullptr) gather(R, p.ldr, rx);
        float* yb = Y + ri * p.ldy + cb;
#pragma unroll
        for (int jj = 0; jj < JB; ++jj)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int j = j0 + jj;
            float x = p.alpha * acc[i][j][v];
            if (has_c) {
              const float c = kind == INFERC_C_ROW    ? cr[j]
                              : kind == INFERC_C_FULL ? cx[jj][v]
                                                      : c0;  // 0 for an unknown kind
              x = x + p.beta * c;
            }
            if (R != nullptr) x = x + rx[jj][v];
            const float y = apply_act(x, ACT);
            if (EDGE) {
              const int64_t row = ri + 8 * (v >> 2) + (v & 3), col = cb + 32 * j;
              if (row < M && col < N) Y[row * p.ldy + col] = y;
            } else {
              yb[(8 * (v >> 2) + (v & 3)) * p.ldy + 32 * j] = y;
            }
          }
      }
    }
  };
  auto by_edge = [&](auto act_tag) {
    if (full) finish(act_tag, std::false_type{});
    else finish(act_tag, std::true_type{});
  };
  switch (p.act) {
    case INFERC_ACT_GELU_ERF: by_edge(std::integral_constant<int, INFERC_ACT_GELU_ERF>{}); break;
    case INFERC_ACT_GELU_TANH: by_edge(std::integral_constant<int, INFERC_ACT_GELU_TANH>{}); break;
    case INFERC_ACT_RELU: by_edge(std::integral_constant<int, INFERC_ACT_RELU>{}); break;
    default: by_edge(std::integral_constant<int, INFERC_ACT_NONE>{}); break;
  }
}

// Sums the split-K partials in split order and applies the epilogue.
__global__ __launch_bounds__(kThreads) void splitk_reduce(GemmParams p) {
  const int slice = blockIdx.y;
  const int64_t MN = p.M * p.N;
  const float* part = p.partial + int64_t(slice) * p.splits * MN;
  const float* C = p.use_table ? p.Ct[slice] : p.C;
  const float* R = p.R ? p.R + slice * p.sr : nullptr;
  float* Y = p.use_table ? p.Yt[slice] : p.Y + slice * p.sy;
  for (int64_t e = int64_t(blockIdx.x) * kThreads + threadIdx.x; e < MN;
       e += int64_t(gridDim.x) * kThreads) {
    float s = 0.0f;
    for (int sp = 0; sp < p.splits; ++sp) s += part[sp * MN + e];
    const int64_t row = e / p.N, col = e % p.N;
    Y[row * p.ldy + col] = epilogue(p, C, R, s, row, col);
  }
}

// ---------------------------------------------------------------------------
// Small-M product (M up to a few hundred rows: the b=1 encoder, GPT-2
// prefill). One block per WM x WN output tile; its W waves split K between
// them, each wave running v_mfma_f32_16x16x4f32 on operands loaded straight
// from global memory into registers (no LDS staging: every operand element is
// used by exactly one wave of the block). The W partial tiles are summed
// through LDS in wave order (deterministic) and the epilogue is applied once.
// This replaces the split-K launch + reduce launch pair for these shapes.
//
// Operand layout (lane l, r = l%16, g = l/16). One k-group is 16 consecutive
// k; MFMA step e (0..3) of the group gives lane-group g the k index 4g+e:
//   A (row-major [M,K]):  float4 A[m0+16i+r][k0+4g .. k0+4g+3]
//   B (TB=0, [K,N]):      row k0+4g+e, CB consecutive columns starting at
//                         n0+CB*r (float4/float2); column block j of the
//                         MFMA takes column n0 + CB*r + j
//   B (TB=1, [N,K]):      float4 B[n0+16j+r][k0+4g .. k0+4g+3]
// Accumulator register v of lane l holds row 4*(l/16)+v, column l%16 of its
// 16x16 block.
// ---------------------------------------------------------------------------



template <int WM, int WN, bool TB>
struct KsFrag {
  static constexpr int RA = WM / 16, CB = WN / 16;
  float4 a[RA];
  float b[4][CB];  // b[e][j]: B operand of MFMA step e, column block j
  bool kin;        // this lane group's 4 k lie inside the wave's K range

  // Loads are unconditional, from addresses clamped into the operands. A row
  // of A past M only feeds output rows that are never stored, and a column
  // of B past N only output columns that are never stored, so those need no
  // masking. k past the wave's range is masked in mma(), where the value is
  // consumed: nothing touches a load result before the MFMA that needs it,
  // so the compiler keeps every ring slot in flight.
  __device__ __forceinline__ void load(const float* __restrict__ A, int64_t lda,
                                       const float* __restrict__ B, int64_t ldb, int64_t M,
                                       int64_t N, int64_t K, int64_t m0, int64_t n0, int64_t k0,
                                       int64_t ke, int r, int g) {
    const int64_t kq = k0 + 4 * g;  // first k of this lane group (a multiple of 4)
    kin = kq < ke;
    const int64_t kc = kq < K - 4 ? kq : K - 4;  // K % 4 == 0 and K >= 4
#pragma unroll
    for (int i = 0; i < RA; ++i) {
      const int64_t row = m0 + 16 * i + r;
      const int64_t rc = row < M ? row : M - 1;
      a[i] = *reinterpret_cast<const float4*>(A + rc * lda + kc);
    }

    if constexpr (TB) {
#pragma unroll
      for (int j = 0; j < CB; ++j) {
        const int64_t n = n0 + 16 * j + r;
        const int64_t nc = n < N ? n : N - 1;
        const float4 t = *reinterpret_cast<const float4*>(B + nc * ldb + kc);
        b[0][j] = t.x; b[1][j] = t.y; b[2][j] = t.z; b[3][j] = t.w;
      }
    } else {
      // N % 4 == 0, so a CB-wide vector at a multiple of CB is all in or all
      // out, and N - CB is a valid start.
      const int64_t n = n0 + CB * r;
      const int64_t nc = n < N ? n : N - CB;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float* src = B + (kc + e) * ldb + nc;
        if constexpr (CB == 4) {
          const float4 t = *reinterpret_cast<const float4*>(src);
          b[e][0] = t.x; b[e][1] = t.y; b[e][2] = t.z; b[e][3] = t.w;
        } else if constexpr (CB == 3) {
          // (the host takes 48-wide tiles only when N % 48 == 0)
          b[e][0] = src[0]; b[e][1] = src[1]; b[e][2] = src[2];
        } else if constexpr (CB == 2) {
          const float2 t = *reinterpret_cast<const float2*>(src);
          b[e][0] = t.x; b[e][1] = t.y;
        } else {
          b[e][0] = *src;
        }
      }
    }
  }

  // Both operands of a masked k are zeroed, so a non-finite value at the
  // clamped address cannot leak into the sum.
  __device__ __forceinline__ void mma(floatx4 (&acc)[RA][CB]) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float av[RA], bv[CB];
#pragma unroll
      for (int i = 0; i < RA; ++i) {
        const float x = e == 0 ? a[i].x : e == 1 ? a[i].y : e == 2 ? a[i].z : a[i].w;
        av[i] = kin ? x : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < CB; ++j) bv[j] = kin ? b[e][j] : 0.0f;
#pragma unroll
      for (int i = 0; i < RA; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
  }
};

// P is the register ring depth: k-groups in flight per wave.
template <int WM, int WN, int W, int P, bool TB, bool LNA, bool LNR>
__global__ __launch_bounds__(64 * W) void gemm_f32_ksplit(const float* __restrict__ A0,
                                                          const float* __restrict__ B0,
                                                          int lda_, int ldb_, int M_, int N_, int K_,
                                                          int kps_, int tiles_m_, int tiles_n_,
                                                          GemmParams p) {
  // The first ring needs only the leading scalar arguments, which the
  // hardware preloads into SGPRs at wave launch; the rest of p (epilogue,
  // LayerNorm terms, other slices) is read while those loads are in flight.
  const int64_t lda = lda_, ldb = ldb_, M = M_, N = N_, K = K_, kps = kps_;
  const int64_t tiles_m = tiles_m_, tiles_n = tiles_n_;
  constexpr int RA = WM / 16, CB = WN / 16;
  static_assert(W * WM * WN * 4 <= 65536, "partial tiles must fit the LDS of one block");
  __shared__ __attribute__((aligned(16))) float red[W * WM * WN];
  __shared__ float2 nstat[2][WM];  // LayerNorm (mean, rstd) of the tile's rows: A, R

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;

  // XCD-aware tile order: consecutive blocks go to different XCDs (round
  // robin over 8), so block b works on tile (b%8)*per + b/8. Each XCD then
  // holds a contiguous run of tiles, n-major, and the m-tiles that share a
  // B column panel read it through the same L2.
  const int64_t T = tiles_m * tiles_n, per = T / 8;
  const int64_t bid = blockIdx.x;
  const int64_t t = bid < 8 * per ? (bid % 8) * per + bid / 8 : bid;
  const int64_t m0 = (t % tiles_m) * WM, n0 = (t / tiles_m) * WN;

  const int slice = blockIdx.y;
  const float* A = A0;  // slice 0's operands
  const float* B = B0;
  if (slice != 0) {
    A = p.A + slice * p.sa;
    B = p.use_table ? p.Bt[slice] : p.B + slice * p.sb;
  }

  // Wave w owns K range [kb, ke); it runs `rings` rounds of P 16-deep
  // k-groups (the host sizes k_per_split so that rounds are mostly full;
  // groups past ke load zeros).
  const int64_t kb = int64_t(wave) * kps;
  const int64_t ke = kb + kps < K ? kb + kps : K;
  const int64_t rings = (kps + 16 * P - 1) / (16 * P);

  floatx4 acc[RA][CB];
#pragma unroll
  for (int i = 0; i < RA; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  KsFrag<WM, WN, TB> f[P];
  const bool has_k = kb < ke;
  // The operands' first ring (unconditional: a wave without a K range
  // loads clamped addresses that mma() masks, and no branch joins before
  // the loads below, whose waits are then counted exactly).
#pragma unroll
  for (int q = 0; q < P; ++q)
    f[q].load(A, lda, B, ldb, M, N, K, m0, n0, kb + 16 * q, ke, r, g);
  __builtin_amdgcn_sched_barrier(0);
  // LayerNorm statistics of the tile's rows (row 4 * wave + lane / 16 per
  // lane group), needed only by the epilogue: loaded behind the first ring
  // and merged after the K loop.
  static_assert(WM <= 4 * W, "a lane group per row of the tile");
  const int si = 4 * wave + (lane >> 4);
  const int64_t srow = m0 + si < M ? m0 + si : M - 1;
  RowStatLoads sla, slr;
  if (LNA) row_stats_load(sla, p.na_stats, srow, K / 16, lane);
  if (LNR) row_stats_load(slr, p.nr_stats, srow, N / 16, lane);
  // This thread's epilogue operands (elements e = tid + 64 W k of the tile),
  // fetched now so the epilogue after the K loop waits on no memory: C, R,
  // the column sums (LNA) and R's gamma and beta (LNR). The loads are
  // unconditional; an absent C or R reads A's first element instead, and
  // indices are clamped into the tile's valid rows and columns.
  constexpr int EPT = (WM * WN + 64 * W - 1) / (64 * W);
  const float* C = p.use_table ? p.Ct[slice] : p.C;
  const float* R = p.R ? p.R + slice * p.sr : nullptr;
  const bool has_c = C != nullptr && p.beta != 0.0f;
  float pc[EPT], pr[EPT], pcs[EPT], pg[EPT], pbt[EPT];
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int e = tid + 64 * W * k < WM * WN ? tid + 64 * W * k : 0;
    const int64_t row = m0 + e / WN < M ? m0 + e / WN : M - 1;
    const int64_t col = n0 + e % WN < N ? n0 + e % WN : N - 1;
    const int64_t ci = p.c_kind == INFERC_C_ROW ? col
                       : p.c_kind == INFERC_C_FULL ? row * p.ldc + col
                                                   : 0;
    pc[k] = (has_c ? C : A)[has_c ? ci : 0];
    pr[k] = (R ? R : A)[R ? row * p.ldr + col : 0];
    pg[k] = LNR ? p.nr_g[col] : 1.0f;
    pbt[k] = LNR ? p.nr_b[col] : 0.0f;
    pcs[k] = LNA ? p.na_c[slice][col] : 0.0f;
  }
  __builtin_amdgcn_sched_barrier(0);
  if (has_k) {
    for (int64_t ring = 1; ring < rings; ++ring) {
      const int64_t k_next = kb + 16 * P * ring;
#pragma unroll
      for (int q = 0; q < P; ++q) {
        // Slot by slot: the scheduler may not merge slots, so each MFMA
        // group waits only for its own loads and the refill of slot q goes
        // out as soon as slot q has been consumed.
        __builtin_amdgcn_sched_barrier(0);
        f[q].mma(acc);
        f[q].load(A, lda, B, ldb, M, N, K, m0, n0, k_next + 16 * q, ke, r, g);
      }
    }
#pragma unroll
    for (int q = 0; q < P; ++q) {
      __builtin_amdgcn_sched_barrier(0);
      f[q].mma(acc);
    }
  }

  // The rows' statistics, merged after the K loop, behind the barrier that
  // publishes the partial tiles.
  if constexpr (LNA) {
    const float2 v = row_stats_merge(sla, K / 16, p.na_eps, lane);
    if ((lane & 15) == 0 && si < WM) nstat[0][si] = v;
  }
  if constexpr (LNR) {
    const float2 v = row_stats_merge(slr, N / 16, p.nr_eps, lane);
    if ((lane & 15) == 0 && si < WM) nstat[1][si] = v;
  }
  // Partial tiles to LDS in [row][col] order of the block's output tile.
  float* mine = red + wave * (WM * WN);
#pragma unroll
  for (int i = 0; i < RA; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      const int col = TB ? 16 * j + r : CB * r + j;
#pragma unroll
      for (int v = 0; v < 4; ++v) mine[(16 * i + 4 * g + v) * WN + col] = acc[i][j][v];
    }
  __syncthreads();

  float* Y = p.use_table ? p.Yt[slice] : p.Y + slice * p.sy;
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int e = tid + 64 * W * k;
    if (e >= WM * WN) break;
    float s = red[e];
#pragma unroll
    for (int w = 1; w < W; ++w) s += red[w * (WM * WN) + e];
    const int64_t row = m0 + e / WN, col = n0 + e % WN;
    if (row < M && col < N) {
      if constexpr (LNA) {
        // A read through its LayerNorm with gamma folded into B:
        // rstd * (sum_k a_k B'_kn - mean * colsum_n); beta's share is in C
        const float2 st = nstat[0][e / WN];
        s = (s - st.x * pcs[k]) * st.y;
      }
      // the epilogue's order: alpha * acc + beta * C, + R, then act
      float v = p.alpha * s;
      if (has_c) v = v + p.beta * pc[k];
      if (R != nullptr) {
        float rv = pr[k];
        if constexpr (LNR) {
          // the residual row read through its LayerNorm
          const float2 st = nstat[1][e / WN];
          rv = fmaf((rv - st.x) * st.y, pg[k], pbt[k]);
        }
        v = v + rv;
      }
      const float y = apply_act(v, p.act);
      Y[row * p.ldy + col] = y;
      red[e] = y;  // only this thread reads red[e]
    }
  }
  if (p.st_out != nullptr) {
    // (mean, M2) of each row's 16-column chunks of Y, two-pass over the
    // stored values (N % 16 == 0, so a chunk is all in or all out)
    __syncthreads();
    constexpr int NCH = WN / 16;
    for (int idx = tid; idx < WM * NCH; idx += 64 * W) {
      const int i = idx / NCH, c = idx % NCH;
      const int64_t row = m0 + i, col0 = n0 + 16 * c;
      if (row >= M || col0 >= N) continue;
      const float* v = red + i * WN + 16 * c;
      float mean = 0.0f;
#pragma unroll
      for (int k = 0; k < 16; ++k) mean += v[k];
      mean *= 1.0f / 16.0f;
      float m2 = 0.0f;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const float d = v[k] - mean;
        m2 += d * d;
      }
      float* o = p.st_out + (int64_t(slice) * M * (N / 16) + row * (N / 16) + col0 / 16) * 2;
      o[0] = mean;
      o[1] = m2;
    }
  }
}

struct KsCfg { int wm, wn, w, p; };

// The small-M kernel takes its extents and leading dimensions as 32-bit
// kernel arguments.
inline bool ks_fits_i32(const GemmParams& p) {
  const int64_t lim = int64_t(1) << 31;
  return p.M < lim && p.N < lim && p.K < lim && p.lda < lim && p.ldb < lim;
}

// K per wave: whole rings of P k-groups, split as evenly as that allows.
inline int64_t ks_k_per_wave(int64_t K, int w, int depth) {
  return ceil_div(ceil_div(K, w), 16 * depth) * 16 * depth;
}

template <int WM, int WN, int W, int P>
void launch_ksplit(GemmParams p, int64_t slices, bool tb, hipStream_t s) {
  p.splits = 1;
  p.partial = nullptr;
  p.k_per_split = ks_k_per_wave(p.K, W, P);
  const int64_t tm = ceil_div(p.M, WM), tn = ceil_div(p.N, WN);
  const dim3 grid(static_cast<unsigned>(tm * tn), static_cast<unsigned>(slices));
  const dim3 block(64 * W);
  const bool lna = p.na_stats != nullptr, lnr = p.nr_stats != nullptr;
  const float* B0 = p.use_table ? p.Bt[0] : p.B;  // slice 0's B
  IH_REQUIRE(ks_fits_i32(p), INFERC_ERR_SHAPE, "gemm: small-M shape beyond 32-bit extents");
#define IH_KS(TB_, LNA_, LNR_)                                                           \
  if (tb == TB_ && lna == LNA_ && lnr == LNR_) {                                         \
    hipLaunchKernelGGL((gemm_f32_ksplit<WM, WN, W, P, TB_, LNA_, LNR_>), grid, block, 0, s, \
                       p.A, B0, int(p.lda), int(p.ldb), int(p.M), int(p.N), int(p.K),   \
                       int(p.k_per_split), int(tm), int(tn), p);                        \
    return;                                                                               \
  }
  IH_KS(false, false, false)
  IH_KS(false, true, false)
  IH_KS(false, false, true)
  IH_KS(false, true, true)
  IH_KS(true, false, false)
  IH_KS(true, true, false)
  IH_KS(true, false, true)
  IH_KS(true, true, true)
#undef IH_KS
}

// Three shapes cover the small-M products (measured on MI355X at M=32..256,
// N=768..3072, K=768..3072). 32x48 tiles with 8 waves and a 2-deep ring when
// N is a multiple of 48 and they give at least 3/4 as many blocks as CUs:
// the b=1 FFN-up (256 blocks, 10.9 us vs 13.3 us for 32x64) and QKV (192
// blocks, 10.4 us vs 12.7 us). Else 32x64 tiles with 8 waves when that
// gives at least half as many blocks as CUs. Else 16x32 tiles with 8 waves
// (out-proj, FFN-down, prefill; 14.9 us for the b=1 FFN-down), trading
// operand reuse for blocks to spread over the CUs, or 16x16 tiles when even
// those give at most a quarter as many blocks as CUs (M=32, N=768 prefill:
// 13.7 us vs 19.2 us).
KsCfg pick_ksplit(int64_t M, int64_t N, int64_t slices, int64_t cus) {
  const int64_t b48 = ceil_div(M, 32) * ceil_div(N, 48) * slices;
  if (N % 48 == 0 && 4 * b48 >= 3 * cus) return KsCfg{32, 48, 8, 2};
  const int64_t big_blocks = ceil_div(M, 32) * ceil_div(N, 64) * slices;
  if (2 * big_blocks >= cus) return KsCfg{32, 64, 8, 3};
  const int64_t b16 = ceil_div(M, 16) * ceil_div(N, 32) * slices;
  if (4 * b16 <= cus) return KsCfg{16, 16, 8, 2};
  return KsCfg{16, 32, 8, 2};
}

bool ksplit_supported(const GemmParams& p, int64_t slices, bool ta, bool vec, int64_t cus,
                      int64_t big_tiles) {
  // Operands need float4 rows (vec), A row-major; the shape must be one the
  // LDS-tiled kernel would have split over K (too few 128x128 tiles).
  return !ta && vec && big_tiles < cus && p.M <= 512 && p.K > 0 && slices < 65536 &&
         ks_fits_i32(p);
}

void run_ksplit(inferc_hip_ctx* ctx, GemmParams p, int64_t slices, bool tb) {
  const KsCfg c = pick_ksplit(p.M, p.N, slices, ctx->num_cus);
  if (c.wn == 48) launch_ksplit<32, 48, 8, 2>(p, slices, tb, ctx->stream);
  else if (c.wm == 32) launch_ksplit<32, 64, 8, 3>(p, slices, tb, ctx->stream);
  else if (c.wn == 16) launch_ksplit<16, 16, 8, 2>(p, slices, tb, ctx->stream);
  else launch_ksplit<16, 32, 8, 2>(p, slices, tb, ctx->stream);
  check_launch("gemm_f32_ksplit");
}

template <int BM, int BN, int BK, int WGM, int WGN, bool TA, bool TB, bool VEC>
void launch_cfg(const GemmParams& p, int64_t slices, hipStream_t s) {
  dim3 grid(unsigned(ceil_div(p.N, BN)), unsigned(ceil_div(p.M, BM)),
            unsigned(slices * p.splits));
  hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, BK, WGM, WGN, TA, TB, VEC>), grid, dim3(kThreads), 0,
                     s, p);
}

template <int BM, int BN, int BK, int WGM, int WGN>
void launch_tile(const GemmParams& p, int64_t slices, bool ta, bool tb, bool vec,
                 hipStream_t s) {
#define IH_GEMM_CASE(TA_, TB_, V_)                                                      \
  if (ta == TA_ && tb == TB_ && vec == V_)                                             \
    return launch_cfg<BM, BN, BK, WGM, WGN, TA_, TB_, V_>(p, slices, s);
  IH_GEMM_CASE(false, false, true)
  IH_GEMM_CASE(false, true, true)
  IH_GEMM_CASE(true, false, true)
  IH_GEMM_CASE(true, true, true)
  IH_GEMM_CASE(false, false, false)
  IH_GEMM_CASE(false, true, false)
  IH_GEMM_CASE(true, false, false)
  IH_GEMM_CASE(true, true, false)
#undef IH_GEMM_CASE
}

// Chooses the tile and the K split, then launches the product (and the
// split-K reduction when K was split). The split-K partials go to
// partial_buf (partial_bytes) when given, else to the context workspace.
void run(inferc_hip_ctx* ctx, GemmParams p, int64_t slices, bool ta, bool tb, bool vec,
         void* partial_buf = nullptr, size_t partial_bytes = 0) {
  struct Cfg { int bm, bn, bk; };
  const int64_t cus = ctx->num_cus;
  const Cfg big{128, 128, 16}, mid{128, 96, 32}, wide{128, 64, 16}, small{64, 64, 32};
  auto tiles = [&](const Cfg& c) { return ceil_div(p.M, c.bm) * ceil_div(p.N, c.bn) * slices; };
  if (ksplit_supported(p, slices, ta, vec, cus, tiles(big))) return run_ksplit(ctx, p, slices, tb);
  IH_REQUIRE(p.na_stats == nullptr && p.nr_stats == nullptr && p.st_out == nullptr,
             INFERC_ERR_UNSUPPORTED,
             "gemm: LayerNorm-on-read operands and row statistics need the small-M path");
  // the kernels address each operand with 32-bit element offsets
  auto extent = [](int64_t rows, int64_t ld, int64_t cols) {
    return rows > 0 && cols > 0 ? (rows - 1) * ld + cols : int64_t(0);
  };
  const int64_t ea = ta ? extent(p.K, p.lda, p.M) : extent(p.M, p.lda, p.K);
  const int64_t eb = tb ? extent(p.N, p.ldb, p.K) : extent(p.K, p.ldb, p.N);
  const int64_t lim32 = (int64_t(1) << 31) - 64;
  IH_REQUIRE(ea < lim32 && eb < lim32 && p.lda < lim32 && p.ldb < lim32 && p.K < lim32,
             INFERC_ERR_UNSUPPORTED, "gemm: an operand spans 2^31 elements or more");
  // 128x128 tiles hold 3 blocks per CU (164 VGPRs). Between one and three
  // tiles per CU a round leaves CUs idle, and 128x64 tiles balance better
  // (the b=32 fused QKV, M=4096 N=3x768 K=768: 175 us against 196 us).
  // 128x96 tiles, waves stacked 4x1 (32x96 each), for N a multiple of 96:
  // the encoder's N = 768 (256 tiles at M = 4096, one per CU), 3x768 and
  // 3072 (at b=32: out-proj 51 us, FFN-down 173-188 us, QKV 140 us, FFN-up
  // 182 us, against 61, 205, 153 and 194 us with the tiles below).
  Cfg c = (p.N % 96 == 0 && tiles(mid) >= cus) ? mid
          : tiles(big) >= 3 * cus             ? big
          : tiles(big) >= cus                 ? wide
                                              : small;
  int64_t splits = 1;
  if (c.bm == small.bm) {
    const int64_t t = tiles(small);
    // Split K until ~2 blocks per CU, keeping >= 4 K-panels per split.
    const int64_t max_splits = p.K / (4 * c.bk);
    while (splits < max_splits && t * splits < 2 * cus) splits *= 2;
    if (splits > max_splits) splits = max_splits;
    if (splits < 1) splits = 1;
  }
  p.splits = int(splits);
  p.k_per_split = splits > 1 ? ceil_div(ceil_div(p.K, splits), c.bk) * c.bk : (p.K > 0 ? p.K : 1);
  if (splits > 1) {
    const size_t need = size_t(slices) * size_t(splits) * size_t(p.M) * size_t(p.N) * sizeof(float);
    if (partial_buf) {
      IH_REQUIRE(need <= partial_bytes, INFERC_ERR_SHAPE,
                 "gemm: split-K partial sums need " + std::to_string(need) +
                     " bytes, more than the " + std::to_string(partial_bytes) +
                     "-byte scratch of the allocation-free entry point");
      p.partial = static_cast<float*>(partial_buf);
    } else {
      p.partial = static_cast<float*>(ctx->ws(need));
    }
  }
  if (c.bn == big.bn) launch_tile<128, 128, 16, 2, 2>(p, slices, ta, tb, vec, ctx->stream);
  else if (c.bn == mid.bn) launch_tile<128, 96, 32, 4, 1>(p, slices, ta, tb, vec, ctx->stream);
  else if (c.bm == wide.bm) launch_tile<128, 64, 16, 2, 2>(p, slices, ta, tb, vec, ctx->stream);
  else launch_tile<64, 64, 32, 2, 2>(p, slices, ta, tb, vec, ctx->stream);
  check_launch("gemm_f32_mfma");
  if (splits > 1) {
    const int64_t blocks = ceil_div(p.M * p.N, kThreads);
    dim3 grid(unsigned(blocks < 4096 ? blocks : 4096), unsigned(slices));
    hipLaunchKernelGGL(splitk_reduce, grid, dim3(kThreads), 0, ctx->stream, p);
    check_launch("splitk_reduce");
  }
}

void validate_common(const GemmArgs& a) {
  IH_REQUIRE(a.M >= 0 && a.N >= 0 && a.K >= 0, INFERC_ERR_SHAPE, "gemm: negative dimension");
  IH_REQUIRE(a.act >= INFERC_ACT_NONE && a.act <= INFERC_ACT_RELU, INFERC_ERR_ARG,
             "gemm: unknown activation");
  IH_REQUIRE(a.c_kind >= INFERC_C_NONE && a.c_kind <= INFERC_C_SCALAR, INFERC_ERR_ARG,
             "gemm: unknown C kind");
  IH_REQUIRE(a.batch >= 1, INFERC_ERR_SHAPE, "gemm: batch must be >= 1");
}

// Copies the LayerNorm-on-read operands and the statistics output into the
// launch parameters, checking the dimensions they need (D % 16 == 0).
void set_row_norms(GemmParams& p, int slices, const RowNorm& na, const RowNorm& nr,
                   float* st_out) {
  if (na.stats) {
    IH_REQUIRE(p.K % 16 == 0 && p.K <= 1024, INFERC_ERR_ARG,
               "gemm: LayerNorm of A needs K % 16 == 0, K <= 1024");
    for (int i = 0; i < slices; ++i) {
      IH_REQUIRE(na.colsum[i] != nullptr, INFERC_ERR_ARG, "gemm: LayerNorm of A needs column sums");
      p.na_c[i] = na.colsum[i];
    }
    p.na_stats = na.stats; p.na_eps = na.eps;
  }
  if (nr.stats) {
    IH_REQUIRE(nr.gamma && nr.beta && p.R && p.N % 16 == 0 && p.N <= 1024, INFERC_ERR_ARG,
               "gemm: LayerNorm of R needs R, gamma, beta and N % 16 == 0, N <= 1024");
    p.nr_stats = nr.stats; p.nr_g = nr.gamma; p.nr_b = nr.beta; p.nr_eps = nr.eps;
  }
  if (st_out) {
    IH_REQUIRE(p.N % 16 == 0, INFERC_ERR_ARG, "gemm: row statistics need N % 16 == 0");
    p.st_out = st_out;
  }
}

}  // namespace

bool gemm_small_m_path(const inferc_hip_ctx* ctx, int64_t M, int64_t N, int64_t K,
                       int64_t slices) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 4 || N % 4) return false;
  GemmParams p{};
  p.M = M; p.N = N; p.K = K;
  const int64_t big_tiles = ceil_div(M, 128) * ceil_div(N, 128) * slices;
  return ksplit_supported(p, slices, false, true, ctx->num_cus, big_tiles);
}

bool gemm_gemv_route(const GemmArgs& a) {
  const bool row_norms = a.norm_a.stats || a.norm_r.stats || a.stats_out;
  return !row_norms && a.M == 1 && a.batch == 1 && !a.trans_a && a.trans_b && a.alpha == 1.0f &&
         a.ldb == a.K && a.K > 0 && a.K <= 16384 &&
         (a.c_kind == INFERC_C_NONE || a.beta == 0.0f ||
          ((a.c_kind == INFERC_C_ROW || a.c_kind == INFERC_C_FULL) && a.beta == 1.0f));
}

void gemm(inferc_hip_ctx* ctx, const GemmArgs& a) {
  validate_common(a);
  if (a.M == 0 || a.N == 0) return;
  IH_REQUIRE(a.Y != nullptr, INFERC_ERR_ARG, "gemm: null output");
  IH_REQUIRE(a.K == 0 || (a.A != nullptr && a.B != nullptr), INFERC_ERR_ARG, "gemm: null operand");
  IH_REQUIRE(a.c_kind == INFERC_C_NONE || a.beta == 0.0f || a.C != nullptr, INFERC_ERR_ARG,
             "gemm: null C with non-zero beta");
  IH_REQUIRE(a.lda >= (a.trans_a ? a.M : a.K), INFERC_ERR_SHAPE, "gemm: lda too small");
  IH_REQUIRE(a.ldb >= (a.trans_b ? a.K : a.N), INFERC_ERR_SHAPE, "gemm: ldb too small");
  IH_REQUIRE(a.ldy >= a.N, INFERC_ERR_SHAPE, "gemm: ldy too small");
  IH_REQUIRE(a.R == nullptr || a.ldr >= a.N, INFERC_ERR_SHAPE, "gemm: ldr too small");
  IH_REQUIRE(a.c_kind != INFERC_C_FULL || a.ldc >= a.N, INFERC_ERR_SHAPE, "gemm: ldc too small");
  IH_REQUIRE(ih::ceil_div(a.M, 64) < 65536 && ih::ceil_div(a.N, 64) < (int64_t(1) << 30) &&
                 a.batch < 4096,
             INFERC_ERR_SHAPE, "gemm: problem too large for one launch grid");

  // One row times a [N,K] row-major B^T is the batch-1 GEMV, which the
  // reference also sends to sgemv (src/kernels/matmul.cc:207-216). The GEMV
  // applies bias, residual and act in the GEMM's order.
  if (gemm_gemv_route(a)) {
    // with one row, a full C is a row of N values like a bias
    const bool has_c = (a.c_kind == INFERC_C_ROW || a.c_kind == INFERC_C_FULL) && a.beta != 0.0f;
    const float* bias = has_c ? a.C : nullptr;
    gemv(ctx, a.N, a.K, a.B, a.A, a.gemv_ln_g, a.gemv_ln_b, a.gemv_ln_eps, bias, a.R, a.act, a.Y);
    return;
  }
  IH_REQUIRE(a.gemv_ln_g == nullptr, INFERC_ERR_UNSUPPORTED,
             "gemm: a LayerNorm of A needs the one-row GEMV route");
  const bool row_norms = a.norm_a.stats || a.norm_r.stats || a.stats_out;

  GemmParams p{};
  p.M = a.M; p.N = a.N; p.K = a.K;
  p.A = a.A; p.lda = a.lda; p.sa = a.stride_a;
  p.B = a.B; p.ldb = a.ldb; p.sb = a.stride_b;
  p.alpha = a.alpha; p.beta = a.beta;
  p.C = a.c_kind == INFERC_C_NONE ? nullptr : a.C; p.c_kind = a.c_kind; p.ldc = a.ldc;
  p.R = a.R; p.ldr = a.ldr; p.sr = a.stride_r;
  p.act = a.act;
  p.Y = a.Y; p.ldy = a.ldy; p.sy = a.stride_y;
  p.use_table = 0;
  if (row_norms) {
    IH_REQUIRE(a.batch == 1 && !a.trans_a && a.lda == a.K && a.ldy == a.N &&
                   (a.R == nullptr || a.ldr == a.N),
               INFERC_ERR_UNSUPPORTED, "gemm: LayerNorm-on-read needs dense unbatched rows");
    set_row_norms(p, 1, a.norm_a, a.norm_r, a.stats_out);
  }

  // float4 global loads need 16-byte aligned rows and a contiguous extent
  // that is a multiple of 4.
  const bool vec = aligned16(a.A) && aligned16(a.B) && a.lda % 4 == 0 && a.ldb % 4 == 0 &&
                   a.stride_a % 4 == 0 && a.stride_b % 4 == 0 &&
                   (a.trans_a ? a.M % 4 == 0 : a.K % 4 == 0) &&
                   (a.trans_b ? a.K % 4 == 0 : a.N % 4 == 0);
  run(ctx, p, a.batch, a.trans_a != 0, a.trans_b != 0, vec, a.partial_buf, a.partial_bytes);
}

void gemm_qkv(inferc_hip_ctx* ctx, int64_t M, int64_t K, int64_t N, const float* X,
              const float* const w[3], const float* const b[3], float* const y[3],
              int64_t ldy, const RowNorm* norm_a) {
  IH_REQUIRE(M >= 0 && K >= 0 && N >= 0, INFERC_ERR_SHAPE, "qkv: negative dimension");
  if (M == 0 || N == 0) return;
  IH_REQUIRE(X && w[0] && w[1] && w[2] && b[0] && b[1] && b[2] && y[0] && y[1] && y[2],
             INFERC_ERR_ARG, "qkv: null pointer");
  GemmParams p{};
  p.M = M; p.N = N; p.K = K;
  p.A = X; p.lda = K; p.sa = 0;
  p.ldb = N;
  p.alpha = 1.0f; p.beta = 1.0f;
  p.c_kind = INFERC_C_ROW;
  p.act = INFERC_ACT_NONE;
  p.ldy = ldy;
  p.use_table = 1;
  bool vec = aligned16(X) && K % 4 == 0 && N % 4 == 0;
  for (int i = 0; i < 3; ++i) {
    p.Bt[i] = w[i]; p.Ct[i] = b[i]; p.Yt[i] = y[i];
    vec = vec && aligned16(w[i]);
  }
  p.C = b[0];  // non-null marker; the table supplies the per-slice bias
  if (norm_a) set_row_norms(p, 3, *norm_a, RowNorm{}, nullptr);
  run(ctx, p, 3, false, false, vec);
}

// ---- scratch of the allocation-free entry point ----
// Split-K partial sums of inferc_hip_gemm_f32_noalloc: a file-scope device
// array, one copy per device, held until the process ends. In host code
// `scratch` names a host-side stand-in, never the device memory; kernels get
// the address looked up by init_gemm_scratch.
constexpr size_t kGemmScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kGemmScratchBytes];

namespace {
std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;  // device address of `scratch`, by device
}  // namespace

void init_gemm_scratch(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  IH_REQUIRE(device >= 0, INFERC_ERR_ARG, "gemm scratch: bad device");
  if (g_scratch_ptr.size() <= size_t(device)) g_scratch_ptr.resize(size_t(device) + 1, nullptr);
  if (g_scratch_ptr[size_t(device)]) return;
  void* ptr = nullptr;
  IH_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  IH_REQUIRE(ptr != nullptr, INFERC_ERR_HIP, "gemm scratch: no device address");
  g_scratch_ptr[size_t(device)] = ptr;
}

void* gemm_scratch(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  IH_REQUIRE(size_t(device) < g_scratch_ptr.size() && g_scratch_ptr[size_t(device)],
             INFERC_ERR_STATE, "gemm scratch: not set up for this device");
  return g_scratch_ptr[size_t(device)];
}

}  // namespace ih

extern "C" {

int inferc_hip_gemm_f32(inferc_hip_ctx* ctx, int trans_a, int trans_b, int64_t M, int64_t N,
                        int64_t K, float alpha, const float* A, int64_t lda, const float* B,
                        int64_t ldb, float beta, const float* C, int c_kind, int64_t ldc,
                        const float* R, int64_t ldr, int act, float* Y, int64_t ldy) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    ih::GemmArgs a;
    a.trans_a = trans_a; a.trans_b = trans_b;
    a.M = M; a.N = N; a.K = K; a.alpha = alpha; a.beta = beta;
    a.A = A; a.lda = lda; a.B = B; a.ldb = ldb;
    a.C = C; a.c_kind = c_kind; a.ldc = ldc;
    a.R = R; a.ldr = ldr; a.act = act; a.Y = Y; a.ldy = ldy;
    ih::gemm(ctx, a);
  });
}

int inferc_hip_gemm_f32_noalloc(inferc_hip_ctx* ctx, int trans_a, int trans_b, int64_t M,
                                int64_t N, int64_t K, float alpha, const float* A, int64_t lda,
                                const float* B, int64_t ldb, float beta, const float* C,
                                int c_kind, int64_t ldc, const float* R, int64_t ldr, int act,
                                float* Y, int64_t ldy) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    ih::GemmArgs a;
    a.trans_a = trans_a; a.trans_b = trans_b;
    a.M = M; a.N = N; a.K = K; a.alpha = alpha; a.beta = beta;
    a.A = A; a.lda = lda; a.B = B; a.ldb = ldb;
    a.C = C; a.c_kind = c_kind; a.ldc = ldc;
    a.R = R; a.ldr = ldr; a.act = act; a.Y = Y; a.ldy = ldy;
    a.partial_buf = ih::gemm_scratch(ctx->device);
    a.partial_bytes = ih::kGemmScratchBytes;
    ih::gemm(ctx, a);
  });
}

int inferc_hip_matmul_f32(inferc_hip_ctx* ctx, int64_t batch, int64_t M, int64_t N, int64_t K,
                          const float* A, int64_t stride_a, const float* B, int64_t stride_b,
                          float* Y) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    IH_REQUIRE(batch >= 0, INFERC_ERR_SHAPE, "matmul: negative batch");
    if (batch == 0) return;
    IH_REQUIRE(batch < 65536, INFERC_ERR_SHAPE, "matmul: batch too large for one launch");
    ih::GemmArgs a;
    a.M = M; a.N = N; a.K = K;
    a.A = A; a.lda = K; a.B = B; a.ldb = N; a.Y = Y; a.ldy = N;
    a.batch = batch; a.stride_a = stride_a; a.stride_b = stride_b; a.stride_y = M * N;
    ih::gemm(ctx, a);
  });
}

int inferc_hip_fused_matmul_add_gelu_f32(inferc_hip_ctx* ctx, int64_t M, int64_t N, int64_t K,
                                         const float* X, const float* W, const float* bias,
                                         float* Y) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    IH_REQUIRE(bias != nullptr, INFERC_ERR_ARG, "fused_matmul_add_gelu: null bias");
    ih::GemmArgs a;
    a.M = M; a.N = N; a.K = K;
    a.A = X; a.lda = K; a.B = W; a.ldb = N;
    a.beta = 1.0f; a.C = bias; a.c_kind = INFERC_C_ROW;
    a.act = INFERC_ACT_GELU_ERF;
    a.Y = Y; a.ldy = N;
    ih::gemm(ctx, a);
  });
}

int inferc_hip_fused_qkv_f32(inferc_hip_ctx* ctx, int64_t M, int64_t K, int64_t N,
                             const float* X, const float* wq, const float* bq, const float* wk,
                             const float* bk, const float* wv, const float* bv, float* q,
                             float* k, float* v) {
  return ih::guard([&] {
    ih::check_ctx(ctx)->make_current();
    const float* w[3] = {wq, wk, wv};
    const float* b[3] = {bq, bk, bv};
    float* y[3] = {q, k, v};
    ih::gemm_qkv(ctx, M, K, N, X, w, b, y, N);
  });
}

}  // extern "C"
