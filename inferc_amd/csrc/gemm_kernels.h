// The fp32 GEMM kernels of gemm.hip and their launchers, shared by the
// translation units that instantiate them: gemm.hip (the small-M kernel
// and the launch logic) and the compiles of gemm_tile.hip (the LDS-tiled
// kernel, one tile form and A orientation each), so that the library's
// kernels compile in parallel. Internal to the library.
#pragma once

#include <type_traits>

#include "common.h"

namespace ih {

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
  // small-M path with K also split over blocks (gridDim.z > 1): each tile's
  // per-block partial sums ([slices][tiles][z][WM*WN] in partial) and its
  // arrival counter (zero between launches)
  unsigned* ks_count;
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

// The LDS-tiled kernel's launcher for one tile form and one A orientation
// (its B orientations and aligned/unaligned forms inside). FORM 0: 128x128
// tiles, BK 16, 2x2 waves; 1: 128x96, BK 32, 4x1; 2: 128x64, BK 16, 2x2;
// 3: 64x64, BK 32, 2x2. Each (FORM, TA) is instantiated by its own compile
// of gemm_tile.hip (inferc_amd/build.py), so that the forms compile in
// parallel.
template <int FORM, bool TA>
void gemm_launch_tile(const GemmParams& p, int64_t slices, bool tb, bool vec, hipStream_t s);
extern template void gemm_launch_tile<0, false>(const GemmParams&, int64_t, bool, bool, hipStream_t);
extern template void gemm_launch_tile<0, true>(const GemmParams&, int64_t, bool, bool, hipStream_t);
extern template void gemm_launch_tile<1, false>(const GemmParams&, int64_t, bool, bool, hipStream_t);
extern template void gemm_launch_tile<1, true>(const GemmParams&, int64_t, bool, bool, hipStream_t);
extern template void gemm_launch_tile<2, false>(const GemmParams&, int64_t, bool, bool, hipStream_t);
extern template void gemm_launch_tile<2, true>(const GemmParams&, int64_t, bool, bool, hipStream_t);
extern template void gemm_launch_tile<3, false>(const GemmParams&, int64_t, bool, bool, hipStream_t);
extern template void gemm_launch_tile<3, true>(const GemmParams&, int64_t, bool, bool, hipStream_t);

namespace {

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
// With gridDim.z = Z > 1 the K range is also split over Z blocks per tile
// (kpb_ each). Every block stores its partial tile, and the last of the Z to
// arrive (an atomic counter per tile) sums the Z partials in z order, so the
// result does not depend on arrival order, and runs the epilogue; it also
// sets the counter back to zero for the next launch.
template <int WM, int WN, int W, int P, bool TB, bool LNA, bool LNR>
__global__ __launch_bounds__(64 * W) void gemm_f32_ksplit(const float* __restrict__ A0,
                                                          const float* __restrict__ B0,
                                                          int lda_, int ldb_, int M_, int N_, int K_,
                                                          int kps_, int tiles_m_, int tiles_n_,
                                                          int kpb_, GemmParams p) {
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

  // Wave w owns K range [kb, ke) of the block's [kbb, keb); it runs `rings`
  // rounds of P 16-deep k-groups (the host sizes k_per_split so that rounds
  // are mostly full; groups past ke load zeros).
  const int64_t kbb = int64_t(blockIdx.z) * kpb_;
  const int64_t keb = kbb + kpb_ < K ? kbb + kpb_ : K;
  const int64_t kb = kbb + int64_t(wave) * kps;
  const int64_t ke = kb + kps < keb ? kb + kps : keb;
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

  float sum[EPT];
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int e = tid + 64 * W * k;
    float s = 0.0f;
    if (e < WM * WN) {
      s = red[e];
#pragma unroll
      for (int w = 1; w < W; ++w) s += red[w * (WM * WN) + e];
    }
    sum[k] = s;
  }
  if (gridDim.z > 1) {
    const int Z = gridDim.z;
    __shared__ int last;
    unsigned* cnt = p.ks_count + int64_t(slice) * T + t;
    float* part = p.partial + (int64_t(slice) * T + t) * Z * (WM * WN);
    // The partials are agent-scope atomic stores and loads, which write
    // through to and read from the device-coherent level, so no fence has
    // to write back or invalidate a whole L2 (a device-scope fence per block
    // made these launches 10x slower). Each thread waits for its stores to
    // complete before the barrier that precedes the count.
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int e = tid + 64 * W * k;
      if (e < WM * WN)
        __hip_atomic_store(part + int64_t(blockIdx.z) * (WM * WN) + e, sum[k], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
      last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             unsigned(Z - 1);
    __syncthreads();
    if (!last) return;
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int e = tid + 64 * W * k;
      if (e >= WM * WN) continue;
      float s = __hip_atomic_load(part + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      for (int z = 1; z < Z; ++z)
        s += __hip_atomic_load(part + int64_t(z) * (WM * WN) + e, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      sum[k] = s;
    }
    if (tid == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  float* Y = p.use_table ? p.Yt[slice] : p.Y + slice * p.sy;
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int e = tid + 64 * W * k;
    if (e >= WM * WN) break;
    float s = sum[k];
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

struct KsCfg { int wm, wn, w, p, z; };  // z: blocks sharing one tile's K

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

// K per block when K is split over z blocks per tile: a multiple of 16.
inline int64_t ks_k_per_block(int64_t K, int z) { return ceil_div(ceil_div(K, z), 16) * 16; }

// Launches the small-M kernel; z > 1 also splits K over z blocks per tile,
// which needs p.partial (z * tiles * slices * WM * WN floats) and p.ks_count
// (tiles * slices counters, zero).
template <int WM, int WN, int W, int P>
void launch_ksplit(GemmParams p, int64_t slices, bool tb, int z, hipStream_t s) {
  p.splits = 1;
  if (z <= 1) {
    z = 1;
    p.partial = nullptr;
    p.ks_count = nullptr;
  }
  const int64_t kpb = z > 1 ? ks_k_per_block(p.K, z) : p.K;
  p.k_per_split = ks_k_per_wave(kpb, W, P);
  const int64_t tm = ceil_div(p.M, WM), tn = ceil_div(p.N, WN);
  const dim3 grid(static_cast<unsigned>(tm * tn), static_cast<unsigned>(slices),
                  static_cast<unsigned>(z));
  const dim3 block(64 * W);
  const bool lna = p.na_stats != nullptr, lnr = p.nr_stats != nullptr;
  const float* B0 = p.use_table ? p.Bt[0] : p.B;  // slice 0's B
  IH_REQUIRE(ks_fits_i32(p), INFERC_ERR_SHAPE, "gemm: small-M shape beyond 32-bit extents");
#define IH_KS(TB_, LNA_, LNR_)                                                           \
  if (tb == TB_ && lna == LNA_ && lnr == LNR_) {                                         \
    hipLaunchKernelGGL((gemm_f32_ksplit<WM, WN, W, P, TB_, LNA_, LNR_>), grid, block, 0, s, \
                       p.A, B0, int(p.lda), int(p.ldb), int(p.M), int(p.N), int(p.K),   \
                       int(p.k_per_split), int(tm), int(tn), int(kpb), p);              \
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

template <int BM, int BN, int BK, int WGM, int WGN, bool TA, bool TB, bool VEC>
void launch_cfg(const GemmParams& p, int64_t slices, hipStream_t s) {
  dim3 grid(unsigned(ceil_div(p.N, BN)), unsigned(ceil_div(p.M, BM)),
            unsigned(slices * p.splits));
  hipLaunchKernelGGL((gemm_f32_mfma<BM, BN, BK, WGM, WGN, TA, TB, VEC>), grid, dim3(kThreads), 0,
                     s, p);
}

template <int BM, int BN, int BK, int WGM, int WGN, bool TA>
void launch_tile(const GemmParams& p, int64_t slices, bool tb, bool vec, hipStream_t s) {
  if (tb && vec) return launch_cfg<BM, BN, BK, WGM, WGN, TA, true, true>(p, slices, s);
  if (!tb && vec) return launch_cfg<BM, BN, BK, WGM, WGN, TA, false, true>(p, slices, s);
  if (tb) return launch_cfg<BM, BN, BK, WGM, WGN, TA, true, false>(p, slices, s);
  return launch_cfg<BM, BN, BK, WGM, WGN, TA, false, false>(p, slices, s);
}

}  // namespace
}  // namespace ih
