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
// and the partial tiles are summed through LDS in the same launch (for a long
// K also over two blocks per tile, the later of which sums both partials in a
// fixed order). Other
// shapes run the 64x64 kernel with K split over blocks; partial sums land in
// the context workspace, and a second kernel reduces them in fixed order
// (deterministic) and applies the epilogue.
#include <mutex>
#include <type_traits>
#include <string>
#include <vector>

#include "gemm_kernels.h"

namespace ih {
namespace {

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
//
// With K >= 2048, where 16x32 tiles leave CUs idle, K is also split over two
// blocks of 16x48 tiles (16 waves each) when that gives between one and two
// blocks per CU: the b=1 FFN-down (M=128, N=768, K=3072) takes 11.3 us on
// 256 blocks against 13.3 us on 192 (16x32, K whole; 8 waves per 16x48
// block: 11.7 us); splitting out-proj, FFN-up or QKV (K=768) the same way
// was slower in every form measured.
KsCfg pick_ksplit(int64_t M, int64_t N, int64_t K, int64_t slices, int64_t cus, bool split_k) {
  const int64_t b48 = ceil_div(M, 32) * ceil_div(N, 48) * slices;
  if (N % 48 == 0 && 4 * b48 >= 3 * cus) return KsCfg{32, 48, 8, 2, 1};
  const int64_t big_blocks = ceil_div(M, 32) * ceil_div(N, 64) * slices;
  if (2 * big_blocks >= cus) return KsCfg{32, 64, 8, 3, 1};
  const int64_t b16 = ceil_div(M, 16) * ceil_div(N, 32) * slices;
  if (4 * b16 <= cus) return KsCfg{16, 16, 8, 2, 1};
  const int64_t z48 = 2 * ceil_div(M, 16) * (N / 48) * slices;
  if (split_k && K >= 2048 && N % 48 == 0 && z48 >= cus && z48 <= 2 * cus &&
      z48 / 2 <= inferc_hip_ctx::kKsCounters)
    return KsCfg{16, 48, 16, 2, 2};
  return KsCfg{16, 32, 8, 2, 1};
}

bool ksplit_supported(const GemmParams& p, int64_t slices, bool ta, bool vec, int64_t cus,
                      int64_t big_tiles) {
  // Operands need float4 rows (vec), A row-major; the shape must be one the
  // LDS-tiled kernel would have split over K (too few 128x128 tiles).
  return !ta && vec && big_tiles < cus && p.M <= 512 && p.K > 0 && slices < 65536 &&
         ks_fits_i32(p);
}

// split_k: K may also be split over blocks (not for the allocation-free
// entry point, whose scratch holds no counters).
void run_ksplit(inferc_hip_ctx* ctx, GemmParams p, int64_t slices, bool tb, bool split_k) {
  const KsCfg c = pick_ksplit(p.M, p.N, p.K, slices, ctx->num_cus, split_k);
  if (c.z > 1) {
    const int64_t tiles = ceil_div(p.M, c.wm) * ceil_div(p.N, c.wn) * slices;
    p.partial = static_cast<float*>(
        ctx->ws(size_t(tiles) * size_t(c.z) * size_t(c.wm) * size_t(c.wn) * sizeof(float)));
    p.ks_count = ctx->ks_count;
  }
  if (c.wm == 16 && c.wn == 48) launch_ksplit<16, 48, 16, 2>(p, slices, tb, c.z, ctx->stream);
  else if (c.wn == 48) launch_ksplit<32, 48, 8, 2>(p, slices, tb, c.z, ctx->stream);
  else if (c.wm == 32) launch_ksplit<32, 64, 8, 3>(p, slices, tb, c.z, ctx->stream);
  else if (c.wn == 16) launch_ksplit<16, 16, 8, 2>(p, slices, tb, c.z, ctx->stream);
  else launch_ksplit<16, 32, 8, 2>(p, slices, tb, c.z, ctx->stream);
  check_launch("gemm_f32_ksplit");
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
  if (ksplit_supported(p, slices, ta, vec, cus, tiles(big)))
    return run_ksplit(ctx, p, slices, tb, partial_buf == nullptr);
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
  auto go = [&](auto form) {
    constexpr int F = decltype(form)::value;
    if (ta)
      gemm_launch_tile<F, true>(p, slices, tb, vec, ctx->stream);
    else
      gemm_launch_tile<F, false>(p, slices, tb, vec, ctx->stream);
  };
  if (c.bn == big.bn) go(std::integral_constant<int, 0>{});
  else if (c.bn == mid.bn) go(std::integral_constant<int, 1>{});
  else if (c.bm == wide.bm) go(std::integral_constant<int, 2>{});
  else go(std::integral_constant<int, 3>{});
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

bool gemm_gemv_route(const inferc_hip_ctx* ctx, const GemmArgs& a) {
  const bool row_norms = a.norm_a.stats || a.norm_r.stats || a.stats_out;
  // (no context: a device-free planning run, which assumes the default)
  return (ctx == nullptr || ctx->gemv_decode) && !row_norms && a.M == 1 && a.batch == 1 && !a.trans_a && a.trans_b && a.alpha == 1.0f &&
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
  if (gemm_gemv_route(ctx, a)) {
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
