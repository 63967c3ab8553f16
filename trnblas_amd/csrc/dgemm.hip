// fp64 GEMM for gfx950 on v_mfma_f64_16x16x4_f64: the products of the metric
// stage (trnblas/level3.py:332-380; the reference's device route is
// torch.linalg.cholesky + a blocked trsm whose updates are GEMMs,
// trnblas/nki/dispatch.py:1740-1799, :1854-1881). Here those are the panels
// and trailing updates of the blocked Cholesky, the block products of the
// triangular inverse, and trsm's block solves and updates, all in fp64.
//
// D = alpha op(A) op(B) + beta C, batched by strides; D may alias C (each
// element is read and written by the same lane). Two options shape the tile
// walk for triangular work:
//  * lower: only tiles on or below the diagonal of a square D are launched,
//    and only elements m >= n are written (a trailing update of a Cholesky);
//  * tri: an operand is triangular, so each tile's k range skips its zero
//    blocks (A lower: k < m0 + BM; A upper: k >= m0; B lower: k >= n0; B
//    upper: k < n0 + BN). The other triangle of such an operand must hold
//    zeros inside the k range a tile still reads (its diagonal blocks).
//
// Layout: a 256-thread workgroup (4 wave64s, 2 x 2) owns a BM x BM tile of D
// (BM 128, or 64 / 32 for launches with fewer 128-tiles than CUs); each wave a
// BM/2 square as 16 x 16 MFMA blocks with fp64 accumulators. k-tiles of BK
// values (16 for BM 128, 64 for BM 64: either way 64 MFMAs per wave per
// k-tile) move by LDS DMA (buffer_load_dwordx4 ... lds) into two LDS stages;
// after the barrier that publishes k-tile t each wave reads all its
// fragments of t, then issues the DMA of t + 1 into the other stage, then
// runs its MFMAs (the compiler makes an LDS read that follows an
// outstanding LDS DMA wait for it, so no read follows the DMA inside a
// k-tile; a deeper pipeline with more stages got such waits anyway).
//  * K-contiguous panel (BM rows of 8 BK bytes): within each 128-byte
//    segment of row r, 16-byte group q sits in slot q ^ ((r >> 1) & 7); a
//    1 KiB DMA block is whole rows. Lane group g = lane / 16 reads k = 4 g ..
//    4 g + 3 of each 16-deep sub-tile of its row (two 16-byte reads): MFMA q
//    (0..3) takes element q, so MFMA q multiplies k = 4 g + q for lane group
//    g, the same permutation of k for both operands.
//  * M/N-contiguous panel (BK rows k of BM values): group q of row k in slot
//    q ^ (8 ((k >> 2) & 1)), which puts the rows k and k + 4 that two lane
//    groups read together on different halves of the banks; a DMA block is
//    1 (BM 128), 2 (BM 64) or 4 (BM 32) rows. A fragment is four 8-byte
//    column reads.
// Ragged M / N edges read zeros (an offset past the buffer's records);
// K and each operand's contiguous extent are even (16-byte groups are
// wholly inside or outside the matrix), checked by the entry point.
//
// MFMA 16x16x4 f64 lane layout (measured with an in-bounds probe): A[i][k]
// from lane i + 16 k, B[k][j] from lane j + 16 k, D[i][j] in lane
// j + 16 (i % 4), register i / 4 (unlike the fp32 16x16 layouts, whose
// registers hold consecutive rows).
#include "common.hpp"

namespace trnblas {

typedef double f64x4 __attribute__((ext_vector_type(4)));

struct DgemmArgs {
  int M, N, K;
  double alpha, beta;
  const double* A;
  int64_t lda, sA;
  const double* B;
  int64_t ldb, sB;
  const double* C;
  int64_t ldc, sC;
  double* D;
  int64_t ldd, sD;
  int batch;
  int tiles_m, tiles_n;  // tile grid of one batch entry
  int ntiles;            // tiles of the launch
  int lower;             // launch the lower-triangle tiles only, write m >= n
  int tri;               // TRNBLAS_TRI_* bits
};

constexpr uint32_t kDOob = 0x80000000u;  // offsets >= this read as zero
constexpr uint32_t kDRecords = 0x7ffffff0u;

__device__ __forceinline__ void dma16(const void* base, void* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)kDRecords,
                                        0x00020000),
      (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

// Lower-triangle tile t -> (tm, tn), tm >= tn, row by row.
__device__ __forceinline__ void dtri_tile(int t, int& tm, int& tn) {
  int r = (int)((sqrtf(8.0f * (float)t + 1.0f) - 1.0f) * 0.5f);
  while (r * (r + 1) / 2 > t) --r;
  while ((r + 1) * (r + 2) / 2 <= t) ++r;
  tm = r;
  tn = t - r * (r + 1) / 2;
}

// A BM x BM output tile, k-tiles of BK values (BK / 2 16-byte groups per
// K-contiguous row) in two LDS stages: 64 KiB for every shape (BM 128: BK 16;
// BM 64: BK 32; BM 32: BK 64), so two workgroups share a CU, or one shares
// it with a 90 KiB diagonal-block kernel of a concurrent stream. Each wave
// has 64 (BM 128), 32 (BM 64) or 16 (BM 32) MFMAs per k-tile behind the
// next k-tile's DMA.
template <int BM, int BK, bool AKC, bool BKC>
__global__ __launch_bounds__(256, 2) void dgemm_kernel(DgemmArgs g) {
  constexpr int WT = BM / 2;        // wave tile
  constexpr int F = WT / 16;        // 16 x 16 blocks per wave side
  constexpr int PANEL = BM * BK;    // doubles per operand panel
  constexpr int KG = BK / 2;        // 16-byte groups in a K-contiguous row
  constexpr int KRB = 64 / KG;      // K-contiguous rows per 1 KiB DMA block
  constexpr int MG = BM / 2;        // 16-byte groups in an M/N-contiguous row
  constexpr int RPB = 64 / MG;      // M/N-contiguous rows per 1 KiB DMA block
  constexpr int NBLK = PANEL / 128 / 4;  // DMA blocks per wave per panel
  constexpr int KS = BK / 16;       // 16-deep sub-tiles per k-tile
  static_assert(KG >= 8 && NBLK >= 1, "tile");
  __shared__ __attribute__((aligned(16))) double st0[2 * PANEL];
  __shared__ __attribute__((aligned(16))) double st1[2 * PANEL];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int lane = tid & 63;
  asm volatile("" : "+v"(lane));
  const int wm0 = (wave >> 1) * WT, wn0 = (wave & 1) * WT;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  int bat, tm, tn;
  if (g.lower) {
    bat = 0;
    dtri_tile(t, tm, tn);
  } else {
    const int per = g.tiles_m * g.tiles_n;
    bat = t / per;
    grouped_tile(t - bat * per, g.tiles_m, g.tiles_n, 8, tm, tn);
  }
  const int m0 = tm * BM, n0 = tn * BM;
  const int M = g.M, N = g.N, K = g.K;
  int kbeg = 0, kend = K;
  if (g.tri & TRNBLAS_TRI_A_LOWER) kend = min(kend, m0 + BM);
  if (g.tri & TRNBLAS_TRI_A_UPPER) kbeg = max(kbeg, m0);
  if (g.tri & TRNBLAS_TRI_B_LOWER) kbeg = max(kbeg, n0);
  if (g.tri & TRNBLAS_TRI_B_UPPER) kend = min(kend, n0 + BM);
  kbeg = kbeg / BK * BK;
  const int kb0 = kbeg / BK, kb1 = kend > kbeg ? (kend + BK - 1) / BK : kb0;
  const double* A = g.A + bat * g.sA;
  const double* B = g.B + bat * g.sB;

  // K-contiguous rows: group q in slot (q & ~7) | ((q & 7) ^ ((r >> 1) & 7)),
  // i.e. each 128-byte segment of a row swizzled by the row (an involution)
  auto kslot = [](int q, int r) __attribute__((always_inline)) {
    return (q & ~7) | ((q & 7) ^ ((r >> 1) & 7));
  };
  // DMA of k-tile kt into stage st (A panel, then B panel); wave w fills
  // blocks NBLK w .. NBLK w + NBLK - 1 of each panel.
  auto dma = [&](double* st, int kt) __attribute__((always_inline)) {
    const int k0 = kt * BK;
    const double* pa = AKC ? A + (int64_t)m0 * g.lda + k0 : A + (int64_t)k0 * g.lda + m0;
    const double* pb = BKC ? B + (int64_t)n0 * g.ldb + k0 : B + (int64_t)k0 * g.ldb + n0;
    const int ra = AKC ? M - m0 : K - k0, ca = AKC ? K - k0 : M - m0;
    const int rb = BKC ? N - n0 : K - k0, cb = BKC ? K - k0 : N - n0;
    auto geo = [&](bool kc, int u, int& row, int& grp) __attribute__((always_inline)) {
      const int b = NBLK * wave + u;
      if (kc) {
        row = KRB * b + lane / KG;
        grp = kslot(lane % KG, row);
      } else {
        row = RPB * b + lane / MG;
        grp = (lane % MG) ^ (8 * ((row >> 2) & 1));
      }
    };
#pragma unroll
    for (int u = 0; u < NBLK; ++u) {
      int rw, gp;
      geo(AKC, u, rw, gp);
      const bool ok = rw < ra && 2 * gp < ca;
      const uint32_t v = ok ? (uint32_t)((int64_t)rw * g.lda * 8 + 16 * gp) : kDOob;
      dma16(pa, st + (NBLK * wave + u) * 128, v);
    }
#pragma unroll
    for (int u = 0; u < NBLK; ++u) {
      int rw, gp;
      geo(BKC, u, rw, gp);
      const bool ok = rw < rb && 2 * gp < cb;
      const uint32_t v = ok ? (uint32_t)((int64_t)rw * g.ldb * 8 + 16 * gp) : kDOob;
      dma16(pb, st + PANEL + (NBLK * wave + u) * 128, v);
    }
  };

  // The lane's four k values kk + 4 g .. kk + 4 g + 3 of row / column r.
  const int lg = lane >> 4;
  auto frag = [&](const double* p, bool kc, int r, int kk, double (&v)[4])
                  __attribute__((always_inline)) {
    if (kc) {
      const double* row = p + r * BK;
      const int q = kk / 2 + 2 * lg;
      const double2 x0 = *reinterpret_cast<const double2*>(row + 2 * kslot(q, r));
      const double2 x1 = *reinterpret_cast<const double2*>(row + 2 * kslot(q + 1, r));
      v[0] = x0.x;
      v[1] = x0.y;
      v[2] = x1.x;
      v[3] = x1.y;
    } else {
      const int col = 2 * ((r >> 1) ^ (8 * (lg & 1))) + (r & 1);
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = p[(kk + 4 * lg + q) * BM + col];
    }
  };

  f64x4 acc[F][F];
#pragma unroll
  for (int i = 0; i < F; ++i)
#pragma unroll
    for (int j = 0; j < F; ++j) acc[i][j] = f64x4{0.0, 0.0, 0.0, 0.0};

  // Waves of a diagonal tile (lower) whose block lies above the diagonal
  // move their share of the panels but run no MFMAs. (For the other cases
  // `busy` is an opaque runtime condition: as a branch it keeps the
  // fragment reads, the DMA and the MFMAs of a k-tile in separate blocks.)
  int on = 1;
  asm volatile("" : "+s"(on));
  const bool busy = g.lower ? !(tm == tn && wn0 > wm0) : on != 0;
  // One k-tile from stage `cur`: every fragment is read before the DMA of
  // k-tile `next` (< 0: none) into the other stage issues; the MFMAs run
  // behind that DMA.
  auto step = [&](const double* cur, double* oth, int next) __attribute__((always_inline)) {
    double fa[KS][F][4], fb[KS][F][4];
    if (busy) {
#pragma unroll
      for (int c = 0; c < KS; ++c) {
#pragma unroll
        for (int i = 0; i < F; ++i) frag(cur, AKC, wm0 + 16 * i + (lane & 15), 16 * c, fa[c][i]);
#pragma unroll
        for (int j = 0; j < F; ++j)
          frag(cur + PANEL, BKC, wn0 + 16 * j + (lane & 15), 16 * c, fb[c][j]);
      }
    }
    if (next >= 0) dma(oth, next);
    if (busy) {
#pragma unroll
      for (int c = 0; c < KS; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int i = 0; i < F; ++i)
#pragma unroll
            for (int j = 0; j < F; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(fa[c][i][q], fb[c][j][q], acc[i][j],
                                                               0, 0, 0);
    }
  };

  if (kb1 > kb0) dma(st0, kb0);
  for (int kt = kb0; kt < kb1; kt += 2) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA of k-tile kt has landed
    __syncthreads();                // every wave's has; every read of st1 is done
    step(st0, st1, kt + 1 < kb1 ? kt + 1 : -1);
    if (kt + 1 >= kb1) break;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    step(st1, st0, kt + 2 < kb1 ? kt + 2 : -1);
  }

  // epilogue: D = alpha acc + beta C
  const double* C = g.C ? g.C + bat * g.sC : nullptr;
  double* D = g.D + bat * g.sD;
#pragma unroll
  for (int i = 0; i < F; ++i)
#pragma unroll
    for (int j = 0; j < F; ++j) {
      const int n = n0 + wn0 + 16 * j + (lane & 15);
      const int mb = m0 + wm0 + 16 * i + lg;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = mb + 4 * e;
        if (m < M && n < N && (!g.lower || n <= m)) {
          double v = g.alpha * acc[i][j][e];
          if (g.beta != 0.0) v = fma(g.beta, C[(int64_t)m * g.ldc + n], v);
          D[(int64_t)m * g.ldd + n] = v;
        }
      }
    }
}

template <int BM, bool AKC, bool BKC>
static int dlaunch(DgemmArgs g, hipStream_t s) {
  g.tiles_m = (g.M + BM - 1) / BM;
  g.tiles_n = (g.N + BM - 1) / BM;
  g.ntiles = g.lower ? g.tiles_m * (g.tiles_m + 1) / 2 : g.tiles_m * g.tiles_n * g.batch;
  constexpr int BK = BM == 128 ? 16 : BM == 64 ? 32 : 64;
  hipLaunchKernelGGL((dgemm_kernel<BM, BK, AKC, BKC>), dim3(g.ntiles), dim3(256), 0, s, g);
  return check_launch("trnblas_hip_dgemm");
}

template <int BM>
static int dlaunch_layout(const DgemmArgs& g, bool akc, bool bkc, hipStream_t s) {
  if (akc && bkc) return dlaunch<BM, true, true>(g, s);
  if (akc) return dlaunch<BM, true, false>(g, s);
  if (bkc) return dlaunch<BM, false, true>(g, s);
  return dlaunch<BM, false, false>(g, s);
}

static bool daligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace trnblas

using namespace trnblas;

extern "C" int trnblas_hip_dgemm(int transA, int transB, int64_t M, int64_t N, int64_t K,
                                 double alpha, const double* A, int64_t lda, int64_t strideA,
                                 const double* B, int64_t ldb, int64_t strideB, double beta,
                                 const double* C, int64_t ldc, int64_t strideC, double* D,
                                 int64_t ldd, int64_t strideD, int64_t batch, int lower, int tri,
                                 void* stream) {
  clear_error();
  TRNBLAS_CHECK_ARG(M >= 0 && N >= 0 && K >= 0 && batch >= 0, "dgemm: negative size");
  TRNBLAS_CHECK_ARG(M < (1ll << 30) && N < (1ll << 30) && K < (1ll << 30),
                    "dgemm: dimension >= 2^30");
  TRNBLAS_CHECK_ARG((tri & ~15) == 0, "dgemm: bad tri flags %d", tri);
  TRNBLAS_CHECK_ARG(!lower || (M == N && batch <= 1), "dgemm: lower needs a square D, batch 1");
  if (M == 0 || N == 0 || batch == 0) return TRNBLAS_OK;
  TRNBLAS_CHECK_ARG(D != nullptr && ldd >= N, "dgemm: bad D / ldd");
  if (beta != 0.0) TRNBLAS_CHECK_ARG(C != nullptr && ldc >= N, "dgemm: beta != 0 needs C, ldc >= N");
  const bool akc = !transA, bkc = transB != 0;
  if (K > 0) {
    TRNBLAS_CHECK_ARG(A != nullptr && B != nullptr, "dgemm: A or B is NULL");
    TRNBLAS_CHECK_ARG(lda >= (akc ? K : M) && ldb >= (bkc ? K : N), "dgemm: lda / ldb too small");
    // 16-byte groups: aligned bases, even leading dimensions, strides and
    // contiguous extents (each group wholly inside or outside the matrix)
    const int64_t a_ext = akc ? K : M, b_ext = bkc ? K : N;
    TRNBLAS_CHECK_ARG(daligned16(A) && daligned16(B) && lda % 2 == 0 && ldb % 2 == 0 &&
                          strideA % 2 == 0 && strideB % 2 == 0 && a_ext % 2 == 0 &&
                          b_ext % 2 == 0,
                      "dgemm: A and B need 16-byte aligned bases and even leading dimensions, "
                      "batch strides and contiguous extents");
    // 32-bit buffer offsets within one k-tile panel
    const int64_t span_a = (akc ? 128 : 64) * lda * 8, span_b = (bkc ? 128 : 64) * ldb * 8;
    TRNBLAS_CHECK_ARG(span_a < (int64_t)kDRecords - 64 && span_b < (int64_t)kDRecords - 64,
                      "dgemm: leading dimension too large for 32-bit panel offsets");
  }
  DgemmArgs g{};
  g.M = (int)M;
  g.N = (int)N;
  g.K = (int)K;
  g.alpha = alpha;
  g.beta = beta;
  g.A = A;
  g.lda = lda;
  g.sA = strideA;
  g.B = B;
  g.ldb = ldb;
  g.sB = strideB;
  g.C = beta != 0.0 ? C : nullptr;
  g.ldc = ldc;
  g.sC = strideC;
  g.D = D;
  g.ldd = ldd;
  g.sD = strideD;
  g.batch = (int)batch;
  g.lower = lower != 0;
  g.tri = tri;
  // 128 x 128 tiles when they fill the chip, smaller ones for narrow launches
  const int cus = device_cus();
  auto tiles = [&](int64_t bm) {
    const int64_t tm = (M + bm - 1) / bm, tn = (N + bm - 1) / bm;
    return lower ? tm * (tm + 1) / 2 : tm * tn * batch;
  };
  if (tiles(128) >= cus) return dlaunch_layout<128>(g, akc, bkc, (hipStream_t)stream);
  if (tiles(64) >= cus) return dlaunch_layout<64>(g, akc, bkc, (hipStream_t)stream);
  return dlaunch_layout<32>(g, akc, bkc, (hipStream_t)stream);
}
