// Diagonal blocks of the metric factorisation, fp64, for gfx950.
//
// metric_inv_half (trnblas/level3.py:365-380; the reference's device route is
// torch.linalg.cholesky + a blocked trsm, trnblas/nki/dispatch.py:1854-1881)
// returns X = L^-T for J = L L^T. On the device this build factors J by a
// right-looking blocked Cholesky whose trailing updates and panels are
// DGEMMs; this kernel is the step those cannot do: the Cholesky factor L_kk
// of one updated diagonal block (nb <= 128) and its inverse L_kk^-1, which
// turns the panel solve into a GEMM and seeds the block inverse of L.
//
// One 1024-thread workgroup per block. The owner of tile (br, bc), br >= bc,
// keeps the 4 x 4 tile at rows 4 br .., columns 4 bc .. of the 128 x 128
// block (padded with the identity past nb) in registers. Both phases are
// right-looking with
// one barrier per column: the owners of the column (and, for the inverse,
// of the row) publish it into an LDS vector (double buffered, so a vector is
// rewritten only two barriers after it was read), every owner then applies
// the rank-1 update to its tile.
#include "common.hpp"

namespace trnblas {

constexpr int kCholNB = 128;

__global__ __launch_bounds__(1024) void chol_block_kernel(int nb, double* A, int64_t lda,
                                                          double* Li, int64_t ldl, int32_t* info,
                                                          int offset) {
  __shared__ double col[2][kCholNB];
  __shared__ double row[2][kCholNB];
  // Thread t < 528 owns lower tile t of the 32 x 32 tile grid in row-major
  // triangle order (br (br + 1) / 2 + bc = t); the others own nothing. A
  // wave whose tiles all lie above the current row skips the update (the
  // tiles of a finished row never change again) but keeps the barriers.
  const int t = threadIdx.x;
  constexpr int kTiles = 32 * 33 / 2;
  const bool own = t < kTiles;
  int br = (int)((sqrtf(8.0f * (float)t + 1.0f) - 1.0f) * 0.5f);
  while (br * (br + 1) / 2 > t) --br;
  while ((br + 1) * (br + 2) / 2 <= t) ++br;
  int bc = t - br * (br + 1) / 2;
  if (!own) br = bc = 0;  // (reads stay in range; nothing is published or written)
  // largest tile row in this wave (wave-uniform; -1 for a wave with no tile)
  const int tl = min((int)(t | 63), kTiles - 1);
  int wrow = (int)((sqrtf(8.0f * (float)tl + 1.0f) - 1.0f) * 0.5f);
  while (wrow * (wrow + 1) / 2 > tl) --wrow;
  while ((wrow + 1) * (wrow + 2) / 2 <= tl) ++wrow;
  if ((t & ~63) >= kTiles) wrow = -1;
  wrow = __builtin_amdgcn_readfirstlane(wrow);

  double a[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int i = 4 * br + r, k = 4 * bc + c;
      double v = 0.0;
      if (own && k <= i) v = (i < nb) ? A[(int64_t)i * lda + k] : (i == k ? 1.0 : 0.0);
      a[r][c] = v;
    }

  // Cholesky: at column j the tile entries (i, k), j < k <= i, lose
  // a_ij a_kj / a_jj; column j becomes a_ij / sqrt(a_jj), its diagonal
  // sqrt(a_jj). A pivot that is not positive (or NaN) is recorded
  // (1-based, plus the block's offset in J) and the factor is garbage.
  int bad = 0;
  for (int j = 0; j < nb; ++j) {
    double* cv = col[j & 1];
    if (own && bc == (j >> 2)) {
      // (static indices only: a runtime index into the tile puts it in scratch)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        double v = a[r][0];
#pragma unroll
        for (int c = 1; c < 4; ++c) v = (j & 3) == c ? a[r][c] : v;
        cv[4 * br + r] = v;
      }
    }
    __syncthreads();
    // every value the step needs is read at once, and the tile is updated
    // with selects: per-entry branches around the LDS reads serialise them
    const double d = cv[j];
    double ci[4], ck[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) ci[r] = cv[4 * br + r];
#pragma unroll
    for (int c = 0; c < 4; ++c) ck[c] = cv[4 * bc + c];
    if (!(d > 0.0) && bad == 0) bad = j + 1;
    if (wrow < (j >> 2)) continue;
    const double rt = sqrt(d), rinv = 1.0 / rt, dinv = rinv * rinv;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int i = 4 * br + r, k = 4 * bc + c;
        const double upd = a[r][c] - ci[r] * ck[c] * dinv;
        const double cj = i == j ? rt : ci[r] * rinv;
        a[r][c] = (k == j && i >= j) ? cj : ((k > j && i >= k) ? upd : a[r][c]);
      }
  }

  // Inverse X = L^-1 (lower), forward substitution by rows: at row i the row
  // is complete up to the factor 1 / l_ii; every later row m loses
  // (l_mi / l_ii) x_i. Row i of X and column i of L are published together.
  double x[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) x[r][c] = (own && 4 * br + r == 4 * bc + c) ? 1.0 : 0.0;
  for (int i = 0; i < nb; ++i) {
    double* lc = col[(nb + i) & 1];
    double* xr = row[i & 1];
    if (own && bc == (i >> 2)) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        double v = a[r][0];
#pragma unroll
        for (int c = 1; c < 4; ++c) v = (i & 3) == c ? a[r][c] : v;
        lc[4 * br + r] = v;
      }
    }
    if (own && br == (i >> 2)) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        double v = x[0][c];
#pragma unroll
        for (int r = 1; r < 4; ++r) v = (i & 3) == r ? x[r][c] : v;
        xr[4 * bc + c] = v;
      }
    }
    __syncthreads();
    if (wrow < (i >> 2)) continue;
    const double inv = 1.0 / lc[i];
    double lm[4], xk[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) lm[r] = lc[4 * br + r];
#pragma unroll
    for (int c = 0; c < 4; ++c) xk[c] = xr[4 * bc + c];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int m = 4 * br + r, k = 4 * bc + c;
        // X is lower triangular: row i is zero past column i (and those
        // entries of the published row are stale), so columns k > i stay
        const double v = m == i ? x[r][c] * inv : x[r][c] - lm[r] * inv * xk[c];
        x[r][c] = (k <= i && m >= i) ? v : x[r][c];
      }
  }

#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int i = 4 * br + r, k = 4 * bc + c;
      if (own && i < nb && k < nb) {
        if (k <= i) A[(int64_t)i * lda + k] = a[r][c];
        Li[(int64_t)i * ldl + k] = k <= i ? x[r][c] : 0.0;
        // the mirrored tile above the diagonal has no owner: its zeros
        if (br > bc) Li[(int64_t)k * ldl + i] = 0.0;
      }
    }
  if (t == 0 && bad && info[0] == 0) info[0] = offset + bad;
}

}  // namespace trnblas

using namespace trnblas;

extern "C" int trnblas_hip_chol_block(int64_t nb, double* A, int64_t lda, double* Linv,
                                      int64_t ldl, int32_t* info, int64_t offset, void* stream) {
  clear_error();
  TRNBLAS_CHECK_ARG(nb >= 0 && nb <= kCholNB, "chol_block: nb %lld not in [0, %d]", (long long)nb,
                    kCholNB);
  if (nb == 0) return TRNBLAS_OK;
  TRNBLAS_CHECK_ARG(A && Linv && info, "chol_block: NULL pointer");
  TRNBLAS_CHECK_ARG(lda >= nb && ldl >= nb, "chol_block: leading dimension below nb");
  TRNBLAS_CHECK_ARG(offset >= 0 && offset < (1ll << 30), "chol_block: bad offset");
  hipLaunchKernelGGL(chol_block_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, (int)nb, A,
                     lda, Linv, ldl, info, (int)offset);
  return check_launch("chol_block");
}
