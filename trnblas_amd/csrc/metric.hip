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
// One workgroup of 576 threads per block, blocked by 4 x 4 tiles: the owner of
// tile (br, bc), br >= bc, keeps the tile at rows 4 br .., columns 4 bc .. of
// the 128 x 128 block (padded with the identity past nb) in registers.
// Cholesky, per tile column jb, one barrier: (A) the owner of the diagonal
// tile factors it (4 x 4 Cholesky) and publishes L_jj^-1 and
// A_jj^-1 = L_jj^-T L_jj^-1; after the barrier (B) the panel tiles below it
// become L_ij = A_ij L_jj^-T while (C) every trailing tile loses
// A_ij A_jj^-1 A_kj^T (= L_ij L_kj^T) from column jb's unscaled tiles, and
// the tiles of column jb + 1 publish themselves for the next step. Inverse X = L^-1, per tile row ib: the
// unscaled row of X and the column M_m = L_m,ib L_ib,ib^-1 are published,
// then the row becomes L_ib,ib^-1 X_ib and every later row m loses
// M_m X_ib (unscaled). Waves whose tiles all lie above the current tile row
// skip the arithmetic (those tiles are final) but keep the barriers.
#include "common.hpp"

namespace trnblas {

constexpr int kCholNB = 128;
constexpr int kCholNT = kCholNB / 4;
constexpr int kCholTiles = kCholNT * (kCholNT + 1) / 2;

constexpr int kCholThreads = (kCholTiles + 63) / 64 * 64;  // 9 waves

// 1 / sqrt(d) for d > 0: the hardware estimate (v_rsq_f64) refined by two
// Newton-Raphson steps y <- y (3 - d y^2) / 2, each of which doubles the
// correct bits; a short FMA chain in place of a correctly rounded sqrt and
// a division on the serial path of the diagonal tile. NaN for d <= 0.
__device__ __forceinline__ double rsqrt_nr(double d) {
  double y = __builtin_amdgcn_rsq(d);
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const double h = 0.5 * d * y;
    y = fma(-h, y, 1.5) * y;
  }
  return d > 0.0 ? y : __builtin_nan("");
}

__global__ __launch_bounds__(kCholThreads) void chol_block_kernel(int nb, double* A, int64_t lda,
                                                          double* Li, int64_t ldl, int32_t* info,
                                                          int offset) {
  __shared__ double dinv[kCholNT][16];    // L_jj^-1 of every diagonal tile, row-major
  __shared__ double ainv[2][16];          // Cholesky: A_jj^-1 = L_jj^-T L_jj^-1 of column j
  __shared__ double pan[2][kCholNT][16];  // Cholesky: column j's tiles before their scaling
  __shared__ double mcol[2][kCholNT][16]; // inverse: M_m of the current tile row
  __shared__ double xrow[2][kCholNT][16]; // inverse: the unscaled tile row of X
  __shared__ int sbad;

  // Thread t < 528 owns lower tile t in row-major triangle order
  // (br (br + 1) / 2 + bc = t); the rest of the last wave owns nothing.
  const int t = threadIdx.x;
  const bool own = t < kCholTiles;
  int br = (int)((sqrtf(8.0f * (float)t + 1.0f) - 1.0f) * 0.5f);
  while (br * (br + 1) / 2 > t) --br;
  while ((br + 1) * (br + 2) / 2 <= t) ++br;
  int bc = t - br * (br + 1) / 2;
  if (!own) br = bc = 0;  // (reads stay in range; nothing is published or written)
  // largest tile row in this wave (wave-uniform; -1 for a wave with no tile)
  const int tl = min((int)(t | 63), kCholTiles - 1);
  int wrow = (int)((sqrtf(8.0f * (float)tl + 1.0f) - 1.0f) * 0.5f);
  while (wrow * (wrow + 1) / 2 > tl) --wrow;
  while ((wrow + 1) * (wrow + 2) / 2 <= tl) ++wrow;
  if ((t & ~63) >= kCholTiles) wrow = -1;
  wrow = __builtin_amdgcn_readfirstlane(wrow);
  const int ntr = (nb + 3) >> 2;  // tile rows holding matrix entries
  if (t == 0) sbad = 0x7fffffff;

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

  // Column 0's tiles below the diagonal, as they are
  if (own && bc == 0 && br > 0) {
#pragma unroll
    for (int e = 0; e < 16; ++e) pan[0][br][e] = a[e >> 2][e & 3];
  }
  for (int jb = 0; jb < ntr; ++jb) {
    double(*pj)[16] = pan[jb & 1];
    double(*pn)[16] = pan[(jb + 1) & 1];
    double* aj = ainv[jb & 1];
    // (A) diagonal tile (updated through column jb - 1 by this same thread):
    // factor (lower part only), invert, and publish L_jj^-1 and A_jj^-1
    if (own && br == jb && bc == jb) {
      double rinv[4];  // 1 / l_cc
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const double d = a[c][c];
        if (!(d > 0.0) && 4 * jb + c < nb) atomicMin(&sbad, 4 * jb + c + 1);
        rinv[c] = rsqrt_nr(d);
        a[c][c] = d * rinv[c];
#pragma unroll
        for (int r = c + 1; r < 4; ++r) a[r][c] *= rinv[c];
#pragma unroll
        for (int r = c + 1; r < 4; ++r)
#pragma unroll
          for (int q = c + 1; q <= r; ++q) a[r][q] -= a[r][c] * a[q][c];
      }
      double m[4][4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int r = 0; r < c; ++r) m[r][c] = 0.0;
        m[c][c] = rinv[c];
#pragma unroll
        for (int r = c + 1; r < 4; ++r) {
          double sum = 0.0;
#pragma unroll
          for (int q = c; q < r; ++q) sum += a[r][q] * m[q][c];
          m[r][c] = -sum * rinv[r];
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          dinv[jb][4 * r + c] = m[r][c];
          if (c > r) a[r][c] = 0.0;
          double sum = 0.0;  // (m^T m)[r][c]
#pragma unroll
          for (int q = 0; q < 4; ++q) sum += m[q][r] * m[q][c];
          aj[4 * r + c] = sum;
        }
    }
    __syncthreads();  // L_jj^-1, A_jj^-1 and column jb's tiles are published
    if (wrow > jb && own && bc == jb && br > jb) {
      // (B) panel tile: L_ij = A_ij L_jj^-T
      double m[4][4], p[4][4];
#pragma unroll
      for (int e = 0; e < 16; ++e) m[e >> 2][e & 3] = dinv[jb][e];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          double sum = 0.0;
#pragma unroll
          for (int q = 0; q <= c; ++q) sum += a[r][q] * m[c][q];
          p[r][c] = sum;
        }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) a[r][c] = p[r][c];
    } else if (wrow > jb && own && bc > jb) {
      // (C) trailing tile: A_ik -= (A_ij A_jj^-1) A_kj^T, from column jb's
      // unscaled tiles (L_ij L_kj^T = A_ij A_jj^-1 A_kj^T), so the panel's
      // scaling (B) runs beside this update instead of before it
      double q4[4][4];  // A_ij A_jj^-1
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        double ai[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) ai[q] = pj[br][4 * r + q];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          double sum = 0.0;
#pragma unroll
          for (int q = 0; q < 4; ++q) sum += ai[q] * aj[4 * q + c];
          q4[r][c] = sum;
        }
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        double ak[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) ak[q] = pj[bc][4 * c + q];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          double sum = 0.0;
#pragma unroll
          for (int q = 0; q < 4; ++q) sum += q4[r][q] * ak[q];
          a[r][c] -= sum;
        }
      }
      // column jb + 1's tiles below the diagonal are now as the next step
      // needs them
      if (bc == jb + 1 && br > bc) {
#pragma unroll
        for (int e = 0; e < 16; ++e) pn[br][e] = a[e >> 2][e & 3];
      }
    }
  }

  double x[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) x[r][c] = (own && br == bc && r == c) ? 1.0 : 0.0;
  for (int ib = 0; ib < ntr; ++ib) {
    double(*mc)[16] = mcol[ib & 1];
    double(*xr)[16] = xrow[ib & 1];
    if (own && br == ib) {
#pragma unroll
      for (int e = 0; e < 16; ++e) xr[bc][e] = x[e >> 2][e & 3];
    }
    if (wrow > ib && own && bc == ib && br > ib) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          double sum = 0.0;
#pragma unroll
          for (int q = c; q < 4; ++q) sum += a[r][q] * dinv[ib][4 * q + c];
          mc[br][4 * r + c] = sum;
        }
    }
    __syncthreads();
    if (wrow < ib || !own || bc > ib || br < ib) continue;
    double xk[4][4];
#pragma unroll
    for (int e = 0; e < 16; ++e) xk[e >> 2][e & 3] = xr[bc][e];
    if (br == ib) {
      // the final row: L_ib,ib^-1 X_ib
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          double sum = 0.0;
#pragma unroll
          for (int q = 0; q <= r; ++q) sum += dinv[ib][4 * r + q] * xk[q][c];
          x[r][c] = sum;
        }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        double mr[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) mr[q] = mc[br][4 * r + q];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          double sum = 0.0;
#pragma unroll
          for (int q = 0; q < 4; ++q) sum += mr[q] * xk[q][c];
          x[r][c] -= sum;
        }
      }
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
  __syncthreads();
  if (t == 0 && sbad != 0x7fffffff && info[0] == 0) info[0] = offset + sbad;
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
  hipLaunchKernelGGL(chol_block_kernel, dim3(1), dim3(kCholThreads), 0, (hipStream_t)stream, (int)nb, A,
                     lda, Linv, ldl, info, (int)offset);
  return check_launch("chol_block");
}
