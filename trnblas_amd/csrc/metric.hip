// 128-wide diagonal blocks of the metric stage, fp64, for gfx950.
//
// metric_inv_half (trnblas/level3.py:365-380; the reference's device route is
// torch.linalg.cholesky + a blocked trsm, trnblas/nki/dispatch.py:1854-1881)
// returns X = L^-T for J = L L^T, and trsm (level3.py:332-362, the blocked
// solve of dispatch.py:1740-1799) solves with a triangular matrix. On the
// device both are blocked by 128: the panels, trailing updates and block
// products are fp64 GEMMs (dgemm.hip); these kernels do what a GEMM cannot,
// on one 128 x 128 diagonal block per workgroup:
//  * chol128_kernel: the Cholesky factor L of an updated SPD block and L^-1
//    (the panel solve then is a GEMM with L^-1, and L^-1 seeds the block
//    inverse of the whole factor);
//  * trinv128_kernel: the inverse of each 128 x 128 diagonal block of a
//    triangular matrix (trsm's diagonal solves become GEMMs).
//
// Inside a workgroup (8 waves) the block is a grid of 8 x 8 sub-blocks of
// 16 x 16 in LDS, lower sub-blocks only, each column-major with column pitch
// 17 doubles. With that pitch the three access patterns of the 16x16x4 f64
// MFMA are cheap: an A fragment (lane l: X[l % 16][4 q + l / 16]) reads 16
// consecutive doubles per 16-lane group, a B fragment (X[4 q + l / 16][l % 16])
// and the accumulator layout (lane l, register e: row 4 e + l / 16, column
// l % 16) fall on distinct banks.
//
// Cholesky, per 16-wide block column p (one barrier after each phase):
//  1. one wave factors the 16 x 16 diagonal sub-block and inverts it
//     (diag16: column by column, the column and the multipliers' row
//     exchanged through LDS; the inverse is built from the same row
//     operations applied to the identity);
//  2. the sub-blocks below it become L_ip = A_ip (L_pp^-1)^T (MFMA);
//  3. the trailing sub-blocks lose L_ip L_kp^T (MFMA).
// Inverse (both kernels), with the diagonal sub-blocks' inverses in place:
// recursive doubling over halves of 16, 32 and 64,
// Y21 = -Y22 (L21 Y11), in place over L21, through an LDS scratch for the
// intermediate product.
#include <type_traits>

#include "common.hpp"

namespace trnblas {

typedef double f64x4 __attribute__((ext_vector_type(4)));

constexpr int kCholNB = 128;
constexpr int kSP = 17;          // column pitch of a sub-block (doubles)
constexpr int kSB = 16 * kSP;    // doubles per sub-block
constexpr int kNS = 8;           // sub-blocks per side
constexpr int kNLow = kNS * (kNS + 1) / 2;  // lower sub-blocks
constexpr int kThreads = 512;    // 8 waves

__device__ __forceinline__ int sidx(int i, int j) { return i * (i + 1) / 2 + j; }  // i >= j

// 1 / sqrt(d) for d > 0: the hardware estimate (v_rsq_f64) refined by two
// Newton-Raphson steps y <- y (3 - d y^2) / 2; NaN for d <= 0.
__device__ __forceinline__ double rsqrt_nr(double d) {
  double y = __builtin_amdgcn_rsq(d);
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const double h = 0.5 * d * y;
    y = fma(-h, y, 1.5) * y;
  }
  return d > 0.0 ? y : __builtin_nan("");
}

// 1 / d: the hardware estimate (v_rcp_f64) refined by two Newton-Raphson
// steps y <- y + y (1 - d y).
__device__ __forceinline__ double rcp_nr(double d) {
  double y = __builtin_amdgcn_rcp(d);
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const double e = fma(-d, y, 1.0);
    y = fma(y, e, y);
  }
  return y;
}

__device__ __forceinline__ double readlane_f64(double v, int l) {
  const long long b = __builtin_bit_cast(long long, v);
  const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)b, l);
  const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(b >> 32), l);
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

// MFMA operand and accumulator access of one sub-block (slice q = 0..3).
__device__ __forceinline__ double frag_a(const double* s, int lane, int q) {
  return s[(4 * q + (lane >> 4)) * kSP + (lane & 15)];  // X[l % 16][4 q + l / 16]
}
__device__ __forceinline__ double frag_b(const double* s, int lane, int q) {
  return s[(lane & 15) * kSP + 4 * q + (lane >> 4)];  // X[4 q + l / 16][l % 16]
}
__device__ __forceinline__ f64x4 load_acc(const double* s, int lane) {
  const double* p = s + (lane & 15) * kSP + (lane >> 4);
  return f64x4{p[0], p[4], p[8], p[12]};
}
__device__ __forceinline__ void store_acc(double* s, int lane, const f64x4& v) {
  double* p = s + (lane & 15) * kSP + (lane >> 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) p[4 * e] = v[e];
}
// acc += sgn X Y^T (BT) or sgn X Y
template <bool BT>
__device__ __forceinline__ void mma16(f64x4& acc, const double* X, const double* Y, double sgn,
                                      int lane) {
  double a[4], b[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    a[q] = sgn * frag_a(X, lane, q);
    b[q] = BT ? frag_a(Y, lane, q) : frag_b(Y, lane, q);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_mfma_f64_16x16x4f64(a[q], b[q], acc, 0, 0, 0);
}

template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (N > 0) {
    static_for<N - 1>(f);
    f(std::integral_constant<int, N - 1>{});
  }
}

// v from lane SRC of the lane's 16-lane row (DPP row_newbcast).
template <int SRC>
__device__ __forceinline__ double row_bcast(double v) {
  const long long b = __builtin_bit_cast(long long, v);
  const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)b, 0x150 + SRC, 0xf, 0xf, false);
  const unsigned hi =
      (unsigned)__builtin_amdgcn_update_dpp(0, (int)(b >> 32), 0x150 + SRC, 0xf, 0xf, false);
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

// One wave on a 16 x 16 diagonal sub-block `blk` (lower part read).
// CHOL: blk becomes L (blk = L L^T, zeros above) and inv receives L^-1;
// a non-positive (or NaN) pivot sets *bad to min(*bad, col0 + column + 1)
// when that column is below nb. Otherwise blk is lower triangular (unit:
// its diagonal taken as ones) and inv receives its inverse; blk is not
// written.
// Lane (h = l / 16, r = l % 16) holds columns 4 e + h of row r (e = 0..3)
// of the matrix and of E, the product of the elimination steps so far
// (unit lower; after the last column E = (unit L)^-1, and L^-1 = diag(1 /
// l_rr) E). Per column c: the pivot by readlane; every lane publishes its
// (scaled) element of column 4 (c / 4) + h through LDS, of which the
// column-c ones are read back (L[r][c] and L[s][c] for the lane's
// columns); row c of E comes from lane c of the lane's own 16-lane row
// (DPP). Updates are unconditional where the arithmetic leaves the final
// values unchanged (zero multipliers, zero entries of E), so the loop has
// no branches; the strict upper part of the matrix collects garbage that
// is never read and is written out as zeros. ex: 80 doubles of this
// wave's LDS.
template <bool CHOL>
__device__ __forceinline__ void diag16(double* blk, double* inv, double* ex, int lane, bool unit,
                                       int* bad, int col0, int nb) {
  double* colb = ex;        // colb[16 h + r]: lane (h, r)'s published value
  double* rinvb = ex + 64;  // 1 / l_cc
  // (an opaque copy of the lane index: otherwise the per-column lane masks
  // are computed once, outside the caller's loop, and spill)
  int ln = lane;
  asm volatile("" : "+v"(ln));
  const int r = ln & 15, h = ln >> 4;
  double a[4], E[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int s = 4 * e + h;
    a[e] = s <= r ? blk[s * kSP + r] : 0.0;
    if (!CHOL && unit && s == r) a[e] = 1.0;
    E[e] = s == r ? 1.0 : 0.0;
  }
  static_for<16>([&](auto cI) {
    constexpr int c = decltype(cI)::value, ch = c & 3, ce = c >> 2;
    const double d = readlane_f64(a[ce], c + 16 * ch);  // the pivot
    const double rinv = CHOL ? rsqrt_nr(d) : (unit ? 1.0 : rcp_nr(d));
    colb[16 * h + r] = CHOL ? a[ce] * rinv : a[ce];
    rinvb[c] = rinv;
    double ev[4];  // E[c][4 e + h]
#pragma unroll
    for (int e = 0; e < 4; ++e) ev[e] = row_bcast<c>(E[e]);
    __builtin_amdgcn_wave_barrier();
    const double lr = colb[16 * ch + r];  // L[r][c] (CHOL) / T[r][c]
    const double m = r > c ? lr * rinv : 0.0;  // the elimination multiplier of row r
    if (CHOL) {
      double cs[4];  // L[4 e + h][c]
#pragma unroll
      for (int e = ce; e < 4; ++e) cs[e] = colb[16 * ch + 4 * e + h];
      a[ce] = h == ch ? lr : a[ce];
#pragma unroll
      for (int e = ce + 1; e < 4; ++e) a[e] = fma(-lr, cs[e], a[e]);
      a[ce] = h > ch ? fma(-lr, cs[ce], a[ce]) : a[ce];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) E[e] = fma(-m, ev[e], E[e]);
    __builtin_amdgcn_wave_barrier();
  });
  const double rr = rinvb[r];
  if (CHOL) {  // the first NaN 1 / l_cc is the first pivot that is not positive
    const bool isbad = ln < 16 && !(rr == rr) && col0 + ln < nb;
    const unsigned long long msk = __ballot(isbad);
    if (msk != 0ull && ln == 0) *bad = min(*bad, col0 + (int)__builtin_ctzll(msk) + 1);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int s = 4 * e + h;
    if (CHOL) blk[s * kSP + r] = s <= r ? a[e] : 0.0;
    inv[s * kSP + r] = s <= r ? E[e] * rr : 0.0;
  }
}

// acc += sgn sum_{t < n} X_t Y_t (n <= NMAX, wave-uniform) over sub-block
// pairs given by the offsets xo[t], yo[t] into G / Y buffers: every
// fragment is read before the first MFMA (offsets past n repeat a valid
// pair and their MFMAs are skipped), so the LDS reads overlap.
template <int NMAX>
__device__ __forceinline__ void mma16_sum(f64x4& acc, const double* X, const int (&xo)[NMAX],
                                          const double* Y, const int (&yo)[NMAX], int n, double sgn,
                                          int lane) {
  double a[NMAX][4], b[NMAX][4];
#pragma unroll
  for (int t = 0; t < NMAX; ++t)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      a[t][q] = sgn * frag_a(X + xo[t], lane, q);
      b[t][q] = frag_b(Y + yo[t], lane, q);
    }
#pragma unroll
  for (int t = 0; t < NMAX; ++t)
    if (t < n) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        acc = __builtin_amdgcn_mfma_f64_16x16x4f64(a[t][q], b[t][q], acc, 0, 0, 0);
    }
}

// The block inverse Y = L^-1 in place over the lower sub-block grid G, whose
// off-diagonal sub-blocks hold L and diagonal ones their inverses: for
// halves of h = 1, 2, 4 sub-blocks and each column j of a half, T = L21 Y11
// (column j) into scr, then Y21 = -Y22 T (column j) over L21. A round
// handles one column of every pair: 4 sub-blocks of T, so scr holds 4
// (later rounds read only columns of L21 that earlier rounds left).
__device__ __forceinline__ void block_inverse(double* G, double* scr, int wave, int lane) {
  static_for<3>([&](auto lI) {
    constexpr int h = 1 << decltype(lI)::value;
    for (int j = 0; j < h; ++j) {
      if (wave < 4) {  // item = (pair pi, row i of the half)
        const int pi = wave / h, i = wave % h, b0 = 2 * h * pi;
        int xo[h], yo[h];
#pragma unroll
        for (int t = 0; t < h; ++t) {  // k = j + t < h
          const int k = min(j + t, h - 1);
          xo[t] = sidx(b0 + h + i, b0 + k) * kSB;
          yo[t] = sidx(b0 + k, b0 + j) * kSB;
        }
        f64x4 acc = {0.0, 0.0, 0.0, 0.0};
        mma16_sum<h>(acc, G, xo, G, yo, h - j, 1.0, lane);
        store_acc(scr + wave * kSB, lane, acc);
      }
      __syncthreads();
      if (wave < 4) {
        const int pi = wave / h, i = wave % h, b0 = 2 * h * pi;
        int xo[h], yo[h];
#pragma unroll
        for (int t = 0; t < h; ++t) {  // k = t <= i
          const int k = min(t, i);
          xo[t] = sidx(b0 + h + i, b0 + h + k) * kSB;
          yo[t] = (pi * h + k) * kSB;
        }
        f64x4 acc = {0.0, 0.0, 0.0, 0.0};
        mma16_sum<h>(acc, G, xo, scr, yo, i + 1, -1.0, lane);
        store_acc(G + sidx(b0 + h + i, b0 + j) * kSB, lane, acc);
      }
      __syncthreads();
    }
  });
}

// The lower triangle of a 128 x 128 block (element (i, k) at
// X[i * ri + k * ci], the identity past nb) into the sub-block grid. Thread
// t takes column k = t % 128 of rows t / 128 + 4 u (u = 0..31), so its
// addresses step by a constant and the sub-block of each u is known at
// compile time; all 32 loads issue before the first LDS store.
template <typename TT>
__device__ __forceinline__ void load_lower(double* G, const TT* X, int64_t ri, int64_t ci, int nb,
                                           int tid) {
  constexpr int PER = kCholNB * kCholNB / kThreads;  // 32
  const int k = tid & 127, i0 = tid >> 7;
  const TT* p = X + i0 * ri + k * ci;
  double v[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = i0 + 4 * u;
    v[u] = (k <= i && i < nb) ? (double)p[(int64_t)(4 * u) * ri] : (i == k ? 1.0 : 0.0);
  }
  double* g = G + (k >> 4) * kSB + (k & 15) * kSP + i0;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = i0 + 4 * u;
    if (k <= i) g[sidx(u >> 2, 0) * kSB + 4 * (u & 3)] = v[u];
  }
}

// The lower triangle of the grid out to Z[i * zr + k * zc] for i, k < nb
// (zeros above the diagonal when `full`, else the strict upper part
// untouched), in the thread mapping of load_lower.
template <typename TT>
__device__ __forceinline__ void store_lower(const double* G, TT* Z, int64_t zr, int64_t zc, int nb,
                                            bool full, int tid, bool skip_diag = false) {
  constexpr int PER = kCholNB * kCholNB / kThreads;
  asm volatile("" : "+v"(tid));  // (its masks and addresses computed here, not at kernel entry)
  const int k = tid & 127, i0 = tid >> 7;
  const double* g = G + (k >> 4) * kSB + (k & 15) * kSP + i0;
  double v[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = i0 + 4 * u;
    v[u] = k <= i ? g[sidx(u >> 2, 0) * kSB + 4 * (u & 3)] : 0.0;
  }
  TT* z = Z + (int64_t)i0 * zr + (int64_t)k * zc;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = i0 + 4 * u;
    if (i < nb && k < nb && (full || k <= i) && !(skip_diag && (i >> 4) == (k >> 4)))
      z[(int64_t)(4 * u) * zr] = (TT)v[u];
  }
}

// LDS: the sub-block grid (78 KB), one diagonal inverse, the block
// inverse's scratch and diag16's exchange: 91 KB, so the workgroup shares a
// CU with a GEMM workgroup (64 KB) of a concurrent stream instead of
// waiting for a whole free CU.
__global__ __launch_bounds__(kThreads) void chol128_kernel(int nb, double* A, int64_t lda,
                                                           double* Li, int64_t ldl, int32_t* info,
                                                           int offset) {
  __shared__ double G[kNLow * kSB];
  __shared__ double D1[kSB];        // inverse of the current diagonal sub-block
  __shared__ double scr[4 * kSB];   // T of the block inverse
  __shared__ double ex[80];         // diag16's exchange
  __shared__ int sbad;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (tid == 0) sbad = 0x7fffffff;
  // the lower triangle, the identity past nb (diag16 reads and writes only
  // the lower part of a diagonal sub-block)
  load_lower(G, A, lda, 1, nb, tid);
  __syncthreads();
  for (int p = 0; p < kNS; ++p) {
    double* Gpp = G + sidx(p, p) * kSB;
    if (wave == 0) diag16<true>(Gpp, D1, ex, lane, false, &sbad, 16 * p, nb);
    __syncthreads();
    for (int i = p + 1 + wave; i < kNS; i += kThreads / 64) {  // panel
      f64x4 acc = {0.0, 0.0, 0.0, 0.0};
      mma16<true>(acc, G + sidx(i, p) * kSB, D1, 1.0, lane);
      store_acc(G + sidx(i, p) * kSB, lane, acc);
    }
    __syncthreads();
    const int nt = kNS - 1 - p, items = nt * (nt + 1) / 2;
    if (wave == 7) {
      // L_pp out to A (its lower part), then L_pp^-1 in its place: the
      // trailing update below does not read the diagonal sub-block
      for (int e = lane; e < 256; e += 64) {
        const int r = e >> 4, c = e & 15, i = 16 * p + r, k = 16 * p + c;
        if (c <= r && i < nb) A[(int64_t)i * lda + k] = Gpp[c * kSP + r];
      }
      for (int e = lane; e < kSB; e += 64) Gpp[e] = D1[e];
    }
    for (int it = wave; it < items; it += kThreads / 64) {  // trailing update
      int ri = 0;
      while ((ri + 1) * (ri + 2) / 2 <= it) ++ri;
      const int i = p + 1 + ri, k = p + 1 + (it - ri * (ri + 1) / 2);
      f64x4 acc = load_acc(G + sidx(i, k) * kSB, lane);
      mma16<true>(acc, G + sidx(i, p) * kSB, G + sidx(k, p) * kSB, -1.0, lane);
      store_acc(G + sidx(i, k) * kSB, lane, acc);
    }
    __syncthreads();
  }
  // the off-diagonal sub-blocks of L out (the diagonal ones went out per
  // step; the diagonal sub-blocks of G now hold their inverses)
  store_lower(G, A, lda, (int64_t)1, nb, false, tid, true);
  __syncthreads();
  block_inverse(G, scr, wave, lane);
  store_lower(G, Li, ldl, (int64_t)1, nb, true, tid);
  if (tid == 0 && sbad != 0x7fffffff && info[0] == 0) info[0] = offset + sbad;
}

// Inverse of diagonal block b of the n x n triangular matrix T: element
// (i, k) of the lower matrix inverted is T[k0 + i][k0 + k] (lower) or
// T[k0 + k][k0 + i] (upper: T^T is inverted and the result transposed back),
// read through the strides (sr, sc) in T's element type. Dinv[b] (128 x 128
// row-major) receives the inverse, the identity past the matrix.
template <typename TT>
__global__ __launch_bounds__(kThreads) void trinv128_kernel(int n, int upper, int unit,
                                                            const TT* T, int64_t sr, int64_t sc,
                                                            TT* Dinv) {
  __shared__ double G[kNLow * kSB];
  __shared__ double scr[4 * kSB];
  __shared__ double ex[kThreads / 64][80];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.x, k0 = b * kCholNB, nb = min(kCholNB, n - k0);
  const int64_t ri = upper ? sc : sr, ci = upper ? sr : sc;  // strides of the lower view
  load_lower(G, T + (int64_t)k0 * (sr + sc), ri, ci, nb, tid);
  __syncthreads();
  // the 8 diagonal sub-blocks' inverses, one wave each, in place (diag16
  // reads the sub-block into registers before it writes the inverse)
  diag16<false>(G + sidx(wave, wave) * kSB, G + sidx(wave, wave) * kSB, ex[wave], lane, unit != 0,
                nullptr, 0, 0);
  __syncthreads();
  block_inverse(G, scr, wave, lane);
  // lower: out[i][k] = Y[i][k]; upper: out[k][i] = Y[i][k]
  TT* out = Dinv + (int64_t)b * kCholNB * kCholNB;
  store_lower(G, out, upper ? (int64_t)1 : (int64_t)kCholNB, upper ? (int64_t)kCholNB : (int64_t)1,
              kCholNB, true, tid);
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
  hipLaunchKernelGGL(chol128_kernel, dim3(1), dim3(kThreads), 0, (hipStream_t)stream, (int)nb, A,
                     lda, Linv, ldl, info, (int)offset);
  return check_launch("chol_block");
}

extern "C" int trnblas_hip_tri_inv_blocks(int dtype, int64_t n, int upper, int unit, const void* T,
                                          int64_t ldt_r, int64_t ldt_c, void* Dinv, void* stream) {
  clear_error();
  TRNBLAS_CHECK_ARG(dtype == TRNBLAS_F32 || dtype == TRNBLAS_F64,
                    "tri_inv_blocks: dtype %d not supported (f32, f64)", dtype);
  TRNBLAS_CHECK_ARG(n >= 0 && n < (1ll << 30), "tri_inv_blocks: bad n %lld", (long long)n);
  if (n == 0) return TRNBLAS_OK;
  TRNBLAS_CHECK_ARG(T && Dinv, "tri_inv_blocks: NULL pointer");
  TRNBLAS_CHECK_ARG(ldt_r > 0 && ldt_c > 0 && (ldt_r >= n || ldt_c >= n || n == 1),
                    "tri_inv_blocks: bad strides");
  const int nblk = (int)((n + kCholNB - 1) / kCholNB);
  if (dtype == TRNBLAS_F64)
    hipLaunchKernelGGL(trinv128_kernel<double>, dim3(nblk), dim3(kThreads), 0, (hipStream_t)stream,
                       (int)n, upper, unit, static_cast<const double*>(T), ldt_r, ldt_c,
                       static_cast<double*>(Dinv));
  else
    hipLaunchKernelGGL(trinv128_kernel<float>, dim3(nblk), dim3(kThreads), 0, (hipStream_t)stream,
                       (int)n, upper, unit, static_cast<const float*>(T), ldt_r, ldt_c,
                       static_cast<float*>(Dinv));
  return check_launch("tri_inv_blocks");
}
