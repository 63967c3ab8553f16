// Native drivers of the metric stage: the blocked Cholesky inverse factor
// (metric_inv_half, trnblas/level3.py:365-380) and the blocked triangular
// solve (trsm, level3.py:332-362; the reference's blocked solve is
// `_nki_trsm_left`, trnblas/nki/dispatch.py:1740-1799). Each is one C-ABI
// call that issues its whole launch sequence from C++: the 128-wide
// diagonal-block kernels (metric.hip) and the GEMMs around them (dgemm.hip,
// and gemm.hip for fp32 trsm). Issued from Python, each launch's host cost
// (~50 us through ctypes) exceeded its GPU time, and the GPU waited.
//
// metric_inv_half: right-looking blocked Cholesky with look-ahead. After the
// panel of block b only the next block column is updated on the caller's
// stream, so block b + 1 is factored while a second stream (per device,
// default priority) applies the rest of the trailing update (lower
// triangle only) with the other CUs; the caller's stream waits for it
// before it next writes there. Y = L^-1 is built beside the factorisation
// on a third stream: once block b is factored (its inverse Y_bb written in
// place by the diagonal kernel), block row b of Y follows from the rows
// above it, Y[b, :b] = -Y_bb (L[b, :b] Y[:b, :b]), two GEMMs that run
// while the caller's stream factors the next blocks (the late steps, bound
// by the one-workgroup diagonal kernel, leave most CUs free). Then X = Y^T.
#include <mutex>

#include "common.hpp"

namespace trnblas {

constexpr int kNB = 128;

// The 2-D helpers walk rows with blockIdx.y and columns with blockIdx.x
// (grid-strided both ways).
__global__ __launch_bounds__(256) void fill_kernel(double* p, int64_t rows, int64_t cols,
                                                   int64_t ld, double v) {
  for (int64_t i = blockIdx.y; i < rows; i += gridDim.y)
    for (int64_t j = blockIdx.x * 256ll + threadIdx.x; j < cols; j += (int64_t)gridDim.x * 256)
      p[i * ld + j] = v;
}

// dst[i * dr + j * dc] = alpha * src[i * sr + j * sc], rows x cols
template <typename TS, typename TD>
__global__ __launch_bounds__(256) void copy2d_kernel(int64_t rows, int64_t cols, const TS* src,
                                                     int64_t sr, int64_t sc, TD* dst,
                                                     int64_t dr, int64_t dc, double alpha) {
  for (int64_t i = blockIdx.y; i < rows; i += gridDim.y)
    for (int64_t j = blockIdx.x * 256ll + threadIdx.x; j < cols; j += (int64_t)gridDim.x * 256)
      dst[i * dr + j * dc] = (TD)(alpha * (double)src[i * sr + j * sc]);
}

__global__ void set_i32_kernel(int32_t* p, int32_t v) { *p = v; }

static dim3 grid2d(int64_t rows, int64_t cols) {
  const int64_t gx = (cols + 255) / 256, gy = rows;
  return dim3((unsigned)(gx < 64 ? (gx > 0 ? gx : 1) : 64), (unsigned)(gy < 4096 ? (gy > 0 ? gy : 1) : 4096));
}

// X[j][i] = Y[i][j] for i, j < n through a 64 x 64 LDS tile (both sides
// coalesced)
__global__ __launch_bounds__(256) void transpose_kernel(int n, const double* Y, int64_t ldy,
                                                        double* X, int64_t ldx) {
  __shared__ double t[64][65];
  const int i0 = blockIdx.y * 64, j0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int i = i0 + r, j = j0 + tx;
    t[r][tx] = (i < n && j < n) ? Y[(int64_t)i * ldy + j] : 0.0;
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int j = j0 + r, i = i0 + tx;
    if (i < n && j < n) X[(int64_t)j * ldx + i] = t[tx][r];
  }
}

static int grid_for(int64_t elems) {
  const int64_t g = (elems + 255) / 256;
  return (int)(g < 4096 ? (g > 0 ? g : 1) : 4096);
}

static int fill(double* p, int64_t rows, int64_t cols, int64_t ld, double v, hipStream_t s) {
  if (rows <= 0 || cols <= 0) return TRNBLAS_OK;
  hipLaunchKernelGGL(fill_kernel, grid2d(rows, cols), dim3(256), 0, s, p, rows, cols, ld, v);
  return check_launch("fill");
}

// Per device: the side stream of the look-ahead and the two events that
// hand work between the streams (re-recorded every step; a wait uses the
// record that precedes it), and the mutex that keeps calls on one device
// from interleaving their use.
struct SideStream {
  std::mutex mu;
  hipStream_t side = nullptr, inv = nullptr;
  hipEvent_t ready = nullptr, done = nullptr, inverted = nullptr;
};

static SideStream* side_stream(int& rc) {
  static SideStream devs[64];
  int dev = 0;
  rc = TRNBLAS_OK;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    set_error("metric_inv_half: no current device");
    rc = TRNBLAS_E_LAUNCH;
    return nullptr;
  }
  return &devs[dev];
}

static int side_init(SideStream* ss) {
  if (ss->side) return TRNBLAS_OK;
  if (hipStreamCreateWithFlags(&ss->side, hipStreamNonBlocking) != hipSuccess ||
      hipStreamCreateWithFlags(&ss->inv, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreateWithFlags(&ss->ready, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ss->done, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ss->inverted, hipEventDisableTiming) != hipSuccess) {
    set_error("metric_inv_half: cannot create the side stream / events");
    return TRNBLAS_E_LAUNCH;
  }
  return TRNBLAS_OK;
}

static void metric_layout(int64_t n, int64_t& nblk, int64_t& npad, size_t off[4]) {
  nblk = (n + kNB - 1) / kNB;
  npad = nblk * kNB;
  const size_t sq = (size_t)npad * npad * 8;
  auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
  off[0] = 0;                                // W: J, updated in place
  off[1] = up(off[0] + sq);                  // L: panels of the factor
  off[2] = up(off[1] + sq);                  // Y: L^-1 (diagonal blocks from the kernel)
  off[3] = up(off[2] + sq);                  // T: a block row's product L[b, :b] Y[:b, :b]
}

#define TRY(x)                        \
  do {                                \
    const int rc_ = (x);              \
    if (rc_ != TRNBLAS_OK) return rc_; \
  } while (0)

}  // namespace trnblas

using namespace trnblas;

extern "C" size_t trnblas_hip_metric_inv_half_workspace(int64_t n) {
  if (n <= 0) return 0;
  int64_t nblk, npad;
  size_t off[4];
  metric_layout(n, nblk, npad, off);
  return off[3] + (size_t)kNB * npad * 8;
}

extern "C" int trnblas_hip_metric_inv_half(int64_t n, const double* J, int64_t ldj, double* X,
                                           int64_t ldx, int32_t* info, void* workspace,
                                           size_t workspace_bytes, void* stream) {
  clear_error();
  TRNBLAS_CHECK_ARG(n >= 0 && n < (1ll << 20), "metric_inv_half: bad n %lld", (long long)n);
  if (n == 0) return TRNBLAS_OK;
  TRNBLAS_CHECK_ARG(J && X && info && workspace, "metric_inv_half: NULL pointer");
  TRNBLAS_CHECK_ARG(ldj >= n && ldx >= n, "metric_inv_half: leading dimension below n");
  TRNBLAS_CHECK_ARG(workspace_bytes >= trnblas_hip_metric_inv_half_workspace(n),
                    "metric_inv_half: workspace %zu bytes, %zu needed", workspace_bytes,
                    trnblas_hip_metric_inv_half_workspace(n));
  TRNBLAS_CHECK_ARG((reinterpret_cast<uintptr_t>(workspace) & 255) == 0,
                    "metric_inv_half: workspace must be 256-byte aligned");
  hipStream_t main = (hipStream_t)stream;
  int64_t nblk, npad;
  size_t off[4];
  metric_layout(n, nblk, npad, off);
  char* ws = static_cast<char*>(workspace);
  double* W = reinterpret_cast<double*>(ws + off[0]);
  double* L = reinterpret_cast<double*>(ws + off[1]);
  double* Y = reinterpret_cast<double*>(ws + off[2]);
  double* T = reinterpret_cast<double*>(ws + off[3]);
  int rc = TRNBLAS_OK;
  SideStream* ss = side_stream(rc);
  if (!ss) return rc;
  std::lock_guard<std::mutex> lock(ss->mu);
  TRY(side_init(ss));
  auto wait = [](hipStream_t s, hipEvent_t e) {
    return hipStreamWaitEvent(s, e, 0) == hipSuccess ? TRNBLAS_OK : TRNBLAS_E_LAUNCH;
  };
  auto record = [](hipEvent_t e, hipStream_t s) {
    return hipEventRecord(e, s) == hipSuccess ? TRNBLAS_OK : TRNBLAS_E_LAUNCH;
  };

  // W = J zero-padded; Y = 0 (the last block's padding stays 0); info = 0
  TRY(fill(W, npad, npad, npad, 0.0, main));
  hipLaunchKernelGGL((copy2d_kernel<double, double>), grid2d(n, n), dim3(256), 0, main, n, n, J,
                     ldj, (int64_t)1, W, npad, (int64_t)1, 1.0);
  TRY(check_launch("metric_inv_half(copy)"));
  TRY(fill(Y, npad, npad, npad, 0.0, main));
  hipLaunchKernelGGL(set_i32_kernel, dim3(1), dim3(1), 0, main, info, 0);
  TRY(check_launch("metric_inv_half(info)"));

  bool rest = false, inv = false;  // the side / inverse stream has work pending
  for (int64_t b = 0; b < nblk; ++b) {
    const int64_t k0 = b * kNB, m = n - k0 < kNB ? n - k0 : kNB;
    double* Ybb = Y + k0 * npad + k0;
    // L_bb into W (lower triangle), L_bb^-1 = Y_bb straight into Y
    TRY(trnblas_hip_chol_block(m, W + k0 * npad + k0, npad, Ybb, npad, info, k0, main));
    // block row b of Y: T = L[b, :b] Y[:b, :b], Y[b, :b] = -Y_bb T, on the
    // inverse stream once `ready` (recorded after this step's GEMMs on the
    // caller's stream, or right here in the last step) follows Y_bb
    auto inv_row = [&]() -> int {
      if (b == 0) return TRNBLAS_OK;
      TRY(wait(ss->inv, ss->ready));
      TRY(trnblas_hip_dgemm(0, 0, kNB, k0, k0, 1.0, L + k0 * npad, npad, 0, Y, npad, 0, 0.0,
                            nullptr, npad, 0, T, npad, 0, 1, 0, TRNBLAS_TRI_B_LOWER, ss->inv));
      TRY(trnblas_hip_dgemm(0, 0, kNB, k0, kNB, -1.0, Ybb, npad, 0, T, npad, 0, 0.0, nullptr,
                            npad, 0, Y + k0 * npad, npad, 0, 1, 0, TRNBLAS_TRI_A_LOWER, ss->inv));
      inv = true;
      return TRNBLAS_OK;
    };
    if (k0 + kNB >= npad) {
      if (b > 0) TRY(record(ss->ready, main));
      TRY(inv_row());
      break;
    }
    const int64_t k1 = k0 + kNB, k2 = k1 + kNB, rows = npad - k1;
    // the panel of L: L[k1:, k0:k1] = W[k1:, k0:k1] Y_bb^T
    TRY(trnblas_hip_dgemm(0, 1, rows, kNB, kNB, 1.0, W + k1 * npad + k0, npad, 0, Ybb, npad, 0,
                          0.0, nullptr, npad, 0, L + k1 * npad + k0, npad, 0, 1, 0, 0, main));
    if (rest) TRY(wait(main, ss->done));
    rest = false;
    // the next block column: W[k1:, k1:k2] -= P P[:128]^T
    TRY(trnblas_hip_dgemm(0, 1, rows, kNB, kNB, -1.0, L + k1 * npad + k0, npad, 0,
                          L + k1 * npad + k0, npad, 0, 1.0, W + k1 * npad + k1, npad, 0,
                          W + k1 * npad + k1, npad, 0, 1, 0, 0, main));
    // one event for both: the side stream's trailing update and the
    // inverse stream's block row (one record per step fewer on the host)
    if (k2 < npad || b > 0) TRY(record(ss->ready, main));
    TRY(inv_row());
    if (k2 < npad) {
      const int64_t r2 = npad - k2;
      const double* R = L + k2 * npad + k0;
      double* Wt = W + k2 * npad + k2;
      TRY(wait(ss->side, ss->ready));
      TRY(trnblas_hip_dgemm(0, 1, r2, r2, kNB, -1.0, R, npad, 0, R, npad, 0, 1.0, Wt, npad, 0, Wt,
                            npad, 0, 1, 1, 0, ss->side));
      TRY(record(ss->done, ss->side));
      rest = true;
    }
  }
  if (rest) TRY(wait(main, ss->done));
  if (inv) {
    TRY(record(ss->inverted, ss->inv));
    TRY(wait(main, ss->inverted));
  }
  const unsigned tb = (unsigned)((n + 63) / 64);
  hipLaunchKernelGGL(transpose_kernel, dim3(tb, tb), dim3(256), 0, main, (int)n, Y, npad, X, ldx);
  return check_launch("metric_inv_half(transpose)");
}

// ── trsm ─────────────────────────────────────────────────────────────────────

static void trsm_layout(int dtype, int64_t n, int64_t nrhs, int64_t& nblk, int64_t& npad,
                        int64_t& mp, size_t off[5]) {
  const size_t es = dtype == TRNBLAS_F64 ? 8 : 4;
  nblk = (n + kNB - 1) / kNB;
  npad = nblk * kNB;
  mp = nrhs + (nrhs & 1);
  auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
  off[0] = 0;                                            // Dinv
  off[1] = up(off[0] + (size_t)nblk * kNB * kNB * es);   // T, padded copy
  off[2] = up(off[1] + (size_t)npad * npad * es);        // R, the running right-hand side
  off[3] = up(off[2] + (size_t)npad * mp * es);          // X, padded
  off[4] = up(off[3] + (size_t)npad * mp * es);          // fp32 GEMM workspace
}

extern "C" size_t trnblas_hip_gemm_workspace(void);

extern "C" size_t trnblas_hip_trsm_workspace(int dtype, int64_t n, int64_t nrhs) {
  if (n <= 0 || nrhs <= 0 || (dtype != TRNBLAS_F32 && dtype != TRNBLAS_F64)) return 0;
  int64_t nblk, npad, mp;
  size_t off[5];
  trsm_layout(dtype, n, nrhs, nblk, npad, mp, off);
  return off[4] + (dtype == TRNBLAS_F32 ? trnblas_hip_gemm_workspace() : 0);
}

namespace trnblas {

struct TrsmCtx {
  int dtype, upper;
  int64_t npad, mp;
  char *Dinv, *T, *R, *X, *gws;
  size_t gws_bytes;
  hipStream_t s;
  size_t es;
  // element pointers
  char* at(char* base, int64_t i, int64_t j, int64_t ld) const {
    return base + (size_t)(i * ld + j) * es;
  }
  // D = alpha A B + beta C (C may be D), row-major operands of this solve
  int mm(int64_t M, int64_t N, int64_t K, double alpha, const char* A, int64_t lda,
         const char* B, int64_t ldb, double beta, char* D, int64_t ldd, int tri) const {
    if (dtype == TRNBLAS_F64)
      return trnblas_hip_dgemm(0, 0, M, N, K, alpha, reinterpret_cast<const double*>(A), lda, 0,
                               reinterpret_cast<const double*>(B), ldb, 0, beta,
                               reinterpret_cast<const double*>(D), ldd, 0,
                               reinterpret_cast<double*>(D), ldd, 0, 1, 0, tri, s);
    return trnblas_hip_gemm(TRNBLAS_F32, 0, 0, M, N, K, alpha, A, lda, 0, B, ldb, 0, beta, D, ldd, 0,
                            D, ldd, 0, 1, gws, gws_bytes, s);
  }
  // blocks [b0, b1): X rows from R rows (R is consumed)
  int solve(int64_t b0, int64_t b1) const {
    if (b1 - b0 == 1) {
      const int64_t r = b0 * kNB;
      return mm(kNB, mp, kNB, 1.0, Dinv + (size_t)b0 * kNB * kNB * es, kNB, at(R, r, 0, mp), mp, 0.0,
                at(X, r, 0, mp), mp, upper ? TRNBLAS_TRI_A_UPPER : TRNBLAS_TRI_A_LOWER);
    }
    const int64_t bm = (b0 + b1) / 2, lo = b0 * kNB, mid = bm * kNB, hi = b1 * kNB;
    if (!upper) {  // forward: the first half, then the rest of R
      TRY(solve(b0, bm));
      TRY(mm(hi - mid, mp, mid - lo, -1.0, at(T, mid, lo, npad), npad, at(X, lo, 0, mp), mp, 1.0,
             at(R, mid, 0, mp), mp, 0));
      return solve(bm, b1);
    }
    TRY(solve(bm, b1));  // backward: the second half first
    TRY(mm(mid - lo, mp, hi - mid, -1.0, at(T, lo, mid, npad), npad, at(X, mid, 0, mp), mp, 1.0,
           at(R, lo, 0, mp), mp, 0));
    return solve(b0, bm);
  }
};

template <typename E>
static int trsm_copies(int64_t n, int64_t nrhs, double alpha, const void* T, int64_t tr, int64_t tc,
                       const void* B, int64_t br, int64_t bc, const TrsmCtx& c) {
  hipLaunchKernelGGL((copy2d_kernel<E, E>), grid2d(n, n), dim3(256), 0, c.s, n, n,
                     static_cast<const E*>(T), tr, tc, reinterpret_cast<E*>(c.T), c.npad,
                     (int64_t)1, 1.0);
  TRY(check_launch("trsm(copy T)"));
  hipLaunchKernelGGL((copy2d_kernel<E, E>), grid2d(n, nrhs), dim3(256), 0, c.s, n, nrhs,
                     static_cast<const E*>(B), br, bc, reinterpret_cast<E*>(c.R), c.mp, (int64_t)1,
                     alpha);
  return check_launch("trsm(copy B)");
}

template <typename E>
__global__ __launch_bounds__(256) void fill_t_kernel(E* p, int64_t n) {
  for (int64_t x = blockIdx.x * 256ll + threadIdx.x; x < n; x += (int64_t)gridDim.x * 256) p[x] = E(0);
}

}  // namespace trnblas

extern "C" int trnblas_hip_trsm(int dtype, int64_t n, int64_t nrhs, int upper, int unit,
                                double alpha, const void* T, int64_t ldt_r, int64_t ldt_c,
                                const void* B, int64_t ldb_r, int64_t ldb_c, void* X,
                                int64_t ldx_r, int64_t ldx_c, void* workspace,
                                size_t workspace_bytes, void* stream) {
  clear_error();
  TRNBLAS_CHECK_ARG(dtype == TRNBLAS_F32 || dtype == TRNBLAS_F64, "trsm: dtype %d not supported",
                    dtype);
  TRNBLAS_CHECK_ARG(n >= 0 && nrhs >= 0 && n < (1ll << 20) && nrhs < (1ll << 30),
                    "trsm: bad sizes");
  if (n == 0 || nrhs == 0) return TRNBLAS_OK;
  TRNBLAS_CHECK_ARG(T && B && X && workspace, "trsm: NULL pointer");
  TRNBLAS_CHECK_ARG(ldt_r > 0 && ldt_c > 0 && ldb_r > 0 && ldb_c > 0 && ldx_r > 0 && ldx_c > 0,
                    "trsm: strides must be positive");
  const size_t need = trnblas_hip_trsm_workspace(dtype, n, nrhs);
  TRNBLAS_CHECK_ARG(workspace_bytes >= need, "trsm: workspace %zu bytes, %zu needed",
                    workspace_bytes, need);
  TRNBLAS_CHECK_ARG((reinterpret_cast<uintptr_t>(workspace) & 255) == 0,
                    "trsm: workspace must be 256-byte aligned");
  TrsmCtx c{};
  int64_t nblk;
  size_t off[5];
  trsm_layout(dtype, n, nrhs, nblk, c.npad, c.mp, off);
  char* ws = static_cast<char*>(workspace);
  c.dtype = dtype;
  c.upper = upper != 0;
  c.es = dtype == TRNBLAS_F64 ? 8 : 4;
  c.Dinv = ws + off[0];
  c.T = ws + off[1];
  c.R = ws + off[2];
  c.X = ws + off[3];
  c.gws = ws + off[4];
  c.gws_bytes = workspace_bytes - off[4];
  c.s = (hipStream_t)stream;
  // zero T, R (their padding takes part in the products) and X
  const int64_t zero_elems = (int64_t)((off[4] - off[1]) / c.es);
  if (dtype == TRNBLAS_F64)
    hipLaunchKernelGGL(fill_t_kernel<double>, dim3(grid_for(zero_elems)), dim3(256), 0, c.s,
                       reinterpret_cast<double*>(c.T), zero_elems);
  else
    hipLaunchKernelGGL(fill_t_kernel<float>, dim3(grid_for(zero_elems)), dim3(256), 0, c.s,
                       reinterpret_cast<float*>(c.T), zero_elems);
  TRY(check_launch("trsm(fill)"));
  if (dtype == TRNBLAS_F64)
    TRY(trsm_copies<double>(n, nrhs, alpha, T, ldt_r, ldt_c, B, ldb_r, ldb_c, c));
  else
    TRY(trsm_copies<float>(n, nrhs, alpha, T, ldt_r, ldt_c, B, ldb_r, ldb_c, c));
  TRY(trnblas_hip_tri_inv_blocks(dtype, n, upper, unit, T, ldt_r, ldt_c, c.Dinv, stream));
  TRY(c.solve(0, nblk));
  if (dtype == TRNBLAS_F64)
    hipLaunchKernelGGL((copy2d_kernel<double, double>), grid2d(n, nrhs), dim3(256), 0, c.s, n, nrhs,
                       reinterpret_cast<const double*>(c.X), c.mp, (int64_t)1,
                       static_cast<double*>(X), ldx_r, ldx_c, 1.0);
  else
    hipLaunchKernelGGL((copy2d_kernel<float, float>), grid2d(n, nrhs), dim3(256), 0, c.s, n, nrhs,
                       reinterpret_cast<const float*>(c.X), c.mp, (int64_t)1,
                       static_cast<float*>(X), ldx_r, ldx_c, 1.0);
  return check_launch("trsm(copy X)");
}
