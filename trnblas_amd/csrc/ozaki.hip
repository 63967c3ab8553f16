// Ozaki fp64-class GEMM on gfx950: native-fp64 digit split + int8 MFMA slice
// products with exact int32 groups + fp32 TwoSum + fused fp64 recombination.
//
// Arithmetic contract (trnblas/ozaki.py): digits as `split` (:123-219), the
// group cut and order of `schedule` / `diag_groups` (:337-365), the TwoSum of
// `_two_sum32` (:378-386) as folded by `reference_from_digits` (:389-415), and
// `combine` (:418-455). Mode 0 reproduces `reference_gemm` bit for bit.
//
// Design for CDNA4 (not a translation of the NKI kernels,
// trnblas/nki/dispatch.py:3768-4354, which emulate fp64 with bit fields and
// run bf16 matmuls on the Tensor Engine):
//  * the split is plain fp64 (rint chain), one pass per operand, writing
//    int8 digits K-contiguous for both operands (B is transposed on the fly
//    through LDS), so both MFMA operands are 16-byte K-contiguous loads;
//  * slice products run on v_mfma_i32_32x32x32_i8 with int32 accumulation:
//    a group of at most 4096 terms of |d| <= 64 digits sums to at most 2^24,
//    exact in int32 and in fp32;
//  * a 256-thread workgroup owns a 128x128 output tile; per lane it keeps the
//    int32 group accumulators and the fp32 (hi, lo) pairs of its 64 outputs
//    in registers for the whole schedule; the operand tiles are staged in
//    LDS, double buffered, and the k-step pipeline runs straight across
//    group and slice-pair boundaries;
//  * the fp64 recombination (hi + lo) 2^(eA + eB + off) is fused into the
//    store (no (hi, lo) round trip through HBM), including the fp64 sum of K
//    blocks for very long K (`plan`'s K blocking).
#include <algorithm>
#include <type_traits>

#include "common.hpp"

namespace trnblas {

constexpr int kSliceBits = 7;
constexpr int kTileK = 128;     // K tile of the schedule
constexpr int kGroupTiles = 32;  // 4096 terms
constexpr int kNonFinite = (int)0x80000000;

// ---------------------------------------------------------------------------
// split

// frexp exponent of |x| (x finite, >= 0): x < 2^e, 0 -> 0.
__device__ __forceinline__ int frexp_exp(double x) {
  int e = 0;
  (void)frexp(x, &e);
  return x == 0.0 ? 0 : e;
}

// Exponent of the largest |x| of each row (per_row) or column; non-finite
// rows / columns get kNonFinite.
__global__ __launch_bounds__(256) void oz_emax_row_kernel(const double* X, int64_t ldx, int R,
                                                          int C, int32_t* exps) {
  __shared__ double smax[4];
  __shared__ int sbad[4];
  const int r = blockIdx.x;
  const double* row = X + (int64_t)r * ldx;
  double m = 0.0;
  int bad = 0;
  for (int c = threadIdx.x; c < C; c += blockDim.x) {
    const double v = fabs(row[c]);
    bad |= !isfinite(v);
    m = v > m ? v : m;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const double o = __shfl_xor(m, off, 64);
    m = o > m ? o : m;
    bad |= __shfl_xor(bad, off, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    smax[threadIdx.x >> 6] = m;
    sbad[threadIdx.x >> 6] = bad;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double mm = 0.0;
    int bb = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
      mm = smax[w] > mm ? smax[w] : mm;
      bb |= sbad[w];
    }
    exps[r] = bb ? kNonFinite : frexp_exp(mm);
  }
}

// Column maxima: a 64-column strip x 256-row chunk per workgroup, 4 row lanes
// per column; the chunk's exponent (frexp is monotonic in |x|) goes into
// exps[c] by atomicMax, a non-finite chunk as kEmaxBad (turned into
// kNonFinite by oz_flags_kernel). exps must hold INT_MIN beforehand.
constexpr int kEmaxRows = 256;
constexpr int kEmaxBad = 0x7fffffff;

__global__ __launch_bounds__(256) void oz_fill_kernel(int32_t* p, int n, int32_t v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__global__ __launch_bounds__(256) void oz_emax_col_kernel(const double* X, int64_t ldx, int R,
                                                          int C, int32_t* exps) {
  __shared__ double smax[4][64];
  __shared__ int sbad[4][64];
  const int cx = threadIdx.x & 63, ry = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + cx;
  const int r0 = blockIdx.y * kEmaxRows, r1 = min(R, r0 + kEmaxRows);
  double m = 0.0;
  int bad = 0;
  if (c < C) {
    for (int r = r0 + ry; r < r1; r += 4) {
      const double v = fabs(X[(int64_t)r * ldx + c]);
      bad |= !isfinite(v);
      m = v > m ? v : m;
    }
  }
  smax[ry][cx] = m;
  sbad[ry][cx] = bad;
  __syncthreads();
  if (ry == 0 && c < C) {
    for (int k = 1; k < 4; ++k) {
      m = smax[k][cx] > m ? smax[k][cx] : m;
      bad |= sbad[k][cx];
    }
    atomicMax(&exps[c], bad ? kEmaxBad : frexp_exp(m));
  }
}

// flags[0] = 1 when some shift 6 - e is not a normal exponent (the global
// two-factor scaling of ozaki.py:185-188); flags[1] = 1 on non-finite input.
// A column exponent of kEmaxBad (non-finite) is rewritten as kNonFinite.
__global__ __launch_bounds__(1024) void oz_flags_kernel(int32_t* exps, int n, int32_t* flags) {
  __shared__ int s2[16], sn[16];
  int two = 0, nf = 0;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int e = exps[i];
    if (e == kNonFinite || e == kEmaxBad) {
      if (e == kEmaxBad) exps[i] = kNonFinite;
      nf = 1;
    } else {
      const int sh = (kSliceBits - 1) - e;
      two |= (sh > 1023 || sh < -1022);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    two |= __shfl_xor(two, off, 64);
    nf |= __shfl_xor(nf, off, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    s2[threadIdx.x >> 6] = two;
    sn[threadIdx.x >> 6] = nf;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int a = 0, b = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
      a |= s2[w];
      b |= sn[w];
    }
    flags[0] = a;
    flags[1] = b;
  }
}

__device__ __forceinline__ double pow2(int n) {  // n a normal exponent
  return __longlong_as_double((long long)(n + 1023) << 52);
}

__device__ __forceinline__ int floor_div2(int v) { return v >= 0 ? v / 2 : -((1 - v) / 2); }

// The k digits of x for exponent e (ozaki.py:191-217), as int8 into d[].
template <int KMAX>
__device__ __forceinline__ void digits_of(double x, int e, int k, bool two, int8_t* d) {
  const int sh = (kSliceBits - 1) - e;
  double rem;
  if (two) {
    const int h = floor_div2(sh);
    rem = x * pow2(h);
    rem = rem * pow2(sh - h);
  } else {
    rem = x * pow2(sh);
  }
#pragma unroll
  for (int s = 0; s < KMAX; ++s) {
    if (s < k) {
      if (s) rem = rem * 128.0;
      const double q = rint(rem);
      if (s + 1 < k) rem = rem - q;
      d[s] = (int8_t)(int)q;
    }
  }
}

// Row split: X (R, C) row-major, one exponent per row, digits
// out[s*ld_slice + r*ld_digit + c]. A workgroup covers 1024 columns of one
// row, each thread 4 consecutive columns: loads and the 4-byte digit stores
// of a wave are contiguous.
__global__ __launch_bounds__(256) void oz_digits_row_kernel(const double* X, int64_t ldx, int R,
                                                            int C, int k, const int32_t* exps,
                                                            const int32_t* flags, int8_t* out,
                                                            int64_t ld_digit, int64_t ld_slice,
                                                            int il) {
  const int cgs = (C + 1023) / 1024;
  const int64_t r = blockIdx.x / cgs;
  const int c0 = (int)(blockIdx.x - r * cgs) * 1024 + 4 * (int)threadIdx.x;
  if (c0 >= C) return;
  const int e = exps[r];
  if (e == kNonFinite) return;
  const bool two = flags[0] != 0;
  const double* src = X + r * ldx + c0;
  double x[4];
  if (c0 + 4 <= C && ((reinterpret_cast<uintptr_t>(src) & 15) == 0)) {
    const double2 a = *reinterpret_cast<const double2*>(src);
    const double2 b = *reinterpret_cast<const double2*>(src + 2);
    x[0] = a.x;
    x[1] = a.y;
    x[2] = b.x;
    x[3] = b.y;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = c0 + i < C ? src[i] : 0.0;
  }
  union {
    int8_t b[4];
    int w;
  } u[12];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int8_t d[12];
    digits_of<12>(x[i], e, k, two, d);
#pragma unroll
    for (int s = 0; s < 12; ++s) u[s].b[i] = s < k ? d[s] : 0;
  }
  for (int s = 0; s < k; ++s) {
    int8_t* dst = il ? out + r * ld_digit + (int64_t)(c0 >> 5) * 32 * k + s * 32 + (c0 & 31)
                     : out + (int64_t)s * ld_slice + r * ld_digit + c0;
    if (c0 + 4 <= C && ((uintptr_t)dst & 3) == 0) {
      *reinterpret_cast<int*>(dst) = u[s].w;
    } else {
      for (int i = 0; i < 4 && c0 + i < C; ++i) dst[i] = u[s].b[i];
    }
  }
}

// Column split, written transposed: X (R, C) row-major, one exponent per
// column c, digits out[s*ld_slice + c*ld_digit + r] (R contiguous). 64 x 64
// tiles through LDS: reads are coalesced along c, writes along r.
__global__ __launch_bounds__(256) void oz_digits_col_kernel(const double* X, int64_t ldx, int R,
                                                            int C, int k, const int32_t* exps,
                                                            const int32_t* flags, int8_t* out,
                                                            int64_t ld_digit, int64_t ld_slice,
                                                            int il) {
  // Block: 64 columns x 64 rows of X. Thread t: column c0 + t / 4, rows
  // r0 + 16 (t % 4) .. +15. Both digit layouts keep a thread's 16 rows of
  // one (slice, column) as 16 contiguous, 16-byte aligned bytes, so each
  // thread writes a slice with one 16-byte store (no transpose through LDS).
  const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
  const int c = c0 + (threadIdx.x >> 2), rq = (threadIdx.x & 3) * 16;
  if (c >= C) return;
  const int e = exps[c];
  if (e == kNonFinite) return;
  const bool two = flags[0] != 0;
  // digit bytes packed into words with static indices only (a byte union
  // indexed by the runtime slice count goes to scratch memory)
  uint32_t u[12][4];
#pragma unroll
  for (int s = 0; s < 12; ++s)
#pragma unroll
    for (int q = 0; q < 4; ++q) u[s][q] = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = r0 + rq + i;
    int8_t d[12];
    const double x = r < R ? X[(int64_t)r * ldx + c] : 0.0;
    digits_of<12>(x, e, k, two, d);
#pragma unroll
    for (int s = 0; s < 12; ++s) u[s][i >> 2] |= (uint32_t)(uint8_t)(s < k ? d[s] : 0) << (8 * (i & 3));
  }
  const bool full = r0 + rq + 16 <= R;
#pragma unroll
  for (int s = 0; s < 12; ++s) {
    if (s < k) {
      const int rr = r0 + rq;
      int8_t* dst = il ? out + (int64_t)c * ld_digit + (int64_t)(rr >> 5) * 32 * k + s * 32 + (rr & 31)
                       : out + (int64_t)s * ld_slice + (int64_t)c * ld_digit + rr;
      if (full && (((uintptr_t)dst) & 15) == 0) {
        *reinterpret_cast<i32x4*>(dst) =
            i32x4{(int)u[s][0], (int)u[s][1], (int)u[s][2], (int)u[s][3]};
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (r0 + rq + i < R) dst[i] = (int8_t)(u[s][i >> 2] >> (8 * (i & 3)));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// slice GEMM

struct OzArgs {
  int k;         // slices
  int M, N;
  int Kp, kb;    // padded K, K block (multiples of 128)
  const int8_t* A;
  int64_t lda, lda_s;
  const int8_t* B;
  int64_t ldb, ldb_s;
  const int32_t* eA;
  const int32_t* eB;
  double* C;      // combine target (mode 0 / 1), or
  float* hilo;    // raw (hi, lo) planes (hilo output)
  int64_t ldc_m, ldc_n, ldh;
  int tiles_m, tiles_n;
  int flush;      // fast mode: k-steps between int32 -> fp64 flushes of the diagonals
  int64_t hl_rs, hl_cs, hl_lo;  // oz_exact_kernel: (hi, lo) output strides (floats)
  int fuse;                     // oz_exact_kernel: combine into C in the epilogue
};

// The fp64 recombination of one exact-mode element (ozaki.py:418-455,
// `combine`): ((double) hi + (double) lo) 2^(eA + off) 2^eB.
__device__ __forceinline__ double oz_combine(float hi, float lo, int ea_raw, int eb, int k);

__device__ __forceinline__ void two_sum32(float& hi, float& lo, float p) {
#pragma clang fp contract(off)
  const float s = hi + p;
  const float bb = s - hi;
  const float t = s - bb;
  const float e = (hi - t) + (p - bb);
  hi = s;
  lo = lo + e;
}

constexpr uint32_t kOzOob = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t oz_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7ffffff0,
                                           0x00020000);
}

// (d, s, kstep) walk of the schedule: diagonals d = k-1 .. 0, pairs
// s = 0 .. d (t = d - s), k-steps of BK bytes over the K block.
struct OzStep {
  int d, s, ks;
};

// Exact mode over K blocks (`plan`'s K blocking, K beyond ~2^16: each block
// its own (hi, lo) chain, the blocks summed in fp64 into C): register-staged
// 64-byte k-steps, one pair's tiles per step. Single-block calls take
// oz_exact_kernel.
template <int BM, int BN, int BK, int OUT>  // OUT: 0 combine into C, 1 raw hilo
__global__ __launch_bounds__(256) void oz_gemm_kernel(OzArgs g) {
  constexpr int NT = 256;
  constexpr int WM = BM / 2, WN = BN / 2;  // 2 x 2 waves
  constexpr int FM = WM / 32, FN = WN / 32;
  constexpr int LD = BK + 16;  // padded LDS row (bytes)
  constexpr int A_SZ = BM * LD, B_SZ = BN * LD;
  constexpr int NVA = BM * BK / 16 / NT, NVB = BN * BK / 16 / NT;
  static_assert(NVA * 16 * NT == BM * BK && NVB * 16 * NT == BN * BK, "tile split");
  constexpr int SUB = kTileK / BK;  // k-steps per 128-K tile
  __shared__ __attribute__((aligned(16))) int8_t lds[2 * (A_SZ + B_SZ)];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  int tm, tn;
  grouped_tile(t, g.tiles_m, g.tiles_n, 8, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int k = g.k;
  const int nkb = (g.Kp + g.kb - 1) / g.kb;  // the last block may be shorter
  const int npairs = k * (k + 1) / 2;
  // per K block: 128-tiles per slice, and the group cut that follows from it
  int kt = 0, steps_per_pair = 0, total = 0, per = 1;

  i32x4 ra[NVA], rb[NVB];
  int kbase = 0;
  auto load = [&](const OzStep& st) {
    const int tt = st.d - st.s;
    const int64_t koff = kbase + (int64_t)st.ks * BK;
    const __amdgpu_buffer_rsrc_t rsa = oz_rsrc(g.A + st.s * g.lda_s + (int64_t)m0 * g.lda + koff);
    const __amdgpu_buffer_rsrc_t rsb = oz_rsrc(g.B + tt * g.ldb_s + (int64_t)n0 * g.ldb + koff);
#pragma unroll
    for (int i = 0; i < NVA; ++i) {
      const int idx = tid + i * NT, r = idx / (BK / 16), c = (idx % (BK / 16)) * 16;
      const uint32_t off = (uint32_t)(r * g.lda + c);
      ra[i] = __builtin_amdgcn_raw_buffer_load_b128(rsa, m0 + r < g.M ? off : kOzOob, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < NVB; ++i) {
      const int idx = tid + i * NT, r = idx / (BK / 16), c = (idx % (BK / 16)) * 16;
      const uint32_t off = (uint32_t)(r * g.ldb + c);
      rb[i] = __builtin_amdgcn_raw_buffer_load_b128(rsb, n0 + r < g.N ? off : kOzOob, 0, 0);
    }
  };
  auto store = [&](int buf) {
    int8_t* la = lds + buf * (A_SZ + B_SZ);
    int8_t* lb = la + A_SZ;
#pragma unroll
    for (int i = 0; i < NVA; ++i) {
      const int idx = tid + i * NT, r = idx / (BK / 16), c = (idx % (BK / 16)) * 16;
      *reinterpret_cast<i32x4*>(la + r * LD + c) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < NVB; ++i) {
      const int idx = tid + i * NT, r = idx / (BK / 16), c = (idx % (BK / 16)) * 16;
      *reinterpret_cast<i32x4*>(lb + r * LD + c) = rb[i];
    }
  };
  auto advance = [&](OzStep st) {
    if (++st.ks == steps_per_pair) {
      st.ks = 0;
      if (++st.s > st.d) {
        st.s = 0;
        --st.d;
      }
    }
    return st;
  };
  // True when the step just computed closes a group (ozaki.py:337-355).
  auto group_end = [&](const OzStep& st) {
    if (st.ks % SUB != SUB - 1) return false;
    const int tile = st.ks / SUB;
    if (kt >= kGroupTiles) return (tile + 1) % kGroupTiles == 0 || tile + 1 == kt;
    return tile + 1 == kt && ((st.s + 1) % per == 0 || st.s == st.d);
  };

  for (int kbi = 0; kbi < nkb; ++kbi) {
    kbase = kbi * g.kb;
    kt = (g.Kp - kbase < g.kb ? g.Kp - kbase : g.kb) / kTileK;
    steps_per_pair = kt * SUB;
    total = npairs * steps_per_pair;
    per = kt >= kGroupTiles ? 1 : kGroupTiles / kt;
    i32x16 acc[FM][FN];
    float hi[FM][FN][16], lo[FM][FN][16];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          acc[i][j][r] = 0;
          hi[i][j][r] = 0.0f;
          lo[i][j][r] = 0.0f;
        }
    OzStep cur{k - 1, 0, 0};
    load(cur);
    store(0);
    __syncthreads();
    for (int n = 0; n < total; ++n) {
      const bool more = n + 1 < total;
      const OzStep nxt = advance(cur);
      if (more) load(nxt);
      const int8_t* la = lds + (n & 1) * (A_SZ + B_SZ);
      const int8_t* lb = la + A_SZ;
#pragma unroll
      for (int c = 0; c < BK / 32; ++c) {
        const int kk = c * 32 + (lane >> 5) * 16;
        i32x4 fa[FM], fb[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
          fa[i] = *reinterpret_cast<const i32x4*>(la + (wm0 + i * 32 + (lane & 31)) * LD + kk);
#pragma unroll
        for (int j = 0; j < FN; ++j)
          fb[j] = *reinterpret_cast<const i32x4*>(lb + (wn0 + j * 32 + (lane & 31)) * LD + kk);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
      }
      if (group_end(cur)) {
        const float scale = __int_as_float((127 + kSliceBits * (k - 1 - cur.d)) << 23);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const float pv = (float)acc[i][j][r] * scale;  // exact: |G| <= 2^24
              two_sum32(hi[i][j][r], lo[i][j][r], pv);
              acc[i][j][r] = 0;
            }
      }
      if (more) store((n + 1) & 1);
      __syncthreads();
      cur = nxt;
    }

    // Epilogue (lane l of a 32x32 block: column l % 32, rows
    // 8 (r/4) + 4 (l/32) + r % 4).
    const int off = -2 * (kSliceBits - 1) - kSliceBits * (k - 1);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = n0 + wn0 + j * 32 + (lane & 31);
        const int eb = n < g.N ? (OUT == 0 ? g.eB[n] : 0) : 0;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm0 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
          if (m >= g.M || n >= g.N) continue;
          if (OUT == 1) {
            g.hilo[(int64_t)m * g.ldh + n] = hi[i][j][r];
            g.hilo[(int64_t)g.M * g.ldh + (int64_t)m * g.ldh + n] = lo[i][j][r];
            continue;
          }
          const int ea = g.eA[m] + off;
          const double v = (double)hi[i][j][r] + (double)lo[i][j][r];
          double c;
          if (ea < 900 && ea > -900 && eb < 900 && eb > -900)
            c = (v * pow2(ea)) * pow2(eb);
          else
            c = ldexp(v, ea + eb);
          double* dst = g.C + (int64_t)m * g.ldc_m + (int64_t)n * g.ldc_n;
          *dst = kbi == 0 ? c : *dst + c;
        }
      }
  }
}

// ---------------------------------------------------------------------------
// Fast mode: all slices per k-step, one int32 accumulator per diagonal.
//
// A 64 x 64 output tile per workgroup (4 waves, one 32 x 32 MFMA block each).
// Each BK-wide k-step stages that K slice of every digit slice of A and B in
// LDS (2 x k x 64 rows x BK bytes) and runs all k (k + 1) / 2 slice products
// from it, so one load feeds (k + 1) / 2 MFMAs per slice instead of one.
// Products on diagonal d = s + t share an int32 accumulator: with
// |digit| <= 64 a term is <= 2^12, and the host sets `flush` so that
// k * K_flush * 2^12 < 2^31. At a flush and at the end each diagonal is
// converted to fp64 exactly and summed, scaled by 2^(7 (k-1-d)), smallest
// diagonal first; flushes before the end add into C. The result is the exact
// digit expansion up to fp64 rounding of that sum: within the truncation
// bound of the reference's fp32 TwoSum chain, but not bitwise equal to it.
//
// Operands go from HBM straight into LDS (buffer_load_dwordx4 ... lds: lane l
// of a wave fills the 16 bytes at the wave's LDS base + 16 l; out-of-range
// lanes write zeros), one 1 KiB block of 1024 / BK rows of one slice of one
// operand per instruction, so no registers hold a stage in flight. LDS rows
// are BK bytes with the 16-byte slots XOR-swizzled by the row (lane l of a
// block loads the global group that belongs in its slot), so 16-byte
// fragment reads of 8 or 16 consecutive rows hit distinct banks; each row is
// one BK-byte request.
template <int BK>
__device__ __forceinline__ int oz_slot(int r, int c) {
  return BK == 64 ? c ^ (((r >> 1) ^ (r >> 2)) & 3) : c ^ (((r >> 2) ^ (r >> 3)) & 1);
}

// KS: the slice count (a template parameter, so the k (k + 1) / 2 MFMAs of a
// k-step are straight-line code). BK = 64 for k <= 8, 32 above. NB LDS
// stages: 2 (double buffered, one workgroup per CU) or 1 (the load of step
// s + 1 waits for every wave to finish step s; two workgroups per CU cover
// each other's loads).
template <int KS, int BK, int NB>
__global__ __launch_bounds__(256, NB == 1 ? 2 : 1) void oz_fast_kernel(OzArgs g) {
  constexpr int T = 64;
  constexpr int SL = T * BK;       // bytes per slice tile
  constexpr int OP = KS * SL;      // bytes per operand stage
  constexpr int STAGE = 2 * OP;
  constexpr int RPI = 1024 / BK;   // rows per 1 KiB load instruction
  constexpr int IPS = T / RPI;     // instructions per slice tile
  constexpr int GPR = BK / 16;     // 16-byte groups per row
  __shared__ __attribute__((aligned(16))) int8_t lds[NB * STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  int tm, tn;
  grouped_tile(t, g.tiles_m, g.tiles_n, 8, tm, tn);
  const int m0 = tm * T, n0 = tn * T;
  constexpr int k = KS;
  const int nsteps = g.Kp / BK;

  // Wave w loads row block w % IPS of the slices sl with sl % (4 / IPS) ==
  // w / IPS, of both operands: one instruction per (operand, slice).
  constexpr int WPB = 4 / IPS;  // waves sharing one row block
  const int blk = w % IPS, jw = w / IPS;
  const int r = blk * RPI + lane / GPR;
  const int cg = oz_slot<BK>(r, lane % GPR);  // the slot map is its own inverse
  const uint32_t voffA = m0 + r < g.M ? (uint32_t)(r * g.lda + 16 * cg) : kOzOob;
  const uint32_t voffB = n0 + r < g.N ? (uint32_t)(r * g.ldb + 16 * cg) : kOzOob;
  const int8_t* baseA = g.A + (int64_t)m0 * g.lda;
  const int8_t* baseB = g.B + (int64_t)n0 * g.ldb;
  auto load = [&](int step, int buf) {
    const int64_t koff = (int64_t)step * BK;
#pragma unroll
    for (int sl = 0; sl < KS; ++sl)
      if (sl < k && sl % WPB == jw) {
        int8_t* dst = lds + buf * STAGE + sl * SL + blk * 1024;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            oz_rsrc(baseA + sl * g.lda_s + koff), (__attribute__((address_space(3))) void*)dst,
            16, voffA, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            oz_rsrc(baseB + sl * g.ldb_s + koff),
            (__attribute__((address_space(3))) void*)(dst + OP), 16, voffB, 0, 0, 0);
      }
  };

  // Wave w: rows 32 (w & 1), columns 32 (w >> 1) of the tile. Lane l reads
  // row l % 32 of its block, bytes 16 (l / 32) .. +15 of each 32-wide chunk.
  const int ar = 32 * (w & 1) + (lane & 31), br = 32 * (w >> 1) + (lane & 31);
  i32x16 acc[KS];
#pragma unroll
  for (int d = 0; d < KS; ++d)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[d][e] = 0;

  // Lane l of a 32x32 block: column l % 32, rows 8 (e/4) + 4 (l/32) + e % 4.
  const int off = -2 * (kSliceBits - 1) - kSliceBits * (k - 1);
  const int n = n0 + 32 * (w >> 1) + (lane & 31);
  const int eb = n < g.N ? g.eB[n] : 0;
  auto flush = [&](bool first) {
    // Convert (all accumulators die here), then scale and store.
    double v[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      v[e] = 0.0;
#pragma unroll
      for (int d = KS - 1; d >= 0; --d)
        if (d < k) v[e] += (double)acc[d][e] * pow2(kSliceBits * (k - 1 - d));
    }
#pragma unroll
    for (int d = 0; d < KS; ++d)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[d][e] = 0;
#pragma unroll 4
    for (int e = 0; e < 16; ++e) {
      const int m = m0 + 32 * (w & 1) + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
      if (m >= g.M || n >= g.N) continue;
      const int ea = g.eA[m] + off;
      double cv;
      if (ea < 900 && ea > -900 && eb < 900 && eb > -900)
        cv = (v[e] * pow2(ea)) * pow2(eb);
      else
        cv = ldexp(v[e], ea + eb);
      double* dst = g.C + (int64_t)m * g.ldc_m + (int64_t)n * g.ldc_n;
      *dst = first ? cv : *dst + cv;
    }
  };

  // K in blocks of `flush` steps; each block drains its pipeline and then
  // flushes (C5-size K is one block). A stage is complete when every wave
  // has waited for its own loads (vmcnt) and passed the barrier.
  for (int s0 = 0; s0 < nsteps; s0 += g.flush) {
    const int s1 = s0 + g.flush < nsteps ? s0 + g.flush : nsteps;
    if (s0 > 0) __syncthreads();  // the previous block's last stage is consumed
    if (NB == 2) {
      load(s0, 0);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
    for (int s = s0; s < s1; ++s) {
      int cur = 0;
      if (NB == 2) {
        if (s + 1 < s1) load(s + 1, (s + 1 - s0) & 1);
        cur = (s - s0) & 1;
      } else {
        // one stage: the other workgroup on the CU computes while this
        // one's loads are in flight
        if (s > s0) __syncthreads();  // every wave is done with the stage
        load(s, 0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
      }
      const int8_t* buf = lds + cur * STAGE;
#pragma unroll
      for (int ch = 0; ch < BK / 32; ++ch) {
        const int c = 2 * ch + (lane >> 5);
        // byte of slice s2's group c of this lane's A / B row
        auto fofs = [&](int row, int s2) { return s2 * SL + row * BK + 16 * oz_slot<BK>(row, c); };
        i32x4 fa[KS];
#pragma unroll
        for (int s2 = 0; s2 < KS; ++s2)
          if (s2 < k) fa[s2] = *reinterpret_cast<const i32x4*>(buf + fofs(ar, s2));
#pragma unroll
        for (int tt = 0; tt < KS; ++tt)
          if (tt < k) {
            const i32x4 fb = *reinterpret_cast<const i32x4*>(buf + OP + fofs(br, tt));
#pragma unroll
            for (int s2 = 0; s2 < KS - tt; ++s2)
              if (s2 + tt < k)
                acc[s2 + tt] =
                    __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[s2], fb, acc[s2 + tt], 0, 0, 0);
          }
      }
      if (NB == 2) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
      }
    }
    flush(s0 == 0);
  }
  if (nsteps == 0) flush(true);
}

// Fast mode on interleaved digits of any slice count KS (1..12): row r's
// 32-wide K chunk kc holds the KS slices' 32 bytes side by side at
// r * ld + kc * 32 KS + s * 32 (trnblas_hip_ozaki_split, per_row bit 1), so
// a k-step of a row is 32 KS contiguous bytes.
//
// A 64 x 64 output tile per workgroup, 4 waves with one 32 x 32 MFMA block
// and KS int32 diagonal accumulators each (the arithmetic and bits of
// oz_fast_kernel), K steps of 32 through two LDS stages. A step reads every
// fragment it needs into registers first and only then issues the DMA of
// the next step into the other stage, so no LDS read is ordered after an
// outstanding LDS DMA (which would make it wait for all of them) and the
// DMA lands while the step's KS (KS + 1) / 2 MFMAs run. Up to 9 slices the
// accumulators and fragments (24 KS VGPRs) leave two waves per SIMD; above,
// one (a second fragment set read ahead of the MFMAs measured slower: 27.1
// against 25.8 ms at C5, k = 10).
//
// LDS rows are 2 KS + 1 groups of 16 bytes (one pad group): with an odd
// pitch the 16 consecutive rows of a fragment read fall on 16 distinct bank
// groups. A panel is loaded as consecutive 1 KiB DMA blocks: lane l of
// block b fills slot q = 64 b + l, i.e. group q % (2 KS + 1) of row
// q / (2 KS + 1); pad slots and rows outside the matrix read zeros without a
// memory access.
//
// KS = 10 is laid out to keep two workgroups per CU ("LZ"): rows of 2 KS =
// 20 groups with no pad, group j of row r in slot j ^ ((r >> 2) & 3) (the
// 16 rows of a fragment read: 4 (r % 4) + the XOR term covers 16 distinct
// bank groups), so a stage is 40 KiB and two workgroups fit the 160 KiB of
// LDS; and B's fragments are read one slice ahead of their MFMAs instead of
// all at once (accumulators 160 + A fragments 40 + B 8 VGPRs fit the 256 of
// two waves per SIMD). Those reads follow the next step's DMA, so that DMA
// is issued by inline asm (lds_dma16_asm) and waited for explicitly.
template <int KS>
__global__ __launch_bounds__(256, KS <= 10 ? 2 : 1) void oz_fast_ilk_kernel(OzArgs g) {
  constexpr int T = 64, W = 4;
  constexpr bool LZ = KS == 10;
  constexpr int RG = 2 * KS, PG = LZ ? RG : RG + 1;  // groups of a row's step, LDS pitch
  constexpr int NIP = (T * PG + 63) / 64;  // 1 KiB DMA blocks per panel
  constexpr int OPA = NIP * 1024, STAGE = 2 * OPA;
  constexpr int PER = (NIP + W - 1) / W;   // blocks per wave, panel and step
  static_assert(!LZ || (RG % 4 == 0 && T * PG % 64 == 0), "LZ layout: 4-group XOR, whole blocks");
  __shared__ __attribute__((aligned(16))) int8_t lds[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  int tm, tn;
  grouped_tile(t, g.tiles_m, g.tiles_n, 8, tm, tn);
  const int m0 = tm * T, n0 = tn * T;
  const int nsteps = g.Kp / 32;

  // wave w moves blocks w, w + W, ... of each panel: per block its lane's
  // row offset and group (or kOzOob)
  uint32_t voffA[PER], voffB[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int q = 64 * (w + u * W) + lane, r = q / PG;
    const int j = LZ ? (q % PG) ^ ((r >> 2) & 3) : q % PG;  // the group slot q holds
    const bool in = j < RG && r < T;
    voffA[u] = (in && m0 + r < g.M) ? (uint32_t)(r * g.lda + 16 * j) : kOzOob;
    voffB[u] = (in && n0 + r < g.N) ? (uint32_t)(r * g.ldb + 16 * j) : kOzOob;
  }
  const int8_t* baseA = g.A + (int64_t)m0 * g.lda;
  const int8_t* baseB = g.B + (int64_t)n0 * g.ldb;
  auto load = [&](int step, int buf) {
    const int soff = step * 32 * KS;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      if (NIP % W != 0 && u + 1 == PER && w + u * W >= NIP) break;
      int8_t* dst = lds + buf * STAGE + (w + u * W) * 1024;
      const uint32_t va = voffA[u], vb = voffB[u];
      if constexpr (LZ) {
        lds_dma16_asm(baseA, dst, va, soff);
        lds_dma16_asm(baseB, dst + OPA, vb, soff);
      } else {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(oz_rsrc(baseA),
                                                 (__attribute__((address_space(3))) void*)dst, 16,
                                                 va, soff, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            oz_rsrc(baseB), (__attribute__((address_space(3))) void*)(dst + OPA), 16, vb, soff, 0,
            0);
      }
    }
  };

  // Wave w: rows 32 (w & 1), columns 32 (w >> 1) of the tile. Lane l reads
  // row l % 32 of its block, bytes 16 (l / 32) .. +15 of each slice's 32.
  // LZ: group 2 s + h sits in slot (2 s + h) ^ x, x = (row >> 2) & 3, i.e.
  // at 32 (s ^ (x >> 1)) + 16 (h ^ (x & 1)): s + x/2 for even s, s - x/2 for
  // odd s (two per-lane bases, the slice offset an immediate).
  const int wm = w & 1, wn = w >> 1;
  const int h = lane >> 5;
  const int x = LZ ? ((lane & 31) >> 2) & 3 : 0;
  const int hx = 16 * (h ^ (x & 1)), x1 = 32 * (x >> 1);
  const int rowA = (32 * wm + (lane & 31)) * 16 * PG + hx;
  const int rowB = OPA + (32 * wn + (lane & 31)) * 16 * PG + hx;
  i32x16 acc[KS];
#pragma unroll
  for (int d = 0; d < KS; ++d)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[d][e] = 0;

  // Lane l of a 32x32 block: column l % 32, rows 8 (e/4) + 4 (l/32) + e % 4.
  constexpr int k = KS;
  const int off = -2 * (kSliceBits - 1) - kSliceBits * (k - 1);
  auto flush = [&](bool first) {
    // (n and B's exponent are formed here, not kept live across the steps)
    const int n = n0 + 32 * wn + (lane & 31);
    const int eb = n < g.N ? g.eB[n] : 0;
    double v[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      v[e] = 0.0;
#pragma unroll
      for (int d = k - 1; d >= 0; --d) v[e] += (double)acc[d][e] * pow2(kSliceBits * (k - 1 - d));
    }
#pragma unroll
    for (int d = 0; d < KS; ++d)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[d][e] = 0;
#pragma unroll 4
    for (int e = 0; e < 16; ++e) {
      const int m = m0 + 32 * wm + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
      if (m >= g.M || n >= g.N) continue;
      const int ea = g.eA[m] + off;
      double cv;
      if (ea < 900 && ea > -900 && eb < 900 && eb > -900)
        cv = (v[e] * pow2(ea)) * pow2(eb);
      else
        cv = ldexp(v[e], ea + eb);
      double* dst = g.C + (int64_t)m * g.ldc_m + (int64_t)n * g.ldc_n;
      *dst = first ? cv : *dst + cv;
    }
  };

  // the fragment of slice s2 from the A (base rowA) or B (rowB) panel
  auto frag = [&](const int8_t* buf, int row, int s2) __attribute__((always_inline)) {
    const int o = LZ ? ((s2 & 1) ? row - x1 : row + x1) : row;
    return *reinterpret_cast<const i32x4*>(buf + o + 32 * s2);
  };
  auto read = [&](const int8_t* buf, i32x4 (&fa)[KS], i32x4 (&fb)[KS]) __attribute__((always_inline)) {
#pragma unroll
    for (int s2 = 0; s2 < KS; ++s2) {
      fa[s2] = frag(buf, rowA, s2);
      fb[s2] = frag(buf, rowB, s2);
    }
  };
  auto mfmas = [&](const i32x4 (&fa)[KS], const i32x4 (&fb)[KS]) __attribute__((always_inline)) {
#pragma unroll
    for (int tt = 0; tt < KS; ++tt)
#pragma unroll
      for (int s2 = 0; s2 < KS - tt; ++s2)
        acc[s2 + tt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[s2], fb[tt], acc[s2 + tt], 0, 0, 0);
  };

  for (int s0 = 0; s0 < nsteps; s0 += g.flush) {
    const int s1 = s0 + g.flush < nsteps ? s0 + g.flush : nsteps;
    if (s0 > 0) __syncthreads();  // every wave is done with the previous block's stages
    load(s0, 0);
    for (int s = s0; s < s1; ++s) {
      const int cur = (s - s0) & 1;
      const int8_t* buf = lds + cur * STAGE;
      if constexpr (LZ) {
        // this wave's DMA of step s has landed, then every wave's has (and
        // every wave is done reading stage cur ^ 1)
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        i32x4 fa[KS];
#pragma unroll
        for (int s2 = 0; s2 < KS; ++s2) fa[s2] = frag(buf, rowA, s2);
        i32x4 fb = frag(buf, rowB, 0);
        if (s + 1 < s1) load(s + 1, cur ^ 1);
#pragma unroll
        for (int tt = 0; tt < KS; ++tt) {
          i32x4 fn = fb;
          if (tt + 1 < KS) fn = frag(buf, rowB, tt + 1);
#pragma unroll
          for (int s2 = 0; s2 < KS - tt; ++s2)
            acc[s2 + tt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[s2], fb, acc[s2 + tt], 0, 0, 0);
          fb = fn;
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
        __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA of step s has landed
        __syncthreads();                // every wave's has; stage cur ^ 1 is free
        i32x4 fa[KS], fb[KS];
        read(buf, fa, fb);
        if (s + 1 < s1) load(s + 1, cur ^ 1);
        mfmas(fa, fb);
      }
    }
    flush(s0 == 0);
  }
  if (nsteps == 0) flush(true);
}

// Exact mode, streamed by slice pair: the reference's groups and fp32 TwoSum
// order (bit for bit the arithmetic of `reference_gemm`), on a 128 x 128
// output tile.
//
// 4 waves (2 x 2), each a 64 x 64 block as 2 x 2 MFMA 32 x 32 blocks with
// its int32 group accumulators and fp32 (hi, lo) pairs in registers (192
// VGPRs); two workgroups per CU, so one computes while the other waits at
// a barrier. The walk is the schedule's (diagonal, pair, K tile) order; each
// step is one 128-byte K tile of the pair's A and B slices, moved by LDS DMA
// (buffer_load_dwordx4 ... lds) into one of two LDS stages. A step reads
// the fragments of its first two 32-byte chunks, runs their MFMAs, reads
// the last two chunks and only then issues the DMA of the next step into
// the other stage (an LDS read ordered after an outstanding LDS DMA would
// wait for it), then runs the last MFMAs: at most two chunks' fragments
// (32 VGPRs) are live.
//
// LDS rows are 128 bytes with the 16-byte groups XOR ((r >> 1) & 7) per
// row r (as the GEMM kernel's K-contiguous panels), so a 1 KiB DMA block is
// 8 whole rows and the 16 rows of a fragment read fall on distinct bank
// groups. Lane l of block b loads row 8 b + l / 8, global group
// (l % 8) ^ ((row >> 1) & 7): within a wave's blocks that is two per-lane
// offsets (even and odd blocks) plus a uniform row offset; rows past M / N
// read zeros.
__global__ __launch_bounds__(256, 2) void oz_exact_kernel(OzArgs g) {
  constexpr int TM = 128, TN = 128;
  constexpr int PA = TM * 128, STG = PA + TN * 128;  // bytes: A panel, stage
  __shared__ __attribute__((aligned(16))) int8_t lds[2 * STG];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int lane = tid & 63;
  const int wm0 = (wave >> 1) * 64, wn0 = (wave & 1) * 64;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  int tm, tn;
  grouped_tile(t, g.tiles_m, g.tiles_n, 8, tm, tn);
  const int m0 = tm * TM, n0 = tn * TN;
  const int k = g.k;
  const int kt = g.Kp / kTileK;  // K tiles per slice (one K block: kb == Kp)
  const int total = k * (k + 1) / 2 * kt;
  const int per = kt >= kGroupTiles ? 1 : kGroupTiles / kt;

  // wave w fills blocks 4 w .. 4 w + 3 of each panel: block 4 w + u holds
  // rows 8 (4 w + u) + l / 8, whose swizzle is ((l / 8) >> 1) + 4 (u & 1)
  const int lr = lane >> 3, lq = lane & 7;
  const uint32_t vA0 = (uint32_t)(lr * g.lda + 16 * (lq ^ (lr >> 1)));
  const uint32_t vA1 = (uint32_t)(lr * g.lda + 16 * (lq ^ ((lr >> 1) + 4)));
  const uint32_t vB0 = (uint32_t)(lr * g.ldb + 16 * (lq ^ (lr >> 1)));
  const uint32_t vB1 = (uint32_t)(lr * g.ldb + 16 * (lq ^ ((lr >> 1) + 4)));
  auto dma = [&](int8_t* st, int d, int sp, int ks) __attribute__((always_inline)) {
    const int64_t koff = (int64_t)ks * kTileK;
    const int8_t* pa = g.A + sp * g.lda_s + (int64_t)m0 * g.lda + koff;
    const int8_t* pb = g.B + (d - sp) * g.ldb_s + (int64_t)n0 * g.ldb + koff;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int rows = 8 * (4 * wave + u);
      int8_t* dst = st + (4 * wave + u) * 1024;
      // rows past M / N (an edge tile) read zeros without a memory access
      const uint32_t va = m0 + rows + lr < g.M ? ((u & 1) ? vA1 : vA0) : kOzOob;
      const uint32_t vb = n0 + rows + lr < g.N ? ((u & 1) ? vB1 : vB0) : kOzOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(oz_rsrc(pa),
                                               (__attribute__((address_space(3))) void*)dst, 16,
                                               va, rows * (int)g.lda, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          oz_rsrc(pb), (__attribute__((address_space(3))) void*)(dst + PA), 16, vb,
          rows * (int)g.ldb, 0, 0);
    }
  };

  {
    // the lane index is made opaque: otherwise the per-lane addresses of
    // the whole walk are hoisted and kept live
    asm volatile("" : "+v"(lane));
    i32x16 acc[2][2];
    float hi[2][2][16], lo[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          acc[i][j][r] = 0;
          hi[i][j][r] = 0.0f;
          lo[i][j][r] = 0.0f;
        }
    // fragments of chunk c: the lane's rows (32 per MFMA block), global
    // group 2 c + l / 32 (rows 32 apart share the swizzle)
    const int sw = ((lane & 31) >> 1) & 7;
    const int ra = (wm0 + (lane & 31)) * 128, rb = PA + (wn0 + (lane & 31)) * 128;
    auto rd = [&](const int8_t* cur, int c, i32x4 (&f)[4]) __attribute__((always_inline)) {
      const int o = 16 * ((2 * c + (lane >> 5)) ^ sw);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        f[i] = *reinterpret_cast<const i32x4*>(cur + ra + o + 32 * 128 * i);
        f[2 + i] = *reinterpret_cast<const i32x4*>(cur + rb + o + 32 * 128 * i);
      }
    };
    auto mm = [&](const i32x4 (&f)[4]) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f[i], f[2 + j], acc[i][j], 0, 0, 0);
    };

    int d = k - 1, sp = 0, ks = 0;  // the step being computed
    dma(lds, d, sp, ks);
    for (int n = 0; n < total; ++n) {
      int8_t* cur = lds + (n & 1) * STG;
      int8_t* oth = lds + ((n & 1) ^ 1) * STG;
      // the next step of the walk: K tiles, then pairs s = 0 .. d (t = d - s),
      // then diagonals d = k-1 .. 0
      int nd = d, ns = sp, nk = ks + 1;
      if (nk == kt) {
        nk = 0;
        if (++ns > nd) {
          ns = 0;
          --nd;
        }
      }
      __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA of step n has landed
      __syncthreads();                // every wave's has; every read of `oth` is done
      i32x4 f0[4], f1[4];
      rd(cur, 0, f0);
      rd(cur, 1, f1);
      mm(f0);
      mm(f1);
      rd(cur, 2, f0);
      rd(cur, 3, f1);
      if (n + 1 < total) dma(oth, nd, ns, nk);
      mm(f0);
      mm(f1);
      // a group closes after this step (ozaki.py:337-355): fold its exact
      // int32 sums, scaled by 2^(7 (k - 1 - d)), into (hi, lo)
      const bool end = kt >= kGroupTiles ? ((ks + 1) % kGroupTiles == 0 || ks + 1 == kt)
                                         : (ks + 1 == kt && ((sp + 1) % per == 0 || sp == d));
      if (end) {
        const float scale = __int_as_float((127 + kSliceBits * (k - 1 - d)) << 23);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const float pv = (float)acc[i][j][r] * scale;  // exact: |G| <= 2^24
              two_sum32(hi[i][j][r], lo[i][j][r], pv);
              acc[i][j][r] = 0;
            }
      }
      d = nd, sp = ns, ks = nk;
    }

    // Epilogue (lane l of a 32x32 block: column l % 32, rows 8 (r/4) +
    // 4 (l/32) + r % 4): the fp64 recombination into C (gemm_fp64), or the
    // raw (hi, lo) pairs into two planes (the hilo surface).
    asm volatile("" : "+v"(lane));
    if (g.fuse) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int n = n0 + wn0 + j * 32 + (lane & 31);
          const int mb = m0 + wm0 + i * 32 + (lane >> 5) * 4;
          if (n >= g.N) continue;
          const int eb = g.eB[n];
          double* cb = g.C + (int64_t)mb * g.ldc_m + (int64_t)n * g.ldc_n;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int dm = (r >> 2) * 8 + (r & 3);
            if (mb + dm >= g.M) continue;
            cb[dm * g.ldc_m] = oz_combine(hi[i][j][r], lo[i][j][r], g.eA[mb + dm], eb, k);
          }
        }
      return;
    }
    // (one base address per 32 x 32 block; the row offsets are uniform)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn0 + j * 32 + (lane & 31);
        const int mb = m0 + wm0 + i * 32 + (lane >> 5) * 4;
        if (n >= g.N) continue;
        // (hi, lo) of element (m, n) at hilo[m rs + n cs] and lo_off floats on
        float* hb = g.hilo + (int64_t)mb * g.hl_rs + (int64_t)n * g.hl_cs;
        const int64_t rs = g.hl_rs, lo_off = g.hl_lo;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dm = (r >> 2) * 8 + (r & 3);
          if (mb + dm >= g.M) continue;
          hb[dm * rs] = hi[i][j][r];
          hb[dm * rs + lo_off] = lo[i][j][r];
        }
      }
  }
}

__device__ __forceinline__ double oz_combine(float hi, float lo, int ea_raw, int eb, int k) {
  const int off = -2 * (kSliceBits - 1) - kSliceBits * (k - 1);
  const int ea = ea_raw + off;
  const double v = (double)hi + (double)lo;
  if (ea < 900 && ea > -900 && eb < 900 && eb > -900) return (v * pow2(ea)) * pow2(eb);
  return ldexp(v, ea + eb);
}

constexpr int kOzBM = 128, kOzBN = 128, kOzBK = 64;

static int oz_launch(OzArgs& g, int out, hipStream_t s) {
  g.tiles_m = (g.M + kOzBM - 1) / kOzBM;
  g.tiles_n = (g.N + kOzBN - 1) / kOzBN;
  const int64_t nt = (int64_t)g.tiles_m * g.tiles_n;
  TRNBLAS_CHECK_ARG(nt < (1ll << 31), "ozaki: too many tiles");
  if (g.kb == g.Kp) {
    // one K block (K up to ~2^16): the streamed kernel (C5: 22.7 ms against
    // 63.8 ms for oz_gemm_kernel, bit-equal), with the fp64 combine in its
    // epilogue (mode 0) or the (hi, lo) planes out (mode 1)
    g.fuse = out == 0;
    if (out != 0) {
      g.hl_rs = g.ldh;
      g.hl_cs = 1;
      g.hl_lo = (int64_t)g.M * g.ldh;
    }
    hipLaunchKernelGGL(oz_exact_kernel, dim3((unsigned)nt), dim3(256), 0, s, g);
    return check_launch("ozaki_gemm");
  }
  if (out == 0)
    hipLaunchKernelGGL((oz_gemm_kernel<kOzBM, kOzBN, kOzBK, 0>), dim3((unsigned)nt), dim3(256),
                       0, s, g);
  else
    hipLaunchKernelGGL((oz_gemm_kernel<kOzBM, kOzBN, kOzBK, 1>), dim3((unsigned)nt), dim3(256),
                       0, s, g);
  return check_launch("ozaki_gemm");
}

// Fast mode launch: 64 x 64 tiles; the int32 diagonals are flushed to fp64
// before k * K_flush * 2^12 could reach 2^31 (K blocks are not needed).
// One LDS stage per workgroup, two workgroups per CU: measured faster at C5
// (17.9 ms against 19.5 ms) than two stages and one workgroup per CU, whose
// single wave per SIMD leaves every barrier and load wait exposed.
constexpr int OZ_NB = 1;
static int oz_fast_launch(OzArgs& g, hipStream_t s, bool il) {
  const int64_t kflush = ((1ll << 31) - 1) / (4096ll * g.k);  // K terms per diagonal
  if (il) {
    // 64 x 64 tiles (two workgroups per CU up to 9 slices): measured faster
    // at C5 (the 8192^3 call 14.2 ms against 15.0 ms) than 128 x 64 tiles
    // with one 8-wave workgroup per CU, whose barriers stall every wave on
    // the CU at once
    g.tiles_m = (g.M + 63) / 64;
    g.tiles_n = (g.N + 63) / 64;
    const int64_t nt = (int64_t)g.tiles_m * g.tiles_n;
    TRNBLAS_CHECK_ARG(nt < (1ll << 31), "ozaki: too many tiles");
    g.flush = (int)std::max<int64_t>(1, kflush / 32);
    const dim3 grid((unsigned)nt), block(256);
    switch (g.k) {
#define OZ_IL(KS) \
  case KS:        \
    hipLaunchKernelGGL((oz_fast_ilk_kernel<KS>), grid, block, 0, s, g); \
    break;
      OZ_IL(1) OZ_IL(2) OZ_IL(3) OZ_IL(4) OZ_IL(5) OZ_IL(6)
      OZ_IL(7) OZ_IL(8) OZ_IL(9) OZ_IL(10) OZ_IL(11) OZ_IL(12)
#undef OZ_IL
      default:
        set_error("ozaki_gemm(fast): slices %d not in [1, 12]", g.k);
        return TRNBLAS_E_ARG;
    }
    return check_launch("ozaki_gemm(fast)");
  }
  g.tiles_m = (g.M + 63) / 64;
  g.tiles_n = (g.N + 63) / 64;
  const int64_t nt = (int64_t)g.tiles_m * g.tiles_n;
  TRNBLAS_CHECK_ARG(nt < (1ll << 31), "ozaki: too many tiles");
  const int bk = g.k <= 8 ? 64 : 32;
  g.flush = (int)std::max<int64_t>(1, kflush / bk);
  const dim3 grid((unsigned)nt), block(256);
  switch (g.k) {
#define OZ_FAST(KS, BK) \
  case KS:              \
    hipLaunchKernelGGL((oz_fast_kernel<KS, BK, OZ_NB>), grid, block, 0, s, g); \
    break;
    OZ_FAST(1, 64) OZ_FAST(2, 64) OZ_FAST(3, 64) OZ_FAST(4, 64)
    OZ_FAST(5, 64) OZ_FAST(6, 64) OZ_FAST(7, 64) OZ_FAST(8, 64)
    OZ_FAST(9, 32) OZ_FAST(10, 32) OZ_FAST(11, 32) OZ_FAST(12, 32)
#undef OZ_FAST
    default:
      set_error("ozaki_gemm(fast): slices %d not in [1, 12]", g.k);
      return TRNBLAS_E_ARG;
  }
  return check_launch("ozaki_gemm(fast)");
}

static int oz_check_operands(int slices, int64_t M, int64_t N, int64_t Kp, int64_t kb,
                             const int8_t* dA, int64_t lda, int64_t lda_slice, const int8_t* dB,
                             int64_t ldb, int64_t ldb_slice) {
  TRNBLAS_CHECK_ARG(slices >= 1 && slices <= 12, "ozaki: slices %d not in [1, 12]", slices);
  TRNBLAS_CHECK_ARG(M >= 0 && N >= 0 && Kp >= 0 && M < (1 << 30) && N < (1 << 30),
                    "ozaki: bad size");
  TRNBLAS_CHECK_ARG(Kp % kTileK == 0, "ozaki: Kp %lld not a multiple of 128", (long long)Kp);
  TRNBLAS_CHECK_ARG(kb > 0 && kb % kTileK == 0,
                    "ozaki: K block %lld must be a positive multiple of 128", (long long)kb);
  TRNBLAS_CHECK_ARG(dA && dB, "ozaki: NULL digits");
  TRNBLAS_CHECK_ARG(lda >= Kp && ldb >= Kp && lda % 16 == 0 && ldb % 16 == 0 &&
                        lda_slice % 16 == 0 && ldb_slice % 16 == 0,
                    "ozaki: digit leading dimensions must be >= Kp and multiples of 16");
  TRNBLAS_CHECK_ARG(((uintptr_t)dA & 15) == 0 && ((uintptr_t)dB & 15) == 0,
                    "ozaki: digit buffers must be 16-byte aligned");
  TRNBLAS_CHECK_ARG((int64_t)kOzBM * lda < 0x7fffff00ll && (int64_t)kOzBN * ldb < 0x7fffff00ll,
                    "ozaki: leading dimension too large for 32-bit tile offsets");
  return TRNBLAS_OK;
}

// ---------------------------------------------------------------------------
// Ozaki scheme II (Ozaki, Uchino and Imamura, 2025): the exact product of
// the integer operands A' = rint(A 2^(p - eA)), B' = rint(B 2^(p - eB))
// (p = 7 slices - 1: the precision of `slices` 7-bit digits) by the Chinese
// remainder theorem over pairwise coprime int8 moduli. Each modulus costs
// one int8 GEMM of balanced residues (|r| <= 128, int32 sums exact), where
// the digit split costs slices (slices + 1) / 2 of them for all moduli
// together being fewer: at C5, 22 GEMMs against 66 for 11 slices.
//
//  * crt_residues_row / _col: A' (by rows) and B' (by columns, written
//    transposed) as int8 residues, K contiguous, one plane per modulus;
//  * crt_gemm_kernel: per modulus t the int8 GEMM A'_t B'_t^T on
//    v_mfma_i32_32x32x32_i8, its int32 sums reduced to balanced residues mod
//    m_t in the epilogue and stored in a 32 x 32 blocked layout (lane l's 16
//    accumulator bytes of block (bm, bn) are 16 contiguous bytes);
//  * crt_combine_kernel: per element, Garner's mixed-radix digits from the
//    residues (exact small-integer fp32 arithmetic), the value by Horner in
//    fp64 fma over digit pairs (radices m_2g m_2g+1), scaled by
//    2^(eA + eB - 2p).

constexpr int kCrtMax = 32;
// pairwise coprime, <= 256, largest first (256 first: the balanced
// mixed-radix range is exactly [-M/2, M/2 - 1])
constexpr int kCrtMod[kCrtMax] = {256, 255, 253, 251, 247, 241, 239, 233, 229, 227, 223,
                                  217, 211, 199, 197, 193, 191, 181, 179, 173, 167, 163,
                                  157, 151, 149, 139, 137, 131, 127, 113, 109, 107};

struct CrtTab {
  int m[kCrtMax];           // the moduli
  int q[kCrtMax][kCrtMax];  // q[s][t] = (m_0 ... m_{s-1}) mod m_t, s < t
  int inv[kCrtMax];         // (m_0 ... m_{t-1})^-1 mod m_t
  int w28[kCrtMax];         // 2^28 mod m_t
  int w56[kCrtMax];         // 2^56 mod m_t
  double rcp[kCrtMax];      // 1 / m_t
};

constexpr int crt_modinv(int a, int m) {  // a^-1 mod m, gcd(a, m) = 1
  int t = 0, nt = 1, r = m, nr = a % m;
  while (nr != 0) {
    const int q = r / nr;
    int x = t - q * nt;
    t = nt;
    nt = x;
    x = r - q * nr;
    r = nr;
    nr = x;
  }
  return t < 0 ? t + m : t;
}

constexpr CrtTab crt_tab() {
  CrtTab c{};
  for (int t = 0; t < kCrtMax; ++t) {
    const int m = kCrtMod[t];
    c.m[t] = m;
    long long P = 1 % m;
    for (int s = 0; s < t; ++s) {
      c.q[s][t] = (int)P;
      P = P * kCrtMod[s] % m;
    }
    c.inv[t] = t ? crt_modinv((int)P, m) : 1;
    long long w = 1;
    for (int i = 0; i < 28; ++i) w = w * 2 % m;
    c.w28[t] = (int)w;
    for (int i = 0; i < 28; ++i) w = w * 2 % m;
    c.w56[t] = (int)w;
    c.rcp[t] = 1.0 / m;
  }
  return c;
}

constexpr CrtTab kCrtTab = crt_tab();

// Paired moduli mu_g = m_2g m_2g+1 (< 2^16) for the recombination: the
// balanced mixed-radix digits in these radices are exactly
// v_2g + m_2g v_2g+1 of the single-modulus digits.
constexpr int kCrtPairs = kCrtMax / 2;
struct CrtPairTab {
  long long mu[kCrtPairs];              // m_2g m_2g+1
  int pinv[kCrtPairs];                  // m_2g^-1 mod m_2g+1
  long long q[kCrtPairs][kCrtPairs];    // q[h][g] = (mu_0 ... mu_h-1) mod mu_g, h < g
  long long inv[kCrtPairs];             // (mu_0 ... mu_g-1)^-1 mod mu_g
  double rcp[kCrtPairs];                // 1 / mu_g
};

constexpr long long crt_modinv64(long long a, long long m) {
  long long t = 0, nt = 1, r = m, nr = a % m;
  while (nr != 0) {
    const long long q = r / nr;
    long long x = t - q * nt;
    t = nt;
    nt = x;
    x = r - q * nr;
    r = nr;
    nr = x;
  }
  return t < 0 ? t + m : t;
}

constexpr CrtPairTab crt_pair_tab() {
  CrtPairTab c{};
  for (int g = 0; g < kCrtPairs; ++g) {
    const long long mu = (long long)kCrtMod[2 * g] * kCrtMod[2 * g + 1];
    c.mu[g] = mu;
    c.pinv[g] = crt_modinv(kCrtMod[2 * g] % kCrtMod[2 * g + 1], kCrtMod[2 * g + 1]);
    long long P = 1 % mu;
    for (int h = 0; h < g; ++h) {
      c.q[h][g] = P;
      P = P * c.mu[h] % mu;
    }
    c.inv[g] = g ? crt_modinv64(P, mu) : 1;
    c.rcp[g] = 1.0 / (double)mu;
  }
  return c;
}

constexpr CrtPairTab kCrtPair = crt_pair_tab();
__constant__ CrtTab c_crt_tab = crt_tab();  // for per-launch (runtime) modulus indices

// y = rint(x 2^sh) (|y| <= 2^p, p <= 90) as sign and 28-bit limbs:
// |y| = y2 2^56 + y1 2^28 + y0, 0 <= yk < 2^28, every step exact (|y| is an
// integer of at most 53 significant bits).
struct CrtLimbs {
  double y0, y1, y2;
  bool neg;
};

__device__ __forceinline__ CrtLimbs crt_limbs(double x, int sh) {
  double y = rint(ldexp(x, sh));
  CrtLimbs l;
  l.neg = y < 0.0;
  y = fabs(y);
  l.y2 = floor(y * 0x1p-56);
  y = fma(-l.y2, 0x1p56, y);
  l.y1 = floor(y * 0x1p-28);
  l.y0 = fma(-l.y1, 0x1p28, y);
  return l;
}

// The balanced residue of sign * |y| modulo m_T: [-m/2, m/2) for even m,
// [-(m-1)/2, (m-1)/2] for odd m. s = y2 w56 + y1 w28 + y0 < 2^37 is exact in
// fp64; floor(s / m) from the reciprocal is off by at most one, fixed below.
template <int T>
__device__ __forceinline__ int crt_residue(const CrtLimbs& l) {
  constexpr int m = kCrtMod[T];
  const double s = fma(l.y2, (double)kCrtTab.w56[T], fma(l.y1, (double)kCrtTab.w28[T], l.y0));
  const double q = floor(s * kCrtTab.rcp[T]);
  double r = fma(-q, (double)m, s);
  r = r < 0.0 ? r + m : r;
  r = r >= (double)m ? r - m : r;
  int ri = (int)r;
  ri = l.neg ? -ri : ri;
  ri = ri >= m - m / 2 ? ri - m : ri;
  ri = ri < -(m / 2) ? ri + m : ri;
  return ri;
}

// Residues of one element for every modulus t < nmod, byte b of word u[t].
template <int T>
__device__ __forceinline__ void crt_residues_of(const CrtLimbs& l, int nmod, uint32_t* u, int b) {
  if constexpr (T < kCrtMax) {
    if (T < nmod) {
      u[T] |= (uint32_t)(uint8_t)(int8_t)crt_residue<T>(l) << (8 * b);
      crt_residues_of<T + 1>(l, nmod, u, b);
    }
  }
}

// Residue planes are blocked: element (row r, k) of modulus t's plane at
// t * ld_plane + ((r / 16) * (kp / 64) + k / 64) * 1024 + (r % 16) * 64 + k % 64,
// so the 16 rows x 64 bytes that one LDS DMA instruction of the GEMM moves
// are one contiguous KiB (eight whole cache lines).
__device__ __forceinline__ int64_t crt_blk(int64_t r, int k, int nkc) {
  return ((r >> 4) * nkc + (k >> 6)) * 1024 + (r & 15) * 64 + (k & 63);
}

// Row residues: X (R, C) row-major with exponent e_r per row, residues of
// row r, k < kp (columns C .. kp - 1 zero). A workgroup covers 16 rows x
// 64 columns (one KiB block per modulus); thread t: row 16 blockIdx.y +
// t / 16, columns 64 blockIdx.x + 4 (t % 16) .. +3. A wave's 4-byte stores
// of a modulus fill 256 contiguous bytes.
__global__ __launch_bounds__(256) void crt_residues_row_kernel(const double* X, int64_t ldx,
                                                               int R, int C, int kp, int p,
                                                               int nmod, const int32_t* exps,
                                                               int8_t* out, int64_t ld_plane) {
  const int64_t r = (int64_t)blockIdx.y * 16 + (threadIdx.x >> 4);
  const int k0 = blockIdx.x * 64 + 4 * (threadIdx.x & 15);
  if (r >= R) return;
  const int e = exps[r];
  if (e == kNonFinite) return;
  uint32_t u[kCrtMax];
#pragma unroll
  for (int t = 0; t < kCrtMax; ++t) u[t] = 0;
  const double* src = X + r * ldx + k0;
  double x[4];
  if (k0 + 4 <= C && ((reinterpret_cast<uintptr_t>(src) & 15) == 0)) {
    const double2 a = *reinterpret_cast<const double2*>(src);
    const double2 b = *reinterpret_cast<const double2*>(src + 2);
    x[0] = a.x;
    x[1] = a.y;
    x[2] = b.x;
    x[3] = b.y;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = k0 + i < C ? src[i] : 0.0;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) crt_residues_of<0>(crt_limbs(x[i], p - e), nmod, u, i);
  int8_t* dst = out + crt_blk(r, k0, kp >> 6);
#pragma unroll
  for (int t = 0; t < kCrtMax; ++t)
    if (t < nmod) *reinterpret_cast<uint32_t*>(dst + t * ld_plane) = u[t];
}

// Column residues: X (R, C) row-major with exponent e_c per column, the
// residues of column c as operand row c, k = r < kp (rows R .. kp - 1
// zero). A workgroup covers 64 rows (k) x 64 columns: the tile is read row
// by row (coalesced) into LDS, then thread t takes column 16 q + t / 16 of
// pass q (q < 4) and rows 4 (t % 16) .. +3 of it, so a wave's 4-byte
// stores of a modulus fill 256 contiguous bytes of the blocked layout.
__global__ __launch_bounds__(256) void crt_residues_col_kernel(const double* X, int64_t ldx,
                                                               int R, int C, int kp, int p,
                                                               int nmod, const int32_t* exps,
                                                               int8_t* out, int64_t ld_plane) {
  __shared__ double tile[64][65];  // [column][row], padded: column reads spread over banks
  const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = r0 + 4 * i + ty, c = c0 + tx;
    tile[tx][4 * i + ty] = (r < R && c < C) ? X[(int64_t)r * ldx + c] : 0.0;
  }
  __syncthreads();
  const int kk = 4 * (threadIdx.x & 15);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int cl = 16 * q + (threadIdx.x >> 4), c = c0 + cl;
    if (c >= C) continue;
    const int e = exps[c];
    if (e == kNonFinite) continue;
    uint32_t u[kCrtMax];
#pragma unroll
    for (int t = 0; t < kCrtMax; ++t) u[t] = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) crt_residues_of<0>(crt_limbs(tile[cl][kk + i], p - e), nmod, u, i);
    int8_t* dst = out + crt_blk(c, r0 + kk, kp >> 6);
#pragma unroll
    for (int t = 0; t < kCrtMax; ++t)
      if (t < nmod) *reinterpret_cast<uint32_t*>(dst + t * ld_plane) = u[t];
  }
}

struct CrtGemmArgs {
  int M, N, Kp;          // Kp a multiple of 64
  const int8_t* A;       // blocked residues (crt_blk): plane t at A + t lda_plane,
  int64_t lda, lda_plane;  // lda = bytes from one 16-row block to the next
  const int8_t* B;       // B^T residues, blocked the same way
  int64_t ldb, ldb_plane;
  int8_t* P;             // product residues, 32 x 32 blocked, plane t at P + t p_plane
  int64_t p_plane;
  int nbm, nbn;          // 32-row / 32-column blocks of the output
  int tiles_m, tiles_n;  // 256 x 256 tiles
};

constexpr int kCrtTM = 256, kCrtTN = 256, kCrtBK = 64, kCrtStages = 4;
constexpr int kCrtPanelA = kCrtTM * kCrtBK;              // 16 KiB per stage
constexpr int kCrtStage = kCrtPanelA + kCrtTN * kCrtBK;  // 32 KiB

// Balanced residue of an int32 modulo m (|a| < 2^31, exact in fp64).
__device__ __forceinline__ int crt_smod32(int a, int m, double rcp) {
  const double x = (double)a;
  const double q = floor(x * rcp);
  int r = (int)fma(-q, (double)m, x);
  r += r < 0 ? m : 0;
  r -= r >= m ? m : 0;
  return r >= m - (m >> 1) ? r - m : r;
}

// The int8 GEMM of one modulus (blockIdx.y) on a 256 x 256 output tile:
// 4 waves (2 x 2) of 128 x 128, each 4 x 4 blocks of v_mfma_i32_32x32x32_i8
// (256 int32 accumulators per lane, in AGPRs), so a 32-byte chunk's 8
// fragment reads (4 of A, 4 of B, 16 bytes per lane each) feed 16 MFMAs:
// half the LDS bytes per MFMA of a 64 x 64 wave tile. K steps of 64 bytes
// through four LDS stages of 32 KiB: the DMA of step s + 3 goes out once
// every wave has passed the barrier of step s (so every wave is done
// reading step s - 1, whose stage it refills), and each chunk's fragments
// are read before the MFMAs of the chunk before issue, so their LDS latency
// hides behind those MFMAs (one wave per SIMD has no other wave to hide
// it). A stage holds 256 rows of A then 256 of B, 64 bytes each; group j of
// row r sits in slot j ^ ((r >> 2) & 3), so the 16 rows of a fragment read
// fall on distinct bank groups and a 1 KiB DMA block is 16 whole rows. The
// DMA (buffer_load_dwordx4 ... lds) is issued by inline asm, out of sight
// of the compiler's wait tracking, and waited for explicitly (vmcnt leaves
// the later steps' DMAs of this wave in flight). Rows past M / N load
// zeros without a memory access. ACCUM: add the residues already in P (a K
// block after the first).
template <bool ACCUM>
__global__ __launch_bounds__(256, 1) void crt_gemm_kernel(CrtGemmArgs g) {
  __shared__ __attribute__((aligned(16))) int8_t lds[kCrtStages * kCrtStage];
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  int lane = tid & 63;
  const int mod = blockIdx.y;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  int tm, tn;
  grouped_tile(t, g.tiles_m, g.tiles_n, 4, tm, tn);
  const int m0 = tm * kCrtTM, n0 = tn * kCrtTN;
  const int8_t* baseA = g.A + mod * g.lda_plane + (int64_t)(m0 >> 4) * g.lda;
  const int8_t* baseB = g.B + mod * g.ldb_plane + (int64_t)(n0 >> 4) * g.ldb;
  const int nsteps = g.Kp / kCrtBK;

  // DMA: wave w moves blocks b = w + 4u (u < 4) of each panel (rows 16 b ..
  // 16 b + 15: one contiguous KiB of the blocked residues per k-step); lane
  // l of a block fills row 16 b + l / 4, slot l % 4, i.e. source group
  // (l % 4) ^ ((l >> 4) & 3) of that row
  uint32_t vA[4], vB[4];
  {
    const int gsrc = (lane & 3) ^ ((lane >> 4) & 3);
    const int in_blk = (lane >> 2) * 64 + 16 * gsrc;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int row = 16 * (w + 4 * u) + (lane >> 2);
      vA[u] = m0 + row < g.M ? (uint32_t)((w + 4 * u) * g.lda + in_blk) : kOzOob;
      vB[u] = n0 + row < g.N ? (uint32_t)((w + 4 * u) * g.ldb + in_blk) : kOzOob;
    }
  }
  // block u (< 4) of both panels of a step
  auto dma_u = [&](int step, int u) __attribute__((always_inline)) {
    int8_t* dst = lds + (step & (kCrtStages - 1)) * kCrtStage;
    const int soff = step * 1024;
    lds_dma16_asm(baseA, dst + (w + 4 * u) * 1024, vA[u], soff);
    lds_dma16_asm(baseB, dst + kCrtPanelA + (w + 4 * u) * 1024, vB[u], soff);
  };
  auto dma = [&](int step) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 4; ++u) dma_u(step, u);
  };

  i32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

  // fragment of chunk c (32 bytes of K): row (l % 32) of the block, group
  // 2 c + l / 32 in slot (2 c + l / 32) ^ ((l % 32 >> 2) & 3)
  const int wm = w & 1, wn = w >> 1;
  const int sw = ((lane & 31) >> 2) & 3;
  const int o0 = (lane & 31) * kCrtBK + 16 * ((lane >> 5) ^ sw);
  const int o1 = (lane & 31) * kCrtBK + 16 * ((2 + (lane >> 5)) ^ sw);
  const int rowA = 128 * wm * kCrtBK, rowB = kCrtPanelA + 128 * wn * kCrtBK;
  // the fragments of chunk c of a step: f[i] = A block i, f[4 + j] = B block j
  auto rd = [&](int step, int c, i32x4 (&f)[8]) __attribute__((always_inline)) {
    const int8_t* cur = lds + (step & (kCrtStages - 1)) * kCrtStage;
    const int o = c ? o1 : o0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[i] = *reinterpret_cast<const i32x4*>(cur + rowA + 32 * i * kCrtBK + o);
      f[4 + i] = *reinterpret_cast<const i32x4*>(cur + rowB + 32 * i * kCrtBK + o);
    }
  };
  auto mm_row = [&](const i32x4 (&f)[8], int i) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f[i], f[4 + j], acc[i][j], 0, 0, 0);
  };
  auto mm = [&](const i32x4 (&f)[8]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) mm_row(f, i);
  };

  // prefetch distance 3: the DMA of step s + 3 refills the stage of s - 1
  dma(0);
  if (nsteps > 1) dma(1);
  if (nsteps > 2) dma(2);
  // this wave's DMA of step 0 has landed (8 DMAs per step and wave)
  if (nsteps > 2)
    asm volatile("s_waitcnt vmcnt(16)\n\ts_barrier" ::: "memory");
  else if (nsteps > 1)
    asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  i32x4 f0[8], f1[8];
  rd(0, 0, f0);
  // step s: chunk 1's reads behind chunk 0's MFMAs; then the barrier that
  // publishes step s + 1 (this wave's DMA of s + 1 has landed; vmcnt(8)
  // leaves the 8 of s + 2 in flight), the DMA of s + 3 and the reads of
  // chunk 0 of s + 1, behind chunk 1's MFMAs. The steady-state loop has no
  // branches (the last steps are peeled), so the compiler's LDS wait counts
  // before chunk 1's MFMAs leave the next step's reads in flight;
  // sched_barrier keeps the compiler from sinking the reads below the
  // MFMAs, which it prefers for register pressure.
  // The 8 DMA issues of s + 3 go out between chunk 1's MFMA rows (2 per
  // row of 4 MFMAs), where the matrix cores have queued work, instead of as
  // one block at the phase boundary (timed: the block cost ~a quarter of
  // the GEMM's time).
  auto body = [&](int s, auto next, auto refill, auto wait8) __attribute__((always_inline)) {
    rd(s, 1, f1);
    __builtin_amdgcn_sched_barrier(0);
    mm(f0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (decltype(next)::value) {
      if constexpr (decltype(wait8)::value)
        asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
      rd(s + 1, 0, f0);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      mm_row(f1, i);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (decltype(next)::value && decltype(refill)::value) dma_u(s + 3, i);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  using Y = std::true_type;
  using N = std::false_type;
  int s = 0;
  for (; s + 3 < nsteps; ++s) body(s, Y{}, Y{}, Y{});
  if (s + 2 < nsteps) body(s++, Y{}, N{}, Y{});
  if (s + 1 < nsteps) body(s++, Y{}, N{}, N{});
  body(s, N{}, N{}, N{});

  // epilogue: balanced residues mod m, 16 bytes per lane per 32 x 32 block
  asm volatile("" : "+v"(lane));
  const int m = c_crt_tab.m[mod];
  const double rcp = c_crt_tab.rcp[mod];
  int8_t* P = g.P + mod * g.p_plane;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int bm = (m0 + 128 * wm + 32 * i) >> 5, bn = (n0 + 128 * wn + 32 * j) >> 5;
      if (bm >= g.nbm || bn >= g.nbn) continue;
      i32x4* dst = reinterpret_cast<i32x4*>(P + (((int64_t)bm * g.nbn + bn) * 64 + lane) * 16);
      i32x4 old = {0, 0, 0, 0};
      if constexpr (ACCUM) old = *dst;
      uint32_t wd[4] = {0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int prev = (int8_t)(uint8_t)((uint32_t)old[e >> 2] >> (8 * (e & 3)));
        wd[e >> 2] |= (uint32_t)(uint8_t)(int8_t)crt_smod32(acc[i][j][e] + prev, m, rcp) << (8 * (e & 3));
      }
      *dst = i32x4{(int)wd[0], (int)wd[1], (int)wd[2], (int)wd[3]};
    }
}

// x mod m for an integer-valued double |x| < 2^52 (exact: floor(x / m)
// from the reciprocal is off by at most one, fixed after the exact fma).
__device__ __forceinline__ double crt_mod(double x, double m, double rcp) {
  const double q = floor(x * rcp);
  double r = fma(-q, m, x);
  r = r < 0.0 ? r + m : r;
  return r >= m ? r - m : r;
}

// Garner's digits of one element in the paired radices and its value by
// Horner. r[t]: the residue mod m_t (t < nmod). Pair g (moduli 2g, 2g + 1)
// first becomes one residue R mod mu_g = m_2g m_2g+1 (two-modulus CRT);
// the last group is a single modulus when nmod is odd. Digit g:
// V_g = ((R_g - sum_{h<g} V_h (mu_0..mu_h-1 mod mu_g)) (mu_0..mu_g-1)^-1)
// mods mu_g; every sum stays below 2^36, exact in fp64. Then
// H = V_top, H = fma(H, mu_g, V_g) down to g = 0 (one rounding per step).
template <int NMOD>
__device__ __forceinline__ double crt_value(const float* r) {
  constexpr int nmod = NMOD;
  double V[kCrtPairs];
  constexpr int top = (nmod - 1) >> 1;
#pragma unroll
  for (int g = 0; g < kCrtPairs; ++g) {
    if (g <= top) {
      const bool pair = 2 * g + 1 < nmod;  // a compile-time constant once unrolled
      const double ma = kCrtMod[2 * g];
      double R, mu, rcp, inv;
      double acc = 0.0;
      if (pair) {
        const double mb = kCrtMod[2 * g + 1], rcpb = 1.0 / kCrtMod[2 * g + 1];
        const double d = crt_mod(crt_mod((double)(r[2 * g + 1] - r[2 * g]), mb, rcpb) * kCrtPair.pinv[g], mb, rcpb);
        R = fma(ma, d, (double)r[2 * g]);
        mu = (double)kCrtPair.mu[g];
        rcp = kCrtPair.rcp[g];
        inv = (double)kCrtPair.inv[g];
#pragma unroll
        for (int h = 0; h < g; ++h) acc = fma(V[h], (double)kCrtPair.q[h][g], acc);
      } else {
        R = r[2 * g];
        mu = ma;
        rcp = kCrtTab.rcp[2 * g];
        inv = (double)kCrtTab.inv[2 * g];
#pragma unroll
        for (int h = 0; h < g; ++h) acc = fma(V[h], (double)kCrtTab.q[2 * h][2 * g], acc);
      }
      const double z = crt_mod(crt_mod(R - acc, mu, rcp) * inv, mu, rcp);
      // balanced: [-mu/2, mu/2) (mu even only for g = 0) or +-(mu - 1)/2
      V[g] = z >= mu - floor(mu * 0.5) ? z - mu : z;
    }
  }
  double H = 0.0;
#pragma unroll
  for (int g = kCrtPairs - 1; g >= 0; --g)
    if (g <= top) H = g == top ? V[g] : fma(H, (double)kCrtPair.mu[g], V[g]);
  return H;
}

struct CrtCombineArgs {
  int M, N, nmod, p;
  const int8_t* P;
  int64_t p_plane;
  int nbm, nbn;
  const int32_t* eA;
  const int32_t* eB;
  double* C;
  int64_t ldc_m, ldc_n;
};

// One wave per 32 x 32 block of the product residues (4 blocks per
// workgroup): lane l holds 16 bytes per modulus, the elements of column
// l % 32, rows 8 (e / 4) + 4 (l / 32) + e % 4 (the MFMA accumulator layout).
// NMOD, the modulus count, is a template parameter: the digit loops then
// have no runtime branches.
template <int NMOD>
__global__ __launch_bounds__(256) void crt_combine_kernel(CrtCombineArgs g) {
  const int lane = threadIdx.x & 63;
  const int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (blk >= (int64_t)g.nbm * g.nbn) return;
  const int bm = (int)(blk / g.nbn), bn = (int)(blk - (int64_t)bm * g.nbn);
  const int n = bn * 32 + (lane & 31);
  if (n >= g.N) return;
  const int eb = g.eB[n];
  const int8_t* src = g.P + blk * 1024 + lane * 16;
  // word q of the lane's 16 bytes holds elements 4 q .. 4 q + 3
#pragma unroll 1
  for (int q = 0; q < 4; ++q) {
    uint32_t wd[NMOD];
#pragma unroll
    for (int t = 0; t < NMOD; ++t) wd[t] = *reinterpret_cast<const uint32_t*>(src + t * g.p_plane + 4 * q);
#pragma unroll 1
    for (int b = 0; b < 4; ++b) {
      const int m = bm * 32 + 8 * q + 4 * (lane >> 5) + b;
      if (m >= g.M) continue;
      float r[NMOD];
#pragma unroll
      for (int t = 0; t < NMOD; ++t) r[t] = (float)(int8_t)(uint8_t)(wd[t] >> (8 * b));
      const double H = crt_value<NMOD>(r);
      g.C[(int64_t)m * g.ldc_m + (int64_t)n * g.ldc_n] = ldexp(H, g.eA[m] + eb - 2 * g.p);
    }
  }
}

// Moduli count for `slices` and K: the fewest leading moduli whose product M
// satisfies M >= 2 K 2^(2p) + 2 (multi-word integers, 32-bit limbs).
static int crt_count(int slices, int64_t K) {
  const int p = 7 * slices - 1;
  constexpr int L = 12;  // 384 bits
  uint32_t need[L] = {0}, M[L] = {0};
  // need = 2 K 2^(2p) + 2 = (K << (2p + 1)) + 2
  const int sh = 2 * p + 1;
  const unsigned __int128 v = (unsigned __int128)(uint64_t)(K > 0 ? K : 1) << (sh % 32);
  for (int i = 0; i < 4 && sh / 32 + i < L; ++i) need[sh / 32 + i] = (uint32_t)(v >> (32 * i));
  // + 2
  uint64_t carry = 2;
  for (int i = 0; i < L && carry; ++i) {
    const uint64_t s = (uint64_t)need[i] + carry;
    need[i] = (uint32_t)s;
    carry = s >> 32;
  }
  M[0] = 1;
  for (int n = 1; n <= kCrtMax; ++n) {
    uint64_t c = 0;
    for (int i = 0; i < L; ++i) {
      const uint64_t s = (uint64_t)M[i] * (uint64_t)kCrtMod[n - 1] + c;
      M[i] = (uint32_t)s;
      c = s >> 32;
    }
    // M >= need ?
    int cmp = 0;
    for (int i = L - 1; i >= 0 && cmp == 0; --i) cmp = M[i] > need[i] ? 1 : (M[i] < need[i] ? -1 : 0);
    if (cmp >= 0) return n;
  }
  return -1;
}

}  // namespace trnblas

using namespace trnblas;

extern "C" int trnblas_hip_ozaki_split(int per_row, int64_t R, int64_t C, const double* X,
                                       int64_t ldx, int slices, int8_t* digits,
                                       int64_t ld_digit, int64_t ld_slice, int32_t* exps,
                                       int32_t* scratch, void* stream) {
  clear_error();
  hipStream_t s = (hipStream_t)stream;
  TRNBLAS_CHECK_ARG((per_row & ~3) == 0, "ozaki_split: per_row %d: bit 0 per row, bit 1 interleaved",
                    per_row);
  const int il = (per_row >> 1) & 1;
  per_row &= 1;
  TRNBLAS_CHECK_ARG(slices >= 1 && slices <= 12, "ozaki_split: slices %d not in [1, 12]",
                    slices);
  TRNBLAS_CHECK_ARG(R >= 0 && C >= 0 && R < (1 << 30) && C < (1 << 30), "ozaki_split: bad size");
  TRNBLAS_CHECK_ARG(scratch && exps, "ozaki_split: NULL exps / scratch");
  const int n = per_row ? (int)R : (int)C;
  if (R == 0 || C == 0) {
    // zero exponents, no digits (the caller zero-fills the digit buffer)
    hipLaunchKernelGGL(oz_flags_kernel, dim3(1), dim3(1024), 0, s, exps, 0,
                       scratch);
    if (n > 0 && hipMemsetAsync(exps, 0, n * sizeof(int32_t), s) != hipSuccess)
      return check_launch("ozaki_split");
    return check_launch("ozaki_split");
  }
  TRNBLAS_CHECK_ARG(X && digits && ldx >= C, "ozaki_split: bad X / digits");
  if (il) {
    const int64_t kd = per_row ? C : R;  // the K extent of the digits
    TRNBLAS_CHECK_ARG(ld_digit >= (kd + 31) / 32 * 32 * slices && ld_digit % 16 == 0 &&
                          ((uintptr_t)digits & 15) == 0,
                      "ozaki_split: bad interleaved digit layout");
  }
  if (per_row) {
    TRNBLAS_CHECK_ARG(il || (ld_digit >= C && ld_slice >= R * ld_digit),
                      "ozaki_split: bad digit layout");
    hipLaunchKernelGGL(oz_emax_row_kernel, dim3((unsigned)R), dim3(256), 0, s, X, ldx, (int)R,
                       (int)C, exps);
  } else {
    TRNBLAS_CHECK_ARG(il || (ld_digit >= R && ld_slice >= C * ld_digit),
                      "ozaki_split: bad digit layout");
    TRNBLAS_CHECK_ARG((R + kEmaxRows - 1) / kEmaxRows < 65536, "ozaki_split: too many rows");
    hipLaunchKernelGGL(oz_fill_kernel, dim3((unsigned)((C + 255) / 256)), dim3(256), 0, s, exps,
                       (int)C, (int32_t)0x80000000);
    hipLaunchKernelGGL(oz_emax_col_kernel,
                       dim3((unsigned)((C + 63) / 64), (unsigned)((R + kEmaxRows - 1) / kEmaxRows)),
                       dim3(256), 0, s, X, ldx, (int)R, (int)C, exps);
  }
  int rc = check_launch("ozaki_split(emax)");
  if (rc) return rc;
  hipLaunchKernelGGL(oz_flags_kernel, dim3(1), dim3(1024), 0, s, exps, n,
                     scratch);
  rc = check_launch("ozaki_split(flags)");
  if (rc) return rc;
  if (per_row) {
    const int64_t blocks = R * ((C + 1023) / 1024);
    TRNBLAS_CHECK_ARG(blocks < (1ll << 31), "ozaki_split: too large");
    hipLaunchKernelGGL(oz_digits_row_kernel, dim3((unsigned)blocks), dim3(256),
                       0, s, X, ldx, (int)R, (int)C, slices, (const int32_t*)exps,
                       (const int32_t*)scratch, digits, ld_digit, ld_slice, il);
  } else {
    TRNBLAS_CHECK_ARG((R + 63) / 64 < 65536, "ozaki_split: too many rows");
    hipLaunchKernelGGL(oz_digits_col_kernel,
                       dim3((unsigned)((C + 63) / 64), (unsigned)((R + 63) / 64)), dim3(256), 0,
                       s, X, ldx, (int)R, (int)C, slices, (const int32_t*)exps,
                       (const int32_t*)scratch, digits, ld_digit, ld_slice, il);
  }
  return check_launch("ozaki_split(digits)");
}

extern "C" int trnblas_hip_ozaki_gemm(int mode, int slices, int64_t M, int64_t N, int64_t Kp,
                                      int64_t kb, const int8_t* dA, int64_t lda,
                                      int64_t lda_slice, const int8_t* dB, int64_t ldb,
                                      int64_t ldb_slice, const int32_t* eA, const int32_t* eB,
                                      double* C, int64_t ldc_m, int64_t ldc_n, void* stream) {
  clear_error();
  TRNBLAS_CHECK_ARG(mode >= 0 && mode <= 2, "ozaki_gemm: mode %d not supported", mode);
  if (M == 0 || N == 0) return TRNBLAS_OK;
  int rc = oz_check_operands(slices, M, N, Kp, kb, dA, lda, lda_slice, dB, ldb, ldb_slice);
  if (rc) return rc;
  if (mode == 2)
    TRNBLAS_CHECK_ARG(lda >= slices * Kp && ldb >= slices * Kp,
                      "ozaki_gemm: interleaved digits need rows of >= slices * Kp bytes");
  TRNBLAS_CHECK_ARG(Kp > 0, "ozaki_gemm: K == 0 (the caller returns zeros)");
  TRNBLAS_CHECK_ARG(C && eA && eB, "ozaki_gemm: NULL C / exponents");
  OzArgs g{};
  g.k = slices;
  g.M = (int)M;
  g.N = (int)N;
  g.Kp = (int)Kp;
  g.kb = (int)kb;
  g.A = dA;
  g.lda = lda;
  g.lda_s = lda_slice;
  g.B = dB;
  g.ldb = ldb;
  g.ldb_s = ldb_slice;
  g.eA = eA;
  g.eB = eB;
  g.C = C;
  g.ldc_m = ldc_m;
  g.ldc_n = ldc_n;
  if (mode >= 1) return oz_fast_launch(g, (hipStream_t)stream, mode == 2);
  return oz_launch(g, 0, (hipStream_t)stream);
}

extern "C" int trnblas_hip_ozaki_hilo(int slices, int64_t M, int64_t N, int64_t Kp,
                                      const int8_t* dA, int64_t lda, int64_t lda_slice,
                                      const int8_t* dB, int64_t ldb, int64_t ldb_slice,
                                      float* hilo, int64_t ldh, void* stream) {
  clear_error();
  if (M == 0 || N == 0) return TRNBLAS_OK;
  int rc = oz_check_operands(slices, M, N, Kp, Kp > 0 ? Kp : kTileK, dA, lda, lda_slice, dB,
                             ldb, ldb_slice);
  if (rc) return rc;
  TRNBLAS_CHECK_ARG(Kp > 0, "ozaki_hilo: K == 0");
  TRNBLAS_CHECK_ARG(hilo && ldh >= N, "ozaki_hilo: bad output");
  OzArgs g{};
  g.k = slices;
  g.M = (int)M;
  g.N = (int)N;
  g.Kp = (int)Kp;
  g.kb = (int)Kp;
  g.A = dA;
  g.lda = lda;
  g.lda_s = lda_slice;
  g.B = dB;
  g.ldb = ldb;
  g.ldb_s = ldb_slice;
  g.hilo = hilo;
  g.ldh = ldh;
  return oz_launch(g, 1, (hipStream_t)stream);
}

extern "C" int trnblas_hip_crt_moduli(int slices, int64_t K) {
  clear_error();
  TRNBLAS_CHECK_ARG(slices >= 1 && slices <= 12, "crt: slices %d not in [1, 12]", slices);
  TRNBLAS_CHECK_ARG(K >= 0 && K < (1ll << 40), "crt: bad K %lld", (long long)K);
  const int n = crt_count(slices, K);
  TRNBLAS_CHECK_ARG(n > 0, "crt: K %lld needs more than %d moduli at %d slices", (long long)K,
                    kCrtMax, slices);
  return n;
}

extern "C" int trnblas_hip_crt_split(int per_row, int64_t R, int64_t C, const double* X,
                                     int64_t ldx, int slices, int nmod, int64_t kp, int8_t* res,
                                     int64_t ld_plane, int32_t* exps, int32_t* flags,
                                     void* stream) {
  clear_error();
  hipStream_t s = (hipStream_t)stream;
  TRNBLAS_CHECK_ARG(per_row == 0 || per_row == 1, "crt_split: per_row %d", per_row);
  TRNBLAS_CHECK_ARG(slices >= 1 && slices <= 12, "crt_split: slices %d not in [1, 12]", slices);
  TRNBLAS_CHECK_ARG(nmod >= 1 && nmod <= kCrtMax, "crt_split: nmod %d not in [1, %d]", nmod,
                    kCrtMax);
  TRNBLAS_CHECK_ARG(R > 0 && C > 0 && R < (1 << 30) && C < (1 << 30), "crt_split: bad size");
  TRNBLAS_CHECK_ARG(X && res && exps && flags && ldx >= C, "crt_split: bad X / residues / exps");
  const int64_t kd = per_row ? C : R;  // the K extent
  const int64_t rows = per_row ? R : C;
  TRNBLAS_CHECK_ARG(kp >= kd && kp % 64 == 0 && kp < (1ll << 30),
                    "crt_split: kp %lld must be a multiple of 64 >= K", (long long)kp);
  TRNBLAS_CHECK_ARG(ld_plane >= (rows + 15) / 16 * 16 * kp && ld_plane % 16 == 0 &&
                        ((uintptr_t)res & 15) == 0,
                    "crt_split: residue planes need ceil(rows / 16) 16 kp bytes, 16-byte aligned");
  if (per_row) {
    hipLaunchKernelGGL(oz_emax_row_kernel, dim3((unsigned)R), dim3(256), 0, s, X, ldx, (int)R,
                       (int)C, exps);
  } else {
    TRNBLAS_CHECK_ARG((R + kEmaxRows - 1) / kEmaxRows < 65536, "crt_split: too many rows");
    hipLaunchKernelGGL(oz_fill_kernel, dim3((unsigned)((C + 255) / 256)), dim3(256), 0, s, exps,
                       (int)C, (int32_t)0x80000000);
    hipLaunchKernelGGL(oz_emax_col_kernel,
                       dim3((unsigned)((C + 63) / 64), (unsigned)((R + kEmaxRows - 1) / kEmaxRows)),
                       dim3(256), 0, s, X, ldx, (int)R, (int)C, exps);
  }
  int rc = check_launch("crt_split(emax)");
  if (rc) return rc;
  hipLaunchKernelGGL(oz_flags_kernel, dim3(1), dim3(1024), 0, s, exps, (int)rows, flags);
  rc = check_launch("crt_split(flags)");
  if (rc) return rc;
  const int p = 7 * slices - 1;
  if (per_row) {
    TRNBLAS_CHECK_ARG((R + 15) / 16 < 65536, "crt_split: too many rows");
    hipLaunchKernelGGL(crt_residues_row_kernel, dim3((unsigned)(kp / 64), (unsigned)((R + 15) / 16)),
                       dim3(256), 0, s, X, ldx, (int)R, (int)C, (int)kp, p, nmod,
                       (const int32_t*)exps, res, ld_plane);
  } else {
    TRNBLAS_CHECK_ARG(kp / 64 < 65536, "crt_split: too many rows");
    hipLaunchKernelGGL(crt_residues_col_kernel, dim3((unsigned)((C + 63) / 64), (unsigned)(kp / 64)),
                       dim3(256), 0, s, X, ldx, (int)R, (int)C, (int)kp, p, nmod,
                       (const int32_t*)exps, res, ld_plane);
  }
  return check_launch("crt_split(residues)");
}

extern "C" int trnblas_hip_crt_gemm(int nmod, int64_t M, int64_t N, int64_t Kp, const int8_t* RA,
                                    int64_t lda_plane, const int8_t* RB, int64_t ldb_plane,
                                    int8_t* P, int64_t p_plane, void* stream) {
  clear_error();
  TRNBLAS_CHECK_ARG(nmod >= 1 && nmod <= kCrtMax, "crt_gemm: nmod %d not in [1, %d]", nmod,
                    kCrtMax);
  TRNBLAS_CHECK_ARG(M > 0 && N > 0 && M < (1 << 30) && N < (1 << 30), "crt_gemm: bad size");
  TRNBLAS_CHECK_ARG(Kp > 0 && Kp % kCrtBK == 0, "crt_gemm: Kp %lld not a positive multiple of 64",
                    (long long)Kp);
  TRNBLAS_CHECK_ARG(RA && RB && P, "crt_gemm: NULL operand");
  TRNBLAS_CHECK_ARG(lda_plane >= (M + 15) / 16 * 16 * Kp && ldb_plane >= (N + 15) / 16 * 16 * Kp &&
                        lda_plane % 16 == 0 && ldb_plane % 16 == 0 &&
                        ((uintptr_t)RA & 15) == 0 && ((uintptr_t)RB & 15) == 0,
                    "crt_gemm: residue planes (trnblas_hip_crt_split's blocked layout) too small or "
                    "not 16-byte aligned");
  // every DMA offset (16 blocks of 16 rows, the K offset) inside the 31-bit buffer range
  TRNBLAS_CHECK_ARG(16 * 16 * Kp + 1024 < 0x7ffffff0ll,
                    "crt_gemm: K too long for 32-bit tile offsets");
  const int nbm = (int)((M + 31) / 32), nbn = (int)((N + 31) / 32);
  TRNBLAS_CHECK_ARG(p_plane >= (int64_t)nbm * nbn * 1024 && p_plane % 16 == 0 &&
                        ((uintptr_t)P & 15) == 0,
                    "crt_gemm: product planes need %lld bytes each, 16-byte aligned",
                    (long long)nbm * nbn * 1024);
  CrtGemmArgs g{};
  g.M = (int)M;
  g.N = (int)N;
  g.Kp = (int)Kp;
  g.A = RA;
  g.lda = 16 * Kp;  // one 16-row block: Kp / 64 KiB blocks
  g.lda_plane = lda_plane;
  g.B = RB;
  g.ldb = 16 * Kp;
  g.ldb_plane = ldb_plane;
  g.P = P;
  g.p_plane = p_plane;
  g.nbm = nbm;
  g.nbn = nbn;
  g.tiles_m = (int)((M + kCrtTM - 1) / kCrtTM);
  g.tiles_n = (int)((N + kCrtTN - 1) / kCrtTN);
  const int64_t nt = (int64_t)g.tiles_m * g.tiles_n;
  TRNBLAS_CHECK_ARG(nt < (1ll << 31), "crt_gemm: too many tiles");
  // |residue| <= 128: a K block of 2^16 sums below 2^30 in int32; longer K
  // runs one launch per block, each adding its residues to the last (mod m)
  constexpr int64_t kKb = 1 << 16;
  for (int64_t k0 = 0; k0 < Kp; k0 += kKb) {
    g.A = RA + k0 * 16;  // K block k0: KiB block k0 / 64 of every 16-row block
    g.B = RB + k0 * 16;
    g.Kp = (int)std::min<int64_t>(kKb, Kp - k0);
    if (k0 == 0)
      hipLaunchKernelGGL(crt_gemm_kernel<false>, dim3((unsigned)nt, (unsigned)nmod), dim3(256), 0,
                         (hipStream_t)stream, g);
    else
      hipLaunchKernelGGL(crt_gemm_kernel<true>, dim3((unsigned)nt, (unsigned)nmod), dim3(256), 0,
                         (hipStream_t)stream, g);
    const int rc = check_launch("crt_gemm");
    if (rc) return rc;
  }
  return TRNBLAS_OK;
}

extern "C" int trnblas_hip_crt_combine(int slices, int nmod, int64_t M, int64_t N,
                                       const int8_t* P, int64_t p_plane, const int32_t* eA,
                                       const int32_t* eB, double* C, int64_t ldc_m,
                                       int64_t ldc_n, void* stream) {
  clear_error();
  TRNBLAS_CHECK_ARG(slices >= 1 && slices <= 12, "crt_combine: slices %d not in [1, 12]", slices);
  TRNBLAS_CHECK_ARG(nmod >= 1 && nmod <= kCrtMax, "crt_combine: nmod %d not in [1, %d]", nmod,
                    kCrtMax);
  TRNBLAS_CHECK_ARG(M > 0 && N > 0 && M < (1 << 30) && N < (1 << 30), "crt_combine: bad size");
  TRNBLAS_CHECK_ARG(P && eA && eB && C, "crt_combine: NULL argument");
  const int nbm = (int)((M + 31) / 32), nbn = (int)((N + 31) / 32);
  TRNBLAS_CHECK_ARG(p_plane >= (int64_t)nbm * nbn * 1024 && p_plane % 16 == 0 &&
                        ((uintptr_t)P & 15) == 0,
                    "crt_combine: bad product planes");
  CrtCombineArgs g{};
  g.M = (int)M;
  g.N = (int)N;
  g.nmod = nmod;
  g.p = 7 * slices - 1;
  g.P = P;
  g.p_plane = p_plane;
  g.nbm = nbm;
  g.nbn = nbn;
  g.eA = eA;
  g.eB = eB;
  g.C = C;
  g.ldc_m = ldc_m;
  g.ldc_n = ldc_n;
  const int64_t blocks = ((int64_t)nbm * nbn + 3) / 4;
  TRNBLAS_CHECK_ARG(blocks < (1ll << 31), "crt_combine: too large");
  const dim3 grid((unsigned)blocks), block(256);
  hipStream_t s = (hipStream_t)stream;
  switch (nmod) {
#define CRT_COMB(N) \
  case N:           \
    hipLaunchKernelGGL(crt_combine_kernel<N>, grid, block, 0, s, g); \
    break;
    CRT_COMB(1) CRT_COMB(2) CRT_COMB(3) CRT_COMB(4) CRT_COMB(5) CRT_COMB(6) CRT_COMB(7)
    CRT_COMB(8) CRT_COMB(9) CRT_COMB(10) CRT_COMB(11) CRT_COMB(12) CRT_COMB(13) CRT_COMB(14)
    CRT_COMB(15) CRT_COMB(16) CRT_COMB(17) CRT_COMB(18) CRT_COMB(19) CRT_COMB(20) CRT_COMB(21)
    CRT_COMB(22) CRT_COMB(23) CRT_COMB(24) CRT_COMB(25) CRT_COMB(26) CRT_COMB(27) CRT_COMB(28)
    CRT_COMB(29) CRT_COMB(30) CRT_COMB(31) CRT_COMB(32)
#undef CRT_COMB
  }
  return check_launch("crt_combine");
}
