// Fused DF-MP2 pair energy on gfx950 fp32 MFMA.
//
//   e_ij = sum_{a,b} T_ab (2 T_ab - T_ba) / (e_i + e_j - v_a - v_b),  T = B_i B_j^T
//
// The reference evaluates this per occupied row with one NKI launch per row,
// materialising T in SBUF and transposing blocks of it on the Tensor Engine
// (trnblas/nki/dispatch.py:4899-5001, driven by :2768-2795; the CPU oracle is
// :2514-2533). Here one launch covers every pair, and T never leaves the
// registers:
//
//  * work item = (pair (i, j), virtual tile pair (A, B) with A <= B), S x S
//    tiles (S = 96: nvir 672 = 7 tiles). For A < B the workgroup computes
//    X = B_i[A] B_j[B]^T and X' = B_j[A] B_i[B]^T, i.e. T[A,B] and T[B,A]^T in
//    the same register layout, and adds
//        sum_{a in A, b in B} 2 (X^2 + X'^2 - X X') / D_ab,
//    which is the (a, b) and (b, a) terms of both tiles (D is symmetric in
//    a, b). For A == B it computes X = T[A,A] only, takes X' = X^T through
//    LDS, and adds sum X (2 X - X') / D. So each T entry is computed once.
//  * pairs: every i <= j with weight 1 (i == j) or 2 (e_ij = e_ji), or an
//    explicit pair list (the per-row / per-window op surface).
//  * the denominator and the energy terms are evaluated in fp64 from the fp32
//    T; each workgroup writes one fp64 partial; a second kernel sums the
//    partials of each pair, then the weighted pair energies, in a fixed order
//    (deterministic, no atomics).
//  * operand panels (four 96 x 16 fp32 panels per k-step) are staged in LDS,
//    double buffered, K-contiguous with 16-byte row padding (conflict-free
//    fragment reads); loads are branch-free buffer loads with zero fill.
//  * items of one pair are consecutive on one XCD (shared L2 for its B_i,
//    B_j panels).
#include "common.hpp"
#include <mutex>
#include <type_traits>

namespace trnblas {

constexpr uint32_t kPeOob = 0x80000000u;

struct PairArgs {
  int nvir, naux;
  const float* Bi;  // fp32 operands (fp32 kernel)
  const uint16_t* Pi;  // bf16x6 / fp16x3 kernels: pieces of Bi / Bj (split kernels)
  const uint16_t* Pj;
  const int32_t* Ei;   // fp16x3: row exponents of Bi / Bj, (occupied row, a) at o * ldE + a
  const int32_t* Ej;
  int ldE;
  int ldv;             // piece row length (naux rounded up to 32)
  int rows_i, rows_j;  // occupied rows of Pi / Pj (pair indices beyond give NaN)
  int64_t ldi_occ;
  const float* Bj;
  int64_t ldj_occ;
  int64_t ld_vir;
  const float* eps_i;
  const float* eps_j;
  const float* eps_vir;
  int nocc;  // implicit mode when pair_i == nullptr
  int npairs;
  const int32_t* pair_i;
  const int32_t* pair_j;
  const double* pair_w;
  int nb, nq;  // virtual tiles, tile pairs (A <= B) per pair
  double* partial;  // [npairs * nq]
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t pe_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7ffffff0,
                                           0x00020000);
}

// Pair index p -> (i, j), i <= j, row-major over the upper triangle of nocc.
__device__ __forceinline__ void tri_pair(int p, int nocc, int& i, int& j) {
  // rows before i: f(i) = i * nocc - i (i - 1) / 2
  const double n = nocc + 0.5;
  int r = (int)(n - sqrt(n * n - 2.0 * (double)p));
  if (r < 0) r = 0;
  if (r > nocc - 1) r = nocc - 1;
  while (r > 0 && (int64_t)r * nocc - (int64_t)r * (r - 1) / 2 > p) --r;
  while (r + 1 < nocc && (int64_t)(r + 1) * nocc - (int64_t)(r + 1) * r / 2 <= p) ++r;
  i = r;
  j = i + (p - (r * nocc - r * (r - 1) / 2));
}

// Tile-pair index q -> (A, B), A <= B, row-major over the upper triangle of nb.
__device__ __forceinline__ void tri_tiles(int q, int nb, int& A, int& B) {
  int a = 0, rem = q;
  while (rem >= nb - a) {
    rem -= nb - a;
    ++a;
  }
  A = a;
  B = a + rem;
}

// Work item -> pair index p (partials at p * nq + q), tile pair q, occupied
// indices (i, j). Items of one pair are consecutive (and xcd_remap keeps
// them on one XCD, sharing that L2 for the pair's panels).
__device__ __forceinline__ void pe_item(const PairArgs& g, int item, int& p, int& q, int& i,
                                        int& j) {
  p = item / g.nq;
  q = item - p * g.nq;
  if (g.pair_i) {
    i = g.pair_i[p];
    j = g.pair_j[p];
  } else {
    tri_pair(p, g.nocc, i, j);
  }
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int S, int BK, bool VEC>
__global__ __launch_bounds__(S / 32 * 64, 2) void pair_energy_kernel(PairArgs g) {
  constexpr int NW = S / 32;  // waves; wave w owns rows 32w..32w+31 of the tile
  constexpr int NT = NW * 64;
  constexpr int NJ = S / 32;  // column blocks per wave
  constexpr int LD = BK + 4;  // padded LDS row (floats)
  constexpr int PANEL = S * LD;
  constexpr int NV = S * BK / 4 / NT;  // float4 groups per thread per panel
  static_assert(NV * 4 * NT == S * BK, "panel split");
  constexpr int STAGE = 4 * PANEL;
  constexpr int XT_LD = S + 1;
  static_assert(2 * STAGE >= S * XT_LD, "transpose buffer fits in the stage buffers");
  __shared__ __attribute__((aligned(16))) float lds[2 * STAGE];
  __shared__ double red[NW];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int item = xcd_remap(blockIdx.x, gridDim.x);
  int p, q, i, j;
  pe_item(g, item, p, q, i, j);
  int TA, TB;
  tri_tiles(q, g.nb, TA, TB);
  const bool diag = TA == TB;
  const int a0 = TA * S, b0 = TB * S;
  const int nvir = g.nvir, naux = g.naux;
  const float* Xi = g.Bi + (int64_t)i * g.ldi_occ;
  const float* Xj = g.Bj + (int64_t)j * g.ldj_occ;

  // panels: 0 = B_i[A], 1 = B_j[A], 2 = B_j[B], 3 = B_i[B]
  const float* pbase[4] = {Xi + (int64_t)a0 * g.ld_vir, Xj + (int64_t)a0 * g.ld_vir,
                           Xj + (int64_t)b0 * g.ld_vir, Xi + (int64_t)b0 * g.ld_vir};
  const int prow[4] = {nvir - a0, nvir - a0, nvir - b0, nvir - b0};
  const int npanel = diag ? 2 : 4;

  i32x4 st[4][NV];
  auto load = [&](int k0) {
#pragma unroll
    for (int pn = 0; pn < 4; ++pn) {
      if (pn >= npanel) break;
      const __amdgpu_buffer_rsrc_t rs = pe_rsrc(pbase[pn] + k0);
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const int idx = tid + v * NT, r = idx / (BK / 4), c = (idx % (BK / 4)) * 4;
        const bool ok = r < prow[pn] && c < naux - k0;
        const uint32_t off = (uint32_t)((r * g.ld_vir + c) * 4);
        if (VEC) {
          st[pn][v] = __builtin_amdgcn_raw_buffer_load_b128(rs, ok ? off : kPeOob, 0, 0);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            st[pn][v][e] = __builtin_amdgcn_raw_buffer_load_b32(
                rs, (ok && c + e < naux - k0) ? off + 4 * e : kPeOob, 0, 0);
        }
      }
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int pn = 0; pn < 4; ++pn) {
      if (pn >= npanel) break;
      float* dst = lds + buf * STAGE + pn * PANEL;
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const int idx = tid + v * NT, r = idx / (BK / 4), c = (idx % (BK / 4)) * 4;
        *reinterpret_cast<i32x4*>(dst + r * LD + c) = st[pn][v];
      }
    }
  };

  f32x16 X[NJ], Xp[NJ];
#pragma unroll
  for (int jb = 0; jb < NJ; ++jb)
#pragma unroll
    for (int r = 0; r < 16; ++r) X[jb][r] = Xp[jb][r] = 0.0f;

  const int nk = (naux + BK - 1) / BK;
  if (nk > 0) {
    load(0);
    store(0);
    __syncthreads();
  }
  const int arow = 32 * w + (lane & 31);
  for (int kt = 0; kt < nk; ++kt) {
    const bool more = kt + 1 < nk;
    if (more) load((kt + 1) * BK);
    const float* buf = lds + (kt & 1) * STAGE;
#pragma unroll
    for (int c = 0; c < BK / 8; ++c) {
      const int kk = c * 8 + (lane >> 5) * 4;
      const f32x4 fai = *reinterpret_cast<const f32x4*>(buf + 0 * PANEL + arow * LD + kk);
      f32x4 fbj[NJ];
#pragma unroll
      for (int jb = 0; jb < NJ; ++jb)
        fbj[jb] = *reinterpret_cast<const f32x4*>(buf + (diag ? 1 : 2) * PANEL +
                                                  (32 * jb + (lane & 31)) * LD + kk);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int jb = 0; jb < NJ; ++jb)
          X[jb] = __builtin_amdgcn_mfma_f32_32x32x2f32(fai[e], fbj[jb][e], X[jb], 0, 0, 0);
      if (!diag) {
        const f32x4 faj = *reinterpret_cast<const f32x4*>(buf + 1 * PANEL + arow * LD + kk);
        f32x4 fbi[NJ];
#pragma unroll
        for (int jb = 0; jb < NJ; ++jb)
          fbi[jb] = *reinterpret_cast<const f32x4*>(buf + 3 * PANEL +
                                                    (32 * jb + (lane & 31)) * LD + kk);
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int jb = 0; jb < NJ; ++jb)
            Xp[jb] = __builtin_amdgcn_mfma_f32_32x32x2f32(faj[e], fbi[jb][e], Xp[jb], 0, 0, 0);
      }
    }
    if (more) store((kt + 1) & 1);
    __syncthreads();
  }

  // Lane l of a 32x32 block holds column l % 32 and rows 8 (r/4) + 4 (l/32) + r % 4.
  if (diag) {
    // X' = X^T through LDS (the stage buffers are free after the last barrier).
    float* xt = lds;
#pragma unroll
    for (int jb = 0; jb < NJ; ++jb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int a = 32 * w + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        const int b = 32 * jb + (lane & 31);
        xt[a * XT_LD + b] = X[jb][r];
      }
    __syncthreads();
#pragma unroll
    for (int jb = 0; jb < NJ; ++jb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int a = 32 * w + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        const int b = 32 * jb + (lane & 31);
        Xp[jb][r] = xt[b * XT_LD + a];
      }
  }

  const double eo = (double)g.eps_i[i] + (double)g.eps_j[j];
  double sum = 0.0;
#pragma unroll
  for (int jb = 0; jb < NJ; ++jb) {
    const int b = b0 + 32 * jb + (lane & 31);
    const double eb = b < nvir ? (double)g.eps_vir[b] : 0.0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int a = a0 + 32 * w + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
      if (a < nvir && b < nvir) {
        const double x = X[jb][r], xp = Xp[jb][r];
        const double d = eo - (double)g.eps_vir[a] - eb;
        const double num = diag ? x * (2.0 * x - xp) : 2.0 * (x * x + xp * xp - x * xp);
        sum += num / d;
      }
    }
  }
  sum = wave_sum(sum);
  if (lane == 0) red[w] = sum;
  __syncthreads();
  if (tid == 0) {
    double t = 0.0;
#pragma unroll
    for (int k = 0; k < NW; ++k) t += red[k];
    g.partial[(int64_t)p * g.nq + q] = t;
  }
}

// Per-pair sums of the partials (fixed order), then the weighted total.
__global__ __launch_bounds__(256) void pair_sum_kernel(const double* partial, int npairs,
                                                       int nq, double* e_pair) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= npairs) return;
  const double* src = partial + (int64_t)p * nq;
  double s = 0.0;
  for (int q = 0; q < nq; ++q) s += src[q];
  e_pair[p] = s;
}

// Zero fill (the empty-sum results): a kernel rather than hipMemsetAsync, so
// the call records no memset node when a caller captures it in a graph.
__global__ __launch_bounds__(256) void zero_f64_kernel(double* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0;
}

__global__ __launch_bounds__(1024) void pair_total_kernel(const double* e_pair, int npairs,
                                                          int nocc, const int32_t* pair_i,
                                                          const int32_t* pair_j,
                                                          const double* pair_w, double* total) {
  __shared__ double red[16];
  const int tid = threadIdx.x;
  double s = 0.0;
  for (int p = tid; p < npairs; p += blockDim.x) {
    double w;
    if (pair_i) {
      w = pair_w ? pair_w[p] : 1.0;
    } else {
      int i, j;
      tri_pair(p, nocc, i, j);
      w = i == j ? 1.0 : 2.0;
    }
    s += w * e_pair[p];
  }
  s = wave_sum(s);
  if ((tid & 63) == 0) red[tid >> 6] = s;
  __syncthreads();
  if (tid == 0) {
    double t = 0.0;
    for (int k = 0; k < (int)(blockDim.x >> 6); ++k) t += red[k];
    *total = t;
  }
}

// ── bf16x6: fp32 products from three bf16 pieces on bf16 MFMA ───────────────
//
// x = hi + mid + lo exactly (each piece an 8-bit-significand bf16), and
//   x y ~= hi_x hi_y + hi_x mid_y + mid_x hi_y + hi_x lo_y + mid_x mid_y + lo_x hi_y,
// dropping mid_x lo_y + lo_x mid_y + lo_x lo_y (< 2^-23 |x y|). Each bf16
// product is exact in fp32; the products of one 32-wide k slice are summed by
// the MFMA, the slices by fp32 adds, so a dot product carries fp32
// accumulation error plus that 2^-23 term. gfx950 runs
// v_mfma_f32_16x16x32_bf16 at 16x the rate of v_mfma_f32_32x32x2_f32, so the
// six products cost 6/16 of one fp32 MFMA product.

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

// Two floats to packed bf16, round to nearest even (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  const bf16x2 h = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, h);
}

// hi = rn_bf16(x), mid = rn_bf16(x - hi), lo = rn_bf16(x - hi - mid) for a
// pair of floats, packed: both differences are exact in fp32 and lo holds the
// last <= 8 bits exactly, so x == hi + mid + lo for every normal x. Eleven
// VALU operations per pair.
__device__ __forceinline__ void split_pair(float x0, float x1, uint32_t& H, uint32_t& M,
                                           uint32_t& L) {
  // The low half goes to the top through a byte permute (v_perm_b32,
  // [b1 b0 0 0]): written as H << 16 the compiler rebuilds it with a second
  // conversion of x0 (two more VALU operations per pair).
  H = cvt_pk_bf16(x0, x1);
  const float r0 = x0 - __uint_as_float(__builtin_amdgcn_perm(H, 0u, 0x05040c0cu)),
              r1 = x1 - __uint_as_float(H & 0xffff0000u);
  M = cvt_pk_bf16(r0, r1);
  const float s0 = r0 - __uint_as_float(__builtin_amdgcn_perm(M, 0u, 0x05040c0cu)),
              s1 = r1 - __uint_as_float(M & 0xffff0000u);
  L = cvt_pk_bf16(s0, s1);
}

__device__ __forceinline__ void split_bf16x3(const f32x4& x, i32x2& hi, i32x2& mid, i32x2& lo) {
  uint32_t h0, m0, l0, h1, m1, l1;
  split_pair(x[0], x[1], h0, m0, l0);
  split_pair(x[2], x[3], h1, m1, l1);
  hi = i32x2{(int)h0, (int)h1};
  mid = i32x2{(int)m0, (int)m1};
  lo = i32x2{(int)l0, (int)l1};
}

// ── fp16x3: fp32 products from two fp16 pieces on f16 MFMA ──────────────────
//
// Each row (o, a) of an operand is scaled by 2^e(o, a) so its largest
// magnitude lies in [2^14, 2^15); then xs = x 2^e = hi + lo + r with
// hi = rn_f16(xs), lo = rn_f16(xs - hi) (xs - hi is exact in fp32) and
// |r| <= 2^-22 |xs| + 2^-25, and
//   xs ys ~= hi_x hi_y + hi_x lo_y + lo_x hi_y,
// dropping lo_x lo_y (<= 2^-22 |xs ys|): the two-piece split of Ootomo and
// Yokota (SGEMM emulation on fp16 tensor cores, 2022) with the scale taken
// per row instead of the lo piece, so no separate correction accumulator is
// needed. The row scale keeps every element above the row maximum times
// 2^-17 inside fp16's normal range; the smaller ones keep an absolute error
// below 2^-39 of the row maximum. Each fp16 product is exact in fp32, and the
// kernels sum a slice's products on the MFMA and the slices in fp32 as for
// bf16x6. T_ab = acc 2^-(e(i, a) + e(j, b)) is formed in fp64. Three products
// instead of six halve the MFMA work, and two pieces move two thirds of the
// operand bytes.

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Arithmetic of the split kernels: NPC pieces per element, the products
// (piece of A, piece of B) smallest first, and the MFMA on 16-byte fragments.
template <int NPC>
struct PeMath;
template <>
struct PeMath<3> {  // bf16x6
  static constexpr int NPROD = 6;
  static constexpr int ka[6] = {2, 1, 0, 1, 0, 0}, kb[6] = {0, 1, 2, 0, 1, 0};
  static __device__ __forceinline__ f32x4 mma(i32x4 a, i32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <>
struct PeMath<2> {  // fp16x3
  static constexpr int NPROD = 3;
  static constexpr int ka[3] = {1, 0, 0}, kb[3] = {0, 1, 0};
  static __device__ __forceinline__ f32x4 mma(i32x4 a, i32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// Scale of T_ab from the row exponents (1 for bf16x6, which is unscaled).
template <int NPC>
__device__ __forceinline__ double pe_scale(const PairArgs& g, const int32_t* Ea, int oa, int a,
                                           const int32_t* Eb, int ob, int b) {
  if constexpr (NPC == 2)
    return ldexp(1.0, -(Ea[(int64_t)oa * g.ldE + a] + Eb[(int64_t)ob * g.ldE + b]));
  else
    return 1.0;
}

__device__ __forceinline__ void split_f16x2(const f32x4& x, int e, i32x2& hi, i32x2& lo) {
  _Float16 h[4], l[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const float xs = ldexpf(x[u], e);
    h[u] = (_Float16)xs;
    l[u] = (_Float16)(xs - (float)h[u]);
  }
  auto pk = [](_Float16 a, _Float16 b) {
    return (int)((uint32_t)__builtin_bit_cast(uint16_t, a) |
                 ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16));
  };
  hi = i32x2{pk(h[0], h[1]), pk(h[2], h[3])};
  lo = i32x2{pk(l[0], l[1]), pk(l[2], l[3])};
}

constexpr int kX3S = 96, kX3BK = 32;

// LDS slot of 16-byte group `grp` of panel row `r` (rows of 64 bytes): the
// XOR makes every 8 (and every 16) consecutive rows of one group land on
// distinct 16-byte bank groups, so fragment reads and stage writes are
// conflict free without padding.
__device__ __forceinline__ int x3_slot(int r, int grp) { return grp ^ (((r >> 1) ^ (r >> 2)) & 3); }

// fp32 operand X (n, nvir, naux), strides (ld_occ, ld_vir, 1), as its NPC
// pieces p (bf16x6: 0 hi, 1 mid, 2 lo; fp16x3: 0 hi, 1 lo of the row-scaled
// value) in 32-wide k slices s, rows taken in pairs: element (o, a, p, k),
// a = 2 m + d, k = 32 s + c, at
//   ((((o * nvp + m) * nk + s) * NPC + p) * 2 + d) * 32 + c,   nvp = ceil(nvir / 2),
// nk = ldv / 32. The 64 bytes of one row's slice of one piece share a
// 128-byte line with the other row of its pair, and the pieces of a row
// pair's slice are NPC x 128 contiguous bytes, so a wave's 16-row load reads
// 8 whole lines (half lines would cost the address path twice as much).
// Columns [naux, ldv) are zero, and so is the second row of the last pair
// of an odd nvir.
__device__ __forceinline__ uint16_t* piece_slot(uint16_t* P, int npc, int nvir, int ldv, int o,
                                                int a, int k0) {
  const int nvp = (nvir + 1) >> 1, nk = ldv >> 5;
  return P + ((((int64_t)o * nvp + (a >> 1)) * nk + (k0 >> 5)) * npc * 2 + (a & 1)) * 32 + (k0 & 31);
}

// 8 consecutive k of row a of X from k0 (zeros past naux and for a >= nvir).
template <bool VEC>
__device__ __forceinline__ void load_row8(const float* src, int nvir, int naux, int a, int k0,
                                          f32x4& x0, f32x4& x1) {
  if (a >= nvir) {
    x0 = x1 = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  } else if (VEC && k0 + 8 <= naux) {
    x0 = *reinterpret_cast<const f32x4*>(src + k0);
    x1 = *reinterpret_cast<const f32x4*>(src + k0 + 4);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x0[e] = k0 + e < naux ? src[k0 + e] : 0.0f;
      x1[e] = k0 + 4 + e < naux ? src[k0 + 4 + e] : 0.0f;
    }
  }
}

// bf16x6 pieces: one thread per 8 consecutive k of a row (rows of the padded
// 2 ceil(nvir / 2)); `total` = n * 2 ceil(nvir / 2) * ldv / 8 threads.
template <bool VEC>
__global__ __launch_bounds__(256) void split_planes_kernel(int nvir, int naux, int ldv, int total,
                                                          const float* X, int64_t ld_occ,
                                                          int64_t ld_vir, uint16_t* P) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int gpr = ldv >> 3, nv2 = (nvir + 1) & ~1;
  const int row = idx / gpr, k0 = (idx - row * gpr) * 8;
  const int o = row / nv2, a = row - o * nv2;
  f32x4 x0, x1;
  load_row8<VEC>(X + (int64_t)o * ld_occ + (int64_t)a * ld_vir, nvir, naux, a, k0, x0, x1);
  uint16_t* dst = piece_slot(P, 3, nvir, ldv, o, a, k0);
  i32x2 h0, m0, l0, h1, m1, l1;
  split_bf16x3(x0, h0, m0, l0);
  split_bf16x3(x1, h1, m1, l1);
  *reinterpret_cast<i32x4*>(dst) = i32x4{h0[0], h0[1], h1[0], h1[1]};
  *reinterpret_cast<i32x4*>(dst + 64) = i32x4{m0[0], m0[1], m1[0], m1[1]};
  *reinterpret_cast<i32x4*>(dst + 128) = i32x4{l0[0], l0[1], l1[0], l1[1]};
}

// fp16x3 pieces and row exponents in one pass over X: one wave per row pair
// (o, m) of the padded layout. Row a's exponent is e = 15 - E for its
// largest magnitude f 2^E, f in [0.5, 1), so the row's values times 2^e lie
// below 2^15; e = 0 for a zero or non-finite row and for the padding row of
// an odd nvir; it goes to E[o * 2 nvp + a]. The wave's first sweep takes both
// rows' maxima, the second splits them, re-reading the same lines (from
// cache, so HBM sees X once). Lane l covers row 2 m + ((l >> 2) & 1), k =
// 256 j + 32 (l >> 3) + 8 (l & 3) .. + 7 in sweep step j: 8 whole slices of
// both rows per step. `nrp` = n ceil(nvir / 2) row pairs.
template <bool VEC>
__global__ __launch_bounds__(256) void split_f16x3_kernel(int nvir, int naux, int ldv, int nrp,
                                                         const float* X, int64_t ld_occ,
                                                         int64_t ld_vir, int32_t* E, uint16_t* P) {
  const int rp = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (rp >= nrp) return;
  const int nvp = (nvir + 1) >> 1, o = rp / nvp, m = rp - o * nvp;
  const int a = 2 * m + ((lane >> 2) & 1);
  const int kl = 32 * (lane >> 3) + 8 * (lane & 3);
  const float* src = X + (int64_t)o * ld_occ + (int64_t)(a < nvir ? a : 0) * ld_vir;
  float mx = 0.0f;
#pragma unroll 4
  for (int k0 = kl; k0 < ldv; k0 += 256) {
    f32x4 x0, x1;
    load_row8<VEC>(src, nvir, naux, a, k0, x0, x1);
#pragma unroll
    for (int u = 0; u < 4; ++u) mx = fmaxf(mx, fmaxf(fabsf(x0[u]), fabsf(x1[u])));
  }
  // the maximum over the 32 lanes of the same row (lane bit 2 picks the row)
#pragma unroll
  for (int off = 1; off < 64; off <<= 1)
    if (off != 4) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  int e = 0;
  if (mx > 0.0f && mx <= 3.402823466e38f) {
    int ex;
    frexpf(mx, &ex);
    e = 15 - ex;
  }
  if ((lane & ~4) == 0) E[(int64_t)o * 2 * nvp + a] = e;
#pragma unroll 4
  for (int k0 = kl; k0 < ldv; k0 += 256) {
    f32x4 x0, x1;
    load_row8<VEC>(src, nvir, naux, a, k0, x0, x1);
    uint16_t* dst = piece_slot(P, 2, nvir, ldv, o, a, k0);
    i32x2 h0, l0, h1, l1;
    split_f16x2(x0, e, h0, l0);
    split_f16x2(x1, e, h1, l1);
    *reinterpret_cast<i32x4*>(dst) = i32x4{h0[0], h0[1], h1[0], h1[1]};
    *reinterpret_cast<i32x4*>(dst + 64) = i32x4{l0[0], l0[1], l1[0], l1[1]};
  }
}

// Work item = (pair, virtual tile pair A <= B) as in pair_energy_kernel, 96 x 96
// tiles, 4 waves, wave w on the 48 x 48 quadrant (w & 1, w >> 1) as 3 x 3
// blocks of 16 x 16. Off-diagonal items run two passes over k in one
// pipeline: X = B_i[A] B_j[B]^T, then X' = B_j[A] B_i[B]^T (both held in
// registers); diagonal items run the first pass only (B = A). The operands
// come pre-split (split_planes_kernel), so a k-step spends no VALU on the
// split. A stage is one 32-wide k slice of the NPC pieces x 2 panels of the
// running pass (36 KiB for bf16x6, 24 KiB for fp16x3); LDS holds two stages
// (the epilogue's 72 KiB, two workgroups per CU) and two register sets hold
// the next two slices in flight: slice t is multiplied from LDS while slices
// t + 1 and t + 2 load, and slice t + 1 goes to LDS at the end of step t.
// The MFMA partial of each block spans two slices (2 NPROD products) before
// it joins the running sum by an fp32 add.
template <int NPC>
__global__ __launch_bounds__(256, 2) void pair_energy_x3_kernel(PairArgs g) {
  using M = PeMath<NPC>;
  constexpr int S = kX3S, BK = kX3BK;
  constexpr int STAGE = 2 * NPC * S * BK;  // 16-bit elements: NPC pieces x 2 panels
  constexpr int NU = NPC * 3;              // 1 KiB loads per wave per stage
  static_assert(STAGE * 2 == NPC * 12 * 1024 && S == 96 && BK == 32, "3 KiB per piece per wave");
  constexpr int LDS_ELEMS = 2 * STAGE > 2 * S * S * 2 ? 2 * STAGE : 2 * S * S * 2;
  __shared__ __attribute__((aligned(16))) uint16_t lds[LDS_ELEMS];  // stages / epilogue
  __shared__ double red[4];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int item = xcd_remap(blockIdx.x, gridDim.x);
  int p, q, i, j;
  pe_item(g, item, p, q, i, j);
  if ((unsigned)i >= (unsigned)g.rows_i || (unsigned)j >= (unsigned)g.rows_j) {
    if (tid == 0) g.partial[(int64_t)p * g.nq + q] = __builtin_nan("");
    return;
  }
  int TA, TB;
  tri_tiles(q, g.nb, TA, TB);
  const bool diag = TA == TB;
  const int a0 = TA * S, b0 = TB * S;
  const int nvir = g.nvir, ldv = g.ldv;
  const int64_t ostride = (int64_t)((nvir + 1) >> 1) * 2 * NPC * ldv;  // one occupied row
  const uint16_t* Xi = g.Pi + i * ostride;
  const uint16_t* Xj = g.Pj + j * ostride;
  const int nk = ldv / BK;  // even: ldv is a multiple of 2 BK
  const int nsteps = diag ? nk : 2 * nk;

  // LDS stage layout [side][piece][row][BK], side 0 the A side (rows a0:
  // B_i in pass 0, B_j in pass 1), side 1 the B side (rows b0: B_j, then
  // B_i). Waves 2 s and 2 s + 1 fill side s, 6 NPC row blocks of 16 rows x 64
  // bytes (one 16-byte load per lane each), block e = piece * 6 + blk at
  // stage offset e KiB; wave h = w >> 1 of the side takes e = h + 2 u. Lane
  // l carries LDS slot l % 4 of row 16 blk + l / 4, i.e. the global 16-byte
  // group x3_slot(row, l % 4), and stores it lane-linearly; lanes 8 v ..
  // 8 v + 7 read one 128-byte line (a row pair of split_planes_kernel's
  // layout). The lane's byte offset from the panel's first row pair is
  // fixed; the slice offset (NPC x 128 bytes per slice) goes into soffset and the
  // panel (operand, rows) into the buffer resource, one per pass. Rows past
  // nvir read as zeros.
  const int side = w & 1, h = w >> 1;
  const int rbase = side ? b0 : a0;
  const int lr = lane >> 2;
  uint32_t voff[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int e = h + 2 * u, pc = e / 6, r = 16 * (e - 6 * pc) + lr;
    voff[u] = r < nvir - rbase ? (uint32_t)(((r >> 1) * nk * (NPC * 64) + pc * 64 + (r & 1) * 32 +
                                             8 * x3_slot(r, lane & 3)) *
                                            2)
                               : kPeOob;
  }
  const int64_t prow = (int64_t)(rbase >> 1) * nk * (NPC * 64);  // rbase is even
  const __amdgpu_buffer_rsrc_t rs0 = pe_rsrc((side ? Xj : Xi) + prow);
  const __amdgpu_buffer_rsrc_t rs1 = pe_rsrc((side ? Xi : Xj) + prow);
  // Past the last slice the loads still issue (every step issues the same
  // NU, which keeps the compiler's wait counts exact), re-reading the last
  // slice (L2-resident); their data is never stored.
  i32x4 stg[2][NU];  // slice t in set t & 1 between its load and its store
  auto load = [&](int t, i32x4(&set)[NU]) {
    if (t >= nsteps) t = nsteps - 1;
    const bool pass1 = t >= nk;
    const int sl = pass1 ? t - nk : t;
    const __amdgpu_buffer_rsrc_t rs = pass1 ? rs1 : rs0;
#pragma unroll
    for (int u = 0; u < NU; ++u)
      set[u] = __builtin_amdgcn_raw_buffer_load_b128(
          rs, voff[u], __builtin_amdgcn_readfirstlane(sl * NPC * 128), 0);
  };
  auto store = [&](const i32x4(&set)[NU], int buf) {
    uint16_t* dst = lds + buf * STAGE + side * (STAGE / 2) + h * 512 + lane * 8;
#pragma unroll
    for (int u = 0; u < NU; ++u) *reinterpret_cast<i32x4*>(dst + u * 1024) = set[u];
  };

  // The fragment row of a lane is row0 + 16 blk + (lane & 15) with row0 a
  // multiple of 16, so its LDS slot depends on the lane only.
  const int ar0 = 48 * (w & 1), br0 = 48 * (w >> 1);
  const int fslot = 8 * x3_slot(lane & 15, lane >> 4);
  f32x4 accX[3][3], accP[3][3], part[3][3];
#pragma unroll
  for (int rb = 0; rb < 3; ++rb)
#pragma unroll
    for (int cb = 0; cb < 3; ++cb) accX[rb][cb] = accP[rb][cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // Step t (global over both passes; P = t & 1 is static): slice t is in LDS
  // buffer P (the barrier publishes it and retires every read of buffer
  // 1 - P), set P is free (its slice t went to LDS in step t - 1) and takes
  // slice t + 2, slice t is multiplied (the NPROD products of each block,
  // smallest first, into its partial: with TWO the partial starts at zero
  // when FIRST and spans two slices, added to the pass's sum below (bf16x6
  // both passes, fp16x3 pass 0); otherwise it starts at zero every slice and
  // is added to the pass's sum at once (fp16x3 pass 1), the order of
  // pair_energy_quad_kernel), then set 1 - P (slice t + 1) goes to buffer
  // 1 - P.
  auto step = [&](auto P_, auto FIRST_, auto TWO_, int t, f32x4(&acc)[3][3]) {
    constexpr int P = decltype(P_)::value;
    constexpr bool FIRST = decltype(FIRST_)::value;
    constexpr bool TWO = decltype(TWO_)::value;  // two-slice partials
    __syncthreads();
    load(t + 2, stg[P]);
    const uint16_t* buf = lds + P * STAGE;
    auto frag = [&](int pc, int sd, int r) {
      return *reinterpret_cast<const i32x4*>(buf + ((sd * NPC + pc) * S + r) * BK + fslot);
    };
    i32x4 fa[3][NPC];
#pragma unroll
    for (int rb = 0; rb < 3; ++rb)
#pragma unroll
      for (int pc = 0; pc < NPC; ++pc) fa[rb][pc] = frag(pc, 0, ar0 + 16 * rb + (lane & 15));
#pragma unroll
    for (int cb = 0; cb < 3; ++cb) {
      i32x4 fb[NPC];
#pragma unroll
      for (int pc = 0; pc < NPC; ++pc) fb[pc] = frag(pc, 1, br0 + 16 * cb + (lane & 15));
      if constexpr (!TWO) {
#pragma unroll
        for (int e = 0; e < M::NPROD; ++e)
#pragma unroll
          for (int rb = 0; rb < 3; ++rb)
            part[rb][cb] = M::mma(fa[rb][M::ka[e]], fb[M::kb[e]],
                                  e == 0 ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : part[rb][cb]);
#pragma unroll
        for (int rb = 0; rb < 3; ++rb) acc[rb][cb] += part[rb][cb];
      } else {
#pragma unroll
        for (int rb = 0; rb < 3; ++rb)
          part[rb][cb] = M::mma(fa[rb][M::ka[0]], fb[M::kb[0]],
                                FIRST ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : part[rb][cb]);
#pragma unroll
        for (int e = 1; e < M::NPROD; ++e) {
#pragma unroll
          for (int rb = 0; rb < 3; ++rb)
            part[rb][cb] = M::mma(fa[rb][M::ka[e]], fb[M::kb[e]], part[rb][cb]);
        }
      }
    }
    if (t + 1 < nsteps) store(stg[1 - P], 1 - P);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using T = std::true_type;
  using F = std::false_type;
  // One pass: slice pairs (t even, t + 1); bf16x6 adds each partial to the
  // pass's sum in fp32.
  auto run_pass = [&](f32x4(&acc)[3][3], int t0, auto TWO_) {
    constexpr bool TWO = decltype(TWO_)::value;
    for (int u = 0; u < nk; u += 2) {
      step(I0(), T(), TWO_, t0 + u, acc);
      step(I1(), F(), TWO_, t0 + u + 1, acc);
      if constexpr (TWO) {
#pragma unroll
        for (int rb = 0; rb < 3; ++rb)
#pragma unroll
          for (int cb = 0; cb < 3; ++cb) acc[rb][cb] += part[rb][cb];
      }
    }
  };

  if (nsteps > 0) {
    load(0, stg[0]);
    load(1, stg[1]);
    store(stg[0], 0);
  }
  // fp16x3 sums X over two-slice partials and X' over one-slice partials,
  // as pair_energy_quad_kernel does; bf16x6 both over two-slice partials
  run_pass(accX, 0, T());
  if (!diag) run_pass(accP, nk, std::integral_constant<bool, NPC != 2>());
  __syncthreads();  // all fragment reads done before the epilogue reuses LDS

  // Lane l of a 16 x 16 block holds column l % 16 and rows 4 (l / 16) + r.
  // Off-diagonal: X at [0, S*S), X' at [S*S, 2 S*S), row stride S.
  // Diagonal: X at row stride S + 1 (conflict-free transposed reads).
  float* xs = reinterpret_cast<float*>(lds);
  const int ldx = diag ? S + 1 : S;
#pragma unroll
  for (int rb = 0; rb < 3; ++rb)
#pragma unroll
    for (int cb = 0; cb < 3; ++cb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int a = ar0 + 16 * rb + 4 * (lane >> 4) + r;
        const int b = br0 + 16 * cb + (lane & 15);
        xs[a * ldx + b] = accX[rb][cb][r];
        if (!diag) xs[S * S + a * S + b] = accP[rb][cb][r];
      }
  __syncthreads();

  const double eo = (double)g.eps_i[i] + (double)g.eps_j[j];
  double sum = 0.0;
#pragma unroll 4
  for (int e = 0; e < S * S / 256; ++e) {
    const int idx = tid + 256 * e, a = idx / S, b = idx - a * S;
    if (a0 + a < nvir && b0 + b < nvir) {
      // X = B_i[A] B_j[B]^T, X' = B_j[A] B_i[B]^T (diagonal: X' = X^T)
      const double x = xs[a * ldx + b] * pe_scale<NPC>(g, g.Ei, i, a0 + a, g.Ej, j, b0 + b);
      const double xp = diag ? xs[b * ldx + a] * pe_scale<NPC>(g, g.Ei, i, a0 + b, g.Ej, j, a0 + a)
                             : xs[S * S + a * S + b] *
                                   pe_scale<NPC>(g, g.Ej, j, a0 + a, g.Ei, i, b0 + b);
      const double d = eo - (double)g.eps_vir[a0 + a] - (double)g.eps_vir[b0 + b];
      sum += (diag ? x * (2.0 * x - xp) : 2.0 * (x * x + xp * xp - x * xp)) / d;
    }
  }
  sum = wave_sum(sum);
  if (lane == 0) red[w] = sum;
  __syncthreads();
  if (tid == 0) g.partial[(int64_t)p * g.nq + q] = (red[0] + red[1]) + (red[2] + red[3]);
}

// Couples of the implicit walk: row i's pairs (i, j), j = i .. nocc - 1,
// two at a time: couple c = (i, j0 = i + 2 h, j0 + 1) for h <
// ceil((nocc - i) / 2); the second pair is absent when j0 + 1 == nocc. Rows
// before i hold C(i) = sum_{t < i} ceil((nocc - t) / 2) = F(nocc + 1) -
// F(nocc + 1 - i) couples, F(x) = sum_{u <= x} floor(u / 2).
__device__ __forceinline__ int64_t half_floor_sum(int64_t x) {
  const int64_t m = x >> 1;
  return (x & 1) ? m * (m + 1) : m * m;
}
__host__ __device__ __forceinline__ int64_t pe_couples(int64_t n) {
  const int64_t m = (n + 1) >> 1;  // F(n + 1)
  return ((n + 1) & 1) ? m * (m + 1) : m * m;
}
__device__ __forceinline__ void couple_of(int c, int n, int& i, int& j0) {
  auto before = [&](int r) { return half_floor_sum(n + 1) - half_floor_sum(n + 1 - r); };
  const double nn = n + 1.0;
  int r = (int)(nn - sqrt(fmax(0.0, nn * nn - 4.0 * (double)c)));
  if (r < 0) r = 0;
  if (r > n - 1) r = n - 1;
  while (r > 0 && before(r) > c) --r;
  while (r + 1 < n && before(r + 1) <= c) ++r;
  i = r;
  j0 = r + 2 * (c - (int)before(r));
}

// The implicit walk two pairs at a time (bf16x6): work item = (couple (i,
// j0, j1), tile pair A <= B). Both pairs share B_i, so a k-step stages three
// 96-row panels (54 KiB) for two 96 x 96 outputs where two single-pair
// workgroups stage four: a quarter fewer operand bytes per product, which is
// what bounds pair_energy_x3_kernel. 8 waves, one workgroup per CU: waves 4 g .. 4 g + 3
// compute pair g of the couple, each the 48 x 48 quadrant (w & 1, w >> 1) as
// in pair_energy_x3_kernel, with the same pieces, MFMA order, two-slice
// partials and two-deep register pipeline. Stage slots: 0 = the shared panel
// (B_i[A] in pass 0, B_i[B] in pass 1), 1 + g = pair g's (B_jg[B], then
// B_jg[A]); a single-pair couple runs pair 0 twice and drops the copy.
template <int NPC>
__global__ __launch_bounds__(512, 1) void pair_energy_x3c_kernel(PairArgs g) {
  static_assert(NPC == 3, "bf16x6; fp16x3 runs pair_energy_quad_kernel");
  using M = PeMath<NPC>;
  constexpr int S = kX3S, BK = kX3BK;
  constexpr int SLOT = NPC * S * BK;  // 16-bit elements of one panel slice, NPC pieces
  constexpr int STAGE = 3 * SLOT;
  constexpr int NQ = STAGE * 2 / 1024;  // 1 KiB load instructions per stage (18 NPC)
  constexpr int NL = (NQ + 7) / 8;      // per wave (the spare ones re-load, unstored)
  constexpr int BPS = NPC * 6;          // load blocks per slot
  static_assert(NQ == 18 * NPC && S == 96 && BK == 32, "stage split");
  constexpr int LDS_ELEMS = 2 * STAGE > S * (S + 1) * 4 ? 2 * STAGE : S * (S + 1) * 4;
  __shared__ __attribute__((aligned(16))) uint16_t lds[LDS_ELEMS];  // stages / diagonal epilogue
  __shared__ double red[8];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gp = w >> 2, qd = w & 3;
  const int item = xcd_remap(blockIdx.x, gridDim.x);
  const int c = item / g.nq, q = item - c * g.nq;
  int i, j0;
  couple_of(c, g.nocc, i, j0);
  const bool two = j0 + 1 < g.nocc;
  const int j1 = two ? j0 + 1 : j0;
  int TA, TB;
  tri_tiles(q, g.nb, TA, TB);
  const bool diag = TA == TB;
  const int a0 = TA * S, b0 = TB * S;
  const int nvir = g.nvir, ldv = g.ldv;
  const int nk = ldv / BK;  // even
  const int nsteps = diag ? nk : 2 * nk;
  const int64_t ostride = (int64_t)((nvir + 1) >> 1) * 2 * NPC * ldv;

  // Load instruction qq = slot * 6 NPC + piece * 6 + blk (rows 16 blk ..
  // 16 blk + 15 of that slot's panel) fills stage offset qq KiB; wave w
  // issues qq = w + 8 u. The lane offsets are those of pair_energy_x3_kernel
  // (row-pair layout, one 128-byte line per 8 lanes): row r = 16 blk + l / 4
  // and x3_slot(r, .) depends on r mod 8 only, so the lane's part (row l / 4
  // of the block) is one offset for every load, and the wave-uniform part
  // (16 blk rows and the piece) moves the resource's base and shortens its
  // range by as much. A panel's resource spans its valid row pairs only (the
  // padding row of an odd nvir is zero), so rows past nvir read as zeros:
  // the range check sees the lane offset (not the soffset, which carries
  // the k slice).
  const int lr = lane >> 2;
  const uint32_t voff =
      (uint32_t)(((lr >> 1) * nk * (NPC * 64) + (lr & 1) * 32 + 8 * x3_slot(lr, lane & 3)) * 2);
  // Panel (slot sl, pass ps): operand rows from rbase; its resource spans the
  // valid row pairs only. Wave-uniform scalars, computed per load.
  const int pairsA = min((nvir - a0 + 1) >> 1, S / 2), pairsB = min((nvir - b0 + 1) >> 1, S / 2);
  const int64_t rowA = (int64_t)(a0 >> 1) * nk * (NPC * 64),
                rowB = (int64_t)(b0 >> 1) * nk * (NPC * 64);
  i32x4 stg[2][NL];
  auto load = [&](int t, i32x4(&set)[NL]) __attribute__((always_inline)) {
    if (t >= nsteps) t = nsteps - 1;  // keeps every step at NL loads (exact wait counts)
    const int ps = t >= nk ? 1 : 0, sl0 = ps ? t - nk : t;
#pragma unroll
    for (int u = 0; u < NL; ++u) {
      const int qq = w + 8 * u < NQ ? w + 8 * u : w + 8 * u - 8;
      const int sl = qq / BPS, e = qq - sl * BPS, pc = e / 6;
      const int uo = ((8 * (e - 6 * pc)) * nk * (NPC * 64) + pc * 64) * 2;  // bytes
      const bool onA = (sl == 0) == (ps == 0);  // the panel's rows are the A tile's
      // operand row i, j0 or j1 by arithmetic (a select chain becomes a table in memory)
      const int o = i + (sl > 0) * (j0 - i) + (sl > 1) * (j1 - j0);
      const int nrec = (onA ? pairsA : pairsB) * nk * NPC * 128 - uo;
      const char* base =
          reinterpret_cast<const char*>(g.Pi + o * ostride + (onA ? rowA : rowB)) + uo;
      // (readfirstlane: an offset the compiler keeps in a VGPR after a select
      // wraps the load in a loop over the lanes' distinct values)
      const int soff = __builtin_amdgcn_readfirstlane(sl0 * NPC * 128);
      set[u] = __builtin_amdgcn_raw_buffer_load_b128(
          __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0, nrec > 0 ? nrec : 0,
                                            0x00020000),
          voff, soff, 0);
    }
  };
  auto store = [&](const i32x4(&set)[NL], int buf) __attribute__((always_inline)) {
    uint16_t* dst = lds + buf * STAGE + w * 512 + lane * 8;
#pragma unroll
    for (int u = 0; u < NL; ++u)
      if (w + 8 * u < NQ) *reinterpret_cast<i32x4*>(dst + u * 8 * 512) = set[u];
  };

  const int ar0 = 48 * (qd & 1), br0 = 48 * (qd >> 1);
  const int fslot = 8 * x3_slot(lane & 15, lane >> 4);
  f32x4 accX[3][3], accP[3][3], part[3][3];
#pragma unroll
  for (int rb = 0; rb < 3; ++rb)
#pragma unroll
    for (int cb = 0; cb < 3; ++cb) accX[rb][cb] = accP[rb][cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  auto step = [&](auto P_, auto FIRST_, int t) __attribute__((always_inline)) {
    constexpr int P = decltype(P_)::value;
    constexpr bool FIRST = decltype(FIRST_)::value;
    __syncthreads();
    const int ps = t >= nk ? 1 : 0;
    const uint16_t* bufA = lds + P * STAGE + (ps ? 1 + gp : 0) * SLOT;
    const uint16_t* bufB = lds + P * STAGE + (ps ? 0 : 1 + gp) * SLOT;
    auto frag = [&](const uint16_t* b, int pc, int r) __attribute__((always_inline)) {
      return *reinterpret_cast<const i32x4*>(b + (pc * S + r) * BK + fslot);
    };
    load(t + 2, stg[P]);
    i32x4 fa[3][NPC];
    // Blocks (rb, cb) in the order cb-major; before a block's NPROD MFMAs
    // the fragments the next block adds (A rows of rb + 1 in column block
    // 0, B columns of cb + 1 at rb = 2) are read, and scheduling barriers
    // keep that order: the LDS reads of a step are spread over its MFMAs
    // instead of all preceding them (C3: 55.5 against 56.4 ms).
    i32x4 fb[3][NPC];
#pragma unroll
    for (int pc = 0; pc < NPC; ++pc) {
      fb[0][pc] = frag(bufB, pc, br0 + (lane & 15));
      fa[0][pc] = frag(bufA, pc, ar0 + (lane & 15));
    }
#pragma unroll
    for (int cb = 0; cb < 3; ++cb)
#pragma unroll
      for (int rb = 0; rb < 3; ++rb) {
        if (cb == 0 && rb < 2) {
#pragma unroll
          for (int pc = 0; pc < NPC; ++pc)
            fa[rb + 1][pc] = frag(bufA, pc, ar0 + 16 * (rb + 1) + (lane & 15));
        } else if (rb == 2 && cb < 2) {
#pragma unroll
          for (int pc = 0; pc < NPC; ++pc)
            fb[cb + 1][pc] = frag(bufB, pc, br0 + 16 * (cb + 1) + (lane & 15));
        }
        __builtin_amdgcn_sched_barrier(0);
        part[rb][cb] = M::mma(fa[rb][M::ka[0]], fb[cb][M::kb[0]],
                              FIRST ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : part[rb][cb]);
#pragma unroll
        for (int e = 1; e < M::NPROD; ++e)
          part[rb][cb] = M::mma(fa[rb][M::ka[e]], fb[cb][M::kb[e]], part[rb][cb]);
        __builtin_amdgcn_sched_barrier(0);
      }
    if (t + 1 < nsteps) store(stg[1 - P], 1 - P);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using T = std::true_type;
  using F = std::false_type;
  auto run_pass = [&](f32x4(&acc)[3][3], int t0) __attribute__((always_inline)) {
    for (int u = 0; u < nk; u += 2) {
      step(I0(), T(), t0 + u);
      step(I1(), F(), t0 + u + 1);
#pragma unroll
      for (int rb = 0; rb < 3; ++rb)
#pragma unroll
        for (int cb = 0; cb < 3; ++cb) acc[rb][cb] += part[rb][cb];
    }
  };

  if (nsteps > 0) {
    load(0, stg[0]);
    load(1, stg[1]);
    store(stg[0], 0);
  }
  run_pass(accX, 0);
  if (!diag) run_pass(accP, nk);

  // Lane l of a 16 x 16 block holds column l % 16 and rows 4 (l / 16) + r.
  const int jg = gp ? j1 : j0;
  const double eo = (double)g.eps_i[i] + (double)g.eps_j[jg];
  double sum = 0.0;
  if (!diag) {
    // X and X' of one (a, b) sit in the same lane: the terms from registers
#pragma unroll
    for (int cb = 0; cb < 3; ++cb) {
      const int b = b0 + br0 + 16 * cb + (lane & 15);
      const double eb = b < nvir ? (double)g.eps_vir[b] : 0.0;
#pragma unroll
      for (int rb = 0; rb < 3; ++rb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int a = a0 + ar0 + 16 * rb + 4 * (lane >> 4) + r;
          if (a < nvir && b < nvir) {
            // X = B_i[A] B_jg[B]^T, X' = B_jg[A] B_i[B]^T
            const double x = accX[rb][cb][r] * pe_scale<NPC>(g, g.Ei, i, a, g.Ei, jg, b);
            const double xp = accP[rb][cb][r] * pe_scale<NPC>(g, g.Ei, jg, a, g.Ei, i, b);
            sum += 2.0 * (x * x + xp * xp - x * xp) / (eo - (double)g.eps_vir[a] - eb);
          }
        }
    }
  } else {
    // diagonal tile: X^T through LDS, one 96 x 97 block per pair
    __syncthreads();  // all fragment reads done before LDS is reused
    float* xs = reinterpret_cast<float*>(lds) + gp * S * (S + 1);
#pragma unroll
    for (int rb = 0; rb < 3; ++rb)
#pragma unroll
      for (int cb = 0; cb < 3; ++cb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          xs[(ar0 + 16 * rb + 4 * (lane >> 4) + r) * (S + 1) + br0 + 16 * cb + (lane & 15)] =
              accX[rb][cb][r];
    __syncthreads();
    const int lt = tid & 255;
#pragma unroll 4
    for (int e = 0; e < S * S / 256; ++e) {
      const int idx = lt + 256 * e, a = idx / S, b = idx - a * S;
      if (a0 + a < nvir && a0 + b < nvir) {
        const double x = xs[a * (S + 1) + b] * pe_scale<NPC>(g, g.Ei, i, a0 + a, g.Ei, jg, a0 + b);
        const double xt = xs[b * (S + 1) + a] * pe_scale<NPC>(g, g.Ei, i, a0 + b, g.Ei, jg, a0 + a);
        sum += x * (2.0 * x - xt) /
               (eo - (double)g.eps_vir[a0 + a] - (double)g.eps_vir[a0 + b]);
      }
    }
  }
  sum = wave_sum(sum);
  if (lane == 0) red[w] = sum;
  __syncthreads();
  if ((tid & 255) == 0 && (gp == 0 || two)) {
    const int p = i * g.nocc - i * (i - 1) / 2 + (jg - i);
    g.partial[(int64_t)p * g.nq + q] = (red[4 * gp] + red[4 * gp + 1]) + (red[4 * gp + 2] + red[4 * gp + 3]);
  }
}

// The implicit walk four pairs at a time (fp16x3): work item = (square of
// pairs (i0, i1) x (j0, j1), i0 = 2 sa, j0 = 2 sb, sa <= sb, tile pair
// A <= B); a square with sa == sb holds three pairs ((i1, j0) is not one),
// and an odd nocc leaves i1 or j1 absent. A 32-wide k-slice stages the four
// operand panels B_i0, B_i1, B_j0, B_j1 (48 KiB) for the four pairs' 96 x 96
// outputs: one panel per pair, where a couple of pairs sharing B_i stages
// 1.5 (pair_energy_x3c_kernel), which is what bounds these kernels (the LDS
// DMA moves ~40 bytes per clock per CU; a couple's step stages as long as
// its MFMAs take). Waves 4 gi .. 4 gi + 3 take i = i_gi and both j, each the
// 48 x 48 quadrant (qd & 1, qd >> 1) of both pairs (X and X', 144 VGPRs):
// the products of one pair (pieces smallest first) chain on the MFMA from
// zero over two slices in pass 0 (both pairs' partials, 72 VGPRs, live
// across the step) and over one slice in pass 1 (where X' takes 72 more
// VGPRs: one pair's partials at a time), and are added to the pair's sum
// in fp32, as pair_energy_x3_kernel<2> sums them; a chain over all slices
// on the MFMA accumulator came out 1.6e-7 low on same-sign sums. Three LDS stages, slice s in stage s % 3; each group DMAs
// its half of a stage (6 DMAs per wave per slice, slices past the walk
// clamped to the last so the waits stay exact).
// The two groups share the SIMDs (waves w and w + 4) and run half a step
// apart, so one group's MFMAs overlap the other's DMA issue and fragment
// reads: in phase A(t) group 0 multiplies slice t while group 1 DMAs its
// half of slice t + 2 and reads slice t's fragments; in B(t) group 1
// multiplies slice t while group 0 DMAs its half of slice t + 3 and reads
// slice t + 1's fragments. A barrier ends each phase; before it, a wave that
// just issued DMAs waits for all of its own but the newest slice's.
// Stage slots: 0 B_i0, 1 B_i1, 2 B_j0, 3 B_j1; the i panels hold tile A's
// rows in pass 0 (X = B_i[A] B_j[B]^T) and tile B's in pass 1 (X' = B_j[A]
// B_i[B]^T). An absent index repeats the one before it; its pairs are
// computed and dropped.
__global__ __launch_bounds__(512, 1) void pair_energy_quad_kernel(PairArgs g) {
  constexpr int NPC = 2;
  using M = PeMath<NPC>;
  constexpr int S = kX3S, BK = kX3BK;
  constexpr int SLOT = NPC * S * BK;
  constexpr int STAGE = 4 * SLOT;
  constexpr int NQ = STAGE * 2 / 1024;  // 48 DMAs of 1 KiB per stage
  constexpr int NL = NQ / 8;            // 6 per wave
  constexpr int BPS = NPC * 6;
  static_assert(NQ == 48 && S == 96 && BK == 32, "stage split");
  constexpr int EPI = 4 * S * (S + 1) * 2;  // four 96 x 97 float blocks, in 16-bit elements
  constexpr int LDS_ELEMS = 3 * STAGE > EPI ? 3 * STAGE : EPI;
  __shared__ __attribute__((aligned(16))) uint16_t lds[LDS_ELEMS];
  __shared__ double red[2][2][4];
  __shared__ int tileE[4][S];   // diagonal tiles: row exponents of i0, i1, j0, j1
  __shared__ float tileEv[S];   // and the rows' orbital energies

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gi = w >> 2, qd = w & 3;
  const int item = xcd_remap(blockIdx.x, gridDim.x);
  const int c = item / g.nq, q = item - c * g.nq;
  int sa, sb;
  tri_tiles(c, (g.nocc + 1) >> 1, sa, sb);
  const bool hi = 2 * sa + 1 < g.nocc, hj = 2 * sb + 1 < g.nocc;
  const int i0 = 2 * sa, i1 = hi ? i0 + 1 : i0, j0 = 2 * sb, j1 = hj ? j0 + 1 : j0;
  const int ig = gi ? i1 : i0;
  int TA, TB;
  tri_tiles(q, g.nb, TA, TB);
  const bool diag = TA == TB;
  const int a0 = TA * S, b0 = TB * S;
  const int nvir = g.nvir, ldv = g.ldv;
  const int nk = ldv / BK;
  const int nsteps = diag ? nk : 2 * nk;
  const int64_t ostride = (int64_t)((nvir + 1) >> 1) * 2 * NPC * ldv;

  const int lr = lane >> 2;
  const uint32_t voff =
      (uint32_t)(((lr >> 1) * nk * (NPC * 64) + (lr & 1) * 32 + 8 * x3_slot(lr, lane & 3)) * 2);
  const int pairsA = min((nvir - a0 + 1) >> 1, S / 2), pairsB = min((nvir - b0 + 1) >> 1, S / 2);
  const int64_t rowA = (int64_t)(a0 >> 1) * nk * (NPC * 64),
                rowB = (int64_t)(b0 >> 1) * nk * (NPC * 64);
  // this group's half of slice t (clamped to the last) into stage buf: slot
  // 0 B_i0, 1 B_i1, 2 B_j0, 3 B_j1; the i panels hold tile A's rows in pass
  // 0, tile B's in pass 1; group gi moves the 1 KiB pieces 24 gi .. 24 gi + 23
  auto dma = [&](int t, int buf) __attribute__((always_inline)) {
    if (t >= nsteps) t = nsteps - 1;
    const int ps = t >= nk ? 1 : 0, sl0 = ps ? t - nk : t;
    const int soff = __builtin_amdgcn_readfirstlane(sl0 * NPC * 128);
#pragma unroll
    for (int u = 0; u < NL; ++u) {
      const int qq = 24 * gi + qd + 4 * u;
      const int sl = qq / BPS, e = qq - sl * BPS, pc = e / 6;
      const int uo = ((8 * (e - 6 * pc)) * nk * (NPC * 64) + pc * 64) * 2;
      const bool onA = (sl < 2) == (ps == 0);
      const int o = i0 + (sl == 1) * (i1 - i0) + (sl == 2) * (j0 - i0) + (sl == 3) * (j1 - i0);
      const int nrec = (onA ? pairsA : pairsB) * nk * NPC * 128 - uo;
      lds_dma16_asm(reinterpret_cast<const char*>(g.Pi + o * ostride + (onA ? rowA : rowB)) + uo,
                lds + buf * STAGE + qq * 512, voff, soff, nrec > 0 ? nrec : 0);
    }
  };

  const int ar0 = 48 * (qd & 1), br0 = 48 * (qd >> 1);
  f32x4 accX[2][3][3], accP[2][3][3];
#pragma unroll
  for (int jj = 0; jj < 2; ++jj)
#pragma unroll
    for (int rb = 0; rb < 3; ++rb)
#pragma unroll
      for (int cb = 0; cb < 3; ++cb) accX[jj][rb][cb] = accP[jj][rb][cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  i32x4 fi[3][2], fj[2][3][2];  // the wave's fragments of one slice, live from its read phase to its MFMAs
  // fragments of slice t from stage bt
  auto rd = [&](int t, int bt) __attribute__((always_inline)) {
    // the lane index is opaque here, so the fragment addresses are computed
    // in each read phase instead of hoisted out of the walk and kept live
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int fs = 8 * x3_slot(ln & 15, ln >> 4);
    const int ps = t >= nk ? 1 : 0;
    const uint16_t* st = lds + bt * STAGE;
    const uint16_t* ip = st + gi * SLOT;
    const int ri = ps == 0 ? ar0 : br0, rj = ps == 0 ? br0 : ar0;
#pragma unroll
    for (int u = 0; u < 3; ++u)
#pragma unroll
      for (int pc = 0; pc < 2; ++pc) {
        fi[u][pc] = *reinterpret_cast<const i32x4*>(ip + (pc * S + ri + 16 * u + (ln & 15)) * BK + fs);
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          fj[jj][u][pc] = *reinterpret_cast<const i32x4*>(st + (2 + jj) * SLOT +
                                                          (pc * S + rj + 16 * u + (ln & 15)) * BK + fs);
      }
  };
  // the slice's products, pair by pair, into one pair's partials at a time:
  // a block's partial is added to the pair's sum three blocks after its
  // last product issued, so the adds run beside the remaining MFMAs; pair
  // 0's last three blocks are added just before pair 1's first products
  // take their registers, and only pair 1's last three trail the MFMAs
  f32x4 part[2][3][3];  // pass 0: both pairs' two-slice partials live across the step
  auto mm = [&](auto PS_, auto FIRST_, auto LAST_) __attribute__((always_inline)) {
    constexpr int PS = decltype(PS_)::value;
    constexpr bool FIRST = decltype(FIRST_)::value, LAST = decltype(LAST_)::value;
    auto fold = [&](int jj, int rb, int cb) __attribute__((always_inline)) {
      if constexpr (PS == 0)
        accX[jj][rb][cb] += part[jj][rb][cb];
      else
        accP[jj][rb][cb] += part[jj][rb][cb];
    };
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
#pragma unroll
      for (int e = 0; e < M::NPROD; ++e)
#pragma unroll
        for (int cb = 0; cb < 3; ++cb)
#pragma unroll
          for (int rb = 0; rb < 3; ++rb) {
            if (LAST && jj == 1 && e == 0 && 3 * cb + rb >= 6) fold(0, rb, cb);
            const f32x4 c0 = FIRST && e == 0 ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : part[jj][rb][cb];
            if constexpr (PS == 0)
              part[jj][rb][cb] = M::mma(fi[rb][M::ka[e]], fj[jj][cb][M::kb[e]], c0);
            else
              part[jj][rb][cb] = M::mma(fj[jj][rb][M::ka[e]], fi[cb][M::kb[e]], c0);
            if (LAST && jj == 1 && e == 0 && 3 * cb + rb >= 6) __builtin_amdgcn_sched_barrier(0);
            if (LAST && e == M::NPROD - 1) {
              const int nb = 3 * cb + rb;  // block order of this loop
              if (nb >= 3) fold(jj, (nb - 3) % 3, (nb - 3) / 3);
              __builtin_amdgcn_sched_barrier(0);
            }
          }
    }
    if constexpr (LAST) {
#pragma unroll
      for (int ob = 6; ob < 9; ++ob) fold(1, ob % 3, ob / 3);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto bar = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
  // this wave's DMAs of all but its newest n slices have landed (6 per slice)
  auto vwait = [&](int n) __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    if (n >= 2)
      asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
  };
  auto m3 = [](int t) { return t - 3 * (t / 3); };
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  // The two passes are separate loops so that the target of the folds (X or
  // X') is fixed at compile time. Group 0 has its half of slices 0 .. 2 in
  // flight before the walk and group 1 of slices 0 and 1; both wait for
  // slice 0, then group 0 reads it.
  if (nsteps > 0) {
    if (gi == 0) {
      dma(0, 0);
      dma(1, 1);
      dma(2, 2);
      vwait(2);
      bar();
      rd(0, 0);
      auto step0 = [&](auto PS_, auto F_, auto L_, int t) __attribute__((always_inline)) {
        const int b0s = m3(t), b1s = b0s == 2 ? 0 : b0s + 1;
        mm(PS_, F_, L_);  // A(t)
        vwait(1);
        bar();
        dma(t + 3, b0s);  // B(t): stage t % 3 was read by both groups in or before A(t)
        rd(t + 1, b1s);   // past the walk it reads a stage nobody uses
        bar();
      };
      auto walk0 = [&](auto PS_, int t0, int t1) __attribute__((always_inline)) {
        using T = std::true_type;
        using F = std::false_type;
        if constexpr (decltype(PS_)::value == 0) {
          for (int t = t0; t < t1; t += 2) {  // nk is even
            step0(PS_, T(), F(), t);
            step0(PS_, F(), T(), t + 1);
          }
        } else {
          for (int t = t0; t < t1; ++t) step0(PS_, T(), T(), t);
        }
      };
      walk0(P0(), 0, nk);
      if (!diag) walk0(P1(), nk, nsteps);
    } else {
      dma(0, 0);
      dma(1, 1);
      vwait(1);
      bar();
      auto step1 = [&](auto PS_, auto F_, auto L_, int t) __attribute__((always_inline)) {
        const int b0s = m3(t), b2s = b0s == 0 ? 2 : b0s - 1;
        dma(t + 2, b2s);  // A(t): stage (t + 2) % 3 held slice t - 1, read before A(t)
        rd(t, b0s);
        vwait(1);
        bar();
        mm(PS_, F_, L_);  // B(t)
        bar();
      };
      auto walk1 = [&](auto PS_, int t0, int t1) __attribute__((always_inline)) {
        using T = std::true_type;
        using F = std::false_type;
        if constexpr (decltype(PS_)::value == 0) {
          for (int t = t0; t < t1; t += 2) {
            step1(PS_, T(), F(), t);
            step1(PS_, F(), T(), t + 1);
          }
        } else {
          for (int t = t0; t < t1; ++t) step1(PS_, T(), T(), t);
        }
      };
      walk1(P0(), 0, nk);
      if (!diag) walk1(P1(), nk, nsteps);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no DMA may land after the workgroup ends

  // The energy terms. The exponents and orbital energies of the lane's rows
  // and columns are loaded once, up front and clamped into the matrix, so
  // their loads overlap instead of each term waiting for its own; 2^-(e1 +
  // e2) is the pe_scale factor. Rows and columns past nvir hold X = X' = 0
  // (their panel rows read as zeros), so their terms are exact zeros with
  // finite denominators and need no branch.
  double sum[2] = {0.0, 0.0};
  const double ei = (double)g.eps_i[ig];
  const int32_t* E = g.Ei;
  const int64_t ldE = g.ldE;
  if (!diag) {
    int xa_i[12], xa_j[2][12], xb_i[3], xb_j[2][3];
    float eva[12], evb[3];
#pragma unroll
    for (int rb = 0; rb < 3; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int a = min(a0 + ar0 + 16 * rb + 4 * (lane >> 4) + r, nvir - 1);
        xa_i[4 * rb + r] = E[ig * ldE + a];
        xa_j[0][4 * rb + r] = E[j0 * ldE + a];
        xa_j[1][4 * rb + r] = E[j1 * ldE + a];
        eva[4 * rb + r] = g.eps_vir[a];
      }
#pragma unroll
    for (int cb = 0; cb < 3; ++cb) {
      const int b = min(b0 + br0 + 16 * cb + (lane & 15), nvir - 1);
      xb_i[cb] = E[ig * ldE + b];
      xb_j[0][cb] = E[j0 * ldE + b];
      xb_j[1][cb] = E[j1 * ldE + b];
      evb[cb] = g.eps_vir[b];
    }
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int jg = jj ? j1 : j0;
      const double eo = ei + (double)g.eps_j[jg];
#pragma unroll
      for (int cb = 0; cb < 3; ++cb) {
        const double eb = (double)evb[cb];
#pragma unroll
        for (int rb = 0; rb < 3; ++rb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int ka = 4 * rb + r;
            const double x = accX[jj][rb][cb][r] * ldexp(1.0, -(xa_i[ka] + xb_j[jj][cb]));
            const double xp = accP[jj][rb][cb][r] * ldexp(1.0, -(xa_j[jj][ka] + xb_i[cb]));
            sum[jj] += 2.0 * (x * x + xp * xp - x * xp) / (eo - (double)eva[ka] - eb);
          }
      }
    }
  } else {
    // diagonal tile: X goes through LDS for its transpose; the tile's
    // exponents (orbitals i0, i1, j0, j1) and orbital energies beside it
    const int o4[4] = {i0, i1, j0, j1};
    for (int x = tid; x < 5 * S; x += 512) {
      const int r = x % S, row = min(a0 + r, nvir - 1), sl = x / S;
      if (sl < 4)
        tileE[sl][r] = E[o4[sl] * ldE + row];
      else
        tileEv[r] = g.eps_vir[row];
    }
    __syncthreads();
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      float* xs = reinterpret_cast<float*>(lds) + (2 * gi + jj) * S * (S + 1);
#pragma unroll
      for (int rb = 0; rb < 3; ++rb)
#pragma unroll
        for (int cb = 0; cb < 3; ++cb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            xs[(ar0 + 16 * rb + 4 * (lane >> 4) + r) * (S + 1) + br0 + 16 * cb + (lane & 15)] =
                accX[jj][rb][cb][r];
    }
    __syncthreads();
    const int lt = tid & 255;
    const int* ti = tileE[gi];  // exponents of i_gi over the tile's rows
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int jg = jj ? j1 : j0;
      const int* tj = tileE[2 + jj];
      const double eo = ei + (double)g.eps_j[jg];
      const float* xs = reinterpret_cast<const float*>(lds) + (2 * gi + jj) * S * (S + 1);
#pragma unroll 4
      for (int e = 0; e < S * S / 256; ++e) {
        const int idx = lt + 256 * e, a = idx / S, b = idx - a * S;
        const double x = xs[a * (S + 1) + b] * ldexp(1.0, -(ti[a] + tj[b]));
        const double xt = xs[b * (S + 1) + a] * ldexp(1.0, -(ti[b] + tj[a]));
        sum[jj] += x * (2.0 * x - xt) / (eo - (double)tileEv[a] - (double)tileEv[b]);
      }
    }
  }
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    const double s = wave_sum(sum[jj]);
    if (lane == 0) red[gi][jj][qd] = s;
  }
  __syncthreads();
  if (tid < 4) {
    const int pg = tid >> 1, pj = tid & 1;  // thread t writes pair (i_pg, j_pj)
    const int pi = pg ? i1 : i0, pjj = pj ? j1 : j0;
    const bool valid = (pg == 0 || hi) && (pj == 0 || hj) && pi <= pjj;
    if (valid) {
      const int p = pi * g.nocc - pi * (pi - 1) / 2 + (pjj - pi);
      g.partial[(int64_t)p * g.nq + q] =
          (red[pg][pj][0] + red[pg][pj][1]) + (red[pg][pj][2] + red[pg][pj][3]);
    }
  }
}

// MP2 energy of a precomputed amplitude block (the `mp2_energy` surface,
// trnblas/nki/dispatch.py:4356-4491): one workgroup per (i, j) pair walks the
// 32 x 32 tile pairs (A <= B) of T_ij, reading T[A,B] and T[B,A] once each
// through LDS (transposed read of the second), so every amplitude is read
// once from HBM. fp64 terms, fixed-order reduction.
__global__ __launch_bounds__(256) void mp2_energy_kernel(int ic, int nocc, int nvir,
                                                         const float* T, int64_t ldt,
                                                         const float* eo_chunk,
                                                         const float* eo_full,
                                                         const float* ev, double* out) {
  __shared__ float x[32][33], y[32][33];
  __shared__ double red[4];
  const int pair = blockIdx.x;
  const int i = pair / nocc, j = pair - i * nocc;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 8 rows of 32
  const double eo = (double)eo_chunk[i] + (double)eo_full[j];
  const float* Tij = T + (int64_t)i * nvir * ldt + (int64_t)j * nvir;
  const int nb = (nvir + 31) / 32;
  double sum = 0.0;
  for (int A = 0; A < nb; ++A)
    for (int B = A; B < nb; ++B) {
      __syncthreads();
      for (int r = ty; r < 32; r += 8) {
        const int a = A * 32 + r, b = B * 32 + tx;
        x[r][tx] = (a < nvir && b < nvir) ? Tij[(int64_t)a * ldt + b] : 0.0f;
        const int a2 = B * 32 + r, b2 = A * 32 + tx;
        y[r][tx] = (a2 < nvir && b2 < nvir) ? Tij[(int64_t)a2 * ldt + b2] : 0.0f;
      }
      __syncthreads();
      for (int r = ty; r < 32; r += 8) {
        const int a = A * 32 + r, b = B * 32 + tx;
        if (a < nvir && b < nvir) {
          const double tab = x[r][tx], tba = y[tx][r];
          const double d = eo - (double)ev[a] - (double)ev[b];
          sum += (A == B ? tab * (2.0 * tab - tba) : 2.0 * (tab * tab + tba * tba - tab * tba)) / d;
        }
      }
    }
  sum = wave_sum(sum);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sum;
  __syncthreads();
  if (threadIdx.x == 0) out[pair] = (red[0] + red[1]) + (red[2] + red[3]);
}

constexpr int kPeS = 96, kPeBK = 16;

static int64_t pe_nq(int64_t nvir) {
  const int64_t nb = (nvir + kPeS - 1) / kPeS;
  return nb * (nb + 1) / 2;
}

}  // namespace trnblas

using namespace trnblas;

extern "C" size_t trnblas_hip_pair_energy_workspace(int64_t nvir, int64_t npairs) {
  if (nvir <= 0 || npairs <= 0) return 0;
  return (size_t)(npairs * pe_nq(nvir) + npairs) * sizeof(double);
}

// Split workspaces (bf16x6: NPC = 3; fp16x3: NPC = 2): the partials of the
// fp32 layout, then the pieces of Bi (ni x ceil(nvir / 2) row pairs of
// 2 NPC x ldv), then those of Bj (nj x ceil(nvir / 2); none when nj == 0,
// where Bj shares Bi's pieces); fp16x3 adds the int32 row exponents of Bi
// (ni x 2 ceil(nvir / 2)), then of Bj. Each region is 256-byte aligned.
static int64_t x3_ldv(int64_t naux) { return (naux + 2 * kX3BK - 1) / (2 * kX3BK) * (2 * kX3BK); }
static size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }
static size_t x3_planes_bytes(int npc, int64_t n, int64_t nvir, int64_t naux) {
  return al256((size_t)(2 * npc * n * ((nvir + 1) / 2) * x3_ldv(naux)) * sizeof(uint16_t));
}
static size_t h3_exps_bytes(int64_t n, int64_t nvir) {
  return al256((size_t)(n * ((nvir + 1) & ~1ll)) * sizeof(int32_t));
}
static size_t split_workspace(int npc, int64_t nvir, int64_t naux, int64_t npairs, int64_t ni,
                              int64_t nj) {
  if (nvir <= 0 || npairs <= 0 || naux < 0 || ni < 0 || nj < 0) return 0;
  size_t b = al256(trnblas_hip_pair_energy_workspace(nvir, npairs)) +
             x3_planes_bytes(npc, ni, nvir, naux) + x3_planes_bytes(npc, nj, nvir, naux);
  if (npc == 2) b += h3_exps_bytes(ni, nvir) + h3_exps_bytes(nj, nvir);
  return b;
}

extern "C" size_t trnblas_hip_pair_energy_bf16x6_workspace(int64_t nvir, int64_t naux,
                                                           int64_t npairs, int64_t ni,
                                                           int64_t nj) {
  return split_workspace(3, nvir, naux, npairs, ni, nj);
}

extern "C" size_t trnblas_hip_pair_energy_fp16x3_workspace(int64_t nvir, int64_t naux,
                                                           int64_t npairs, int64_t ni,
                                                           int64_t nj) {
  return split_workspace(2, nvir, naux, npairs, ni, nj);
}

// Split n x nvir rows (o, a) of X into the pieces at P (bf16x6:
// split_planes_kernel; fp16x3: split_f16x3_kernel, row exponents into E).
template <int NPC>
static void x3_split(const float* X, int64_t n, int64_t ld_occ, int64_t ld_vir, int nvir,
                     int naux, int ldv, uint16_t* P, int32_t* E, hipStream_t s) {
  const int64_t threads = n * ((nvir + 1) & ~1) * (ldv / 8);
  if (threads == 0) return;
  const bool vec = (reinterpret_cast<uintptr_t>(X) & 15) == 0 && ld_occ % 4 == 0 &&
                   ld_vir % 4 == 0;
  if (NPC == 2) {
    const int64_t nrp = n * ((nvir + 1) >> 1);
    const unsigned blocks = (unsigned)((nrp + 3) / 4);
    if (vec)
      hipLaunchKernelGGL(split_f16x3_kernel<true>, dim3(blocks), dim3(256), 0, s, nvir, naux, ldv,
                         (int)nrp, X, ld_occ, ld_vir, E, P);
    else
      hipLaunchKernelGGL(split_f16x3_kernel<false>, dim3(blocks), dim3(256), 0, s, nvir, naux, ldv,
                         (int)nrp, X, ld_occ, ld_vir, E, P);
    return;
  }
  const unsigned blocks = (unsigned)((threads + 255) / 256);
  if (vec)
    hipLaunchKernelGGL(split_planes_kernel<true>, dim3(blocks), dim3(256), 0, s, nvir, naux, ldv,
                       (int)threads, X, ld_occ, ld_vir, P);
  else
    hipLaunchKernelGGL(split_planes_kernel<false>, dim3(blocks), dim3(256), 0, s, nvir, naux, ldv,
                       (int)threads, X, ld_occ, ld_vir, P);
}

template <int NPC>
static void split_launch(const PairArgs& g, bool implicit, int64_t citems, int64_t items,
                         hipStream_t s) {
  if (implicit && NPC == 2)
    hipLaunchKernelGGL(pair_energy_quad_kernel, dim3((unsigned)citems), dim3(512), 0, s, g);
  else if (implicit)
    hipLaunchKernelGGL(pair_energy_x3c_kernel<3>, dim3((unsigned)citems), dim3(512), 0, s, g);
  else
    hipLaunchKernelGGL(pair_energy_x3_kernel<NPC>, dim3((unsigned)items), dim3(256), 0, s, g);
}

// Shared driver of the fp32 (npc 0), bf16x6 (npc 3) and fp16x3 (npc 2)
// pair-energy entry points: argument checks, the split, the fused kernel,
// then the per-pair and total reductions.
static int pair_energy_run(int npc, const char* name, int64_t nvir, int64_t naux, const float* Bi,
                           int64_t ni, int64_t ldi_occ, const float* Bj, int64_t nj,
                           int64_t ldj_occ, int64_t ld_vir, const float* eps_i, const float* eps_j,
                           const float* eps_vir, int64_t nocc, int64_t npairs,
                           const int32_t* pair_i, const int32_t* pair_j, const double* pair_w,
                           double* out_pairs, double* out_total, void* workspace,
                           size_t workspace_bytes, hipStream_t s) {
  TRNBLAS_CHECK_ARG(nvir >= 0 && naux >= 0 && nocc >= 0 && npairs >= 0, "%s: negative size", name);
  TRNBLAS_CHECK_ARG(nvir < (1 << 30) && naux < (1 << 30), "%s: size too large", name);
  if (pair_i == nullptr) {
    TRNBLAS_CHECK_ARG(Bi == Bj && eps_i == eps_j && ldi_occ == ldj_occ,
                      "%s: the implicit i <= j walk needs Bi == Bj, eps_i == eps_j", name);
    npairs = nocc * (nocc + 1) / 2;
  } else {
    TRNBLAS_CHECK_ARG(pair_j != nullptr, "%s: pair_j is NULL", name);
  }
  if (npairs == 0 || nvir == 0) {
    // Empty sums: zero energies.
    if (out_total) hipLaunchKernelGGL(zero_f64_kernel, dim3(1), dim3(256), 0, s, out_total, 1);
    if (out_pairs && npairs > 0)
      hipLaunchKernelGGL(zero_f64_kernel, dim3((unsigned)((npairs + 255) / 256)), dim3(256), 0, s,
                         out_pairs, npairs);
    return check_launch(name);
  }
  TRNBLAS_CHECK_ARG(Bi && Bj && eps_i && eps_j && eps_vir, "%s: NULL operand", name);
  TRNBLAS_CHECK_ARG(ld_vir >= naux, "%s: ld_vir < naux", name);
  TRNBLAS_CHECK_ARG((int64_t)kPeS * ld_vir * 4 < 0x7fffff00ll,
                    "%s: ld_vir too large for 32-bit panel offsets", name);
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const int64_t nq = pe_nq(nvir);
  const int64_t items = npairs * nq;
  TRNBLAS_CHECK_ARG(items < (1ll << 31), "%s: too many work items", name);
  const bool x3 = npc != 0;
  if (x3) {
    TRNBLAS_CHECK_ARG(ni >= 0 && nj >= 0 && ni < (1 << 30) && nj < (1 << 30),
                      "%s: bad row count", name);
    TRNBLAS_CHECK_ARG(pair_i != nullptr || (ni >= nocc && nj == 0),
                      "%s: the implicit walk needs ni >= nocc and nj == 0", name);
    TRNBLAS_CHECK_ARG(nj > 0 || (Bj == Bi && ldj_occ == ldi_occ),
                      "%s: nj == 0 shares Bi's pieces and needs Bj == Bi", name);
    TRNBLAS_CHECK_ARG((int64_t)kX3S * npc * x3_ldv(naux) * 2 < 0x7fffff00ll,
                      "%s: naux too large for 32-bit panel offsets", name);
    TRNBLAS_CHECK_ARG((ni > nj ? ni : nj) * (nvir + 1) * (x3_ldv(naux) / 8) < (1ll << 31),
                      "%s: operands too large for one split launch", name);
  }
  const size_t need = x3 ? split_workspace(npc, nvir, naux, npairs, ni, nj)
                         : trnblas_hip_pair_energy_workspace(nvir, npairs);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("%s: workspace of %zu bytes needed, %zu given", name, need, workspace_bytes);
    return TRNBLAS_E_WORKSPACE;
  }
  PairArgs g;
  g.nvir = (int)nvir;
  g.naux = (int)naux;
  g.Bi = Bi;
  g.ldi_occ = ldi_occ;
  g.Bj = Bj;
  g.ldj_occ = ldj_occ;
  g.ld_vir = ld_vir;
  g.eps_i = eps_i;
  g.eps_j = eps_j;
  g.eps_vir = eps_vir;
  g.nocc = (int)nocc;
  g.npairs = (int)npairs;
  g.pair_i = pair_i;
  g.pair_j = pair_j;
  g.pair_w = pair_w;
  g.nb = (int)((nvir + kPeS - 1) / kPeS);
  g.nq = (int)nq;
  g.partial = static_cast<double*>(workspace);
  double* e_pair = out_pairs ? out_pairs : g.partial + items;
  const bool vec = al16(Bi) && al16(Bj) && naux % 4 == 0 && ld_vir % 4 == 0 &&
                   ldi_occ % 4 == 0 && ldj_occ % 4 == 0;
  if (x3) {
    static_assert(kX3S == kPeS, "one tile size: one partials layout");
    const int ldv = (int)x3_ldv(naux);
    char* pieces =
        static_cast<char*>(workspace) + al256(trnblas_hip_pair_energy_workspace(nvir, npairs));
    const size_t pbi = x3_planes_bytes(npc, ni, nvir, naux), pbj = x3_planes_bytes(npc, nj, nvir, naux);
    uint16_t* Pi = reinterpret_cast<uint16_t*>(pieces);
    uint16_t* Pj = nj ? reinterpret_cast<uint16_t*>(pieces + pbi) : Pi;
    int32_t* Ei = npc == 2 ? reinterpret_cast<int32_t*>(pieces + pbi + pbj) : nullptr;
    int32_t* Ej = npc == 2 && nj ? reinterpret_cast<int32_t*>(pieces + pbi + pbj +
                                                             h3_exps_bytes(ni, nvir))
                                 : Ei;
    g.Pi = Pi;
    g.Pj = Pj;
    g.Ei = Ei;
    g.Ej = Ej;
    g.ldE = (int)((nvir + 1) & ~1ll);
    g.ldv = ldv;
    g.rows_i = (int)ni;
    g.rows_j = (int)(nj ? nj : ni);
    // implicit walk items: squares of pairs (fp16x3), couples (bf16x6)
    const int64_t nb2 = (nocc + 1) / 2;
    const int64_t citems =
        pair_i == nullptr ? (npc == 2 ? nb2 * (nb2 + 1) / 2 : pe_couples(nocc)) * nq : 0;
    TRNBLAS_CHECK_ARG(citems < (1ll << 31), "%s: too many work items", name);
    if (npc == 3) {
      x3_split<3>(Bi, ni, ldi_occ, ld_vir, (int)nvir, (int)naux, ldv, Pi, nullptr, s);
      if (nj) x3_split<3>(Bj, nj, ldj_occ, ld_vir, (int)nvir, (int)naux, ldv, Pj, nullptr, s);
    } else {
      x3_split<2>(Bi, ni, ldi_occ, ld_vir, (int)nvir, (int)naux, ldv, Pi, Ei, s);
      if (nj) x3_split<2>(Bj, nj, ldj_occ, ld_vir, (int)nvir, (int)naux, ldv, Pj, Ej, s);
    }
    int rc = check_launch(name);
    if (rc) return rc;
    // the implicit walk: four pairs (fp16x3) or two sharing B_i (bf16x6) per workgroup
    if (npc == 3)
      split_launch<3>(g, pair_i == nullptr, citems, items, s);
    else
      split_launch<2>(g, pair_i == nullptr, citems, items, s);
  } else {
    constexpr int NT = kPeS / 32 * 64;
    if (vec)
      hipLaunchKernelGGL((pair_energy_kernel<kPeS, kPeBK, true>), dim3((unsigned)items),
                         dim3(NT), 0, s, g);
    else
      hipLaunchKernelGGL((pair_energy_kernel<kPeS, kPeBK, false>), dim3((unsigned)items),
                         dim3(NT), 0, s, g);
  }
  int rc = check_launch(name);
  if (rc) return rc;
  hipLaunchKernelGGL(pair_sum_kernel, dim3((unsigned)((npairs + 255) / 256)), dim3(256), 0, s,
                     (const double*)g.partial, (int)npairs, (int)nq, e_pair);
  rc = check_launch(name);
  if (rc) return rc;
  if (out_total) {
    hipLaunchKernelGGL(pair_total_kernel, dim3(1), dim3(1024), 0, s, (const double*)e_pair,
                       (int)npairs, (int)nocc, pair_i, pair_j, pair_w, out_total);
    rc = check_launch(name);
  }
  return rc;
}

extern "C" int trnblas_hip_pair_energy(int64_t nvir, int64_t naux, const float* Bi,
                                       int64_t ldi_occ, const float* Bj, int64_t ldj_occ,
                                       int64_t ld_vir, const float* eps_i, const float* eps_j,
                                       const float* eps_vir, int64_t nocc, int64_t npairs,
                                       const int32_t* pair_i, const int32_t* pair_j,
                                       const double* pair_w, double* out_pairs,
                                       double* out_total, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  clear_error();
  return pair_energy_run(0, "pair_energy", nvir, naux, Bi, 0, ldi_occ, Bj, 0, ldj_occ, ld_vir,
                         eps_i, eps_j, eps_vir, nocc, npairs, pair_i, pair_j, pair_w,
                         out_pairs, out_total, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int trnblas_hip_pair_energy_bf16x6(int64_t nvir, int64_t naux, const float* Bi,
                                              int64_t ni, int64_t ldi_occ, const float* Bj,
                                              int64_t nj, int64_t ldj_occ,
                                              int64_t ld_vir, const float* eps_i,
                                              const float* eps_j, const float* eps_vir,
                                              int64_t nocc, int64_t npairs,
                                              const int32_t* pair_i, const int32_t* pair_j,
                                              const double* pair_w, double* out_pairs,
                                              double* out_total, void* workspace,
                                              size_t workspace_bytes, void* stream) {
  clear_error();
  return pair_energy_run(3, "pair_energy_bf16x6", nvir, naux, Bi, ni, ldi_occ, Bj, nj, ldj_occ,
                         ld_vir, eps_i, eps_j, eps_vir, nocc, npairs, pair_i, pair_j, pair_w,
                         out_pairs, out_total, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int trnblas_hip_pair_energy_fp16x3(int64_t nvir, int64_t naux, const float* Bi,
                                              int64_t ni, int64_t ldi_occ, const float* Bj,
                                              int64_t nj, int64_t ldj_occ,
                                              int64_t ld_vir, const float* eps_i,
                                              const float* eps_j, const float* eps_vir,
                                              int64_t nocc, int64_t npairs,
                                              const int32_t* pair_i, const int32_t* pair_j,
                                              const double* pair_w, double* out_pairs,
                                              double* out_total, void* workspace,
                                              size_t workspace_bytes, void* stream) {
  clear_error();
  return pair_energy_run(2, "pair_energy_fp16x3", nvir, naux, Bi, ni, ldi_occ, Bj, nj, ldj_occ,
                         ld_vir, eps_i, eps_j, eps_vir, nocc, npairs, pair_i, pair_j, pair_w,
                         out_pairs, out_total, workspace, workspace_bytes, (hipStream_t)stream);
}

// ── No-allocation variant of trnblas_hip_pair_energy ───────────────────────
//
// The partials live in `scratch`, a file-scope device array: each GPU the
// library runs on holds its own copy at its own address until the process
// ends. In host code `scratch` names a host-side stand-in, never the device
// memory, so its device address is looked up per device (hipGetSymbolAddress,
// with that device current, on the first call there) and only that address
// is handed to the kernels. Every partial is written before it is read, so
// nothing needs clearing between calls; calls that overlap on one GPU (other
// streams, other host threads) share the array and race.
constexpr size_t kPeScratchBytes = (size_t)16 << 20;  // 2 Mi fp64 partials
static __device__ __align__(256) double scratch[kPeScratchBytes / sizeof(double)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};
}  // namespace

static int scratch_address(const char* name, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("%s: no current device (or device index >= %d)", name, kMaxDevices);
    return TRNBLAS_E_LAUNCH;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("%s: hipGetSymbolAddress(scratch) on device %d: %s", name, dev,
                hipGetErrorString(e));
      return TRNBLAS_E_LAUNCH;
    }
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return TRNBLAS_OK;
}

extern "C" size_t trnblas_hip_pair_energy_noalloc_max_bytes(void) { return kPeScratchBytes; }

extern "C" int trnblas_hip_pair_energy_noalloc(int64_t nvir, int64_t naux, const float* Bi,
                                               int64_t ldi_occ, const float* Bj, int64_t ldj_occ,
                                               int64_t ld_vir, const float* eps_i,
                                               const float* eps_j, const float* eps_vir,
                                               int64_t nocc, int64_t npairs,
                                               const int32_t* pair_i, const int32_t* pair_j,
                                               const double* pair_w, double* out_pairs,
                                               double* out_total, void* stream) {
  clear_error();
  static const char* name = "pair_energy_noalloc";
  TRNBLAS_CHECK_ARG(nvir >= 0 && nocc >= 0 && npairs >= 0 && nvir < (1 << 30) &&
                        nocc < (1 << 30),
                    "%s: bad size", name);
  const int64_t np = pair_i == nullptr ? nocc * (nocc + 1) / 2 : npairs;
  const size_t need = trnblas_hip_pair_energy_workspace(nvir, np);
  if (need > kPeScratchBytes) {
    set_error("%s: %lld pairs at nvir %lld need %zu bytes of partials; the static scratch holds "
              "%zu (use trnblas_hip_pair_energy with a workspace)",
              name, (long long)np, (long long)nvir, need, kPeScratchBytes);
    return TRNBLAS_E_WORKSPACE;
  }
  void* ws = nullptr;
  const int rc = scratch_address(name, &ws);
  if (rc) return rc;
  return pair_energy_run(0, name, nvir, naux, Bi, 0, ldi_occ, Bj, 0, ldj_occ, ld_vir, eps_i,
                         eps_j, eps_vir, nocc, npairs, pair_i, pair_j, pair_w, out_pairs,
                         out_total, ws, kPeScratchBytes, (hipStream_t)stream);
}

extern "C" int trnblas_hip_mp2_energy(int64_t ic, int64_t nocc, int64_t nvir, const float* T_flat,
                                      int64_t ldt, const float* eps_occ_chunk,
                                      const float* eps_occ_full, const float* eps_vir,
                                      double* out_pairs, void* stream) {
  clear_error();
  TRNBLAS_CHECK_ARG(ic >= 0 && nocc >= 0 && nvir >= 0, "mp2_energy: negative size");
  if (ic == 0 || nocc == 0) return TRNBLAS_OK;
  TRNBLAS_CHECK_ARG(ic * nocc < (1ll << 31) && nvir < (1 << 30), "mp2_energy: size too large");
  TRNBLAS_CHECK_ARG(out_pairs && eps_occ_chunk && eps_occ_full, "mp2_energy: NULL operand");
  if (nvir > 0)
    TRNBLAS_CHECK_ARG(T_flat && eps_vir && ldt >= nocc * nvir, "mp2_energy: bad T_flat / ldt");
  hipLaunchKernelGGL(mp2_energy_kernel, dim3((unsigned)(ic * nocc)), dim3(256), 0,
                     (hipStream_t)stream, (int)ic, (int)nocc, (int)nvir, T_flat, ldt,
                     eps_occ_chunk, eps_occ_full, eps_vir, out_pairs);
  return check_launch("mp2_energy");
}
