// Level-3 GEMM and SYRK for gfx950 on MFMA: fp32 (v_mfma_f32_32x32x2_f32) and
// bf16 / fp16 (v_mfma_f32_32x32x16_{bf16,f16}, fp32 accumulate).
//
// Semantics follow trnblas/level3.py:69-134 (`gemm`, `batched_gemm`:
// D = alpha op(A) op(B) + beta C into a fresh output, C never written) and
// :243-302 (`syrk`: full symmetric result from the `uplo` triangle of C).
// The kernels are written for CDNA4, not translated from the reference's NKI
// tiling (trnblas/nki/dispatch.py:3324-3760, :4493-4544):
//  * a 256-thread workgroup (4 wave64s) owns a 128x128 tile of D; each wave a
//    64x64 sub-tile as 2x2 MFMA 32x32 blocks with the accumulators in
//    AGPR/VGPRs;
//  * operand panels are staged in LDS, double buffered: the loads of k-tile
//    t+1 are in flight while the MFMAs of k-tile t run, one barrier per
//    k-tile (16-byte aligned operands: direct-to-LDS DMA, gemm_dma_kernel;
//    otherwise through registers, gemm_kernel);
//  * an operand whose K dimension is contiguous in HBM is kept K-contiguous
//    in LDS (rows padded by 16 bytes, so each 16-byte fragment read is
//    bank-conflict free); one whose M / N dimension is contiguous (a
//    transposed operand: transA / transB, the C1 `Aᵀ B`) is kept that way and
//    read a column at a time — no transposed copy is ever made in HBM;
//  * the K order inside an 8-wide (fp32) / 16-wide (16-bit) chunk is permuted
//    the same way for both operands (lane half h takes k = h*EV .. h*EV+EV-1),
//    so a fragment is one 16-byte LDS read;
//  * ragged M / N / K edges are zero-filled at load and masked at store;
//  * the alpha / beta epilogue is fused into the store;
//  * SYRK launches only the lower-triangle tiles (n(n+1)/2 of them for n
//    tiles) and writes each value to D[i][j] and D[j][i];
//  * the tile walk is XCD-aware: each of the 8 XCDs (own L2) walks a
//    contiguous range of tiles in grouped order.
#include <algorithm>
#include <type_traits>

#include "common.hpp"

namespace trnblas {

struct GemmArgs {
  int M, N, K;
  float alpha, beta;
  const void* A;
  int64_t lda, sA;
  const void* B;
  int64_t ldb, sB;
  const void* C;
  int64_t ldc, sC;
  void* D;
  int64_t ldd, sD;
  int batch;
  int tiles_m, tiles_n;  // tile grid of one batch entry
  int ntiles;            // tiles of the launch (all batch entries, or the SYRK triangle)
  int nk;                // k-tiles per tile
  int uplo;              // SYRK: 0 = lower triangle of C referenced, 1 = upper
  const int32_t* tri;    // SYRK: triangle flags of C (device), or null; see syrk_upper
  int vec4;              // SYRK: C and D take 4-element vector accesses (aligned, ld % 4 == 0)
  int vec2;              // sgemm_pipe_kernel: C and D take 2-element accesses (aligned, ld even)
  int sk_groups;         // stream-K workgroups (0 = data-parallel)
  int dp_tiles;          // under stream-K: leading tiles computed whole
  float* ws;             // stream-K partial tiles [sk_groups][2][BM * BN]
  int span;              // k-tiles per MFMA accumulation chain (chain_length / k-tile)
};

template <typename T>
struct Zero {
  __device__ static T v() { return T(0.0f); }
};

template <typename T>
__device__ __forceinline__ float to_f32(T x) {
  return (float)x;
}

// Buffer-resource loads: an offset at or beyond num_records reads zero with
// no memory access, so ragged edges are masked by a select on the offset
// (no branches around loads).
constexpr uint32_t kOob = 0x80000000u;  // offsets >= this read as zero
constexpr uint32_t kRecords = 0x7ffffff0u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)kRecords,
                                           0x00020000);
}

// One 16-byte group of EV consecutive elements at byte offset `off` from the
// resource base. VEC: all EV elements are valid or none is (`ok`); otherwise
// `nvalid` (0..EV) leading elements are valid.
template <typename T, bool VEC>
__device__ __forceinline__ i32x4 load_group(__amdgpu_buffer_rsrc_t rs, uint32_t off, bool ok,
                                            int nvalid) {
  constexpr int EV = 16 / sizeof(T);
  if (VEC) return __builtin_amdgcn_raw_buffer_load_b128(rs, ok ? off : kOob, 0, 0);
  union {
    i32x4 v;
    T e[EV];
    unsigned short h[EV];
    int w[EV];
  } u;
#pragma unroll
  for (int e = 0; e < EV; ++e) {
    const uint32_t o = (ok && e < nvalid) ? off + e * (uint32_t)sizeof(T) : kOob;
    if (sizeof(T) == 4)
      u.w[e] = __builtin_amdgcn_raw_buffer_load_b32(rs, o, 0, 0);
    else
      u.h[e] = __builtin_amdgcn_raw_buffer_load_b16(rs, o, 0, 0);
  }
  return u.v;
}

// Accumulation: the MFMA accumulator of a tile restarts from zero every
// chain_length(K) k values and each finished chain is added into a separate
// fp32 sum with a VALU add (fold_span). One chain over all of K rounds the
// running sum at every step: a sum of 8192 same-sign products (a SYRK
// diagonal) came out 5.3e-6 off. With chains of L values folded into the sum
// the error is that of one L-long chain (averaged over the K / L chains)
// plus that of K / L folds. Measured on the MI355X, largest componentwise
// error over the whole output with U(0, 1) operands, L = 64 / 128 / 256:
// SYRK 1030 x 260 (one chain dominates) 3.5e-7 / 5.7e-7 / 1.05e-6; SYRK
// 4096 x 8192 (the folds dominate) 7.8e-7 / 6.2e-7 / 4.5e-7; C2a (N(0, 1))
// 6.1e-7 / 4.2e-7 / 3.6e-7, at 1.094 / 1.057 / 1.046 ms. Hence L grows with
// K. 16-bit operands keep L >= 128 (two of their 64-wide k-tiles: the DMA
// kernel folds after an even number of k-tiles).
static inline int chain_length(int64_t K, int elem_bytes) {
  const int L = K <= 1024 ? 64 : K <= 4096 ? 128 : K < 16384 ? 256 : K < 65536 ? 512 : 1024;
  return elem_bytes == 2 && L < 128 ? 128 : L;
}

__device__ __forceinline__ void fold_span(f32x16& sum, f32x16& acc) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    sum[r] += acc[r];
    acc[r] = 0.0f;
  }
}

// acc += a * b over one fragment: 4 fp32 MFMAs (one per element) or one
// 16-bit MFMA.
__device__ __forceinline__ void mma_frag(f32x16& acc, const i32x4& a, const i32x4& b, float*) {
  const f32x4 av = __builtin_bit_cast(f32x4, a);
  const f32x4 bv = __builtin_bit_cast(f32x4, b);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[0], bv[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[1], bv[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[2], bv[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[3], bv[3], acc, 0, 0, 0);
}
__device__ __forceinline__ void mma_frag(f32x16& acc, const i32x4& a, const i32x4& b, __bf16*) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
}
__device__ __forceinline__ void mma_frag(f32x16& acc, const i32x4& a, const i32x4& b,
                                         _Float16*) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                               __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
}

// Fragment of 32 rows (row index `row` for this lane) at k offset `kk`:
// from a K-contiguous LDS panel (one 16-byte read) or an M/N-contiguous one
// (EV column reads).
template <typename T, bool KC, int ROWS, int BK>
__device__ __forceinline__ i32x4 read_frag(const T* buf, int row, int kk) {
  constexpr int EV = 16 / sizeof(T);
  if (KC) {
    return *reinterpret_cast<const i32x4*>(buf + row * (BK + EV) + kk);
  } else {
    union {
      i32x4 v;
      T e[EV];
    } u;
#pragma unroll
    for (int e = 0; e < EV; ++e) u.e[e] = buf[(kk + e) * (ROWS + EV) + row];
    return u.v;
  }
}

// Lower-triangle tile t -> (tm, tn), tm >= tn, of a triangle T tiles on a
// side, in groups of 8 tile rows: group G (rows 8G .. 8G + R - 1, R = 8 but
// for the last) lists its whole columns tn < 8G (R tiles each, top to
// bottom), then its own R-row triangle column by column; groups start at
// tile 32 G^2 + 4 G. Consecutive tiles (one XCD's share of a round) then
// cover an 8-row, 8-column block of operand panels (13-20 distinct panels per
// 64 tiles of a 32-tile side, against ~35 for a row-major walk).
__device__ __forceinline__ void tri_tile(int t, int T, int& tm, int& tn) {
  int G = (int)((sqrtf(16.0f + 128.0f * (float)t) - 4.0f) * (1.0f / 64.0f));
  while (G > 0 && 32 * G * G + 4 * G > t) --G;
  while ((G + 1) * 8 < T && 32 * (G + 1) * (G + 1) + 4 * (G + 1) <= t) ++G;
  int u = t - (32 * G * G + 4 * G);
  const int R = min(8, T - 8 * G);
  if (u < 8 * G * R) {
    tm = 8 * G + u % R;
    tn = u / R;
    return;
  }
  u -= 8 * G * R;
  int c = 0;
  while (u >= R - c) {
    u -= R - c;
    ++c;
  }
  tm = 8 * G + c + u;
  tn = 8 * G + c;
}

// SYRK: whether the upper triangle of C is the one referenced: g.uplo, or,
// with triangle flags (flags[0]: the strict upper triangle holds a nonzero,
// flags[1]: the strict lower one), the other triangle when only that one
// holds off-diagonal entries (the rule of trnblas/level3.py:305-329, decided
// on the device so the host need not wait for the flags before the launch).
__device__ __forceinline__ int syrk_upper(const GemmArgs& g) {
  int up = g.uplo;
  if (g.tri != nullptr) {
    const int has_up = g.tri[0], has_lo = g.tri[1];
    if (up ? (has_lo && !has_up) : (has_up && !has_lo)) up ^= 1;
  }
  return up;
}

// D = alpha acc + beta C for one output element (C not read when beta == 0);
// SYRK: m >= n only, written to both triangles, C read from the side `up`
// (syrk_upper).
template <typename T, bool SYRK>
__device__ __forceinline__ void store_out(const GemmArgs& g, const T* C, T* D, int m, int n,
                                          float acc, int up = 0) {
  if (SYRK) {
    if (m < g.M && n <= m) {
      float v = g.alpha * acc;
      if (g.beta != 0.0f) {
        const int64_t ci = up ? (int64_t)n * g.ldc + m : (int64_t)m * g.ldc + n;
        v = __builtin_fmaf(g.beta, to_f32(C[ci]), v);  // one rounding, in every epilogue
      }
      const T o = (T)v;
      D[(int64_t)m * g.ldd + n] = o;
      D[(int64_t)n * g.ldd + m] = o;
    }
  } else if (m < g.M && n < g.N) {
    float v = g.alpha * acc;
    if (g.beta != 0.0f) v = __builtin_fmaf(g.beta, to_f32(C[(int64_t)m * g.ldc + n]), v);
    D[(int64_t)m * g.ldd + n] = (T)v;
  }
}

// Four consecutive values of T at p (4-element aligned) as floats, and back
// (one 16-byte access for fp32, 8 bytes for 16-bit types).
template <typename T>
__device__ __forceinline__ void load4(const T* p, float (&v)[4]) {
  union {
    u32x2 u2;
    f32x4 f;
    T e[4];
  } x;
  if constexpr (sizeof(T) == 4)
    x.f = *reinterpret_cast<const f32x4*>(p);
  else
    x.u2 = *reinterpret_cast<const u32x2*>(p);
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = to_f32(x.e[e]);
}
template <typename T>
__device__ __forceinline__ void store4(T* p, const float (&v)[4]) {
  union {
    u32x2 u2;
    f32x4 f;
    T e[4];
  } x;
#pragma unroll
  for (int e = 0; e < 4; ++e) x.e[e] = (T)v[e];
  if constexpr (sizeof(T) == 4)
    *reinterpret_cast<f32x4*>(p) = x.f;
  else
    *reinterpret_cast<u32x2*>(p) = x.u2;
}

// Tile t -> (batch, tile row, tile column).
template <bool SYRK>
__device__ __forceinline__ void decode_tile(const GemmArgs& g, int t, int& bat, int& tm, int& tn) {
  if (SYRK) {
    bat = 0;
    tri_tile(t, g.tiles_m, tm, tn);
  } else {
    const int per = g.tiles_m * g.tiles_n;
    bat = t / per;
    grouped_tile(t - bat * per, g.tiles_m, g.tiles_n, 8, tm, tn);
  }
}

// Stream-K: workgroup w owns k-iterations [sk_start(w), sk_start(w + 1)) of
// the tiles x nk iteration space.
__device__ __forceinline__ int64_t sk_start(int w, int64_t total, int groups) {
  return (int64_t)w * total / groups;
}

// Epilogue of one segment: alpha / beta into D (slot < 0, whole tile) or the
// raw partial into workspace slot `slot` of workgroup w (stream-K).
// Lane l of an MFMA 32x32 block holds column l % 32 and rows
// 8 (r / 4) + 4 (l / 32) + r % 4 of its 16 registers r.
template <typename T, bool SYRK, int FM, int FN, int BM, int BN>
__device__ __forceinline__ void store_tile(const GemmArgs& g, const f32x16 (&acc)[FM][FN], int bat,
                                           int m0, int n0, int wm0, int wn0, int lane, int slot,
                                           int w) {
  if (slot < 0) {
    const T* C = static_cast<const T*>(g.C) + (g.C ? bat * g.sC : 0);
    T* D = static_cast<T*>(g.D) + bat * g.sD;
    const int up = SYRK ? syrk_upper(g) : 0;
    if (SYRK && m0 > n0 && m0 + BM <= g.M && g.vec4) {
      // A SYRK tile strictly below the diagonal with every row inside: each
      // lane's registers r = 4 s .. 4 s + 3 are 4 consecutive rows of one
      // column, so the mirrored values D[n][m .. m + 3] (and C[n][m .. m + 3]
      // when the upper triangle is referenced) move as one vector per lane.
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int mb = m0 + wm0 + i * 32 + (lane >> 5) * 4;
          const int n = n0 + wn0 + j * 32 + (lane & 31);
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int m = mb + 8 * s;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = g.alpha * acc[i][j][4 * s + e];
            if (g.beta != 0.0f) {
              if (up) {
                float c[4];
                load4(C + (int64_t)n * g.ldc + m, c);
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = __builtin_fmaf(g.beta, c[e], v[e]);
              } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                  v[e] = __builtin_fmaf(g.beta, to_f32(C[(int64_t)(m + e) * g.ldc + n]), v[e]);
              }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) D[(int64_t)(m + e) * g.ldd + n] = (T)v[e];
            store4(D + (int64_t)n * g.ldd + m, v);
          }
        }
      return;
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int mb = m0 + wm0 + i * 32 + (lane >> 5) * 4;
        const int n = n0 + wn0 + j * 32 + (lane & 31);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          store_out<T, SYRK>(g, C, D, mb + (r >> 2) * 8 + (r & 3), n, acc[i][j][r], up);
      }
  } else {
    float* P = g.ws + ((int64_t)w * 2 + slot) * (BM * BN);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int mb = wm0 + i * 32 + (lane >> 5) * 4;
        const int n = wn0 + j * 32 + (lane & 31);
#pragma unroll
        for (int r = 0; r < 16; ++r) P[(mb + (r >> 2) * 8 + (r & 3)) * BN + n] = acc[i][j][r];
      }
  }
}

// Each workgroup computes whole tiles (data-parallel: one tile per
// workgroup) or, under stream-K, a contiguous range of the k-iterations of
// all tiles: whole tiles it covers get the epilogue directly, the partial
// tiles at either end of its range are written to its two workspace slots
// and summed by gemm_fixup_kernel.
template <typename T, int BM, int BN, int BK, int WM, int WN, bool AKC, bool BKC, bool VEC,
          bool SYRK>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64, 1) void gemm_kernel(GemmArgs g) {
  constexpr int EV = 16 / sizeof(T);
  constexpr int NT = (BM / WM) * (BN / WN) * 64;
  constexpr int WAVES_N = BN / WN;
  constexpr int FM = WM / 32, FN = WN / 32;
  constexpr int CH = 2 * EV;  // k per fragment read
  static_assert(BK % CH == 0, "BK must be a multiple of the fragment k");
  // LDS panels: [row][k] (K-contiguous) or [k][row], rows padded by EV.
  constexpr int A_LC = AKC ? BK : BM, A_LR = AKC ? BM : BK;
  constexpr int B_LC = BKC ? BK : BN, B_LR = BKC ? BN : BK;
  constexpr int A_SZ = A_LR * (A_LC + EV), B_SZ = B_LR * (B_LC + EV);
  constexpr int A_NV = A_LR * A_LC / EV / NT, B_NV = B_LR * B_LC / EV / NT;
  static_assert(A_NV * EV * NT == A_LR * A_LC && B_NV * EV * NT == B_LR * B_LC, "tile split");
  constexpr int NB = (sizeof(T) == 4 && BK == 64) ? 1 : 2;  // LDS stages
  __shared__ __attribute__((aligned(16))) T lds[NB * (A_SZ + B_SZ)];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave / WAVES_N) * WM, wn0 = (wave % WAVES_N) * WN;
  const int M = g.M, N = g.N, K = g.K;
  const int nk = g.nk;

  // One segment: k-iterations [kb0, kb1) of tile t; slot < 0 = whole tile.
  auto segment = [&](int t, int kb0, int kb1, int slot, int w) {
    int bat, tm, tn;
    decode_tile<SYRK>(g, t, bat, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const T* A = static_cast<const T*>(g.A) + bat * g.sA;
    const T* B = static_cast<const T*>(g.B) + bat * g.sB;

    // Per-thread offsets inside a k-tile are loop invariant; the tile corner
    // moves with k0 (scalar base of the buffer resource).
    i32x4 ra[A_NV], rb[B_NV];
    auto load_tiles = [&](int k0) {
      const __amdgpu_buffer_rsrc_t rsa =
          make_rsrc(AKC ? A + (int64_t)m0 * g.lda + k0 : A + (int64_t)k0 * g.lda + m0);
      const __amdgpu_buffer_rsrc_t rsb =
          make_rsrc(BKC ? B + (int64_t)n0 * g.ldb + k0 : B + (int64_t)k0 * g.ldb + n0);
#pragma unroll
      for (int i = 0; i < A_NV; ++i) {
        const int idx = tid + i * NT, r = idx / (A_LC / EV), c = (idx % (A_LC / EV)) * EV;
        const uint32_t off = (uint32_t)((r * g.lda + c) * (int64_t)sizeof(T));
        // AKC: rows are m, columns k. Otherwise rows are k, columns m.
        const int rl = AKC ? M - m0 : K - k0, cl = AKC ? K - k0 : M - m0;
        ra[i] = load_group<T, VEC>(rsa, off, r < rl && c < cl, cl - c);
      }
#pragma unroll
      for (int i = 0; i < B_NV; ++i) {
        const int idx = tid + i * NT, r = idx / (B_LC / EV), c = (idx % (B_LC / EV)) * EV;
        const uint32_t off = (uint32_t)((r * g.ldb + c) * (int64_t)sizeof(T));
        // BKC: rows are n, columns k. Otherwise rows are k, columns n.
        const int rl = BKC ? N - n0 : K - k0, cl = BKC ? K - k0 : N - n0;
        rb[i] = load_group<T, VEC>(rsb, off, r < rl && c < cl, cl - c);
      }
    };
    auto store_tiles = [&](int buf) {
      T* la = lds + buf * (A_SZ + B_SZ);
      T* lb = la + A_SZ;
#pragma unroll
      for (int i = 0; i < A_NV; ++i) {
        const int idx = tid + i * NT, r = idx / (A_LC / EV), c = (idx % (A_LC / EV)) * EV;
        *reinterpret_cast<i32x4*>(la + r * (A_LC + EV) + c) = ra[i];
      }
#pragma unroll
      for (int i = 0; i < B_NV; ++i) {
        const int idx = tid + i * NT, r = idx / (B_LC / EV), c = (idx % (B_LC / EV)) * EV;
        *reinterpret_cast<i32x4*>(lb + r * (B_LC + EV) + c) = rb[i];
      }
    };

    f32x16 acc[FM][FN], sum[FM][FN];  // current MFMA chain, folded chains
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = sum[i][j][r] = 0.0f;

    if (kb1 > kb0) {
      load_tiles(kb0 * BK);
      store_tiles(0);
      if (NB == 1 && kb0 + 1 < kb1) load_tiles((kb0 + 1) * BK);
      __syncthreads();
    }
    int chain = g.span;  // k-tiles left in the current MFMA chain
    for (int kt = kb0; kt < kb1; ++kt) {
      const int cur = NB == 1 ? 0 : (kt - kb0) & 1;
      const bool more = kt + 1 < kb1;
      if (NB == 2 && more) load_tiles((kt + 1) * BK);
      const T* la = lds + cur * (A_SZ + B_SZ);
      const T* lb = la + A_SZ;
#pragma unroll
      for (int c = 0; c < BK / CH; ++c) {
        const int kk = c * CH + (lane >> 5) * EV;
        i32x4 fa[FM], fb[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
          fa[i] = read_frag<T, AKC, BM, BK>(la, wm0 + i * 32 + (lane & 31), kk);
#pragma unroll
        for (int j = 0; j < FN; ++j)
          fb[j] = read_frag<T, BKC, BN, BK>(lb, wn0 + j * 32 + (lane & 31), kk);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) mma_frag(acc[i][j], fa[i], fb[j], (T*)nullptr);
      }
      if (--chain == 0) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) fold_span(sum[i][j], acc[i][j]);
        chain = g.span;
      }
      if (NB == 2) {
        if (more) store_tiles(cur ^ 1);
        __syncthreads();
      } else {
        // One stage: every wave is done reading before tile kt + 1 is
        // stored; tile kt + 2 is then requested into the freed registers.
        __syncthreads();
        if (more) {
          store_tiles(0);
          if (kt + 2 < kb1) load_tiles((kt + 2) * BK);
          __syncthreads();
        }
      }
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) fold_span(sum[i][j], acc[i][j]);

    store_tile<T, SYRK, FM, FN, BM, BN>(g, sum, bat, m0, n0, wm0, wn0, lane, slot, w);
  };

  if (g.sk_groups == 0) {
    segment(xcd_remap(blockIdx.x, gridDim.x), 0, nk, -1, 0);
    return;
  }
  // Hybrid schedule: the first dp_tiles tiles whole (G per round), then the
  // k-iterations of the remaining tiles split evenly over the G workgroups.
  const int G = g.sk_groups;
  const int w = xcd_remap(blockIdx.x, gridDim.x);
  for (int t = w; t < g.dp_tiles; t += G) segment(t, 0, nk, -1, w);
  const int64_t total = (int64_t)(g.ntiles - g.dp_tiles) * nk;
  const int64_t x0 = sk_start(w, total, G), x1 = sk_start(w + 1, total, G);
  for (int64_t x = x0; x < x1;) {
    const int tt = (int)(x / nk);
    const int kb0 = (int)(x - (int64_t)tt * nk);
    const int kb1 = (int)((int64_t)kb0 + (x1 - x) < nk ? kb0 + (x1 - x) : nk);
    const bool whole = kb0 == 0 && kb1 == nk;
    segment(g.dp_tiles + tt, kb0, kb1, whole ? -1 : (x == x0 ? 0 : 1), w);
    x += kb1 - kb0;
  }
}

// One 16-byte-per-lane LDS DMA (buffer_load_dwordx4 ... lds) of the wave:
// lane l's group at offset voff of the resource lands at lds + 16 l. (A
// non-template helper: the builtin with a type-dependent LDS pointer does
// not instantiate in a kernel template's host pass.)
__device__ __forceinline__ void lds_dma16(const void* base, void* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(base),
                                           (__attribute__((address_space(3))) void*)lds, 16, voff,
                                           0, 0, 0);
}

// Lane layout of ds_read_b64_tr_b16 (gfx950), measured with an in-bounds
// probe: in each group of 16 lanes every lane loads 8 bytes (four 16-bit
// values) at its own address, and lane i receives, for j = 0..3, value i % 4
// of the 8 bytes loaded by lane 4 j + i / 4 of its group.
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ s16x4 lds_tr16(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(const_cast<void*>(p)));
}

// GEMM / SYRK on 16-byte aligned operands (fp32, bf16, fp16): the tile,
// wave split, MFMA (v_mfma_f32_32x32x2_f32, v_mfma_f32_32x32x16_{bf16,f16})
// and k order of gemm_kernel, with the operand panels moved by LDS DMA
// (buffer_load_dwordx4 ... lds) instead of through registers. k-tiles of
// 128 bytes per K-contiguous row (32 fp32 / 64 bf16 or fp16 values) in two
// LDS stages; after the barrier that publishes k-tile t every wave reads all
// its fragments of k-tile t, then issues the DMA of k-tile t + 1 into the
// other stage, which lands behind k-tile t's MFMAs: one barrier per k-tile,
// no staging registers and no LDS stores. (The compiler makes an LDS read
// that follows an outstanding LDS DMA wait for it, so no read may follow
// the DMA inside a k-tile.)
//
// The panels have no row padding; their 16-byte groups are XOR-swizzled, so
// a 1 KiB DMA block (lane l writes bytes 16 l .. 16 l + 15) is a set of
// whole rows and the fragment reads are bank-conflict free:
//  * K-contiguous panel, 128 rows of 128 bytes: group q of row r sits in
//    slot q ^ ((r >> 1) & 7); a DMA block is 8 rows;
//  * M/N-contiguous panel, rows k of 128 values (512 or 256 bytes): fp32,
//    group q of row k sits in slot q ^ (8 ((k / 4) & 1)), which moves the
//    second lane half's column reads (k + 4) onto the other half of the
//    banks; 16-bit, in slot q ^ (4 (k & 3)): the transposing reads of a
//    16-lane group take rows k .. k + 3 at the same columns, and the 64-byte
//    shift per row puts them on distinct banks (the 64-value rows of BN = 64
//    keep q ^ (4 ((k / 8) & 1))); a DMA block is 2 (fp32) or 4 rows.
// Lane l of a DMA block loads the global group that belongs in its slot
// (the swizzles are their own inverses), so each row's lanes still read the
// row's bytes exactly once. Ragged edges: a group outside the matrix gets
// an offset past the buffer's records and reads as zeros (VEC operands:
// every 16-byte group is wholly inside or outside).
//
// BN = 64 (GEMM only): 128 x 64 tiles, waves of 64 x 32 (one MFMA block
// column), a 64-row B panel (8 DMA blocks, two per wave; M/N-contiguous rows
// of 64 values keep the same swizzle), for launches whose 128 x 128 tiles
// would fill at most one workgroup slot per CU (launch_narrow).
template <typename T, bool AKC, bool BKC, bool SYRK, int BN = 128>
__global__ __launch_bounds__(256, 2) void gemm_dma_kernel(GemmArgs g) {
  constexpr int EV = 16 / sizeof(T);  // values per 16-byte group
  constexpr int BM = 128, BK = 128 / sizeof(T), WM = 64, WN = BN / 2, FM = 2, FN = WN / 32;
  static_assert(BN == 128 || (BN == 64 && !SYRK), "tile shapes: 128 x 128, or 128 x 64 for GEMM");
  constexpr int CH = 2 * EV;          // k per fragment chunk (both lane halves)
  constexpr int PANEL = 128 * BK;     // values of the A panel (16 KiB)
  constexpr int BPANEL = BN * BK;     // values of the B panel
  constexpr int MGA = 128 / EV, MGB = BN / EV;  // 16-byte groups in an M/N-contiguous row
  constexpr int NBW = BPANEL * (int)sizeof(T) / 4096;  // B DMA blocks per wave (4 or 2)
  constexpr int MSW = 2 * sizeof(T);  // M/N swizzle (groups)
  // slot XOR of row k of an M/N-contiguous panel with mg 16-byte groups per row
  auto mn_swz = [](int k, int mg) __attribute__((always_inline)) {
    return (sizeof(T) == 2 && mg == 16) ? 4 * (k & 3) : MSW * ((k / EV) & 1);
  };
  __shared__ __attribute__((aligned(16))) T st0[PANEL + BPANEL];
  __shared__ __attribute__((aligned(16))) T st1[PANEL + BPANEL];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
  const int M = g.M, N = g.N, K = g.K, nk = g.nk;

  auto segment = [&](int t, int kb0, int kb1, int slot, int w) {
    // The lane index is made opaque per segment: otherwise every per-lane LDS
    // address of the segment is hoisted out of the work loop and kept live
    // across it, which spills.
    int lane = tid & 63;
    asm volatile("" : "+v"(lane));
    int bat, tm, tn;
    decode_tile<SYRK>(g, t, bat, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const T* A = static_cast<const T*>(g.A) + bat * g.sA;
    const T* B = static_cast<const T*>(g.B) + bat * g.sB;

    // the DMA of k-tile kt into stage st (A panel, then B panel)
    auto dma = [&](T* st, int kt) {
      const int k0 = kt * BK;
      const T* pa = AKC ? A + (int64_t)m0 * g.lda + k0 : A + (int64_t)k0 * g.lda + m0;
      const T* pb = BKC ? B + (int64_t)n0 * g.ldb + k0 : B + (int64_t)k0 * g.ldb + n0;
      // rows / columns of the matrix left from the panel's corner
      const int ra = AKC ? M - m0 : K - k0, ca = AKC ? K - k0 : M - m0;
      const int rb = BKC ? N - n0 : K - k0, cb = BKC ? K - k0 : N - n0;
      // wave w fills blocks nb w .. nb w + nb - 1 of a panel (nb = 4 for A,
      // NBW for B). KC block b: row 8 b + l / 8, global group (l % 8) ^
      // swizzle; MN block b (rows of mg groups): row (64 / mg) b + l / mg,
      // global group (l % mg) ^ swizzle.
      auto geo = [&](bool kc, int mg, int nb, int u, int& row, int& grp)
                     __attribute__((always_inline)) {
        const int b = nb * wave + u;
        if (kc) {
          row = 8 * b + (lane >> 3);
          grp = (lane & 7) ^ ((row >> 1) & 7);
        } else {
          row = (64 / mg) * b + lane / mg;
          grp = (lane % mg) ^ mn_swz(row, mg);
        }
      };
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        int rw, gp;
        geo(AKC, MGA, 4, u, rw, gp);
        const bool oka = rw < ra && EV * gp < ca;
        const uint32_t va =
            oka ? (uint32_t)((int64_t)rw * g.lda * (int64_t)sizeof(T) + 16 * gp) : kOob;
        lds_dma16(pa, st + (4 * wave + u) * (1024 / sizeof(T)), va);
      }
#pragma unroll
      for (int u = 0; u < NBW; ++u) {
        int rw, gp;
        geo(BKC, MGB, NBW, u, rw, gp);
        const bool okb = rw < rb && EV * gp < cb;
        const uint32_t vb =
            okb ? (uint32_t)((int64_t)rw * g.ldb * (int64_t)sizeof(T) + 16 * gp) : kOob;
        lds_dma16(pb, st + PANEL + (NBW * wave + u) * (1024 / sizeof(T)), vb);
      }
    };

    f32x16 acc[FM][FN], sum[FM][FN];  // current MFMA chain, folded chains
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = sum[i][j][r] = 0.0f;
    auto fold = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) fold_span(sum[i][j], acc[i][j]);
    };

    // Fragment of the lane's row r (32 rows per MFMA block) at k offset kk
    // (EV consecutive k, kk a multiple of EV): one 16-byte read from a
    // K-contiguous panel, EV column reads from an M/N-contiguous one (rows
    // of W values: the panel's width).
    auto frag = [&](const T* p, bool kc, int r, int kk, int W) __attribute__((always_inline)) {
      if (kc)
        return *reinterpret_cast<const i32x4*>(p + r * BK + EV * ((kk / EV) ^ ((r >> 1) & 7)));
      if constexpr (sizeof(T) == 2) {
        // Two transposing reads: in each 16-lane group (rows rb .. rb + 15,
        // one k-octet) lane i loads row k + i / 4, columns rb + 4 (i % 4) ..
        // + 3 of the panel (8 bytes of one swizzled 16-byte slot), and
        // receives column rb + i of rows k .. k + 3.
        const int i = lane & 15;
        const int c0 = r - i + 4 * (i & 3);
        const int k1 = kk + (i >> 2);
        const T* s0 = p + k1 * W + EV * ((c0 / EV) ^ mn_swz(k1, W / EV)) + (c0 & 4);
        union {
          s16x4 h[2];
          i32x4 v;
        } u;
        u.h[0] = lds_tr16(s0);
        u.h[1] = lds_tr16(s0 + 4 * W);
        return u.v;
      }
      const T* q = p + EV * ((r / EV) ^ (MSW * ((kk / EV) & 1))) + (r % EV);
      union {
        i32x4 v;
        T e[EV];
      } u;
#pragma unroll
      for (int e = 0; e < EV; ++e) u.e[e] = q[(kk + e) * W];
      return u.v;
    };
    // One k-tile from stage `cur`: every fragment of the k-tile is read into
    // registers (64 VGPRs) before the DMA of k-tile `next` (< 0: none) into
    // the other stage issues, then the 64 MFMAs run behind that DMA.
    // On a SYRK diagonal tile the wave of rows 0-63, columns 64-127 holds
    // only entries above the diagonal: it moves its share of the panels and
    // keeps the barriers, but reads no fragments and runs no MFMAs (its
    // accumulators stay zero and its store writes nothing).
    // `busy` is also a runtime (opaque) condition for GEMM: as a branch it
    // keeps the fragment reads, the DMA and the MFMAs of a k-tile in separate
    // blocks; scheduled as one block they hold the folded sums, the chain and
    // the fragments live together with hoisted addresses, and spill.
    int on = 1;
    asm volatile("" : "+s"(on));
    const bool busy = SYRK ? !(tm == tn && wn0 > wm0) : on != 0;
    auto step = [&](const T* cur, T* oth, int next) __attribute__((always_inline)) {
      i32x4 fa[BK / CH][FM], fb[BK / CH][FN];
      if (busy) {
#pragma unroll
        for (int c = 0; c < BK / CH; ++c) {
          const int kk = c * CH + (lane >> 5) * EV;
#pragma unroll
          for (int i = 0; i < FM; ++i)
            fa[c][i] = frag(cur, AKC, wm0 + i * 32 + (lane & 31), kk, 128);
#pragma unroll
          for (int j = 0; j < FN; ++j)
            fb[c][j] = frag(cur + PANEL, BKC, wn0 + j * 32 + (lane & 31), kk, BN);
        }
      }
      if (next >= 0) dma(oth, next);
      if (busy) {
#pragma unroll
        for (int c = 0; c < BK / CH; ++c)
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) mma_frag(acc[i][j], fa[c][i], fb[c][j], (T*)nullptr);
      }
    };

    __syncthreads();  // a previous segment's reads of both stages are done
    if (kb1 > kb0) dma(st0, kb0);
    int chain = g.span;  // k-tiles left in the current MFMA chain (span is even)
    for (int kt = kb0; kt < kb1; kt += 2) {
      __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA of k-tile kt has landed
      __syncthreads();                // every wave's has; every read of st1 is done
      step(st0, st1, kt + 1 < kb1 ? kt + 1 : -1);
      if (kt + 1 >= kb1) break;
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      step(st1, st0, kt + 2 < kb1 ? kt + 2 : -1);
      chain -= 2;
      if (chain == 0) {
        fold();
        chain = g.span;
      }
    }
    fold();
    store_tile<T, SYRK, FM, FN, BM, BN>(g, sum, bat, m0, n0, wm0, wn0, lane, slot, w);
  };

  // Work of this workgroup, walked with one call site of `segment` (two
  // inlined copies of it do not fit the register budget): data-parallel, the
  // tile w; under stream-K, whole tiles w, w + G, ... below dp_tiles, then
  // the k-iteration range [x0, x1) of the remaining tiles.
  const int w = xcd_remap(blockIdx.x, gridDim.x);
  const bool sk = g.sk_groups != 0;
  const int G = sk ? g.sk_groups : 1;
  const int64_t total = sk ? (int64_t)(g.ntiles - g.dp_tiles) * nk : 0;
  int64_t x = sk ? sk_start(w, total, G) : 0;
  const int64_t x1 = sk ? sk_start(w + 1, total, G) : 0;
  const int64_t x0 = x;
  int tw = w;  // next whole tile
  const int tw_end = sk ? g.dp_tiles : w + 1;
  for (;;) {
    int t, kb0, kb1, slot;
    if (tw < tw_end) {
      t = tw;
      kb0 = 0;
      kb1 = nk;
      slot = -1;
      tw += G;
    } else if (x < x1) {
      const int tt = (int)(x / nk);
      kb0 = (int)(x - (int64_t)tt * nk);
      kb1 = (int)((int64_t)kb0 + (x1 - x) < nk ? kb0 + (x1 - x) : nk);
      t = g.dp_tiles + tt;
      slot = (kb0 == 0 && kb1 == nk) ? -1 : (x == x0 ? 0 : 1);
      x += kb1 - kb0;
    } else {
      break;
    }
    segment(t, kb0, kb1, slot, w);
  }
}

// 16-bit GEMM on 256 x 256 tiles (aligned operands, whole tiles, one
// workgroup per CU). A 128 x 128 tile stages 32 KiB per 64-wide k-tile for
// 512 cycles of MFMA issue per SIMD, less than its LDS DMA takes at ~40
// bytes per clock per CU; a 256 x 256 tile stages twice the bytes for four
// times the MFMAs. 512 threads: wave w owns rows 128 (w & 1) .. + 127 and
// columns 64 (w >> 1) .. + 63 (4 x 2 MFMA 32x32x16 blocks). The K-contiguous
// panels, DMA blocks and fragment reads are those of gemm_dma_kernel with
// 256-row panels; an M/N-contiguous panel has rows k of 256 values (a DMA
// block is two rows) with group q of row k in slot q ^ (4 (k & 3)): the
// transposing reads of a 16-lane group take rows k .. k + 3 at the same
// columns, and the 64-byte shift per row puts them on distinct banks (with
// gemm_dma_kernel's swizzle, half of the kernel's LDS cycles were bank
// conflicts). Two LDS stages of 64 KiB; each wave moves 4 blocks of each
// panel per k-tile. The DMA is issued by inline asm (invisible to the compiler's
// wait tracking), so fragment reads of the current stage may follow it; the
// kernel waits for its own DMAs (vmcnt(0)) before the barrier that
// publishes the next stage. Fragments are read one 16-wide k chunk ahead of
// the MFMAs (two sets of six). One MFMA chain over all of K (no folded
// partial sums: 16-bit results are held to 2^-8 |A||B|, far above an fp32
// chain's rounding).
template <typename T, bool AKC, bool BKC>
__global__ __launch_bounds__(512, 1) void hgemm256_kernel(GemmArgs g) {
  static_assert(sizeof(T) == 2, "16-bit operands");
  constexpr int EV = 8, BM = 256, BN = 256, BK = 64, WM = 128, WN = 64, FM = 4, FN = 2;
  constexpr int NB = 4;                // DMA blocks per panel per wave
  constexpr int CH = 2 * EV;           // k per fragment chunk
  constexpr int PANEL = BM * BK;       // values of one panel (32 KiB)
  constexpr int MG = 256 / EV;         // 16-byte groups in an M/N-contiguous row
  __shared__ __attribute__((aligned(16))) T lds[2][2 * PANEL];

  const int tid = threadIdx.x;
  int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm0 = (wave & 1) * WM, wn0 = (wave >> 1) * WN;
  const int M = g.M, N = g.N, K = g.K, nk = g.nk;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  int bat, tm, tn;
  decode_tile<false>(g, t, bat, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const T* A = static_cast<const T*>(g.A) + bat * g.sA;
  const T* B = static_cast<const T*>(g.B) + bat * g.sB;

  // DMA block b = 4 wave + u of a panel. KC: row 8 b + l / 8, global group
  // (l % 8) ^ swizzle; MN: row 2 b + l / 32, global group (l % 32) ^ swizzle.
  auto geo = [&](bool kc, int u, int& row, int& grp) __attribute__((always_inline)) {
    const int b = NB * wave + u;
    if (kc) {
      row = 8 * b + (lane >> 3);
      grp = (lane & 7) ^ ((row >> 1) & 7);
    } else {
      row = 2 * b + lane / MG;
      grp = (lane % MG) ^ (4 * (row & 3));
    }
  };
  auto dma = [&](T* st, int kt) __attribute__((always_inline)) {
    const int k0 = kt * BK;
    const T* pa = AKC ? A + (int64_t)m0 * g.lda + k0 : A + (int64_t)k0 * g.lda + m0;
    const T* pb = BKC ? B + (int64_t)n0 * g.ldb + k0 : B + (int64_t)k0 * g.ldb + n0;
    const int ra = AKC ? M - m0 : K - k0, ca = AKC ? K - k0 : M - m0;
    const int rb = BKC ? N - n0 : K - k0, cb = BKC ? K - k0 : N - n0;
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      int rw, gp;
      geo(AKC, u, rw, gp);
      const uint32_t va = rw < ra && EV * gp < ca
                              ? (uint32_t)((int64_t)rw * g.lda * (int64_t)sizeof(T) + 16 * gp)
                              : kOob;
      lds_dma16_asm(pa, st + (NB * wave + u) * (1024 / sizeof(T)), va, 0);
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      int rw, gp;
      geo(BKC, u, rw, gp);
      const uint32_t vb = rw < rb && EV * gp < cb
                              ? (uint32_t)((int64_t)rw * g.ldb * (int64_t)sizeof(T) + 16 * gp)
                              : kOob;
      lds_dma16_asm(pb, st + PANEL + (NB * wave + u) * (1024 / sizeof(T)), vb, 0);
    }
  };

  // Fragment of the lane's row r at k offset kk (a multiple of EV): one
  // 16-byte read from a K-contiguous panel, two transposing 8-byte reads
  // from an M/N-contiguous one (rows of 256 values).
  auto frag = [&](const T* p, bool kc, int r, int kk) __attribute__((always_inline)) {
    if (kc)
      return *reinterpret_cast<const i32x4*>(p + r * BK + EV * ((kk / EV) ^ ((r >> 1) & 7)));
    const int i = lane & 15;
    const int c0 = r - i + 4 * (i & 3);
    const int k1 = kk + (i >> 2);
    const T* s0 = p + k1 * BM + EV * ((c0 / EV) ^ (4 * (k1 & 3))) + (c0 & 4);
    union {
      s16x4 h[2];
      i32x4 v;
    } u;
    u.h[0] = lds_tr16(s0);
    u.h[1] = lds_tr16(s0 + 4 * BM);
    return u.v;
  };
  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  i32x4 fa[2][FM], fb[2][FN];
  auto rd = [&](const T* cur, int c, int set) __attribute__((always_inline)) {
    const int kk = c * CH + (lane >> 5) * EV;
#pragma unroll
    for (int i = 0; i < FM; ++i) fa[set][i] = frag(cur, AKC, wm0 + i * 32 + (lane & 31), kk);
#pragma unroll
    for (int j = 0; j < FN; ++j) fb[set][j] = frag(cur + PANEL, BKC, wn0 + j * 32 + (lane & 31), kk);
  };
  auto mm = [&](int set) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) mma_frag(acc[i][j], fa[set][i], fb[set][j], (T*)nullptr);
  };
  auto publish = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  // One k-tile per iteration with the stage chosen at run time (unrolled
  // copies per stage give the accumulators different registers in each copy
  // and spill at the joins): chunk 0's fragments, the DMA of k-tile kt + 1
  // into the other stage, then chunk c's MFMAs behind chunk c + 1's reads,
  // with scheduling barriers that keep each chunk's reads behind the MFMAs
  // two chunks back (else all four chunks' fragments are live at once).
  if (nk > 0) dma(lds[0], 0);
  for (int kt = 0; kt < nk; ++kt) {
    publish();  // k-tile kt has landed; every read of the other stage is done
    // the lane index is opaque per k-tile, so its LDS and DMA addresses are
    // recomputed here instead of hoisted out of the loop and kept live
    asm volatile("" : "+v"(lane));
    const T* cur = lds[kt & 1];
    rd(cur, 0, 0);
    if (kt + 1 < nk) dma(lds[(kt & 1) ^ 1], kt + 1);
    rd(cur, 1, 1);
    __builtin_amdgcn_sched_barrier(0);
    mm(0);
    __builtin_amdgcn_sched_barrier(0);
    rd(cur, 2, 0);
    __builtin_amdgcn_sched_barrier(0);
    mm(1);
    __builtin_amdgcn_sched_barrier(0);
    rd(cur, 3, 1);
    __builtin_amdgcn_sched_barrier(0);
    mm(0);
    __builtin_amdgcn_sched_barrier(0);
    mm(1);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  store_tile<T, false, FM, FN, BM, BN>(g, acc, bat, m0, n0, wm0, wn0, lane, -1, 0);
}

// Sums the stream-K partials of each split tile in workgroup order
// (deterministic) and applies the epilogue. Grid: (split tiles, BM / 8):
// each workgroup finishes 8 rows of one tile, one float4 of partials per
// thread and contributor (all contributors' loads in flight at once).
template <typename T, int BM, int BN, bool SYRK>
__global__ __launch_bounds__(256) void gemm_fixup_kernel(GemmArgs g) {
  constexpr int MAXC = 64;  // contributors per tile (choose_sk keeps to it)
  constexpr int ROWS = 1024 / BN;
  static_assert(ROWS * BN / 4 == 256, "one float4 per thread");
  __shared__ int64_t src[MAXC];
  __shared__ int ncontrib;
  const int t = g.dp_tiles + blockIdx.x;
  const int nk = g.nk, G = g.sk_groups;
  const int64_t total = (int64_t)(g.ntiles - g.dp_tiles) * nk;
  const int64_t lo = (int64_t)blockIdx.x * nk, hi = lo + nk;
  if (threadIdx.x == 0) {
    int w0 = (int)(lo * G / total);
    while (w0 + 1 < G && sk_start(w0 + 1, total, G) <= lo) ++w0;
    while (w0 > 0 && sk_start(w0, total, G) > lo) --w0;
    int n = 0;
    if (!(sk_start(w0, total, G) <= lo && sk_start(w0 + 1, total, G) >= hi)) {
      for (int w = w0; w < G && n < MAXC; ++w) {
        const int64_t st = sk_start(w, total, G);
        if (st >= hi) break;
        src[n++] = ((int64_t)w * 2 + (st >= lo ? 0 : 1)) * (BM * BN);
      }
    }
    ncontrib = n;
  }
  __syncthreads();
  const int nc = ncontrib;
  if (nc == 0) return;  // whole tile, already written
  int bat, tm, tn;
  decode_tile<SYRK>(g, t, bat, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const T* C = static_cast<const T*>(g.C) + (g.C ? bat * g.sC : 0);
  T* D = static_cast<T*>(g.D) + bat * g.sD;
  const int r = blockIdx.y * ROWS + threadIdx.x / (BN / 4);
  const int c = (threadIdx.x % (BN / 4)) * 4;
  const int e = r * BN + c;
  const int up = SYRK ? syrk_upper(g) : 0;
  // contributors summed in order; their loads issued 8 at a time (a plain
  // loop would wait for each load before the next add)
  f32x4 v = *reinterpret_cast<const f32x4*>(g.ws + src[0] + e);
  int q = 1;
  for (; q + 8 <= nc; q += 8) {
    f32x4 p[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) p[u] = *reinterpret_cast<const f32x4*>(g.ws + src[q + u] + e);
#pragma unroll
    for (int u = 0; u < 8; ++u) v += p[u];
  }
  for (; q < nc; ++q) v += *reinterpret_cast<const f32x4*>(g.ws + src[q] + e);
#pragma unroll
  for (int u = 0; u < 4; ++u) store_out<T, SYRK>(g, C, D, m0 + r, n0 + c + u, v[u], up);
}

// fp32 GEMM with one workgroup per CU (sgemm_pipe_kernel), both operands
// M/N-contiguous (A^T B). A 128 x 128 tile per workgroup: eight compute
// waves of 64 x 32, two per SIMD (4 x 2 blocks of v_mfma_f32_16x16x4_f32),
// and four movers, waves that only move operands: k-tiles of 32 are loaded
// into the movers' registers two k-tiles ahead and stored into four LDS
// stages of 32 KiB (A panel, then B panel, each 32 k rows of 128 values).
// (LDS DMA was measured slower here: a wave's LDS DMAs complete one at a
// time, so compute waves that issued their share stalled at the issue, 124
// TFLOP/s at 8192^3 against 140 with the DMAs left out; two and four
// DMA-only waves gave 118 and 130.) The fragments of each 8-wide k slice
// (k-oct) are read before the MFMAs of the k-oct before issue, and the
// barrier that publishes k-tile s + 1 comes before the last k-oct's MFMAs of
// k-tile s. Rows and columns past M / N and k past K read as zeros (offsets
// past the buffer's records). The accumulation follows gemm_dma_kernel: MFMA
// chains of span k-tiles folded into a separate sum.
constexpr int kPipeBK = 32;
constexpr int kPipeStages = 4;
constexpr int kPipePanel = 128 * kPipeBK;   // floats per panel (16 KiB)
constexpr int kPipeStage = 2 * kPipePanel;  // floats per stage (32 KiB)
constexpr int kPipeThreads = 768;           // 8 compute waves + 4 movers

typedef float f32x2 __attribute__((ext_vector_type(2)));

__global__ __launch_bounds__(kPipeThreads, 1) void sgemm_pipe_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) float lds[kPipeStages * kPipeStage];
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  int lane = tid & 63;
  const int t = xcd_remap(blockIdx.x, gridDim.x);
  int bat, tm, tn;
  decode_tile<false>(g, t, bat, tm, tn);
  const int m0 = tm * 128, n0 = tn * 128;
  const int K = g.K, nk = g.nk;

  if (w >= 8) {
    // The movers: wave 8 + m (m < 4) moves blocks 8 (m & 1) .. + 7 of the A
    // panel (m < 2) or the B panel (m >= 2) of each stage, 1 KiB per block:
    // a 16-byte buffer load per lane into registers two k-tiles ahead, then
    // one 16-byte LDS store per lane (lane l of block b: bytes 16 l of the
    // block's KiB). Block b holds k rows 2 b, 2 b + 1; lane l holds k row
    // 2 b + l / 32, values 4 (l % 32) .. + 3. A lane's load is valid while
    // its columns are inside the matrix and kq <= K - k0 (kq: one past the
    // lane's k); others read zeros.
    const int m = w - 8;
    const bool onB = m >= 2;
    const float* X = static_cast<const float*>(onB ? g.B : g.A) + bat * (onB ? g.sB : g.sA);
    const int64_t ld = onB ? g.ldb : g.lda;
    const int r0 = onB ? n0 : m0, left = (onB ? g.N : g.M) - r0;
    uint32_t v[8];
    int kq[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int b = 8 * (m & 1) + u;
      const int krow = 2 * b + (lane >> 5);
      const int col = 4 * (lane & 31);
      v[u] = (uint32_t)((int64_t)krow * ld * 4 + 4 * col);
      kq[u] = col < left ? krow + 1 : 1 << 30;
    }
    auto gload = [&](int kt, i32x4(&r)[8]) __attribute__((always_inline)) {
      const int k0 = kt * kPipeBK, kl = K - k0;
      const float* base = X + (int64_t)k0 * ld + r0;
      const __amdgpu_buffer_rsrc_t rs = make_rsrc(base);
#pragma unroll
      for (int u = 0; u < 8; ++u)
        r[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, kq[u] <= kl ? v[u] : kOob, 0, 0);
    };
    auto lwrite = [&](int kt, const i32x4(&r)[8]) __attribute__((always_inline)) {
      float* dst = lds + (kt & (kPipeStages - 1)) * kPipeStage + (onB ? kPipePanel : 0) +
                   8 * (m & 1) * 256 + 4 * lane;
#pragma unroll
      for (int u = 0; u < 8; ++u) *reinterpret_cast<i32x4*>(dst + u * 256) = r[u];
    };
    if (nk == 0) return;
    // Barrier s publishes k-tile s: the movers' stores of it are done
    // (lgkmcnt(0)). Between barriers s and s + 1 a mover stores k-tile s + 1
    // (loaded two steps before) into the stage of k-tile s - 3 and loads
    // k-tile s + 3 into the registers it freed. Register set s & 1 holds
    // k-tiles s and s + 2.
    i32x4 ra[8], rb[8];
    gload(0, ra);
    if (nk > 1) gload(1, rb);
    lwrite(0, ra);
    if (nk > 2) gload(2, ra);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    auto step = [&](int s, i32x4(&r)[8]) __attribute__((always_inline)) {
      lwrite(s + 1, r);
      if (s + 3 < nk) gload(s + 3, r);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    int s = 0;
    for (; s + 2 < nk; s += 2) {
      step(s, rb);
      step(s + 1, ra);
    }
    if (s + 1 < nk) step(s, rb);
    return;
  }

  const int wm0 = 64 * (w & 1), wn0 = 32 * (w >> 1);
  const int kg = lane >> 4, li = lane & 15;
  // v_mfma_f32_16x16x4_f32: lane l holds k = l / 16 of A (row l % 16) and
  // of B (column l % 16); block p (0..3) of the wave's rows is rows
  // wm0 + 4 r + p, block q (0..1) of its columns is columns wn0 + 2 c + q,
  // so one 16-byte read gives a lane its A values of all four row blocks and
  // one 8-byte read its B values of both column blocks.
  struct Frag {
    float a[2][4], b[2][2];  // [k-step of the k-oct][block]
  };
  auto rd = [&](const float* st, int o, Frag& f) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(st + (8 * o + 4 * j + kg) * 128 + wm0 + 4 * li);
#pragma unroll
      for (int p = 0; p < 4; ++p) f.a[j][p] = v[p];
      const f32x2 u = *reinterpret_cast<const f32x2*>(st + kPipePanel + (8 * o + 4 * j + kg) * 128 + wn0 + 2 * li);
      f.b[j][0] = u[0];
      f.b[j][1] = u[1];
    }
  };
  f32x4 acc[4][2], sum[4][2];
#pragma unroll
  for (int p = 0; p < 4; ++p)
#pragma unroll
    for (int q = 0; q < 2; ++q) acc[p][q] = sum[p][q] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  auto mm = [&](const Frag& f) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int p = 0; p < 4; ++p)
#pragma unroll
        for (int q = 0; q < 2; ++q)
          acc[p][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.a[j][p], f.b[j][q], acc[p][q], 0, 0, 0);
  };

  const float* C = static_cast<const float*>(g.C) + (g.C ? bat * g.sC : 0);
  const int M = g.M, Nn = g.N;
  const float beta = g.beta;
  // lane l, register i of block (p, q): row 4 (4 (l / 16) + i) + p, column 2 (l % 16) + q
  auto row_of = [&](int p, int i) __attribute__((always_inline)) {
    return m0 + wm0 + 4 * (4 * kg + i) + p;
  };
  const int col = n0 + wn0 + 2 * li;
  float cv[4][4][2];
  auto load_c = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int mr = row_of(p, i);
        const bool ok = mr < M && beta != 0.0f && col < Nn;
        if (ok && g.vec2) {
          const f32x2 c = *reinterpret_cast<const f32x2*>(C + (int64_t)mr * g.ldc + col);
          cv[p][i][0] = c[0];
          cv[p][i][1] = c[1];
        } else {
          cv[p][i][0] = ok ? C[(int64_t)mr * g.ldc + col] : 0.0f;
          cv[p][i][1] = ok ? C[(int64_t)mr * g.ldc + col + 1] : 0.0f;
        }
      }
  };

  Frag f0, f1;
  // k-tile s: the reads of k-octs 1..3 go out before the MFMAs of the k-oct
  // before; then the barrier that publishes s + 1, the reads of k-oct 0 of
  // s + 1, and the last k-oct's MFMAs. The loop has no branch but the fold,
  // and the last k-tile is peeled, so the compiler's LDS wait counts stay
  // exact; sched_barrier keeps the reads ahead of the MFMAs. The last
  // k-tile loads C first (beta != 0).
  auto body = [&](int s, auto next) __attribute__((always_inline)) {
    constexpr bool NEXT = decltype(next)::value;
    if constexpr (!NEXT) load_c();
    const float* cur = lds + (s & (kPipeStages - 1)) * kPipeStage;
    rd(cur, 1, f1);
    __builtin_amdgcn_sched_barrier(0);
    mm(f0);
    __builtin_amdgcn_sched_barrier(0);
    rd(cur, 2, f0);
    __builtin_amdgcn_sched_barrier(0);
    mm(f1);
    __builtin_amdgcn_sched_barrier(0);
    rd(cur, 3, f1);
    __builtin_amdgcn_sched_barrier(0);
    mm(f0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NEXT) {
      asm volatile("s_barrier" ::: "memory");
      rd(lds + ((s + 1) & (kPipeStages - 1)) * kPipeStage, 0, f0);
    }
    __builtin_amdgcn_sched_barrier(0);
    mm(f1);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto fold = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        sum[p][q] += acc[p][q];
        acc[p][q] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
  };
  using Y = std::true_type;
  using N = std::false_type;
  if (nk > 0) {
    asm volatile("s_barrier" ::: "memory");  // k-tile 0 is in LDS
    rd(lds, 0, f0);
    int chain = g.span, s = 0;
    for (; s + 1 < nk; ++s) {
      body(s, Y{});
      if (--chain == 0) {
        fold();
        chain = g.span;
      }
    }
    body(s, N{});
    fold();
  } else {
    load_c();
  }
  // D = alpha sum + beta C
  asm volatile("" : "+v"(lane));
  float* D = static_cast<float*>(g.D) + bat * g.sD;
  const float alpha = g.alpha;
#pragma unroll
  for (int p = 0; p < 4; ++p)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int mr = row_of(p, i);
      if (mr >= M || col >= Nn) continue;
      const float v0 = __builtin_fmaf(beta, cv[p][i][0], alpha * sum[p][0][i]);
      const float v1 = __builtin_fmaf(beta, cv[p][i][1], alpha * sum[p][1][i]);
      if (g.vec2) {
        *reinterpret_cast<f32x2*>(D + (int64_t)mr * g.ldd + col) = f32x2{v0, v1};
      } else {
        D[(int64_t)mr * g.ldd + col] = v0;
        D[(int64_t)mr * g.ldd + col + 1] = v1;
      }
    }
}

template <typename T>
struct Cfg {
  static constexpr int BM = 128, BN = 128, WM = 64, WN = 64;
  // k-tile of gemm_kernel: 32 (two LDS stages). (16-byte aligned operands
  // run gemm_dma_kernel, with 128-byte k-tiles.)
  template <bool VEC>
  static constexpr int bk() {
    return 32;
  }
  static constexpr int NT = (BM / WM) * (BN / WN) * 64;
};

constexpr int kTileM = 128, kTileN = 128;
constexpr size_t kSkSlotBytes = (size_t)kTileM * kTileN * sizeof(float);

int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        v <= 0)
      v = 256;
    cus[dev] = v;
  }
  return cus[dev];
}

// Stream-K groups for this launch, or 0 for data-parallel: stream-K when the
// last round of one-tile workgroups would leave more than 10 % of the
// resident slots idle and the workspace holds two partial tiles per group.
static int choose_sk(GemmArgs& g, int occupancy, size_t ws_bytes) {
  g.dp_tiles = 0;
  if (g.ws == nullptr || g.nk < 8) return 0;
  const int64_t slots = (int64_t)device_cus() * (occupancy > 0 ? occupancy : 1);
  const int64_t rounds = (g.ntiles + slots - 1) / slots;
  const double eff = (double)g.ntiles / (double)(rounds * slots);
  // At most one tile per CU leaves one wave per SIMD (no second workgroup to
  // fill the MFMA pipe behind the barriers): split it too when each tile has
  // k-iterations enough (16) for the partial-tile traffic to pay (1024^2 x
  // 4096 fp32: 277 -> 83 us; 2048^3 with its 256 tiles: 175 -> 163 us;
  // 512^3: 51.5 -> 28.7 us, 768^3: 67 -> 35 us; below 16 no further gain).
  if (eff >= 0.9 || rounds > 8 || (g.ntiles <= device_cus() && g.nk < 16)) return 0;
  int64_t groups = slots;
  const int64_t dp = (g.ntiles / groups) * groups;  // whole rounds
  const int64_t tail = (int64_t)(g.ntiles - dp) * g.nk;
  // at least 4 k-iterations per group, and few enough groups per tile for
  // gemm_fixup_kernel's 64 contributors (a tile spans at most
  // ceil(nk / per) + 1 groups)
  const int64_t per = std::max<int64_t>(4, (g.nk + 62) / 63);
  if (tail / groups < per) groups = tail / per;
  if (groups < 1 || (size_t)groups * 2 * kSkSlotBytes > ws_bytes) return 0;
  if (dp > 0 && groups != slots) return 0;  // keep one workgroup per slot
  g.dp_tiles = (int)dp;
  return (int)groups;
}

// 128 x 64 tiles pay where 128 x 128 tiles fill at most one workgroup slot
// per CU (k-iterations >= 16): twice the tiles for the same grid, so a
// one-round grid of 128 x 128 tiles split by stream-K becomes whole 128 x 64
// tiles (no partials, no fixup launch), and a smaller one is split into half
// as many pieces per tile, with half the partial-tile bytes. Measured (fp32,
// microseconds, against the stream-K split of 128 x 128 tiles): 512^3 14.5 /
// 19.3, 1024^3 31.1 / 35.0, 1280^3 53.2 / 62.1, 512^2 x 8192 49.0 / 54.8,
// 2048^2 x 512 (102.6 / 74.8 TFLOP/s), 1900 x 2100 x 1000 (107.4 / 79.2
// TFLOP/s), C1 (2048^3 A^T B + 0.5 C) 148.5 / 151.9; 1536^2 x 2048 and
// 256^2 x 16384 unchanged. bf16 / fp16 (64-wide k-tiles): 2048^3 28.1 / 38.1,
// 1280^3 22.9 / 26.5, 1024^2 x 4096 24.6 / 27.9, 512^2 x 8192 25.5 / 29.7;
// at 1024^3 (16 k-tiles) 20.9 / 20.1, hence 20 k-tiles at least there.
static bool narrow_tiles_pay(const GemmArgs& g, int elem_bytes) {
  return g.ntiles <= device_cus() && g.nk >= (elem_bytes == 4 ? 16 : 20);
}

constexpr size_t kNarrowLdsPad = 16384;
static int choose_sk(GemmArgs& g, int occupancy, size_t ws_bytes);

template <typename T, bool AKC, bool BKC>
static int launch_narrow(GemmArgs g, size_t ws_bytes, hipStream_t s) {
  g.tiles_n = (g.N + 63) / 64;
  g.ntiles = g.tiles_m * g.tiles_n * g.batch;
  // 48 KiB of LDS and ~150 VGPRs would let three workgroups share a CU, so
  // a one-round grid of 2 per CU could land 3 + 1 on some CUs; 16 KiB of
  // unused dynamic LDS caps it at two (64 KiB each)
  g.sk_groups = choose_sk(g, 2, ws_bytes);  // (its slot check assumes 64 KiB partials: 32 here)
  const int grid = g.sk_groups ? g.sk_groups : g.ntiles;
  hipLaunchKernelGGL((gemm_dma_kernel<T, AKC, BKC, false, 64>), dim3(grid), dim3(256),
                     kNarrowLdsPad, s, g);
  int rc = check_launch("trnblas_hip_gemm");
  if (rc || !g.sk_groups) return rc;
  hipLaunchKernelGGL((gemm_fixup_kernel<T, 128, 64, false>),
                     dim3(g.ntiles - g.dp_tiles, 128 / 16), dim3(256), 0, s, g);
  return check_launch("trnblas_hip_gemm(fixup)");
}

// fp32 GEMM on sgemm_pipe_kernel (whole 128 x 128 tiles, one workgroup per
// CU); C and D take 2-element accesses when 8-byte aligned with even ld.
static int launch_pipe(GemmArgs g, hipStream_t s) {
  g.nk = (g.K + kPipeBK - 1) / kPipeBK;
  g.span = chain_length(g.K, 4) / kPipeBK;
  g.vec2 = g.ldd % 2 == 0 && (reinterpret_cast<uintptr_t>(g.D) & 7) == 0 &&
           (g.C == nullptr || (g.ldc % 2 == 0 && (reinterpret_cast<uintptr_t>(g.C) & 7) == 0));
  hipLaunchKernelGGL(sgemm_pipe_kernel, dim3(g.ntiles), dim3(kPipeThreads), 0, s, g);
  return check_launch("trnblas_hip_gemm");
}

// sgemm_pipe_kernel where it was measured faster than gemm_dma_kernel: both
// operands M/N-contiguous (A^T B, C1's layout) and one round of 128 x 128
// tiles that fills 90 % of the CUs or more, with 32 k-tiles or more. C1
// (2048^3 A^T B + 0.5 C) 0.1375 against 0.149 ms (0.139 with four compute
// waves of 64 x 64 on v_mfma_f32_32x32x2_f32, one per SIMD; 0.1397 with eight
// on 32x32x2). With K-contiguous operands gemm_dma_kernel's 16-byte
// fragment reads win (A B^T, A^T B^T at 2048^3: 0.159 / 0.161 against 0.135
// / 0.141 ms with the four-wave version), as they do for fewer tiles than
// CUs (gemm_dma_kernel splits them by stream-K) and at 8192^3 (133.7 against
// 138 TFLOP/s with the four-wave version: ~4800 cycles per 4096-cycle
// k-tile, timed in-kernel).
static bool pipe_pays(const GemmArgs& g) {
  const int cus = device_cus();
  return g.ntiles <= cus && 10 * g.ntiles >= 9 * cus &&
         (g.K + kPipeBK - 1) / kPipeBK >= 32;
}

// hgemm256_kernel where its 256 x 256 tiles fill every CU at least once, in
// rounds that keep 90 % of the CUs busy, and K spans 8 k-tiles or more
// (16-bit GEMM on aligned operands, 32-bit panel offsets for 256-row
// panels). Measured against gemm_dma_kernel (bf16, ms, NN / NT): 4096^2 x
// 1024 0.053 / 0.051 against 0.063 / 0.061, 4096^3 0.146 / 0.142 against
// 0.166 / 0.157, 8192^3 1.030 / 0.956 against 1.213 / 1.093, 16384 x 4096 x
// 2048 0.301 / 0.279 against 0.343 / 0.324; with a partial last round it
// loses (5120^3: 400 tiles, 0.328 / 0.299 against 0.317 / 0.301; 6144^3:
// 576 tiles, 0.541 / 0.530 against 0.531 / 0.485; 7168^3: 784 tiles).
static bool wide_tiles_pay(const GemmArgs& g) {
  const int64_t tiles = (int64_t)((g.M + 255) / 256) * ((g.N + 255) / 256) * g.batch;
  const int64_t cus = device_cus(), rounds = (tiles + cus - 1) / cus;
  return tiles >= cus && 10 * tiles >= 9 * rounds * cus && g.K >= 512;
}

template <typename T, bool AKC, bool BKC>
static int launch_wide(GemmArgs g, hipStream_t s) {
  g.tiles_m = (g.M + 255) / 256;
  g.tiles_n = (g.N + 255) / 256;
  g.ntiles = g.tiles_m * g.tiles_n * g.batch;
  g.nk = (g.K + 63) / 64;
  hipLaunchKernelGGL((hgemm256_kernel<T, AKC, BKC>), dim3(g.ntiles), dim3(512), 0, s, g);
  return check_launch("trnblas_hip_gemm");
}

template <typename T, bool AKC, bool BKC, bool VEC, bool SYRK>
static int launch_t(GemmArgs g, size_t ws_bytes, hipStream_t s) {
  using C = Cfg<T>;
  constexpr bool DMA = VEC;  // aligned operands: gemm_dma_kernel
  constexpr int BK = DMA ? 128 / (int)sizeof(T) : C::template bk<VEC>();
  g.nk = (g.K + BK - 1) / BK;
  g.span = chain_length(g.K, (int)sizeof(T)) / BK;  // even for the DMA kernel's k-tiles
  if constexpr (DMA && !SYRK && sizeof(T) == 4 && !AKC && !BKC) {
    if (pipe_pays(g)) return launch_pipe(g, s);
  }
  if constexpr (DMA && !SYRK && sizeof(T) == 2) {
    const int64_t span_a = (AKC ? 256 : 64) * g.lda * 2, span_b = (BKC ? 256 : 64) * g.ldb * 2;
    if (wide_tiles_pay(g) && span_a < (int64_t)kRecords - 64 && span_b < (int64_t)kRecords - 64)
      return launch_wide<T, AKC, BKC>(g, s);
  }
  if constexpr (DMA && !SYRK) {
    if (narrow_tiles_pay(g, (int)sizeof(T))) return launch_narrow<T, AKC, BKC>(g, ws_bytes, s);
  }
  void (*kern)(GemmArgs);
  if constexpr (DMA)
    kern = gemm_dma_kernel<T, AKC, BKC, SYRK>;
  else
    kern = gemm_kernel<T, C::BM, C::BN, BK, C::WM, C::WN, AKC, BKC, VEC, SYRK>;
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, C::NT, 0) != hipSuccess) occ = 1;
  g.sk_groups = choose_sk(g, occ, ws_bytes);
  const int grid = g.sk_groups ? g.sk_groups : g.ntiles;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(C::NT), 0, s, g);
  int rc = check_launch(SYRK ? "trnblas_hip_syrk" : "trnblas_hip_gemm");
  if (rc || !g.sk_groups) return rc;
  hipLaunchKernelGGL((gemm_fixup_kernel<T, C::BM, C::BN, SYRK>),
                     dim3(g.ntiles - g.dp_tiles, C::BM / 8), dim3(256), 0, s, g);
  return check_launch(SYRK ? "trnblas_hip_syrk(fixup)" : "trnblas_hip_gemm(fixup)");
}

template <typename T, bool SYRK>
static int launch_dtype(const GemmArgs& g, bool akc, bool bkc, bool vec, size_t ws_bytes,
                        hipStream_t s) {
#define TRNBLAS_L(a, b, v)                                 \
  if (akc == a && bkc == b && vec == v)                    \
    return launch_t<T, a, b, v, SYRK>(g, ws_bytes, s);
  TRNBLAS_L(true, true, true)
  TRNBLAS_L(true, true, false)
  TRNBLAS_L(false, false, true)
  TRNBLAS_L(false, false, false)
  if (!SYRK) {
    TRNBLAS_L(true, false, true)
    TRNBLAS_L(true, false, false)
    TRNBLAS_L(false, true, true)
    TRNBLAS_L(false, true, false)
  }
#undef TRNBLAS_L
  set_error("gemm: unsupported layout combination");
  return TRNBLAS_E_ARG;
}

static int elem_size(int dtype) { return dtype == TRNBLAS_F32 ? 4 : 2; }

// Largest k-tile of the launch configurations for `dtype` (panel-span check).
static int k_tile(int dtype) {
  return 128 / elem_size(dtype);  // gemm_dma_kernel's (gemm_kernel's is 32, no larger)
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <bool SYRK>
static int dispatch(int dtype, const GemmArgs& g, bool akc, bool bkc, size_t ws_bytes,
                    hipStream_t s) {
  const int ev = 16 / elem_size(dtype);
  // Buffer offsets inside one k-tile panel are 32-bit: the panel (tile rows
  // times the leading dimension) must stay below 2 GiB.
  const int64_t es = elem_size(dtype), bk = k_tile(dtype);
  const int64_t span_a = (akc ? 128 : bk) * g.lda * es, span_b = (bkc ? 128 : bk) * g.ldb * es;
  if (span_a >= (int64_t)kRecords - 64 || span_b >= (int64_t)kRecords - 64) {
    set_error("gemm: leading dimension too large for 32-bit panel offsets (lda %lld, ldb %lld)",
              (long long)g.lda, (long long)g.ldb);
    return TRNBLAS_E_ARG;
  }
  // VEC: 16-byte aligned groups that are wholly inside or outside the matrix
  // (the contiguous extent of each operand is a multiple of EV).
  const int a_ext = akc ? g.K : g.M, b_ext = bkc ? g.K : g.N;
  const bool vec = aligned16(g.A) && aligned16(g.B) && g.lda % ev == 0 && g.ldb % ev == 0 &&
                   g.sA % ev == 0 && g.sB % ev == 0 && a_ext % ev == 0 && b_ext % ev == 0;
  switch (dtype) {
    case TRNBLAS_F32:
      return launch_dtype<float, SYRK>(g, akc, bkc, vec, ws_bytes, s);
    case TRNBLAS_BF16:
      return launch_dtype<__bf16, SYRK>(g, akc, bkc, vec, ws_bytes, s);
    case TRNBLAS_F16:
      return launch_dtype<_Float16, SYRK>(g, akc, bkc, vec, ws_bytes, s);
  }
  set_error("unsupported dtype %d", dtype);
  return TRNBLAS_E_ARG;
}

// Operand packing (trnblas_hip_pack_k): X (R x K, element (r, k) at
// X + r sr + k sk) copied into row-major P (R x kp) with zero columns
// K .. kp - 1, one 64 x 64 block per workgroup, moved as raw bits (U: the
// element's size). A K-contiguous source (sk == 1) is copied along k; any
// other is read along r (coalesced for a transposed view, sr == 1) into an
// LDS block and written along k.
struct PackArgs {
  const void* X;
  void* P;
  int64_t R, K, kp, sr, sk, sxb, spb, tiles_r, tiles_k;
};

template <typename U>
__global__ __launch_bounds__(256) void pack_k_kernel(PackArgs p) {
  __shared__ U blk[64][65];
  int64_t b = blockIdx.x;
  const int64_t ik = b % p.tiles_k;
  b /= p.tiles_k;
  const int64_t ir = b % p.tiles_r;
  b /= p.tiles_r;
  const int64_t r0 = ir * 64, k0 = ik * 64;
  const U* X = static_cast<const U*>(p.X) + b * p.sxb;
  U* P = static_cast<U*>(p.P) + b * p.spb;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  if (p.sk == 1) {
#pragma unroll 4
    for (int i = 0; i < 16; ++i) {
      const int64_t r = r0 + ty + 4 * i, k = k0 + tx;
      if (r < p.R && k < p.kp) P[r * p.kp + k] = k < p.K ? X[r * p.sr + k] : U(0);
    }
    return;
  }
#pragma unroll 4
  for (int i = 0; i < 16; ++i) {
    const int64_t r = r0 + tx, k = k0 + ty + 4 * i;
    blk[ty + 4 * i][tx] = (r < p.R && k < p.K) ? X[r * p.sr + k * p.sk] : U(0);
  }
  __syncthreads();
#pragma unroll 4
  for (int i = 0; i < 16; ++i) {
    const int64_t r = r0 + ty + 4 * i, k = k0 + tx;
    if (r < p.R && k < p.kp) P[r * p.kp + k] = blk[tx][ty + 4 * i];
  }
}

}  // namespace trnblas

using namespace trnblas;

extern "C" size_t trnblas_hip_gemm_workspace(void) {
  // two fp32 partial tiles per resident workgroup slot (at most 2 per CU)
  return (size_t)device_cus() * 2 * 2 * kSkSlotBytes;
}

extern "C" int trnblas_hip_pack_k(int dtype, int64_t R, int64_t K, const void* X, int64_t sr,
                                  int64_t sk, int64_t sxb, void* P, int64_t kp, int64_t spb,
                                  int64_t batch, void* stream) {
  clear_error();
  TRNBLAS_CHECK_ARG(dtype == TRNBLAS_F32 || dtype == TRNBLAS_BF16 || dtype == TRNBLAS_F16,
                    "pack_k: dtype %d not supported", dtype);
  TRNBLAS_CHECK_ARG(R >= 0 && K >= 0 && batch >= 0 && kp >= K, "pack_k: bad sizes");
  TRNBLAS_CHECK_ARG(sr >= 0 && sk >= 0 && sxb >= 0 && spb >= 0, "pack_k: negative stride");
  if (R == 0 || kp == 0 || batch == 0) return TRNBLAS_OK;
  TRNBLAS_CHECK_ARG(batch == 1 || spb >= R * kp, "pack_k: batch stride of P below R * kp");
  TRNBLAS_CHECK_ARG(P != nullptr && (K == 0 || X != nullptr), "pack_k: NULL operand");
  PackArgs a{X, P, R, K, kp, sr, sk, sxb, spb, (R + 63) / 64, (kp + 63) / 64};
  const int64_t blocks = a.tiles_r * a.tiles_k * batch;
  TRNBLAS_CHECK_ARG(blocks < (1ll << 31), "pack_k: too many 64 x 64 blocks");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TRNBLAS_F32)
    hipLaunchKernelGGL(pack_k_kernel<uint32_t>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(pack_k_kernel<uint16_t>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  return check_launch("trnblas_hip_pack_k");
}

extern "C" int trnblas_hip_gemm(int dtype, int transA, int transB, int64_t M, int64_t N,
                                int64_t K, double alpha, const void* A, int64_t lda,
                                int64_t strideA, const void* B, int64_t ldb, int64_t strideB,
                                double beta, const void* C, int64_t ldc, int64_t strideC,
                                void* D, int64_t ldd, int64_t strideD, int64_t batch,
                                void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  TRNBLAS_CHECK_ARG(dtype == TRNBLAS_F32 || dtype == TRNBLAS_BF16 || dtype == TRNBLAS_F16,
                    "gemm: dtype %d not supported", dtype);
  TRNBLAS_CHECK_ARG(M >= 0 && N >= 0 && K >= 0 && batch >= 0, "gemm: negative size");
  TRNBLAS_CHECK_ARG(M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31),
                    "gemm: dimension >= 2^31");
  if (M == 0 || N == 0 || batch == 0) return TRNBLAS_OK;
  TRNBLAS_CHECK_ARG(D != nullptr, "gemm: D is NULL");
  TRNBLAS_CHECK_ARG(ldd >= N, "gemm: ldd %lld < N %lld", (long long)ldd, (long long)N);
  if (K > 0) {
    TRNBLAS_CHECK_ARG(A != nullptr && B != nullptr, "gemm: A or B is NULL");
    TRNBLAS_CHECK_ARG(lda >= (transA ? M : K), "gemm: lda too small");
    TRNBLAS_CHECK_ARG(ldb >= (transB ? K : N), "gemm: ldb too small");
  }
  if (beta != 0.0) {
    TRNBLAS_CHECK_ARG(C != nullptr, "gemm: beta != 0 needs C");
    TRNBLAS_CHECK_ARG(ldc >= N, "gemm: ldc too small");
  }
  GemmArgs g{};
  g.M = (int)M;
  g.N = (int)N;
  g.K = (int)K;
  g.alpha = (float)alpha;
  g.beta = (float)beta;
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
  g.uplo = 0;
  g.tiles_m = (int)((M + kTileM - 1) / kTileM);
  g.tiles_n = (int)((N + kTileN - 1) / kTileN);
  const int64_t ntiles = (int64_t)g.tiles_m * g.tiles_n * batch;
  TRNBLAS_CHECK_ARG(ntiles < (1ll << 31), "gemm: too many tiles");
  g.ntiles = (int)ntiles;
  g.nk = (int)((K + k_tile(dtype) - 1) / k_tile(dtype));
  g.ws = static_cast<float*>(workspace);
  // A is K-contiguous unless transposed; B is K-contiguous only when transposed.
  return dispatch<false>(dtype, g, !transA, transB != 0, workspace ? workspace_bytes : 0,
                         (hipStream_t)stream);
}

static int syrk_impl(int dtype, int uplo, int trans, int64_t N, int64_t K, double alpha,
                     const void* A, int64_t lda, double beta, const void* C, int64_t ldc, void* D,
                     int64_t ldd, const int32_t* tri, void* workspace, size_t workspace_bytes,
                     void* stream) {
  TRNBLAS_CHECK_ARG(dtype == TRNBLAS_F32 || dtype == TRNBLAS_BF16 || dtype == TRNBLAS_F16,
                    "syrk: dtype %d not supported", dtype);
  TRNBLAS_CHECK_ARG(N >= 0 && K >= 0, "syrk: negative size");
  TRNBLAS_CHECK_ARG(N < (1ll << 31) && K < (1ll << 31), "syrk: dimension >= 2^31");
  if (N == 0) return TRNBLAS_OK;
  TRNBLAS_CHECK_ARG(D != nullptr && ldd >= N, "syrk: bad D / ldd");
  if (K > 0) {
    TRNBLAS_CHECK_ARG(A != nullptr, "syrk: A is NULL");
    TRNBLAS_CHECK_ARG(lda >= (trans ? N : K), "syrk: lda too small");
  }
  if (beta != 0.0) TRNBLAS_CHECK_ARG(C != nullptr && ldc >= N, "syrk: bad C / ldc");
  GemmArgs g{};
  g.M = (int)N;
  g.N = (int)N;
  g.K = (int)K;
  g.alpha = (float)alpha;
  g.beta = (float)beta;
  g.A = A;
  g.lda = lda;
  g.sA = 0;
  g.B = A;  // B(k, n) = op(A)[n][k]
  g.ldb = lda;
  g.sB = 0;
  g.C = beta != 0.0 ? C : nullptr;
  g.ldc = ldc;
  g.sC = 0;
  g.D = D;
  g.ldd = ldd;
  g.sD = 0;
  g.batch = 1;
  g.uplo = uplo ? 1 : 0;
  g.tri = beta != 0.0 ? tri : nullptr;
  const size_t vb = 4 * (size_t)elem_size(dtype);
  g.vec4 = (ldd % 4 == 0) && ((uintptr_t)D % vb == 0) &&
           (beta == 0.0 || ((ldc % 4 == 0) && ((uintptr_t)C % vb == 0)));
  const int t = (int)((N + kTileM - 1) / kTileM);
  g.tiles_m = g.tiles_n = t;
  g.ntiles = (int)((int64_t)t * (t + 1) / 2);
  g.nk = (int)((K + k_tile(dtype) - 1) / k_tile(dtype));
  g.ws = static_cast<float*>(workspace);
  // trans == 0: op(A) = A (N x K, K-contiguous) and B(k, n) = A[n][k] (K-contiguous).
  // trans != 0: op(A) = A^T with A K x N (N-contiguous), B(k, n) = A[k][n].
  return dispatch<true>(dtype, g, !trans, !trans, workspace ? workspace_bytes : 0,
                        (hipStream_t)stream);
}

extern "C" int trnblas_hip_syrk(int dtype, int uplo, int trans, int64_t N, int64_t K,
                                double alpha, const void* A, int64_t lda, double beta,
                                const void* C, int64_t ldc, void* D, int64_t ldd,
                                void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return syrk_impl(dtype, uplo, trans, N, K, alpha, A, lda, beta, C, ldc, D, ldd, nullptr,
                   workspace, workspace_bytes, stream);
}

extern "C" int trnblas_hip_syrk_flagged(int dtype, int uplo, int trans, int64_t N, int64_t K,
                                        double alpha, const void* A, int64_t lda, double beta,
                                        const void* C, int64_t ldc, void* D, int64_t ldd,
                                        const int32_t* flags, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  clear_error();
  TRNBLAS_CHECK_ARG(flags != nullptr || beta == 0.0, "syrk_flagged: NULL flags");
  return syrk_impl(dtype, uplo, trans, N, K, alpha, A, lda, beta, C, ldc, D, ldd, flags,
                   workspace, workspace_bytes, stream);
}

// Which strict triangles of an n x n matrix hold a nonzero (NaN counts), for
// the SYRK triangle rule (trnblas/level3.py:305-329): flags[0] = upper,
// flags[1] = lower.
namespace trnblas {

// Sets the flags from a sample: wave w reads the 1024 columns around the
// diagonal of row {n/2, n/4, 3n/4, n-1}[w] (n = 0: zeros). A C with entries
// in both triangles is decided here, by two plain stores, so the waves of
// the full pass that follows find both flags set and stop at once (stores
// from thousands of waves to one address serialise in the L2).
template <typename T>
__global__ __launch_bounds__(256) void tri_sample_kernel(int n, const T* C, int64_t ldc,
                                                         int32_t* flags) {
  __shared__ int s_up[4], s_lo[4];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int up = 0, lo = 0;
  if (n > 0) {
    const int rows[4] = {n / 2, n / 4, (int)((3ll * n) / 4), n - 1};
    const int r = __builtin_amdgcn_readfirstlane(w == 0 ? rows[0] : w == 1 ? rows[1] : w == 2 ? rows[2] : rows[3]);
    const int cb = r - 512;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(C + (int64_t)r * ldc);
    T v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int c = cb + 64 * u + lane;
      const uint32_t off = (c >= 0 && c < n && c != r) ? (uint32_t)c * (uint32_t)sizeof(T) : kOob;
      if constexpr (sizeof(T) == 4) {
        v[u] = __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0));
      } else {
        v[u] = __builtin_bit_cast(T, (unsigned short)__builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0));
      }
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int c = cb + 64 * u + lane;
      const int nz = !(to_f32(v[u]) == 0.0f);
      up |= nz & (c > r);
      lo |= nz & (c < r);
    }
  }
  up = __any(up);
  lo = __any(lo);
  if (lane == 0) {
    s_up[w] = up;
    s_lo[w] = lo;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    flags[0] = s_up[0] | s_up[1] | s_up[2] | s_up[3];
    flags[1] = s_lo[0] | s_lo[1] | s_lo[2] | s_lo[3];
  }
}

// Work items are (row, 1024-column chunk) pairs, one per wave at a time
// over a grid of 2048 waves; a wave's lanes read 16 columns each (64 apart,
// all loads in flight at once; columns outside the row's strict triangles
// of interest read as zero through the buffer resource, with no access).
// Before each item a wave reads both flags (one 8-byte load at device scope)
// and skips the triangles already known to hold a nonzero; it stops once
// both are known, from the flags or from its own items. A flag is set by a
// plain store of 1 (every writer writes the same value: no read-modify-
// write, so thousands of waves finding entries at once do not serialise on
// atomics). A filled C is decided after about one item per wave; an empty
// triangle costs one pass over it.
template <typename T>
__global__ __launch_bounds__(256) void triangle_nonzero_kernel(int n, const T* C, int64_t ldc,
                                                               int32_t* flags) {
  const int lane = threadIdx.x & 63;
  const int nch = (n + 1023) >> 10;
  const int64_t items = (int64_t)n * nch;
  const int64_t stride = (int64_t)gridDim.x * 4;
  int64_t* both = reinterpret_cast<int64_t*>(flags);
  int fu = 0, fl = 0;  // known by this wave
  for (int64_t q = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); q < items; q += stride) {
    const int64_t f = __hip_atomic_load(both, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    fu |= (int)(f & 0xffffffff) != 0;
    fl |= (int)(f >> 32) != 0;
    fu = __builtin_amdgcn_readfirstlane(fu);
    fl = __builtin_amdgcn_readfirstlane(fl);
    if (fu && fl) break;
    const int r = (int)(q / nch);
    const int c0 = (int)(q - (int64_t)r * nch) * 1024;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(C + (int64_t)r * ldc);
    T v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int c = c0 + 64 * u + lane;
      const bool want = c < n && ((c > r && !fu) || (c < r && !fl));
      const uint32_t off = want ? (uint32_t)c * (uint32_t)sizeof(T) : kOob;
      if constexpr (sizeof(T) == 4) {
        v[u] = __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0));
      } else {
        v[u] = __builtin_bit_cast(T, (unsigned short)__builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0));
      }
    }
    int up = 0, lo = 0;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int c = c0 + 64 * u + lane;
      const int nz = !(to_f32(v[u]) == 0.0f);  // NaN counts as nonzero
      up |= nz & (c > r);
      lo |= nz & (c < r);
    }
    up = __any(up);
    lo = __any(lo);
    if (lane == 0) {
      if (up && !fu) __hip_atomic_store(&flags[0], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (lo && !fl) __hip_atomic_store(&flags[1], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    fu |= up;
    fl |= lo;
  }
}

}  // namespace trnblas

template <typename T>
static void launch_triangle(int64_t n, const void* C, int64_t ldc, int32_t* flags, hipStream_t s) {
  const T* c = static_cast<const T*>(C);
  hipLaunchKernelGGL(tri_sample_kernel<T>, dim3(1), dim3(256), 0, s, (int)n, c, ldc, flags);
  if (n < 2) return;
  const int64_t items = n * ((n + 1023) / 1024);
  const int64_t blocks = std::min<int64_t>((items + 3) / 4, 512);
  hipLaunchKernelGGL(triangle_nonzero_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, s, (int)n,
                     c, ldc, flags);
}

extern "C" int trnblas_hip_triangle_nonzero(int dtype, int64_t n, const void* C, int64_t ldc,
                                            int32_t* flags, void* stream) {
  clear_error();
  hipStream_t s = (hipStream_t)stream;
  TRNBLAS_CHECK_ARG(n >= 0 && n < (1 << 30), "triangle_nonzero: bad n");
  TRNBLAS_CHECK_ARG(flags != nullptr && (uintptr_t)flags % 8 == 0,
                    "triangle_nonzero: flags NULL or not 8-byte aligned");
  if (n > 0) TRNBLAS_CHECK_ARG(C != nullptr && ldc >= n, "triangle_nonzero: bad C / ldc");
  switch (dtype) {
    case TRNBLAS_F32:
      launch_triangle<float>(n, C, ldc, flags, s);
      break;
    case TRNBLAS_BF16:
      launch_triangle<__bf16>(n, C, ldc, flags, s);
      break;
    case TRNBLAS_F16:
      launch_triangle<_Float16>(n, C, ldc, flags, s);
      break;
    default:
      set_error("triangle_nonzero: dtype %d not supported", dtype);
      return TRNBLAS_E_ARG;
  }
  return check_launch("triangle_nonzero");
}
