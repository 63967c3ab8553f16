/*
 * trnblas_hip.h — C ABI of the MI355X (gfx950) Level-3 op library.
 *
 * One function per kernel family. Every pointer argument is a device pointer
 * unless stated otherwise; every function is asynchronous on `stream` (a
 * hipStream_t passed as void*; NULL = the null stream), allocates nothing and
 * returns 0 on success or a negative TRNBLAS_E_* code. The message of the
 * last failure on the calling thread is returned by trnblas_hip_last_error().
 * Outputs are caller-allocated; inputs are never written.
 *
 * Global state. The library keeps an immutable kernel table, a thread-local
 * error message, and two pieces of mutable per-device state:
 *  - trnblas_hip_metric_inv_half creates, on its first call on a device,
 *    two side streams and their events for that device and keeps them until
 *    the process ends; calls on one device share them and are serialised on
 *    the host by a mutex (two threads calling it on one device do not
 *    overlap);
 *  - trnblas_hip_pair_energy_noalloc keeps its partial sums in one static
 *    device array per GPU: calls that overlap on one GPU (two streams, or
 *    two threads) race on it and must be serialised by the caller.
 * Every other function is reentrant: it touches only its arguments.
 *
 * The reference (trnsci/trnblas 0.13.0) has no native code: its device path is
 * the NKI kernels behind the `torch.ops.trnblas.*` custom ops registered in
 * trnblas/nki/_native.py:49-259 and called from trnblas/nki/dispatch.py
 * (`_call_kernel` :2168-2184, `_launch` :2187-2194). Each entry point below
 * names the reference interface it replaces.
 */
#ifndef TRNBLAS_HIP_H
#define TRNBLAS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types */
#define TRNBLAS_F32 0
#define TRNBLAS_BF16 1
#define TRNBLAS_F16 2
#define TRNBLAS_F64 3 /* trnblas_hip_tri_inv_blocks only (fp64 work has its own entry points) */

/* error codes */
#define TRNBLAS_OK 0
#define TRNBLAS_E_ARG (-1)       /* invalid argument (shape, stride, dtype, flag) */
#define TRNBLAS_E_LAUNCH (-2)    /* a kernel launch failed (hipGetLastError) */
#define TRNBLAS_E_NONFINITE (-3) /* reserved: non-finite data where the op cannot represent it */
#define TRNBLAS_E_WORKSPACE (-4) /* workspace too small */

/* Version of this ABI (bumped on any signature change). */
int trnblas_hip_abi_version(void);

/* Message of the last failure on the calling thread ("" if none). */
const char* trnblas_hip_last_error(void);

/*
 * GEMM, strided-batched:  D[b] = alpha * op(A[b]) * op(B[b]) + beta * C[b]
 *
 * Replaces the GEMM kernel family behind torch.ops.trnblas.gemm_{64,128}_128_
 * {128,256,512}, gemm_ragged, gemm_lnc and gemm_lnc_tn
 * (trnblas/nki/_native.py:49-74; kernels trnblas/nki/dispatch.py:3324-3760),
 * plus the `_scale_add` epilogue of trnblas/level3.py:42-66, which is fused
 * here, and the per-slice launch loop of `nki_batched_gemm`
 * (dispatch.py:1384-1427), which is one launch here (grid over the batch).
 *
 * dtype: TRNBLAS_F32 (fp32 MFMA) or TRNBLAS_BF16 / TRNBLAS_F16 (16-bit MFMA,
 * fp32 accumulate). A, B, C, D all have that element type.
 * op(A) is M x K: A is row-major M x K (lda >= K) when transA == 0, row-major
 * K x M (lda >= M) when transA != 0; likewise op(B) is K x N. C and D are
 * row-major M x N with leading dimensions ldc, ldd. C may be NULL when
 * beta == 0 (then C is not read, as in BLAS). Any M, N, K >= 0 (ragged edges
 * are handled in the kernel; K == 0 gives D = beta * C). Batch strides are in
 * elements; a stride of 0 broadcasts that operand over the batch. D must not
 * overlap A or B; it may be C itself (an in-place update: each element of C
 * is read and written by the same thread), but must not partly overlap C.
 */
int trnblas_hip_gemm(int dtype, int transA, int transB, int64_t M, int64_t N, int64_t K,
                     double alpha, const void* A, int64_t lda, int64_t strideA,
                     const void* B, int64_t ldb, int64_t strideB, double beta,
                     const void* C, int64_t ldc, int64_t strideC, void* D, int64_t ldd,
                     int64_t strideD, int64_t batch, void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * Workspace that lets trnblas_hip_gemm / trnblas_hip_syrk balance a launch
 * whose tiles do not fill the GPU evenly (stream-K: the k-iterations of all
 * tiles are split evenly over the resident workgroups; split tiles are summed
 * by a second, deterministic kernel). Bytes for the current device; with a
 * NULL or smaller workspace the calls run one tile per workgroup. Calls on
 * one stream may share a workspace; calls that can overlap (other streams)
 * need one each.
 */
size_t trnblas_hip_gemm_workspace(void);

/*
 * Operand packing:  P[b] (R x kp, row-major) = X[b] (R x K) with zero
 * columns K .. kp - 1.
 *
 * Replaces the zero padding of GEMM operands to the kernel's tile multiples,
 * `_pad_gemm_operands` (trnblas/nki/dispatch.py:2344-2368). Here it serves
 * operands that trnblas_hip_gemm / trnblas_hip_syrk cannot read by LDS DMA
 * in place: packed K-contiguous with kp a multiple of 16 bytes, they take the
 * DMA kernel (zero products add nothing to any sum).
 * Element (r, k) of X[b] is at X + b * sxb + r * sr + k * sk (strides in
 * elements, >= 0; sk == 1 is copied along k, any other layout through an LDS
 * transpose). P[b] starts at P + b * spb (spb >= R * kp when batch > 1).
 * dtype: TRNBLAS_F32, TRNBLAS_BF16 or TRNBLAS_F16 (bits are copied as they are).
 * P must not overlap X. Asynchronous on `stream`.
 */
int trnblas_hip_pack_k(int dtype, int64_t R, int64_t K, const void* X, int64_t sr, int64_t sk,
                       int64_t sxb, void* P, int64_t kp, int64_t spb, int64_t batch,
                       void* stream);

/*
 * SYRK:  D = alpha * op(A) * op(A)^T + beta * sym_uplo(C), returned full.
 *
 * Replaces torch.ops.trnblas.syrk (trnblas/nki/_native.py:124-132; kernel
 * dispatch.py:4493-4544) together with the host symmetrisation
 * `_symmetrize` (dispatch.py:3167-3199) and the triangle rule
 * `_sym_from_triangle` of trnblas/level3.py:298-302. Only the lower triangle
 * of op(A) op(A)^T is computed (n(n+1)k flops); each value is written to
 * both D[i][j] and D[j][i], so D is exactly symmetric.
 * op(A) is N x K: A row-major N x K (trans == 0) or K x N (trans != 0).
 * uplo: 0 = the lower triangle of C is referenced, 1 = the upper. C may be
 * NULL when beta == 0. dtype and workspace as in trnblas_hip_gemm.
 */
int trnblas_hip_syrk(int dtype, int uplo, int trans, int64_t N, int64_t K, double alpha,
                     const void* A, int64_t lda, double beta, const void* C, int64_t ldc,
                     void* D, int64_t ldd, void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * SYRK as trnblas_hip_syrk, with the referenced triangle of C chosen on the
 * device from `flags` (device int32[2] as written by
 * trnblas_hip_triangle_nonzero on the same stream): the `uplo` triangle, or
 * the other one when only that one holds off-diagonal entries. Replaces
 * `_resolve_syrk_uplo` + syrk of trnblas/level3.py:285-287, :305-329 without
 * a host round trip between the triangle check and the product (the host
 * reads the flags afterwards, for the DeprecationWarning). flags may be NULL
 * only when beta == 0.
 */
int trnblas_hip_syrk_flagged(int dtype, int uplo, int trans, int64_t N, int64_t K, double alpha,
                             const void* A, int64_t lda, double beta, const void* C, int64_t ldc,
                             void* D, int64_t ldd, const int32_t* flags, void* workspace,
                             size_t workspace_bytes, void* stream);

/*
 * Which strict triangles of the n x n matrix C hold a nonzero entry (NaN
 * counts as nonzero): flags[0] = strictly upper, flags[1] = strictly lower
 * (device int32[2], 8-byte aligned, written by this call). The triangle rule of SYRK's C
 * argument, trnblas/level3.py:305-329 (`_resolve_syrk_uplo`), as one pass
 * over C on the device. dtype as in trnblas_hip_gemm.
 */
int trnblas_hip_triangle_nonzero(int dtype, int64_t n, const void* C, int64_t ldc,
                                 int32_t* flags, void* stream);

/*
 * DF-MP2 pair energies, fused (T never leaves the chip).
 *
 * For each pair p = (i, j):
 *   e_p = sum_{a,b < nvir} T_ab (2 T_ab - T_ba) / (eps_i[i] + eps_j[j] - eps_vir[a] - eps_vir[b]),
 *   T = X_i X_j^T,  X_i = Bi + i*ldi_occ,  X_j = Bj + j*ldj_occ,
 * each X an nvir x naux fp32 matrix with rows ld_vir elements apart (naux
 * contiguous).
 *
 * Pair set: when pair_i == NULL, every unordered pair i <= j of
 * [0, nocc) with weight 1 (i == j) or 2 (i != j) — the symmetric walk of the
 * reference (e_ij = e_ji); this needs Bi == Bj, eps_i == eps_j, ldi_occ ==
 * ldj_occ. Otherwise the npairs pairs (pair_i[p], pair_j[p]) (device int32
 * arrays) with weights pair_w[p] (device double array, NULL = all 1).
 *
 * out_pairs (device double[npairs], may be NULL) receives the unweighted e_p;
 * out_total (device double[1], may be NULL) receives sum_p w_p e_p. Both are
 * deterministic (fixed reduction order). workspace must hold
 * trnblas_hip_pair_energy_workspace(nvir, npairs) bytes (npairs =
 * nocc (nocc + 1) / 2 in the implicit mode).
 *
 * Replaces torch.ops.trnblas.pair_energy_sym and the per-row launch loop of
 * `_nki_pair_energy_sym_impl` (trnblas/nki/_native.py:221-239,
 * dispatch.py:2768-2795, kernel :4899-5001), and is the engine of the
 * batched_pair / j_batched / fused_gemm_energy op surface
 * (_native.py:168-218).
 */
size_t trnblas_hip_pair_energy_workspace(int64_t nvir, int64_t npairs);
int trnblas_hip_pair_energy(int64_t nvir, int64_t naux, const float* Bi, int64_t ldi_occ,
                            const float* Bj, int64_t ldj_occ, int64_t ld_vir,
                            const float* eps_i, const float* eps_j, const float* eps_vir,
                            int64_t nocc, int64_t npairs, const int32_t* pair_i,
                            const int32_t* pair_j, const double* pair_w, double* out_pairs,
                            double* out_total, void* workspace, size_t workspace_bytes,
                            void* stream);

/*
 * DF-MP2 pair energies as trnblas_hip_pair_energy — same pair set, weights,
 * outputs and determinism — with every fp32 product formed on bf16 MFMA
 * (v_mfma_f32_16x16x32_bf16, fp32 accumulation) from the three bf16 pieces
 * of each operand:
 *   x = hi + mid + lo exactly (hi = rn_bf16(x), mid = rn_bf16(x - hi),
 *   lo = x - hi - mid), and
 *   x y ~= hi_x hi_y + hi_x mid_y + mid_x hi_y + hi_x lo_y + mid_x mid_y + lo_x hi_y,
 * the three dropped products being below 2^-23 |x y|. Each T entry then
 * carries fp32 accumulation error plus that term (fp32-class accuracy) at
 * 6/16 of the MFMA time of an fp32 product.
 *
 * A first pass writes the pieces of Bi and Bj into the workspace (three bf16
 * planes per operand), so the call takes the row counts of the operands:
 * ni rows of Bi (>= every pair_i, >= nocc in the implicit mode) and nj rows
 * of Bj (>= every pair_j), or nj == 0 when Bj == Bi with ldj_occ == ldi_occ
 * (one set of planes serves both; required in the implicit mode); a pair
 * index beyond these rows gives a NaN energy for its pair. workspace
 * must hold trnblas_hip_pair_energy_bf16x6_workspace(nvir, naux, npairs, ni,
 * nj) bytes.
 *
 * Replaces the same reference interface as trnblas_hip_pair_energy
 * (torch.ops.trnblas.pair_energy_sym, trnblas/nki/_native.py:221-239).
 */
size_t trnblas_hip_pair_energy_bf16x6_workspace(int64_t nvir, int64_t naux, int64_t npairs,
                                                int64_t ni, int64_t nj);
int trnblas_hip_pair_energy_bf16x6(int64_t nvir, int64_t naux, const float* Bi, int64_t ni,
                                   int64_t ldi_occ, const float* Bj, int64_t nj,
                                   int64_t ldj_occ, int64_t ld_vir, const float* eps_i,
                                   const float* eps_j, const float* eps_vir, int64_t nocc,
                                   int64_t npairs, const int32_t* pair_i, const int32_t* pair_j,
                                   const double* pair_w, double* out_pairs, double* out_total,
                                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * DF-MP2 pair energies as trnblas_hip_pair_energy_bf16x6 (same arguments,
 * pair set, weights, outputs, determinism and row-count rules) with every
 * fp32 product formed on f16 MFMA (v_mfma_f32_16x16x32_f16, fp32
 * accumulation) from two fp16 pieces of each operand. Each row (o, a) is
 * first scaled by 2^e(o, a) so its largest magnitude lies in [2^14, 2^15);
 * then xs = x 2^e = hi + lo + r (hi = rn_f16(xs), lo = rn_f16(xs - hi),
 * |r| <= 2^-22 |xs| + 2^-25) and
 *   xs ys ~= hi_x hi_y + hi_x lo_y + lo_x hi_y,
 * dropping lo_x lo_y (<= 2^-22 |xs ys|); T_ab = sum 2^-(e(i, a) + e(j, b)) is
 * formed in fp64. Each T entry carries fp32 accumulation error plus about
 * 3 2^-22 relative per product (fp32-class accuracy) at 3/16 of the MFMA time
 * of an fp32 product. workspace must hold
 * trnblas_hip_pair_energy_fp16x3_workspace(nvir, naux, npairs, ni, nj) bytes
 * (the pieces plus one int32 exponent per row).
 *
 * Replaces the same reference interface as trnblas_hip_pair_energy
 * (torch.ops.trnblas.pair_energy_sym, trnblas/nki/_native.py:221-239).
 */
size_t trnblas_hip_pair_energy_fp16x3_workspace(int64_t nvir, int64_t naux, int64_t npairs,
                                                int64_t ni, int64_t nj);
int trnblas_hip_pair_energy_fp16x3(int64_t nvir, int64_t naux, const float* Bi, int64_t ni,
                                   int64_t ldi_occ, const float* Bj, int64_t nj,
                                   int64_t ldj_occ, int64_t ld_vir, const float* eps_i,
                                   const float* eps_j, const float* eps_vir, int64_t nocc,
                                   int64_t npairs, const int32_t* pair_i, const int32_t* pair_j,
                                   const double* pair_w, double* out_pairs, double* out_total,
                                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * trnblas_hip_pair_energy without a workspace argument: same arguments
 * (minus workspace), pair set, weights, outputs, kernels and bits. It
 * allocates nothing: the fp64 partials live in a static device array of
 * trnblas_hip_pair_energy_noalloc_max_bytes() bytes (16 MiB) per GPU, held
 * until the process ends, so npairs * (nb (nb + 1) / 2 + 1) * 8 bytes, with
 * nb = ceil(nvir / 96), must fit (C3: 1.1 MB; nocc 256 / nvir 768: 9.7 MB);
 * larger calls return TRNBLAS_E_WORKSPACE. Nothing needs clearing between
 * calls (every partial is written before it is read), but calls that overlap
 * on one GPU share the array and race.
 *
 * No counterpart in the reference: this is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).
 */
size_t trnblas_hip_pair_energy_noalloc_max_bytes(void);
int trnblas_hip_pair_energy_noalloc(int64_t nvir, int64_t naux, const float* Bi, int64_t ldi_occ,
                                    const float* Bj, int64_t ldj_occ, int64_t ld_vir,
                                    const float* eps_i, const float* eps_j,
                                    const float* eps_vir, int64_t nocc, int64_t npairs,
                                    const int32_t* pair_i, const int32_t* pair_j,
                                    const double* pair_w, double* out_pairs, double* out_total,
                                    void* stream);

/*
 * MP2 energy of a precomputed amplitude block (no GEMM), HBM-bound.
 *
 * T[i][j][a][b] = T_flat[(i*nvir + a) * ldt + j*nvir + b] for i < ic,
 * j < nocc. out_pairs (device double[ic*nocc], row-major (i, j)) receives
 *   sum_ab T_ijab (2 T_ijab - T_ijba) / (eo_chunk[i] + eo_full[j] - ev[a] - ev[b]).
 * Replaces torch.ops.trnblas.mp2_energy (trnblas/nki/_native.py:135-158,
 * kernel dispatch.py:4356-4491).
 */
int trnblas_hip_mp2_energy(int64_t ic, int64_t nocc, int64_t nvir, const float* T_flat,
                           int64_t ldt, const float* eps_occ_chunk, const float* eps_occ_full,
                           const float* eps_vir, double* out_pairs, void* stream);

/*
 * Ozaki split of a finite fp64 matrix into `slices` int8 digits (per row or
 * per column), as trnblas/ozaki.py:123-219 `split` (digit_0 = rint(x 2^(6-e)),
 * digit_s = rint(2^7 * remainder), |digit| <= 64, e = frexp exponent of the
 * row / column maximum), with native fp64 arithmetic. Replaces
 * torch.ops.trnblas.ozaki_emax / ozaki_emax_col / ozaki_split /
 * ozaki_split_col (trnblas/nki/_native.py:77-121; kernels
 * dispatch.py:3994-4354), which derive the same digits from raw bits
 * because Trainium has no fp64.
 *
 * X: R x C fp64, element (r, c) at X[r*ldx + c].
 * per_row != 0: one exponent per row (the A operand); digits are written as
 *   digits[s*ld_slice + r*ld_digit + c] (K = C contiguous).
 * per_row == 0: one exponent per column (the B operand); digits are written
 *   transposed, digits[s*ld_slice + c*ld_digit + r] (K = R contiguous).
 * per_row | 2: the interleaved layout of the fast GEMM (mode 2 of
 *   trnblas_hip_ozaki_gemm): digit (s, row, kk) of the digit row `row` (r or
 *   c as above) and K index kk at
 *   digits[row*ld_digit + (kk/32)*32*slices + s*32 + kk%32], i.e. the slices
 *   of each 32-wide K chunk side by side; ld_digit >= round_up(K, 32) *
 *   slices and a multiple of 16, digits 16-byte aligned; ld_slice unused.
 * The digit buffer must be zero beyond the matrix (the caller pads to the
 * kernel's tile; entries beyond R x C are not written). exps (device int32,
 * R or C entries) receives e. scratch: device int32[2] (scale-mode flag and
 * non-finite flag). Returns TRNBLAS_OK; a non-finite X is reported through
 * scratch[1] != 0 (checked by the caller after synchronising), the digits
 * are then undefined.
 */
int trnblas_hip_ozaki_split(int per_row, int64_t R, int64_t C, const double* X, int64_t ldx,
                            int slices, int8_t* digits, int64_t ld_digit, int64_t ld_slice,
                            int32_t* exps, int32_t* scratch, void* stream);

/*
 * Ozaki slice GEMM with fused recombination:
 *   C[m][n] = sum over K blocks of (hi + lo) * 2^(eA[m] + eB[n] + off),
 * where (hi, lo) is the fp32 TwoSum chain of trnblas/ozaki.py:358-415
 * (`schedule`, `_two_sum32`, `reference_from_digits`) over exact int32
 * group sums of int8 digit products (int8 MFMA). With mode 0 the result
 * equals `ozaki.reference_gemm` bit for bit (same groups, same TwoSum order,
 * same combine, ozaki.py:418-455). Mode 1 (fast) accumulates each diagonal
 * of slice pairs exactly in int32 and recombines in fp64 (error within the
 * same bound, not bitwise). Mode 2 is mode 1 on interleaved digits
 * (trnblas_hip_ozaki_split with per_row | 2; any slice count, lda / ldb
 * the digit row strides >= slices * Kp, lda_slice / ldb_slice unused): the
 * same result bit for bit, each row's k-step one contiguous load.
 *
 * dA: digits (slices, >= M, Kp) with dA[s*lda_slice + m*lda + k];
 * dB: digits (slices, >= N, Kp) with dB[s*ldb_slice + n*ldb + k]; both K
 * contiguous, zero beyond M / N / K. Kp is K padded to 128. kb: K block
 * (a multiple of 128, `ozaki.plan`; the last block holds what remains of
 * Kp), blocks summed in fp64 in order. C element (m, n) at C[m*ldc_m + n*ldc_n] (ldc_m, ldc_n
 * let the caller write C^T for the narrow-N swap of `ozaki.run`).
 * Replaces torch.ops.trnblas.ozaki_gemm (trnblas/nki/_native.py:77-85;
 * kernel dispatch.py:3887-3918) and the host `combine`.
 */
int trnblas_hip_ozaki_gemm(int mode, int slices, int64_t M, int64_t N, int64_t Kp,
                           int64_t kb, const int8_t* dA, int64_t lda, int64_t lda_slice,
                           const int8_t* dB, int64_t ldb, int64_t ldb_slice, const int32_t* eA,
                           const int32_t* eB, double* C, int64_t ldc_m, int64_t ldc_n,
                           void* stream);

/*
 * Raw (hi, lo) output of the Ozaki slice GEMM, mode 0, for one K block:
 * hilo[0][m][n] = hi, hilo[1][m][n] = lo (fp32, row-major M x N each,
 * leading dimension ldh). The `torch.ops.trnblas.ozaki_gemm` surface
 * (trnblas/nki/_native.py:77-85: (k, Kp, Mp) x (k, Kp, N) -> (2, Mp, N)).
 */
int trnblas_hip_ozaki_hilo(int slices, int64_t M, int64_t N, int64_t Kp, const int8_t* dA,
                           int64_t lda, int64_t lda_slice, const int8_t* dB, int64_t ldb,
                           int64_t ldb_slice, float* hilo, int64_t ldh, void* stream);

/*
 * gemm_fp64 by Ozaki scheme II (the "crt" mode of trnblas_amd.gemm_fp64):
 * the same precision knob as the digit split of `nki_gemm_fp64`
 * (trnblas/nki/dispatch.py:958-980, trnblas/ozaki.py:123-455), which these
 * four calls replace in that mode. Each operand is represented as one
 * integer per element, A'_il = rint(a_il 2^(p - eA_i)) and B'_lj =
 * rint(b_lj 2^(p - eB_j)) with p = 7 slices - 1 (the precision of `slices`
 * 7-bit digits) and eA_i / eB_j the frexp exponents of the row / column
 * maxima; A'B' is computed exactly from int8 GEMMs modulo pairwise coprime
 * moduli m_t <= 256 (256, 255, 253, 251, 247, 241, ...; 32 at most) and the
 * Chinese remainder theorem; C = A'B' 2^(eA_i + eB_j - 2p). The error is
 * the operand rounding alone, within the `slices`-digit truncation bound.
 *
 * trnblas_hip_crt_moduli: the number of moduli for `slices` and inner
 * dimension K (the fewest whose product M >= 2 K 2^(2p) + 2), or a negative
 * code.
 *
 * trnblas_hip_crt_split: exponents and balanced int8 residues (r in
 * [-m/2, m/2)) of X (R x C fp64, row-major, ldx) for the first nmod moduli.
 * per_row = 1 (A): one exponent per row, operand row r = row r of X (K = C);
 * per_row = 0 (B): one exponent per column, operand row c = column c of X
 * (K = R). The residues are blocked: residue (t, row r, k) at
 * res[t * ld_plane + ((r / 16) (kp / 64) + k / 64) 1024 + (r % 16) 64 + k % 64]
 * (16 rows x 64 bytes per contiguous KiB; ld_plane >= ceil(rows / 16) 16 kp),
 * K runs to kp (a multiple of 64, >= the K extent), padded with zero
 * residues. exps: int32 per row / column; flags: int32[2], flags[1] = 1
 * when X holds inf / nan (the residues are then undefined).
 *
 * trnblas_hip_crt_gemm: for t < nmod, P_t = RA_t RB_t^T mod m_t as balanced
 * int8 residues, RA (M operand rows) and RB (N operand rows) in the blocked
 * layout of trnblas_hip_crt_split with K extent Kp (16-byte aligned). P is
 * 32 x 32 blocked: plane t at P + t * p_plane (p_plane >= ceil(M / 32)
 * ceil(N / 32) 1024 bytes), block (bm, bn) at 1024 (bm ceil(N / 32) + bn),
 * where byte 16 l + e is element (32 bm + 8 (e / 4) + 4 (l / 32) + e % 4,
 * 32 bn + l % 32) (the layout of the MFMA accumulators).
 *
 * trnblas_hip_crt_combine: C[m * ldc_m + n * ldc_n] (fp64) from the residue
 * planes and exponents: Garner's mixed-radix digits, the value by fp64 fma
 * Horner over digit pairs, times 2^(eA_m + eB_n - 2p).
 */
int trnblas_hip_crt_moduli(int slices, int64_t K);
int trnblas_hip_crt_split(int per_row, int64_t R, int64_t C, const double* X, int64_t ldx,
                          int slices, int nmod, int64_t kp, int8_t* res, int64_t ld_plane,
                          int32_t* exps, int32_t* flags, void* stream);
int trnblas_hip_crt_gemm(int nmod, int64_t M, int64_t N, int64_t Kp, const int8_t* RA,
                         int64_t lda_plane, const int8_t* RB, int64_t ldb_plane, int8_t* P,
                         int64_t p_plane, void* stream);
int trnblas_hip_crt_combine(int slices, int nmod, int64_t M, int64_t N, const int8_t* P,
                            int64_t p_plane, const int32_t* eA, const int32_t* eB, double* C,
                            int64_t ldc_m, int64_t ldc_n, void* stream);

/*
 * One diagonal block of the blocked Cholesky of metric_inv_half, fp64:
 * A (nb x nb, 0 <= nb <= 128, row-major, leading dimension lda; only its lower
 * triangle is read) is overwritten in its lower triangle by the Cholesky
 * factor L (A = L L^T) and Linv (nb x nb, ldl) receives L^-1, lower
 * triangular with zeros above. A pivot that is not positive (A not positive
 * definite, or NaN) sets *info = offset + its 1-based column unless *info is
 * already nonzero (the host zeroes info once and checks it after the last
 * block); L and Linv are then garbage. Device pointers, asynchronous on
 * `stream`. Replaces the factorisation inside metric_inv_half
 * (trnblas/level3.py:365-380: torch.linalg.cholesky + trsm,
 * trnblas/nki/dispatch.py:1854-1881); the panels, trailing updates and the
 * block inverse of L around it are DGEMMs on the host side of the op.
 */
int trnblas_hip_chol_block(int64_t nb, double* A, int64_t lda, double* Linv, int64_t ldl,
                           int32_t* info, int64_t offset, void* stream);

/*
 * Inverses of the 128 x 128 diagonal blocks of a triangular n x n matrix T
 * (trsm's diagonal solves, as GEMMs with these inverses): element (i, k) of
 * T at T[i * ldt_r + k * ldt_c] (any two positive strides: a transposed view
 * is passed as is); upper != 0: T is upper triangular, else lower; only
 * that triangle is read, and with unit != 0 its diagonal is taken as ones.
 * Dinv receives ceil(n / 128) row-major 128 x 128 blocks: block b is the
 * inverse of T[128 b : 128 b + 128, 128 b : 128 b + 128] (zeros in the other
 * triangle; the identity past n). dtype TRNBLAS_F32 or TRNBLAS_F64 (T and
 * Dinv); the arithmetic is fp64 either way. A zero pivot gives inf / NaN, as
 * a triangular solve does. Replaces the per-block
 * torch.linalg.solve_triangular calls of the reference's blocked trsm
 * (`_nki_trsm_left`, trnblas/nki/dispatch.py:1740-1799).
 */
int trnblas_hip_tri_inv_blocks(int dtype, int64_t n, int upper, int unit, const void* T,
                               int64_t ldt_r, int64_t ldt_c, void* Dinv, void* stream);

/* operand triangles of trnblas_hip_dgemm (bits of `tri`) */
#define TRNBLAS_TRI_A_LOWER 1 /* A[m][k] == 0 for k > m: a tile reads k < m0 + tile */
#define TRNBLAS_TRI_A_UPPER 2 /* A[m][k] == 0 for k < m: a tile reads k >= m0 */
#define TRNBLAS_TRI_B_LOWER 4 /* B[k][n] == 0 for k < n: a tile reads k >= n0 */
#define TRNBLAS_TRI_B_UPPER 8 /* B[k][n] == 0 for k > n: a tile reads k < n0 + tile */

/*
 * fp64 GEMM, strided-batched: D[b] = alpha * op(A[b]) * op(B[b]) + beta * C[b]
 * on the fp64 MFMA. The products of the metric stage: the reference runs
 * them as the GEMM updates of its blocked trsm (`_nki_trsm_left`,
 * trnblas/nki/dispatch.py:1740-1799, `mm(...)`) after torch.linalg.cholesky
 * (`_device_inv_chol_factor`, :1866-1870); here they are the panels and
 * trailing updates of the blocked Cholesky, the block products of the
 * triangular inverse and trsm's block solves and updates.
 *
 * op(A) is M x K: row-major M x K (lda >= K) when transA == 0, row-major
 * K x M (lda >= M) otherwise; likewise op(B) K x N. C and D are row-major
 * M x N (ldc, ldd >= N); D may be C itself (an in-place update); C is not
 * read when beta == 0. A and B need 16-byte aligned bases and even leading
 * dimensions, batch strides and contiguous extents (K when K is the
 * contiguous dimension, else M / N). lower != 0 (M == N, batch <= 1): only
 * the elements m >= n of D are computed and written. tri: TRNBLAS_TRI_* bits
 * of triangular operands whose zero blocks are skipped (their other
 * triangle must hold zeros).
 */
int trnblas_hip_dgemm(int transA, int transB, int64_t M, int64_t N, int64_t K, double alpha,
                      const double* A, int64_t lda, int64_t strideA, const double* B,
                      int64_t ldb, int64_t strideB, double beta, const double* C, int64_t ldc,
                      int64_t strideC, double* D, int64_t ldd, int64_t strideD, int64_t batch,
                      int lower, int tri, void* stream);

/*
 * metric_inv_half: X = L^-T for an SPD n x n fp64 J = L L^T (row-major,
 * ldj; only its lower triangle is read), X row-major (ldx), exactly upper
 * triangular. Replaces `nki_metric_inv_half` (trnblas/nki/dispatch.py:
 * 1883-1905; its device route `_device_inv_chol_factor` :1866-1870 is
 * torch.linalg.cholesky + the blocked trsm against the identity). One call
 * issues the whole sequence: a right-looking blocked Cholesky (128-wide
 * blocks; trnblas_hip_chol_block on the diagonal, trnblas_hip_dgemm panels
 * and lower-triangle trailing updates, the trailing update on a second
 * stream of the same device so the next diagonal block runs beside it),
 * then L^-1 by recursive doubling over block halves and its transpose.
 * info (device int32) is set to the order of the first leading minor that
 * is not positive definite, else 0 (X is then garbage). workspace: at least
 * trnblas_hip_metric_inv_half_workspace(n) bytes, 256-byte aligned. Calls on
 * one device share its second stream and are serialised on the host.
 */
size_t trnblas_hip_metric_inv_half_workspace(int64_t n);
int trnblas_hip_metric_inv_half(int64_t n, const double* J, int64_t ldj, double* X, int64_t ldx,
                                int32_t* info, void* workspace, size_t workspace_bytes,
                                void* stream);

/*
 * Triangular solve T X = alpha B, T n x n triangular (upper != 0: upper,
 * else lower; only that triangle read; unit != 0: its diagonal taken as
 * ones), B n x nrhs, X n x nrhs; element (i, j) of each matrix at
 * base[i * ld_r + j * ld_c] (any positive strides: a transposed view is
 * passed as is, which is how the left / right and trans forms of trsm map
 * to this one). dtype TRNBLAS_F32 or TRNBLAS_F64. Replaces the reference's
 * blocked `_nki_trsm_left` (trnblas/nki/dispatch.py:1740-1799): the
 * 128 x 128 diagonal blocks are all inverted in one launch
 * (trnblas_hip_tri_inv_blocks), then the solve recurses over block halves
 * with GEMM updates (fp64: trnblas_hip_dgemm; fp32: trnblas_hip_gemm).
 * workspace: at least trnblas_hip_trsm_workspace(dtype, n, nrhs) bytes,
 * 256-byte aligned. X may not overlap T or B.
 */
size_t trnblas_hip_trsm_workspace(int dtype, int64_t n, int64_t nrhs);
int trnblas_hip_trsm(int dtype, int64_t n, int64_t nrhs, int upper, int unit, double alpha,
                     const void* T, int64_t ldt_r, int64_t ldt_c, const void* B, int64_t ldb_r,
                     int64_t ldb_c, void* X, int64_t ldx_r, int64_t ldx_c, void* workspace,
                     size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* TRNBLAS_HIP_H */
