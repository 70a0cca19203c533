/* fermix_amd C ABI: batched fp32 (and fp64) slogdet / slogpf (and the factors and inverses their
 * gradients need) on AMD Instinct MI355X (gfx950), as hand-written HIP kernels.
 *
 * This is the drop-in boundary for the hot path of ChenAo-Phys/fermix: each entry
 * point replaces the group of Pallas calls the reference issues through
 * `_pcall` (src/fermix/_field.py:357-389) for one role, cited per function below. The
 * reference binds its kernels inside JAX; a maintainer would bind this header from an
 * XLA FFI handler (one typed-buffer handler per entry point, the stream taken from the
 * call's platform stream).
 *
 * Conventions (all entry points):
 *  - matrices are row-major, contiguous, batch-major: a[b * n * n + i * n + j];
 *  - the caller owns every buffer; the library never allocates device memory, never
 *    synchronises, and only enqueues work on `stream` (a hipStream_t; NULL = the legacy
 *    default stream);
 *  - `workspace` is caller-provided device memory of at least the size reported by the
 *    matching *_workspace function (0 means no workspace is needed; NULL allowed then);
 *  - alignment: every matrix-shaped pointer (a, lu, perm, inv_t, adj_t, gbuf, d, g) and
 *    the workspace must be 16-byte aligned, and sign / logabs / scale aligned to their
 *    element size; a misaligned pointer returns FX_ERR_INVALID_ARGUMENT before any work is
 *    enqueued (memory from hipMalloc, or a tensor allocator, satisfies this; a slice of a
 *    batch at an odd member offset of an odd-n batch does not and must be copied);
 *  - any batch size up to 2^31 - 1 is accepted: entry points whose kernels put the
 *    batch on a grid dimension limited to 65535 run it in consecutive chunks of 65528
 *    members on the stream, and their *_workspace sizes are those of one chunk;
 *  - the return value is a status code (FX_OK on success); numerical edge cases are
 *    encoded in the values (an exactly zero pivot gives sign 0 and logabs -inf);
 *  - calls are reentrant; the library keeps no mutable global state apart from the
 *    once-per-device address of the scratch array of fx_slogdet_f32_noalloc, the
 *    once-per-device second stream (and its two events) on which the blocked LU runs
 *    half of a large batch (ordered after the caller's stream and joined back to it
 *    before the call returns; held under a per-device lock while in use) and the
 *    tuning-table override of fx_tune_override;
 *  - the kernel family is chosen from n alone (never from the batch): several matrices
 *    per wave (n <= 32 for slogdet, 16 for slogpf), one fused workgroup per matrix
 *    (n <= fx_tune.fused_max_n, 128 in the gfx950 table), blocked kernels with workspace
 *    (float32: the Parlett-Reid to n = 8192, the LU to fx_tune.lu_generic_above_n, 4096,
 *    then the field-generic blocked kernels to 16384); the blocked kernels' own choices follow the tuning table below, whose
 *    fx_tune_override is the reference's OVERRIDE hook. The environment variable
 *    FERMIX_AMD_KERNELS = tiny | fused | blocked | generic, read on every call, forces a
 *    family where it covers n (generic: the field-generic blocked kernels that run
 *    float32 above 8192, for any n > 128; FX_ERR_UNSUPPORTED elsewhere); the padded orders, block widths
 *    and workspace sizes reported below follow it, so query them under the same setting
 *    as the call (a test hook like the reference's OVERRIDE, src/fermix/_common.py:
 *    363-378).
 */
#ifndef FERMIX_AMD_H
#define FERMIX_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FX_OK 0
#define FX_ERR_INVALID_ARGUMENT 1 /* bad pointer, batch < 0, n < 0, ... */
#define FX_ERR_WORKSPACE 2        /* workspace missing or too small */
#define FX_ERR_LAUNCH 3           /* a HIP launch failed (hipGetLastError) */
#define FX_ERR_UNSUPPORTED 4      /* size not covered by the compiled kernels */

typedef void* fx_stream_t; /* hipStream_t */

/* prec: the arithmetic of the MFMA products (the reference's `prec`, src/fermix/_field.py:
 * 20-23, 173-190, 262-275, whose fp32 modes are "ieee" and "tf32x3"):
 *  - FX_PREC_IEEE: fp32 MFMA (v_mfma_f32_32x32x2f32 / 16x16x4f32);
 *  - FX_PREC_BF16X3: every fp32 operand split as hi + mid + lo bf16 (round to nearest, the
 *    residues exact in fp32) and the six products with terms down to 2^-16 of the leading
 *    one on v_mfma_f32_32x32x16_bf16, fp32 accumulation -- gfx950's counterpart of the
 *    reference's tf32x3 (three reduced-precision passes at fp32 accuracy).
 * It applies to the blocked (n > 128) LU trailing updates and to every GEMM of the
 * inverses (A^-T, S^-1, the adjugates). The n <= 128 kernels, the panels, the U-row solves,
 * the diagonal-block inverses and the Parlett-Reid trailing update (bound by memory
 * traffic, not by the MFMA rate) compute in fp32 in both modes; the slogpf forward entry
 * points therefore take no prec. */
#define FX_PREC_IEEE 0
#define FX_PREC_BF16X3 1

/* Option bits or-ed into the prec argument of the slogdet / det entry points (float32):
 * the outer LU block of the blocked family (n > 128), the reference's per-call `block`
 * (src/fermix/api.py:92-97, _common.py:31-41). The factorisation is built from 64-column
 * panels whose trailing updates go either one block at a time (K = 64) or in pairs of
 * blocks (one K = 128 update per pair):
 *  - FX_LU_BLOCK_TABLE (0): the tuning table's choice (pairs for padded N above
 *    fx_tune.lu_pair_above_n);
 *  - FX_LU_BLOCK_64: single 64-column blocks;
 *  - FX_LU_BLOCK_128: blocks in pairs, K = 128 updates.
 * The choice changes the rounding of the factorisation, so a gradient call must pass the
 * option of the forward call it differentiates (sign / logabs are then bit-identical).
 * fx_slogdet_inverse_f32 and the slogpf entry points accept prec values without option
 * bits only. */
#define FX_PREC_MASK 0x0f
#define FX_LU_BLOCK_TABLE 0x000
#define FX_LU_BLOCK_64 0x100
#define FX_LU_BLOCK_128 0x200
#define FX_LU_BLOCK_MASK 0x300

/* ---------------------------------------------------------------- tuning table
 * The library's launch choices for one GPU architecture: the counterpart of the
 * reference's Tune / TUNES[arch][kind] / OVERRIDE (src/fermix/_common.py:17-378), whose
 * fields are Triton tiles and warps; here every field is a size threshold of a dispatch
 * decision the host code makes from n alone (never from the batch). The float32 fields
 * steer the fp32 kernels, the f64_ fields the float64 ones. Ranges are those the compiled
 * kernels support; values outside them are rejected by fx_tune_override. */
typedef struct fx_tune {
  /* float32 families: n <= fused_max_n (above the several-matrices-per-wave sizes,
   * n <= 32 for slogdet and n <= 16 for slogpf, which are fixed) runs one workgroup per
   * matrix with the matrix in LDS; larger n runs the blocked kernels. 32 .. 128 */
  int32_t fused_max_n;
  /* blocked LU: 64-column blocks in pairs (one K = 128 trailing update per pair) for
   * padded order N > lu_pair_above_n (FX_LU_BLOCK_TABLE). >= 0 */
  int32_t lu_pair_above_n;
  /* blocked LU: the first block pair reads the input in place of a copy into the
   * workspace when n = N <= lu_direct_max_n (16-byte aligned input). 0 .. 1024 */
  int32_t lu_direct_max_n;
  /* blocked Parlett-Reid (N <= 2048): 64-column blocks once the trailing order is at most
   * pf_block64_max_m, for padded orders N >= pf_block64_min_n that are multiples of 64;
   * 32-column blocks otherwise (16 above N = 2048, 8 above N = 4096). 128 .. 4096 / 0 .. 1024 */
  int32_t pf_block64_min_n;
  int32_t pf_block64_max_m;
  /* GEMMs of the inverses and adjugates in FX_PREC_IEEE: 128 x 128 tiles when M, N >=
   * gemm128_min_mn and K >= gemm128_min_k, else 64 x 64 (bit-identical results); the
   * product with A^-T's transposed, row-permuted output too if gemm128_tout (0 / 1).
   * >= 128 / >= 64 */
  int32_t gemm128_min_mn;
  int32_t gemm128_min_k;
  int32_t gemm128_tout;
  /* the same three for FX_PREC_BF16X3 (the 128 x 128 kernel splits each operand once
   * into bf16 planes in LDS, the 64 x 64 one at every use) */
  int32_t gemm128_x3_min_mn;
  int32_t gemm128_x3_min_k;
  int32_t gemm128_x3_tout;
  /* float64: the matrix in registers for n <= f64_reg_max_n (0 .. 128), with rows split
   * in 16-column strips for n <= f64_strip16_max_n (0 .. 64) and 32-column ones above;
   * larger n runs one workgroup per matrix in LDS or in the workspace */
  int32_t f64_reg_max_n;
  int32_t f64_strip16_max_n;
  /* blocked float32 Parlett-Reid: the batch runs as two halves, each launch holding one
   * half's 1024-thread panels beside the other half's trailing update, when a half holds
   * at most pf_overlap_max_half matrices and batch * N^2 >= pf_overlap_min_work * 2^20
   * (the same bits as unsplit). >= 0 / >= 0 */
  int32_t pf_overlap_max_half;
  int32_t pf_overlap_min_work;
  /* blocked float32 LU of padded order N <= 4096: batches of at least two matrices with
   * batch * N^2 >= lu_split_min_work * 2^20 run as two halves on two streams (the same
   * bits as unsplit); 0 never. >= 0 */
  int32_t lu_split_min_work;
  /* float32 LU (slogdet, det and their gradients): n > lu_generic_above_n runs the
   * field-generic blocked kernels (multi-workgroup panels, fp64 MFMA products) in place
   * of the float32 blocked ones, whose register panels spill for very tall panels (the
   * reference's lu_generic_above_n, src/fermix/_common.py:126,211-281). 128 .. 8192 */
  int32_t lu_generic_above_n;
  int32_t reserved[3]; /* zero */
} fx_tune;

/* The table of an architecture ("gfx950"; FX_ERR_UNSUPPORTED for any other name: the
 * library holds gfx950 code only). */
int fx_tune_table(const char* arch, fx_tune* out);

/* Replace the table for every later call in the process (NULL: back to the table) -- the
 * reference's OVERRIDE hook, for tuning sweeps and tests. FX_ERR_INVALID_ARGUMENT (and no
 * change) for a field outside its range. Workspace sizes follow the active values, so
 * query them after setting an override. Not to be changed while another thread is inside
 * an entry point of the library. */
int fx_tune_override(const fx_tune* t);

/* The values in effect (the override if one is set, else the gfx950 table). */
int fx_tune_active(fx_tune* out);

/* Human-readable text of a status code (static storage). */
const char* fx_status_string(int status);

/* ABI version of this header (major * 100 + minor). */
int fx_abi_version(void);

/* Padded order N >= n of the LU factors returned by fx_slogdet_parts_f32 (identity
 * padding; the reference pads to its block size the same way, src/fermix/_common.py:
 * 527-539). */
int32_t fx_lu_padded_size(int32_t n);

/* Padded order N of the Parlett-Reid factors of fx_slogpf_factors_f32. */
int32_t fx_pf_padded_size(int32_t n);

/* ---------------------------------------------------------------- slogdet
 * sign[b], logabs[b] of det(a[b]) for b < batch: sign exactly +1 / -1, or 0 with
 * logabs = -inf for an exactly zero pivot. Sizes: the float64 and complex entry points
 * cover 0 <= n <= 8192, the float32 ones 0 <= n <= 16384, and return FX_ERR_UNSUPPORTED
 * above. float32 above n = 4096: the Parlett-Reid blocks are 8 columns wide (latency-bound;
 * the trailing updates and GEMMs are those of the smaller orders); the LU above
 * fx_tune.lu_generic_above_n (4096) and the Parlett-Reid above 8192 run the field-generic
 * blocked kernels of the float64 path on float storage (32-column panels, tall ones on
 * several workgroups per matrix, the trailing products in fp64 on the MFMA, prec without
 * effect), for the values and the parts runs (fx_slogdet_parts_f32 with zero_singular and
 * no lu / perm, fx_det_parts_f32, fx_slogpf_parts_f32); the packed factor exports and
 * their inverses (fx_slogdet_factors_f32, fx_slogdet_inverse_f32, fx_lu_padded_size:
 * above lu_generic_above_n; fx_slogpf_factors_f32, fx_slogpf_inverse_f32,
 * fx_pf_padded_size: above 8192) return FX_ERR_UNSUPPORTED / 0 / -1 there.
 * Replaces `_lu_core` (src/fermix/_lu.py:543-611) as called by `_slogdet_core`
 * (src/fermix/_diff.py:42-49); kernels K1-K4 of the reference (_lu.py:54-393). */
size_t fx_slogdet_f32_workspace(int64_t batch, int32_t n);
int fx_slogdet_f32(const float* a, int64_t batch, int32_t n, float* sign, float* logabs, int32_t prec,
                   void* workspace, size_t workspace_bytes, fx_stream_t stream);

/* The same factorisation as fx_slogdet_f32 (identical arithmetic, so sign / logabs are
 * bit-identical to it) plus, each optional (NULL to skip):
 *  - inv_t (batch, n, n): A^-T formed with the zero pivots of U replaced by 1; zero for
 *    members with a non-finite result and, if zero_singular != 0, for members with an
 *    exactly zero pivot;
 *  - lu (batch, N, N), N = fx_lu_padded_size(n): packed L (unit, strictly lower) and U
 *    of P A' where A' = [[A, 0], [0, I]];
 *  - perm (batch, N): (P A')[c] = A'[perm[c]].
 * Replaces `_lu_parts` (src/fermix/_inverse.py:502-531) as called by `_parts`
 * (src/fermix/_diff.py:62-77); kernels K7-K10 (_inverse.py:35-499). */
size_t fx_slogdet_parts_f32_workspace(int64_t batch, int32_t n);
int fx_slogdet_parts_f32(const float* a, int64_t batch, int32_t n, int32_t zero_singular,
                         float* sign, float* logabs, float* inv_t, float* lu, int32_t* perm, int32_t prec,
                         void* workspace, size_t workspace_bytes, fx_stream_t stream);

/* The factors of fx_slogdet_parts_f32 alone, formed straight in the caller's lu
 * (batch, N, N) and perm (batch, N) (N = fx_lu_padded_size(n); same layout), with sign /
 * logabs bit-identical to fx_slogdet_f32. Together with fx_slogdet_inverse_f32 this
 * splits `_lu_parts` (src/fermix/_inverse.py:502-531) into its factorisation, run by the
 * forward pass, and the inverse, run by the backward pass once the cotangent is known. */
size_t fx_slogdet_factors_f32_workspace(int64_t batch, int32_t n);
int fx_slogdet_factors_f32(const float* a, int64_t batch, int32_t n, float* sign, float* logabs, float* lu,
                           int32_t* perm, int32_t prec, void* workspace, size_t workspace_bytes, fx_stream_t stream);

/* inv_t (batch, n, n) = scale[b] * A^-T (scale NULL: 1) from the factors lu / perm of
 * fx_slogdet_factors_f32 (or fx_slogdet_parts_f32) and their sign, with the guards of
 * fx_slogdet_parts_f32's inv_t (zero pivots of U replaced by 1; zero for non-finite
 * results and, if zero_singular != 0, for members with sign 0). lu is used as scratch
 * and overwritten. With scale = the logabs cotangent, inv_t is the slogdet VJP itself:
 * `_permT` with the guard of `_lu_parts` (src/fermix/_inverse.py:478-531) and the
 * cotangent product of the jvp rule (src/fermix/_diff.py:92-126) in one pass. */
size_t fx_slogdet_inverse_f32_workspace(int64_t batch, int32_t n);
int fx_slogdet_inverse_f32(float* lu, const int32_t* perm, const float* sign, const float* scale, int64_t batch,
                           int32_t n, int32_t zero_singular, float* inv_t, int32_t prec, void* workspace,
                           size_t workspace_bytes, fx_stream_t stream);

/* adj_t (batch, n, n) = adj(A)^T = d det(A) / dA, finite and exact for singular A, plus
 * sign / logabs bit-identical to fx_slogdet_f32 (det = sign * exp(logabs) is the value
 * the reference's det returns with this gradient). From the packed LU of the same run:
 * det(factors) * A^-T for members without an exact zero pivot; with zero pivots at
 * k1 <= ... <= km (U~ = U with them replaced by 1, d_K = product of the other pivots) the
 * rank-1 form sgn(P) d_K c (U~^-1 e_k1)(e_km^T U~^-1 L^-1 P), c = (U~^-1)[k1, km] for
 * m = 2 and 1 for m = 1; 0 for m >= 3. Non-finite inverses give 0.
 * Replaces `_det_gradT` (src/fermix/_diff.py:205-246) with `_lu_det` (:184-202) and
 * `_perm_sign` (:160-176) on top of `_parts(zero_singular=False)`, as called by the jvp
 * rule of `_det_diff` (:288-301). */
size_t fx_det_parts_f32_workspace(int64_t batch, int32_t n);
int fx_det_parts_f32(const float* a, int64_t batch, int32_t n, float* sign, float* logabs, float* adj_t,
                     int32_t prec, void* workspace, size_t workspace_bytes, fx_stream_t stream);

/* No counterpart in the reference: fx_slogdet_f32 for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments without the workspace (and prec: FX_PREC_IEEE); sign / logabs
 * bit-identical to fx_slogdet_f32 with FX_PREC_IEEE. The blocked kernels' workspace (n > 128) is a device array of the
 * library of FX_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends); a batch whose
 * workspace exceeds it runs in consecutive sub-batches that fit. n whose single-matrix
 * workspace exceeds the array (n > 4032) returns FX_ERR_UNSUPPORTED. The call allocates
 * nothing. Calls that overlap on one GPU share its array and race: serialise them. */
#define FX_NOALLOC_SCRATCH_BYTES (64u << 20)
int fx_slogdet_f32_noalloc(const float* a, int64_t batch, int32_t n, float* sign, float* logabs,
                           fx_stream_t stream);
/* Host-only plan query of fx_slogdet_f32_noalloc (no counterpart in the reference): the
 * number of members per sub-batch it runs for (batch, n) -- batch itself when one sub-batch
 * suffices, a multiple of 8 when at least 8 fit -- and 0 when it returns
 * FX_ERR_UNSUPPORTED. */
int64_t fx_slogdet_f32_noalloc_batch(int64_t batch, int32_t n);

/* ---------------------------------------------------------------- slogpf
 * sign[b], logabs[b] of pf(S[b]), S = (a - a^T) / 2 if skew_symmetrize != 0, else
 * S = a (which must then be exactly skew-symmetric). Odd n gives (0, -inf).
 * Replaces `_pf_core` (src/fermix/_pf.py:497-570) as called by `_slogpf_core`
 * (src/fermix/_diff.py:52-59), with the skew-symmetrisation of `_slogpf`
 * (src/fermix/api.py:124-125) fused into the load; kernels K5-K6 (_pf.py:59-382). */
size_t fx_slogpf_f32_workspace(int64_t batch, int32_t n);
int fx_slogpf_f32(const float* a, int64_t batch, int32_t n, int32_t skew_symmetrize, float* sign,
                  float* logabs, void* workspace, size_t workspace_bytes, fx_stream_t stream);

/* Columns per chunk of the Parlett-Reid factors: 16 for n <= 128, 32 for n <= 2048, 16
 * above (a chunk holds 16 or 8 pair steps; a 64-column block of the factorisation spans
 * two chunks). */
int32_t fx_pf_block_columns(int32_t n);

/* The Parlett-Reid factors P S' P^T = L D L^T of the same run (S' = S padded with
 * [[0,1],[-1,0]] blocks to N = fx_pf_padded_size(n)), PB = fx_pf_block_columns(n):
 *  - gbuf (batch, N/PB, N, PB): chunk k's tau_t (column 2t) and w_t (column 2t+1) of the
 *    pair steps PB/2 k + t, indexed by the original row; entries of rows assigned before
 *    the pair step are zero, rows assigned before chunk k are unspecified;
 *  - d (batch, N/2): the pair pivots d_s = (P S' P^T reduced)[2s, 2s+1];
 *  - perm (batch, N): final position -> original row.
 * sign / logabs are bit-identical to fx_slogpf_f32. Replaces `_pf_core_factors`
 * (src/fermix/_pf.py:497-514). */
size_t fx_slogpf_factors_f32_workspace(int64_t batch, int32_t n);
int fx_slogpf_factors_f32(const float* a, int64_t batch, int32_t n, int32_t skew_symmetrize,
                          float* sign, float* logabs, float* gbuf, float* d, int32_t* perm,
                          void* workspace, size_t workspace_bytes, fx_stream_t stream);

/* g (batch, n, n) = scale[b] * S^-1 (adjugate = 0) or scale[b] * pf(S) S^-1 (adjugate
 * != 0) from the factors of fx_slogpf_factors_f32 (read only; scale NULL: 1), with the
 * guards of fx_slogpf_parts_f32's g. With scale = -cotangent / 2 it is the slogpf VJP:
 * `_pf_parts` (src/fermix/_pfinv.py:196-269) on saved factors, with the cotangent
 * product of the jvp rule (src/fermix/_diff.py:129-156) in its final gather. */
size_t fx_slogpf_inverse_f32_workspace(int64_t batch, int32_t n);
int fx_slogpf_inverse_f32(const float* gbuf, const float* d, const int32_t* perm, const float* scale,
                          int64_t batch, int32_t n, int32_t adjugate, float* g, int32_t prec, void* workspace,
                          size_t workspace_bytes, fx_stream_t stream);

/* The same run as fx_slogpf_f32 (bit-identical sign / logabs) plus g (batch, n, n)
 * formed from the run's own factors (no second factorisation):
 *  - adjugate = 0: S^-1, zero for members with an exactly zero pivot or a non-finite
 *    result (the slogpf gradient is -g / 2);
 *  - adjugate != 0: pf(S) S^-1, the Pfaffian adjugate, finite and exact for singular S
 *    (a second exact zero pivot is lifted to +1 and -1 and the two evaluations averaged;
 *    the pf gradient is -g / 2). Odd n gives g = 0 in both modes.
 * Replaces `_pf_parts` (src/fermix/_pfinv.py:196-269) as called by `_pf_grad_parts`
 * (src/fermix/_diff.py:80-89); kernels K11-K12 (_pfinv.py:80-192) and the adjugate
 * helpers `_pf_adj_coeffs` / `_lifted_mean` (src/fermix/_fallback.py:138-176). */
size_t fx_slogpf_parts_f32_workspace(int64_t batch, int32_t n);
int fx_slogpf_parts_f32(const float* a, int64_t batch, int32_t n, int32_t skew_symmetrize,
                        int32_t adjugate, float* sign, float* logabs, float* g, int32_t prec, void* workspace,
                        size_t workspace_bytes, fx_stream_t stream);

/* ---------------------------------------------------------------- float64
 * The reference takes float64 through the same API (`_prep`, src/fermix/api.py:24-31,
 * with 64-bit fields, src/fermix/_field.py:20-120 and :265-275). These entry points are
 * the float64 counterparts of the ones above, with the same argument meaning, outputs
 * in float64 and 0 <= n <= 8192. For n <= fx_tune.f64_reg_max_n (128) one workgroup per
 * matrix holds it in registers: an LU / Gauss-Jordan with partial pivoting
 * (`_slogdet_generic`, `_lu_parts_generic`, src/fermix/_fallback.py:36-97) and
 * Parlett-Reid (`_slogpf_generic`, :266-300), no workspace. Above, slogdet / det and the
 * inverses run a blocked LU (32-column panels, the trailing updates on the fp64 MFMA) and
 * blocked solves of it in a workspace of two padded matrix copies per member, and slogpf
 * a blocked Parlett-Reid (16 pair steps per panel, the pivot swapped into c + 1 as the
 * generic path does, the K = 32 trailing update on the fp64 MFMA; one padded matrix copy
 * plus 64 columns per member). The kernel family override FERMIX_AMD_KERNELS does not
 * apply to them. */
size_t fx_slogdet_f64_workspace(int64_t batch, int32_t n);
int fx_slogdet_f64(const double* a, int64_t batch, int32_t n, double* sign, double* logabs, void* workspace,
                   size_t workspace_bytes, fx_stream_t stream);

/* sign / logabs bit-identical to fx_slogdet_f64, plus inv_t (batch, n, n) = A^-T (NULL to
 * skip), zero for members with an exactly zero pivot or a non-finite inverse (the
 * zero_singular = 1 convention of fx_slogdet_parts_f32). */
size_t fx_slogdet_parts_f64_workspace(int64_t batch, int32_t n);
int fx_slogdet_parts_f64(const double* a, int64_t batch, int32_t n, double* sign, double* logabs, double* inv_t,
                         void* workspace, size_t workspace_bytes, fx_stream_t stream);

size_t fx_slogpf_f64_workspace(int64_t batch, int32_t n);
int fx_slogpf_f64(const double* a, int64_t batch, int32_t n, int32_t skew_symmetrize, double* sign, double* logabs,
                  void* workspace, size_t workspace_bytes, fx_stream_t stream);

/* sign / logabs bit-identical to fx_slogpf_f64, plus g (batch, n, n) (NULL to skip):
 * adjugate = 0: g = S^-1, zero where pf(S) = 0 (odd n, an exactly zero pivot) or S^-1 is
 * not finite;
 * adjugate != 0: g = pf(S) S^-1, the Pfaffian adjugate (pf's gradient, -g / 2 = d pf / dS),
 * finite and exact for singular S (rank n - 2: the rank-2 adjugate; rank <= n - 4: 0),
 * zero for odd n: the reference's formula (_pf_adj_blocks / _pf_adj_coeffs / _second_zero,
 * src/fermix/_fallback.py:101-192) from a Parlett-Reid run of its own (the smallest
 * pivot K by modulus, exact zero pivots and d_K replaced by 1) and one Gauss-Jordan
 * inverse of the replaced factorisation, a second exact zero pivot lifted to +1 and -1
 * (two inverses for those members); above n = 128 only the members with pf = 0 or a
 * numerically singular S (the forward's pair pivots spanning more than 2^18 in modulus)
 * take that route, the others pf(S) times S^-1 from the blocked LU solves; sign / logabs
 * stay those of the plain forward. */
size_t fx_slogpf_parts_f64_workspace(int64_t batch, int32_t n);
int fx_slogpf_parts_f64(const double* a, int64_t batch, int32_t n, int32_t skew_symmetrize, int32_t adjugate,
                        double* sign, double* logabs, double* g, void* workspace, size_t workspace_bytes,
                        fx_stream_t stream);

/* ---------------------------------------------------------------- complex
 * The reference's complex kinds (complex64 / complex128 through the same API: `_prep`,
 * src/fermix/api.py:24-31; the complex field, src/fermix/_field.py:32-120, 129-162). A
 * complex matrix is interleaved (re, im) pairs, row-major and batch-major (the memory of
 * a C99 complex array, or of torch's complex tensors): a[2 (b n n + i n + j) + {0, 1}];
 * sign is one complex value per member (2 floats / doubles), logabs real. Conventions of
 * the generic path (src/fermix/_fallback.py:36-55, 266-300): the pivot is the candidate
 * of largest |re| + |im| (LAPACK's cabs1, the reference's `abs1`), sign = parity *
 * prod(d / |d|), logabs = sum log|d|, an exactly zero pivot gives sign 0 and logabs -inf;
 * inv_t = A^-T without conjugation (the holomorphic derivative of log det, as in
 * `_lu_parts_generic`, :63-97). 0 <= n <= 8192. Up to n = 64 one workgroup per matrix,
 * the matrix in LDS when it fits (else one copy per member in the workspace; twice that
 * with the inverse); above, the blocked kernels of the float64 path on the complex field
 * (32-column LU panels, 16-pair Parlett-Reid panels, the trailing updates as four real
 * MFMA products per complex one). The complex64 entry points take prec:
 * FX_PREC_BF16X3 (the fp32-accuracy mode, the Python API's default as for float32) forms
 * those products on the fp64 MFMA with the operands widened to double; FX_PREC_IEEE as
 * four fp32 MFMA products (the reference's complex64 fp32-rate products, _field.py:173-190;
 * the fp32 MFMA's rate and rounding). Any other value: FX_ERR_INVALID_ARGUMENT. Up to
 * n = 64 (no blocked products) both give the same bits. complex128 has no prec (IEEE
 * fp64). */
size_t fx_slogdet_c64_workspace(int64_t batch, int32_t n);
int fx_slogdet_c64(const float* a, int64_t batch, int32_t n, float* sign, float* logabs, int32_t prec,
                   void* workspace, size_t workspace_bytes, fx_stream_t stream);
size_t fx_slogdet_c128_workspace(int64_t batch, int32_t n);
int fx_slogdet_c128(const double* a, int64_t batch, int32_t n, double* sign, double* logabs, void* workspace,
                    size_t workspace_bytes, fx_stream_t stream);

/* sign / logabs bit-identical to fx_slogdet_c64 / _c128, plus inv_t (batch, n, n) = A^-T
 * (NULL to skip), zero for members with an exactly zero pivot or a non-finite inverse. */
size_t fx_slogdet_parts_c64_workspace(int64_t batch, int32_t n);
int fx_slogdet_parts_c64(const float* a, int64_t batch, int32_t n, float* sign, float* logabs, float* inv_t,
                         int32_t prec, void* workspace, size_t workspace_bytes, fx_stream_t stream);
size_t fx_slogdet_parts_c128_workspace(int64_t batch, int32_t n);
int fx_slogdet_parts_c128(const double* a, int64_t batch, int32_t n, double* sign, double* logabs, double* inv_t,
                          void* workspace, size_t workspace_bytes, fx_stream_t stream);

/* pf of complex skew-symmetric S (S^T = -S; S = (a - a^T) / 2 if skew_symmetrize != 0):
 * Parlett-Reid with the pivot swapped into column c + 1 (`_slogpf_generic`,
 * src/fermix/_fallback.py:266-300); odd n gives (0, -inf). */
size_t fx_slogpf_c64_workspace(int64_t batch, int32_t n);
int fx_slogpf_c64(const float* a, int64_t batch, int32_t n, int32_t skew_symmetrize, float* sign, float* logabs,
                  int32_t prec, void* workspace, size_t workspace_bytes, fx_stream_t stream);
size_t fx_slogpf_c128_workspace(int64_t batch, int32_t n);
int fx_slogpf_c128(const double* a, int64_t batch, int32_t n, int32_t skew_symmetrize, double* sign,
                   double* logabs, void* workspace, size_t workspace_bytes, fx_stream_t stream);

/* sign / logabs bit-identical to fx_slogpf_c64 / _c128, plus g (batch, n, n) (NULL to
 * skip): adjugate = 0: g = S^-1, zero where pf(S) = 0 (odd n, an exactly zero pivot) or
 * S^-1 is not finite;
 * adjugate != 0: g = pf(S) S^-1, the Pfaffian adjugate (pf's gradient, -g / 2 = d pf / dS),
 * finite and exact for singular S (rank n - 2: the rank-2 adjugate; rank <= n - 4: 0),
 * zero for odd n: the reference's formula (_pf_adj_blocks / _pf_adj_coeffs / _second_zero,
 * src/fermix/_fallback.py:101-192) from a Parlett-Reid run of its own (the smallest
 * pivot K by modulus, exact zero pivots and d_K replaced by 1) and one Gauss-Jordan
 * inverse of the replaced factorisation, a second exact zero pivot lifted to +1 and -1
 * (two inverses for those members); above n = 64 only the members with pf = 0 or a
 * numerically singular S (the forward's pair pivots spanning more than 2^8 in modulus for
 * complex64, 2^18 for complex128) take that route, the others pf(S) times S^-1 from the
 * blocked LU solves; sign / logabs stay those of the plain forward. */
size_t fx_slogpf_parts_c64_workspace(int64_t batch, int32_t n);
int fx_slogpf_parts_c64(const float* a, int64_t batch, int32_t n, int32_t skew_symmetrize, int32_t adjugate,
                        float* sign, float* logabs, float* g, int32_t prec, void* workspace, size_t workspace_bytes,
                        fx_stream_t stream);
size_t fx_slogpf_parts_c128_workspace(int64_t batch, int32_t n);
int fx_slogpf_parts_c128(const double* a, int64_t batch, int32_t n, int32_t skew_symmetrize, int32_t adjugate,
                         double* sign, double* logabs, double* g, void* workspace, size_t workspace_bytes,
                         fx_stream_t stream);

/* adj_t (batch, n, n) = adj(A)^T = d det(A) / dA (holomorphic for complex A, no
 * conjugation) plus sign / logabs of the same Gauss-Jordan run, for float64, complex64
 * and complex128 -- fx_det_parts_f32's contract: det(A) A^-T from the run's own pivots
 * when no pivot is exactly zero; with zero pivots at columns k1 <= ... <= km (U~ = U with
 * them taken as 1, d_K = the product of the other pivots) the rank-1 continuation
 * sgn(P) d_K c (U~^-1 e_k1)(e_km^T U~^-1 L^-1 P) with c = (U~^-1)[k1, km] for m = 2 and 1
 * for m = 1; 0 for m >= 3 and for a non-finite result. Replaces `_det_gradT` with `_lu_det`
 * and `_perm_sign` (src/fermix/_diff.py:160-246) for the 64-bit and complex kinds. One
 * workgroup per matrix up to n = 128 (float64) / 64 (complex; no workspace while [A | I]
 * fits in 60 KiB of LDS); above, the blocked LU, whose solves give the regular members'
 * det(A) A^-T, the Gauss-Jordan continuation then running only for the exactly singular
 * members. The sign / logabs equal those of fx_slogdet_f64 / _c64 / _c128 (the same
 * pivots and per-element updates). */
size_t fx_det_parts_f64_workspace(int64_t batch, int32_t n);
int fx_det_parts_f64(const double* a, int64_t batch, int32_t n, double* sign, double* logabs, double* adj_t,
                     void* workspace, size_t workspace_bytes, fx_stream_t stream);
size_t fx_det_parts_c64_workspace(int64_t batch, int32_t n);
int fx_det_parts_c64(const float* a, int64_t batch, int32_t n, float* sign, float* logabs, float* adj_t,
                     int32_t prec, void* workspace, size_t workspace_bytes, fx_stream_t stream);
size_t fx_det_parts_c128_workspace(int64_t batch, int32_t n);
int fx_det_parts_c128(const double* a, int64_t batch, int32_t n, double* sign, double* logabs, double* adj_t,
                      void* workspace, size_t workspace_bytes, fx_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FERMIX_AMD_H */
