// Internal launcher declarations of the fermix_amd HIP library (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "../../include/fermix.h"

namespace fx {

// The tuning values in effect (tune.hip): the gfx950 table, or the fx_tune_override.
const fx_tune& tune();
// Held by every C entry point for the length of the call: pins the tuning table that is
// active when the call begins (nested entry points keep the outer pin), so a concurrent
// fx_tune_override takes effect at a thread's next call, never part-way through one.
struct TunePin {
  TunePin();
  ~TunePin();
  TunePin(const TunePin&) = delete;
  TunePin& operator=(const TunePin&) = delete;

 private:
  bool own_;
};

// The device's second stream (side.hip) for a driver that runs two halves of a batch side
// by side. With want and the stream available (not under graph capture), ok() holds and
// the device's side stream is reserved until the destructor: fork() orders the side
// stream after the work enqueued so far on s, join() (also run by the destructor) orders
// s after the side stream's work.
class SideStream {
 public:
  SideStream(hipStream_t s, bool want);
  ~SideStream();
  SideStream(const SideStream&) = delete;
  SideStream& operator=(const SideStream&) = delete;
  bool ok() const { return side_ != nullptr; }
  hipStream_t side() const { return side_ ? *side_ : s_; }
  int fork();
  int join();

 private:
  hipStream_t s_;
  hipStream_t* side_ = nullptr;
  hipEvent_t* fork_ = nullptr;
  hipEvent_t* join_ = nullptr;
  bool forked_ = false;
  std::unique_lock<std::mutex> lk_;
};

// Compute units of the current device (side.hip; queried once per device, 256 if the
// query fails).
int device_cus();

// dst[i] = src[i] for i < count: count a multiple of 4, both pointers 16-byte aligned.
int launch_copy(const float* src, float* dst, int64_t count, hipStream_t s);

// n <= TINY_MAXN (LU) / PF_TINY_MAXN (Parlett-Reid): several matrices per wave, one lane
// per row (tiny.hip). Same outputs
// and factor formats as the n <= 128 kernels below (N = tiny_padded(n) = 16 or 32),
// which dispatch to them for these n.
constexpr int TINY_MAXN = 32;     // LU
constexpr int PF_TINY_MAXN = 16;  // Parlett-Reid
int tiny_padded(int n);
int launch_lu_tiny(const float* A, int n, int64_t batch, float* sign, float* logabs, float* lu, int* perm,
                   hipStream_t s);
int launch_pf_tiny(const float* A, int n, int skew, int64_t batch, float* sign, float* logabs, float* gbuf, float* d,
                   int* perm, hipStream_t s);
// sign / logabs (bit-identical to launch_lu_tiny) and A^-T in one pass (Gauss-Jordan).
int launch_lu_tiny_inv(const float* A, int n, int64_t batch, int zero_singular, float* sign, float* logabs,
                       float* invT, hipStream_t s);

// n <= 128 fused kernels (one workgroup per matrix).
int lu_small_padded(int n);
int pf_small_padded(int n);
// slogdet; with lu != nullptr also the packed LU of P A (B, N, N) in the final row order
// and perm (B, N) with (P A)[c] = A[perm[c]], N = lu_small_padded(n).
int launch_lu_small(const float* A, int n, int64_t batch, float* sign, float* logabs, float* lu,
                    int* perm, hipStream_t s);
// slogpf; with gbuf != nullptr also the Parlett-Reid factors: gbuf (B, N/16, N, 16) with
// block k's tau_t / w_t in columns 2t / 2t+1 indexed by original row, d (B, N/2) the pair
// pivots, perm (B, N) final position -> original row. N = pf_small_padded(n).
int launch_pf_small(const float* A, int n, int skew, int64_t batch, float* sign, float* logabs,
                    float* gbuf, float* d, int* perm, hipStream_t s);

// 128 < n <= LU_LARGE_MAXN: blocked LU in a workspace (see lu_large.hip). W_out / g0_out
// return the packed LU (B, N, N) and, with parts, the composed row map (B, N),
// N = lu_large_padded. With W_ext (and, with parts, g0_ext) the LU and the row map are
// formed in those caller buffers instead of the workspace (external = true sizes it).
constexpr int LU_LARGE_MAXN = 8192;
int lu_large_padded(int n);
size_t lu_large_workspace(int64_t batch, int n, bool parts, bool external = false);
// x3 != 0 runs the trailing updates in the split-bf16x3 mode (FX_PREC_BF16X3); lu_block is
// FX_LU_BLOCK_TABLE, FX_LU_BLOCK_64 or FX_LU_BLOCK_128 (block pairs from the table, never,
// always). split = false keeps every launch on s (no side stream).
int launch_lu_large(const float* A, int n, int64_t batch, float* sign, float* logabs, void* ws,
                    size_t ws_bytes, bool parts, float** W_out, int** g0_out, hipStream_t s,
                    float* W_ext = nullptr, int* g0_ext = nullptr, int x3 = 0, int lu_block = FX_LU_BLOCK_TABLE,
                    bool split = true);

// A^-T from the packed LU (B, N, N) and row map g0 (B, N) into invT (B, n, n); LU is
// overwritten when in_place and N is a power-of-two multiple of 32 (inverse.hip).
int inv_padded(int N);
size_t lu_inverse_workspace(int64_t batch, int N, bool need_copy);
// With scale != nullptr every member's invT is multiplied by scale[b] (the non-finite
// check applies to the unscaled values).
// x3 != 0 runs the GEMMs in the split-bf16x3 mode.
int launch_lu_inverse(float* LU, const int* g0, int N, int n, int64_t batch, const float* sign,
                      int zero_singular, float* invT, bool in_place, void* ws, size_t ws_bytes,
                      hipStream_t s, const float* scale = nullptr, int x3 = 0);

// 128 < n <= PF_LARGE_MAXN Parlett-Reid (pf_large.hip); with gbuf the factors
// (B, N/PB, N, PB) by original row (PB = pf_large_block_cols(N)), d (B, N/2) and perm (B, N).
constexpr int PF_LARGE_MAXN = 8192;
int pf_large_padded(int n);
int pf_large_block_cols(int N);  // columns per factor chunk: 32 for N <= 2048, 16 to 4096, 8 above
size_t pf_large_workspace(int64_t batch, int n, bool fact);
int launch_pf_large(const float* A, int n, int skew, int64_t batch, float* sign, float* logabs,
                    float* gbuf, float* dout, int* perm, void* ws, size_t ws_bytes, hipStream_t s);

// In-place unit-lower (and upper) triangular inverses of a packed (B, Ninv, Ninv) buffer;
// with active != nullptr only the members with active[b] != 0 are processed.
int launch_tri_inverse(float* T, int Ninv, int64_t batch, float* Tmp, bool upper, hipStream_t s,
                       const int* active = nullptr, int x3 = 0);
int launch_unit_lower_inverse(float* T, int Ninv, int64_t batch, float* Tmp, hipStream_t s,
                              const int* active = nullptr, int x3 = 0);

// S^-1 (adjugate = 0) or pf(S) S^-1 (adjugate != 0) as (B, n, n) from the Parlett-Reid
// factors (gbuf with PB columns per block, d, perm), read only; every member multiplied
// by scale[b] when scale is given.
size_t pf_inverse_workspace(int64_t batch, int N);
int launch_pf_inverse(const float* gbuf, int PB, const float* d, const int* perm, int N, int n, int64_t batch,
                      int adjugate, float* out, void* ws, size_t ws_bytes, hipStream_t s,
                      const float* scale = nullptr, int x3 = 0);

// parity[b] = parity (0 even, 1 odd) of the permutation perm[b] of 0..N-1, N <= 2048.
int launch_perm_parity(const int* perm, int N, int64_t batch, int* parity, hipStream_t s);

// det adjugate (adjugate.hip): prep reads the packed LU (before the in-place inverse
// overwrites it) and returns the per-member scale of the inverse's scatter; finish
// turns the members with one or two zero pivots into their rank-1 adjugate.
size_t det_adjugate_workspace(int64_t batch, int n);
int launch_det_adjugate_prep(const float* LU, const int* g0, int N, int n, int64_t batch, void* ws,
                             float** scale_out, hipStream_t s);
int launch_det_adjugate_finish(int n, int64_t batch, void* ws, float* G, hipStream_t s);

// ------------------------------------------------------------------ batched GEMM
// Masks apply to op(X) in global coordinates (row + off*r, col + off*c): elements
// outside the triangle read as zero (unit diagonal for the *_UNIT kinds).
enum { MASK_NONE = 0, MASK_LOWER_UNIT = 1, MASK_UPPER = 2, MASK_UPPER_UNIT = 3 };

struct GemmDesc {
  const float* A;
  const float* B;
  float* C;
  int64_t sA, sB, sC;     // stride of the batch index (blockIdx.y)
  int64_t sA2, sB2, sC2;  // stride of the second batch index (blockIdx.z)
  int lda, ldb, ldc;
  int M, N, K;
  float alpha, beta;
  int transA, transB;  // op(A) = A (M x K, row-major) or A^T (A stored K x M)
  int maskA, maskB;
  int offAr, offAc, offBr, offBc;
  int lower_only;  // only tiles on/below the diagonal; C[j][i] = mirror * C[i][j]
  float mirror;
  int xcd8;  // set by launch_gemm: the batch is a multiple of 8 (XCD-aware tile order)
  int x3;    // products in the split-bf16x3 mode (FX_PREC_BF16X3) instead of fp32 MFMA
  const int* active;  // optional (batch,) mask: members with active[b] == 0 are skipped
  // Optional transposed, row-permuted output in place of C (64 x 64 tiles, one batch
  // index, not lower_only): tout[b][g0[b][j]][i] = scale[b] * alpha (op(A) op(B))[i][j]
  // for i < nout and g0[b][j] < nout (tout (batch, nout, nout), g0 (batch, N)), and
  // flags[b][tile] = the tile holds a non-finite value (tiles row-major, ceil(M/64) x
  // ceil(N/64) per member). scale is optional.
  float* tout;
  const int* g0;
  int nout;
  const float* scale;
  int* flags;
  // Optional row transform of B (maskB must be MASK_NONE, transB 0): op(B) row k is
  // s_k B[k ^ 1] with s_k = bscale[b][k / 2], negated for odd k (bscale (batch, K / 2)).
  const float* bscale;
};

// C = alpha op(A) op(B) + beta C for every (batch, second-batch) index.
int launch_gemm(const GemmDesc& d, int64_t batch, int nb2, hipStream_t s);

// float64 blocked LU (sign, logabs) for the orders above the register kernels (lu64_impl.inc)
size_t lu64_workspace(int64_t batch, int n);
int launch_lu64(const double* A, int n, int64_t batch, double* sign, double* logabs, void* ws, size_t ws_bytes,
                hipStream_t s);
// ... and the inverse from the same factorisation (A skew-symmetrised when skew): out =
// A^-T (out_t) or A^-1, times ssign exp(slog) when ssign is given, zero where gate
// (default: the factorisation's own sign) is 0 or the result is not finite; sign / logabs
// those of the factorisation.
size_t lu64_inverse_workspace(int64_t batch, int n);
int launch_lu64_inverse(const double* A, int n, int skew, int64_t batch, double* sign, double* logabs,
                        const double* gate, const double* ssign, const double* slog, double* out, int out_t,
                        void* ws, size_t ws_bytes, hipStream_t s);
// float64 Parlett-Reid sign / logabs for n above the register kernels (lu64_impl.inc): 16 pair
// steps per panel, the trailing update on the fp64 MFMA
size_t pr64_workspace(int64_t batch, int n);
int launch_pr64_blocked(const double* A, int n, int skew, int64_t batch, double* sign, double* logabs, void* ws,
                        size_t ws_bytes, hipStream_t s, double* spread = nullptr);

// float64 Pfaffian adjugate pf(S) S^-1 (cplx.hip; zero for odd n); psign / plog / spread:
// the Parlett-Reid run's sign, log|pf| and pair-pivot spread (launch_pr64's) of the same S
size_t pf_adjugate_f64_ws(int64_t batch, int n);
int pf_adjugate_f64(const double* a, int64_t batch, int n, int skew, double* g, const double* psign,
                    const double* plog, const double* spread, void* ws, size_t wsb, hipStream_t s);

// float32 above LU_LARGE_MAXN / PF_LARGE_MAXN up to GEN32_MAXN (cplx.hip): the blocked
// kernels of lu64_impl.inc on float storage; the caller checks the arguments. slogdet_parts:
// A^-T zero for singular members; det_parts: adj(A)^T; slogpf_parts: S^-1 (zero where
// pf = 0) or, with adjugate, pf(S) S^-1.
constexpr int GEN32_MAXN = 16384;
size_t gen32_slogdet_ws(int64_t batch, int n);
int gen32_slogdet(const float* a, int64_t batch, int n, float* sign, float* logabs, void* ws, size_t wsb,
                  hipStream_t s);
size_t gen32_slogdet_parts_ws(int64_t batch, int n);
int gen32_slogdet_parts(const float* a, int64_t batch, int n, float* sign, float* logabs, float* inv_t, void* ws,
                        size_t wsb, hipStream_t s);
size_t gen32_det_parts_ws(int64_t batch, int n);
int gen32_det_parts(const float* a, int64_t batch, int n, float* sign, float* logabs, float* adj_t, void* ws,
                    size_t wsb, hipStream_t s);
size_t gen32_slogpf_ws(int64_t batch, int n);
int gen32_slogpf(const float* a, int64_t batch, int n, int skew, float* sign, float* logabs, void* ws, size_t wsb,
                 hipStream_t s);
size_t gen32_slogpf_parts_ws(int64_t batch, int n);
int gen32_slogpf_parts(const float* a, int64_t batch, int n, int skew, int adjugate, float* sign, float* logabs,
                       float* g, void* ws, size_t wsb, hipStream_t s);

// complex64's product mode for the calls of this thread: 1 while a complex64 entry point
// called with FX_PREC_IEEE runs (the blocked products as fp32 MFMA products), else 0 (the
// products on the fp64 MFMA, complex64 widened). CxPrecPin sets it for one call.
int cx32_ieee();
struct CxPrecPin {
  explicit CxPrecPin(int ieee);
  ~CxPrecPin();
  CxPrecPin(const CxPrecPin&) = delete;
  CxPrecPin& operator=(const CxPrecPin&) = delete;
  int old_;
};

}  // namespace fx
