// Blocked LU with partial pivoting (sign, logabs) for the float64 and complex kinds above
// the orders of their one-workgroup kernels, n <= 8192: the reference's `_lu_core` block
// loop (src/fermix/_lu.py:543-611: panel, row swaps, U rows, trailing GEMM) for the 64-bit
// and complex fields, with the trailing update on the fp64 MFMA (v_mfma_f64_16x16x4f64;
// a complex product as four real ones, complex64 operands widened to double). Every
// kernel is generic over the field F (double, cx<float>, cx<double>: field.h); the pivot
// magnitude of a complex value is |re| + |im|, its sign the product of the pivots'
// phases d / |d|. The matrix is copied into a workspace of padded order N (a
// multiple of 32, identity padding) and factored in place, 32 columns per block:
//   1. lu64_panel_reg_kernel / lu64_panel_kernel (one workgroup per matrix): the 32
//      columns of rows >= r0, one column step at a time -- the pivot is the row of
//      largest |x| among rows >= c (lowest row on ties), swapped into row c over the
//      panel's columns, then the multipliers and the rank-1 update of the panel's
//      remaining columns; with the rows in registers up to 512 rows (1024 for 8-byte
//      elements), else in memory;
//   2. lu64_rows_kernel<0> (matrix x 256 trailing columns): the panel's row swaps on the
//      trailing columns and U12 = L11^-1 A12 by forward substitution (L11 in LDS);
//   3. lu64_gemm_kernel / lucx_gemm_kernel (matrix x 64 x 64 tile): A22 -= L21 U12 at
//      K = 32, the products in accumulators of their own, subtracted from A22 at the end;
//   4. lu64_finish_kernel: sign = (-1)^swaps * prod sign(d), logabs = sum log|d| in
//      pivot order (one wave, lane-strided partial sums and a fixed tree).
// The column steps of a panel are latency-bound (two or three workgroup barriers each);
// the work that grows as n^3 runs on the MFMA in many workgroups per matrix. The inverse
// (blk_lu_inverse: A^-T, S^-1, det A^-T, pf S^-1) solves with the same row and GEMM
// kernels, and the blocked Parlett-Reid below (blk_pr: slogpf) updates its trailing
// matrix with the same GEMMs.
#include <algorithm>

#include "common.h"
#include "fermix_internal.h"
#include "field.h"

namespace fx {
namespace {

constexpr int P64 = 32;    // panel width
constexpr int NT64 = 256;  // threads of the panel and U-row workgroups

typedef double v4d __attribute__((ext_vector_type(4)));

int lu64_padded(int n) { return (n + P64 - 1) / P64 * P64; }

template <class F>
using RealOf = typename Fd<F>::R;

template <class F>
constexpr bool is_real() {
  return sizeof(F) == sizeof(RealOf<F>);
}

// W (B, N, N) = A (B, n, n) with identity padding (skew: (A - A^T) / 2), or, with pfpad
// (n even), padding by 2 x 2 blocks [[0, 1], [-1, 0]] on the diagonal (skew, Pfaffian 1);
// a grid-stride loop over B N N elements.
template <class F>
__global__ void lu64_copy_kernel(const F* __restrict__ A, int n, int skew, F* __restrict__ W, int N, int64_t total,
                                 int pfpad) {
  using D = Fd<F>;
  const int64_t NN = (int64_t)N * N;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = e / NN;
    const int64_t f = e - b * NN;
    const int r = (int)(f / N), c = (int)(f - (int64_t)r * N);
    const F* Ab = A + b * (int64_t)n * n;
    F v = pfpad ? (c == (r ^ 1) ? ((r & 1) ? D::neg(D::one()) : D::one()) : D::zero()) : (r == c ? D::one() : D::zero());
    if (r < n && c < n) v = skew ? half_diff(Ab[(int64_t)r * n + c], Ab[(int64_t)c * n + r]) : Ab[(int64_t)r * n + c];
    W[e] = v;
  }
}

// Panel of columns r0 .. r0 + 31, rows r0 .. N - 1, in place; ipiv / d: the pivot row and
// pivot of each column; nsw: the block's row swaps.
template <class F, int NT>
__global__ __launch_bounds__(NT) void lu64_panel_kernel(F* __restrict__ W, int N, int r0, int* __restrict__ ipiv,
                                                        F* __restrict__ dpiv, int* __restrict__ nsw) {
  using D = Fd<F>;
  __shared__ unsigned long long redk[2][NT / 64];
  __shared__ int redr[2][NT / 64];
  __shared__ F prow[P64];
  const int64_t b = blockIdx.x;
  F* Wb = W + b * (int64_t)N * N;
  const int tid = threadIdx.x;
  int swaps = 0;
  for (int j = 0; j < P64; ++j) {
    const int c = r0 + j;
    unsigned long long k = 0;
    int row = 0x7fffffff;
    for (int r = c + tid; r < N; r += NT) take_better(k, row, D::key(Wb[(int64_t)r * N + c]), r);
    const int p = block_argmax<NT>(k, row, redk[j & 1], redr[j & 1]);  // >= c: every key is >= 1
    if (p != c) {
      if (tid < P64) {
        F* Rc = Wb + (int64_t)c * N + r0;
        F* Rp = Wb + (int64_t)p * N + r0;
        const F u = Rc[tid], v = Rp[tid];
        Rc[tid] = v;
        Rp[tid] = u;
      }
      ++swaps;
    }
    __syncthreads();
    if (tid < P64) prow[tid] = Wb[(int64_t)c * N + r0 + tid];
    __syncthreads();
    const F d = prow[j];
    if (tid == 0) {
      ipiv[b * N + c] = p;
      dpiv[b * N + c] = d;
    }
    const F rd = D::rcp(d);  // a zero pivot: its column is zero below, rd = 0
    for (int r = c + 1 + tid; r < N; r += NT) {
      F* R = Wb + (int64_t)r * N + r0;
      const F l = D::mul(R[j], rd);
      R[j] = l;
      for (int q = j + 1; q < P64; ++q) R[q] = D::fms(R[q], l, prow[q]);
    }
    __syncthreads();
  }
  if (tid == 0) nsw[b * (N / P64) + r0 / P64] = swaps;
}

// The same panel with its rows in registers (m = N - r0 <= NTR: thread t holds row r0 + t,
// columns r0 .. r0 + 31; NTR = 1024 only for 8-byte elements, whose 32-entry rows fit the
// 128 registers of a 1024-thread workgroup): per column step one workgroup argmax, the
// pivot row and row c
// posted through LDS and exchanged by their owners, then the multipliers and the rank-1
// update in registers -- the arithmetic of lu64_panel_kernel element for element (same
// pivots, same rounding), without its global stores and reloads between column steps.
template <class F, int NTR>
__global__ __launch_bounds__(NTR) void lu64_panel_reg_kernel(F* __restrict__ W, int N, int r0,
                                                             int* __restrict__ ipiv, F* __restrict__ dpiv,
                                                             int* __restrict__ nsw) {
  using D = Fd<F>;
  __shared__ unsigned long long redk[2][NTR / 64];
  __shared__ int redr[2][NTR / 64];
  __shared__ F prow[P64], crow[P64];
  const int64_t b = blockIdx.x;
  F* Wb = W + b * (int64_t)N * N;
  const int tid = threadIdx.x;
  const int r = r0 + tid;
  const bool own = r < N;
  F a[P64];
#pragma unroll
  for (int q = 0; q < P64; ++q) a[q] = own ? Wb[(int64_t)r * N + r0 + q] : D::zero();
  int swaps = 0;
  // column steps with compile-time j (the row stays in registers, no dynamic index)
  static_for<0, P64>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    const int c = r0 + j;
    const unsigned long long k = own && tid >= j ? D::key(a[j]) : 0ull;
    const int p = block_argmax<NTR>(k, own ? r : 0x7fffffff, redk[j & 1], redr[j & 1]);  // >= c
    if (r == p) {
#pragma unroll
      for (int q = 0; q < P64; ++q) prow[q] = a[q];
    }
    if (tid == j && p != c) {
#pragma unroll
      for (int q = 0; q < P64; ++q) crow[q] = a[q];
    }
    __syncthreads();
    if (p != c) {
      ++swaps;
      if (tid == j) {
#pragma unroll
        for (int q = 0; q < P64; ++q) a[q] = prow[q];
      } else if (r == p) {
#pragma unroll
        for (int q = 0; q < P64; ++q) a[q] = crow[q];
      }
    }
    const F d = prow[j];
    if (tid == 0) {
      ipiv[b * N + c] = p;
      dpiv[b * N + c] = d;
    }
    if (own && tid > j) {
      const F l = D::mul(a[j], D::rcp(d));
      a[j] = l;
#pragma unroll
      for (int q = j + 1; q < P64; ++q) a[q] = D::fms(a[q], l, prow[q]);
    }
  });
  if (own) {
#pragma unroll
    for (int q = 0; q < P64; ++q) Wb[(int64_t)r * N + r0 + q] = a[q];
  }
  if (tid == 0) nsw[b * (N / P64) + r0 / P64] = swaps;
}

// 32 rows r0 .. r0 + 31 of a target matrix T, columns c0 + 256 cb + tid (< cend), against
// the diagonal block D = W[r0 .. r0 + 31][r0 .. r0 + 31] of the factorisation:
//   MODE 0 / 1: the panel's row swaps (row r0 + j with ipiv[r0 + j] >= r0 + j, in order),
//     then the forward substitution with the unit lower part of D (MODE 0: T = W, the
//     U rows of the trailing columns; MODE 1: T = Y, the forward solve of L Y = P I);
//   MODE 2: the backward substitution with the upper part of D (the solve U X = Y).
template <class F, int MODE>
__global__ __launch_bounds__(NT64) void lu64_rows_kernel(const F* __restrict__ W, F* __restrict__ T, int N, int r0,
                                                         const int* __restrict__ ipiv, int c0, int cend, int ncb) {
  using Q = Fd<F>;
  __shared__ F D[P64][P64 + 1];
  const int64_t b = blockIdx.x / ncb;
  const int cb = (int)(blockIdx.x - b * ncb);
  const F* Wb = W + b * (int64_t)N * N;
  F* Tb = T + b * (int64_t)N * N;
  const int tid = threadIdx.x;
  for (int e = tid; e < P64 * P64; e += NT64) {
    const int i = e / P64, k = e % P64;
    D[i][k] = Wb[(int64_t)(r0 + i) * N + r0 + k];
  }
  __syncthreads();
  const int col = c0 + NT64 * cb + tid;
  if (col >= cend) return;
  F x[P64];
#pragma unroll
  for (int i = 0; i < P64; ++i) x[i] = Tb[(int64_t)(r0 + i) * N + col];
  if constexpr (MODE != 2) {
    const int* ip = ipiv + b * N + r0;
    // rows beyond the block rows exchange with the column's entries below
#pragma unroll
    for (int j = 0; j < P64; ++j) {
      const int p = ip[j];
      if (p != r0 + j) {
        if (p < r0 + P64) {
          F t = x[j];
#pragma unroll
          for (int i = j + 1; i < P64; ++i)
            if (p - r0 == i) {
              const F u = x[i];
              x[i] = t;
              t = u;
            }
          x[j] = t;
        } else {
          F* e = Tb + (int64_t)p * N + col;
          const F u = *e;
          *e = x[j];
          x[j] = u;
        }
      }
    }
#pragma unroll
    for (int i = 1; i < P64; ++i) {
      F v = x[i];
#pragma unroll
      for (int k = 0; k < i; ++k) v = Q::fms(v, D[i][k], x[k]);
      x[i] = v;
    }
  } else {
#pragma unroll
    for (int i = P64 - 1; i >= 0; --i) {
      F v = x[i];
#pragma unroll
      for (int k = i + 1; k < P64; ++k) v = Q::fms(v, D[i][k], x[k]);
      x[i] = Q::div(v, D[i][i]);
    }
  }
#pragma unroll
  for (int i = 0; i < P64; ++i) Tb[(int64_t)(r0 + i) * N + col] = x[i];
}

// C -= A B with K = 32: A = rows 0 .. M - 1 of a 32-column block, B = its 32 rows of
// columns 0 .. NC - 1, C = M x NC (every operand given at its first element in matrix 0,
// with its own row and matrix strides). One 64 x 64 tile per workgroup (tiles t = tile row *
// ntc + tile column), four waves of 32 x 32, each as 2 x 2 16 x 16 fp64 MFMA
// accumulators over eight K = 4 steps; the products in accumulators of their own,
// subtracted from C in fp64 at the end. Lane l supplies A[l % 16][l / 16] and
// B[l / 16][l % 16]; accumulator element v of lane l is row l / 16 + 4 v, column l % 16
// (measured with a one-wave probe: unlike the fp32 16x16x4 layout, a lane's four rows
// are 4 apart). Serves the trailing update A22 -= L21 U12 and both solves' updates.
template <class E>
__global__ __launch_bounds__(256) void lu64_gemm_kernel(const E* __restrict__ A, int lda, int64_t sA,
                                                        const E* __restrict__ Bm, int ldb, int64_t sB,
                                                        E* __restrict__ C, int ldc, int64_t sC, int M, int NC,
                                                        int ntr, int ntc) {
  __shared__ double As[64][P64 + 1];
  __shared__ double Bs[P64][64 + 1];
  const int nt = ntr * ntc;
  const int64_t b = blockIdx.x / nt;
  const int t = (int)(blockIdx.x - b * nt);
  const int i0 = 64 * (t / ntc), j0 = 64 * (t % ntc);
  const E* Ab = A + b * sA;
  const E* Bb = Bm + b * sB;
  E* Cb = C + b * sC;
  const int tid = threadIdx.x;
  for (int e = tid; e < 64 * P64; e += 256) {
    const int i = e / P64, k = e % P64;
    As[i][k] = i0 + i < M ? (double)Ab[(int64_t)(i0 + i) * lda + k] : 0.0;
    const int kk = e / 64, j = e % 64;
    Bs[kk][j] = j0 + j < NC ? (double)Bb[(int64_t)kk * ldb + j0 + j] : 0.0;
  }
  __syncthreads();
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  const int l16 = lane & 15, lk = lane >> 4;
  v4d acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[a][c][v] = 0.0;
#pragma unroll
  for (int s = 0; s < P64 / 4; ++s) {
    double av[2], bv[2];
#pragma unroll
    for (int a = 0; a < 2; ++a) av[a] = As[wm + 16 * a + l16][4 * s + lk];
#pragma unroll
    for (int c = 0; c < 2; ++c) bv[c] = Bs[4 * s + lk][wn + 16 * c + l16];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int c = 0; c < 2; ++c) acc[a][c] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[a], bv[c], acc[a][c], 0, 0, 0);
  }
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int col = j0 + wn + 16 * c + l16;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = i0 + wm + 16 * a + lk + 4 * v;
        if (row < M && col < NC) {
          E* e = Cb + (int64_t)row * ldc + col;
          *e = E((double)*e - acc[a][c][v]);
        }
      }
    }
}

// The complex C -= A B (K = 32, same tiling and lane layout): each operand staged as its
// real and imaginary planes in double (K in two halves of 16, 34 KiB of LDS), four real
// MFMA products per complex one, Re = Ar Br - Ai Bi and Im = Ar Bi + Ai Br in accumulators
// of their own, subtracted from C at the end (rounded once to T).
template <class T>
__global__ __launch_bounds__(256) void lucx_gemm_kernel(const cx<T>* __restrict__ A, int lda, int64_t sA,
                                                        const cx<T>* __restrict__ Bm, int ldb, int64_t sB,
                                                        cx<T>* __restrict__ C, int ldc, int64_t sC, int M, int NC,
                                                        int ntr, int ntc) {
  __shared__ double Ar[64][17], Ai[64][17];
  __shared__ double Br[16][65], Bi[16][65];
  const int nt = ntr * ntc;
  const int64_t b = blockIdx.x / nt;
  const int t = (int)(blockIdx.x - b * nt);
  const int i0 = 64 * (t / ntc), j0 = 64 * (t % ntc);
  const cx<T>* Ab = A + b * sA;
  const cx<T>* Bb = Bm + b * sB;
  cx<T>* Cb = C + b * sC;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  const int l16 = lane & 15, lk = lane >> 4;
  v4d cr[2][2], ci[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        cr[a][c][v] = 0.0;
        ci[a][c][v] = 0.0;
      }
  for (int h = 0; h < 2; ++h) {
    if (h) __syncthreads();
    for (int e = tid; e < 64 * 16; e += 256) {
      const int i = e / 16, k = e % 16;
      const cx<T> u = i0 + i < M ? Ab[(int64_t)(i0 + i) * lda + 16 * h + k] : cx<T>{T(0), T(0)};
      Ar[i][k] = u.re;
      Ai[i][k] = u.im;
      const int kk = e / 64, j = e % 64;
      const cx<T> w = j0 + j < NC ? Bb[(int64_t)(16 * h + kk) * ldb + j0 + j] : cx<T>{T(0), T(0)};
      Br[kk][j] = w.re;
      Bi[kk][j] = w.im;
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      double ar[2], ai[2], br[2], bi[2];
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        ar[a] = Ar[wm + 16 * a + l16][4 * s + lk];
        ai[a] = Ai[wm + 16 * a + l16][4 * s + lk];
      }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        br[c] = Br[4 * s + lk][wn + 16 * c + l16];
        bi[c] = Bi[4 * s + lk][wn + 16 * c + l16];
      }
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          cr[a][c] = __builtin_amdgcn_mfma_f64_16x16x4f64(ar[a], br[c], cr[a][c], 0, 0, 0);
          cr[a][c] = __builtin_amdgcn_mfma_f64_16x16x4f64(-ai[a], bi[c], cr[a][c], 0, 0, 0);
          ci[a][c] = __builtin_amdgcn_mfma_f64_16x16x4f64(ar[a], bi[c], ci[a][c], 0, 0, 0);
          ci[a][c] = __builtin_amdgcn_mfma_f64_16x16x4f64(ai[a], br[c], ci[a][c], 0, 0, 0);
        }
    }
  }
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int col = j0 + wn + 16 * c + l16;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = i0 + wm + 16 * a + lk + 4 * v;
        if (row < M && col < NC) {
          cx<T>* e = Cb + (int64_t)row * ldc + col;
          const cx<T> o = *e;
          *e = cx<T>{T((double)o.re - cr[a][c][v]), T((double)o.im - ci[a][c][v])};
        }
      }
    }
}

// (sign, logabs) per matrix, one wave each: lane-strided partial sums of log|d| over the
// pivots in order, a fixed xor tree; the sign from the count of negative pivots and swaps
// (complex: the product of the pivots' phases, times (-1)^swaps).
template <class F>
__global__ void lu64_finish_kernel(const F* __restrict__ dpiv, const int* __restrict__ nsw, int N,
                                   F* __restrict__ sign, RealOf<F>* __restrict__ logabs, int64_t batch) {
  using D = Fd<F>;
  const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (b >= batch) return;
  double lg = 0.0;
  double2 ph = make_double2(1.0, 0.0);
  int neg = 0, zero = 0;
  for (int i = lane; i < N; i += 64) {
    const F d = dpiv[b * N + i];
    zero |= D::is0(d);
    if constexpr (is_real<F>()) {
      neg += D::to2(d).x < 0.0;
      lg += !D::is0(d) ? log(fabs(D::to2(d).x)) : 0.0;
    } else if (!D::is0(d)) {
      const double2 u = D::to2(d);
      const double m = hypot(u.x, u.y);
      lg += log(m);
      ph = c2mul(ph, make_double2(u.x / m, u.y / m));
    }
  }
  int sw = 0;
  for (int i = lane; i < N / P64; i += 64) sw += nsw[b * (N / P64) + i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    lg += __shfl_xor(lg, off);
    neg += __shfl_xor(neg, off);
    zero |= __shfl_xor(zero, off);
    sw += __shfl_xor(sw, off);
    if constexpr (!is_real<F>()) ph = c2mul(ph, make_double2(__shfl_xor(ph.x, off), __shfl_xor(ph.y, off)));
  }
  if (lane == 0) {
    const double par = ((neg + sw) & 1) ? -1.0 : 1.0;
    sign[b] = zero ? D::zero() : D::from(make_double2(par * ph.x, par * ph.y));
    logabs[b] = zero ? RealOf<F>(-INFINITY) : RealOf<F>(lg);
  }
}

// out[b][i][j] (i, j < n) = scale_b X[j][i] (out_t) or scale_b X[i][j], X the solve's
// N x N result, scale_b = ssign_b exp(slog_b) when ssign is given; zero where gate[b] == 0
// (the member's own sign, or a caller's gate); any non-finite value of a member raises
// flag[b] (every writer stores 1).
template <class F>
__global__ void lu64_out_kernel(const F* __restrict__ X, int N, int n, int out_t, const F* __restrict__ gate,
                                const F* __restrict__ ssign, const RealOf<F>* __restrict__ slog, F* __restrict__ out,
                                int* __restrict__ flag, int64_t total) {
  using D = Fd<F>;
  const int64_t nn = (int64_t)n * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = e / nn;
    const int64_t f = e - b * nn;
    const int i = (int)(f / n), j = (int)(f - (int64_t)i * n);
    F v = D::zero();
    if (!D::is0(gate[b])) {
      v = X[b * (int64_t)N * N + (out_t ? (int64_t)j * N + i : (int64_t)i * N + j)];
      if (ssign) {
        const double2 sg = D::to2(ssign[b]);
        const double m = exp((double)slog[b]);
        v = D::scale(v, make_double2(sg.x * m, sg.y * m));
      }
      if (!D::finite(v)) flag[b] = 1;
    }
    out[e] = v;
  }
}

template <class F>
__global__ void lu64_zero_kernel(F* __restrict__ out, int n, const int* __restrict__ flag, int64_t total) {
  const int64_t nn = (int64_t)n * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x)
    if (flag[e / nn]) out[e] = Fd<F>::zero();
}

template <class F>
__global__ void lu64_fill_kernel(F* __restrict__ Y, int N, int* __restrict__ flag, int64_t batch, int64_t total) {
  const int64_t NN = (int64_t)N * N;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t f = e % NN;
    Y[e] = (f / N == f % N) ? Fd<F>::one() : Fd<F>::zero();
    if (f == 0) flag[e / NN] = 0;
  }
}

unsigned grid_of(int64_t total) { return (unsigned)std::min<int64_t>((total + 255) / 256, 1 << 20); }

size_t al256(size_t x) { return (x + 255) / 256 * 256; }

template <class F>
struct Lu64Bufs {
  F* W;
  int* ipiv;
  F* dpiv;
  int* nsw;
};

template <class F>
Lu64Bufs<F> lu64_take(char*& p, int64_t batch, int N) {
  auto take = [&](size_t x) {
    char* q = p;
    p += al256(x);
    return (void*)q;
  };
  Lu64Bufs<F> f;
  f.W = (F*)take((size_t)batch * N * N * sizeof(F));
  f.ipiv = (int*)take((size_t)batch * N * 4);
  f.dpiv = (F*)take((size_t)batch * N * sizeof(F));
  f.nsw = (int*)take((size_t)batch * (N / P64) * 4);
  return f;
}

// C -= A B (K = 32) over M x NC, operands at their first elements of matrix 0
template <class F>
int lu64_gemm_strided(const F* A, int lda, int64_t sA, const F* Bm, int ldb, int64_t sB, F* C, int ldc, int64_t sC,
                      int M, int NC, int64_t batch, hipStream_t s) {
  if (M <= 0 || NC <= 0) return FX_OK;
  const int ntr = (M + 63) / 64, ntc = (NC + 63) / 64;
  const dim3 grid((unsigned)(batch * ntr * ntc));
  if constexpr (is_real<F>())
    lu64_gemm_kernel<F><<<grid, 256, 0, s>>>(A, lda, sA, Bm, ldb, sB, C, ldc, sC, M, NC, ntr, ntc);
  else
    lucx_gemm_kernel<RealOf<F>><<<grid, 256, 0, s>>>(A, lda, sA, Bm, ldb, sB, C, ldc, sC, M, NC, ntr, ntc);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

// the same with every operand inside an N x N matrix of the batch
template <class F>
int lu64_gemm(const F* A, const F* Bm, F* C, int N, int M, int NC, int64_t batch, hipStream_t s) {
  const int64_t NN = (int64_t)N * N;
  return lu64_gemm_strided<F>(A, N, NN, Bm, N, NN, C, N, NN, M, NC, batch, s);
}

template <class F, int MODE>
int lu64_rows(const F* W, F* T, int N, int r0, const int* ipiv, int c0, int cend, int64_t batch, hipStream_t s) {
  if (cend <= c0) return FX_OK;
  const int ncb = (cend - c0 + NT64 - 1) / NT64;
  lu64_rows_kernel<F, MODE><<<dim3((unsigned)(batch * ncb)), NT64, 0, s>>>(W, T, N, r0, ipiv, c0, cend, ncb);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

// Copy (with skew symmetrisation) and factor in place; sign / logabs of the factorisation.
template <class F>
int lu64_factor(const F* A, int n, int skew, int64_t batch, const Lu64Bufs<F>& f, int N, F* sign, RealOf<F>* logabs,
                hipStream_t s) {
  const int64_t total = batch * (int64_t)N * N;
  lu64_copy_kernel<F><<<dim3(grid_of(total)), 256, 0, s>>>(A, n, skew, f.W, N, total, 0);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  for (int r0 = 0; r0 < N; r0 += P64) {
    bool in_regs = N - r0 <= 512;  // the panel's rows in registers
    if (in_regs) {
      lu64_panel_reg_kernel<F, 512><<<dim3((unsigned)batch), 512, 0, s>>>(f.W, N, r0, f.ipiv, f.dpiv, f.nsw);
    } else if constexpr (sizeof(F) <= 8) {
      in_regs = N - r0 <= 1024;
      if (in_regs)
        lu64_panel_reg_kernel<F, 1024><<<dim3((unsigned)batch), 1024, 0, s>>>(f.W, N, r0, f.ipiv, f.dpiv, f.nsw);
    }
    if (!in_regs)  // latency-bound column steps on rows in memory: more threads per matrix
      lu64_panel_kernel<F, 1024><<<dim3((unsigned)batch), 1024, 0, s>>>(f.W, N, r0, f.ipiv, f.dpiv, f.nsw);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
    const int r1 = r0 + P64;
    if (r1 >= N) break;
    int st = lu64_rows<F, 0>(f.W, f.W, N, r0, f.ipiv, r1, N, batch, s);
    if (st == FX_OK)
      st = lu64_gemm<F>(f.W + (int64_t)r1 * N + r0, f.W + (int64_t)r0 * N + r1, f.W + (int64_t)r1 * N + r1, N, N - r1,
                        N - r1, batch, s);
    if (st != FX_OK) return st;
  }
  lu64_finish_kernel<F><<<dim3((unsigned)((batch + 3) / 4)), 256, 0, s>>>(f.dpiv, f.nsw, N, sign, logabs, batch);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

// ---- blocked Parlett-Reid (slogpf of the float64 and complex kinds above their
// one-workgroup kernels)
//
// The reference's Parlett-Reid block loop (src/fermix/_pf.py:59-382: pair steps with a
// pivot search in the eliminated column, a symmetric row / column swap and the rank-2
// skew update S22 -= u v^T - v u^T, u = S[c, :] / S[c, c + 1], v = S[c + 1, :]) with the
// updates of 16 pair steps deferred: within a panel each pair step forms its two rows
// left-looking from the panel's earlier (u, v), and after the panel the trailing matrix
// takes all 16 at once, S22 -= [U, -V] [V, U]^T, a K = 32 product on the fp64 MFMA
// (the LU's GEMM kernels). The pair's Pfaffian factor is d = S[c, c + 1] after the swap;
// pf = (-1)^swaps prod d (no conjugation for the complex kinds).
constexpr int PRB = P64 / 2;  // pair steps per panel

// Panel of positions r0 .. r0 + 31 (one workgroup per matrix), W the full skew matrix of
// padded order N (rows and columns >= c + 1 swapped symmetrically, in place). Ar (B, N,
// 32): row x = (U[x][0..15], -V[x][0..15]); Bk (B, 32, N): rows 0..15 = V^T, 16..31 =
// U^T (the two operands of the trailing product, and the left-looking coefficients).
// rc: the current row c of the pair step; lacc / sacc / stat: log|pf| and the sign
// (phase) so far and the zero-pivot flag (a flagged member skips its later panels).
template <class F, int NT>
__global__ __launch_bounds__(NT) void pr64_panel_kernel(F* __restrict__ W, int N, int n, int r0, F* __restrict__ Ar,
                                                        F* __restrict__ Bk, F* __restrict__ rcg,
                                                        double* __restrict__ lacc, double2* __restrict__ sacc,
                                                        int* __restrict__ stat, double2* __restrict__ lr) {
  using D = Fd<F>;
  __shared__ unsigned long long redk[2][NT / 64];
  __shared__ int redr[2][NT / 64];
  __shared__ F cu[PRB], cv[PRB];
  const int64_t b = blockIdx.x;
  if (stat[b]) return;
  const int tid = threadIdx.x;
  F* Wb = W + b * (int64_t)N * N;
  F* Ab = Ar + b * (int64_t)N * P64;
  F* Bb = Bk + b * (int64_t)P64 * N;
  F* rc = rcg + b * (int64_t)N;
  double lg = 0.0;  // thread 0's running sums, in pivot order
  double2 sg = make_double2(1.0, 0.0);
  double lo = INFINITY, hi = -INFINITY;  // thread 0's range of log |d|
  bool sing = false;
  for (int p = 0; p < PRB; ++p) {
    const int c = r0 + 2 * p, q = c + 1;
    // row c: S[c][x] - sum_j (U[c][j] V[x][j] - V[c][j] U[x][j]) for x > c
    if (tid < p) {
      cu[tid] = Bb[(int64_t)(PRB + tid) * N + c];
      cv[tid] = Bb[(int64_t)tid * N + c];
    }
    __syncthreads();
    unsigned long long k = 0;
    int row = 0x7fffffff;
    for (int x = q + tid; x < N; x += NT) {
      F a = Wb[(int64_t)c * N + x];
      for (int j = 0; j < p; ++j) {
        a = D::fms(a, cu[j], Bb[(int64_t)j * N + x]);
        a = D::fms(a, D::neg(cv[j]), Bb[(int64_t)(PRB + j) * N + x]);
      }
      rc[x] = a;
      take_better(k, row, D::key(a), x);
    }
    // |S[x][c]| = |S[c][x]|: the largest, lowest index on ties, moves to position q
    const int pv = block_argmax<NT>(k, row, redk[p & 1], redr[p & 1]);
    if (pv != q) {
      for (int x = q + tid; x < N; x += NT) {
        const F u = Wb[(int64_t)pv * N + x], v = Wb[(int64_t)q * N + x];
        Wb[(int64_t)pv * N + x] = v;
        Wb[(int64_t)q * N + x] = u;
      }
      if (tid < P64) {
        const F u = Ab[(int64_t)pv * P64 + tid], v = Ab[(int64_t)q * P64 + tid];
        Ab[(int64_t)pv * P64 + tid] = v;
        Ab[(int64_t)q * P64 + tid] = u;
        const F y = Bb[(int64_t)tid * N + pv], z = Bb[(int64_t)tid * N + q];
        Bb[(int64_t)tid * N + pv] = z;
        Bb[(int64_t)tid * N + q] = y;
      }
      if (tid == 0) {
        const F u = rc[pv];
        rc[pv] = rc[q];
        rc[q] = u;
        sg = make_double2(-sg.x, -sg.y);
      }
      __syncthreads();
      for (int r = q + tid; r < N; r += NT) {
        const F u = Wb[(int64_t)r * N + pv], v = Wb[(int64_t)r * N + q];
        Wb[(int64_t)r * N + pv] = v;
        Wb[(int64_t)r * N + q] = u;
      }
    }
    __syncthreads();
    if (tid < p) {
      cu[tid] = Bb[(int64_t)(PRB + tid) * N + q];
      cv[tid] = Bb[(int64_t)tid * N + q];
    }
    __syncthreads();
    const F d = rc[q];
    if (D::is0(d)) {  // row c is zero beyond c: pf = 0
      sing = true;
      break;
    }
    const F rd = D::rcp(d);
    // u = row c / d, v = row q (left-looking like row c) beyond q; zero at positions <= q
    for (int x = r0 + tid; x < N; x += NT) {
      F u = D::zero(), v = D::zero();
      if (x > q) {
        F a = Wb[(int64_t)q * N + x];
        for (int j = 0; j < p; ++j) {
          a = D::fms(a, cu[j], Bb[(int64_t)j * N + x]);
          a = D::fms(a, D::neg(cv[j]), Bb[(int64_t)(PRB + j) * N + x]);
        }
        v = a;
        u = D::mul(rc[x], rd);
      }
      Ab[(int64_t)x * P64 + p] = u;
      Ab[(int64_t)x * P64 + PRB + p] = D::neg(v);
      Bb[(int64_t)p * N + x] = v;
      Bb[(int64_t)(PRB + p) * N + x] = u;
    }
    if (tid == 0) {
      D::acc(sg, lg, d);
      if (c < n) {  // the pairs of the matrix, not of its padding
        const double ld = log(D::mag(d));
        lo = fmin(lo, ld);
        hi = fmax(hi, ld);
      }
    }
    __syncthreads();
  }
  if (tid == 0) {
    if (sing) stat[b] = 1;
    lacc[b] += lg;
    sacc[b] = c2mul(sacc[b], sg);
    lr[b] = make_double2(fmin(lr[b].x, lo), fmax(lr[b].y, hi));
  }
}

// The same panel with the panel's (U, V) entries in registers (m = N - r0 <= NTR: thread
// t owns position r0 + t, its U / V entries of the pair steps so far and its entry of the
// current row c): the left-looking sums read registers instead of the (U, V) block, the
// swap exchanges the two positions' registers through LDS, and the block is written once
// at the end -- the arithmetic of pr64_panel_kernel element for element.
template <class F, int NTR>
__global__ __launch_bounds__(NTR) void pr64_panel_reg_kernel(F* __restrict__ W, int N, int n, int r0,
                                                             F* __restrict__ Ar,
                                                             F* __restrict__ Bk, double* __restrict__ lacc,
                                                             double2* __restrict__ sacc, int* __restrict__ stat,
                                                             double2* __restrict__ lr) {
  using D = Fd<F>;
  __shared__ unsigned long long redk[2][NTR / 64];
  __shared__ int redr[2][NTR / 64];
  __shared__ F cu[PRB], cv[PRB];
  __shared__ F xs[2][2 * PRB + 1];
  __shared__ F dsh;
  const int64_t b = blockIdx.x;
  if (stat[b]) return;
  const int tid = threadIdx.x;
  const int x = r0 + tid;
  const bool own = x < N;
  F* Wb = W + b * (int64_t)N * N;
  F u[PRB], v[PRB];
#pragma unroll
  for (int j = 0; j < PRB; ++j) u[j] = v[j] = D::zero();
  F rcx = D::zero();
  double lg = 0.0;  // thread 0's running sums, in pivot order
  double2 sg = make_double2(1.0, 0.0);
  double lo = INFINITY, hi = -INFINITY;  // thread 0's range of log |d|
  bool sing = false;
  static_for<0, PRB>([&](auto pc) {
    constexpr int p = decltype(pc)::value;
    if (sing) return;
    const int c = r0 + 2 * p, q = c + 1;
    if (x == c) {
#pragma unroll
      for (int j = 0; j < p; ++j) {
        cu[j] = u[j];
        cv[j] = v[j];
      }
    }
    __syncthreads();
    unsigned long long k = 0;
    if (own && x > c) {
      F a = Wb[(int64_t)c * N + x];
#pragma unroll
      for (int j = 0; j < p; ++j) {
        a = D::fms(a, cu[j], v[j]);
        a = D::fms(a, D::neg(cv[j]), u[j]);
      }
      rcx = a;
      k = D::key(a);
    }
    const int pv = block_argmax<NTR>(k, own && x > c ? x : 0x7fffffff, redk[p & 1], redr[p & 1]);
    if (pv != q) {
      for (int y = q + tid; y < N; y += NTR) {
        const F a = Wb[(int64_t)pv * N + y], e = Wb[(int64_t)q * N + y];
        Wb[(int64_t)pv * N + y] = e;
        Wb[(int64_t)q * N + y] = a;
      }
      if (x == pv || x == q) {
        F* o = xs[x == q];
#pragma unroll
        for (int j = 0; j < p; ++j) {
          o[j] = u[j];
          o[PRB + j] = v[j];
        }
        o[2 * PRB] = rcx;
      }
      if (tid == 0) sg = make_double2(-sg.x, -sg.y);
      __syncthreads();
      if (x == pv || x == q) {
        const F* o = xs[x == pv];
#pragma unroll
        for (int j = 0; j < p; ++j) {
          u[j] = o[j];
          v[j] = o[PRB + j];
        }
        rcx = o[2 * PRB];
      }
      for (int r = q + tid; r < N; r += NTR) {
        const F a = Wb[(int64_t)r * N + pv], e = Wb[(int64_t)r * N + q];
        Wb[(int64_t)r * N + pv] = e;
        Wb[(int64_t)r * N + q] = a;
      }
    }
    __syncthreads();
    if (x == q) {
#pragma unroll
      for (int j = 0; j < p; ++j) {
        cu[j] = u[j];
        cv[j] = v[j];
      }
      dsh = rcx;
    }
    __syncthreads();
    const F d = dsh;
    if (D::is0(d)) {  // row c is zero beyond c: pf = 0
      sing = true;
      return;
    }
    const F rd = D::rcp(d);
    F un = D::zero(), vn = D::zero();
    if (own && x > q) {
      F a = Wb[(int64_t)q * N + x];
#pragma unroll
      for (int j = 0; j < p; ++j) {
        a = D::fms(a, cu[j], v[j]);
        a = D::fms(a, D::neg(cv[j]), u[j]);
      }
      vn = a;
      un = D::mul(rcx, rd);
    }
    u[p] = un;
    v[p] = vn;
    if (tid == 0) {
      D::acc(sg, lg, d);
      if (c < n) {  // the pairs of the matrix, not of its padding
        const double ld = log(D::mag(d));
        lo = fmin(lo, ld);
        hi = fmax(hi, ld);
      }
    }
    __syncthreads();
  });
  if (own && !sing) {
    F* Ab = Ar + b * (int64_t)N * P64;
    F* Bb = Bk + b * (int64_t)P64 * N;
#pragma unroll
    for (int j = 0; j < PRB; ++j) {
      Ab[(int64_t)x * P64 + j] = u[j];
      Ab[(int64_t)x * P64 + PRB + j] = D::neg(v[j]);
      Bb[(int64_t)j * N + x] = v[j];
      Bb[(int64_t)(PRB + j) * N + x] = u[j];
    }
  }
  if (tid == 0) {
    if (sing) stat[b] = 1;
    lacc[b] += lg;
    sacc[b] = c2mul(sacc[b], sg);
    lr[b] = make_double2(fmin(lr[b].x, lo), fmax(lr[b].y, hi));
  }
}

__global__ void pr64_init_kernel(double* __restrict__ lacc, double2* __restrict__ sacc, int* __restrict__ stat,
                                 double2* __restrict__ lr, int64_t batch) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  lacc[b] = 0.0;
  sacc[b] = make_double2(1.0, 0.0);
  stat[b] = 0;
  lr[b] = make_double2(INFINITY, -INFINITY);
}

// (sign, logabs): the running sums, (0, -inf) for flagged members and for odd n (odd);
// spread (when given): log max |d| - log min |d| over the pair pivots, +inf where pf = 0
template <class F>
__global__ void pr64_finish_kernel(const double* __restrict__ lacc, const double2* __restrict__ sacc,
                                   const int* __restrict__ stat, const double2* __restrict__ lr, int odd,
                                   F* __restrict__ sign, RealOf<F>* __restrict__ logabs, double* __restrict__ spread,
                                   int64_t batch) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  const bool zero = odd || stat[b];
  sign[b] = zero ? Fd<F>::zero() : Fd<F>::from(sacc[b]);
  logabs[b] = zero ? RealOf<F>(-INFINITY) : RealOf<F>(lacc[b]);
  if (spread) spread[b] = zero ? INFINITY : lr[b].y - lr[b].x;
}

template <class F>
struct Pr64Bufs {
  F* W;
  F* Ar;
  F* Bk;
  F* rc;
  double* lacc;
  double2* sacc;
  int* stat;
  double2* lr;  // (min, max) of log |d| over the pair pivots so far
};

template <class F>
Pr64Bufs<F> pr64_take(char* p, int64_t batch, int N) {
  auto take = [&](size_t x) {
    char* q = p;
    p += al256(x);
    return (void*)q;
  };
  Pr64Bufs<F> f;
  f.W = (F*)take((size_t)batch * N * N * sizeof(F));
  f.Ar = (F*)take((size_t)batch * N * P64 * sizeof(F));
  f.Bk = (F*)take((size_t)batch * N * P64 * sizeof(F));
  f.rc = (F*)take((size_t)batch * N * sizeof(F));
  f.lacc = (double*)take((size_t)batch * 8);
  f.sacc = (double2*)take((size_t)batch * 16);
  f.stat = (int*)take((size_t)batch * 4);
  f.lr = (double2*)take((size_t)batch * 16);
  return f;
}

}  // namespace

template <class F>
size_t blk_lu_workspace(int64_t batch, int n) {
  if (batch <= 0 || n <= 0) return 0;
  const int N = lu64_padded(n);
  return al256((size_t)batch * N * N * sizeof(F)) + al256((size_t)batch * N * 4) +
         al256((size_t)batch * N * sizeof(F)) + al256((size_t)batch * (N / P64) * 4);
}

template <class F>
int blk_lu(const F* A, int n, int64_t batch, F* sign, RealOf<F>* logabs, void* ws, size_t ws_bytes, hipStream_t s) {
  if (batch <= 0) return FX_OK;
  if (n <= 0 || n > blk_max_n<F>()) return FX_ERR_UNSUPPORTED;
  if (!ws || ws_bytes < blk_lu_workspace<F>(batch, n)) return FX_ERR_WORKSPACE;
  const int N = lu64_padded(n);
  char* p = (char*)ws;
  const Lu64Bufs<F> f = lu64_take<F>(p, batch, N);
  return lu64_factor<F>(A, n, 0, batch, f, N, sign, logabs, s);
}

template <class F>
size_t blk_lu_inverse_workspace(int64_t batch, int n) {
  if (batch <= 0 || n <= 0) return 0;
  const int N = lu64_padded(n);
  return blk_lu_workspace<F>(batch, n) + al256((size_t)batch * N * N * sizeof(F)) + al256((size_t)batch * 4);
}

// The factorisation of A (skew: of (A - A^T) / 2) with its sign / logabs, then X = A^-1 by
// the blocked solves L Y = P I (the panels' swaps applied to Y as they were to A, column
// by column, rows in the order of their panel) and U X = Y (bottom block first), each a
// 32-row substitution per column and a K = 32 MFMA update of the rows below / above per
// block. out = X^T (out_t) or X, times ssign exp(slog) when ssign is given (the
// factorisation's own sign / logabs: the det adjugate of a regular member; a Parlett-Reid
// run's: the Pfaffian adjugate), zero where gate is 0 (default: the member's own sign) or
// X is not finite. 2 n^3 flops of the solves on the MFMA against 2 n^3 of a Gauss-Jordan
// run on one workgroup per matrix.
template <class F>
int blk_lu_inverse(const F* A, int n, int skew, int64_t batch, F* sign, RealOf<F>* logabs, const F* gate,
                   const F* ssign, const RealOf<F>* slog, F* out, int out_t, void* ws, size_t ws_bytes, hipStream_t s) {
  if (batch <= 0) return FX_OK;
  if (n <= 0 || n > blk_max_n<F>()) return FX_ERR_UNSUPPORTED;
  if (!ws || ws_bytes < blk_lu_inverse_workspace<F>(batch, n)) return FX_ERR_WORKSPACE;
  const int N = lu64_padded(n);
  char* p = (char*)ws;
  const Lu64Bufs<F> f = lu64_take<F>(p, batch, N);
  F* Y = (F*)p;
  p += al256((size_t)batch * N * N * sizeof(F));
  int* flag = (int*)p;
  int st = lu64_factor<F>(A, n, skew, batch, f, N, sign, logabs, s);
  if (st != FX_OK) return st;
  const int64_t tot = batch * (int64_t)N * N;
  lu64_fill_kernel<F><<<dim3(grid_of(tot)), 256, 0, s>>>(Y, N, flag, batch, tot);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  for (int r0 = 0; r0 < N && st == FX_OK; r0 += P64) {
    const int r1 = r0 + P64;
    st = lu64_rows<F, 1>(f.W, Y, N, r0, f.ipiv, 0, N, batch, s);
    if (st == FX_OK && r1 < N)
      st = lu64_gemm<F>(f.W + (int64_t)r1 * N + r0, Y + (int64_t)r0 * N, Y + (int64_t)r1 * N, N, N - r1, N, batch, s);
  }
  for (int r0 = N - P64; r0 >= 0 && st == FX_OK; r0 -= P64) {
    st = lu64_rows<F, 2>(f.W, Y, N, r0, f.ipiv, 0, N, batch, s);
    if (st == FX_OK && r0 > 0) st = lu64_gemm<F>(f.W + r0, Y + (int64_t)r0 * N, Y, N, r0, N, batch, s);
  }
  if (st != FX_OK) return st;
  const int64_t on = batch * (int64_t)n * n;
  lu64_out_kernel<F><<<dim3(grid_of(on)), 256, 0, s>>>(Y, N, n, out_t, gate ? gate : sign, ssign, slog, out, flag, on);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  lu64_zero_kernel<F><<<dim3(grid_of(on)), 256, 0, s>>>(out, n, flag, on);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

template <class F>
size_t blk_pr_workspace(int64_t batch, int n) {
  if (batch <= 0 || n <= 0 || (n & 1)) return 0;
  const int N = lu64_padded(n);
  return al256((size_t)batch * N * N * sizeof(F)) + 2 * al256((size_t)batch * N * P64 * sizeof(F)) +
         al256((size_t)batch * N * sizeof(F)) + al256((size_t)batch * 8) + al256((size_t)batch * 16) +
         al256((size_t)batch * 4) + al256((size_t)batch * 16);
}

// sign / logabs of pf(A) (skew: of (A - A^T) / 2) by the blocked Parlett-Reid: copy with
// [[0, 1], [-1, 0]] padding to order N (a multiple of 32), 16 pair steps per panel
// kernel, the K = 32 trailing update after each; (0, -inf) for odd n. spread (optional,
// B doubles): log max |d| - log min |d| over the pair pivots of the matrix (not of its
// padding), +inf where pf = 0.
template <class F>
int blk_pr(const F* A, int n, int skew, int64_t batch, F* sign, RealOf<F>* logabs, void* ws, size_t ws_bytes,
           hipStream_t s, double* spread) {
  if (batch <= 0) return FX_OK;
  if (n <= 0 || n > blk_max_n<F>()) return FX_ERR_UNSUPPORTED;
  const unsigned gb = (unsigned)((batch + 255) / 256);
  if (n & 1) {
    pr64_finish_kernel<F><<<dim3(gb), 256, 0, s>>>(nullptr, nullptr, nullptr, nullptr, 1, sign, logabs, spread, batch);
    return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
  }
  if (!ws || ws_bytes < blk_pr_workspace<F>(batch, n)) return FX_ERR_WORKSPACE;
  const int N = lu64_padded(n);
  const Pr64Bufs<F> f = pr64_take<F>((char*)ws, batch, N);
  const int64_t total = batch * (int64_t)N * N;
  lu64_copy_kernel<F><<<dim3(grid_of(total)), 256, 0, s>>>(A, n, skew, f.W, N, total, 1);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  pr64_init_kernel<<<dim3(gb), 256, 0, s>>>(f.lacc, f.sacc, f.stat, f.lr, batch);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  const int64_t NN = (int64_t)N * N, NP = (int64_t)N * P64;
  for (int r0 = 0; r0 < N; r0 += P64) {
    // the panel's (U, V) in registers for 8-byte elements up to 512 rows (the 16-byte
    // complex128 entries, and 1024-thread workgroups, would spill)
    bool in_regs = false;
    if constexpr (sizeof(F) <= 8) {
      in_regs = N - r0 <= 512;
      if (in_regs)
        pr64_panel_reg_kernel<F, 512><<<dim3((unsigned)batch), 512, 0, s>>>(f.W, N, n, r0, f.Ar, f.Bk, f.lacc, f.sacc,
                                                                            f.stat, f.lr);
    }
    if (!in_regs)  // latency-bound column loops: more threads per matrix
      pr64_panel_kernel<F, 1024><<<dim3((unsigned)batch), 1024, 0, s>>>(f.W, N, n, r0, f.Ar, f.Bk, f.rc, f.lacc, f.sacc,
                                                                        f.stat, f.lr);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
    const int r1 = r0 + P64;
    if (r1 >= N) break;
    // S22 -= [U, -V] [V, U]^T over positions r1 .. N - 1
    const int st = lu64_gemm_strided<F>(f.Ar + (int64_t)r1 * P64, P64, NP, f.Bk + r1, N, NP,
                                        f.W + (int64_t)r1 * N + r1, N, NN, N - r1, N - r1, batch, s);
    if (st != FX_OK) return st;
  }
  pr64_finish_kernel<F><<<dim3(gb), 256, 0, s>>>(f.lacc, f.sacc, f.stat, f.lr, 0, sign, logabs, spread, batch);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

#define FX_BLK_INST(F)                                                                                            \
  template size_t blk_lu_workspace<F>(int64_t, int);                                                             \
  template int blk_lu<F>(const F*, int, int64_t, F*, RealOf<F>*, void*, size_t, hipStream_t);                    \
  template size_t blk_lu_inverse_workspace<F>(int64_t, int);                                                     \
  template int blk_lu_inverse<F>(const F*, int, int, int64_t, F*, RealOf<F>*, const F*, const F*,                \
                                 const RealOf<F>*, F*, int, void*, size_t, hipStream_t);                         \
  template size_t blk_pr_workspace<F>(int64_t, int);                                                             \
  template int blk_pr<F>(const F*, int, int, int64_t, F*, RealOf<F>*, void*, size_t, hipStream_t, double*);
FX_BLK_INST(double)
FX_BLK_INST(float)
FX_BLK_INST(cx<float>)
FX_BLK_INST(cx<double>)
#undef FX_BLK_INST

// the float64 names used by f64.hip and cplx.hip
size_t lu64_workspace(int64_t batch, int n) { return blk_lu_workspace<double>(batch, n); }
int launch_lu64(const double* A, int n, int64_t batch, double* sign, double* logabs, void* ws, size_t ws_bytes,
                hipStream_t s) {
  return blk_lu<double>(A, n, batch, sign, logabs, ws, ws_bytes, s);
}
size_t lu64_inverse_workspace(int64_t batch, int n) { return blk_lu_inverse_workspace<double>(batch, n); }
int launch_lu64_inverse(const double* A, int n, int skew, int64_t batch, double* sign, double* logabs,
                        const double* gate, const double* ssign, const double* slog, double* out, int out_t,
                        void* ws, size_t ws_bytes, hipStream_t s) {
  return blk_lu_inverse<double>(A, n, skew, batch, sign, logabs, gate, ssign, slog, out, out_t, ws, ws_bytes, s);
}
size_t pr64_workspace(int64_t batch, int n) { return blk_pr_workspace<double>(batch, n); }
int launch_pr64_blocked(const double* A, int n, int skew, int64_t batch, double* sign, double* logabs, void* ws,
                        size_t ws_bytes, hipStream_t s, double* spread) {
  return blk_pr<double>(A, n, skew, batch, sign, logabs, ws, ws_bytes, s, spread);
}

}  // namespace fx
