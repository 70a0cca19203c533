// Blocked float64 LU with partial pivoting (sign, logabs) for 128 < n <= 4096: the
// reference's `_lu_core` block loop (src/fermix/_lu.py:543-611: panel, row swaps, U rows,
// trailing GEMM) for the 64-bit kind, with the trailing update on the fp64 MFMA
// (v_mfma_f64_16x16x4f64). The matrix is copied into a workspace of padded order N (a
// multiple of 32, identity padding) and factored in place, 32 columns per block:
//   1. lu64_panel_kernel (one workgroup per matrix): the 32 columns of rows >= r0, one
//      column step at a time -- the pivot is the row of largest |x| among rows >= c
//      (lowest row on ties), swapped into row c over the panel's columns, then the
//      multipliers and the rank-1 update of the panel's remaining columns;
//   2. lu64_rows_kernel<0> (matrix x 256 trailing columns): the panel's row swaps on the
//      trailing columns and U12 = L11^-1 A12 by forward substitution (L11 in LDS);
//   3. lu64_gemm_kernel (matrix x 64 x 64 tile): A22 -= L21 U12 at K = 32, the products
//      in an accumulator of their own, subtracted from A22 in fp64 at the end;
//   4. lu64_finish_kernel: sign = (-1)^swaps * prod sign(d), logabs = sum log|d| in
//      pivot order (one wave, lane-strided partial sums and a fixed tree).
// The column steps of a panel are latency-bound (three workgroup barriers each); the
// work that grows as n^3 runs on the MFMA in many workgroups per matrix. The inverse
// (launch_lu64_inverse: A^-T, S^-1, det A^-T) solves with the same row and GEMM kernels,
// and the blocked Parlett-Reid below (launch_pr64_blocked: float64 slogpf) updates its
// trailing matrix with the same GEMM.
#include <algorithm>

#include "common.h"
#include "fermix_internal.h"

namespace fx {
namespace {

constexpr int P64 = 32;    // panel width
constexpr int NT64 = 256;  // threads of the panel and U-row workgroups

typedef double v4d __attribute__((ext_vector_type(4)));

int lu64_padded(int n) { return (n + P64 - 1) / P64 * P64; }

// W (B, N, N) = A (B, n, n) with identity padding (skew: (A - A^T) / 2), or, with pfpad
// (n even), padding by 2 x 2 blocks [[0, 1], [-1, 0]] on the diagonal (skew, Pfaffian 1);
// a grid-stride loop over B N N elements.
__global__ void lu64_copy_kernel(const double* __restrict__ A, int n, int skew, double* __restrict__ W, int N,
                                 int64_t total, int pfpad = 0) {
  const int64_t NN = (int64_t)N * N;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = e / NN;
    const int64_t f = e - b * NN;
    const int r = (int)(f / N), c = (int)(f - (int64_t)r * N);
    const double* Ab = A + b * (int64_t)n * n;
    double v = pfpad ? (c == (r ^ 1) ? ((r & 1) ? -1.0 : 1.0) : 0.0) : (r == c ? 1.0 : 0.0);
    if (r < n && c < n) v = skew ? (Ab[(int64_t)r * n + c] - Ab[(int64_t)c * n + r]) * 0.5 : Ab[(int64_t)r * n + c];
    W[e] = v;
  }
}

// Panel of columns r0 .. r0 + 31, rows r0 .. N - 1, in place; ipiv / d: the pivot row and
// pivot of each column; nsw: the block's row swaps.
template <int NT>
__global__ __launch_bounds__(NT) void lu64_panel_kernel(double* __restrict__ W, int N, int r0,
                                                        int* __restrict__ ipiv, double* __restrict__ dpiv,
                                                        int* __restrict__ nsw) {
  __shared__ unsigned long long redk[2][NT / 64];
  __shared__ int redr[2][NT / 64];
  __shared__ double prow[P64];
  const int64_t b = blockIdx.x;
  double* Wb = W + b * (int64_t)N * N;
  const int tid = threadIdx.x;
  int swaps = 0;
  for (int j = 0; j < P64; ++j) {
    const int c = r0 + j;
    unsigned long long k = 0;
    int row = 0x7fffffff;
    for (int r = c + tid; r < N; r += NT) take_better(k, row, key64(Wb[(int64_t)r * N + c]), r);
    const int p = block_argmax<NT>(k, row, redk[j & 1], redr[j & 1]);  // >= c: every key is >= 1
    if (p != c) {
      if (tid < P64) {
        double* Rc = Wb + (int64_t)c * N + r0;
        double* Rp = Wb + (int64_t)p * N + r0;
        const double u = Rc[tid], v = Rp[tid];
        Rc[tid] = v;
        Rp[tid] = u;
      }
      ++swaps;
    }
    __syncthreads();
    if (tid < P64) prow[tid] = Wb[(int64_t)c * N + r0 + tid];
    __syncthreads();
    const double d = prow[j];
    if (tid == 0) {
      ipiv[b * N + c] = p;
      dpiv[b * N + c] = d;
    }
    const double rd = d != 0.0 ? 1.0 / d : 0.0;  // a zero pivot: its column is zero below
    for (int r = c + 1 + tid; r < N; r += NT) {
      double* R = Wb + (int64_t)r * N + r0;
      const double l = R[j] * rd;
      R[j] = l;
      for (int q = j + 1; q < P64; ++q) R[q] = fma(-l, prow[q], R[q]);
    }
    __syncthreads();
  }
  if (tid == 0) nsw[b * (N / P64) + r0 / P64] = swaps;
}

// 32 rows r0 .. r0 + 31 of a target matrix T, columns c0 + 256 cb + tid (< cend), against
// the diagonal block D = W[r0 .. r0 + 31][r0 .. r0 + 31] of the factorisation:
//   MODE 0 / 1: the panel's row swaps (row r0 + j with ipiv[r0 + j] >= r0 + j, in order),
//     then the forward substitution with the unit lower part of D (MODE 0: T = W, the
//     U rows of the trailing columns; MODE 1: T = Y, the forward solve of L Y = P I);
//   MODE 2: the backward substitution with the upper part of D (the solve U X = Y).
template <int MODE>
__global__ __launch_bounds__(NT64) void lu64_rows_kernel(const double* __restrict__ W, double* __restrict__ T,
                                                         int N, int r0, const int* __restrict__ ipiv, int c0,
                                                         int cend, int ncb) {
  __shared__ double D[P64][P64 + 1];
  const int64_t b = blockIdx.x / ncb;
  const int cb = (int)(blockIdx.x - b * ncb);
  const double* Wb = W + b * (int64_t)N * N;
  double* Tb = T + b * (int64_t)N * N;
  const int tid = threadIdx.x;
  for (int e = tid; e < P64 * P64; e += NT64) {
    const int i = e / P64, k = e % P64;
    D[i][k] = Wb[(int64_t)(r0 + i) * N + r0 + k];
  }
  __syncthreads();
  const int col = c0 + NT64 * cb + tid;
  if (col >= cend) return;
  double x[P64];
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
          double t = x[j];
#pragma unroll
          for (int i = j + 1; i < P64; ++i)
            if (p - r0 == i) {
              const double u = x[i];
              x[i] = t;
              t = u;
            }
          x[j] = t;
        } else {
          double* e = Tb + (int64_t)p * N + col;
          const double u = *e;
          *e = x[j];
          x[j] = u;
        }
      }
    }
#pragma unroll
    for (int i = 1; i < P64; ++i) {
      double v = x[i];
#pragma unroll
      for (int k = 0; k < i; ++k) v = fma(-D[i][k], x[k], v);
      x[i] = v;
    }
  } else {
#pragma unroll
    for (int i = P64 - 1; i >= 0; --i) {
      double v = x[i];
#pragma unroll
      for (int k = i + 1; k < P64; ++k) v = fma(-D[i][k], x[k], v);
      x[i] = v / D[i][i];
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
__global__ __launch_bounds__(256) void lu64_gemm_kernel(const double* __restrict__ A, int lda, int64_t sA,
                                                        const double* __restrict__ Bm, int ldb, int64_t sB,
                                                        double* __restrict__ C, int ldc, int64_t sC, int M, int NC,
                                                        int ntr, int ntc) {
  __shared__ double As[64][P64 + 1];
  __shared__ double Bs[P64][64 + 1];
  const int nt = ntr * ntc;
  const int64_t b = blockIdx.x / nt;
  const int t = (int)(blockIdx.x - b * nt);
  const int i0 = 64 * (t / ntc), j0 = 64 * (t % ntc);
  const double* Ab = A + b * sA;
  const double* Bb = Bm + b * sB;
  double* Cb = C + b * sC;
  const int tid = threadIdx.x;
  for (int e = tid; e < 64 * P64; e += 256) {
    const int i = e / P64, k = e % P64;
    As[i][k] = i0 + i < M ? Ab[(int64_t)(i0 + i) * lda + k] : 0.0;
    const int kk = e / 64, j = e % 64;
    Bs[kk][j] = j0 + j < NC ? Bb[(int64_t)kk * ldb + j0 + j] : 0.0;
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
          double* e = Cb + (int64_t)row * ldc + col;
          *e = *e - acc[a][c][v];
        }
      }
    }
}

// (sign, logabs) per matrix, one wave each: lane-strided partial sums of log|d| over the
// pivots in order, a fixed xor tree, the sign from the count of negative pivots and swaps.
__global__ void lu64_finish_kernel(const double* __restrict__ dpiv, const int* __restrict__ nsw, int N,
                                   double* __restrict__ sign, double* __restrict__ logabs, int64_t batch) {
  const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (b >= batch) return;
  double lg = 0.0;
  int neg = 0, zero = 0;
  for (int i = lane; i < N; i += 64) {
    const double d = dpiv[b * N + i];
    zero |= d == 0.0;
    neg += d < 0.0;
    lg += d != 0.0 ? log(fabs(d)) : 0.0;
  }
  int sw = 0;
  for (int i = lane; i < N / P64; i += 64) sw += nsw[b * (N / P64) + i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    lg += __shfl_xor(lg, off);
    neg += __shfl_xor(neg, off);
    zero |= __shfl_xor(zero, off);
    sw += __shfl_xor(sw, off);
  }
  if (lane == 0) {
    sign[b] = zero ? 0.0 : (((neg + sw) & 1) ? -1.0 : 1.0);
    logabs[b] = zero ? -INFINITY : lg;
  }
}

// out[b][i][j] (i, j < n) = scale_b X[j][i] (out_t) or scale_b X[i][j], X the solve's
// N x N result; zero where gate[b] == 0 (the member's own sign, or a caller's gate); any
// non-finite value of a member raises flag[b] (every writer stores 1).
__global__ void lu64_out_kernel(const double* __restrict__ X, int N, int n, int out_t,
                                const double* __restrict__ gate, const double* __restrict__ ssign,
                                const double* __restrict__ slog, double* __restrict__ out, int* __restrict__ flag,
                                int64_t total) {
  const int64_t nn = (int64_t)n * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = e / nn;
    const int64_t f = e - b * nn;
    const int i = (int)(f / n), j = (int)(f - (int64_t)i * n);
    double v = 0.0;
    if (gate[b] != 0.0) {
      v = X[b * (int64_t)N * N + (out_t ? (int64_t)j * N + i : (int64_t)i * N + j)];
      if (ssign) v *= ssign[b] * exp(slog[b]);
      if (!isfinite(v)) flag[b] = 1;
    }
    out[e] = v;
  }
}

__global__ void lu64_zero_kernel(double* __restrict__ out, int n, const int* __restrict__ flag, int64_t total) {
  const int64_t nn = (int64_t)n * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x)
    if (flag[e / nn]) out[e] = 0.0;
}

__global__ void lu64_fill_kernel(double* __restrict__ Y, int N, int* __restrict__ flag, int64_t batch,
                                 int64_t total) {
  const int64_t NN = (int64_t)N * N;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t f = e % NN;
    Y[e] = (f / N == f % N) ? 1.0 : 0.0;
    if (f == 0) flag[e / NN] = 0;
  }
}

unsigned grid_of(int64_t total) { return (unsigned)std::min<int64_t>((total + 255) / 256, 1 << 20); }

struct Lu64Bufs {
  double* W;
  int* ipiv;
  double* dpiv;
  int* nsw;
};

Lu64Bufs lu64_take(char*& p, int64_t batch, int N) {
  auto take = [&](size_t x) {
    char* q = p;
    p += (x + 255) / 256 * 256;
    return (void*)q;
  };
  Lu64Bufs f;
  f.W = (double*)take((size_t)batch * N * N * 8);
  f.ipiv = (int*)take((size_t)batch * N * 4);
  f.dpiv = (double*)take((size_t)batch * N * 8);
  f.nsw = (int*)take((size_t)batch * (N / P64) * 4);
  return f;
}

// C -= A B (K = 32) over M x NC, operands at their first elements of matrix 0
int lu64_gemm_strided(const double* A, int lda, int64_t sA, const double* Bm, int ldb, int64_t sB, double* C,
                      int ldc, int64_t sC, int M, int NC, int64_t batch, hipStream_t s) {
  if (M <= 0 || NC <= 0) return FX_OK;
  const int ntr = (M + 63) / 64, ntc = (NC + 63) / 64;
  lu64_gemm_kernel<<<dim3((unsigned)(batch * ntr * ntc)), 256, 0, s>>>(A, lda, sA, Bm, ldb, sB, C, ldc, sC, M, NC,
                                                                      ntr, ntc);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

// the same with every operand inside an N x N matrix of the batch
int lu64_gemm(const double* A, const double* Bm, double* C, int N, int M, int NC, int64_t batch, hipStream_t s) {
  const int64_t NN = (int64_t)N * N;
  return lu64_gemm_strided(A, N, NN, Bm, N, NN, C, N, NN, M, NC, batch, s);
}

template <int MODE>
int lu64_rows(const double* W, double* T, int N, int r0, const int* ipiv, int c0, int cend, int64_t batch,
              hipStream_t s) {
  if (cend <= c0) return FX_OK;
  const int ncb = (cend - c0 + NT64 - 1) / NT64;
  lu64_rows_kernel<MODE><<<dim3((unsigned)(batch * ncb)), NT64, 0, s>>>(W, T, N, r0, ipiv, c0, cend, ncb);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

// Copy (with skew symmetrisation) and factor in place; sign / logabs of the factorisation.
int lu64_factor(const double* A, int n, int skew, int64_t batch, const Lu64Bufs& f, int N, double* sign,
                double* logabs, hipStream_t s) {
  const int64_t total = batch * (int64_t)N * N;
  lu64_copy_kernel<<<dim3(grid_of(total)), 256, 0, s>>>(A, n, skew, f.W, N, total);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  for (int r0 = 0; r0 < N; r0 += P64) {
    if (N > 512)  // latency-bound column steps: more threads per matrix
      lu64_panel_kernel<1024><<<dim3((unsigned)batch), 1024, 0, s>>>(f.W, N, r0, f.ipiv, f.dpiv, f.nsw);
    else
      lu64_panel_kernel<NT64><<<dim3((unsigned)batch), NT64, 0, s>>>(f.W, N, r0, f.ipiv, f.dpiv, f.nsw);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
    const int r1 = r0 + P64;
    if (r1 >= N) break;
    int st = lu64_rows<0>(f.W, f.W, N, r0, f.ipiv, r1, N, batch, s);
    if (st == FX_OK)
      st = lu64_gemm(f.W + (int64_t)r1 * N + r0, f.W + (int64_t)r0 * N + r1, f.W + (int64_t)r1 * N + r1, N, N - r1,
                     N - r1, batch, s);
    if (st != FX_OK) return st;
  }
  lu64_finish_kernel<<<dim3((unsigned)((batch + 3) / 4)), 256, 0, s>>>(f.dpiv, f.nsw, N, sign, logabs, batch);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

// ---- blocked Parlett-Reid (float64 slogpf above the register kernels)
//
// The reference's Parlett-Reid block loop (src/fermix/_pf.py:59-382: pair steps with a
// pivot search in the eliminated column, a symmetric row / column swap and the rank-2
// skew update S22 -= u v^T - v u^T, u = S[c, :] / S[c, c + 1], v = S[c + 1, :]) with the
// updates of 16 pair steps deferred: within a panel each pair step forms its two rows
// left-looking from the panel's earlier (u, v), and after the panel the trailing matrix
// takes all 16 at once, S22 -= [U, -V] [V, U]^T, a K = 32 product on the fp64 MFMA
// (lu64_gemm_kernel). The pair's Pfaffian factor is d = S[c, c + 1] after the swap; pf =
// (-1)^swaps prod d.
constexpr int PRB = P64 / 2;  // pair steps per panel

// Panel of positions r0 .. r0 + 31 (one workgroup per matrix), W the full skew matrix of
// padded order N (rows and columns >= c + 1 swapped symmetrically, in place). Ar (B, N,
// 32): row x = (U[x][0..15], -V[x][0..15]); Bk (B, 32, N): rows 0..15 = V^T, 16..31 =
// U^T (the two operands of the trailing product, and the left-looking coefficients).
// rc: the current row c of the pair step; lacc / sacc / stat: log|pf| and sign so far and
// the zero-pivot flag (a flagged member skips its later panels).
template <int NT>
__global__ __launch_bounds__(NT) void pr64_panel_kernel(double* __restrict__ W, int N, int r0,
                                                        double* __restrict__ Ar, double* __restrict__ Bk,
                                                        double* __restrict__ rcg, double* __restrict__ lacc,
                                                        double* __restrict__ sacc, int* __restrict__ stat) {
  __shared__ unsigned long long redk[2][NT / 64];
  __shared__ int redr[2][NT / 64];
  __shared__ double cu[PRB], cv[PRB];
  const int64_t b = blockIdx.x;
  if (stat[b]) return;
  const int tid = threadIdx.x;
  double* Wb = W + b * (int64_t)N * N;
  double* Ab = Ar + b * (int64_t)N * P64;
  double* Bb = Bk + b * (int64_t)P64 * N;
  double* rc = rcg + b * (int64_t)N;
  double lg = 0.0, sg = 1.0;  // thread 0's running sums, in pivot order
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
      double a = Wb[(int64_t)c * N + x];
      for (int j = 0; j < p; ++j) {
        a = fma(-cu[j], Bb[(int64_t)j * N + x], a);
        a = fma(cv[j], Bb[(int64_t)(PRB + j) * N + x], a);
      }
      rc[x] = a;
      take_better(k, row, key64(a), x);
    }
    // |S[x][c]| = |S[c][x]|: the largest, lowest index on ties, moves to position q
    const int pv = block_argmax<NT>(k, row, redk[p & 1], redr[p & 1]);
    if (pv != q) {
      for (int x = q + tid; x < N; x += NT) {
        const double u = Wb[(int64_t)pv * N + x], v = Wb[(int64_t)q * N + x];
        Wb[(int64_t)pv * N + x] = v;
        Wb[(int64_t)q * N + x] = u;
      }
      if (tid < P64) {
        const double u = Ab[(int64_t)pv * P64 + tid], v = Ab[(int64_t)q * P64 + tid];
        Ab[(int64_t)pv * P64 + tid] = v;
        Ab[(int64_t)q * P64 + tid] = u;
        const double y = Bb[(int64_t)tid * N + pv], z = Bb[(int64_t)tid * N + q];
        Bb[(int64_t)tid * N + pv] = z;
        Bb[(int64_t)tid * N + q] = y;
      }
      if (tid == 0) {
        const double u = rc[pv];
        rc[pv] = rc[q];
        rc[q] = u;
        sg = -sg;
      }
      __syncthreads();
      for (int r = q + tid; r < N; r += NT) {
        const double u = Wb[(int64_t)r * N + pv], v = Wb[(int64_t)r * N + q];
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
    const double d = rc[q];
    if (d == 0.0) {  // row c is zero beyond c: pf = 0
      sing = true;
      break;
    }
    const double rd = 1.0 / d;
    // u = row c / d, v = row q (left-looking like row c) beyond q; zero at positions <= q
    for (int x = r0 + tid; x < N; x += NT) {
      double u = 0.0, v = 0.0;
      if (x > q) {
        double a = Wb[(int64_t)q * N + x];
        for (int j = 0; j < p; ++j) {
          a = fma(-cu[j], Bb[(int64_t)j * N + x], a);
          a = fma(cv[j], Bb[(int64_t)(PRB + j) * N + x], a);
        }
        v = a;
        u = rc[x] * rd;
      }
      Ab[(int64_t)x * P64 + p] = u;
      Ab[(int64_t)x * P64 + PRB + p] = -v;
      Bb[(int64_t)p * N + x] = v;
      Bb[(int64_t)(PRB + p) * N + x] = u;
    }
    if (tid == 0) {
      lg += log(fabs(d));
      if (d < 0.0) sg = -sg;
    }
    __syncthreads();
  }
  if (tid == 0) {
    if (sing) stat[b] = 1;
    lacc[b] += lg;
    sacc[b] *= sg;
  }
}

__global__ void pr64_init_kernel(double* __restrict__ lacc, double* __restrict__ sacc, int* __restrict__ stat,
                                 int64_t batch) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  lacc[b] = 0.0;
  sacc[b] = 1.0;
  stat[b] = 0;
}

// (sign, logabs): the running sums, (0, -inf) for flagged members and for odd n (odd)
__global__ void pr64_finish_kernel(const double* __restrict__ lacc, const double* __restrict__ sacc,
                                   const int* __restrict__ stat, int odd, double* __restrict__ sign,
                                   double* __restrict__ logabs, int64_t batch) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  const bool zero = odd || stat[b];
  sign[b] = zero ? 0.0 : sacc[b];
  logabs[b] = zero ? -INFINITY : lacc[b];
}

struct Pr64Bufs {
  double* W;
  double* Ar;
  double* Bk;
  double* rc;
  double* lacc;
  double* sacc;
  int* stat;
};

Pr64Bufs pr64_take(char* p, int64_t batch, int N) {
  auto take = [&](size_t x) {
    char* q = p;
    p += (x + 255) / 256 * 256;
    return (void*)q;
  };
  Pr64Bufs f;
  f.W = (double*)take((size_t)batch * N * N * 8);
  f.Ar = (double*)take((size_t)batch * N * P64 * 8);
  f.Bk = (double*)take((size_t)batch * N * P64 * 8);
  f.rc = (double*)take((size_t)batch * N * 8);
  f.lacc = (double*)take((size_t)batch * 8);
  f.sacc = (double*)take((size_t)batch * 8);
  f.stat = (int*)take((size_t)batch * 4);
  return f;
}

}  // namespace

size_t lu64_workspace(int64_t batch, int n) {
  if (batch <= 0 || n <= 0) return 0;
  const int N = lu64_padded(n);
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  return al((size_t)batch * N * N * 8) + al((size_t)batch * N * 4) + al((size_t)batch * N * 8) +
         al((size_t)batch * (N / P64) * 4);
}

int launch_lu64(const double* A, int n, int64_t batch, double* sign, double* logabs, void* ws, size_t ws_bytes,
                hipStream_t s) {
  if (batch <= 0) return FX_OK;
  if (n <= 0 || n > 4096) return FX_ERR_UNSUPPORTED;
  if (!ws || ws_bytes < lu64_workspace(batch, n)) return FX_ERR_WORKSPACE;
  const int N = lu64_padded(n);
  char* p = (char*)ws;
  const Lu64Bufs f = lu64_take(p, batch, N);
  return lu64_factor(A, n, 0, batch, f, N, sign, logabs, s);
}

size_t lu64_inverse_workspace(int64_t batch, int n) {
  if (batch <= 0 || n <= 0) return 0;
  const int N = lu64_padded(n);
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  return lu64_workspace(batch, n) + al((size_t)batch * N * N * 8) + al((size_t)batch * 4);
}

// The factorisation of A (skew: of (A - A^T) / 2) with its sign / logabs, then X = A^-1 by
// the blocked solves L Y = P I (the panels' swaps applied to Y as they were to A, column
// by column, rows in the order of their panel) and U X = Y (bottom block first), each a
// 32-row substitution per column and a K = 32 fp64 MFMA update of the rows below / above
// per block. out = X^T (out_t) or X, times ssign exp(slog) when ssign is given (the
// factorisation's own sign / logabs: the det adjugate of a regular member; a Parlett-Reid
// run's: the Pfaffian adjugate), zero where gate is 0 (default: the member's own sign) or
// X is not finite. 2 n^3 flops of the solves on the MFMA against 2 n^3 of a Gauss-Jordan
// run on one workgroup per matrix.
int launch_lu64_inverse(const double* A, int n, int skew, int64_t batch, double* sign, double* logabs,
                        const double* gate, const double* ssign, const double* slog, double* out, int out_t,
                        void* ws, size_t ws_bytes, hipStream_t s) {
  if (batch <= 0) return FX_OK;
  if (n <= 0 || n > 4096) return FX_ERR_UNSUPPORTED;
  if (!ws || ws_bytes < lu64_inverse_workspace(batch, n)) return FX_ERR_WORKSPACE;
  const int N = lu64_padded(n);
  char* p = (char*)ws;
  const Lu64Bufs f = lu64_take(p, batch, N);
  double* Y = (double*)p;
  p += ((size_t)batch * N * N * 8 + 255) / 256 * 256;
  int* flag = (int*)p;
  int st = lu64_factor(A, n, skew, batch, f, N, sign, logabs, s);
  if (st != FX_OK) return st;
  const int64_t tot = batch * (int64_t)N * N;
  lu64_fill_kernel<<<dim3(grid_of(tot)), 256, 0, s>>>(Y, N, flag, batch, tot);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  for (int r0 = 0; r0 < N && st == FX_OK; r0 += P64) {
    const int r1 = r0 + P64;
    st = lu64_rows<1>(f.W, Y, N, r0, f.ipiv, 0, N, batch, s);
    if (st == FX_OK && r1 < N)
      st = lu64_gemm(f.W + (int64_t)r1 * N + r0, Y + (int64_t)r0 * N, Y + (int64_t)r1 * N, N, N - r1, N, batch, s);
  }
  for (int r0 = N - P64; r0 >= 0 && st == FX_OK; r0 -= P64) {
    st = lu64_rows<2>(f.W, Y, N, r0, f.ipiv, 0, N, batch, s);
    if (st == FX_OK && r0 > 0) st = lu64_gemm(f.W + r0, Y + (int64_t)r0 * N, Y, N, r0, N, batch, s);
  }
  if (st != FX_OK) return st;
  const int64_t on = batch * (int64_t)n * n;
  lu64_out_kernel<<<dim3(grid_of(on)), 256, 0, s>>>(Y, N, n, out_t, gate ? gate : sign, ssign, slog, out, flag, on);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  lu64_zero_kernel<<<dim3(grid_of(on)), 256, 0, s>>>(out, n, flag, on);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

size_t pr64_workspace(int64_t batch, int n) {
  if (batch <= 0 || n <= 0 || (n & 1)) return 0;
  const int N = lu64_padded(n);
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  return al((size_t)batch * N * N * 8) + 2 * al((size_t)batch * N * P64 * 8) + al((size_t)batch * N * 8) +
         2 * al((size_t)batch * 8) + al((size_t)batch * 4);
}

// sign / logabs of pf(A) (skew: of (A - A^T) / 2) by the blocked Parlett-Reid: copy with
// [[0, 1], [-1, 0]] padding to order N (a multiple of 32), 16 pair steps per panel
// kernel, the K = 32 trailing update after each; (0, -inf) for odd n.
int launch_pr64_blocked(const double* A, int n, int skew, int64_t batch, double* sign, double* logabs, void* ws,
                        size_t ws_bytes, hipStream_t s) {
  if (batch <= 0) return FX_OK;
  if (n <= 0 || n > 4096) return FX_ERR_UNSUPPORTED;
  const unsigned gb = (unsigned)((batch + 255) / 256);
  if (n & 1) {
    pr64_finish_kernel<<<dim3(gb), 256, 0, s>>>(nullptr, nullptr, nullptr, 1, sign, logabs, batch);
    return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
  }
  if (!ws || ws_bytes < pr64_workspace(batch, n)) return FX_ERR_WORKSPACE;
  const int N = lu64_padded(n);
  const Pr64Bufs f = pr64_take((char*)ws, batch, N);
  const int64_t total = batch * (int64_t)N * N;
  lu64_copy_kernel<<<dim3(grid_of(total)), 256, 0, s>>>(A, n, skew, f.W, N, total, 1);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  pr64_init_kernel<<<dim3(gb), 256, 0, s>>>(f.lacc, f.sacc, f.stat, batch);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  const int64_t NN = (int64_t)N * N, NP = (int64_t)N * P64;
  for (int r0 = 0; r0 < N; r0 += P64) {
    if (N > 512)  // latency-bound column loops: more threads per matrix
      pr64_panel_kernel<1024><<<dim3((unsigned)batch), 1024, 0, s>>>(f.W, N, r0, f.Ar, f.Bk, f.rc, f.lacc, f.sacc,
                                                                     f.stat);
    else
      pr64_panel_kernel<NT64><<<dim3((unsigned)batch), NT64, 0, s>>>(f.W, N, r0, f.Ar, f.Bk, f.rc, f.lacc, f.sacc,
                                                                     f.stat);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
    const int r1 = r0 + P64;
    if (r1 >= N) break;
    // S22 -= [U, -V] [V, U]^T over positions r1 .. N - 1
    const int st = lu64_gemm_strided(f.Ar + (int64_t)r1 * P64, P64, NP, f.Bk + r1, N, NP, f.W + (int64_t)r1 * N + r1,
                                     N, NN, N - r1, N - r1, batch, s);
    if (st != FX_OK) return st;
  }
  pr64_finish_kernel<<<dim3(gb), 256, 0, s>>>(f.lacc, f.sacc, f.stat, 0, sign, logabs, batch);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

}  // namespace fx
