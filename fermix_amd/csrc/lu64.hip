// Blocked float64 LU with partial pivoting (sign, logabs) for 128 < n <= 4096: the
// reference's `_lu_core` block loop (src/fermix/_lu.py:543-611: panel, row swaps, U rows,
// trailing GEMM) for the 64-bit kind, with the trailing update on the fp64 MFMA
// (v_mfma_f64_16x16x4f64). The matrix is copied into a workspace of padded order N (a
// multiple of 32, identity padding) and factored in place, 32 columns per block:
//   1. lu64_panel_kernel (one workgroup per matrix): the 32 columns of rows >= r0, one
//      column step at a time -- the pivot is the row of largest |x| among rows >= c
//      (lowest row on ties), swapped into row c over the panel's columns, then the
//      multipliers and the rank-1 update of the panel's remaining columns;
//   2. lu64_urow_kernel (matrix x 256 trailing columns): the panel's row swaps on the
//      trailing columns and U12 = L11^-1 A12 by forward substitution (L11 in LDS);
//   3. lu64_update_kernel (matrix x 64 x 64 tile): A22 -= L21 U12 at K = 32, the products
//      in an accumulator of their own, subtracted from A22 in fp64 at the end;
//   4. lu64_finish_kernel: sign = (-1)^swaps * prod sign(d), logabs = sum log|d| in
//      pivot order (one wave, lane-strided partial sums and a fixed tree).
// The column steps of a panel are latency-bound (three workgroup barriers each); the
// work that grows as n^3 runs on the MFMA in many workgroups per matrix.
#include <algorithm>

#include "common.h"
#include "fermix_internal.h"

namespace fx {
namespace {

constexpr int P64 = 32;    // panel width
constexpr int NT64 = 256;  // threads of the panel and U-row workgroups

typedef double v4d __attribute__((ext_vector_type(4)));

int lu64_padded(int n) { return (n + P64 - 1) / P64 * P64; }

// W (B, N, N) = A (B, n, n) with identity padding; a grid-stride loop over B N N elements.
__global__ void lu64_copy_kernel(const double* __restrict__ A, int n, double* __restrict__ W, int N,
                                 int64_t total) {
  const int64_t NN = (int64_t)N * N;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = e / NN;
    const int64_t f = e - b * NN;
    const int r = (int)(f / N), c = (int)(f - (int64_t)r * N);
    W[e] = (r < n && c < n) ? A[b * (int64_t)n * n + (int64_t)r * n + c] : (r == c ? 1.0 : 0.0);
  }
}

// Panel of columns r0 .. r0 + 31, rows r0 .. N - 1, in place; ipiv / d: the pivot row and
// pivot of each column; nsw: the block's row swaps.
__global__ __launch_bounds__(NT64) void lu64_panel_kernel(double* __restrict__ W, int N, int r0,
                                                          int* __restrict__ ipiv, double* __restrict__ dpiv,
                                                          int* __restrict__ nsw) {
  __shared__ unsigned long long redk[2][NT64 / 64];
  __shared__ int redr[2][NT64 / 64];
  __shared__ double prow[P64];
  const int64_t b = blockIdx.x;
  double* Wb = W + b * (int64_t)N * N;
  const int tid = threadIdx.x;
  int swaps = 0;
  for (int j = 0; j < P64; ++j) {
    const int c = r0 + j;
    unsigned long long k = 0;
    int row = 0x7fffffff;
    for (int r = c + tid; r < N; r += NT64) take_better(k, row, key64(Wb[(int64_t)r * N + c]), r);
    const int p = block_argmax<NT64>(k, row, redk[j & 1], redr[j & 1]);  // >= c: every key is >= 1
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
    for (int r = c + 1 + tid; r < N; r += NT64) {
      double* R = Wb + (int64_t)r * N + r0;
      const double l = R[j] * rd;
      R[j] = l;
      for (int q = j + 1; q < P64; ++q) R[q] = fma(-l, prow[q], R[q]);
    }
    __syncthreads();
  }
  if (tid == 0) nsw[b * (N / P64) + r0 / P64] = swaps;
}

// Trailing columns r0 + 32 + 256 cb + tid: the panel's swaps, then U12 = L11^-1 A12.
__global__ __launch_bounds__(NT64) void lu64_urow_kernel(double* __restrict__ W, int N, int r0,
                                                         const int* __restrict__ ipiv, int ncb) {
  __shared__ double L11[P64][P64 + 1];
  const int64_t b = blockIdx.x / ncb;
  const int cb = (int)(blockIdx.x - b * ncb);
  double* Wb = W + b * (int64_t)N * N;
  const int tid = threadIdx.x;
  for (int e = tid; e < P64 * P64; e += NT64) {
    const int i = e / P64, k = e % P64;
    L11[i][k] = Wb[(int64_t)(r0 + i) * N + r0 + k];
  }
  __syncthreads();
  const int col = r0 + P64 + NT64 * cb + tid;
  if (col >= N) return;
  const int* ip = ipiv + b * N + r0;
  double x[P64];
#pragma unroll
  for (int i = 0; i < P64; ++i) x[i] = Wb[(int64_t)(r0 + i) * N + col];
  // swaps in column order: row r0 + j with row ip[j] (>= r0 + j); rows beyond the panel
  // rows exchange with the column's entries below
#pragma unroll
  for (int j = 0; j < P64; ++j) {
    const int p = ip[j];
    if (p != r0 + j) {
      if (p < r0 + P64) {
        // both rows inside the panel rows: exchange x[j] and x[p - r0]
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
        double* e = Wb + (int64_t)p * N + col;
        const double u = *e;
        *e = x[j];
        x[j] = u;
      }
    }
  }
  // forward substitution with the unit lower L11
#pragma unroll
  for (int i = 1; i < P64; ++i) {
    double v = x[i];
#pragma unroll
    for (int k = 0; k < i; ++k) v = fma(-L11[i][k], x[k], v);
    x[i] = v;
  }
#pragma unroll
  for (int i = 0; i < P64; ++i) Wb[(int64_t)(r0 + i) * N + col] = x[i];
}

// A22 -= L21 U12 over the trailing rows / columns >= r1 = r0 + 32, one 64 x 64 tile per
// workgroup (tiles t = tile row * ntl + tile column), four waves of 32 x 32, each as
// 2 x 2 16 x 16 fp64 MFMA accumulators over K = 32 (eight K = 4 steps). Lane l supplies
// A[l % 16][l / 16] and B[l / 16][l % 16]; accumulator element v of lane l is row
// l / 16 + 4 v, column l % 16 (measured with a one-wave probe: unlike the fp32 16x16x4
// layout, the four rows of a lane are 4 apart).
__global__ __launch_bounds__(256) void lu64_update_kernel(double* __restrict__ W, int N, int r0, int ntl) {
  __shared__ double As[64][P64 + 1];  // L21 tile rows
  __shared__ double Bs[P64][64 + 1];  // U12 tile columns
  const int nt = ntl * ntl;
  const int64_t b = blockIdx.x / nt;
  const int t = (int)(blockIdx.x - b * nt);
  const int r1 = r0 + P64;
  const int i0 = r1 + 64 * (t / ntl), j0 = r1 + 64 * (t % ntl);
  double* Wb = W + b * (int64_t)N * N;
  const int tid = threadIdx.x;
  for (int e = tid; e < 64 * P64; e += 256) {
    const int i = e / P64, k = e % P64;
    As[i][k] = i0 + i < N ? Wb[(int64_t)(i0 + i) * N + r0 + k] : 0.0;
    const int kk = e / 64, j = e % 64;
    Bs[kk][j] = j0 + j < N ? Wb[(int64_t)(r0 + kk) * N + j0 + j] : 0.0;
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
        if (row < N && col < N) {
          double* e = Wb + (int64_t)row * N + col;
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
  auto take = [&](size_t x) {
    char* q = p;
    p += (x + 255) / 256 * 256;
    return (void*)q;
  };
  double* W = (double*)take((size_t)batch * N * N * 8);
  int* ipiv = (int*)take((size_t)batch * N * 4);
  double* dpiv = (double*)take((size_t)batch * N * 8);
  int* nsw = (int*)take((size_t)batch * (N / P64) * 4);
  const int64_t total = batch * (int64_t)N * N;
  const int64_t cblocks = std::min<int64_t>((total + 255) / 256, 1 << 20);
  lu64_copy_kernel<<<dim3((unsigned)cblocks), 256, 0, s>>>(A, n, W, N, total);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  for (int r0 = 0; r0 < N; r0 += P64) {
    lu64_panel_kernel<<<dim3((unsigned)batch), NT64, 0, s>>>(W, N, r0, ipiv, dpiv, nsw);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
    const int rest = N - r0 - P64;
    if (rest <= 0) break;
    const int ncb = (rest + NT64 - 1) / NT64;
    lu64_urow_kernel<<<dim3((unsigned)(batch * ncb)), NT64, 0, s>>>(W, N, r0, ipiv, ncb);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
    const int ntl = (rest + 63) / 64;
    lu64_update_kernel<<<dim3((unsigned)(batch * ntl * ntl)), 256, 0, s>>>(W, N, r0, ntl);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  }
  lu64_finish_kernel<<<dim3((unsigned)((batch + 3) / 4)), 256, 0, s>>>(dpiv, nsw, N, sign, logabs, batch);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

}  // namespace fx
