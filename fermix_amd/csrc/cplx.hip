// complex64 / complex128 slogdet and slogpf (values, A^-T and S^-1) -- the reference's
// complex kinds (src/fermix/_field.py:32-120: a complex value as a (re, im) pair, the
// pivot magnitude |re| + |im| (`abs1`, LAPACK's cabs1), the guarded reciprocal
// conj(x) / |x|^2 (`recip`), the pivot phase x / |x| (`unit`) and log of the modulus
// (`mag`)), with the conventions of the generic path (src/fermix/_fallback.py:36-97,
// 266-300): sign = parity * prod(d / |d|), logabs = sum log|d|, an exact zero pivot gives
// (0, -inf); A^-T without conjugation (the holomorphic derivative of log det).
//
// Layout: interleaved (re, im) pairs, row-major, batch-major -- the memory of torch's
// complex64 / complex128 tensors; sign is one complex value per member, logabs real.
//
// Kernels (one workgroup of 1024 threads per matrix; the matrix in LDS when it fits in
// 60 KiB, else in a per-matrix slice of the workspace, served from L2):
//  - cgj_kernel<T, INV>: Gauss-Jordan with virtual partial pivoting (the pivot of column
//    j is the unassigned row of largest |re| + |im|, lowest row on ties). Without INV only
//    the unassigned rows are updated (an LU); with INV the assigned rows and the identity
//    block [A | I] too, and row j of A^-1 is row prow[j] of the right block times the
//    pivot's reciprocal. The element update is the same in both, so the forward and the
//    inverse call give bit-identical sign / logabs;
//  - cpr_kernel<T>: Parlett-Reid with the pivot row / column swapped into position c + 1,
//    d = S[c, c+1], tau = -S[:, c] / d, w = S[:, c+1] and the rank-2 update
//    tau w^T - w tau^T on the rows and columns after c + 1.
// The phase and the log are accumulated in double for both kinds.
#include "common.h"
#include "fermix_internal.h"

namespace fx {
namespace {

constexpr int CX_MAXN = 4096;
constexpr size_t CX_LDS_MAX = 60 * 1024;  // matrix bytes kept in LDS
constexpr int CX_NT = 1024;

template <class T>
struct cx {
  T re, im;
};

template <class T>
__device__ __forceinline__ cx<T> cmul(cx<T> a, cx<T> b) {
  return {a.re * b.re - a.im * b.im, a.re * b.im + a.im * b.re};
}

// r - l p with fused products
template <class T>
__device__ __forceinline__ cx<T> cfms(cx<T> r, cx<T> l, cx<T> p) {
  return {fma(-l.re, p.re, fma(l.im, p.im, r.re)), fma(-l.re, p.im, fma(-l.im, p.re, r.im))};
}

// 1 / x = conj(x) / |x|^2, 0 -> 0
template <class T>
__device__ __forceinline__ cx<T> crecip(cx<T> x) {
  const T s = x.re * x.re + x.im * x.im;
  const T inv = s != T(0) ? T(1) / s : T(0);
  return {x.re * inv, -(x.im * inv)};
}

template <class T>
__device__ __forceinline__ bool czero(cx<T> x) {
  return x.re == T(0) && x.im == T(0);
}

// pivot key: |re| + |im| (exact in double for both kinds), order-preserving bits + 1
template <class T>
__device__ __forceinline__ unsigned long long ckey(cx<T> x) {
  return key64((double)(fabs(x.re) + fabs(x.im)));
}

// the pivot's phase and log-modulus, accumulated in double
__device__ __forceinline__ void acc_pivot(double2& sgn, double& logabs, double re, double im) {
  const double m = hypot(re, im);
  logabs += log(m);
  const double ur = re / m, ui = im / m;
  sgn = make_double2(sgn.x * ur - sgn.y * ui, sgn.x * ui + sgn.y * ur);
}

template <class T>
__device__ __forceinline__ void write_sl(cx<T>* sign_out, T* logabs_out, int64_t b, bool singular, double2 sgn,
                                         double logabs) {
  sign_out[b] = singular ? cx<T>{T(0), T(0)} : cx<T>{T(sgn.x), T(sgn.y)};
  logabs_out[b] = singular ? T(-INFINITY) : T(logabs);
}

// S (skew != 0: (a - a^T) / 2) into M with row stride ld; with ident, M[:, n:2n] = I.
template <class T>
__device__ __forceinline__ void cload(const cx<T>* __restrict__ a, int n, int skew, cx<T>* M, int ld, bool ident) {
  for (int e = threadIdx.x; e < n * n; e += CX_NT) {
    const int r = e / n, k = e - r * n;
    cx<T> v = a[e];
    if (skew) {
      const cx<T> u = a[(size_t)k * n + r];
      v = {(v.re - u.re) * T(0.5), (v.im - u.im) * T(0.5)};
    }
    M[(size_t)r * ld + k] = v;
    if (ident) M[(size_t)r * ld + n + k] = cx<T>{(r == k) ? T(1) : T(0), T(0)};
  }
}

template <class T, bool INV>
__global__ __launch_bounds__(CX_NT) void cgj_kernel(const cx<T>* __restrict__ a, int n, int skew, cx<T>* Wg,
                                                    int use_lds, cx<T>* __restrict__ sign_out,
                                                    T* __restrict__ logabs_out, cx<T>* __restrict__ out,
                                                    int out_t, const cx<T>* __restrict__ gate) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ unsigned long long redk[2][CX_NT / 64];
  __shared__ int redr[2][CX_NT / 64];
  const int ld = INV ? 2 * n : n;
  const size_t mat = (size_t)n * ld;
  const int64_t b = blockIdx.x;
  cx<T>* M = use_lds ? (cx<T>*)smem : Wg + (size_t)b * mat;
  int* prow = (int*)(smem + (use_lds ? mat * sizeof(cx<T>) : 0));
  unsigned char* asg = (unsigned char*)(prow + n);

  cload<T>(a + (size_t)b * n * n, n, skew, M, ld, INV);
  for (int r = threadIdx.x; r < n; r += CX_NT) asg[r] = 0;
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  double logabs = 0.0;
  double2 sgn = make_double2(1.0, 0.0);
  bool singular = false;
  for (int j = 0; j < n; ++j) {
    unsigned long long k = 0;
    int row = 0x7fffffff;
    for (int r = threadIdx.x; r < n; r += CX_NT)
      if (!asg[r]) take_better(k, row, ckey<T>(M[(size_t)r * ld + j]), r);
    const int p = block_argmax<CX_NT>(k, row, redk[j & 1], redr[j & 1]);
    const cx<T> piv = M[(size_t)p * ld + j];
    if (czero(piv))
      singular = true;
    else
      acc_pivot(sgn, logabs, (double)piv.re, (double)piv.im);
    const cx<T> rinv = crecip(piv);  // recip(0) = 0: a zero pivot updates nothing
    if (threadIdx.x == 0) {
      prow[j] = p;
      asg[p] = 1;
    }
    const cx<T>* P = M + (size_t)p * ld;
    for (int r = wave; r < n; r += CX_NT / 64) {
      if (r == p || (!INV && asg[r])) continue;
      cx<T>* R = M + (size_t)r * ld;
      const cx<T> l = cmul(R[j], rinv);
      for (int c = j + 1 + lane; c < ld; c += 64) R[c] = cfms(R[c], l, P[c]);
    }
    __syncthreads();
  }

  // parity of j -> prow[j] (n - number of cycles) by thread 0; asg reused as the marks
  if (threadIdx.x == 0) {
    for (int r = 0; r < n; ++r) asg[r] = 0;
    int cycles = 0;
    for (int s = 0; s < n; ++s) {
      if (asg[s]) continue;
      ++cycles;
      for (int t = s; !asg[t]; t = prow[t]) asg[t] = 1;
    }
    if ((n - cycles) & 1) sgn = make_double2(-sgn.x, -sgn.y);
    write_sl<T>(sign_out, logabs_out, b, singular, sgn, logabs);
  }
  if constexpr (INV) {
    cx<T>* O = out + (size_t)b * n * n;
    const bool zero = singular || (gate && czero(gate[b]));
    bool bad = false;
    if (!zero) {
      // A^-1[j, c] = M[prow[j], n + c] / pivot_j; out_t: O[c, j] (A^-T), else O[j, c]
      for (int e = threadIdx.x; e < n * n; e += CX_NT) {
        const int r = e / n, q = e - r * n;
        const int j = out_t ? q : r, c = out_t ? r : q;
        const cx<T>* Pj = M + (size_t)prow[j] * ld;
        const cx<T> v = cmul(Pj[n + c], crecip(Pj[j]));
        bad |= !(isfinite(v.re) && isfinite(v.im));
        O[e] = v;
      }
    }
    if (zero || __syncthreads_or(bad))
      for (int e = threadIdx.x; e < n * n; e += CX_NT) O[e] = cx<T>{T(0), T(0)};
  }
}

template <class T>
__global__ __launch_bounds__(CX_NT) void cpr_kernel(const cx<T>* __restrict__ a, int n, int skew, cx<T>* Wg,
                                                    int use_lds, cx<T>* __restrict__ sign_out,
                                                    T* __restrict__ logabs_out) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ unsigned long long redk[2][CX_NT / 64];
  __shared__ int redr[2][CX_NT / 64];
  const size_t mat = (size_t)n * n;
  const int64_t b = blockIdx.x;
  if (n & 1) {  // odd n: pf = 0
    if (threadIdx.x == 0) write_sl<T>(sign_out, logabs_out, b, true, make_double2(0.0, 0.0), 0.0);
    return;
  }
  cx<T>* M = use_lds ? (cx<T>*)smem : Wg + (size_t)b * mat;
  cload<T>(a + (size_t)b * mat, n, skew, M, n, false);
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  double logabs = 0.0;
  double2 sgn = make_double2(1.0, 0.0);
  bool singular = false;
  for (int c = 0; c + 1 < n; c += 2) {
    unsigned long long k = 0;
    int row = 0x7fffffff;
    // |S[r, c]| = |S[c, r]|: the candidates read along row c
    for (int r = c + 1 + threadIdx.x; r < n; r += CX_NT) take_better(k, row, ckey<T>(M[(size_t)c * n + r]), r);
    const int p = block_argmax<CX_NT>(k, row, redk[(c >> 1) & 1], redr[(c >> 1) & 1]);
    const int q = c + 1;
    if (p != q) {  // swap rows p, q over columns >= c, then columns p, q over rows >= c
      sgn = make_double2(-sgn.x, -sgn.y);
      for (int x = c + threadIdx.x; x < n; x += CX_NT) {
        const cx<T> u = M[(size_t)p * n + x], v = M[(size_t)q * n + x];
        M[(size_t)p * n + x] = v;
        M[(size_t)q * n + x] = u;
      }
      __syncthreads();
      for (int x = c + threadIdx.x; x < n; x += CX_NT) {
        const cx<T> u = M[(size_t)x * n + p], v = M[(size_t)x * n + q];
        M[(size_t)x * n + p] = v;
        M[(size_t)x * n + q] = u;
      }
      __syncthreads();
    }
    const cx<T> d = M[(size_t)c * n + q];
    if (czero(d)) {
      singular = true;
      break;
    }
    acc_pivot(sgn, logabs, (double)d.re, (double)d.im);
    const cx<T> rd = crecip(d);
    // tau = -S[:, c] / d = S[c, :] / d, w = S[:, q] = -S[q, :] (rows c and q contiguous);
    // S[r, x] += tau_r w_x - w_r tau_x
    const cx<T>* Rc = M + (size_t)c * n;
    const cx<T>* Rq = M + (size_t)q * n;
    for (int r = q + 1 + wave; r < n; r += CX_NT / 64) {
      cx<T>* R = M + (size_t)r * n;
      const cx<T> tr = cmul(Rc[r], rd);
      const cx<T> wr = {-Rq[r].re, -Rq[r].im};
      for (int x = q + 1 + lane; x < n; x += 64) {
        const cx<T> wx = {-Rq[x].re, -Rq[x].im};
        const cx<T> tx = cmul(Rc[x], rd);
        const cx<T> t1 = cmul(tr, wx), t2 = cmul(wr, tx);
        R[x] = cx<T>{R[x].re + (t1.re - t2.re), R[x].im + (t1.im - t2.im)};
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) write_sl<T>(sign_out, logabs_out, b, singular, sgn, logabs);
}

template <class T>
bool cx_in_lds(int n, int ld) {
  return (size_t)n * ld * sizeof(cx<T>) <= CX_LDS_MAX;
}

template <class T>
size_t cx_matrix_ws(int64_t batch, int n, int ld) {
  if (batch <= 0 || n <= 0 || cx_in_lds<T>(n, ld)) return 0;
  return (size_t)batch * n * ld * sizeof(cx<T>);
}

size_t cx_lds_bytes(size_t mat_bytes, int n, bool lds, bool maps) {
  size_t bytes = lds ? mat_bytes : 0;
  if (maps) bytes += (size_t)n * sizeof(int) + ((n + 15) / 16) * 16;
  return bytes ? bytes : 16;
}

size_t align_up(size_t x) { return (x + 255) / 256 * 256; }

template <class T>
int launch_cgj(const T* a, int n, int skew, int64_t batch, T* sign, T* logabs, T* out, int out_t, const T* gate,
               void* ws, size_t ws_bytes, hipStream_t s) {
  const bool inv = out != nullptr;
  const int ld = inv ? 2 * n : n;
  const bool lds = cx_in_lds<T>(n, ld);
  if (!lds && (!ws || ws_bytes < cx_matrix_ws<T>(batch, n, ld))) return FX_ERR_WORKSPACE;
  const size_t shm = cx_lds_bytes((size_t)n * ld * sizeof(cx<T>), n, lds, true);
  const dim3 grid((unsigned)batch);
  const cx<T>* A = reinterpret_cast<const cx<T>*>(a);
  cx<T>* W = (cx<T>*)ws;
  cx<T>* sg = reinterpret_cast<cx<T>*>(sign);
  if (inv)
    cgj_kernel<T, true><<<grid, CX_NT, shm, s>>>(A, n, skew, W, lds, sg, logabs, reinterpret_cast<cx<T>*>(out),
                                                 out_t, reinterpret_cast<const cx<T>*>(gate));
  else
    cgj_kernel<T, false><<<grid, CX_NT, shm, s>>>(A, n, skew, W, lds, sg, logabs, nullptr, 0, nullptr);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

template <class T>
int launch_cpr(const T* a, int n, int skew, int64_t batch, T* sign, T* logabs, void* ws, size_t ws_bytes,
               hipStream_t s) {
  const bool lds = cx_in_lds<T>(n, n);
  if (!lds && (!ws || ws_bytes < cx_matrix_ws<T>(batch, n, n))) return FX_ERR_WORKSPACE;
  const size_t shm = cx_lds_bytes((size_t)n * n * sizeof(cx<T>), n, lds, false);
  cpr_kernel<T><<<dim3((unsigned)batch), CX_NT, shm, s>>>(reinterpret_cast<const cx<T>*>(a), n, skew, (cx<T>*)ws,
                                                          lds, reinterpret_cast<cx<T>*>(sign), logabs);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

// The alignment contract of the ABI (matrix-shaped and workspace pointers 16-byte
// aligned; sign / logabs aligned to their element size) and the size limits.
template <class T>
int check_cx_args(const void* a, int64_t batch, int n, const void* sign, const void* logabs, const void* out,
                  const void* ws) {
  if (batch < 0 || n < 0) return FX_ERR_INVALID_ARGUMENT;
  if (n > CX_MAXN) return FX_ERR_UNSUPPORTED;
  if (batch > 0 && (!sign || !logabs || (n > 0 && !a))) return FX_ERR_INVALID_ARGUMENT;
  auto mis = [](const void* p, uintptr_t m) { return ((uintptr_t)p & m) != 0; };
  if (mis(a, 15) || mis(out, 15) || mis(ws, 15) || mis(sign, 2 * sizeof(T) - 1) || mis(logabs, sizeof(T) - 1))
    return FX_ERR_INVALID_ARGUMENT;
  if (batch > 0x7fffffff) return FX_ERR_UNSUPPORTED;
  return FX_OK;
}

// sign = 1, logabs = 0 for every member (n = 0)
template <class T>
__global__ void cx_empty_kernel(T* sign, T* logabs, int64_t batch) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < batch) {
    sign[2 * i] = T(1);
    sign[2 * i + 1] = T(0);
    logabs[i] = T(0);
  }
}

template <class T>
int cx_empty(T* sign, T* logabs, int64_t batch, hipStream_t s) {
  cx_empty_kernel<T><<<dim3((unsigned)((batch + 255) / 256)), 256, 0, s>>>(sign, logabs, batch);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

template <class T>
size_t slogdet_ws(int64_t batch, int n) {
  return n > CX_MAXN ? 0 : cx_matrix_ws<T>(batch, n, n);
}
template <class T>
size_t slogdet_parts_ws(int64_t batch, int n) {
  return n > CX_MAXN ? 0 : cx_matrix_ws<T>(batch, n, 2 * n);
}

template <class T>
int slogdet(const T* a, int64_t batch, int n, T* sign, T* logabs, void* ws, size_t wsb, hipStream_t s) {
  const int st = check_cx_args<T>(a, batch, n, sign, logabs, nullptr, ws);
  if (st != FX_OK || batch == 0) return st;
  if (n == 0) return cx_empty<T>(sign, logabs, batch, s);
  return launch_cgj<T>(a, n, 0, batch, sign, logabs, nullptr, 0, nullptr, ws, wsb, s);
}

template <class T>
int slogdet_parts(const T* a, int64_t batch, int n, T* sign, T* logabs, T* inv_t, void* ws, size_t wsb,
                  hipStream_t s) {
  const int st = check_cx_args<T>(a, batch, n, sign, logabs, inv_t, ws);
  if (st != FX_OK || batch == 0) return st;
  if (n == 0) return cx_empty<T>(sign, logabs, batch, s);
  return launch_cgj<T>(a, n, 0, batch, sign, logabs, inv_t, 1, nullptr, ws, wsb, s);
}

template <class T>
size_t slogpf_ws(int64_t batch, int n) {
  return n > CX_MAXN ? 0 : cx_matrix_ws<T>(batch, n, n);
}

template <class T>
size_t slogpf_parts_ws(int64_t batch, int n) {
  if (n > CX_MAXN || batch <= 0) return 0;
  return align_up(slogpf_ws<T>(batch, n)) + align_up(cx_matrix_ws<T>(batch, n, 2 * n)) +
         align_up((size_t)batch * 3 * sizeof(T));
}

template <class T>
int slogpf(const T* a, int64_t batch, int n, int skew, T* sign, T* logabs, void* ws, size_t wsb, hipStream_t s) {
  const int st = check_cx_args<T>(a, batch, n, sign, logabs, nullptr, ws);
  if (st != FX_OK || batch == 0) return st;
  if (n == 0) return cx_empty<T>(sign, logabs, batch, s);
  return launch_cpr<T>(a, n, skew != 0, batch, sign, logabs, ws, wsb, s);
}

// S^-1 by Gauss-Jordan on the same S (zeroed where the Parlett-Reid run found pf = 0;
// every member for odd n), after the Parlett-Reid run for sign / logabs.
template <class T>
int slogpf_parts(const T* a, int64_t batch, int n, int skew, int adjugate, T* sign, T* logabs, T* g, void* ws,
                 size_t wsb, hipStream_t s) {
  int st = check_cx_args<T>(a, batch, n, sign, logabs, g, ws);
  if (st != FX_OK || batch == 0) return st;
  if (adjugate) return FX_ERR_UNSUPPORTED;
  if (!g) return slogpf<T>(a, batch, n, skew, sign, logabs, ws, wsb, s);
  if (n == 0) return cx_empty<T>(sign, logabs, batch, s);
  if (wsb < slogpf_parts_ws<T>(batch, n) || (!ws && slogpf_parts_ws<T>(batch, n))) return FX_ERR_WORKSPACE;
  const size_t pr = align_up(slogpf_ws<T>(batch, n));
  const size_t gj = align_up(cx_matrix_ws<T>(batch, n, 2 * n));
  char* base = (char*)ws;
  st = launch_cpr<T>(a, n, skew != 0, batch, sign, logabs, base, pr, s);
  if (st != FX_OK) return st;
  T* gsign = (T*)(base + pr + gj);
  T* glog = gsign + 2 * batch;
  return launch_cgj<T>(a, n, skew != 0, batch, gsign, glog, g, 0, sign, base + pr, gj, s);
}

}  // namespace
}  // namespace fx

using namespace fx;

extern "C" {

size_t fx_slogdet_c64_workspace(int64_t batch, int32_t n) { return slogdet_ws<float>(batch, n); }
size_t fx_slogdet_c128_workspace(int64_t batch, int32_t n) { return slogdet_ws<double>(batch, n); }

int fx_slogdet_c64(const float* a, int64_t batch, int32_t n, float* sign, float* logabs, void* workspace,
                   size_t workspace_bytes, fx_stream_t stream) {
  return slogdet<float>(a, batch, n, sign, logabs, workspace, workspace_bytes, (hipStream_t)stream);
}
int fx_slogdet_c128(const double* a, int64_t batch, int32_t n, double* sign, double* logabs, void* workspace,
                    size_t workspace_bytes, fx_stream_t stream) {
  return slogdet<double>(a, batch, n, sign, logabs, workspace, workspace_bytes, (hipStream_t)stream);
}

size_t fx_slogdet_parts_c64_workspace(int64_t batch, int32_t n) { return slogdet_parts_ws<float>(batch, n); }
size_t fx_slogdet_parts_c128_workspace(int64_t batch, int32_t n) { return slogdet_parts_ws<double>(batch, n); }

int fx_slogdet_parts_c64(const float* a, int64_t batch, int32_t n, float* sign, float* logabs, float* inv_t,
                         void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  return slogdet_parts<float>(a, batch, n, sign, logabs, inv_t, workspace, workspace_bytes, (hipStream_t)stream);
}
int fx_slogdet_parts_c128(const double* a, int64_t batch, int32_t n, double* sign, double* logabs, double* inv_t,
                          void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  return slogdet_parts<double>(a, batch, n, sign, logabs, inv_t, workspace, workspace_bytes, (hipStream_t)stream);
}

size_t fx_slogpf_c64_workspace(int64_t batch, int32_t n) { return slogpf_ws<float>(batch, n); }
size_t fx_slogpf_c128_workspace(int64_t batch, int32_t n) { return slogpf_ws<double>(batch, n); }

int fx_slogpf_c64(const float* a, int64_t batch, int32_t n, int32_t skew_symmetrize, float* sign, float* logabs,
                  void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  return slogpf<float>(a, batch, n, skew_symmetrize, sign, logabs, workspace, workspace_bytes, (hipStream_t)stream);
}
int fx_slogpf_c128(const double* a, int64_t batch, int32_t n, int32_t skew_symmetrize, double* sign,
                   double* logabs, void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  return slogpf<double>(a, batch, n, skew_symmetrize, sign, logabs, workspace, workspace_bytes,
                        (hipStream_t)stream);
}

size_t fx_slogpf_parts_c64_workspace(int64_t batch, int32_t n) { return slogpf_parts_ws<float>(batch, n); }
size_t fx_slogpf_parts_c128_workspace(int64_t batch, int32_t n) { return slogpf_parts_ws<double>(batch, n); }

int fx_slogpf_parts_c64(const float* a, int64_t batch, int32_t n, int32_t skew_symmetrize, int32_t adjugate,
                        float* sign, float* logabs, float* g, void* workspace, size_t workspace_bytes,
                        fx_stream_t stream) {
  return slogpf_parts<float>(a, batch, n, skew_symmetrize, adjugate, sign, logabs, g, workspace, workspace_bytes,
                             (hipStream_t)stream);
}
int fx_slogpf_parts_c128(const double* a, int64_t batch, int32_t n, int32_t skew_symmetrize, int32_t adjugate,
                         double* sign, double* logabs, double* g, void* workspace, size_t workspace_bytes,
                         fx_stream_t stream) {
  return slogpf_parts<double>(a, batch, n, skew_symmetrize, adjugate, sign, logabs, g, workspace,
                              workspace_bytes, (hipStream_t)stream);
}

}  // extern "C"
