// float64 path: slogdet / slogpf forward and their gradients (A^-T, S^-1) for
// 0 <= n <= 8192: one workgroup per matrix up to n = 128, the blocked kernels of lu64_impl.inc
// above.
//
// The reference takes float64 through the same entry points as float32 (dtype check
// `_prep`, src/fermix/api.py:24-31; 64-bit fields in src/fermix/_field.py:20-120, where
// "tf32x3" is rejected for 64-bit types, :265-275). Its arithmetic for these types is
// the generic path: LU with partial pivoting (`_slogdet_generic` / `_slog_from_lu`,
// src/fermix/_fallback.py:36-60), the inverse for the gradient (`_lu_parts_generic`,
// :63-97) and Parlett-Reid with the pivot swapped into column c + 1 and the rank-2
// update tau w^T - w tau^T (`_slogpf_generic`, :266-300).
//
// Kernels (each a single workgroup per matrix):
//  - n <= 128 (fx_tune.f64_reg_max_n), gjreg64_kernel<RW, NC, CH, INV> /
//    pfreg64_kernel<RW, NC, CH>: the matrix in registers, each thread a 16-column (n <= 64,
//    fx_tune.f64_strip16_max_n) or 32-column strip of one row; per column (pair) step the
//    owners post the pivot candidates and the pivot row(s) through LDS, two barriers;
//  - larger n, gj64_kernel<NT, INV>: the matrix in LDS when it fits in 60 KiB, else in a
//    per-matrix slice of the workspace (rows served from L2); it serves the inverse and
//    adjugate runs that the blocked kernels of lu64_impl.inc (LU, Parlett-Reid and the solves,
//    used above 128 for sign / logabs and A^-T, S^-1) leave to it.
// Gauss-Jordan (gj*): virtual partial pivoting (the pivot row of column j is the
// unassigned row of largest |x|, lowest row index on ties). Without INV only the
// unassigned rows are updated (an LU); with INV the assigned rows and an identity block
// [A | I] are eliminated too, and row j of A^-1 is row prow[j] of the right block over
// pivot j. Every element update is fma(-l, P[c], M[r, c]), l = M[r, j] * (1 / pivot), in
// both modes, so sign / logabs of the gradient call are bit-identical to the forward.
// Parlett-Reid (pfreg64_kernel): virtual pivoting (pair a = the lowest unassigned index,
// p = argmax |S[p, a]|; pf = sgn(pi) prod d_k); it adds round(tau_r w_x) - round(w_r
// tau_x) (no contraction), so the matrix stays exactly skew-symmetric. Above n = 128 the
// blocked Parlett-Reid of lu64_impl.inc swaps the pivot row / column into position c + 1 as the
// reference's generic path does. The register kernels are latency-bound per matrix
// (barriers per column step).
#include <algorithm>

#include "common.h"
#include "fermix_internal.h"

namespace fx {
namespace {

constexpr int F64_MAXN = 8192;
constexpr size_t F64_LDS_MAX = 60 * 1024;  // matrix bytes kept in LDS

size_t align_up_256(size_t x) { return (x + 255) / 256 * 256; }

// Loads S (skew != 0: (a - a^T) / 2) into M with row stride ld; with ident, M[:, n:2n] = I.
template <int NT>
__device__ __forceinline__ void load_matrix(const double* __restrict__ a, int n, int skew, double* M, int ld,
                                            bool ident) {
  for (int e = threadIdx.x; e < n * n; e += NT) {
    const int r = e / n, k = e - r * n;
    double v = a[e];
    if (skew) v = (v - a[(size_t)k * n + r]) * 0.5;
    M[(size_t)r * ld + k] = v;
    if (ident) M[(size_t)r * ld + n + k] = (r == k) ? 1.0 : 0.0;
  }
}

template <int NT, bool INV>
__global__ __launch_bounds__(NT) void gj64_kernel(const double* __restrict__ a, int n, int skew, double* Wg,
                                                 int use_lds, double* __restrict__ sign_out,
                                                 double* __restrict__ logabs_out, double* __restrict__ out, int out_t,
                                                 const double* __restrict__ gate) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ unsigned long long redk[2][NT / 64];
  __shared__ int redr[2][NT / 64];
  const int ld = INV ? 2 * n : n;
  const size_t mat = (size_t)n * ld;
  const int64_t b = blockIdx.x;
  double* M = use_lds ? (double*)smem : Wg + (size_t)b * mat;
  int* prow = (int*)(smem + (use_lds ? mat * sizeof(double) : 0));
  unsigned char* asg = (unsigned char*)(prow + n);
  const double* A = a + (size_t)b * n * n;

  load_matrix<NT>(A, n, skew, M, ld, INV);
  for (int r = threadIdx.x; r < n; r += NT) asg[r] = 0;
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  double logabs = 0.0, sgn = 1.0;
  bool singular = false;
  for (int j = 0; j < n; ++j) {
    unsigned long long k = 0;
    int row = 0x7fffffff;
    for (int r = threadIdx.x; r < n; r += NT)
      if (!asg[r]) take_better(k, row, key64(M[(size_t)r * ld + j]), r);
    const int p = block_argmax<NT>(k, row, redk[j & 1], redr[j & 1]);
    const double piv = M[(size_t)p * ld + j];
    double rinv = 0.0;  // recip(0) = 0: a zero pivot updates nothing
    if (piv == 0.0) {
      singular = true;
    } else {
      rinv = 1.0 / piv;
      logabs += log(fabs(piv));
      if (piv < 0.0) sgn = -sgn;
    }
    if (threadIdx.x == 0) {
      prow[j] = p;
      asg[p] = 1;
    }
    const double* P = M + (size_t)p * ld;
    for (int r = wave; r < n; r += NT / 64) {
      if (r == p || (!INV && asg[r])) continue;
      double* R = M + (size_t)r * ld;
      const double l = R[j] * rinv;
      for (int c = j + 1 + lane; c < ld; c += 64) R[c] = fma(-l, P[c], R[c]);
    }
    __syncthreads();
  }

  // parity of j -> prow[j] (n - number of cycles), by thread 0; asg reused as the marks
  if (threadIdx.x == 0) {
    for (int r = 0; r < n; ++r) asg[r] = 0;
    int cycles = 0;
    for (int s = 0; s < n; ++s) {
      if (asg[s]) continue;
      ++cycles;
      for (int t = s; !asg[t]; t = prow[t]) asg[t] = 1;
    }
    if ((n - cycles) & 1) sgn = -sgn;
    if (singular) {
      sign_out[b] = 0.0;
      logabs_out[b] = -INFINITY;
    } else {
      sign_out[b] = sgn;
      logabs_out[b] = logabs;
    }
  }
  if constexpr (INV) {
    double* O = out + (size_t)b * n * n;
    const bool zero = singular || (gate && gate[b] == 0.0);
    bool bad = false;
    if (!zero) {
      // A^-1[j, c] = M[prow[j], n + c] / pivot_j; out_t: O[c, j], else O[j, c]
      for (int e = threadIdx.x; e < n * n; e += NT) {
        const int r = e / n, c = e - r * n;
        const int j = out_t ? c : r, col = out_t ? r : c;
        const double* Pj = M + (size_t)prow[j] * ld;
        const double v = Pj[n + col] / Pj[j];
        bad |= !isfinite(v);
        O[e] = v;
      }
    }
    if (zero || __syncthreads_or(bad))
      for (int e = threadIdx.x; e < n * n; e += NT) O[e] = 0.0;
  }
}

// n <= RW (64 or 128): the same Gauss-Jordan with the matrix in registers. Thread t owns
// row r = t % RW, columns [q NC, q NC + NC) of [A | I] (q = t / RW, CH chunks); per column
// j the chunk holding column j posts its values (the multipliers' sources and the pivot
// candidates) and, after the pivot is known, the pivot row's owners post that row: two
// workgroup barriers per column, every element updated by its owner with the formula of
// gj64_kernel (fma(-l, P[c], M[r, c]), l = M[r, j] * rinv), so sign / logabs equal its
// bits, and the forward (INV = false) and the inverse (INV = true) agree bit for bit.
template <int RW, int NC, int CH, bool INV>
__global__ __launch_bounds__(RW* CH) void gjreg64_kernel(const double* __restrict__ a, int n, int skew,
                                                         double* __restrict__ sign_out,
                                                         double* __restrict__ logabs_out, double* __restrict__ out,
                                                         int out_t, const double* __restrict__ gate) {
  constexpr int NW = RW / 64;
  __shared__ double colj[2][RW];
  __shared__ double prowv[2][NC * CH];
  __shared__ unsigned long long redk[2][NW];
  __shared__ int redr[2][NW];
  __shared__ int pidx[RW];      // pivot row of column j
  __shared__ int pos[RW];       // column whose pivot row is r
  __shared__ double pivs[RW];   // pivot of column j
  const int t = threadIdx.x, r = t % RW, q = t / RW;
  const int64_t b = blockIdx.x;
  const double* A = a + (size_t)b * n * n;

  double M[NC];
  static_for<0, NC>([&](auto I) {
    const int c = q * NC + I.value;
    double v = 0.0;
    if (r < n) {
      if (c < n) {
        v = A[(size_t)r * n + c];
        if (skew) v = (v - A[(size_t)c * n + r]) * 0.5;
      } else if (INV && c < 2 * n) {
        v = (c - n == r) ? 1.0 : 0.0;
      }
    }
    M[I.value] = v;
  });

  bool asg = false, singular = false;
  double logabs = 0.0, sgn = 1.0;
  for (int j = 0; j < n; ++j) {
    const int buf = j & 1, qj = j / NC, ij = j - qj * NC;
    if (q == qj) {
      double v = 0.0;
      static_for<0, NC>([&](auto I) {
        if (I.value == ij) v = M[I.value];
      });
      // exact wave argmax of the 64-bit keys: the high words' maximum, then the low
      // words' maximum among the lanes holding it (DPP reductions), then the lowest such
      // lane (a ballot; lanes are consecutive rows)
      const unsigned long long k = (r < n && !asg) ? key64(v) : 0ull;
      const unsigned hi = (unsigned)(k >> 32), lo = (unsigned)k;
      const unsigned mh = wave_max_u32(hi);
      const unsigned ml = wave_max_u32(hi == mh ? lo : 0u);
      const unsigned long long win = __ballot(hi == mh && lo == ml);
      if ((r & 63) == 0) {
        redk[buf][r >> 6] = ((unsigned long long)mh << 32) | ml;
        redr[buf][r >> 6] = r + __ffsll((long long)win) - 1;
      }
      colj[buf][r] = v;
    }
    __syncthreads();
    unsigned long long k = redk[buf][0];
    int p = redr[buf][0];
#pragma unroll
    for (int i = 1; i < NW; ++i) take_better(k, p, redk[buf][i], redr[buf][i]);
    const double piv = colj[buf][p];
    double rinv = 0.0;  // the logs of the pivots are taken after the loop
    if (piv == 0.0) {
      singular = true;
    } else {
      rinv = 1.0 / piv;
      if (piv < 0.0) sgn = -sgn;
    }
    if (r == p) static_for<0, NC>([&](auto I) { prowv[buf][q * NC + I.value] = M[I.value]; });
    if (t == 0) {
      pidx[j] = p;
      pivs[j] = piv;
    }
    __syncthreads();
    if (r < n && r != p && (INV || !asg)) {
      const double l = colj[buf][r] * rinv;
      static_for<0, NC>([&](auto I) {
        const int c = q * NC + I.value;
        if (c > j) M[I.value] = fma(-l, prowv[buf][c], M[I.value]);
      });
    }
    if (r == p) asg = true;
  }

  // log|pivot_j| in parallel into colj[0] (free after the loop), summed in order by
  // thread 0 (sequential pivot order, as the reference's running logabs)
  __syncthreads();
  double* lg = colj[0];
  for (int j = t; j < n; j += RW * CH) lg[j] = log(fabs(pivs[j]));
  __syncthreads();
  if (t == 0) {  // parity of j -> pidx[j]; pos doubles as the visit marks first
    if (!singular)
      for (int j = 0; j < n; ++j) logabs += lg[j];
    for (int s = 0; s < n; ++s) pos[s] = 0;
    int cycles = 0;
    for (int s = 0; s < n; ++s) {
      if (pos[s]) continue;
      ++cycles;
      for (int u = s; !pos[u]; u = pidx[u]) pos[u] = 1;
    }
    if ((n - cycles) & 1) sgn = -sgn;
    sign_out[b] = singular ? 0.0 : sgn;
    logabs_out[b] = singular ? -INFINITY : logabs;
  }
  if constexpr (INV) {
    __syncthreads();
    for (int j = t; j < n; j += RW * CH) pos[pidx[j]] = j;
    __syncthreads();
    double* O = out + (size_t)b * n * n;
    const bool zero = singular || (gate && gate[b] == 0.0);
    bool bad = false;
    if (!zero && r < n) {
      // row r of the right block is row pos[r] of A^-1 times its pivot
      const int j = pos[r];
      const double pj = pivs[j];
      static_for<0, NC>([&](auto I) {
        const int c = q * NC + I.value - n;
        if (c >= 0 && c < n) {
          const double v = M[I.value] / pj;
          bad |= !isfinite(v);
          O[out_t ? (size_t)c * n + j : (size_t)j * n + c] = v;
        }
      });
    }
    if (zero || __syncthreads_or(bad))
      for (int e = t; e < n * n; e += RW * CH) O[e] = 0.0;
  }
}

// Exact wave argmax of 64-bit keys over the 64 lanes of a wave whose lanes hold the
// consecutive rows r0 .. r0 + 63: the high words' maximum, then the low words' maximum
// among the lanes holding it (DPP reductions), then the lowest such lane (ballot).
__device__ __forceinline__ void wave_argmax64(unsigned long long k, int r0, unsigned long long& kout, int& rout) {
  const unsigned hi = (unsigned)(k >> 32), lo = (unsigned)k;
  const unsigned mh = wave_max_u32(hi);
  const unsigned ml = wave_max_u32(hi == mh ? lo : 0u);
  const unsigned long long win = __ballot(hi == mh && lo == ml);
  kout = ((unsigned long long)mh << 32) | ml;
  rout = r0 + __ffsll((long long)win) - 1;
}

// Even n <= RW: Parlett-Reid with the matrix in registers (layout of gjreg64_kernel) and
// virtual pivoting: pair step k takes a = the lowest unassigned index and p = the
// unassigned row != a of largest |S[p, a]| (lowest index on ties); rows a and p are
// posted, d = S[a, p], and every unassigned row r adds
// round(tau_r w_x) - round(w_r tau_x) (tau = S[a, :] / d, w = -S[p, :], no contraction)
// to its entries, so the unassigned block stays exactly skew. pf(S) = sgn(pi) prod d_k
// for pi = (a_0, p_0, a_1, p_1, ...).
template <int RW, int NC, int CH>
__global__ __launch_bounds__(RW* CH) void pfreg64_kernel(const double* __restrict__ a, int n, int skew,
                                                         double* __restrict__ sign_out,
                                                         double* __restrict__ logabs_out) {
  constexpr int NW = RW / 64;
  __shared__ double rowa[2][NC * CH];
  __shared__ double rowp[2][NC * CH];
  __shared__ unsigned long long redk[2][NW];
  __shared__ int redr[2][NW];
  __shared__ int perm[RW];
  __shared__ double dv[RW / 2];
  const int t = threadIdx.x, r = t % RW, q = t / RW;
  const int64_t b = blockIdx.x;
  if (n & 1) {
    if (t == 0) {
      sign_out[b] = 0.0;
      logabs_out[b] = -INFINITY;
    }
    return;
  }
  const double* A = a + (size_t)b * n * n;
  double M[NC];
  static_for<0, NC>([&](auto I) {
    const int c = q * NC + I.value;
    double v = 0.0;
    if (r < n && c < n) {
      v = A[(size_t)r * n + c];
      if (skew) v = (v - A[(size_t)c * n + r]) * 0.5;
    }
    M[I.value] = v;
  });

  unsigned long long used0 = 0, used1 = 0;  // assigned indices (uniform)
  bool asg = false, singular = false;
  double sgn = 1.0;
  int steps = 0;
  for (int k = 0; 2 * k < n; ++k) {
    const int buf = k & 1;
    const int ai = ~used0 ? __ffsll((long long)~used0) - 1 : 64 + __ffsll((long long)~used1) - 1;
    const int qa = ai / NC, ia = ai - qa * NC;
    if (q == qa) {
      double v = 0.0;
      static_for<0, NC>([&](auto I) {
        if (I.value == ia) v = M[I.value];
      });
      unsigned long long kw;
      int rw;
      wave_argmax64((r < n && !asg && r != ai) ? key64(v) : 0ull, r & ~63, kw, rw);
      if ((r & 63) == 0) {
        redk[buf][r >> 6] = kw;
        redr[buf][r >> 6] = rw;
      }
    }
    if (r == ai) static_for<0, NC>([&](auto I) { rowa[buf][q * NC + I.value] = M[I.value]; });
    __syncthreads();
    unsigned long long kk = redk[buf][0];
    int p = redr[buf][0];
#pragma unroll
    for (int i = 1; i < NW; ++i) take_better(kk, p, redk[buf][i], redr[buf][i]);
    if (r == p) static_for<0, NC>([&](auto I) { rowp[buf][q * NC + I.value] = M[I.value]; });
    const double d = rowa[buf][p];
    if (t == 0) {
      perm[2 * k] = ai;
      perm[2 * k + 1] = p;
      dv[k] = d;
    }
    steps = k + 1;
    if (d == 0.0) {
      singular = true;
      break;
    }
    if (d < 0.0) sgn = -sgn;
    const double rd = 1.0 / d;
    __syncthreads();
    if (r < n && !asg && r != ai && r != p) {
      const double tr = rowa[buf][r] * rd, wr = -rowp[buf][r];
      static_for<0, NC>([&](auto I) {
#pragma clang fp contract(off)
        const int x = q * NC + I.value;
        const double tt = tr * (-rowp[buf][x]) - wr * (rowa[buf][x] * rd);
        M[I.value] = M[I.value] + tt;
      });
    }
    if (r == ai || r == p) asg = true;
    if (ai < 64) used0 |= 1ull << ai; else used1 |= 1ull << (ai - 64);
    if (p < 64) used0 |= 1ull << p; else used1 |= 1ull << (p - 64);
  }
  __syncthreads();
  if (t == 0) {
    double logabs = 0.0;
    if (!singular) {
      for (int k = 0; k < steps; ++k) logabs += log(fabs(dv[k]));
      // parity of i -> perm[i]: marks in the sign bit of a copy (perm values < n)
      int cycles = 0;
      for (int s = 0; s < n; ++s) {
        if (perm[s] < 0) continue;
        ++cycles;
        for (int u = s; perm[u] >= 0;) {
          const int nx = perm[u];
          perm[u] = -1;
          u = nx;
        }
      }
      if ((n - cycles) & 1) sgn = -sgn;
    }
    sign_out[b] = singular ? 0.0 : sgn;
    logabs_out[b] = singular ? -INFINITY : logabs;
  }
}

bool f64_in_lds(int n, int ld) { return (size_t)n * ld * sizeof(double) <= F64_LDS_MAX; }

size_t f64_matrix_ws(int64_t batch, int n, int ld) {
  if (batch <= 0 || n <= 0 || f64_in_lds(n, ld)) return 0;
  return (size_t)batch * n * ld * sizeof(double);
}

size_t f64_lds_bytes(int n, int ld, bool lds, bool maps) {
  size_t bytes = lds ? (size_t)n * ld * sizeof(double) : 0;
  if (maps) bytes += (size_t)n * sizeof(int) + ((n + 15) / 16) * 16;
  return bytes ? bytes : 16;
}

// slogdet forward for n <= TINY64_MAXN with several matrices per wave: G lanes per matrix
// (16 for n <= 16, else 32), lane r of a group holding row r in registers, no workgroup
// barrier. The arithmetic is gjreg64_kernel's forward element for element -- the same
// pivots (the exact 64-bit argmax: the high words' maximum, then the low words' among the
// lanes holding it, then the lowest such row), l = a[r][j] * (1 / piv) and one fma per
// entry of the unassigned rows, the logs summed in pivot order, the sign from the
// negative pivots and the permutation's parity -- so the gradient call
// (gjreg64_kernel<..., true>) returns this forward's bits. The pivot row reaches the
// group through LDS.
constexpr int TINY64_MAXN = 32;

template <int G>
__global__ __launch_bounds__(256) void lutiny64_kernel(const double* __restrict__ a, int n, int64_t batch,
                                                       double* __restrict__ sign_out,
                                                       double* __restrict__ logabs_out) {
  constexpr int MPW = 256 / G;  // matrices per workgroup
  __shared__ double ubuf[256], pbuf[256];
  __shared__ int ibuf[256];
  const int tid = threadIdx.x, lane = tid & 63;
  const int r = tid % G;       // row within the matrix
  const int gbase = lane - r;  // first lane of the group
  double* const ub = ubuf + (tid - r);  // the group's pivot row
  double* const pv = pbuf + (tid - r);  // its pivots, in column order
  int* const pi = ibuf + (tid - r);     // and their rows
  const int64_t mi = (int64_t)blockIdx.x * MPW + tid / G;
  const bool live = mi < batch;
  const double* Ab = a + (live ? mi : 0) * (int64_t)n * n;
  double M[G];
  const int rr = min(r, n - 1);
#pragma unroll
  for (int c = 0; c < G; ++c) M[c] = Ab[(int64_t)rr * n + min(c, n - 1)];
#pragma unroll
  for (int c = 0; c < G; ++c) M[c] = (r < n && c < n) ? M[c] : 0.0;
  bool asg = false, singular = false;
  double sgn = 1.0;
  static_for<0, G>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    if (j < n) {
      const unsigned long long k = (r < n && !asg) ? key64(M[j]) : 0ull;
      const unsigned hi = (unsigned)(k >> 32), lo = (unsigned)k;
      const unsigned mh = group_max_u32<G>(hi);
      const unsigned ml = group_max_u32<G>(hi == mh ? lo : 0u);
      const int p = group_first<G>(k != 0 && hi == mh && lo == ml, gbase);
      const double piv = __shfl(M[j], gbase + p);
      double rinv = 0.0;
      if (piv == 0.0) {
        singular = true;
      } else {
        rinv = 1.0 / piv;
        if (piv < 0.0) sgn = -sgn;
      }
      if (r == p) {
#pragma unroll
        for (int c = j + 1; c < G; ++c) ub[c] = M[c];
        pv[j] = piv;
        pi[j] = p;
      }
      wave_lds_fence();
      if (r < n && r != p && !asg) {
        const double l = M[j] * rinv;
#pragma unroll
        for (int c = j + 1; c < G; ++c) M[c] = fma(-l, ub[c], M[c]);
      }
      if (r == p) asg = true;
      wave_lds_fence();  // every read of ub precedes the next step's writes
    }
  });
  if (live && r == 0) {
    double logabs = 0.0;
    if (!singular)
      for (int j = 0; j < n; ++j) logabs += log(fabs(pv[j]));
    unsigned seen = 0;  // parity of j -> pi[j] from its cycles
    int cycles = 0;
    for (int s0 = 0; s0 < n; ++s0) {
      if ((seen >> s0) & 1u) continue;
      ++cycles;
      for (int u = s0; !((seen >> u) & 1u); u = pi[u]) seen |= 1u << u;
    }
    if ((n - cycles) & 1) sgn = -sgn;
    sign_out[mi] = singular ? 0.0 : sgn;
    logabs_out[mi] = singular ? -INFINITY : logabs;
  }
}

int launch_gj64(const double* a, int n, int skew, int64_t batch, double* sign, double* logabs, double* out,
                int out_t, const double* gate, void* ws, size_t ws_bytes, hipStream_t s) {
  const bool inv = out != nullptr;
  const int ld = inv ? 2 * n : n;
  if (!inv && !skew && n >= 1 && n <= TINY64_MAXN) {  // several matrices per wave
    if (n <= 16)
      lutiny64_kernel<16><<<dim3((unsigned)((batch + 15) / 16)), 256, 0, s>>>(a, n, batch, sign, logabs);
    else
      lutiny64_kernel<32><<<dim3((unsigned)((batch + 7) / 8)), 256, 0, s>>>(a, n, batch, sign, logabs);
    return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
  }
  if (n <= tune().f64_reg_max_n) {  // register-resident
    const dim3 grid((unsigned)batch);
    if (n <= tune().f64_strip16_max_n) {
      if (inv)
        gjreg64_kernel<64, 16, 8, true><<<grid, 512, 0, s>>>(a, n, skew, sign, logabs, out, out_t, gate);
      else
        gjreg64_kernel<64, 16, 4, false><<<grid, 256, 0, s>>>(a, n, skew, sign, logabs, out, out_t, gate);
    } else {
      if (inv)
        gjreg64_kernel<128, 32, 8, true><<<grid, 1024, 0, s>>>(a, n, skew, sign, logabs, out, out_t, gate);
      else
        gjreg64_kernel<128, 32, 4, false><<<grid, 512, 0, s>>>(a, n, skew, sign, logabs, out, out_t, gate);
    }
    return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
  }
  const bool lds = f64_in_lds(n, ld);
  if (!lds && (!ws || ws_bytes < f64_matrix_ws(batch, n, ld))) return FX_ERR_WORKSPACE;
  const size_t shm = f64_lds_bytes(n, ld, lds, true);
  const dim3 grid((unsigned)batch);
  double* W = (double*)ws;
  if (inv)
    gj64_kernel<1024, true><<<grid, 1024, shm, s>>>(a, n, skew, W, lds, sign, logabs, out, out_t, gate);
  else
    gj64_kernel<1024, false><<<grid, 1024, shm, s>>>(a, n, skew, W, lds, sign, logabs, out, out_t, gate);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

// spread: the blocked run's pair-pivot spread (lu64_impl.inc), left unwritten by the register
// kernels
int launch_pr64(const double* a, int n, int skew, int64_t batch, double* sign, double* logabs, void* ws,
                size_t ws_bytes, hipStream_t s, double* spread = nullptr) {
  if (n <= tune().f64_reg_max_n) {  // register-resident
    const dim3 grid((unsigned)batch);
    if (n <= tune().f64_strip16_max_n)
      pfreg64_kernel<64, 32, 2><<<grid, 128, 0, s>>>(a, n, skew, sign, logabs);
    else
      pfreg64_kernel<128, 32, 4><<<grid, 512, 0, s>>>(a, n, skew, sign, logabs);
    return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
  }
  return launch_pr64_blocked(a, n, skew, batch, sign, logabs, ws, ws_bytes, s, spread);  // lu64_impl.inc
}

// Workspace of the Gauss-Jordan path: none in registers (n <= f64_reg_max_n) or LDS.
size_t gj64_ws(int64_t batch, int n, bool inv) {
  return n <= tune().f64_reg_max_n ? 0 : f64_matrix_ws(batch, n, inv ? 2 * n : n);
}

// Argument checks shared by the float64 entry points: the alignment contract of the ABI
// (matrix-shaped and workspace pointers 16-byte aligned, sign / logabs 8-byte aligned).
int check_f64_args(const void* a, int64_t batch, int n, const void* sign, const void* logabs, const void* out,
                   const void* ws) {
  if (batch < 0 || n < 0) return FX_ERR_INVALID_ARGUMENT;
  if (n > F64_MAXN) return FX_ERR_UNSUPPORTED;
  if (batch > 0 && (!sign || !logabs || (n > 0 && !a))) return FX_ERR_INVALID_ARGUMENT;
  auto mis = [](const void* p, uintptr_t m) { return ((uintptr_t)p & m) != 0; };
  if (mis(a, 15) || mis(out, 15) || mis(ws, 15) || mis(sign, 7) || mis(logabs, 7)) return FX_ERR_INVALID_ARGUMENT;
  if (batch > 0x7fffffff) return FX_ERR_UNSUPPORTED;
  return FX_OK;
}

}  // namespace
}  // namespace fx

using namespace fx;

extern "C" {


// Above the register kernels the values come from the blocked LU (lu64_impl.inc) and the
// gradient's A^-T from the blocked solves of the same factorisation, so that a gradient
// call returns the forward's bits.
static bool lu64_path(int n) { return n > tune().f64_reg_max_n; }

size_t fx_slogdet_f64_workspace(int64_t batch, int32_t n) {
  fx::TunePin pin_;
  if (n > F64_MAXN) return 0;
  return lu64_path(n) ? lu64_workspace(batch, n) : gj64_ws(batch, n, false);
}

int fx_slogdet_f64(const double* a, int64_t batch, int32_t n, double* sign, double* logabs, void* workspace,
                   size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  const int st = check_f64_args(a, batch, n, sign, logabs, nullptr, workspace);
  if (st != FX_OK || batch == 0) return st;
  if (lu64_path(n)) return launch_lu64(a, n, batch, sign, logabs, workspace, workspace_bytes, (hipStream_t)stream);
  return launch_gj64(a, n, 0, batch, sign, logabs, nullptr, 0, nullptr, workspace, workspace_bytes,
                     (hipStream_t)stream);
}

size_t fx_slogdet_parts_f64_workspace(int64_t batch, int32_t n) {
  fx::TunePin pin_;
  if (n > F64_MAXN) return 0;
  return lu64_path(n) ? lu64_inverse_workspace(batch, n) : gj64_ws(batch, n, true);
}

int fx_slogdet_parts_f64(const double* a, int64_t batch, int32_t n, double* sign, double* logabs, double* inv_t,
                         void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  const int st = check_f64_args(a, batch, n, sign, logabs, inv_t, workspace);
  if (st != FX_OK || batch == 0) return st;
  if (!inv_t) return fx_slogdet_f64(a, batch, n, sign, logabs, workspace, workspace_bytes, stream);
  hipStream_t s = (hipStream_t)stream;
  if (!lu64_path(n))
    return launch_gj64(a, n, 0, batch, sign, logabs, inv_t, 1, nullptr, workspace, workspace_bytes, s);
  return launch_lu64_inverse(a, n, 0, batch, sign, logabs, nullptr, nullptr, nullptr, inv_t, 1, workspace,
                             workspace_bytes, s);
}

size_t fx_slogpf_f64_workspace(int64_t batch, int32_t n) {
  fx::TunePin pin_;
  return n > F64_MAXN || n <= tune().f64_reg_max_n ? 0 : pr64_workspace(batch, n);
}

int fx_slogpf_f64(const double* a, int64_t batch, int32_t n, int32_t skew_symmetrize, double* sign, double* logabs,
                  void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  const int st = check_f64_args(a, batch, n, sign, logabs, nullptr, workspace);
  if (st != FX_OK || batch == 0) return st;
  return launch_pr64(a, n, skew_symmetrize != 0, batch, sign, logabs, workspace, workspace_bytes,
                     (hipStream_t)stream);
}

size_t fx_slogpf_parts_f64_workspace(int64_t batch, int32_t n) {
  fx::TunePin pin_;
  if (n > F64_MAXN || batch <= 0) return 0;
  const size_t pr = fx_slogpf_f64_workspace(batch, n);
  const size_t inv = (lu64_path(n) ? align_up_256(lu64_inverse_workspace(batch, n)) : align_up_256(gj64_ws(batch, n, true))) +
                     align_up_256((size_t)batch * 2 * sizeof(double));
  // + the blocked Parlett-Reid run's pair-pivot spread (the adjugate's route gate)
  return align_up_256(pr) + std::max(inv, pf_adjugate_f64_ws(batch, n)) +
         (lu64_path(n) ? align_up_256((size_t)batch * sizeof(double)) : 0);
}

int fx_slogpf_parts_f64(const double* a, int64_t batch, int32_t n, int32_t skew_symmetrize, int32_t adjugate,
                        double* sign, double* logabs, double* g, void* workspace, size_t workspace_bytes,
                        fx_stream_t stream) {
  fx::TunePin pin_;
  int st = check_f64_args(a, batch, n, sign, logabs, g, workspace);
  if (st != FX_OK || batch == 0) return st;
  hipStream_t s = (hipStream_t)stream;
  if (!g) return fx_slogpf_f64(a, batch, n, skew_symmetrize, sign, logabs, workspace, workspace_bytes, stream);
  const size_t need = fx_slogpf_parts_f64_workspace(batch, n);
  if (workspace_bytes < need || (!workspace && need)) return FX_ERR_WORKSPACE;
  const size_t pr = align_up_256(fx_slogpf_f64_workspace(batch, n));
  const size_t gj = align_up_256(gj64_ws(batch, n, true));
  char* base = (char*)workspace;
  double* spread = lu64_path(n) ? (double*)(base + need - align_up_256((size_t)batch * sizeof(double))) : nullptr;
  st = launch_pr64(a, n, skew_symmetrize != 0, batch, sign, logabs, base, pr, s, spread);
  if (st != FX_OK || n == 0) return st;
  // the Pfaffian adjugate (cplx.hip): the LU route, or the pivot-replaced Parlett-Reid
  // formula for pf = 0 and numerically singular members
  if (adjugate)
    return pf_adjugate_f64(a, batch, n, skew_symmetrize != 0, g, sign, logabs, spread, base + pr,
                           need - pr - (spread ? align_up_256((size_t)batch * sizeof(double)) : 0), s);
  // S^-1 by Gauss-Jordan (register kernels' orders) or the blocked LU solves on the same S,
  // zeroed where the Parlett-Reid run found pf = 0 (every member for odd n)
  if (lu64_path(n)) {
    const size_t lw = align_up_256(lu64_inverse_workspace(batch, n));
    double* gsign = (double*)(base + pr + lw);
    return launch_lu64_inverse(a, n, skew_symmetrize != 0, batch, gsign, gsign + batch, sign, nullptr, nullptr, g, 0,
                               base + pr, lw, s);
  }
  double* gsign = (double*)(base + pr + gj);
  double* glog = gsign + batch;
  return launch_gj64(a, n, skew_symmetrize != 0, batch, gsign, glog, g, 0, sign, base + pr, gj, s);
}

}  // extern "C"
