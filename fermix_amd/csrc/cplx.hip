// complex64 / complex128 slogdet and slogpf (values, A^-T, S^-1, the det and pf adjugates;
// the latter two also for float64) -- the reference's
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
//  - cgj_kernel<F, MODE>: Gauss-Jordan with virtual partial pivoting (the pivot of column
//    j is the unassigned row of largest |re| + |im|, lowest row on ties), generic over the
//    field F (cx<float>, cx<double>, and double for the float64 det gradient). GJ_FWD
//    updates only the unassigned rows (an LU); GJ_INV / GJ_ADJ also the assigned rows and
//    the identity block [A | I], and row j of A^-1 is row prow[j] of the right block times
//    the pivot's reciprocal; GJ_ADJ forms det's gradient adj(A)^T from it, continued to
//    exactly singular A. The element update is the same in every mode, so the gradient
//    calls give bit-identical sign / logabs;
//  - cpr_kernel<T>: Parlett-Reid with the pivot row / column swapped into position c + 1,
//    d = S[c, c+1], tau = -S[:, c] / d, w = S[:, c+1] and the rank-2 update
//    tau w^T - w tau^T on the rows and columns after c + 1;
//  - the Pfaffian adjugate pf(S) S^-1 (pf's gradient) of the float64 and complex kinds:
//    cpfa_factor_kernel<F> (Parlett-Reid keeping the permutation, the pivots and the
//    factor column of the smallest pivot) and cgj_kernel<F, GJ_PFA> (the inverse of the
//    factorisation with that pivot and the zero pivots replaced by 1, formed from S while
//    it is loaded, and the reference's rank-2 correction on the way out).
// The phase and the log are accumulated in double for both kinds.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "fermix_internal.h"
#include "field.h"

namespace fx {
namespace {

constexpr int CX_MAXN = 8192;
constexpr size_t CX_LDS_MAX = 60 * 1024;  // matrix bytes kept in LDS
constexpr int CX_NT = 1024;
// complex orders above this run the blocked kernels of lu64_impl.inc (LU, solves, Parlett-Reid
// with the trailing updates on the fp64 MFMA); up to it, the one-workgroup kernels here
constexpr int CX_BLK_MIN = 64;

template <class F>
bool blocked(int n) {
  return !std::is_same<F, double>::value && n > CX_BLK_MIN;
}


template <class F>
__device__ __forceinline__ void write_sl(F* sign_out, typename Fd<F>::R* logabs_out, int64_t b, bool singular,
                                         double2 sgn, double logabs) {
  using R = typename Fd<F>::R;
  sign_out[b] = singular ? Fd<F>::zero() : Fd<F>::from(sgn);
  logabs_out[b] = singular ? R(-INFINITY) : R(logabs);
}

// S (skew != 0: (a - a^T) / 2) into M with row stride ld; with ident, M[:, n:2n] = I.

template <class F>
__device__ __forceinline__ void cload(const F* __restrict__ a, int n, int skew, F* M, int ld, bool ident) {
  for (int e = threadIdx.x; e < n * n; e += CX_NT) {
    const int r = e / n, k = e - r * n;
    F v = a[e];
    if (skew) v = half_diff(v, a[(size_t)k * n + r]);
    M[(size_t)r * ld + k] = v;
    if (ident) M[(size_t)r * ld + n + k] = (r == k) ? Fd<F>::one() : Fd<F>::zero();
  }
}

enum { GJ_FWD = 0, GJ_INV = 1, GJ_ADJ = 2, GJ_PFA = 3 };

// ---- the Pfaffian adjugate pf(S) S^-1 (the pf gradient) of the 64-bit and complex kinds.
// Parlett-Reid with the rows and columns permuted (P), P S P^T = L D L^T with D = diag_s(
// d_s J); K = the pair of the smallest |d| (the first exact zero if any); d~ = d with d_K
// and the exact zeros replaced by 1; L~ = L with the a-columns scaled by 1/d~ (columns
// a_s = 2s: w_s / d~_s, p_s = 2s + 1: tau_s). The reference's formula (src/fermix/
// _fallback.py:101-192, _pfinv.py:196-269) is
//   G = -P^T [a1 R + a2 (w v^T - v w^T)] P,  R = Y^T DY, Y = L~^-1,
//   w = R e_aK, v = Y^T e_aK, (a1, a2) = sgn(P) D_K (d_K, 1 - d_K), D_K = prod_{s != K} d_s.
// Here R comes from one inverse: R = -(T~)^-1 with T~ = L~ D~ L~^T, and T~ differs from
// P S P^T only in pair K (its entry d_K -> 1, its a-row / column beyond p_K scaled by 1/d_K:
// + (1 - d_K)(e_a e_p^T + e_a tau^T - transposes)) and at the zero pivots' pair entries
// (0 -> 1), so T~ is formed from S while it is loaded; v = Y^T e_aK is row a_K of L~^-1,
// = (L~^T X~)[p_K, :] = X~^T l with l = L~ e_pK (l = e_pK + tau_K) and X~ = (T~)^-1. With
// X~: G' = a1 X~ - a2 (w v^T - v w^T), w = -X~ e_aK, and G = P^T G' P. A second exact zero
// pivot z is lifted as in the reference: G = (G(d_z = 1) + G(d_z = -1)) / 2 (two
// evaluations, the second only for the members that have one); three or more give G = 0.
template <class F>
struct PfaHead {
  int K;     // pair of the smallest |d|
  int z;     // second zero pivot (lifted), -1 none, -2 three or more zero pivots (G = 0)
  int pad[2];
  F dK;
  F a1[2], a2[2];  // per evaluation (z = +1, z = -1), the 1/2 of the mean included
};

// byte offsets inside one member's slice of the adjugate's metadata
struct PfaLayout {
  size_t perm, ell, d, v, w, rp, stride;
};

template <class F>
PfaLayout pfa_layout(int n) {
  auto up = [](size_t x) { return (x + 15) / 16 * 16; };
  PfaLayout L;
  L.perm = up(sizeof(PfaHead<F>));
  L.ell = L.perm + up((size_t)n * sizeof(int));
  L.d = L.ell + up((size_t)n * sizeof(F));
  L.v = L.d + up((size_t)(n / 2) * sizeof(F));
  L.w = L.v + up((size_t)n * sizeof(F));
  L.rp = L.w + up((size_t)n * sizeof(F));
  L.stride = (L.rp + (size_t)n * sizeof(F) + 255) / 256 * 256;
  return L;
}

// Gauss-Jordan on [A | I] (MODE != GJ_FWD) or A. A zero pivot is taken as 1 for the
// elimination (the U~ convention: its column has no nonzero candidate, so only the
// assigned rows change), which leaves the forward unchanged and makes the right block
// X~ = (P^T L U~)^-1 in GJ_ADJ.
//  - GJ_INV: out = A^-1 (out_t: A^-T), zero for a zero pivot, a zero `gate` value or a
//    non-finite result;
//  - GJ_ADJ: out = adj(A)^T = d det / dA, from the same pivots: det(A) A^-T when no pivot
//    is zero; with zero pivots at columns k1 <= ... <= km (km the last) the rank-1
//    continuation s X~[km, i] X~[j, g(k1)] at (i, j), s = sgn(P) d_K (times
//    X~[k1, g(km)] for m = 2), g(k) = the row assigned at column k, d_K the product of
//    the nonzero pivots; m >= 3 gives 0 -- reference _det_gradT (src/fermix/_diff.py:
//    205-246) with U~^-1 e_k1 = X~ P^T L e_k1 = X~[:, g(k1)] (a zero pivot's multipliers
//    are zero) and (U~^-1)[k1, km] = X~[k1, g(km)]; a non-finite result gives 0.
template <class F, int MODE>
__global__ __launch_bounds__(CX_NT) void cgj_kernel(const F* __restrict__ a, int n, int skew, F* Wg, int use_lds,
                                                    F* __restrict__ sign_out, typename Fd<F>::R* __restrict__ logabs_out,
                                                    F* __restrict__ out, int out_t, const F* __restrict__ gate,
                                                    unsigned char* __restrict__ meta, PfaLayout PL, int eval) {
  using D = Fd<F>;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ unsigned long long redk[2][CX_NT / 64];
  __shared__ int redr[2][CX_NT / 64];
  constexpr bool RIGHT = MODE != GJ_FWD;
  const int ld = RIGHT ? 2 * n : n;
  const size_t mat = (size_t)n * ld;
  const int64_t b = blockIdx.x;
  F* M = use_lds ? (F*)smem : Wg + (size_t)b * mat;
  int* prow = (int*)(smem + (use_lds ? mat * sizeof(F) : 0));
  unsigned char* asg = (unsigned char*)(prow + n);

  if constexpr (MODE == GJ_PFA) {
    // with a gate: only the members whose gate value is 0 (pf = 0; the others' adjugate
    // formed by the caller)
    if (gate && !Fd<F>::is0(gate[b])) return;
    unsigned char* mb = meta + (size_t)b * PL.stride;
    const PfaHead<F>& h = *(const PfaHead<F>*)mb;
    if (h.z == -2) {  // three or more zero pivots: G = 0
      if (eval == 0)
        for (int e = threadIdx.x; e < n * n; e += CX_NT) out[(size_t)b * n * n + e] = D::zero();
      return;
    }
    if (eval == 1 && h.z < 0) return;
    // T~ (rows and columns permuted, pair K and the zero pivots' entries replaced)
    const int* perm = (const int*)(mb + PL.perm);
    const F* ell = (const F*)(mb + PL.ell);
    const F* dm = (const F*)(mb + PL.d);
    const int aK = 2 * h.K, pK = aK + 1;
    const F eK = D::sub(D::one(), h.dK);
    const F lift = eval ? D::sub(D::zero(), D::one()) : D::one();
    const F* A = a + (size_t)b * n * n;
    for (int e = threadIdx.x; e < n * n; e += CX_NT) {
      const int r = e / n, k = e - r * n;
      const int pr = perm[r], pk = perm[k];
      F v = A[(size_t)pr * n + pk];
      if (skew) v = half_diff(v, A[(size_t)pk * n + pr]);
      if (r == aK) {
        if (k == pK) v = D::add(v, eK);
        else if (k > pK) v = D::add(v, D::mul(eK, ell[k]));
      } else if (k == aK) {
        if (r == pK) v = D::sub(v, eK);
        else if (r > pK) v = D::sub(v, D::mul(eK, ell[r]));
      } else if ((r ^ k) == 1 && D::is0(dm[r >> 1])) {
        const F val = (r >> 1) == h.z ? lift : D::one();
        v = (r & 1) ? D::sub(v, val) : D::add(v, val);
      }
      M[(size_t)r * ld + k] = v;
      M[(size_t)r * ld + n + k] = (r == k) ? D::one() : D::zero();
    }
  } else {
    // GJ_ADJ with a gate: only the members whose gate value is 0 (exactly singular ones,
    // the others' adjugate formed by the caller)
    if (MODE == GJ_ADJ && gate && !Fd<F>::is0(gate[b])) return;
    cload<F>(a + (size_t)b * n * n, n, skew, M, ld, RIGHT);
  }
  for (int r = threadIdx.x; r < n; r += CX_NT) asg[r] = 0;
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  double logabs = 0.0;
  double2 sgn = make_double2(1.0, 0.0);
  int nzero = 0, k1 = 0, km = 0;  // zero pivots: count, first and last column
  for (int j = 0; j < n; ++j) {
    unsigned long long k = 0;
    int row = 0x7fffffff;
    for (int r = threadIdx.x; r < n; r += CX_NT)
      if (!asg[r]) take_better(k, row, D::key(M[(size_t)r * ld + j]), r);
    const int p = block_argmax<CX_NT>(k, row, redk[j & 1], redr[j & 1]);
    const F piv = M[(size_t)p * ld + j];
    F rinv;
    if (D::is0(piv)) {
      k1 = nzero ? k1 : j;
      km = j;
      ++nzero;
      rinv = D::one();
    } else {
      D::acc(sgn, logabs, piv);
      rinv = D::rcp(piv);
    }
    if (threadIdx.x == 0) {
      prow[j] = p;
      asg[p] = 1;
    }
    const F* P = M + (size_t)p * ld;
    for (int r = wave; r < n; r += CX_NT / 64) {
      if (r == p || (!RIGHT && asg[r])) continue;
      F* R = M + (size_t)r * ld;
      const F l = D::mul(R[j], rinv);
      for (int c = j + 1 + lane; c < ld; c += 64) R[c] = D::fms(R[c], l, P[c]);
    }
    __syncthreads();
  }

  if constexpr (MODE == GJ_PFA) {
    // X~[i, c] = M[prow[i], n + c] rp[i] (a zero pivot of T~, which exact arithmetic
    // excludes, taken as 1); v = X~^T l over the rows i >= p_K; w = -X~[:, a_K]
    unsigned char* mb = meta + (size_t)b * PL.stride;
    const PfaHead<F>& h = *(const PfaHead<F>*)mb;
    const int* perm = (const int*)(mb + PL.perm);
    const F* ell = (const F*)(mb + PL.ell);
    F* vv = (F*)(mb + PL.v);
    F* ww = (F*)(mb + PL.w);
    F* rp = (F*)(mb + PL.rp);
    const int aK = 2 * h.K, pK = aK + 1;
    for (int i = threadIdx.x; i < n; i += CX_NT) {
      const F* Pi = M + (size_t)prow[i] * ld;
      const F pv = Pi[i];
      const F r = D::is0(pv) ? D::one() : D::rcp(pv);
      rp[i] = r;
      ww[i] = D::sub(D::zero(), D::mul(Pi[n + aK], r));
    }
    __syncthreads();
    for (int j = threadIdx.x; j < n; j += CX_NT) {
      F acc = D::zero();
      for (int i = pK; i < n; ++i) acc = D::add(acc, D::mul(D::mul(ell[i], rp[i]), M[(size_t)prow[i] * ld + n + j]));
      vv[j] = acc;
    }
    __syncthreads();
    const F a1 = eval ? h.a1[1] : h.a1[0], a2 = eval ? h.a2[1] : h.a2[0];
    F* O = out + (size_t)b * n * n;
    for (int e = threadIdx.x; e < n * n; e += CX_NT) {
      const int i = e / n, j = e - i * n;
      const F x = D::mul(M[(size_t)prow[i] * ld + n + j], rp[i]);
      const F c = D::sub(D::mul(ww[i], vv[j]), D::mul(vv[i], ww[j]));
      F g = D::sub(D::mul(a1, x), D::mul(a2, c));
      F* o = O + (size_t)perm[i] * n + perm[j];
      if (eval) g = D::add(*o, g);
      *o = g;
    }
    return;
  }

  // parity of j -> prow[j] (n - number of cycles) by thread 0; asg reused as the marks
  if (threadIdx.x == 0) {
    int cycles = 0;
    for (int r = 0; r < n; ++r) asg[r] = 0;
    for (int s = 0; s < n; ++s) {
      if (asg[s]) continue;
      ++cycles;
      for (int t = s; !asg[t]; t = prow[t]) asg[t] = 1;
    }
    const bool odd = (n - cycles) & 1;
    write_sl<F>(sign_out, logabs_out, b, nzero > 0, odd ? make_double2(-sgn.x, -sgn.y) : sgn, logabs);
    if (MODE == GJ_ADJ) redk[0][0] = odd ? 1ull : 0ull;
  }
  if constexpr (MODE == GJ_INV) {
    F* O = out + (size_t)b * n * n;
    const bool zero = nzero > 0 || (gate && D::is0(gate[b]));
    bool bad = false;
    if (!zero) {
      // A^-1[j, c] = M[prow[j], n + c] / pivot_j; out_t: O[c, j], else O[j, c]
      for (int e = threadIdx.x; e < n * n; e += CX_NT) {
        const int r = e / n, q = e - r * n;
        const int j = out_t ? q : r, c = out_t ? r : q;
        const F* Pj = M + (size_t)prow[j] * ld;
        const F v = D::mul(Pj[n + c], D::rcp(Pj[j]));
        bad |= !D::finite(v);
        O[e] = v;
      }
    }
    if (zero || __syncthreads_or(bad))
      for (int e = threadIdx.x; e < n * n; e += CX_NT) O[e] = D::zero();
  }
  if constexpr (MODE == GJ_ADJ) {
    __syncthreads();
    const bool odd = redk[0][0] != 0;
    // X~[j, c] = M[g(j), n + c] / pivot_j, with a zero pivot taken as 1
    auto X = [&](int j, int c) {
      const F* Pj = M + (size_t)prow[j] * ld;
      const F pj = Pj[j];
      return D::mul(Pj[n + c], D::is0(pj) ? D::one() : D::rcp(pj));
    };
    // s = sgn(P) prod of the nonzero pivots (det itself when none is zero)
    const double e = exp(logabs);
    double2 sd = make_double2(sgn.x * e, sgn.y * e);
    if (odd) sd = make_double2(-sd.x, -sd.y);
    F s = D::from(sd);
    F* O = out + (size_t)b * n * n;
    bool bad = false;
    if (nzero == 0) {
      for (int q = threadIdx.x; q < n * n; q += CX_NT) {
        const int i = q / n, j = q - i * n;
        const F v = D::mul(s, X(j, i));
        bad |= !D::finite(v);
        O[q] = v;
      }
    } else if (nzero <= 2) {
      if (nzero == 2) s = D::mul(s, X(k1, prow[km]));
      const int g1 = prow[k1];
      for (int q = threadIdx.x; q < n * n; q += CX_NT) {
        const int i = q / n, j = q - i * n;
        const F v = D::mul(D::mul(s, X(km, i)), X(j, g1));
        bad |= !D::finite(v);
        O[q] = v;
      }
    }
    if (nzero > 2 || __syncthreads_or(bad))
      for (int q = threadIdx.x; q < n * n; q += CX_NT) O[q] = D::zero();
  }
}

template <class T>
__global__ __launch_bounds__(CX_NT) void cpr_kernel(const cx<T>* __restrict__ a, int n, int skew, cx<T>* Wg,
                                                    int use_lds, cx<T>* __restrict__ sign_out,
                                                    T* __restrict__ logabs_out) {
  using F = cx<T>;
  using D = Fd<F>;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ unsigned long long redk[2][CX_NT / 64];
  __shared__ int redr[2][CX_NT / 64];
  const size_t mat = (size_t)n * n;
  const int64_t b = blockIdx.x;
  if (n & 1) {  // odd n: pf = 0
    if (threadIdx.x == 0) write_sl<F>(sign_out, logabs_out, b, true, make_double2(0.0, 0.0), 0.0);
    return;
  }
  F* M = use_lds ? (F*)smem : Wg + (size_t)b * mat;
  cload<F>(a + (size_t)b * mat, n, skew, M, n, false);
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  double logabs = 0.0;
  double2 sgn = make_double2(1.0, 0.0);
  bool singular = false;
  for (int c = 0; c + 1 < n; c += 2) {
    unsigned long long k = 0;
    int row = 0x7fffffff;
    // |S[r, c]| = |S[c, r]|: the candidates read along row c
    for (int r = c + 1 + threadIdx.x; r < n; r += CX_NT) take_better(k, row, D::key(M[(size_t)c * n + r]), r);
    const int p = block_argmax<CX_NT>(k, row, redk[(c >> 1) & 1], redr[(c >> 1) & 1]);
    const int q = c + 1;
    if (p != q) {  // swap rows p, q over columns >= c, then columns p, q over rows >= c
      sgn = make_double2(-sgn.x, -sgn.y);
      for (int x = c + threadIdx.x; x < n; x += CX_NT) {
        const F u = M[(size_t)p * n + x], v = M[(size_t)q * n + x];
        M[(size_t)p * n + x] = v;
        M[(size_t)q * n + x] = u;
      }
      __syncthreads();
      for (int x = c + threadIdx.x; x < n; x += CX_NT) {
        const F u = M[(size_t)x * n + p], v = M[(size_t)x * n + q];
        M[(size_t)x * n + p] = v;
        M[(size_t)x * n + q] = u;
      }
      __syncthreads();
    }
    const F d = M[(size_t)c * n + q];
    if (D::is0(d)) {
      singular = true;
      break;
    }
    D::acc(sgn, logabs, d);
    const F rd = D::rcp(d);
    // tau = -S[:, c] / d = S[c, :] / d, w = S[:, q] = -S[q, :] (rows c and q contiguous);
    // S[r, x] += tau_r w_x - w_r tau_x
    const F* Rc = M + (size_t)c * n;
    const F* Rq = M + (size_t)q * n;
    for (int r = q + 1 + wave; r < n; r += CX_NT / 64) {
      F* R = M + (size_t)r * n;
      const F tr = D::mul(Rc[r], rd);
      const F wr = {-Rq[r].re, -Rq[r].im};
      for (int x = q + 1 + lane; x < n; x += 64) {
        const F wx = {-Rq[x].re, -Rq[x].im};
        const F tx = D::mul(Rc[x], rd);
        const F t1 = D::mul(tr, wx), t2 = D::mul(wr, tx);
        R[x] = F{R[x].re + (t1.re - t2.re), R[x].im + (t1.im - t2.im)};
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) write_sl<F>(sign_out, logabs_out, b, singular, sgn, logabs);
}

// Parlett-Reid of the Pfaffian adjugate (any field): the pair steps of cpr_kernel with
// whole rows swapped (so the factor's columns below each pair, which the L~ formula reads,
// move with the permutation), the permutation kept, and no stop at a zero pivot (tau = 0
// there: the step changes nothing, as in the reference's masked step). Thread 0 keeps the
// pivot statistics; the end writes the member's PfaHead, the permutation, d and
// l = L~ e_pK (e_pK + tau_K).
template <class F>
__global__ __launch_bounds__(CX_NT) void cpfa_factor_kernel(const F* __restrict__ a, int n, int skew, F* Wg,
                                                            int use_lds, unsigned char* __restrict__ meta,
                                                            PfaLayout PL, const F* __restrict__ gate) {
  using D = Fd<F>;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ unsigned long long redk[2][CX_NT / 64];
  __shared__ int redr[2][CX_NT / 64];
  __shared__ int sK;
  const size_t mat = (size_t)n * n;
  const int64_t b = blockIdx.x;
  if (gate && !D::is0(gate[b])) return;  // formed by the caller
  F* M = use_lds ? (F*)smem : Wg + (size_t)b * mat;
  int* perm = (int*)(smem + (use_lds ? mat * sizeof(F) : 0));
  unsigned char* mb = meta + (size_t)b * PL.stride;
  F* dm = (F*)(mb + PL.d);
  cload<F>(a + (size_t)b * mat, n, skew, M, n, false);
  for (int r = threadIdx.x; r < n; r += CX_NT) perm[r] = r;
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int par = 0, nzero = 0, z2 = -1, K = 0;  // thread 0's statistics
  double best = INFINITY, lsum = 0.0;
  double2 ph = make_double2(1.0, 0.0);
  for (int c = 0; c + 1 < n; c += 2) {
    unsigned long long k = 0;
    int row = 0x7fffffff;
    for (int r = c + 1 + threadIdx.x; r < n; r += CX_NT) take_better(k, row, D::key(M[(size_t)c * n + r]), r);
    const int p = block_argmax<CX_NT>(k, row, redk[(c >> 1) & 1], redr[(c >> 1) & 1]);
    const int q = c + 1;
    if (p != q) {
      par ^= 1;
      for (int x = threadIdx.x; x < n; x += CX_NT) {
        const F u = M[(size_t)p * n + x], v = M[(size_t)q * n + x];
        M[(size_t)p * n + x] = v;
        M[(size_t)q * n + x] = u;
      }
      if (threadIdx.x == 0) {
        const int t = perm[p];
        perm[p] = perm[q];
        perm[q] = t;
      }
      __syncthreads();
      for (int x = c + threadIdx.x; x < n; x += CX_NT) {
        const F u = M[(size_t)x * n + p], v = M[(size_t)x * n + q];
        M[(size_t)x * n + p] = v;
        M[(size_t)x * n + q] = u;
      }
      __syncthreads();
    }
    const F d = M[(size_t)c * n + q];
    if (threadIdx.x == 0) {
      dm[c >> 1] = d;
      const double m = D::mag(d);
      if (m < best) {  // first index on ties; the first zero pivot once there is one
        best = m;
        K = c >> 1;
      }
      if (D::is0(d)) {
        if (nzero == 1) z2 = c >> 1;
        ++nzero;
      } else {
        D::acc(ph, lsum, d);
      }
    }
    if (D::is0(d)) continue;  // tau = 0: the step leaves the matrix as it is
    const F rd = D::rcp(d);
    const F* Rc = M + (size_t)c * n;
    const F* Rq = M + (size_t)q * n;
    for (int r = q + 1 + wave; r < n; r += CX_NT / 64) {
      F* R = M + (size_t)r * n;
      const F tr = D::mul(Rc[r], rd);
      const F wr = D::sub(D::zero(), Rq[r]);
      for (int x = q + 1 + lane; x < n; x += 64) {
        const F wx = D::sub(D::zero(), Rq[x]);
        const F tx = D::mul(Rc[x], rd);
        R[x] = D::add(R[x], D::sub(D::mul(tr, wx), D::mul(wr, tx)));
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    PfaHead<F>& h = *(PfaHead<F>*)mb;
    h.K = K;
    h.pad[0] = h.pad[1] = 0;
    const F dK = dm[K];
    h.dK = dK;
    // D_K = prod_{s != K} d_s as phase * exp(log sum), without d_K (a zero d_K was never
    // accumulated) and without the lifted zero
    if (!D::is0(dK)) {
      lsum -= log(D::mag(dK));
      const double2 u = D::to2(dK);
      const double m = D::mag(dK);
      ph = c2mul(ph, make_double2(u.x / m, -u.y / m));
    }
    const double e = exp(lsum);
    const double sP = par ? -1.0 : 1.0;
    const double2 DK = make_double2(sP * ph.x * e, sP * ph.y * e);
    const double2 dK2 = D::to2(dK);
    double2 a1 = c2mul(DK, dK2), a2 = c2mul(DK, make_double2(1.0 - dK2.x, -dK2.y));
    h.z = nzero >= 3 ? -2 : nzero == 2 ? z2 : -1;
    if (nzero == 2) {  // mean of the lifted evaluations d_z = +1 and d_z = -1
      a1 = make_double2(0.5 * a1.x, 0.5 * a1.y);
      a2 = make_double2(0.5 * a2.x, 0.5 * a2.y);
    }
    h.a1[0] = D::from(a1);
    h.a2[0] = D::from(a2);
    h.a1[1] = D::from(make_double2(-a1.x, -a1.y));
    h.a2[1] = D::from(make_double2(-a2.x, -a2.y));
    sK = K;
  }
  __syncthreads();
  const int aK = 2 * sK, pK = aK + 1;
  const F rK = D::rcp(M[(size_t)aK * n + pK]);  // d_K (0 -> 0: tau_K = 0)
  int* po = (int*)(mb + PL.perm);
  F* ell = (F*)(mb + PL.ell);
  for (int r = threadIdx.x; r < n; r += CX_NT) {
    po[r] = perm[r];
    ell[r] = r < pK ? D::zero() : r == pK ? D::one() : D::sub(D::zero(), D::mul(M[(size_t)r * n + aK], rK));
  }
}

template <class F>
bool cx_in_lds(int n, int ld) {
  return (size_t)n * ld * sizeof(F) <= CX_LDS_MAX;
}

template <class F>
size_t cx_matrix_ws(int64_t batch, int n, int ld) {
  if (batch <= 0 || n <= 0 || cx_in_lds<F>(n, ld)) return 0;
  return (size_t)batch * n * ld * sizeof(F);
}

size_t cx_lds_bytes(size_t mat_bytes, int n, bool lds, bool maps) {
  size_t bytes = lds ? mat_bytes : 0;
  if (maps) bytes += (size_t)n * sizeof(int) + ((n + 15) / 16) * 16;
  return bytes ? bytes : 16;
}

size_t align_up(size_t x) { return (x + 255) / 256 * 256; }

// The element type of a kind's buffers (interleaved pairs for complex) and its real type.
template <class F>
struct Kind;
template <class T>
struct Kind<cx<T>> {
  using R = T;
};
template <>
struct Kind<double> {
  using R = double;
};
template <>
struct Kind<float> {
  using R = float;
};

// the largest order of a field's entry points here: float32 reaches these templates only
// above its own blocked kernels, up to the blocked kernels' float32 limit
template <class F>
constexpr int max_n() {
  return sizeof(F) == 4 ? GEN32_MAXN : CX_MAXN;
}

template <class F>
int launch_cgj(const void* a, int n, int skew, int64_t batch, void* sign, void* logabs, void* out, int mode,
               int out_t, const void* gate, void* ws, size_t ws_bytes, hipStream_t s) {
  using R = typename Kind<F>::R;
  const int ld = mode != GJ_FWD ? 2 * n : n;
  const bool lds = cx_in_lds<F>(n, ld);
  if (!lds && (!ws || ws_bytes < cx_matrix_ws<F>(batch, n, ld))) return FX_ERR_WORKSPACE;
  const size_t shm = cx_lds_bytes((size_t)n * ld * sizeof(F), n, lds, true);
  const dim3 grid((unsigned)batch);
  const F* A = (const F*)a;
  F* W = (F*)ws;
  F* sg = (F*)sign;
  R* lg = (R*)logabs;
  if (mode == GJ_INV)
    cgj_kernel<F, GJ_INV><<<grid, CX_NT, shm, s>>>(A, n, skew, W, lds, sg, lg, (F*)out, out_t, (const F*)gate, nullptr, PfaLayout{}, 0);
  else if (mode == GJ_ADJ)
    cgj_kernel<F, GJ_ADJ><<<grid, CX_NT, shm, s>>>(A, n, skew, W, lds, sg, lg, (F*)out, 1, (const F*)gate, nullptr,
                                                   PfaLayout{}, 0);
  else
    cgj_kernel<F, GJ_FWD><<<grid, CX_NT, shm, s>>>(A, n, skew, W, lds, sg, lg, nullptr, 0, nullptr, nullptr,
                                                  PfaLayout{}, 0);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

template <class T>
int launch_cpr(const void* a, int n, int skew, int64_t batch, void* sign, void* logabs, void* ws, size_t ws_bytes,
               hipStream_t s) {
  using F = cx<T>;
  const bool lds = cx_in_lds<F>(n, n);
  if (!lds && (!ws || ws_bytes < cx_matrix_ws<F>(batch, n, n))) return FX_ERR_WORKSPACE;
  const size_t shm = cx_lds_bytes((size_t)n * n * sizeof(F), n, lds, false);
  cpr_kernel<T><<<dim3((unsigned)batch), CX_NT, shm, s>>>((const F*)a, n, skew, (F*)ws, lds, (F*)sign, (T*)logabs);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

// The alignment contract of the ABI (matrix-shaped and workspace pointers 16-byte
// aligned; sign / logabs aligned to their element size) and the size limits.
template <class F>
int check_cx_args(const void* a, int64_t batch, int n, const void* sign, const void* logabs, const void* out,
                  const void* ws) {
  using R = typename Kind<F>::R;
  if (batch < 0 || n < 0) return FX_ERR_INVALID_ARGUMENT;
  if (n > max_n<F>()) return FX_ERR_UNSUPPORTED;
  if (batch > 0 && (!sign || !logabs || (n > 0 && !a))) return FX_ERR_INVALID_ARGUMENT;
  auto mis = [](const void* p, uintptr_t m) { return ((uintptr_t)p & m) != 0; };
  if (mis(a, 15) || mis(out, 15) || mis(ws, 15) || mis(sign, sizeof(F) - 1) || mis(logabs, sizeof(R) - 1))
    return FX_ERR_INVALID_ARGUMENT;
  if (batch > 0x7fffffff) return FX_ERR_UNSUPPORTED;
  return FX_OK;
}

// sign = 1, logabs = 0 for every member (n = 0)
template <class F>
__global__ void cx_empty_kernel(F* sign, typename Kind<F>::R* logabs, int64_t batch) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < batch) {
    sign[i] = Fd<F>::one();
    logabs[i] = 0;
  }
}

template <class F>
int cx_empty(void* sign, void* logabs, int64_t batch, hipStream_t s) {
  cx_empty_kernel<F><<<dim3((unsigned)((batch + 255) / 256)), 256, 0, s>>>((F*)sign, (typename Kind<F>::R*)logabs,
                                                                          batch);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

template <class F>
size_t slogdet_ws(int64_t batch, int n) {
  if (n > max_n<F>()) return 0;
  return blocked<F>(n) ? blk_lu_workspace<F>(batch, n) : cx_matrix_ws<F>(batch, n, n);
}
template <class F>
size_t slogdet_parts_ws(int64_t batch, int n) {
  if (n > max_n<F>()) return 0;
  return blocked<F>(n) ? blk_lu_inverse_workspace<F>(batch, n) : cx_matrix_ws<F>(batch, n, 2 * n);
}
// det's gradient: blocked, the LU solves plus the Gauss-Jordan run for the singular members
// (its [A | I] and its sign / logabs in scratch)
template <class F>
size_t det_parts_ws(int64_t batch, int n) {
  if (n > max_n<F>() || !blocked<F>(n) || batch <= 0) return slogdet_parts_ws<F>(batch, n);
  return align_up(blk_lu_inverse_workspace<F>(batch, n)) + align_up(cx_matrix_ws<F>(batch, n, 2 * n)) +
         align_up((size_t)batch * 2 * sizeof(F));
}

template <class F>
int slogdet(const void* a, int64_t batch, int n, void* sign, void* logabs, void* ws, size_t wsb, hipStream_t s) {
  const int st = check_cx_args<F>(a, batch, n, sign, logabs, nullptr, ws);
  if (st != FX_OK || batch == 0) return st;
  if (n == 0) return cx_empty<F>(sign, logabs, batch, s);
  using R = typename Kind<F>::R;
  if (blocked<F>(n)) return blk_lu<F>((const F*)a, n, batch, (F*)sign, (R*)logabs, ws, wsb, s);
  return launch_cgj<F>(a, n, 0, batch, sign, logabs, nullptr, GJ_FWD, 0, nullptr, ws, wsb, s);
}

template <class F>
int slogdet_parts(const void* a, int64_t batch, int n, void* sign, void* logabs, void* inv_t, void* ws, size_t wsb,
                  hipStream_t s) {
  const int st = check_cx_args<F>(a, batch, n, sign, logabs, inv_t, ws);
  if (st != FX_OK || batch == 0) return st;
  if (n == 0) return cx_empty<F>(sign, logabs, batch, s);
  using R = typename Kind<F>::R;
  if (blocked<F>(n)) {
    if (!inv_t) return blk_lu<F>((const F*)a, n, batch, (F*)sign, (R*)logabs, ws, wsb, s);
    return blk_lu_inverse<F>((const F*)a, n, 0, batch, (F*)sign, (R*)logabs, nullptr, nullptr, nullptr, (F*)inv_t, 1,
                             ws, wsb, s);
  }
  if (!inv_t) return launch_cgj<F>(a, n, 0, batch, sign, logabs, nullptr, GJ_FWD, 0, nullptr, ws, wsb, s);
  return launch_cgj<F>(a, n, 0, batch, sign, logabs, inv_t, GJ_INV, 1, nullptr, ws, wsb, s);
}

// det's gradient adj(A)^T with sign / logabs of the same run
template <class F>
int det_parts(const void* a, int64_t batch, int n, void* sign, void* logabs, void* adj_t, void* ws, size_t wsb,
              hipStream_t s) {
  const int st = check_cx_args<F>(a, batch, n, sign, logabs, adj_t, ws);
  if (st != FX_OK || batch == 0) return st;
  if (n > 0 && !adj_t) return FX_ERR_INVALID_ARGUMENT;
  if (n == 0) return cx_empty<F>(sign, logabs, batch, s);
  if (blocked<F>(n)) {  // as det_parts_f64 below: the regular members from the LU solves
    using R = typename Kind<F>::R;
    if (!ws || wsb < det_parts_ws<F>(batch, n)) return FX_ERR_WORKSPACE;
    const size_t lw = align_up(blk_lu_inverse_workspace<F>(batch, n)), gw = align_up(cx_matrix_ws<F>(batch, n, 2 * n));
    char* base = (char*)ws;
    const int r = blk_lu_inverse<F>((const F*)a, n, 0, batch, (F*)sign, (R*)logabs, nullptr, (const F*)sign,
                                    (const R*)logabs, (F*)adj_t, 1, base, lw, s);
    if (r != FX_OK) return r;
    F* gsign = (F*)(base + lw + gw);
    return launch_cgj<F>(a, n, 0, batch, gsign, gsign + batch, adj_t, GJ_ADJ, 1, sign, base + lw, gw, s);
  }
  return launch_cgj<F>(a, n, 0, batch, sign, logabs, adj_t, GJ_ADJ, 1, nullptr, ws, wsb, s);
}

// float64 above the register kernels' orders: sign / logabs (the forward's bits) and the
// regular members' adjugate det(A) A^-T from the blocked LU and its solves, the exactly
// singular members' from a Gauss-Jordan run gated to them (its values in scratch).
size_t det_parts_f64_ws(int64_t batch, int n) {
  if (n > CX_MAXN || batch <= 0) return 0;
  if (n <= tune().f64_reg_max_n) return slogdet_parts_ws<double>(batch, n);
  return align_up(lu64_inverse_workspace(batch, n)) + align_up(slogdet_parts_ws<double>(batch, n)) +
         align_up((size_t)batch * 2 * sizeof(double));
}

int det_parts_f64(const double* a, int64_t batch, int n, double* sign, double* logabs, double* adj_t, void* ws,
                  size_t wsb, hipStream_t s) {
  if (n <= tune().f64_reg_max_n) return det_parts<double>(a, batch, n, sign, logabs, adj_t, ws, wsb, s);
  const int st = check_cx_args<double>(a, batch, n, sign, logabs, adj_t, ws);
  if (st != FX_OK || batch == 0) return st;
  if (!adj_t) return FX_ERR_INVALID_ARGUMENT;
  const size_t need = det_parts_f64_ws(batch, n);
  if (!ws || wsb < need) return FX_ERR_WORKSPACE;
  const size_t lw = align_up(lu64_inverse_workspace(batch, n)), gw = align_up(slogdet_parts_ws<double>(batch, n));
  char* base = (char*)ws;
  const int r = launch_lu64_inverse(a, n, 0, batch, sign, logabs, nullptr, sign, logabs, adj_t, 1, base, lw, s);
  if (r != FX_OK) return r;
  double* gsign = (double*)(base + lw + gw);
  return launch_cgj<double>(a, n, 0, batch, gsign, gsign + batch, adj_t, GJ_ADJ, 1, sign, base + lw, gw, s);
}

template <class T>
size_t slogpf_ws(int64_t batch, int n) {
  if (n > CX_MAXN) return 0;
  return blocked<cx<T>>(n) ? blk_pr_workspace<cx<T>>(batch, n) : cx_matrix_ws<cx<T>>(batch, n, n);
}

template <class T>
int launch_pf(const T* a, int n, int skew, int64_t batch, T* sign, T* logabs, void* ws, size_t wsb, hipStream_t s,
              double* spread = nullptr) {
  if (blocked<cx<T>>(n))
    return blk_pr<cx<T>>((const cx<T>*)a, n, skew, batch, (cx<T>*)sign, logabs, ws, wsb, s, spread);
  return launch_cpr<T>(a, n, skew, batch, sign, logabs, ws, wsb, s);
}

// The blocked Pfaffian adjugate takes pf(S) S^-1 from an LU of S scaled by the
// Parlett-Reid run's pf. That is accurate while S is well away from singular; near a
// rank-(n - 2) S the LU's two small pivots and the Parlett-Reid run's small pair pivot
// come from different factorisations, so the product is off by O(1). Members whose
// Parlett-Reid pair pivots span more than this (log max |d| - log min |d|: |d_min| below
// 2^-18 |d_max| in double precision, 2^-8 in single) take the pivot-replaced
// Parlett-Reid formula instead (exact for singular S, as the reference's
// src/fermix/_pfinv.py:196-269). Random members sit far inside it: |d_min| / |d_max| is
// 0.03 .. 0.1 for N(0, 1/n) skew matrices at n = 256 .. 1024.
template <class R>
constexpr double pf_lu_spread_max() {
  return (sizeof(R) == 8 ? 18.0 : 8.0) * 0.69314718055994531;
}

// gate[b] = sign[b] where the member takes the LU route (spread within the limit), else 0
template <class F>
__global__ void pf_gate_kernel(const F* __restrict__ sign, const double* __restrict__ spread, double lim,
                               F* __restrict__ gate, int64_t batch) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  gate[b] = spread[b] <= lim ? sign[b] : Fd<F>::zero();
}

template <class F>
int pf_gate(const F* sign, const double* spread, F* gate, int64_t batch, hipStream_t s) {
  pf_gate_kernel<F><<<dim3((unsigned)((batch + 255) / 256)), 256, 0, s>>>(sign, spread,
                                                                        pf_lu_spread_max<typename Fd<F>::R>(), gate,
                                                                        batch);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

// The Pfaffian adjugate's workspace: the Parlett-Reid matrix and then [T~ | I] (the same
// bytes; none while they fit in LDS) and the per-member metadata.
template <class F>
size_t pf_adjugate_ws(int64_t batch, int n) {
  if (batch <= 0 || n <= 0 || (n & 1) || n > max_n<F>()) return 0;
  const size_t mats = std::max(cx_matrix_ws<F>(batch, n, n), cx_matrix_ws<F>(batch, n, 2 * n));
  return align_up(mats) + align_up((size_t)batch * pfa_layout<F>(n).stride);
}

template <class F>
__global__ void cx_zero_kernel(F* g, int64_t count) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < count; e += (int64_t)gridDim.x * blockDim.x)
    g[e] = Fd<F>::zero();
}

template <class F>
int cx_zero(F* g, int64_t count, hipStream_t s) {
  if (count <= 0) return FX_OK;
  const int64_t blocks = std::min<int64_t>((count + 255) / 256, 65536);
  cx_zero_kernel<F><<<dim3((unsigned)blocks), 256, 0, s>>>(g, count);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

// g = pf(S) S^-1 for even n > 0: the Parlett-Reid factor, then one [T~ | I] Gauss-Jordan
// per evaluation (the second returns at once for the members without a lifted pivot);
// with a gate, only the members whose gate value is 0.
template <class F>
int pf_adjugate(const F* a, int64_t batch, int n, int skew, F* g, void* ws, size_t wsb, hipStream_t s,
                const F* gate = nullptr) {
  const size_t need = pf_adjugate_ws<F>(batch, n);
  if (need && (!ws || wsb < need)) return FX_ERR_WORKSPACE;
  const PfaLayout PL = pfa_layout<F>(n);
  char* base = (char*)ws;
  const size_t mats = align_up(std::max(cx_matrix_ws<F>(batch, n, n), cx_matrix_ws<F>(batch, n, 2 * n)));
  F* W = (F*)base;
  unsigned char* meta = (unsigned char*)(base + mats);
  const dim3 grid((unsigned)batch);
  {
    const bool lds = cx_in_lds<F>(n, n);
    const size_t shm = cx_lds_bytes((size_t)n * n * sizeof(F), n, lds, true);
    cpfa_factor_kernel<F><<<grid, CX_NT, shm, s>>>(a, n, skew, W, lds, meta, PL, gate);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  }
  const bool lds = cx_in_lds<F>(n, 2 * n);
  const size_t shm = cx_lds_bytes((size_t)n * 2 * n * sizeof(F), n, lds, true);
  for (int ev = 0; ev < 2; ++ev) {
    cgj_kernel<F, GJ_PFA><<<grid, CX_NT, shm, s>>>(a, n, skew, W, lds, nullptr, nullptr, g, 0, gate, meta, PL, ev);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  }
  return FX_OK;
}

// The blocked parts run of a field (complex above CX_BLK_MIN, float32 above its own
// blocked kernels): the blocked Parlett-Reid for sign / logabs and the pair pivots'
// spread, then g: S^-1 from the blocked LU solves of the same S (zero where pf = 0), or the
// Pfaffian adjugate pf(S) S^-1 -- from the same solves scaled by the Parlett-Reid pf for
// the members the gate passes, from the pivot-replaced Parlett-Reid formula for the others
// (pf = 0, or pair pivots spanning more than pf_lu_spread_max). Workspace: the
// Parlett-Reid run's, then max(LU solves + their sign / logabs, the formula's), then the
// spread and the gate.
template <class F>
size_t blk_pf_parts_body(int64_t batch, int n) {
  using R = typename Fd<F>::R;
  return std::max(align_up(blk_lu_inverse_workspace<F>(batch, n)) + align_up((size_t)batch * (sizeof(F) + sizeof(R))),
                  pf_adjugate_ws<F>(batch, n));
}
template <class F>
size_t blk_pf_parts_ws(int64_t batch, int n) {
  if (batch <= 0 || n <= 0 || n > max_n<F>()) return 0;
  return align_up(blk_pr_workspace<F>(batch, n)) + blk_pf_parts_body<F>(batch, n) +
         align_up((size_t)batch * sizeof(double)) + align_up((size_t)batch * sizeof(F));
}
template <class F>
int blk_pf_parts(const F* A, int64_t batch, int n, int skew, int adjugate, F* sign, typename Fd<F>::R* logabs, F* g,
                 void* ws, size_t wsb, hipStream_t s) {
  using R = typename Fd<F>::R;
  if (!ws || wsb < blk_pf_parts_ws<F>(batch, n)) return FX_ERR_WORKSPACE;
  const size_t pr = align_up(blk_pr_workspace<F>(batch, n));
  const size_t body = blk_pf_parts_body<F>(batch, n);
  const size_t lw = align_up(blk_lu_inverse_workspace<F>(batch, n));
  char* base = (char*)ws;
  double* spread = (double*)(base + pr + body);
  F* gz = (F*)(base + pr + body + align_up((size_t)batch * sizeof(double)));
  int st = blk_pr<F>(A, n, skew, batch, sign, logabs, base, pr, s, spread);
  if (st != FX_OK) return st;
  if (adjugate && (n & 1)) return cx_zero<F>(g, batch * (int64_t)n * n, s);
  F* gsign = (F*)(base + pr + lw);
  R* glog = (R*)(gsign + batch);
  const F* gate = sign;
  if (adjugate) {
    st = pf_gate<F>(sign, spread, gz, batch, s);
    if (st != FX_OK) return st;
    gate = gz;
  }
  st = blk_lu_inverse<F>(A, n, skew, batch, gsign, glog, gate, adjugate ? sign : nullptr, adjugate ? logabs : nullptr,
                         g, 0, base + pr, lw, s);
  if (st != FX_OK || !adjugate) return st;
  return pf_adjugate<F>(A, batch, n, skew, g, base + pr, body, s, gate);
}

template <class T>
size_t slogpf_parts_ws(int64_t batch, int n) {
  if (n > CX_MAXN || batch <= 0) return 0;
  if (blocked<cx<T>>(n)) return blk_pf_parts_ws<cx<T>>(batch, n);
  const size_t inv = align_up(cx_matrix_ws<cx<T>>(batch, n, 2 * n)) + align_up((size_t)batch * 3 * sizeof(T));
  return align_up(slogpf_ws<T>(batch, n)) + std::max(inv, pf_adjugate_ws<cx<T>>(batch, n));
}

template <class T>
int slogpf(const T* a, int64_t batch, int n, int skew, T* sign, T* logabs, void* ws, size_t wsb, hipStream_t s) {
  const int st = check_cx_args<cx<T>>(a, batch, n, sign, logabs, nullptr, ws);
  if (st != FX_OK || batch == 0) return st;
  if (n == 0) return cx_empty<cx<T>>(sign, logabs, batch, s);
  return launch_pf<T>(a, n, skew != 0, batch, sign, logabs, ws, wsb, s);
}

// The Parlett-Reid run for sign / logabs, then g: S^-1 by Gauss-Jordan on the same S
// (zeroed where the Parlett-Reid run found pf = 0; every member for odd n), or the
// Pfaffian adjugate pf(S) S^-1 (zero for odd n).
template <class T>
int slogpf_parts(const T* a, int64_t batch, int n, int skew, int adjugate, T* sign, T* logabs, T* g, void* ws,
                 size_t wsb, hipStream_t s) {
  int st = check_cx_args<cx<T>>(a, batch, n, sign, logabs, g, ws);
  if (st != FX_OK || batch == 0) return st;
  if (!g) return slogpf<T>(a, batch, n, skew, sign, logabs, ws, wsb, s);
  if (n == 0) return cx_empty<cx<T>>(sign, logabs, batch, s);
  if (blocked<cx<T>>(n))
    return blk_pf_parts<cx<T>>((const cx<T>*)a, batch, n, skew != 0, adjugate, (cx<T>*)sign, logabs, (cx<T>*)g, ws,
                               wsb, s);
  if (wsb < slogpf_parts_ws<T>(batch, n) || (!ws && slogpf_parts_ws<T>(batch, n))) return FX_ERR_WORKSPACE;
  const size_t pr = align_up(slogpf_ws<T>(batch, n));
  char* base = (char*)ws;
  st = launch_pf<T>(a, n, skew != 0, batch, sign, logabs, base, pr, s);
  if (st != FX_OK) return st;
  if (adjugate && (n & 1)) return cx_zero<cx<T>>((cx<T>*)g, batch * (int64_t)n * n, s);
  if (adjugate)
    return pf_adjugate<cx<T>>((const cx<T>*)a, batch, n, skew != 0, (cx<T>*)g, base + pr, wsb - pr, s);
  const size_t gj = align_up(cx_matrix_ws<cx<T>>(batch, n, 2 * n));
  T* gsign = (T*)(base + pr + gj);
  T* glog = gsign + 2 * batch;
  return launch_cgj<cx<T>>(a, n, skew != 0, batch, gsign, glog, g, GJ_INV, 0, sign, base + pr, gj, s);
}

}  // namespace

// the float64 Pfaffian adjugate (fx_slogpf_parts_f64 with adjugate != 0): zero for odd n.
// Above the register kernels (n > f64_reg_max_n) the members the gate passes (pf != 0 and
// the pair pivots' spread within pf_lu_spread_max; psign, the Parlett-Reid run's sign,
// plog its log|pf|, spread its pivot spread) take pf(S) S^-1 from the blocked LU solves,
// and the others run the pivot-replaced Parlett-Reid factor and Gauss-Jordan above.
static size_t pf_adjugate_f64_body(int64_t batch, int n) {
  return std::max(pf_adjugate_ws<double>(batch, n),
                  align_up(lu64_inverse_workspace(batch, n)) + align_up((size_t)batch * 2 * sizeof(double)));
}
size_t pf_adjugate_f64_ws(int64_t batch, int n) {
  if (n <= tune().f64_reg_max_n || batch <= 0 || (n & 1)) return pf_adjugate_ws<double>(batch, n);
  return pf_adjugate_f64_body(batch, n) + align_up((size_t)batch * sizeof(double));
}
int pf_adjugate_f64(const double* a, int64_t batch, int n, int skew, double* g, const double* psign,
                    const double* plog, const double* spread, void* ws, size_t wsb, hipStream_t s) {
  if (batch <= 0 || n == 0) return FX_OK;
  if (n & 1) return cx_zero<double>(g, batch * (int64_t)n * n, s);
  if (n <= tune().f64_reg_max_n) return pf_adjugate<double>(a, batch, n, skew, g, ws, wsb, s);
  if (!ws || !spread || wsb < pf_adjugate_f64_ws(batch, n)) return FX_ERR_WORKSPACE;
  const size_t body = pf_adjugate_f64_body(batch, n);
  const size_t lw = align_up(lu64_inverse_workspace(batch, n));
  double* lsign = (double*)((char*)ws + lw);
  double* gate = (double*)((char*)ws + body);
  int r = pf_gate<double>(psign, spread, gate, batch, s);
  if (r == FX_OK)
    r = launch_lu64_inverse(a, n, skew, batch, lsign, lsign + batch, gate, psign, plog, g, 0, ws, lw, s);
  if (r != FX_OK) return r;
  return pf_adjugate<double>(a, batch, n, skew, g, ws, body, s, gate);
}

// complex64's product mode, per thread and per call (FX_PREC_IEEE: fp32 products)
static thread_local int t_cx32_ieee = 0;
int cx32_ieee() { return t_cx32_ieee; }
CxPrecPin::CxPrecPin(int ieee) : old_(t_cx32_ieee) { t_cx32_ieee = ieee; }
CxPrecPin::~CxPrecPin() { t_cx32_ieee = old_; }

// ---- float32 above its own blocked kernels (LU_LARGE_MAXN < n <= GEN32_MAXN): the
// field-generic blocked kernels of lu64_impl.inc on float storage (32-column panels, the
// trailing products on the fp64 MFMA), with the entry points' argument checks done by the
// caller. det's and pf's gradients as for the complex kinds: the LU solves for the regular
// members, the Gauss-Jordan continuation / pivot-replaced Parlett-Reid formula (one
// workgroup per member) for the exactly singular and, for pf, numerically singular ones.
size_t gen32_slogdet_ws(int64_t batch, int n) { return blk_lu_workspace<float>(batch, n); }
int gen32_slogdet(const float* a, int64_t batch, int n, float* sign, float* logabs, void* ws, size_t wsb,
                  hipStream_t s) {
  return blk_lu<float>(a, n, batch, sign, logabs, ws, wsb, s);
}
size_t gen32_slogdet_parts_ws(int64_t batch, int n) { return blk_lu_inverse_workspace<float>(batch, n); }
int gen32_slogdet_parts(const float* a, int64_t batch, int n, float* sign, float* logabs, float* inv_t, void* ws,
                        size_t wsb, hipStream_t s) {
  return slogdet_parts<float>(a, batch, n, sign, logabs, inv_t, ws, wsb, s);
}
size_t gen32_det_parts_ws(int64_t batch, int n) { return det_parts_ws<float>(batch, n); }
int gen32_det_parts(const float* a, int64_t batch, int n, float* sign, float* logabs, float* adj_t, void* ws,
                    size_t wsb, hipStream_t s) {
  return det_parts<float>(a, batch, n, sign, logabs, adj_t, ws, wsb, s);
}
size_t gen32_slogpf_ws(int64_t batch, int n) { return blk_pr_workspace<float>(batch, n); }
int gen32_slogpf(const float* a, int64_t batch, int n, int skew, float* sign, float* logabs, void* ws, size_t wsb,
                 hipStream_t s) {
  return blk_pr<float>(a, n, skew, batch, sign, logabs, ws, wsb, s);
}
size_t gen32_slogpf_parts_ws(int64_t batch, int n) { return blk_pf_parts_ws<float>(batch, n); }
int gen32_slogpf_parts(const float* a, int64_t batch, int n, int skew, int adjugate, float* sign, float* logabs,
                       float* g, void* ws, size_t wsb, hipStream_t s) {
  return blk_pf_parts<float>(a, batch, n, skew, adjugate, sign, logabs, g, ws, wsb, s);
}

}  // namespace fx

using namespace fx;

extern "C" {

size_t fx_slogdet_c64_workspace(int64_t batch, int32_t n) { fx::TunePin pin_; return slogdet_ws<cx<float>>(batch, n); }
size_t fx_slogdet_c128_workspace(int64_t batch, int32_t n) { fx::TunePin pin_; return slogdet_ws<cx<double>>(batch, n); }

// complex64's prec: FX_PREC_BF16X3 (the fp32-accuracy mode) the products on the fp64
// MFMA, FX_PREC_IEEE four fp32 MFMA products per complex one
static bool bad_cx_prec(int32_t prec) { return prec != FX_PREC_IEEE && prec != FX_PREC_BF16X3; }

int fx_slogdet_c64(const float* a, int64_t batch, int32_t n, float* sign, float* logabs, int32_t prec,
                   void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  if (bad_cx_prec(prec)) return FX_ERR_INVALID_ARGUMENT;
  fx::CxPrecPin pp_(prec == FX_PREC_IEEE);
  return slogdet<cx<float>>(a, batch, n, sign, logabs, workspace, workspace_bytes, (hipStream_t)stream);
}
int fx_slogdet_c128(const double* a, int64_t batch, int32_t n, double* sign, double* logabs, void* workspace,
                    size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  return slogdet<cx<double>>(a, batch, n, sign, logabs, workspace, workspace_bytes, (hipStream_t)stream);
}

size_t fx_slogdet_parts_c64_workspace(int64_t batch, int32_t n) { fx::TunePin pin_; return slogdet_parts_ws<cx<float>>(batch, n); }
size_t fx_slogdet_parts_c128_workspace(int64_t batch, int32_t n) { fx::TunePin pin_; return slogdet_parts_ws<cx<double>>(batch, n); }

int fx_slogdet_parts_c64(const float* a, int64_t batch, int32_t n, float* sign, float* logabs, float* inv_t,
                         int32_t prec, void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  if (bad_cx_prec(prec)) return FX_ERR_INVALID_ARGUMENT;
  fx::CxPrecPin pp_(prec == FX_PREC_IEEE);
  return slogdet_parts<cx<float>>(a, batch, n, sign, logabs, inv_t, workspace, workspace_bytes, (hipStream_t)stream);
}
int fx_slogdet_parts_c128(const double* a, int64_t batch, int32_t n, double* sign, double* logabs, double* inv_t,
                          void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  return slogdet_parts<cx<double>>(a, batch, n, sign, logabs, inv_t, workspace, workspace_bytes, (hipStream_t)stream);
}

size_t fx_slogpf_c64_workspace(int64_t batch, int32_t n) { fx::TunePin pin_; return slogpf_ws<float>(batch, n); }
size_t fx_slogpf_c128_workspace(int64_t batch, int32_t n) { fx::TunePin pin_; return slogpf_ws<double>(batch, n); }

int fx_slogpf_c64(const float* a, int64_t batch, int32_t n, int32_t skew_symmetrize, float* sign, float* logabs,
                  int32_t prec, void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  if (bad_cx_prec(prec)) return FX_ERR_INVALID_ARGUMENT;
  fx::CxPrecPin pp_(prec == FX_PREC_IEEE);
  return slogpf<float>(a, batch, n, skew_symmetrize, sign, logabs, workspace, workspace_bytes, (hipStream_t)stream);
}
int fx_slogpf_c128(const double* a, int64_t batch, int32_t n, int32_t skew_symmetrize, double* sign,
                   double* logabs, void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  return slogpf<double>(a, batch, n, skew_symmetrize, sign, logabs, workspace, workspace_bytes,
                        (hipStream_t)stream);
}

size_t fx_slogpf_parts_c64_workspace(int64_t batch, int32_t n) { fx::TunePin pin_; return slogpf_parts_ws<float>(batch, n); }
size_t fx_slogpf_parts_c128_workspace(int64_t batch, int32_t n) { fx::TunePin pin_; return slogpf_parts_ws<double>(batch, n); }

int fx_slogpf_parts_c64(const float* a, int64_t batch, int32_t n, int32_t skew_symmetrize, int32_t adjugate,
                        float* sign, float* logabs, float* g, int32_t prec, void* workspace, size_t workspace_bytes,
                        fx_stream_t stream) {
  fx::TunePin pin_;
  if (bad_cx_prec(prec)) return FX_ERR_INVALID_ARGUMENT;
  fx::CxPrecPin pp_(prec == FX_PREC_IEEE);
  return slogpf_parts<float>(a, batch, n, skew_symmetrize, adjugate, sign, logabs, g, workspace, workspace_bytes,
                             (hipStream_t)stream);
}
int fx_slogpf_parts_c128(const double* a, int64_t batch, int32_t n, int32_t skew_symmetrize, int32_t adjugate,
                         double* sign, double* logabs, double* g, void* workspace, size_t workspace_bytes,
                         fx_stream_t stream) {
  fx::TunePin pin_;
  return slogpf_parts<double>(a, batch, n, skew_symmetrize, adjugate, sign, logabs, g, workspace,
                              workspace_bytes, (hipStream_t)stream);
}

size_t fx_det_parts_c64_workspace(int64_t batch, int32_t n) { fx::TunePin pin_; return det_parts_ws<cx<float>>(batch, n); }
size_t fx_det_parts_c128_workspace(int64_t batch, int32_t n) { fx::TunePin pin_; return det_parts_ws<cx<double>>(batch, n); }
size_t fx_det_parts_f64_workspace(int64_t batch, int32_t n) { fx::TunePin pin_; return det_parts_f64_ws(batch, n); }

int fx_det_parts_c64(const float* a, int64_t batch, int32_t n, float* sign, float* logabs, float* adj_t,
                     int32_t prec, void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  if (bad_cx_prec(prec)) return FX_ERR_INVALID_ARGUMENT;
  fx::CxPrecPin pp_(prec == FX_PREC_IEEE);
  return det_parts<cx<float>>(a, batch, n, sign, logabs, adj_t, workspace, workspace_bytes, (hipStream_t)stream);
}
int fx_det_parts_c128(const double* a, int64_t batch, int32_t n, double* sign, double* logabs, double* adj_t,
                      void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  return det_parts<cx<double>>(a, batch, n, sign, logabs, adj_t, workspace, workspace_bytes, (hipStream_t)stream);
}
int fx_det_parts_f64(const double* a, int64_t batch, int32_t n, double* sign, double* logabs, double* adj_t,
                     void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  return det_parts_f64(a, batch, n, sign, logabs, adj_t, workspace, workspace_bytes, (hipStream_t)stream);
}

}  // extern "C"
