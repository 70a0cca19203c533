// Field types of the float64 and complex kernels: cx<T> is one complex value as its (re,
// im) pair -- the memory of torch's complex64 / complex128 elements -- and Fd<F> the
// operations the generic kernels use on F = double, cx<float> or cx<double>, after the
// reference's value fields (src/fermix/_field.py:32-120: `abs1` as the pivot magnitude,
// the guarded reciprocal `recip`, the phase `unit`, `mag`).
#pragma once

#include "common.h"
#include "fermix_internal.h"

namespace fx {

template <class T>
struct cx {
  T re, im;
};

// ---- field operations: F = cx<float> / cx<double> (complex kinds) or double (the
// float64 adjugate, which shares the Gauss-Jordan kernel below)
template <class F>
struct Fd;
template <class T>
struct Fd<cx<T>> {
  using R = T;  // real component type (logabs)
  static __device__ __forceinline__ cx<T> zero() { return {T(0), T(0)}; }
  static __device__ __forceinline__ cx<T> one() { return {T(1), T(0)}; }
  static __device__ __forceinline__ bool is0(cx<T> x) { return x.re == T(0) && x.im == T(0); }
  // pivot magnitude |re| + |im| (LAPACK's cabs1), exact in double for both kinds
  static __device__ __forceinline__ unsigned long long key(cx<T> x) {
    return key64((double)(fabs(x.re) + fabs(x.im)));
  }
  static __device__ __forceinline__ cx<T> mul(cx<T> a, cx<T> b) {
    return {a.re * b.re - a.im * b.im, a.re * b.im + a.im * b.re};
  }
  // r - l p with fused products
  static __device__ __forceinline__ cx<T> fms(cx<T> r, cx<T> l, cx<T> p) {
    return {fma(-l.re, p.re, fma(l.im, p.im, r.re)), fma(-l.re, p.im, fma(-l.im, p.re, r.im))};
  }
  // 1 / x = conj(x) / |x|^2, 0 -> 0
  static __device__ __forceinline__ cx<T> rcp(cx<T> x) {
    const T s = x.re * x.re + x.im * x.im;
    const T inv = s != T(0) ? T(1) / s : T(0);
    return {x.re * inv, -(x.im * inv)};
  }
  static __device__ __forceinline__ bool finite(cx<T> x) { return isfinite(x.re) && isfinite(x.im); }
  // the pivot's phase and log-modulus, accumulated in double
  static __device__ __forceinline__ void acc(double2& sgn, double& logabs, cx<T> x) {
    const double re = x.re, im = x.im, m = hypot(re, im);
    logabs += log(m);
    const double ur = re / m, ui = im / m;
    sgn = make_double2(sgn.x * ur - sgn.y * ui, sgn.x * ui + sgn.y * ur);
  }
  static __device__ __forceinline__ cx<T> from(double2 v) { return {T(v.x), T(v.y)}; }
  static __device__ __forceinline__ double2 to2(cx<T> x) { return make_double2(x.re, x.im); }
  // the modulus |x| (the Pfaffian adjugate's choice of the smallest pivot), in double
  static __device__ __forceinline__ double mag(cx<T> x) { return hypot((double)x.re, (double)x.im); }
  static __device__ __forceinline__ cx<T> add(cx<T> a, cx<T> b) { return {a.re + b.re, a.im + b.im}; }
  static __device__ __forceinline__ cx<T> sub(cx<T> a, cx<T> b) { return {a.re - b.re, a.im - b.im}; }
  static __device__ __forceinline__ cx<T> neg(cx<T> a) { return {-a.re, -a.im}; }
  // a / b as a times the guarded reciprocal
  static __device__ __forceinline__ cx<T> div(cx<T> a, cx<T> b) { return mul(a, rcp(b)); }
  static __device__ __forceinline__ cx<T> scale(cx<T> a, double2 s) {
    return {T(a.re * s.x - a.im * s.y), T(a.re * s.y + a.im * s.x)};
  }
};
template <>
struct Fd<double> {
  using R = double;
  static __device__ __forceinline__ double zero() { return 0.0; }
  static __device__ __forceinline__ double one() { return 1.0; }
  static __device__ __forceinline__ bool is0(double x) { return x == 0.0; }
  static __device__ __forceinline__ unsigned long long key(double x) { return key64(x); }
  static __device__ __forceinline__ double mul(double a, double b) { return a * b; }
  static __device__ __forceinline__ double fms(double r, double l, double p) { return fma(-l, p, r); }
  static __device__ __forceinline__ double rcp(double x) { return x != 0.0 ? 1.0 / x : 0.0; }
  static __device__ __forceinline__ bool finite(double x) { return isfinite(x); }
  // the float64 kernels' order: log|d| added in pivot order, the sign flipped per
  // negative pivot
  static __device__ __forceinline__ void acc(double2& sgn, double& logabs, double x) {
    logabs += log(fabs(x));
    if (x < 0.0) sgn.x = -sgn.x;
  }
  static __device__ __forceinline__ double from(double2 v) { return v.x; }
  static __device__ __forceinline__ double2 to2(double x) { return make_double2(x, 0.0); }
  static __device__ __forceinline__ double mag(double x) { return fabs(x); }
  static __device__ __forceinline__ double add(double a, double b) { return a + b; }
  static __device__ __forceinline__ double sub(double a, double b) { return a - b; }
  static __device__ __forceinline__ double neg(double a) { return -a; }
  static __device__ __forceinline__ double div(double a, double b) { return a / b; }
  static __device__ __forceinline__ double scale(double a, double2 s) { return a * s.x; }
};

// float32 above the orders of the float32 blocked kernels: the generic blocked path of the
// 64-bit kinds on float storage (the products of its GEMMs in fp64), with the float64
// conventions (sign flipped per negative pivot, log|d| summed in double in pivot order)
template <>
struct Fd<float> {
  using R = float;
  static __device__ __forceinline__ float zero() { return 0.0f; }
  static __device__ __forceinline__ float one() { return 1.0f; }
  static __device__ __forceinline__ bool is0(float x) { return x == 0.0f; }
  static __device__ __forceinline__ unsigned long long key(float x) { return key64((double)x); }
  static __device__ __forceinline__ float mul(float a, float b) { return a * b; }
  static __device__ __forceinline__ float fms(float r, float l, float p) { return fmaf(-l, p, r); }
  static __device__ __forceinline__ float rcp(float x) { return x != 0.0f ? 1.0f / x : 0.0f; }
  static __device__ __forceinline__ bool finite(float x) { return isfinite(x); }
  static __device__ __forceinline__ void acc(double2& sgn, double& logabs, float x) {
    logabs += log(fabs((double)x));
    if (x < 0.0f) sgn.x = -sgn.x;
  }
  static __device__ __forceinline__ float from(double2 v) { return (float)v.x; }
  static __device__ __forceinline__ double2 to2(float x) { return make_double2(x, 0.0); }
  static __device__ __forceinline__ double mag(float x) { return fabs((double)x); }
  static __device__ __forceinline__ float add(float a, float b) { return a + b; }
  static __device__ __forceinline__ float sub(float a, float b) { return a - b; }
  static __device__ __forceinline__ float neg(float a) { return -a; }
  static __device__ __forceinline__ float div(float a, float b) { return a / b; }
  static __device__ __forceinline__ float scale(float a, double2 s) { return (float)(a * s.x); }
};

// largest order of the blocked kernels of lu64_impl.inc per field: float32 runs them only
// above its own blocked kernels' 8192
constexpr int BLK_MAXN = 8192;
template <class F>
constexpr int blk_max_n() {
  return sizeof(F) == 4 ? GEN32_MAXN : BLK_MAXN;
}

__device__ __forceinline__ double2 c2mul(double2 a, double2 b) {
  return make_double2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}

// (v - u) / 2 per component (the skew part of a pair of mirrored entries)
template <class T>
__device__ __forceinline__ cx<T> half_diff(cx<T> v, cx<T> u) {
  return {(v.re - u.re) * T(0.5), (v.im - u.im) * T(0.5)};
}
__device__ __forceinline__ double half_diff(double v, double u) { return (v - u) * 0.5; }
__device__ __forceinline__ float half_diff(float v, float u) { return (v - u) * 0.5f; }

// The blocked LU, its solves and the blocked Parlett-Reid for F = double, cx<float>,
// cx<double> (lu64_impl.inc): sign / logabs, and out = A^-T / A^-1 (times ssign exp(slog) when
// ssign is given, zero where gate -- default: the factorisation's own sign -- is 0 or the
// result is not finite); 0 < n <= blk_max_n<F>(), every buffer of the batch.
template <class F>
size_t blk_lu_workspace(int64_t batch, int n);
template <class F>
int blk_lu(const F* A, int n, int64_t batch, F* sign, typename Fd<F>::R* logabs, void* ws, size_t ws_bytes,
           hipStream_t s);
template <class F>
size_t blk_lu_inverse_workspace(int64_t batch, int n);
template <class F>
int blk_lu_inverse(const F* A, int n, int skew, int64_t batch, F* sign, typename Fd<F>::R* logabs, const F* gate,
                   const F* ssign, const typename Fd<F>::R* slog, F* out, int out_t, void* ws, size_t ws_bytes,
                   hipStream_t s);
template <class F>
size_t blk_pr_workspace(int64_t batch, int n);
template <class F>
int blk_pr(const F* A, int n, int skew, int64_t batch, F* sign, typename Fd<F>::R* logabs, void* ws, size_t ws_bytes,
           hipStream_t s, double* spread = nullptr);

}  // namespace fx
