// slogdet for n <= 32 and slogpf for n <= 16 with several matrices per wave: a group of G
// lanes (G = 16 for n <= 16, 32 above) holds one matrix, lane r of the group its row r in
// registers.
// Nothing is shared between groups except the wave's instructions, so a 256-thread
// workgroup factors 256 / G matrices at once with no workgroup barrier.
//
// LU (partial pivoting, rows in place): per column j the group's largest |a[j]| among
// the unassigned rows (ties: lowest row) is found with a DPP max over order-preserving
// keys, the pivot row is broadcast through LDS, and every other unassigned row
// subtracts its multiple. Parlett-Reid (pair steps c = 0, 2, ..): column a of the
// current matrix is minus row a (skew), broadcast through LDS; the pivot is the
// largest |M[i][a]| over the unassigned rows, swapped into position c + 1; the rank-2
// update M += tau w^T - w tau^T uses the group's tau / w vectors, exchanged through LDS.
// The permutation stays virtual (a position per row); its parity is the swap count.
//
// With FACT the kernels also write the factors in the formats of the n <= 128 kernels
// (packed LU of P A' in the final row order + the row map; Parlett-Reid tau / w by
// original row, the pair pivots and the final position -> original row map), padded to
// N = G, so the gradient path and the forward run the same arithmetic.
//
// Reference roles replaced (ChenAo-Phys/fermix): for n <= 32 the reference dispatches to
// its generic path (src/fermix/api.py:57-73, _common.py:105-126: jnp LU / masked
// Parlett-Reid, _fallback.py:36-60,266-300); the pivoting, sign and zero-pivot
// conventions followed here are those.
#include "common.h"
#include "fermix_internal.h"

namespace fx {


template <int G>
__device__ __forceinline__ float group_sum_f32(float v) {
  v += dpp_f32<0xB1>(v);
  v += dpp_f32<0x4E>(v);
  v += dpp_f32<0x141>(v);
  v += dpp_f32<0x140>(v);
  if constexpr (G == 32) v += __shfl_xor(v, 16);
  return v;
}


// Row r of matrix Ab (n x n, row-major) into a[0..G): columns >= n and rows >= n are 0
// (the callers write the padding). Every load is unconditional at a clamped, in-bounds
// address (Ab is a valid matrix even for a dead group), the padding applied after.
template <int G>
__device__ __forceinline__ void load_row(float (&a)[G], const float* __restrict__ Ab, int n, int r, bool live,
                                         int vec) {
  const bool rowok = live && r < n;
  const int rr = min(r, n - 1);
  if (vec) {  // n == G and 16-byte aligned rows
    const float4* rp = reinterpret_cast<const float4*>(Ab + rr * G);
#pragma unroll
    for (int q = 0; q < G / 4; ++q) {
      const float4 v = rp[q];
      a[4 * q] = rowok ? v.x : 0.0f;
      a[4 * q + 1] = rowok ? v.y : 0.0f;
      a[4 * q + 2] = rowok ? v.z : 0.0f;
      a[4 * q + 3] = rowok ? v.w : 0.0f;
    }
  } else {
    const float* rp = Ab + rr * n;
#pragma unroll
    for (int k = 0; k < G; ++k) a[k] = rp[min(k, n - 1)];
#pragma unroll
    for (int k = 0; k < G; ++k) a[k] = (rowok && k < n) ? a[k] : 0.0f;
  }
}

template <int G, bool FACT>
__global__ __launch_bounds__(256) void lu_tiny_kernel(const float* __restrict__ A, int n, int vec, int64_t batch,
                                                      float* __restrict__ sign_out, float* __restrict__ logabs_out,
                                                      float* __restrict__ lu_out, int* __restrict__ perm_out) {
  constexpr int MPW = 256 / G;  // matrices per workgroup
  __shared__ __align__(16) float ubuf[256];
  const int tid = threadIdx.x, lane = tid & 63;
  const int r = tid % G;                 // row within the matrix
  const int gbase = lane - r;            // first lane of the group
  float* const ub = ubuf + (tid - r);    // the group's pivot-row buffer (G floats)
  const int64_t mi = (int64_t)blockIdx.x * MPW + tid / G;
  const bool live = mi < batch;
  const float* Ab = A + (live ? mi : 0) * (int64_t)n * n;
  float a[G];
  load_row<G>(a, Ab, n, r, live, vec);
#pragma unroll
  for (int k = 0; k < G; ++k)
    if (r >= n && k == r) a[k] = 1.0f;
  int pos = r;
  int nsw = 0;
  float mypiv = 1.0f;  // the pivot of position r
  static_for<0, G>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    if (j < n) {
      const bool cand = r < n && pos >= j;
      const unsigned key = cand_key(a[j], cand);
      const unsigned gk = group_max_u32<G>(key);
      const int prow = group_first<G>(cand && key == gk, gbase);
      const int pl = gbase + prow;
      const float piv = __shfl(a[j], pl);
      const int pp = __shfl(pos, pl);
      // the pivot row's U entries j+1 .. G-1 to the group
      if (r == prow) {
#pragma unroll
        for (int k = j + 1; k < G; ++k) ub[k] = a[k];
      }
      wave_lds_fence();
      if (pos == j) pos = pp;
      if (r == prow) pos = j;
      nsw += (pp != j) ? 1 : 0;
      if (r == j) mypiv = piv;
      const float rcp = safe_rcp(piv);
      if (r < n && pos > j) {
        const float l = a[j] * rcp;
        a[j] = l;
#pragma unroll
        for (int k = j + 1; k < G; ++k) a[k] = fmaf(-l, ub[k], a[k]);
      }
      wave_lds_fence();  // every read of ub precedes the next step's writes
    }
  });
  // (sign, logabs): sum of log|pivot| over the group, zero and negative pivots
  const bool real = r < n;
  const bool z = real && mypiv == 0.0f;
  const float lg = group_sum_f32<G>((real && mypiv != 0.0f) ? logf(fabsf(mypiv)) : 0.0f);
  const int anyz = group_first<G>(z, gbase) < G;
  const unsigned long long nm = __ballot(real && mypiv < 0.0f);
  const int negs = __popc((unsigned)(nm >> gbase) & (G == 32 ? 0xFFFFFFFFu : 0xFFFFu)) + nsw;
  if (live && r == 0) {
    sign_out[mi] = anyz ? 0.0f : ((negs & 1) ? -1.0f : 1.0f);
    logabs_out[mi] = anyz ? -INFINITY : lg;
  }
  if (FACT && live) {
    float4* lr = reinterpret_cast<float4*>(lu_out + (mi * G + pos) * (int64_t)G);
#pragma unroll
    for (int q = 0; q < G / 4; ++q) lr[q] = make_float4(a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]);
    perm_out[mi * G + pos] = r;
  }
}

// Gauss-Jordan on [A | I] with the pivots of lu_tiny_kernel: sign / logabs bit-identical
// to it (the unassigned rows take exactly its update) plus A^-T. Every other row i takes
// row_i -= m_i row_p with m_i = a_i[j] / d~ (d~ = the pivot, 1 for an exact zero, as in
// U~): for the unassigned rows this is the LU step, for the assigned ones the upward
// elimination, and the augmented half collects E with E A~ = diag(d~) Pi, so row pos_i of
// A~^-1 is (row i of E) / d~_{pos_i}. zero_singular zeroes members with a zero pivot;
// members with a non-finite result are zeroed always (the slogdet gradient convention).
template <int G>
__global__ __launch_bounds__(256) void lu_tiny_inv_kernel(const float* __restrict__ A, int n, int vec, int64_t batch,
                                                          int zero_singular, float* __restrict__ sign_out,
                                                          float* __restrict__ logabs_out, float* __restrict__ invT) {
  constexpr int MPW = 256 / G;
  __shared__ __align__(16) float ubuf[256];
  __shared__ __align__(16) float ebuf[256];
  const int tid = threadIdx.x, lane = tid & 63;
  const int r = tid % G;
  const int gbase = lane - r;
  float* const ub = ubuf + (tid - r);
  float* const eb = ebuf + (tid - r);
  const int64_t mi = (int64_t)blockIdx.x * MPW + tid / G;
  const bool live = mi < batch;
  const float* Ab = A + (live ? mi : 0) * (int64_t)n * n;
  float a[G], e[G];
  load_row<G>(a, Ab, n, r, live, vec);
#pragma unroll
  for (int k = 0; k < G; ++k) {
    if (r >= n && k == r) a[k] = 1.0f;
    e[k] = (k == r) ? 1.0f : 0.0f;
  }
  int pos = r;
  int nsw = 0;
  float mypiv = 1.0f;
  static_for<0, G>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    if (j < n) {
      const bool cand = r < n && pos >= j;
      const unsigned key = cand_key(a[j], cand);
      const unsigned gk = group_max_u32<G>(key);
      const int prow = group_first<G>(cand && key == gk, gbase);
      const int pl = gbase + prow;
      const float piv = __shfl(a[j], pl);
      const int pp = __shfl(pos, pl);
      if (r == prow) {
#pragma unroll
        for (int k = j + 1; k < G; ++k) ub[k] = a[k];
#pragma unroll
        for (int k = 0; k < G; k += 4) *reinterpret_cast<float4*>(eb + k) = make_float4(e[k], e[k + 1], e[k + 2], e[k + 3]);
      }
      wave_lds_fence();
      const bool was_assigned = pos < j;
      if (pos == j) pos = pp;
      if (r == prow) pos = j;
      nsw += (pp != j) ? 1 : 0;
      if (r == j) mypiv = piv;
      // d~: 1 for an exact zero pivot; a zero pivot column is zero on every unassigned
      // row, so their multipliers stay 0 as in the LU
      const float rcp = piv != 0.0f ? __builtin_amdgcn_rcpf(piv) : 1.0f;
      if (r < n && r != prow && (pos > j || was_assigned)) {
        const float l = a[j] * rcp;
        a[j] = l;
#pragma unroll
        for (int k = j + 1; k < G; ++k) a[k] = fmaf(-l, ub[k], a[k]);
#pragma unroll
        for (int k = 0; k < G; k += 4) {
          const float4 ev = *reinterpret_cast<const float4*>(eb + k);
          e[k] = fmaf(-l, ev.x, e[k]);
          e[k + 1] = fmaf(-l, ev.y, e[k + 1]);
          e[k + 2] = fmaf(-l, ev.z, e[k + 2]);
          e[k + 3] = fmaf(-l, ev.w, e[k + 3]);
        }
      }
      wave_lds_fence();
    }
  });
  const bool real = r < n;
  const bool z = real && mypiv == 0.0f;
  const float lg = group_sum_f32<G>((real && mypiv != 0.0f) ? logf(fabsf(mypiv)) : 0.0f);
  const int anyz = group_first<G>(z, gbase) < G;
  const unsigned long long nm = __ballot(real && mypiv < 0.0f);
  const int negs = __popc((unsigned)(nm >> gbase) & (G == 32 ? 0xFFFFFFFFu : 0xFFFFu)) + nsw;
  if (live && r == 0) {
    sign_out[mi] = anyz ? 0.0f : ((negs & 1) ? -1.0f : 1.0f);
    logabs_out[mi] = anyz ? -INFINITY : lg;
  }
  // row pos of A~^-1 = e / d~_pos, written as column pos of A^-T; d~_pos comes from the
  // lane that holds pivot pos
  const float dpos = __shfl(mypiv, gbase + pos);
  const float s = dpos != 0.0f ? 1.0f / dpos : 1.0f;
  bool nf = false;
#pragma unroll
  for (int k = 0; k < G; ++k) {
    e[k] *= s;
    nf = nf || (real && k < n && !isfinite(e[k]));
  }
  const bool bad = (group_first<G>(nf, gbase) < G) || (zero_singular && anyz);
  if (live && real) {
    float* ob = invT + mi * (int64_t)n * n + pos;
#pragma unroll
    for (int k = 0; k < G; ++k)
      if (k < n) ob[(int64_t)k * n] = bad ? 0.0f : e[k];
  }
}

// Skew row r of S (n x n): S = (A - A^T) / 2 if skew, else A; rows >= n (n even) are the
// [[0, 1], [-1, 0]] padding.
template <int G>
__device__ __forceinline__ void load_skew_row(float (&a)[G], const float* __restrict__ Ab, int n, int r, bool live,
                                              int skew, int vec) {
  load_row<G>(a, Ab, n, r, live, vec);
  if (skew) {
    const bool rowok = live && r < n;
    const int rr = min(r, n - 1);
    float t[G];
#pragma unroll
    for (int k = 0; k < G; ++k) t[k] = Ab[min(k, n - 1) * n + rr];
#pragma unroll
    for (int k = 0; k < G; ++k) a[k] = a[k] * 0.5f - ((rowok && k < n) ? t[k] : 0.0f) * 0.5f;
  }
  if (r >= n) {
#pragma unroll
    for (int k = 0; k < G; ++k) a[k] = (k == (r ^ 1)) ? ((r & 1) ? -1.0f : 1.0f) : 0.0f;
  }
}

template <int G, bool FACT>
__global__ __launch_bounds__(256) void pf_tiny_kernel(const float* __restrict__ A, int n, int skew, int vec,
                                                      int64_t batch,
                                                      float* __restrict__ sign_out, float* __restrict__ logabs_out,
                                                      float* __restrict__ gbuf_out, float* __restrict__ d_out,
                                                      int* __restrict__ perm_out) {
  constexpr int MPW = 256 / G;
  __shared__ __align__(16) float rbuf[4][256];  // row a, row p, tau, w of each group
  const int tid = threadIdx.x, lane = tid & 63;
  const int r = tid % G;
  const int gbase = lane - r;
  float* const ra = rbuf[0] + (tid - r);
  float* const rp = rbuf[1] + (tid - r);
  float* const tb = rbuf[2] + (tid - r);
  float* const wb = rbuf[3] + (tid - r);
  const int64_t mi = (int64_t)blockIdx.x * MPW + tid / G;
  const bool live = mi < batch;
  const float* Ab = A + (live ? mi : 0) * (int64_t)n * n;
  float a[G];
  load_skew_row<G>(a, Ab, n, r, live, skew, vec);
  int pos = r;
  int nsw = 0;
  float myd = 1.0f;  // the pivot of pair r (lanes r < G / 2)
  static_for<0, G / 2>([&](auto tc) {
    constexpr int t = decltype(tc)::value;
    constexpr int c = 2 * t;
    float tau = 0.0f, w = 0.0f;
    if (c < n) {
      // row a (position c) to the group: x_i = M[i][a] = -M[a][i]
      if (pos == c) {
#pragma unroll
        for (int k = 0; k < G; k += 4) *reinterpret_cast<float4*>(ra + k) = make_float4(a[k], a[k + 1], a[k + 2], a[k + 3]);
      }
      wave_lds_fence();
      const float x = -ra[r];
      const bool cand = r < n && pos > c;
      const unsigned key = cand_key(x, cand);
      const unsigned gk = group_max_u32<G>(key);
      const int prow = group_first<G>(cand && key == gk, gbase);
      const int pl = gbase + prow;
      const int pp = __shfl(pos, pl);
      const float d = ra[prow];  // M[a][p]
      if (r == prow) {
#pragma unroll
        for (int k = 0; k < G; k += 4) *reinterpret_cast<float4*>(rp + k) = make_float4(a[k], a[k + 1], a[k + 2], a[k + 3]);
      }
      wave_lds_fence();
      const float y = -rp[r];  // M[i][p]
      if (pos == c + 1) pos = pp;
      if (r == prow) pos = c + 1;
      nsw += (pp != c + 1) ? 1 : 0;
      if (r == t) myd = d;
      const float inv = safe_rcp(d);
      const bool act = pos > c + 1;  // rows still to be eliminated (padding rows included)
      tau = act ? -x * inv : 0.0f;
      w = act ? y : 0.0f;
      tb[r] = tau;
      wb[r] = w;
      wave_lds_fence();
      if (act) {
#pragma unroll
        for (int k = 0; k < G; k += 4) {
          const float4 tk = *reinterpret_cast<const float4*>(tb + k);
          const float4 wk = *reinterpret_cast<const float4*>(wb + k);
          a[k] = fmaf(tau, wk.x, fmaf(-w, tk.x, a[k]));
          a[k + 1] = fmaf(tau, wk.y, fmaf(-w, tk.y, a[k + 1]));
          a[k + 2] = fmaf(tau, wk.z, fmaf(-w, tk.z, a[k + 2]));
          a[k + 3] = fmaf(tau, wk.w, fmaf(-w, tk.w, a[k + 3]));
        }
      }
      wave_lds_fence();  // every read of the buffers precedes the next step's writes
    } else if (r == t) {
      myd = 1.0f;  // padding pair: [[0, 1], [-1, 0]] in place
    }
    if (FACT && live) {
      // block t / 8 of gbuf (B, G / 16, G, 16): tau in column 2 (t % 8), w in column 2 (t % 8) + 1
      float* gr = gbuf_out + ((mi * (G / 16) + t / 8) * G + r) * (int64_t)16 + 2 * (t % 8);
      *reinterpret_cast<float2*>(gr) = make_float2(tau, w);
    }
  });
  const bool real = r < n / 2;  // real pairs
  const bool z = real && myd == 0.0f;
  const float lg = group_sum_f32<G>((real && myd != 0.0f) ? logf(fabsf(myd)) : 0.0f);
  const int anyz = group_first<G>(z, gbase) < G;
  const unsigned long long nm = __ballot(real && myd < 0.0f);
  const int negs = __popc((unsigned)(nm >> gbase) & (G == 32 ? 0xFFFFFFFFu : 0xFFFFu)) + nsw;
  if (live && r == 0) {
    sign_out[mi] = anyz ? 0.0f : ((negs & 1) ? -1.0f : 1.0f);
    logabs_out[mi] = anyz ? -INFINITY : lg;
  }
  if (FACT && live) {
    if (r < G / 2) d_out[mi * (G / 2) + r] = myd;
    perm_out[mi * G + pos] = r;
  }
}

int tiny_padded(int n) { return n <= 16 ? 16 : 32; }

// 16-byte row loads need n == G and an aligned base (n * n * 4 is then a multiple of 16).
static int tiny_vec(const float* A, int n) { return n == tiny_padded(n) && ((uintptr_t)A & 15) == 0; }

int launch_lu_tiny(const float* A, int n, int64_t batch, float* sign, float* logabs, float* lu, int* perm,
                   hipStream_t s) {
  if (n < 1 || n > TINY_MAXN) return FX_ERR_UNSUPPORTED;
  const int G = tiny_padded(n), vec = tiny_vec(A, n);
  const unsigned blocks = (unsigned)((batch * G + 255) / 256);
  if (G == 16) {
    if (lu)
      hipLaunchKernelGGL((lu_tiny_kernel<16, true>), dim3(blocks), dim3(256), 0, s, A, n, vec, batch, sign, logabs,
                         lu, perm);
    else
      hipLaunchKernelGGL((lu_tiny_kernel<16, false>), dim3(blocks), dim3(256), 0, s, A, n, vec, batch, sign, logabs,
                         nullptr, nullptr);
  } else {
    if (lu)
      hipLaunchKernelGGL((lu_tiny_kernel<32, true>), dim3(blocks), dim3(256), 0, s, A, n, vec, batch, sign, logabs,
                         lu, perm);
    else
      hipLaunchKernelGGL((lu_tiny_kernel<32, false>), dim3(blocks), dim3(256), 0, s, A, n, vec, batch, sign, logabs,
                         nullptr, nullptr);
  }
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

// Parlett-Reid for n <= PF_TINY_MAXN only: at G = 32 (two matrices per wave, three LDS
// round trips per pair step) the one-workgroup-per-matrix kernel is faster.
int launch_lu_tiny_inv(const float* A, int n, int64_t batch, int zero_singular, float* sign, float* logabs,
                       float* invT, hipStream_t s) {
  if (n < 1 || n > TINY_MAXN) return FX_ERR_UNSUPPORTED;
  const int G = tiny_padded(n), vec = tiny_vec(A, n);
  const unsigned blocks = (unsigned)((batch * G + 255) / 256);
  if (G == 16)
    hipLaunchKernelGGL((lu_tiny_inv_kernel<16>), dim3(blocks), dim3(256), 0, s, A, n, vec, batch, zero_singular, sign,
                       logabs, invT);
  else
    hipLaunchKernelGGL((lu_tiny_inv_kernel<32>), dim3(blocks), dim3(256), 0, s, A, n, vec, batch, zero_singular, sign,
                       logabs, invT);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

int launch_pf_tiny(const float* A, int n, int skew, int64_t batch, float* sign, float* logabs, float* gbuf, float* d,
                   int* perm, hipStream_t s) {
  if (n < 2 || n > PF_TINY_MAXN || (n & 1)) return FX_ERR_UNSUPPORTED;
  const int vec = tiny_vec(A, n);
  const unsigned blocks = (unsigned)((batch * 16 + 255) / 256);
  if (gbuf)
    hipLaunchKernelGGL((pf_tiny_kernel<16, true>), dim3(blocks), dim3(256), 0, s, A, n, skew, vec, batch, sign, logabs,
                       gbuf, d, perm);
  else
    hipLaunchKernelGGL((pf_tiny_kernel<16, false>), dim3(blocks), dim3(256), 0, s, A, n, skew, vec, batch, sign,
                       logabs, nullptr, nullptr, nullptr);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

}  // namespace fx
