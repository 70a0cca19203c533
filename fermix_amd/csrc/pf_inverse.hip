// S^-1 (inverse mode) or pf(S) S^-1 (adjugate mode) from the forward's own Parlett-Reid
// factors (the slogpf / pf backward), any N. With P S' P^T = L D L^T, D = diag_s(d_s J),
// the pivot K of smallest |d| and d~ = d with d_K and exact zeros replaced by 1:
//   L~ = L with the a-columns scaled by 1/d~ (unit lower), Y = L~^-1,
//   DY = rows (Y[p_s], -Y[a_s]) / d~_s,   R = Y^T DY (exactly skew),
//   G = -P^T [a1 R + a2 (w v^T - v w^T)] P,  w = R e_{a_K}, v = Y^T e_{a_K},
// inverse:   (a1, a2) = (1, (1 - d_K) / d_K), zeroed for d_K = 0 or a non-finite result;
// adjugate:  (a1, a2) = sgn(P) D_K (d_K, 1 - d_K), D_K = prod_{s != K} d_s -- finite and
//            exact for singular S (d_K enters linearly). A second exact zero pivot z is
//            lifted: G is affine in that pair entry, so G = (G(d_z = +1) + G(d_z = -1)) / 2,
//            the second evaluation running only for the members that have such a pivot.
// Kernels: pivot / coefficient prep (one wave per matrix), L~ assembly, the triangular
// inverse of inverse.hip (lower half only), DY, the skew GEMM R (lower tiles + mirror),
// the rank-2 correction with the non-finite flags, and the permutation gather.
//
// Reference roles replaced (ChenAo-Phys/fermix): _pf_parts (src/fermix/_pfinv.py:196-269)
// with _pf_assemble_kernel (:80-137), _pf_maps (:140-157), the skew _bgemm for R and
// _adj_perm_kernel (:161-192); the scalar helpers _pivot_index / _pair_scale /
// _pf_adj_coeffs / _second_zero / _lifted_mean (src/fermix/_fallback.py:101-176).
#include "common.h"
#include "fermix_internal.h"

namespace fx {

struct PfCoef {
  int K;      // pair index of the smallest |d| among the real pairs
  int bad;    // d_K == 0 (inverse mode: zero the result)
  float a1;   // coefficient of R
  float a2;   // coefficient of (w v^T - v w^T)
  int z;      // adjugate mode: first exact zero pivot other than K (lifted), or -1
};

// One wave per matrix: K, 1/d~, coefficients, and the inverse permutation. In adjugate
// mode parity[b] is the permutation's parity; lift[b] = 1 marks a member with a second
// exact zero pivot, whose coefficients here are those of the d_z = +1 evaluation, halved.
__global__ void pf_prep_kernel(const float* __restrict__ d, int H, int hreal, const int* __restrict__ perm, int N,
                               int adjugate, const int* __restrict__ parity, float* __restrict__ dinv,
                               int* __restrict__ iperm, PfCoef* __restrict__ coef, int* __restrict__ lift,
                               int64_t batch) {
  const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (b >= batch) return;
  const float* db = d + b * H;
  // argmin |d| over s < hreal, first index on ties
  unsigned best = 0xffffffffu;
  int bi = 0;
  for (int s = lane; s < hreal; s += 64) {
    const unsigned k = __float_as_uint(fabsf(db[s]));
    if (k < best) { best = k; bi = s; }
  }
  // wave argmin (key, index): reduce keys, then the lowest index holding the minimum
  unsigned m = best;
  for (int off = 32; off >= 1; off >>= 1) m = min(m, (unsigned)__shfl_xor((int)m, off));
  int cand = (best == m) ? bi : 0x7fffffff;
  for (int off = 32; off >= 1; off >>= 1) cand = min(cand, __shfl_xor(cand, off));
  const int K = cand;
  const float dK = db[K];
  // over s != K: sum log|d_s| of the nonzero pivots, the number of negative and of zero
  // pivots, and the first zero
  float lg = 0.0f;
  int negs = 0, zeros = 0, zfirst = 0x7fffffff;
  for (int s = lane; s < H; s += 64) {
    const float v = db[s];
    const float dt = (s == K || v == 0.0f) ? 1.0f : v;
    dinv[b * H + s] = 1.0f / dt;
    if (s != K) {
      lg += v != 0.0f ? logf(fabsf(v)) : 0.0f;
      negs += v < 0.0f;
      if (v == 0.0f) {
        ++zeros;
        zfirst = min(zfirst, s);
      }
    }
  }
  for (int f = lane; f < N; f += 64) iperm[b * N + perm[b * N + f]] = f;
  if (!adjugate) {
    if (lane == 0) {
      PfCoef c;
      c.K = K;
      c.bad = dK == 0.0f;
      c.a1 = 1.0f;
      c.a2 = dK != 0.0f ? (1.0f - dK) / dK : 0.0f;
      c.z = -1;
      coef[b] = c;
    }
    return;
  }
  lg = wave_sum_f32(lg);
  for (int off = 32; off >= 1; off >>= 1) {
    negs += __shfl_xor(negs, off);
    zeros += __shfl_xor(zeros, off);
    zfirst = min(zfirst, __shfl_xor(zfirst, off));
  }
  if (lane == 0) {
    const bool has2 = zeros >= 1;
    // D_K with d_z = +1: zero if a third zero pivot remains
    const float phase = (zeros - (has2 ? 1 : 0)) > 0 ? 0.0f : ((negs & 1) ? -1.0f : 1.0f);
    const float sgnP = parity[b] ? -1.0f : 1.0f;
    const float D = sgnP * phase * expf(lg) * (has2 ? 0.5f : 1.0f);
    PfCoef c;
    c.K = K;
    c.bad = 0;
    c.a1 = D * dK;
    c.a2 = D * (1.0f - dK);
    c.z = has2 ? zfirst : -1;
    coef[b] = c;
    lift[b] = has2 ? 1 : 0;
  }
}

// Second evaluation of the lifted members: d~_z = -1 (1/d~ flips sign at z). The
// coefficients of that evaluation are those of the first negated (D_K flips with d_z).
__global__ void pf_lift_kernel(const PfCoef* __restrict__ coef, int H, float* __restrict__ dinv, int64_t batch) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  const int z = coef[b].z;
  if (z >= 0) dinv[b * H + z] = -1.0f;
}

// T[f][c] = L~[f][c] (f > c), 1 on the diagonal, 0 above; identity beyond N. One
// workgroup per row f (original row o = perm[f]), four columns per thread step: a group
// of 4 columns lies in one PB-column block of gbuf, read as one 16-byte vector.
__global__ __launch_bounds__(256) void pf_assemble_kernel(const float* __restrict__ gbuf, int PB, int N,
                                                          const int* __restrict__ perm,
                                                          const float* __restrict__ dinv, float* __restrict__ T,
                                                          int Ninv, const int* __restrict__ active) {
  const int64_t b = blockIdx.y;
  if (active && !active[b]) return;
  const int f = blockIdx.x;
  float4* row = reinterpret_cast<float4*>(T + b * (int64_t)Ninv * Ninv + (int64_t)f * Ninv);
  const int nb = N / PB;
  const int o = f < N ? perm[b * N + f] : 0;
  const float* db = dinv + b * (N / 2);
  for (int c4 = threadIdx.x; c4 < Ninv / 4; c4 += 256) {
    const int c = 4 * c4;
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (f < N && c < N && f > c) {
      const int k = c / PB, col = c % PB;
      const float4 g = *reinterpret_cast<const float4*>(gbuf + ((b * nb + k) * (int64_t)N + o) * PB + col);
      const float2 di = *reinterpret_cast<const float2*>(db + (c >> 1));
      // column a = 2s holds w / d~ (w in G column 2t+1), column p = 2s+1 holds tau (G column 2t)
      v.x = f > (c | 1) ? g.y * di.x : 0.0f;
      v.y = f > (c | 1) ? g.x : 0.0f;
      v.z = f > ((c + 2) | 1) ? g.w * di.y : 0.0f;
      v.w = f > ((c + 2) | 1) ? g.z : 0.0f;
    }
    if (f >= c && f < c + 4) (&v.x)[f - c] = 1.0f;
    row[c4] = v;
  }
}

// DY[2s] = Y[2s+1] / d~_s, DY[2s+1] = -Y[2s] / d~_s with Y the unit-lower part of T.
// One workgroup per row r, 16-byte vectors along the row.
__global__ __launch_bounds__(256) void pf_dy_kernel(const float* __restrict__ T, int Ninv, int N,
                                                    const float* __restrict__ dinv, float* __restrict__ DY,
                                                    const int* __restrict__ active) {
  const int64_t b = blockIdx.y;
  if (active && !active[b]) return;
  const int r = blockIdx.x, src = r ^ 1;
  const float4* y4 = reinterpret_cast<const float4*>(T + b * (int64_t)Ninv * Ninv + (int64_t)src * Ninv);
  float4* o4 = reinterpret_cast<float4*>(DY + b * (int64_t)N * N + (int64_t)r * N);
  const float d = dinv[b * (N / 2) + (r >> 1)];
  const float sc = (r & 1) ? -d : d;
  for (int c4 = threadIdx.x; c4 < N / 4; c4 += 256) {
    const int c = 4 * c4;
    float4 y = c < src ? y4[c4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // unit lower: entries with column > src are 0, the diagonal is 1
    y.x = c < src ? y.x : (c == src ? 1.0f : 0.0f);
    y.y = c + 1 < src ? y.y : (c + 1 == src ? 1.0f : 0.0f);
    y.z = c + 2 < src ? y.z : (c + 2 == src ? 1.0f : 0.0f);
    y.w = c + 3 < src ? y.w : (c + 3 == src ? 1.0f : 0.0f);
    o4[c4] = make_float4(y.x * sc, y.y * sc, y.z * sc, y.w * sc);
  }
}

// PT = -sg (a1 R + a2 (w v^T - v w^T)); flags non-finite 64x64 tiles.
__global__ void pf_adj_kernel(const float* __restrict__ R, float* __restrict__ PT, int N, const float* __restrict__ T,
                              int Ninv, const PfCoef* __restrict__ coef, float sg, int* __restrict__ flags,
                              const int* __restrict__ active) {
  const int64_t b = blockIdx.y;
  if (active && !active[b]) return;
  const int nt = (N + 63) / 64;
  const int tile = blockIdx.x;
  const int f0 = (tile / nt) * 64, c0 = (tile % nt) * 64;
  const PfCoef cf = coef[b];
  const float a1 = sg * cf.a1, a2 = sg * cf.a2;
  const int aK = 2 * cf.K;
  const float* Rb = R + b * (int64_t)N * N;
  float* Pb = PT + b * (int64_t)N * N;
  const float* Tb = T + b * (int64_t)Ninv * Ninv;
  bool badv = false;
  // this thread's column c is fixed (64 columns, 4 rows per pass); all reads are in-bounds
  // (clamped) and issued before use
  const int cth = c0 + (threadIdx.x & 63), ccl = min(cth, N - 1);
  const float wc = Rb[ccl * N + aK];
  const float tcv = Tb[aK * Ninv + ccl];
  const float v_c = cth < aK ? tcv : (cth == aK ? 1.0f : 0.0f);
  float rv[16], wv[16], tv[16];
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int f = min(f0 + (threadIdx.x >> 6) + 4 * u, N - 1);
    rv[u] = Rb[f * N + ccl];
    wv[u] = Rb[f * N + aK];
    tv[u] = Tb[aK * Ninv + f];
  }
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int f = f0 + (threadIdx.x >> 6) + 4 * u;
    if (f < N && cth < N) {
      // v = Y^T e_aK: v[j] = Y[aK][j] (unit lower: j < aK stored, j == aK one, j > aK zero)
      const float v_f = f < aK ? tv[u] : (f == aK ? 1.0f : 0.0f);
      const float val = -(a1 * rv[u] + a2 * (wv[u] * v_c - v_f * wc));
      badv = badv || !isfinite(val);
      Pb[(int64_t)f * N + cth] = val;
    }
  }
  const int any = __syncthreads_or(badv ? 1 : 0);
  if (threadIdx.x == 0) flags[b * (nt * nt) + tile] = any;
}

// bad[b]: inverse mode only (the adjugate is returned as computed).
__global__ void pf_reduce_bad_kernel(const int* __restrict__ flags, int ntiles, const PfCoef* __restrict__ coef,
                                     int adjugate, int* __restrict__ bad, int64_t batch) {
  const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (b >= batch) return;
  bool f = false;
  for (int k = lane; k < ntiles; k += 64) f = f || flags[b * ntiles + k] != 0;
  const bool any = __ballot(f) != 0ull;
  if (lane == 0) bad[b] = (!adjugate && (any || coef[b].bad)) ? 1 : 0;
}

// out[i][j] = sc PT[iperm i][iperm j] for i, j < n (or 0 for a bad member), sc = scale[b]
// or 1; with accumulate out[i][j] += sc PT[..] for the active members. One workgroup per
// output row: source row iperm[i] is read contiguously into LDS and the column
// permutation is applied there.
__global__ __launch_bounds__(256) void pf_gather_kernel(const float* __restrict__ PT, int N,
                                                        const int* __restrict__ iperm, int n,
                                                        const int* __restrict__ bad, float* __restrict__ out,
                                                        const int* __restrict__ active, int accumulate,
                                                        const float* __restrict__ scale) {
  __shared__ __align__(16) float rowb[PF_LARGE_MAXN];
  const int64_t b = blockIdx.y;
  if (active && !active[b]) return;
  const int i = blockIdx.x;
  float* o = out + b * (int64_t)n * n + (int64_t)i * n;
  if (bad[b]) {
    for (int j = threadIdx.x; j < n; j += 256) o[j] = 0.0f;
    return;
  }
  const int* ip = iperm + b * N;
  const float4* s4 = reinterpret_cast<const float4*>(PT + b * (int64_t)N * N + (int64_t)ip[i] * N);
  for (int c4 = threadIdx.x; c4 < N / 4; c4 += 256) reinterpret_cast<float4*>(rowb)[c4] = s4[c4];
  __syncthreads();
  if (scale) {
    const float sc = scale[b];
    if (accumulate) {
      for (int j = threadIdx.x; j < n; j += 256) o[j] += sc * rowb[ip[j]];
    } else {
      for (int j = threadIdx.x; j < n; j += 256) o[j] = sc * rowb[ip[j]];
    }
  } else if (accumulate) {
    for (int j = threadIdx.x; j < n; j += 256) o[j] += rowb[ip[j]];
  } else {
    for (int j = threadIdx.x; j < n; j += 256) o[j] = rowb[ip[j]];
  }
}

size_t pf_inverse_workspace(int64_t batch, int N) {
  const int Ninv = inv_padded(N);
  const int nt = (N + 63) / 64;
  size_t bytes = 0;
  auto add = [&](size_t x) { bytes += (x + 255) / 256 * 256; };
  add((size_t)batch * Ninv * Ninv * 4);  // T (L~, then Y)
  add((size_t)batch * Ninv * Ninv);      // Tmp (Ninv/2 x Ninv/2 floats)
  add((size_t)batch * N * N * 4);        // DY
  add((size_t)batch * N * N * 4);        // R / PT
  add((size_t)batch * N / 2 * 4);        // dinv
  add((size_t)batch * N * 4);            // iperm
  add((size_t)batch * sizeof(PfCoef));
  add((size_t)batch * nt * nt * 4);      // flags
  add((size_t)batch * 4);                // bad
  add((size_t)batch * 4);                // parity
  add((size_t)batch * 4);                // lift
  return bytes;
}

int launch_pf_inverse(const float* gbuf, int PB, const float* d, const int* perm, int N, int n, int64_t batch,
                      int adjugate, float* out, void* ws, size_t ws_bytes, hipStream_t s, const float* scale) {
  const int Ninv = inv_padded(N);
  if (!ws || ws_bytes < pf_inverse_workspace(batch, N)) return FX_ERR_WORKSPACE;
  char* p = (char*)ws;
  auto take = [&](size_t x) {
    char* q = p;
    p += (x + 255) / 256 * 256;
    return (void*)q;
  };
  float* T = (float*)take((size_t)batch * Ninv * Ninv * 4);
  float* Tmp = (float*)take((size_t)batch * Ninv * Ninv);
  float* DY = (float*)take((size_t)batch * N * N * 4);
  float* R = (float*)take((size_t)batch * N * N * 4);
  float* dinv = (float*)take((size_t)batch * N / 2 * 4);
  int* iperm = (int*)take((size_t)batch * N * 4);
  PfCoef* coef = (PfCoef*)take((size_t)batch * sizeof(PfCoef));
  const int nt = (N + 63) / 64;
  int* flags = (int*)take((size_t)batch * nt * nt * 4);
  int* bad = (int*)take((size_t)batch * 4);
  int* parity = (int*)take((size_t)batch * 4);
  int* lift = (int*)take((size_t)batch * 4);
  const int64_t NN = (int64_t)Ninv * Ninv;
  const int64_t MM = (int64_t)N * N;
  const unsigned wb = (unsigned)((batch + 3) / 4);
  if (adjugate) {
    const int st = launch_perm_parity(perm, N, batch, parity, s);
    if (st != FX_OK) return st;
  }
  hipLaunchKernelGGL(pf_prep_kernel, dim3(wb), dim3(256), 0, s, d, N / 2, n / 2, perm, N, adjugate, parity, dinv,
                     iperm, coef, lift, batch);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  // One evaluation of -(a1 R + a2 (w v^T - v w^T)) for the current dinv, written to (or,
  // with accumulate, added to) out; `active` restricts it to the marked members.
  auto evaluate = [&](const int* active, float sg, int accumulate) -> int {
    hipLaunchKernelGGL(pf_assemble_kernel, dim3((unsigned)Ninv, (unsigned)batch), dim3(256), 0, s, gbuf, PB, N,
                       perm, dinv, T, Ninv, active);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
    int st = launch_unit_lower_inverse(T, Ninv, batch, Tmp, s, active);
    if (st != FX_OK) return st;
    hipLaunchKernelGGL(pf_dy_kernel, dim3((unsigned)N, (unsigned)batch), dim3(256), 0, s, T, Ninv, N, dinv, DY,
                       active);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
    {
      // R = Y^T DY: op(A) = Y^T (upper, unit diagonal), lower tiles, mirrored skew
      GemmDesc g = {};
      g.M = g.N = g.K = N;
      g.A = T;
      g.transA = 1;
      g.maskA = MASK_UPPER_UNIT;
      g.lda = Ninv;
      g.sA = NN;
      g.B = DY;
      g.ldb = N;
      g.sB = MM;
      g.C = R;
      g.ldc = N;
      g.sC = MM;
      g.alpha = 1.0f;
      g.beta = 0.0f;
      g.lower_only = 1;
      g.mirror = -1.0f;
      g.active = active;
      st = launch_gemm(g, batch, 1, s);
      if (st != FX_OK) return st;
    }
    float* PT = DY;  // DY is dead once R is formed
    hipLaunchKernelGGL(pf_adj_kernel, dim3(nt * nt, (unsigned)batch), dim3(256), 0, s, R, PT, N, T, Ninv, coef, sg,
                       flags, active);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
    if (!accumulate) {
      hipLaunchKernelGGL(pf_reduce_bad_kernel, dim3(wb), dim3(256), 0, s, flags, nt * nt, coef, adjugate, bad,
                         batch);
      if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
    }
    hipLaunchKernelGGL(pf_gather_kernel, dim3((unsigned)n, (unsigned)batch), dim3(256), 0, s, PT, N, iperm, n, bad,
                       out, active, accumulate, scale);
    return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
  };
  int st = evaluate(nullptr, 1.0f, 0);
  if (st != FX_OK || !adjugate) return st;
  // the lifted members' second evaluation (every other member's workgroups exit at once)
  hipLaunchKernelGGL(pf_lift_kernel, dim3((unsigned)((batch + 255) / 256)), dim3(256), 0, s, coef, N / 2, dinv,
                     batch);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  return evaluate(lift, -1.0f, 1);
}

}  // namespace fx
