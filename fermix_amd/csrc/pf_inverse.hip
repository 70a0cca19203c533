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
// inverse of inverse.hip (lower half only), the skew GEMM R (lower tiles + mirror; its
// B operand DY is read from Y through the GEMM's row pair swap and per-row scale, so DY
// is never stored),
// and the permutation gather with the rank-2 correction and the non-finite flags formed
// on the way (no corrected matrix is stored between them).
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

// The two vectors of the rank-2 correction in output order, vw (B, 2, N): w_c = R[c][2K]
// (a column of R) and v_c = Y[2K][c] for c < 2K, 1 at 2K, 0 after (v = Y^T e_2K), stored
// at j with c = iperm[j]; one thread per j.
__global__ void pf_wvec_kernel(const float* __restrict__ R, int N, const float* __restrict__ T, int Ninv,
                               const PfCoef* __restrict__ coef, const int* __restrict__ iperm,
                               float* __restrict__ vw, const int* __restrict__ active) {
  const int64_t b = blockIdx.y;
  if (active && !active[b]) return;
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= N) return;
  const int aK = 2 * coef[b].K, c = iperm[b * N + j];
  vw[2 * b * N + j] = R[b * (int64_t)N * N + (int64_t)c * N + aK];
  const float y = T[b * (int64_t)Ninv * Ninv + (int64_t)aK * Ninv + c];
  vw[(2 * b + 1) * N + j] = c < aK ? y : (c == aK ? 1.0f : 0.0f);
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

// The final matrix straight from R (skew, both triangles stored): with f = iperm[i],
// c = iperm[j] (the factor order of output row i / column j),
//   out[i][j] = sc * -(a1 R[f][c] + a2 (w_f v_c - v_f w_c)),
// w = R[:, 2K], v = Y^T e_2K (both in output order in vw), a1 / a2 the member's
// coefficients times sg, sc = scale[b] or 1; with accumulate the value is added for the
// active members. One workgroup per RPW rows i < N: the source rows f of R are read
// contiguously into LDS and the column permutation applied there; rows / columns >= n
// are evaluated (flags[b][i] marks a non-finite value among the workgroup's rows) but
// not stored. MAXJ >= N / 256: the columns per thread, a template parameter so that the
// per-thread column tables (three registers per column) match N.
template <int RPW, int MAXJ>
__global__ __launch_bounds__(256) void pf_adj_gather_kernel(const float* __restrict__ R, int N,
                                                            const PfCoef* __restrict__ coef, float sg,
                                                            const float* __restrict__ vw,
                                                            const int* __restrict__ iperm, int n,
                                                            int* __restrict__ flags, float* __restrict__ out,
                                                            const int* __restrict__ active, int accumulate,
                                                            const float* __restrict__ scale) {
  extern __shared__ __align__(16) float pf_gather_lds[];  // RPW N floats (launch-time size)
  const int64_t b = blockIdx.y;
  if (active && !active[b]) return;
  const int i0 = RPW * blockIdx.x;
  const int* ip = iperm + b * N;
  const float* wp = vw + 2 * b * N;
  const float* vp = wp + N;
  int f[RPW];
  float wf[RPW], vf[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int i = min(i0 + r, N - 1);
    f[r] = ip[i];
    wf[r] = wp[i];
    vf[r] = vp[i];
  }
  const PfCoef cf = coef[b];
  const float a1 = sg * cf.a1, a2 = sg * cf.a2;
  const float* Rb = R + b * (int64_t)N * N;
  // the column permutation and the correction vectors of this thread's outputs, loaded
  // with the rows (one round trip)
  int cj[MAXJ];
  float wj[MAXJ], vj[MAXJ];
#pragma unroll
  for (int u = 0; u < MAXJ; ++u) {
    const int j = min((int)threadIdx.x + 256 * u, N - 1);
    cj[u] = ip[j];
    wj[u] = wp[j];
    vj[u] = vp[j];
  }
  for (int c4 = threadIdx.x; c4 < N / 4; c4 += 256) {
#pragma unroll
    for (int r = 0; r < RPW; ++r)
      reinterpret_cast<float4*>(pf_gather_lds + r * N)[c4] = reinterpret_cast<const float4*>(Rb + (int64_t)f[r] * N)[c4];
  }
  const float sc = scale ? scale[b] : 1.0f;
  __syncthreads();
  bool nf = false;
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int i = i0 + r;
    if (i >= N) break;
    const float* rowb = pf_gather_lds + r * N;
    float* o = out + b * (int64_t)n * n + (int64_t)i * n;
#pragma unroll
    for (int u = 0; u < MAXJ; ++u) {
      const int j = threadIdx.x + 256 * u;
      if (j < N) {
        const float val = -(a1 * rowb[cj[u]] + a2 * (wf[r] * vj[u] - vf[r] * wj[u]));
        nf = nf || !isfinite(val);
        if (i < n && j < n) {
          if (accumulate) o[j] += sc * val;
          else o[j] = sc * val;
        }
      }
    }
  }
  const int any = __syncthreads_or(nf ? 1 : 0);
  if (threadIdx.x < RPW && i0 + threadIdx.x < N) flags[b * N + i0 + threadIdx.x] = any;
}

// out[b] = 0 for the flagged members (one workgroup per member; others exit at once).
__global__ __launch_bounds__(256) void pf_zero_bad_kernel(const int* __restrict__ bad, float* __restrict__ out,
                                                          int64_t nn) {
  const int64_t b = blockIdx.x;
  if (!bad[b]) return;
  float* o = out + b * nn;
  for (int64_t e = threadIdx.x; e < nn; e += 256) o[e] = 0.0f;
}

size_t pf_inverse_workspace(int64_t batch, int N) {
  const int Ninv = inv_padded(N);
  size_t bytes = 0;
  auto add = [&](size_t x) { bytes += (x + 255) / 256 * 256; };
  add((size_t)batch * Ninv * Ninv * 4);  // T (L~, then Y)
  add((size_t)batch * Ninv * Ninv);      // Tmp (Ninv/2 x Ninv/2 floats)
  add((size_t)batch * N * N * 4);        // R
  add((size_t)batch * 2 * N * 4);        // vw: w and v in output order
  add((size_t)batch * N / 2 * 4);        // dinv
  add((size_t)batch * N * 4);            // iperm
  add((size_t)batch * sizeof(PfCoef));
  add((size_t)batch * N * 4);            // flags (one per row)
  add((size_t)batch * 4);                // bad
  add((size_t)batch * 4);                // parity
  add((size_t)batch * 4);                // lift
  return bytes;
}

int launch_pf_inverse(const float* gbuf, int PB, const float* d, const int* perm, int N, int n, int64_t batch,
                      int adjugate, float* out, void* ws, size_t ws_bytes, hipStream_t s, const float* scale,
                      int x3) {
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
  float* R = (float*)take((size_t)batch * N * N * 4);
  float* vw = (float*)take((size_t)batch * 2 * N * 4);
  float* dinv = (float*)take((size_t)batch * N / 2 * 4);
  int* iperm = (int*)take((size_t)batch * N * 4);
  PfCoef* coef = (PfCoef*)take((size_t)batch * sizeof(PfCoef));
  int* flags = (int*)take((size_t)batch * N * 4);
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
    int st = launch_unit_lower_inverse(T, Ninv, batch, Tmp, s, active, x3);
    if (st != FX_OK) return st;
    {
      // R = Y^T DY: op(A) = Y^T (upper, unit diagonal), lower tiles, mirrored skew
      GemmDesc g = {};
      g.x3 = x3;
      g.M = g.N = g.K = N;
      g.A = T;
      g.transA = 1;
      g.maskA = MASK_UPPER_UNIT;
      g.lda = Ninv;
      g.sA = NN;
      // B = DY = rows (Y[p_s], -Y[a_s]) / d~_s, read from Y by the GEMM's row transform
      // (Y keeps exact zeros above and ones on its diagonal)
      g.B = T;
      g.ldb = Ninv;
      g.sB = NN;
      g.bscale = dinv;
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
    hipLaunchKernelGGL(pf_wvec_kernel, dim3((unsigned)((N + 255) / 256), (unsigned)batch), dim3(256), 0, s, R, N,
                       T, Ninv, coef, iperm, vw, active);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
    // two rows per workgroup: measured 383 us at B = 64, N = 2048 against 520 (one), 463 (four);
    // the column tables sized for N (sized for 8192 at every N: 673 us there)
    constexpr int RPW = 2;
    const dim3 gg((unsigned)((N + RPW - 1) / RPW), (unsigned)batch);
    const size_t gl = RPW * N * sizeof(float);
    if (N <= 2048)
      hipLaunchKernelGGL((pf_adj_gather_kernel<RPW, 8>), gg, dim3(256), gl, s, R, N, coef, sg, vw, iperm, n, flags, out,
                         active, accumulate, scale);
    else if (N <= 4096)
      hipLaunchKernelGGL((pf_adj_gather_kernel<RPW, 16>), gg, dim3(256), gl, s, R, N, coef, sg, vw, iperm, n, flags,
                         out, active, accumulate, scale);
    else
      hipLaunchKernelGGL((pf_adj_gather_kernel<RPW, PF_LARGE_MAXN / 256>), gg, dim3(256), gl, s, R, N, coef, sg, vw,
                         iperm, n, flags, out, active, accumulate, scale);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
    if (accumulate) return FX_OK;
    // inverse mode: members with d_K = 0 or a non-finite value anywhere are zeroed
    hipLaunchKernelGGL(pf_reduce_bad_kernel, dim3(wb), dim3(256), 0, s, flags, N, coef, adjugate, bad, batch);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
    hipLaunchKernelGGL(pf_zero_bad_kernel, dim3((unsigned)batch), dim3(256), 0, s, bad, out, (int64_t)n * n);
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
