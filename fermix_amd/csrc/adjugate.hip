// Gradients of det and pf that stay finite (and exact) for singular inputs: the
// permutation parity of a row map, and the determinant adjugate adj(A)^T = d det / dA
// from the packed LU of the slogdet backward.
//
// det adjugate (P A' = L U, A' = A padded with I, pivots d = diag(U)):
//   regular:   adj(A)^T = det * A^-T with det = sgn(P) prod(d) of these very factors, so
//              the round-off-level pivot of a numerically singular A cancels exactly
//              between det and the 1/d inside A^-T;
//   zero pivots at k1 <= ... <= km, U~ = U with them replaced by 1, d_K = product of
//   the other pivots:
//              adj(A)^T[i][j] = s * (A~^-T)[i][k_m] * (U~^-1 e_k1)[j],
//              s = sgn(P) d_K (m = 1),  sgn(P) d_K (U~^-1)[k1][k2] (m = 2),  0 (m >= 3),
//   with A~^-T the transposed inverse formed from U~ (the slogdet backward's invT).
//
// Reference roles replaced (ChenAo-Phys/fermix): _perm_sign (src/fermix/_diff.py:160-176),
// _lu_det (:184-202) and _det_gradT (:205-246), which the reference evaluates in XLA on
// top of _lu_parts(zero_singular=False); here they are three kernels around the inverse.
#include "common.h"
#include "fermix_internal.h"

namespace fx {

// parity[b] = (N - number of cycles of perm[b]) mod 2, i.e. 1 for an odd permutation. The
// cycles are found by pointer jumping in LDS: after r rounds lab[i] is the smallest index
// among the 2^r orbit elements starting at i and nx[i] = perm^(2^r)(i), so after
// ceil(log2 N) rounds every element carries its cycle's minimum and each cycle has exactly
// one element labelled by itself. One workgroup per member, N <= PARITY_MAXN.
constexpr int PARITY_MAXN = 8192;

__global__ __launch_bounds__(256) void perm_parity_kernel(const int* __restrict__ perm, int N,
                                                          int* __restrict__ parity) {
  constexpr int U = PARITY_MAXN / 256;
  __shared__ int lab[PARITY_MAXN], nx[PARITY_MAXN];
  __shared__ int wcount[4];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  const int* g = perm + b * N;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int i = tid + 256 * u;
    if (i < N) {
      lab[i] = i;
      nx[i] = min(max(g[i], 0), N - 1);
    }
  }
  __syncthreads();
  for (int span = 1; span < N; span *= 2) {
    int nl[U], nn[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = tid + 256 * u;
      nl[u] = 0;
      nn[u] = 0;
      if (i < N) {
        const int q = nx[i];
        nl[u] = min(lab[i], lab[q]);
        nn[u] = nx[q];
      }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = tid + 256 * u;
      if (i < N) {
        lab[i] = nl[u];
        nx[i] = nn[u];
      }
    }
    __syncthreads();
  }
  int cnt = 0;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int i = tid + 256 * u;
    cnt += __popcll(__ballot(i < N && lab[i] == i));
  }
  if ((tid & 63) == 0) wcount[tid >> 6] = cnt;
  __syncthreads();
  if (tid == 0) parity[b] = (N - (wcount[0] + wcount[1] + wcount[2] + wcount[3])) & 1;
}

int launch_perm_parity(const int* perm, int N, int64_t batch, int* parity, hipStream_t s) {
  if (N > PARITY_MAXN) return FX_ERR_UNSUPPORTED;
  if (batch <= 0) return FX_OK;
  hipLaunchKernelGGL(perm_parity_kernel, dim3((unsigned)batch), dim3(256), 0, s, perm, N, parity);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

// ------------------------------------------------------------------ det adjugate

constexpr int DET_ADJ_MAXN = LU_LARGE_MAXN;

// Per-member result of det_prep_kernel.
struct DetCoef {
  int mode;     // 0: G = scale * invT; 1: G = (scale * invT)[:, k2] (x) u1; 2: G = 0
  int k2;       // largest zero-pivot index (mode 1)
  float scale;  // det of the factors (mode 0), s (mode 1), 0 (mode 2)
  int m;        // number of exact zero pivots
};

// Block sums over the 256 threads (4 waves) of a workgroup, deterministic order.
__device__ __forceinline__ float block_sum_f32(float v, float* red) {
  v = wave_sum_f32(v);
  const int tid = threadIdx.x;
  if ((tid & 63) == 0) red[tid >> 6] = v;
  __syncthreads();
  const float r = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return r;
}

__device__ __forceinline__ int block_sum_i32(int v, int* red) {
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  const int tid = threadIdx.x;
  if ((tid & 63) == 0) red[tid >> 6] = v;
  __syncthreads();
  const int r = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return r;
}

__device__ __forceinline__ int block_min_i32(int v, int* red) {
  for (int off = 32; off >= 1; off >>= 1) v = min(v, __shfl_xor(v, off));
  const int tid = threadIdx.x;
  if ((tid & 63) == 0) red[tid >> 6] = v;
  __syncthreads();
  const int r = min(min(red[0], red[1]), min(red[2], red[3]));
  __syncthreads();
  return r;
}

// xs[i] for kbot <= i < ktop of the solution of U~ x = e_ktop (U~ = the upper triangle of
// the packed LU LUb with exact zero pivots replaced by 1); xs must hold e_ktop on entry.
// Rows are processed in blocks of 64 from the top: the four waves first form the
// contribution of the already solved entries (j >= r1) to the block's rows -- independent,
// coalesced row reads -- and wave 0 then solves the block's 64 x 64 triangle from LDS by
// column updates, one lane per row.
__device__ void back_solve(const float* __restrict__ LUb, int N, int ktop, int kbot, float* xs, float* ub,
                           float* accs) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  for (int r1 = ktop; r1 > kbot; r1 -= 64) {
    const int r0 = max(kbot, r1 - 64), rows = r1 - r0;
    // (1) accs[l] = sum_{r1 <= j <= ktop} U[r0 + l][j] xs[j]; wave w takes rows w, w+4, ..
    float part[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) part[q] = 0.0f;
    for (int j0 = r1; j0 <= ktop; j0 += 64) {
      const int j = j0 + lane;
      const bool okj = j <= ktop;
      const float xj = okj ? xs[j] : 0.0f;
      const int jc = okj ? j : ktop;
      float uv[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int l = wave + 4 * q;
        const int row = r0 + min(l, rows - 1);
        uv[q] = LUb[(int64_t)row * N + jc];
      }
#pragma unroll
      for (int q = 0; q < 16; ++q) part[q] = fmaf(uv[q], xj, part[q]);
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const float sum = wave_sum_f32(part[q]);
      const int l = wave + 4 * q;
      if (lane == 0 && l < rows) accs[l] = sum;
    }
    // (2) the block's triangle ub[l][c] = U[r0 + l][r0 + c] (c >= l) into LDS
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int e = tid + 256 * u;
      const int l = e >> 6, c = e & 63;
      float v = 0.0f;
      if (l < rows && c < rows && c >= l) v = LUb[(int64_t)(r0 + l) * N + r0 + c];
      ub[l * 65 + c] = v;
    }
    __syncthreads();
    if (wave == 0) {
      float a = lane < rows ? accs[lane] : 0.0f;
      const float dg = lane < rows ? ub[lane * 65 + lane] : 1.0f;
      const float dinv = 1.0f / (dg == 0.0f ? 1.0f : dg);
      float xmine = 0.0f;
      for (int li = rows - 1; li >= 0; --li) {
        const float xi = -readlane_f(a, li) * readlane_f(dinv, li);
        if (lane == li) xmine = xi;
        if (lane < li) a = fmaf(ub[lane * 65 + li], xi, a);
      }
      if (lane < rows) xs[r0 + lane] = xmine;
    }
    __syncthreads();
  }
}

// One workgroup per member: the pivots' zero pattern, the determinant of the factors and,
// for one or two zero pivots, the vector u1 = (U~^-1 e_k1)[:n] and s.
__global__ __launch_bounds__(256) void det_prep_kernel(const float* __restrict__ LU, int N, int n,
                                                       const int* __restrict__ parity, DetCoef* __restrict__ coef,
                                                       float* __restrict__ scale, float* __restrict__ u1) {
  __shared__ float xs[DET_ADJ_MAXN];
  __shared__ float ub[64 * 65];
  __shared__ float accs[64];
  __shared__ float redf[4];
  __shared__ int redi[4];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  const float* LUb = LU + b * (int64_t)N * N;
  constexpr int DU = DET_ADJ_MAXN / 256;
  float dv[DU];
#pragma unroll
  for (int u = 0; u < DU; ++u) {
    const int i = min(tid + 256 * u, N - 1);
    dv[u] = LUb[(int64_t)i * (N + 1)];
  }
  int zc = 0, negs = 0, kmin = N, kmax = -1;
  float lg = 0.0f;
#pragma unroll
  for (int u = 0; u < DU; ++u) {
    const int i = tid + 256 * u;
    if (i < N) {
      const bool z = dv[u] == 0.0f;
      zc += z;
      negs += dv[u] < 0.0f;
      kmin = z ? min(kmin, i) : kmin;
      kmax = z ? max(kmax, i) : kmax;
      lg += z ? 0.0f : logf(fabsf(dv[u]));
    }
  }
  const int m = block_sum_i32(zc, redi);
  const int ng = block_sum_i32(negs, redi);
  const int k1 = block_min_i32(kmin, redi);
  const int k2 = -block_min_i32(-kmax, redi);
  lg = block_sum_f32(lg, redf);
  const float sgnP = parity[b] ? -1.0f : 1.0f;
  const float dK = ((ng & 1) ? -1.0f : 1.0f) * expf(lg);  // product of the nonzero pivots
  // m >= 3: rank <= n - 2 up to the one case the two-pivot formula does not cover, and G
  // = 0 (the reference's convention). A zero pivot in the identity padding (k2 >= n) does
  // not occur with the lowest-row tie-breaking of the LU kernels; it is mapped to 0 too so
  // that the column read of det_rank1_kernel stays inside the n x n block.
  if (m == 0 || m >= 3 || k2 >= n) {
    if (tid == 0) {
      DetCoef c;
      c.mode = m == 0 ? 0 : 2;
      c.k2 = 0;
      c.scale = m == 0 ? sgnP * dK : 0.0f;
      c.m = m;
      coef[b] = c;
      scale[b] = c.scale;
    }
    return;
  }
  // m is 1 or 2: (U~^-1)[k1][k2] from U~ y = e_k2 (m = 2), then u1 from U~ x = e_k1
  float cval = 1.0f;
  if (m == 2) {
    for (int i = tid; i < N; i += 256) xs[i] = i == k2 ? 1.0f : 0.0f;
    __syncthreads();
    back_solve(LUb, N, k2, k1, xs, ub, accs);
    cval = xs[k1];
    __syncthreads();
  }
  for (int i = tid; i < N; i += 256) xs[i] = i == k1 ? 1.0f : 0.0f;
  __syncthreads();
  back_solve(LUb, N, k1, 0, xs, ub, accs);
  float* ob = u1 + b * (int64_t)n;
  for (int j = tid; j < n; j += 256) ob[j] = xs[j];
  if (tid == 0) {
    DetCoef c;
    c.mode = 1;
    c.k2 = k2;
    c.scale = sgnP * dK * cval;
    c.m = m;
    coef[b] = c;
    scale[b] = c.scale;
  }
}

// G[i][j] = G[i][k2] * u1[j] for the members in mode 1 (G already holds scale * invT); the
// column is staged in LDS before any row is rewritten. One workgroup per member.
__global__ __launch_bounds__(256) void det_rank1_kernel(const DetCoef* __restrict__ coef,
                                                        const float* __restrict__ u1, int n,
                                                        float* __restrict__ G) {
  __shared__ float colv[DET_ADJ_MAXN], uv[DET_ADJ_MAXN];
  const int64_t b = blockIdx.x;
  const DetCoef c = coef[b];
  if (c.mode != 1) return;
  float* Gb = G + b * (int64_t)n * n;
  for (int i = threadIdx.x; i < n; i += 256) {
    colv[i] = Gb[(int64_t)i * n + c.k2];
    uv[i] = u1[b * (int64_t)n + i];
  }
  __syncthreads();
  const int64_t nn = (int64_t)n * n;
  for (int64_t e = threadIdx.x; e < nn; e += 256) {
    const int i = (int)(e / n), j = (int)(e - (int64_t)i * n);
    Gb[e] = colv[i] * uv[j];
  }
}

size_t det_adjugate_workspace(int64_t batch, int n) {
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  return al((size_t)batch * sizeof(DetCoef)) + al((size_t)batch * 4) * 2 + al((size_t)batch * n * 4);
}

int launch_det_adjugate_prep(const float* LU, const int* g0, int N, int n, int64_t batch, void* ws,
                             float** scale_out, hipStream_t s) {
  if (N > DET_ADJ_MAXN) return FX_ERR_UNSUPPORTED;
  char* p = (char*)ws;
  auto take = [&](size_t x) {
    char* q = p;
    p += (x + 255) / 256 * 256;
    return (void*)q;
  };
  take((size_t)batch * sizeof(DetCoef));
  int* parity = (int*)take((size_t)batch * 4);
  float* scale = (float*)take((size_t)batch * 4);
  float* u1 = (float*)take((size_t)batch * n * 4);
  DetCoef* coef = (DetCoef*)ws;
  int st = launch_perm_parity(g0, N, batch, parity, s);
  if (st != FX_OK) return st;
  hipLaunchKernelGGL(det_prep_kernel, dim3((unsigned)batch), dim3(256), 0, s, LU, N, n, parity, coef, scale, u1);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  *scale_out = scale;
  return FX_OK;
}

int launch_det_adjugate_finish(int n, int64_t batch, void* ws, float* G, hipStream_t s) {
  char* p = (char*)ws;
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  const DetCoef* coef = (const DetCoef*)p;
  const float* u1 = (const float*)(p + al((size_t)batch * sizeof(DetCoef)) + al((size_t)batch * 4) * 2);
  hipLaunchKernelGGL(det_rank1_kernel, dim3((unsigned)batch), dim3(256), 0, s, coef, u1, n, G);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

}  // namespace fx
