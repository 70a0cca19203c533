// A^-T from the packed LU of P A' (the slogdet backward), any N: the factors are
// embedded in T (Ninv x Ninv, Ninv = 32 * 2^k >= N, identity padded) and
//   1. the 128x128 (or Ninv x Ninv, if smaller) diagonal blocks are inverted in place in
//      LDS: strictly-lower part of L^-1, upper part of U~^-1 (U~ = U with exact zero
//      pivots replaced by 1, so singular inputs stay finite);
//   2. the block-recursive levels s = 128, 256, .., Ninv/2 complete L^-1 and U~^-1 with
//      four batched MFMA GEMMs per level (all block pairs of a level in one launch):
//        X21 = -X22 (L21 X11),   Y12 = -Y11 (U12 Y22);
//   3. Z = U~^-1 L^-1 by one GEMM whose tiles only run over k >= max(row, col), its
//      epilogue storing invT[g0[c]][i] = Z[i][c] (transpose + row permutation through
//      LDS) and flagging tiles with a non-finite value; Z itself is never stored;
//   4. invT is zeroed for members with a non-finite Z or, if requested, an exactly zero
//      pivot.
// Total 4/3 N^3 of MFMA work (L^-1 and U^-1 N^3/3 each, the triangular product 2N^3/3).
//
// Reference roles replaced (ChenAo-Phys/fermix): _packed_lu / _diag_kernel leaf
// inverses (src/fermix/_inverse.py:75-221), _inv_unit_lower (:429-452), _solve_upper
// (:455-474) and _permT with the singular guard (:478-531).
#include "common.h"
#include "fermix_internal.h"

namespace fx {

// 32-bit index math (Ninv <= 2048).
__global__ void embed_kernel(const float* __restrict__ src, int N, float* __restrict__ T, int Ninv) {
  const int64_t b = blockIdx.y;
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= Ninv * Ninv) return;
  const int r = e / Ninv, c = e - r * Ninv;
  T[b * Ninv * Ninv + e] = (r < N && c < N) ? src[b * (int64_t)N * N + r * N + c] : (r == c ? 1.0f : 0.0f);
}

typedef float v16f __attribute__((ext_vector_type(16)));

// op values of the packed block in LDS: the unit-lower factor (strictly lower entries,
// 1 on the diagonal) and the upper factor (upper entries incl. the diagonal)
__device__ __forceinline__ float lunit_at(const float* Ts, int ld, int r, int c) {
  return r > c ? Ts[r * ld + c] : (r == c ? 1.0f : 0.0f);
}
__device__ __forceinline__ float upper_at(const float* Ts, int ld, int r, int c) {
  return r <= c ? Ts[r * ld + c] : 0.0f;
}

// In-place inverses of the D x D diagonal blocks of the packed T (D = min(128, Ninv)):
// the strictly-lower part becomes L^-1, and with upper the upper part U~^-1, over the
// whole block, in one workgroup with the block in LDS:
//   1. the 32x32 leaves by substitution, one wave per leaf: lane c (< 32) forms column c
//      of L^-1 by forward substitution, lane 32 + c column c of U~^-1 by back
//      substitution (zero pivots divided as 1);
//   2. the recursion levels s = 32, 64 < D on MFMA (32x32x2): X21 = -X22 (L21 X11) and
//      Y12 = -Y11 (U12 Y22), one (pair, factor, 32-column block) per wave. The inner
//      product stays in registers and enters the outer one as it stands (lane (h, c)
//      holding rows 8 (v / 4) + 4 h + v % 4: one MFMA per v over those K indices, the
//      left operand read from LDS in that order); a barrier separates the reads of
//      L21 / U12 from the in-place stores of X21 / Y12.
template <int D>
__global__ __launch_bounds__(256) void diag_inverse_kernel(float* __restrict__ T, int Ninv,
                                                           const int* __restrict__ active, int upper) {
  constexpr int LDT = D + 1;
  __shared__ float Ts[D * LDT];
  const int64_t b = blockIdx.y;
  if (active && !active[b]) return;
  const int t0 = D * blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  float* base = T + b * (int64_t)Ninv * Ninv + (int64_t)t0 * Ninv + t0;
  {
    constexpr int NV = D * D / 4, PER = (NV + 255) / 256;
    float4 v[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int e = tid + 256 * u;
      if (NV % 256 == 0 || e < NV) v[u] = *reinterpret_cast<const float4*>(base + (e / (D / 4)) * Ninv + 4 * (e % (D / 4)));
    }
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int e = tid + 256 * u;
      if (NV % 256 == 0 || e < NV) {
        float* d = Ts + (e / (D / 4)) * LDT + 4 * (e % (D / 4));
        d[0] = v[u].x;
        d[1] = v[u].y;
        d[2] = v[u].z;
        d[3] = v[u].w;
      }
    }
  }
  __syncthreads();
  // 1. leaves
  if (wave < D / 32) {
    const int lo = 32 * wave, c = lane & 31;
    float x[32];
    if (lane < 32) {
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < i; ++k) acc = fmaf(Ts[(lo + i) * LDT + lo + k], x[k], acc);
        x[i] = (i == c) ? 1.0f : (i > c ? -acc : 0.0f);
      }
    } else if (upper) {
#pragma unroll
      for (int i = 31; i >= 0; --i) {
        float acc = (i == c) ? 1.0f : 0.0f;
#pragma unroll
        for (int k = i + 1; k < 32; ++k) acc = fmaf(-Ts[(lo + i) * LDT + lo + k], x[k], acc);
        const float dg = Ts[(lo + i) * LDT + lo + i];
        x[i] = (i > c) ? 0.0f : acc / (dg == 0.0f ? 1.0f : dg);
      }
    }
    // both halves of the wave have read the leaf (the branches run one after the other)
    if (lane < 32 || upper) {
#pragma unroll
      for (int i = 0; i < 32; ++i)
        if (lane < 32 ? (i > c) : (i <= c)) Ts[(lo + i) * LDT + lo + c] = x[i];
    }
  }
  __syncthreads();
  // 2. levels s = 32, 64 below D
  const int l32 = lane & 31, lh = lane >> 5;
  static_for<0, 2>([&](auto lc) {
    constexpr int s = 32 << decltype(lc)::value;
    if constexpr (s < D) {
      constexpr int NCB = s / 32;  // 32-column blocks (and 32-row tiles) of an s x s block
      const int chains = upper ? 2 : 1;
      const int items = (D / (2 * s)) * chains * NCB;  // <= 4
      const bool act = wave < items;
      const int J = wave % NCB, rest = wave / NCB;
      const int chain = rest % chains, o = (rest / chains) * 2 * s;
      v16f tacc[NCB];
#pragma unroll
      for (int I = 0; I < NCB; ++I)
#pragma unroll
        for (int v = 0; v < 16; ++v) tacc[I][v] = 0.0f;
      if (act) {
        if (chain == 0) {
          // T = L21 X11, column block J: k >= 32 J (X11 unit lower)
          for (int k0 = 32 * J; k0 < s; k0 += 2) {
            const float bv = lunit_at(Ts, LDT, o + k0 + lh, o + 32 * J + l32);
#pragma unroll
            for (int I = 0; I < NCB; ++I)
              tacc[I] = __builtin_amdgcn_mfma_f32_32x32x2f32(Ts[(o + s + 32 * I + l32) * LDT + o + k0 + lh], bv,
                                                              tacc[I], 0, 0, 0);
          }
        } else {
          // T = U12 Y22, column block J: k < 32 J + 32 (Y22 upper)
          for (int k0 = 0; k0 < 32 * J + 32; k0 += 2) {
            const float bv = upper_at(Ts, LDT, o + s + k0 + lh, o + s + 32 * J + l32);
#pragma unroll
            for (int I = 0; I < NCB; ++I)
              tacc[I] = __builtin_amdgcn_mfma_f32_32x32x2f32(Ts[(o + 32 * I + l32) * LDT + o + s + k0 + lh], bv,
                                                              tacc[I], 0, 0, 0);
          }
        }
      }
      __syncthreads();  // every read of L21 / U12 is done
      if (act) {
#pragma unroll
        for (int I = 0; I < NCB; ++I) {
          v16f out;
#pragma unroll
          for (int v = 0; v < 16; ++v) out[v] = 0.0f;
          if (chain == 0) {
            // X21 = -X22 T, row tile I: k <= 32 I + 31 (X22 unit lower)
#pragma unroll
            for (int K = 0; K <= I; ++K)
#pragma unroll
              for (int v = 0; v < 16; ++v) {
                const int k = 32 * K + 8 * (v >> 2) + 4 * lh + (v & 3);
                out = __builtin_amdgcn_mfma_f32_32x32x2f32(lunit_at(Ts, LDT, o + s + 32 * I + l32, o + s + k),
                                                           tacc[K][v], out, 0, 0, 0);
              }
#pragma unroll
            for (int v = 0; v < 16; ++v)
              Ts[(o + s + 32 * I + 8 * (v >> 2) + 4 * lh + (v & 3)) * LDT + o + 32 * J + l32] = -out[v];
          } else {
            // Y12 = -Y11 T, row tile I: k >= 32 I (Y11 upper)
#pragma unroll
            for (int K = I; K < NCB; ++K)
#pragma unroll
              for (int v = 0; v < 16; ++v) {
                const int k = 32 * K + 8 * (v >> 2) + 4 * lh + (v & 3);
                out = __builtin_amdgcn_mfma_f32_32x32x2f32(upper_at(Ts, LDT, o + 32 * I + l32, o + k), tacc[K][v],
                                                           out, 0, 0, 0);
              }
#pragma unroll
            for (int v = 0; v < 16; ++v)
              Ts[(o + 32 * I + 8 * (v >> 2) + 4 * lh + (v & 3)) * LDT + o + s + 32 * J + l32] = -out[v];
          }
        }
      }
      __syncthreads();
    }
  });
  for (int e = tid; e < D * D; e += 256) base[(e / D) * Ninv + e % D] = Ts[(e / D) * LDT + e % D];
}

// bad[b] = any tile flag, or (zero_singular and sign[b] == 0)
__global__ void reduce_bad_kernel(const int* __restrict__ flags, int ntiles, const float* __restrict__ sign,
                                  int zero_singular, int* __restrict__ bad, int64_t batch) {
  const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (b >= batch) return;
  bool f = false;
  for (int k = lane; k < ntiles; k += 64) f = f || flags[b * ntiles + k] != 0;
  const bool any = __ballot(f) != 0ull;
  if (lane == 0) bad[b] = (any || (zero_singular && sign[b] == 0.0f)) ? 1 : 0;
}

// invT[b] = 0 for the flagged members (one workgroup per member; others exit at once).
__global__ __launch_bounds__(256) void zero_bad_kernel(const int* __restrict__ bad, float* __restrict__ invT,
                                                       int64_t nn) {
  const int64_t b = blockIdx.x;
  if (!bad[b]) return;
  float* o = invT + b * nn;
  for (int64_t e = threadIdx.x; e < nn; e += 256) o[e] = 0.0f;
}

// In-place inverses of the unit-lower L (strictly lower part) and, with upper, of the
// upper U~ (upper part incl. diagonal) packed in T (B, Ninv, Ninv); Tmp holds
// B * Ninv^2 / 4 floats.
int launch_tri_inverse(float* T, int Ninv, int64_t batch, float* Tmp, bool upper, hipStream_t s,
                       const int* active, int x3) {
  const int64_t NN = (int64_t)Ninv * Ninv;
  const int D = Ninv < 128 ? Ninv : 128;  // diagonal blocks inverted whole in LDS
  if (D == 32)
    hipLaunchKernelGGL((diag_inverse_kernel<32>), dim3(Ninv / 32, (unsigned)batch), dim3(256), 0, s, T, Ninv, active,
                       (int)upper);
  else if (D == 64)
    hipLaunchKernelGGL((diag_inverse_kernel<64>), dim3(Ninv / 64, (unsigned)batch), dim3(256), 0, s, T, Ninv, active,
                       (int)upper);
  else
    hipLaunchKernelGGL((diag_inverse_kernel<128>), dim3(Ninv / 128, (unsigned)batch), dim3(256), 0, s, T, Ninv,
                       active, (int)upper);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  for (int sz = D; sz < Ninv; sz *= 2) {
    const int pairs = Ninv / (2 * sz);
    const int64_t dstride = (int64_t)2 * sz * (Ninv + 1);  // next pair along the diagonal
    GemmDesc d = {};
    d.active = active;
    d.x3 = x3;
    d.M = d.N = d.K = sz;
    d.sA = d.sB = NN;
    d.sC = NN;
    d.lda = d.ldb = d.ldc = Ninv;
    // L: Tmp = L21 * X11
    d.A = T + (int64_t)sz * Ninv;
    d.B = T;
    d.maskB = MASK_LOWER_UNIT;
    d.C = Tmp;
    d.ldc = sz;
    d.sC = (int64_t)pairs * sz * sz;
    d.sA2 = d.sB2 = dstride;
    d.sC2 = (int64_t)sz * sz;
    d.alpha = 1.0f;
    d.beta = 0.0f;
    int st = launch_gemm(d, batch, pairs, s);
    if (st != FX_OK) return st;
    // X21 = -X22 * Tmp
    GemmDesc e = {};
    e.active = active;
    e.x3 = x3;
    e.M = e.N = e.K = sz;
    e.A = T + (int64_t)sz * Ninv + sz;
    e.maskA = MASK_LOWER_UNIT;
    e.lda = Ninv;
    e.sA = NN;
    e.sA2 = dstride;
    e.B = Tmp;
    e.ldb = sz;
    e.sB = (int64_t)pairs * sz * sz;
    e.sB2 = (int64_t)sz * sz;
    e.C = T + (int64_t)sz * Ninv;
    e.ldc = Ninv;
    e.sC = NN;
    e.sC2 = dstride;
    e.alpha = -1.0f;
    e.beta = 0.0f;
    st = launch_gemm(e, batch, pairs, s);
    if (st != FX_OK) return st;
    if (!upper) continue;
    // U: Tmp = U12 * Y22
    GemmDesc f = {};
    f.active = active;
    f.x3 = x3;
    f.M = f.N = f.K = sz;
    f.A = T + sz;
    f.lda = Ninv;
    f.sA = NN;
    f.sA2 = dstride;
    f.B = T + (int64_t)sz * Ninv + sz;
    f.maskB = MASK_UPPER;
    f.ldb = Ninv;
    f.sB = NN;
    f.sB2 = dstride;
    f.C = Tmp;
    f.ldc = sz;
    f.sC = (int64_t)pairs * sz * sz;
    f.sC2 = (int64_t)sz * sz;
    f.alpha = 1.0f;
    f.beta = 0.0f;
    st = launch_gemm(f, batch, pairs, s);
    if (st != FX_OK) return st;
    // Y12 = -Y11 * Tmp
    GemmDesc h = {};
    h.active = active;
    h.x3 = x3;
    h.M = h.N = h.K = sz;
    h.A = T;
    h.maskA = MASK_UPPER;
    h.lda = Ninv;
    h.sA = NN;
    h.sA2 = dstride;
    h.B = Tmp;
    h.ldb = sz;
    h.sB = (int64_t)pairs * sz * sz;
    h.sB2 = (int64_t)sz * sz;
    h.C = T + sz;
    h.ldc = Ninv;
    h.sC = NN;
    h.sC2 = dstride;
    h.alpha = -1.0f;
    h.beta = 0.0f;
    st = launch_gemm(h, batch, pairs, s);
    if (st != FX_OK) return st;
  }
  return FX_OK;
}

int launch_unit_lower_inverse(float* T, int Ninv, int64_t batch, float* Tmp, hipStream_t s,
                              const int* active, int x3) {
  return launch_tri_inverse(T, Ninv, batch, Tmp, false, s, active, x3);
}

int inv_padded(int N) {
  int p = 32;
  while (p < N) p *= 2;
  return p;
}

size_t lu_inverse_workspace(int64_t batch, int N, bool need_copy) {
  const int Ninv = inv_padded(N);
  const int nt = (N + 63) / 64;  // 64x64 tiles of the Z product
  size_t bytes = 0;
  auto add = [&](size_t x) { bytes += (x + 255) / 256 * 256; };
  if (need_copy) add((size_t)batch * Ninv * Ninv * 4);  // T
  add((size_t)batch * Ninv * Ninv / 4 * 4);              // Tmp (largest level: Ninv/2 x Ninv/2)
  add((size_t)batch * nt * nt * 4);                      // flags
  add((size_t)batch * 4);                                // bad
  return bytes;
}

int launch_lu_inverse(float* LU, const int* g0, int N, int n, int64_t batch, const float* sign,
                      int zero_singular, float* invT, bool in_place, void* ws, size_t ws_bytes,
                      hipStream_t s, const float* scale, int x3) {
  const int Ninv = inv_padded(N);
  const bool need_copy = !(in_place && Ninv == N);
  if (!ws || ws_bytes < lu_inverse_workspace(batch, N, need_copy)) return FX_ERR_WORKSPACE;
  char* p = (char*)ws;
  auto take = [&](size_t x) {
    char* q = p;
    p += (x + 255) / 256 * 256;
    return (void*)q;
  };
  float* T = need_copy ? (float*)take((size_t)batch * Ninv * Ninv * 4) : LU;
  float* Tmp = (float*)take((size_t)batch * Ninv * Ninv / 4 * 4);
  const int nt = (N + 63) / 64;  // 64x64 tiles of the Z product, one non-finite flag each
  int* flags = (int*)take((size_t)batch * nt * nt * 4);
  int* bad = (int*)take((size_t)batch * 4);
  const int64_t NN = (int64_t)Ninv * Ninv;
  if (need_copy) {
    hipLaunchKernelGGL(embed_kernel, dim3((unsigned)((NN + 255) / 256), (unsigned)batch), dim3(256), 0, s,
                       LU, N, T, Ninv);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  }
  int st0 = launch_tri_inverse(T, Ninv, batch, Tmp, true, s, nullptr, x3);
  if (st0 != FX_OK) return st0;
  // Z = U~^-1 L^-1 (the leading N x N block) stored straight as invT = P^T Z^T:
  // invT[g0[c]][i] = Z[i][c] for i < n and g0[c] < n, with the non-finite tile flags
  {
    GemmDesc d = {};
    d.x3 = x3;
    d.M = d.N = N;
    d.K = Ninv;
    d.A = T;
    d.maskA = MASK_UPPER;
    d.B = T;
    d.maskB = MASK_LOWER_UNIT;
    d.lda = d.ldb = Ninv;
    d.sA = d.sB = NN;
    d.alpha = 1.0f;
    d.beta = 0.0f;
    d.tout = invT;
    d.g0 = g0;
    d.nout = n;
    d.scale = scale;
    d.flags = flags;
    const int st = launch_gemm(d, batch, 1, s);
    if (st != FX_OK) return st;
  }
  // the flagged members (and, with zero_singular, those with a zero pivot) are cleared
  hipLaunchKernelGGL(reduce_bad_kernel, dim3((unsigned)((batch + 3) / 4)), dim3(256), 0, s, flags, nt * nt,
                     sign, zero_singular, bad, batch);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  hipLaunchKernelGGL(zero_bad_kernel, dim3((unsigned)batch), dim3(256), 0, s, bad, invT, (int64_t)n * n);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

}  // namespace fx
