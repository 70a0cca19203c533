// Device helpers shared by the fermix_amd HIP kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fx {

typedef float v4f __attribute__((ext_vector_type(4)));

template <int V>
struct ic {
  static constexpr int value = V;
};

// Compile-time loop: f(ic<B>{}), ..., f(ic<E-1>{}). Register arrays indexed by the loop
// variable then always resolve to fixed registers (a runtime index would make the
// compiler fall back to s_set_gpr_idx / v_movrel indexing).
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(ic<B>{});
    static_for<B + 1, E>(f);
  }
}

constexpr int WAVE = 64;

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// Order-preserving key of a pivot candidate: the bits of |x| with the top bit set (one OR:
// setting the sign bit of x gives the same word), 0 for "not a candidate". Non-negative
// floats order like their bit patterns, so an integer max over keys is an exact max over
// magnitudes, and the top bit lifts |x| = 0 above "no candidate".
__device__ __forceinline__ unsigned cand_key(float x, bool ok) {
  return ok ? (__float_as_uint(x) | 0x80000000u) : 0u;
}

template <int CTRL>
__device__ __forceinline__ unsigned dpp_u32(unsigned v) {
  return (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

// Maximum of v over the 64 lanes, returned wave-uniform: a 16-lane all-reduce with DPP
// (quad xor 1, quad xor 2, half-row mirror, row mirror), then row_bcast:15 into rows 1
// and 3 and row_bcast:31 into rows 2 and 3, after which lane 63 holds the maximum.
__device__ __forceinline__ unsigned wave_max_u32(unsigned v) {
  v = max(v, dpp_u32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = max(v, dpp_u32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = max(v, dpp_u32<0x141>(v));  // row_half_mirror
  v = max(v, dpp_u32<0x140>(v));  // row_mirror
  // rows outside the mask read 0, the identity of the max, so each step folds into one
  // v_max_u32_dpp
  v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false));
  v = max(v, (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false));
  return __builtin_amdgcn_readlane(v, 63);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum of v over the 64 lanes in a fixed order (deterministic, wave-uniform result).
__device__ __forceinline__ float wave_sum_f32(float v) {
  v += dpp_f32<0xB1>(v);
  v += dpp_f32<0x4E>(v);
  v += dpp_f32<0x141>(v);
  v += dpp_f32<0x140>(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ int readlane_i(int v, int l) { return __builtin_amdgcn_readlane(v, l); }

// Lowest lane whose predicate holds (wave-uniform); 64 if none.
__device__ __forceinline__ int first_lane(bool p) {
  unsigned long long m = __ballot(p);
  return m ? (int)__builtin_ctzll(m) : 64;
}

// Split-bf16x3 products (the fp32-accuracy reduced-precision MFMA mode): x = hi + mid + lo,
// each part the round-to-nearest bf16 of what the previous parts leave (the residues are
// exact in fp32), so the three parts hold x to about 24 significant bits. A product over
// a K = 16 slice takes the six bf16 MFMAs whose terms are at least 2^-16 of the leading
// one (hi*hi, hi*mid, mid*hi, hi*lo, mid*mid, lo*hi; smallest first), accumulated in fp32:
// about 2^-24 relative per term, against 2^-24 for the fp32 MFMA.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float v16f_t __attribute__((ext_vector_type(16)));

// The split of four values (one staged group of consecutive k, for operands that are
// split once when a K stage goes to LDS) and of eight (an operand split at its use).
// Two values per conversion (v_cvt_pk_bf16_f32 rounds a pair into one register; the
// parts come back to fp32 by a shift or a mask), the same bits as the scalar split.
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void split4_bf16x3(const float (&x)[4], bf16x4 (&p)[3]) {
  // residues of the values as given: no contraction with a product that formed them
#pragma clang fp contract(off)
#pragma unroll
  for (int u = 0; u < 4; u += 2) {
    const f32x2_t v = {x[u], x[u + 1]};
    const bf16x2_t h = __builtin_convertvector(v, bf16x2_t);
    const f32x2_t hf = __builtin_convertvector(h, f32x2_t);
    const f32x2_t r1 = {v[0] - hf[0], v[1] - hf[1]};
    const bf16x2_t m = __builtin_convertvector(r1, bf16x2_t);
    const f32x2_t mf = __builtin_convertvector(m, f32x2_t);
    const f32x2_t r2 = {r1[0] - mf[0], r1[1] - mf[1]};
    const bf16x2_t l = __builtin_convertvector(r2, bf16x2_t);
    p[0][u] = h[0];
    p[0][u + 1] = h[1];
    p[1][u] = m[0];
    p[1][u + 1] = m[1];
    p[2][u] = l[0];
    p[2][u + 1] = l[1];
  }
}
__device__ __forceinline__ void split_bf16x3(const float (&x)[8], bf16x8 (&p)[3]) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const float y[4] = {x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]};
    bf16x4 t[3];
    split4_bf16x3(y, t);
#pragma unroll
    for (int s = 0; s < 3; ++s)
#pragma unroll
      for (int u = 0; u < 4; ++u) p[s][4 * q + u] = t[s][u];
  }
}

// Split operand planes in LDS: a staged operand is three bf16 planes (hi, mid, lo) of
// rows of consecutive k (one row per i of A / j of B), so an MFMA operand -- eight k of
// one row -- is one 16-byte read per plane. Rows of 16 k (32 bytes) swap their two
// 16-byte halves on every other group of four rows, rows of 64 k (128 bytes) permute
// their eight 16-byte chunks by the row's low three bits: either way the 16-byte reads of
// eight consecutive rows at one k fall on distinct banks. Offsets in bf16 elements of
// the group of k .. k+3 (k % 4 == 0) or k .. k+7 (k % 8 == 0) of row r.
__device__ __forceinline__ int x3_off16(int r, int k) { return 16 * r + ((((k >> 3) ^ (r >> 2)) & 1) << 3) + (k & 7); }
__device__ __forceinline__ int x3_off64(int r, int k) { return 64 * r + ((((k >> 3) ^ r) & 7) << 3) + (k & 7); }

// Store one split group to the three planes (plane stride PS elements) / read one
// operand's eight k from them.
template <int PS>
__device__ __forceinline__ void x3_put(__bf16* planes, int off, const float (&x)[4]) {
  bf16x4 p[3];
  split4_bf16x3(x, p);
#pragma unroll
  for (int s = 0; s < 3; ++s) *reinterpret_cast<bf16x4*>(planes + s * PS + off) = p[s];
}
template <int PS>
__device__ __forceinline__ void x3_get(const __bf16* planes, int off, bf16x8 (&p)[3]) {
#pragma unroll
  for (int s = 0; s < 3; ++s) p[s] = *reinterpret_cast<const bf16x8*>(planes + s * PS + off);
}

// acc += A B over K = 16 with v_mfma_f32_32x32x16_bf16: lane l supplies the parts of
// A[l % 32][8 (l / 32) + u] and B[8 (l / 32) + u][l % 32], u < 8; D is the 32x32 fp32
// accumulator layout of the 32x32x2 fp32 MFMA.
__device__ __forceinline__ v16f_t mfma_bf16x3(const bf16x8 (&a)[3], const bf16x8 (&b)[3], v16f_t acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], acc, 0, 0, 0);
  return acc;
}

// The same six products into two accumulators: hh += hi*hi, sm += the five smaller terms.
// The bf16 MFMA adds each product to its accumulator truncated to about three bits
// below the accumulator's last place (measured on gfx950: sixteen products of 0.1 ulp
// each leave a 1.0 accumulator unchanged), so small terms added to a large accumulator
// are biased toward zero; in their own accumulator, about 2^-8 of hh, that loss is
// 2^-8 smaller, and the caller adds the accumulators (and any seed) in fp32.
__device__ __forceinline__ void mfma_bf16x3_2(const bf16x8 (&a)[3], const bf16x8 (&b)[3], v16f_t& hh, v16f_t& sm) {
  sm = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b[0], sm, 0, 0, 0);
  sm = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], sm, 0, 0, 0);
  sm = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[2], sm, 0, 0, 0);
  sm = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], sm, 0, 0, 0);
  sm = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], sm, 0, 0, 0);
  hh = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], hh, 0, 0, 0);
}

// fp32 MFMA 16x16x4: D = A(16x4) * B(4x16) + C. Lane l supplies A[l%16][l/16] and
// B[l/16][l%16]; D/C element (4*(l/16)+v, l%16) sits in item v of lane l.
__device__ __forceinline__ v4f mfma16(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Groups of G = 16 or 32 consecutive lanes of a wave (several small matrices per wave):
// Maximum over the G-lane group (G = 16: DPP within a row; G = 32: one more exchange).
template <int G>
__device__ __forceinline__ unsigned group_max_u32(unsigned v) {
  v = max(v, dpp_u32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = max(v, dpp_u32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = max(v, dpp_u32<0x141>(v));  // row_half_mirror
  v = max(v, dpp_u32<0x140>(v));  // row_mirror
  if constexpr (G == 32) v = max(v, (unsigned)__shfl_xor((int)v, 16));
  return v;
}

// Lowest lane of the group (relative index) whose predicate holds; gbase = first lane of
// the group in the wave.
template <int G>
__device__ __forceinline__ int group_first(bool p, int gbase) {
  const unsigned long long m = __ballot(p);
  const unsigned bits = (unsigned)(m >> gbase) & (G == 32 ? 0xFFFFFFFFu : 0xFFFFu);
  return bits ? (int)__builtin_ctz(bits) : G;
}

// Compiler-level ordering point for LDS traffic exchanged between the lanes of one
// wave (the hardware executes one wave's LDS instructions in order).
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Guarded reciprocal: 1/0 -> 0 (a zero pivot contributes nothing to the multipliers).
// v_rcp_f32 (1 ulp) -- the multipliers it scales are within 2 ulp of a / d.
__device__ __forceinline__ float safe_rcp(float d) {
  return d != 0.0f ? __builtin_amdgcn_rcpf(d) : 0.0f;
}

// x unchanged, through an empty register constraint the optimiser cannot look into. Used
// on values copied out of one of several per-row register arrays under a per-row
// predicate: without it the copies merge into one copy from a selected address, which
// indexes the arrays dynamically and moves them to scratch memory.
__device__ __forceinline__ float opaque(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Materialise a running counter where it stands: otherwise the increments of a fully
// unrolled loop can sink to the counter's single use, keeping every operand live.
__device__ __forceinline__ void pin(int& x) { asm volatile("" : "+v"(x)); }

// Pivots of one matrix collected across a wave: pivot g lives in slot g / 64 of lane
// g % 64, so the logs and signs are formed once at the end, off the elimination's
// dependency chain.
template <int NS>
struct PivotLog {
  float v[NS];
  __device__ __forceinline__ void init() {
#pragma unroll
    for (int i = 0; i < NS; ++i) v[i] = 1.0f;
  }
  __device__ __forceinline__ void put(int g, float d, int lane) {
    const int sl = g >> 6;
    const bool mine = (g & 63) == lane;
#pragma unroll
    for (int i = 0; i < NS; ++i) v[i] = (mine && sl == i) ? d : v[i];
  }
  // (sign, logabs) of the product of the pivots times (-1)^nswap; (0, -inf) if any is 0.
  __device__ __forceinline__ void finish(int nswap, float& sign, float& logabs) const {
    float lg = 0.0f;
    bool z = false, ng = false;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      z = z || (v[i] == 0.0f);
      ng = ng != (v[i] < 0.0f);
      lg += (v[i] != 0.0f) ? logf(fabsf(v[i])) : 0.0f;
    }
    lg = wave_sum_f32(lg);
    const unsigned long long zm = __ballot(z);
    const int negs = __popcll(__ballot(ng)) + nswap;
    sign = zm ? 0.0f : ((negs & 1) ? -1.0f : 1.0f);
    logabs = zm ? -INFINITY : lg;
  }
};

// Copy the row-major n x n matrix g into an N x N LDS tile (row stride LDA) with NT
// threads, writing pad(r, c) outside the n x n block. Every global load of a chunk is
// issued before its LDS stores, so a thread keeps several loads in flight; with n == N
// (n a multiple of 16) the loads are 16-byte vectors.
template <int N, int LDA, int NT, class Pad>
__device__ __forceinline__ void load_tile(float* As, const float* __restrict__ g, int n, int tid,
                                          Pad pad) {
  if (n == N) {
    constexpr int NV = N * N / 4;
    constexpr int PER = (NV + NT - 1) / NT;
    const float4* g4 = reinterpret_cast<const float4*>(g);
    float4 v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = tid + NT * i;
      if (NV % NT == 0 || e < NV) v[i] = g4[e];
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = tid + NT * i;
      if (NV % NT == 0 || e < NV) {
        const int r = (4 * e) / N, c = (4 * e) % N;
        float* d = As + r * LDA + c;
        d[0] = v[i].x;
        d[1] = v[i].y;
        d[2] = v[i].z;
        d[3] = v[i].w;
      }
    }
  } else {
    constexpr int CH = 8;
    for (int base = 0; base < N * N; base += NT * CH) {
      float v[CH];
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int e = base + tid + NT * u;
        const int r = e / N, c = e % N;
        v[u] = (e < N * N && r < n && c < n) ? g[r * n + c] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int e = base + tid + NT * u;
        const int r = e / N, c = e % N;
        if (e < N * N) As[r * LDA + c] = (r < n && c < n) ? v[u] : pad(r, c);
      }
    }
  }
}

// ---- 64-bit workgroup argmax (the float64 and complex kernels)

// Order-preserving key of a pivot candidate: |x| bits plus one (0 = no candidate).
__device__ __forceinline__ unsigned long long key64(double x) {
  return (unsigned long long)__double_as_longlong(fabs(x)) + 1ull;
}

__device__ __forceinline__ void take_better(unsigned long long& k, int& r, unsigned long long k2, int r2) {
  if (k2 > k || (k2 == k && r2 < r)) {
    k = k2;
    r = r2;
  }
}

// Workgroup argmax of (key, row), larger key first, then lower row; every thread returns
// the winning row (-1 if no thread had a candidate). redk / redr: NT / 64 slots; the
// caller alternates two slot sets between consecutive calls, so no extra barrier guards
// their reuse.
template <int NT>
__device__ __forceinline__ int block_argmax(unsigned long long k, int r, unsigned long long* redk, int* redr) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long k2 = __shfl_xor(k, off);
    const int r2 = __shfl_xor(r, off);
    take_better(k, r, k2, r2);
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    redk[w] = k;
    redr[w] = r;
  }
  __syncthreads();
  k = redk[0];
  r = redr[0];
#pragma unroll
  for (int i = 1; i < NT / 64; ++i) take_better(k, r, redk[i], redr[i]);
  return k ? r : -1;
}

}  // namespace fx
