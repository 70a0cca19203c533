// Batched fp32 GEMM on MFMA (v_mfma_f32_32x32x2f32) for the sub-block products of the
// large-n paths: C = alpha * op(A) op(B) + beta * C over a batch of matrices (and an
// optional second batch dimension, e.g. the block pairs of one recursion level).
//
// Reference role replaced: the batched sub-block GEMM `_bgemm` (ChenAo-Phys/fermix
// src/fermix/_inverse.py:230-426) and the trailing GEMMs of the LU / Parlett-Reid
// (src/fermix/_lu.py:334-393, src/fermix/_pf.py:287-382).
//
// Design (gfx950): a workgroup of 4 waves computes a BM x BN tile (64 x 64, or 128 x 128
// in gemm128_kernel for the products with M, N >= 1024); each wave owns a (BM/2) x (BN/2)
// quarter as 32x32 MFMA accumulators. K advances in BK = 16 stages
// staged through LDS K-major (so every MFMA operand read is 32 consecutive floats),
// double-buffered, with the next stage's global loads in flight during the current
// stage's MFMAs. The split-bf16x3 mode (X3) runs each K = 16 stage as six bf16 MFMAs
// (v_mfma_f32_32x32x16_bf16) per accumulator.
//
// Options:
//  * operand masks: op(A)(i, k) / op(B)(k, j) read as zero outside a triangle (lower
//    with unit diagonal, or upper), compared on global indices, so packed LU storage
//    can be used directly as L or U; the K range of each tile is trimmed to the
//    triangle at tile granularity;
//  * lower_only: only tiles with tile_row >= tile_col are computed, and each element
//    is also stored mirrored, C[j][i] = mirror * C[i][j] (mirror = -1 gives an exactly
//    skew result with a zero diagonal);
//  * tout (64 x 64 tiles): the product is stored transposed and row-permuted,
//    tout[g0[j]][i] = scale[b] alpha C[i][j], through an LDS transpose in the epilogue,
//    with a non-finite flag per tile (the slogdet backward's A^-T = P^T Z^T);
//  * bscale: op(B) row k is +-bscale[k / 2] B[k ^ 1] (pair swap and per-row scale,
//    applied between the stage load and the LDS store), a compile-time variant.
// The mask combination is a template parameter for the combinations the library uses,
// so a masked element costs one compare and a plain stage carries no mask code.
#include <type_traits>

#include "common.h"
#include "fermix_internal.h"

namespace fx {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int GBK = 16;

// Word 3 of a raw buffer descriptor on gfx9 (untyped 32-bit data, range-checked offsets).
constexpr int BUF_RSRC_WORD3 = 0x00020000;
typedef unsigned v4u __attribute__((ext_vector_type(4)));

// Element (r, c) of op(X) in the mask's global coordinates.
__device__ __forceinline__ float mask_val(float v, int mask, int r, int c) {
  if (mask == MASK_LOWER_UNIT) return r > c ? v : (r == c ? 1.0f : 0.0f);
  if (mask == MASK_UPPER) return r <= c ? v : 0.0f;
  if (mask == MASK_UPPER_UNIT) return r < c ? v : (r == c ? 1.0f : 0.0f);
  return v;
}
__device__ __forceinline__ bool mask_lower(int m) { return m == MASK_LOWER_UNIT; }
__device__ __forceinline__ bool mask_upper(int m) { return m == MASK_UPPER || m == MASK_UPPER_UNIT; }

// Tile loads: VEC uses 16-byte global loads along the operand's contiguous dimension
// (requires that dimension, the leading dimensions, batch strides and base pointers to be
// multiples of 4 floats), otherwise one float per load. Masks are applied in registers.
template <int BM, int BN, bool VEC, int MK, bool BS = false, bool X3 = false>
__global__ __launch_bounds__(256) void gemm_kernel(GemmDesc d) {
  // operand masks: MK = 4 maskA + maskB fixed at compile time (the combinations this
  // library uses), so each mask test folds to one compare per element; MK < 0 reads them
  // from the descriptor
  const int maskA = MK >= 0 ? (MK >> 2) : d.maskA;
  const int maskB = MK >= 0 ? (MK & 3) : d.maskB;
  constexpr int LDSA = BM + 4, LDSB = BN + 4;
  constexpr int WM = BM / 2, WN = BN / 2;   // per-wave quarter
  constexpr int TM = WM / 32, TN = WN / 32;  // 32x32 tiles per wave
  // one LDS block: the two operand stages, reused by the transposed-output epilogue
  constexpr int LDS_AB = 2 * GBK * LDSA + 2 * GBK * LDSB;
  static_assert(LDS_AB >= BN * (BM + 1), "transposed tile fits the operand stages");
  __shared__ __align__(16) float smem[LDS_AB];
  float(*As)[GBK * LDSA] = reinterpret_cast<float(*)[GBK * LDSA]>(smem);
  float(*Bs)[GBK * LDSB] = reinterpret_cast<float(*)[GBK * LDSB]>(smem + 2 * GBK * LDSA);

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  int64_t bat = blockIdx.y;
  const int64_t bat2 = blockIdx.z;
  int tx = blockIdx.x;
  if (d.xcd8) {
    // Workgroups are handed to the 8 XCDs round-robin by linear id, each XCD with its own
    // L2: renumber so that all tiles of one matrix run on one XCD and every XCD gets the
    // same mix of (triangle-trimmed, unequal) tiles.
    const int64_t lin = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
    const int64_t slot = lin >> 3;
    tx = (int)(slot % gridDim.x);
    bat = (slot / gridDim.x) * 8 + (lin & 7);
  }
  // members switched off by the caller's mask (uniform per workgroup, before any barrier)
  if (d.active && !d.active[bat]) return;
  int ti, tj;
  const int ntn = (d.N + BN - 1) / BN;
  if (d.lower_only) {
    // blockIdx.x enumerates the lower triangle of tiles row-major
    const int t = tx;
    int I = (int)((sqrtf(8.0f * t + 1.0f) - 1.0f) * 0.5f);
    while ((I + 1) * (I + 2) / 2 <= t) ++I;
    while (I * (I + 1) / 2 > t) --I;
    ti = I;
    tj = t - I * (I + 1) / 2;
  } else {
    ti = tx / ntn;
    tj = tx % ntn;
  }
  const int i0 = ti * BM, j0 = tj * BN;
  const float* A = d.A + bat * d.sA + bat2 * d.sA2;
  const float* B = d.B + bat * d.sB + bat2 * d.sB2;
  float* C = d.C + bat * d.sC + bat2 * d.sC2;

  // K range of this tile from the operand triangles
  int klo = 0, khi = d.K;
  // op(A)(i, k): lower -> k <= i + offAr - offAc, upper -> k >= i + offAr - offAc;
  // op(B)(k, j): lower -> k >= j + offBc - offBr, upper -> k <= j + offBc - offBr
  if (mask_upper(maskA)) klo = max(klo, i0 + d.offAr - d.offAc);
  if (mask_lower(maskA)) khi = min(khi, i0 + BM + d.offAr - d.offAc);
  if (mask_lower(maskB)) klo = max(klo, j0 + d.offBc - d.offBr);
  if (mask_upper(maskB)) khi = min(khi, j0 + BN + d.offBc - d.offBr);
  klo = max(0, (klo / GBK) * GBK);

  // A stage is plain when no element of it needs a bound or mask fix (a uniform test):
  // an interior tile, a full K stage, and both operands' stage blocks strictly inside
  // their triangles. Plain stages skip the per-element fixes, which otherwise dominate
  // the instruction count of a stage.
  const bool interior = i0 + BM <= d.M && j0 + BN <= d.N;
  auto plain_stage = [&](int k0) {
    if (!VEC || !interior || k0 + GBK > d.K) return false;
    bool ok = true;
    if (maskA == MASK_LOWER_UNIT) ok = ok && i0 + d.offAr > k0 + GBK - 1 + d.offAc;
    if (maskA == MASK_UPPER) ok = ok && i0 + BM - 1 + d.offAr <= k0 + d.offAc;
    if (maskA == MASK_UPPER_UNIT) ok = ok && i0 + BM - 1 + d.offAr < k0 + d.offAc;
    if (maskB == MASK_LOWER_UNIT) ok = ok && k0 + d.offBr > j0 + BN - 1 + d.offBc;
    if (maskB == MASK_UPPER) ok = ok && k0 + GBK - 1 + d.offBr <= j0 + d.offBc;
    if (maskB == MASK_UPPER_UNIT) ok = ok && k0 + GBK - 1 + d.offBr < j0 + d.offBc;
    return ok;
  };

  const int wm = (wave >> 1) * WM, wn = (wave & 1) * WN;
  const int l32 = lane & 31, lh = lane >> 5;

  // global -> register staging of one K stage: A tile BM x GBK, B tile GBK x BN. The
  // loads take clamped (always valid) addresses and nothing reads their data until
  // store_stage, which runs after the MFMAs of the current stage; out-of-range zeros and
  // the triangle masks are applied there.
  constexpr int AV = BM * GBK / 1024, BV = BN * GBK / 1024;  // float4 per thread
  constexpr int AE = BM * GBK / 256, BE = BN * GBK / 256;      // floats per thread
  float4 va[VEC ? AV : 1], vb[VEC ? BV : 1];
  float bsv[VEC ? BV : 1];  // B row scales (bscale), loaded with the stage
  float ra[VEC ? 1 : AE], rb[VEC ? 1 : BE];
  // element coordinates of staging slot e (global row / k / column)
  auto a_coord = [&](int idx, int k0, int& gi, int& gk) {
    if (VEC) {
      if (!d.transA) { gi = i0 + idx / (GBK / 4); gk = k0 + 4 * (idx % (GBK / 4)); }
      else { gk = k0 + idx / (BM / 4); gi = i0 + 4 * (idx % (BM / 4)); }
    } else {
      if (!d.transA) { gi = i0 + idx / GBK; gk = k0 + idx % GBK; }   // row-major A: k fastest
      else { gk = k0 + idx / BM; gi = i0 + idx % BM; }               // A^T stored: i fastest
    }
  };
  auto b_coord = [&](int idx, int k0, int& gk, int& gj) {
    if (VEC) {
      if (!d.transB) { gk = k0 + idx / (BN / 4); gj = j0 + 4 * (idx % (BN / 4)); }
      else { gj = j0 + idx / (GBK / 4); gk = k0 + 4 * (idx % (GBK / 4)); }
    } else {
      if (!d.transB) { gk = k0 + idx / BN; gj = j0 + idx % BN; }     // row-major B: j fastest
      else { gj = j0 + idx / GBK; gk = k0 + idx % GBK; }             // B^T stored: k fastest
    }
  };
  // the last valid vector / element along each dimension (K and the contiguous
  // dimension are multiples of 4 on the VEC path)
  const int lastA_i = d.M - (VEC && d.transA ? 4 : 1), lastA_k = d.K - (VEC && !d.transA ? 4 : 1);
  const int lastB_j = d.N - (VEC && !d.transB ? 4 : 1), lastB_k = d.K - (VEC && d.transB ? 4 : 1);
  auto load_stage = [&](int k0) {
    if constexpr (VEC) {
#pragma unroll
      for (int e = 0; e < AV; ++e) {
        int gi, gk;
        a_coord(tid + 256 * e, k0, gi, gk);
        gi = min(gi, lastA_i);
        gk = min(gk, lastA_k);
        va[e] = *reinterpret_cast<const float4*>(d.transA ? A + (int64_t)gk * d.lda + gi
                                                          : A + (int64_t)gi * d.lda + gk);
      }
#pragma unroll
      for (int e = 0; e < BV; ++e) {
        int gk, gj;
        b_coord(tid + 256 * e, k0, gk, gj);
        gj = min(gj, lastB_j);
        gk = min(gk, lastB_k);
        if (BS) {  // row pair swap (K is even) and the row's scale
          bsv[e] = d.bscale[bat * (d.K / 2) + (gk >> 1)];
          gk ^= 1;
        }
        vb[e] = *reinterpret_cast<const float4*>(d.transB ? B + (int64_t)gj * d.ldb + gk
                                                          : B + (int64_t)gk * d.ldb + gj);
      }
    } else {
#pragma unroll
      for (int e = 0; e < AE; ++e) {
        int gi, gk;
        a_coord(tid + 256 * e, k0, gi, gk);
        gi = min(gi, lastA_i);
        gk = min(gk, lastA_k);
        ra[e] = d.transA ? A[(int64_t)gk * d.lda + gi] : A[(int64_t)gi * d.lda + gk];
      }
#pragma unroll
      for (int e = 0; e < BE; ++e) {
        int gk, gj;
        b_coord(tid + 256 * e, k0, gk, gj);
        gj = min(gj, lastB_j);
        gk = min(gk, lastB_k);
        rb[e] = d.transB ? B[(int64_t)gj * d.ldb + gk] : B[(int64_t)gk * d.ldb + gj];
      }
    }
  };
  // op(A)(gi, gk) after masking (zero outside the matrix)
  auto fixA = [&](float v, int gi, int gk) {
    if (gi >= d.M || gk >= d.K) return 0.0f;
    return maskA ? mask_val(v, maskA, gi + d.offAr, gk + d.offAc) : v;
  };
  auto fixB = [&](float v, int gk, int gj) {
    if (gj >= d.N || gk >= d.K) return 0.0f;
    return maskB ? mask_val(v, maskB, gk + d.offBr, gj + d.offBc) : v;
  };
  // registers -> LDS, K-major (As[k][i], Bs[k][j]) so each MFMA operand read is 32
  // consecutive floats
  auto store_stage = [&](int buf, int k0, bool plain) {
    if constexpr (VEC) {
#pragma unroll
      for (int e = 0; e < AV; ++e) {
        const int idx = tid + 256 * e;
        int gi, gk;
        a_coord(idx, k0, gi, gk);
        const int dr = d.transA, dc = 1 - d.transA;  // step of the vector's components
        float4 v = va[e];
        if (!plain) {
          v.x = fixA(v.x, gi, gk);
          v.y = fixA(v.y, gi + dr, gk + dc);
          v.z = fixA(v.z, gi + 2 * dr, gk + 2 * dc);
          v.w = fixA(v.w, gi + 3 * dr, gk + 3 * dc);
        }
        const int i = gi - i0, k = gk - k0;
        if (!d.transA) {
          As[buf][k * LDSA + i] = v.x;
          As[buf][(k + 1) * LDSA + i] = v.y;
          As[buf][(k + 2) * LDSA + i] = v.z;
          As[buf][(k + 3) * LDSA + i] = v.w;
        } else {
          *reinterpret_cast<float4*>(&As[buf][k * LDSA + i]) = v;
        }
      }
#pragma unroll
      for (int e = 0; e < BV; ++e) {
        const int idx = tid + 256 * e;
        int gk, gj;
        b_coord(idx, k0, gk, gj);
        const int dk = d.transB, dj = 1 - d.transB;
        float4 v = vb[e];
        if (BS) {  // row gk of op(B) = s_gk B[gk ^ 1] (one row per vector: transB is 0)
          const float sg = (gk & 1) ? -bsv[e] : bsv[e];
          v.x *= sg;
          v.y *= sg;
          v.z *= sg;
          v.w *= sg;
        }
        if (!plain) {
          v.x = fixB(v.x, gk, gj);
          v.y = fixB(v.y, gk + dk, gj + dj);
          v.z = fixB(v.z, gk + 2 * dk, gj + 2 * dj);
          v.w = fixB(v.w, gk + 3 * dk, gj + 3 * dj);
        }
        const int k = gk - k0, j = gj - j0;
        if (!d.transB) {
          *reinterpret_cast<float4*>(&Bs[buf][k * LDSB + j]) = v;
        } else {
          Bs[buf][k * LDSB + j] = v.x;
          Bs[buf][(k + 1) * LDSB + j] = v.y;
          Bs[buf][(k + 2) * LDSB + j] = v.z;
          Bs[buf][(k + 3) * LDSB + j] = v.w;
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < AE; ++e) {
        int gi, gk;
        a_coord(tid + 256 * e, k0, gi, gk);
        As[buf][(gk - k0) * LDSA + (gi - i0)] = fixA(ra[e], gi, gk);
      }
#pragma unroll
      for (int e = 0; e < BE; ++e) {
        int gk, gj;
        b_coord(tid + 256 * e, k0, gk, gj);
        Bs[buf][(gk - k0) * LDSB + (gj - j0)] = fixB(rb[e], gk, gj);
      }
    }
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;
  if (klo < khi) load_stage(klo);

  int buf = 0;
  if (klo < khi) {
    store_stage(0, klo, plain_stage(klo));
    __syncthreads();
    for (int k0 = klo; k0 < khi; k0 += GBK) {
      const bool more = k0 + GBK < khi;
      if (more) load_stage(k0 + GBK);
      if constexpr (X3) {
        // the stage's K = 16 in one bf16x3 product per accumulator: lane operands are the
        // eight k = 8 lh + u of its row (A) / column (B), split in registers
        bf16x8 ap[TM][3], bp[TN][3];
#pragma unroll
        for (int a = 0; a < TM; ++a) {
          float f[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) f[u] = As[buf][(8 * lh + u) * LDSA + wm + 32 * a + l32];
          split_bf16x3(f, ap[a]);
        }
#pragma unroll
        for (int b = 0; b < TN; ++b) {
          float f[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) f[u] = Bs[buf][(8 * lh + u) * LDSB + wn + 32 * b + l32];
          split_bf16x3(f, bp[b]);
        }
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
          for (int b = 0; b < TN; ++b) acc[a][b] = mfma_bf16x3(ap[a], bp[b], acc[a][b]);
      } else {
#pragma unroll
        for (int kp = 0; kp < GBK / 2; ++kp) {
          float av[TM], bv[TN];
#pragma unroll
          for (int a = 0; a < TM; ++a) av[a] = As[buf][(2 * kp + lh) * LDSA + wm + 32 * a + l32];
#pragma unroll
          for (int b = 0; b < TN; ++b) bv[b] = Bs[buf][(2 * kp + lh) * LDSB + wn + 32 * b + l32];
#pragma unroll
          for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b)
              acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[a], bv[b], acc[a][b], 0, 0, 0);
        }
      }
      if (more) {
        store_stage(buf ^ 1, k0 + GBK, plain_stage(k0 + GBK));
        __syncthreads();
        buf ^= 1;
      }
    }
  }

  if (d.tout) {
    // transposed, row-permuted output: the tile goes through LDS transposed (Ts[c][r])
    // so that each tile column j is stored as one contiguous run of row g0[j] of tout
    constexpr int LDT = BM + 1;
    float* Ts = smem;
    __syncthreads();  // every wave is done with the last stage's operands
    bool nf = false;
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int b = 0; b < TN; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int r = wm + 32 * a + 8 * (v >> 2) + 4 * lh + (v & 3), c = wn + 32 * b + l32;
          Ts[c * LDT + r] = acc[a][b][v];
          nf = nf || (i0 + r < d.M && j0 + c < d.N && !isfinite(acc[a][b][v]));
        }
    const int any = __syncthreads_or(nf ? 1 : 0);
    if (tid == 0) d.flags[bat * (int64_t)gridDim.x + tx] = any;
    // lane l holds the target row of tile column l (BN == 64: one per lane), so each store
    // pass takes its row with a lane read instead of a load; column cc = wave + 4 u
    static_assert(BN == 64 && BM == 64, "one tile column per lane");
    const int* gb = d.g0 + bat * d.N;
    const int rl = j0 + lane < d.N ? gb[j0 + lane] : d.nout;
    const float sc = d.scale ? d.alpha * d.scale[bat] : d.alpha;
    float* ob = d.tout + bat * (int64_t)d.nout * d.nout;
    const int i = i0 + lane;
#pragma unroll
    for (int u = 0; u < BN / 4; ++u) {
      const int cc = wave + 4 * u;
      const int r = __builtin_amdgcn_readlane(rl, cc);
      if (i < d.nout && r < d.nout) ob[(int64_t)r * d.nout + i] = sc * Ts[cc * LDT + lane];
    }
    return;
  }

  // epilogue: C = alpha * acc + beta * C (and the mirror), one 32x32 accumulator at a
  // time with its 16 reads of C issued before any store (C is read and written through
  // the same pointer, so reads placed after a store could not be hoisted)
  const bool diag_tile = d.lower_only && ti == tj;
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) {
      const int c = j0 + wn + 32 * b + l32;
      float cv[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = i0 + wm + 32 * a + 8 * (v >> 2) + 4 * lh + (v & 3);
        cv[v] = (d.beta != 0.0f && r < d.M && c < d.N) ? C[(int64_t)r * d.ldc + c] : 0.0f;
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = i0 + wm + 32 * a + 8 * (v >> 2) + 4 * lh + (v & 3);
        if (r >= d.M || c >= d.N) continue;
        if (diag_tile && r < c) continue;
        float val = d.alpha * acc[a][b][v];
        if (d.beta != 0.0f) val = fmaf(d.beta, cv[v], val);
        if (d.lower_only && r == c && d.mirror < 0.0f) val = 0.0f;
        C[(int64_t)r * d.ldc + c] = val;
        if (d.lower_only && r != c) C[(int64_t)c * d.ldc + r] = d.mirror * val;
      }
    }
}

// 128 x 128 tiles for the large products (16-byte aligned operands, op(B) = B, op(A) = A
// or A^T by TA): each wave owns a 64 x 64 quarter as 2 x 2 32x32 accumulators, so a
// K = 16 stage is 32 MFMAs per wave against four 16-byte loads per thread. The staging
// code carries no per-element work: offsets are formed once per tile, loads use clamped
// (always valid) addresses, and the raw values go to LDS. Only a stage that touches a
// matrix edge or an operand triangle's diagonal (tested uniformly) is then fixed in LDS
// -- zeros outside the matrix, the triangle masks -- between two barriers.
// Launch bound of 4 waves per SIMD: the compiler then fits the kernel in 116 VGPRs
// (accumulators included) without scratch, against 168 + 64 left to itself.
// The split-bf16x3 variant (X3) splits each staged element once, into three bf16 planes
// (48 KiB of LDS for two stages), and reads each MFMA operand as one 16-byte read per
// plane: measured 17-30 % faster than the fp32 MFMA on the n = 2048 slogpf backward's
// products. (The 64 x 64 kernel keeps the split at the point of use: with one
// accumulator per wave its products are bound by latency, and the larger staged LDS
// footprint made them slower.)
template <bool TA, int MK, bool BS = false, bool X3 = false>
__global__ __launch_bounds__(256, X3 ? 2 : 4) void gemm128_kernel(GemmDesc d) {
  const int maskA = MK >= 0 ? (MK >> 2) : d.maskA;  // compile-time masks as in gemm_kernel
  const int maskB = MK >= 0 ? (MK & 3) : d.maskB;
  constexpr int BM = 128, BN = 128, LDA_ = BM + 4, LDB_ = BN + 4;
  // fp32 stages K-major, or (X3) three split bf16 planes per operand and stage
  constexpr int XPA = BM * GBK, XPB = BN * GBK;  // bf16 per plane
  constexpr int SMEM = X3 ? 2 * 3 * (XPA + XPB) * 2 : 2 * GBK * (LDA_ + LDB_) * 4;
  __shared__ __align__(16) char smem[SMEM];
  float(*As)[GBK * LDA_] = reinterpret_cast<float(*)[GBK * LDA_]>(smem);
  float(*Bs)[GBK * LDB_] = reinterpret_cast<float(*)[GBK * LDB_]>(smem + 2 * GBK * LDA_ * 4);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  int64_t bat = blockIdx.y;
  const int64_t bat2 = blockIdx.z;
  int tx = blockIdx.x;
  if (d.xcd8) {
    const int64_t lin = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
    const int64_t slot = lin >> 3;
    tx = (int)(slot % gridDim.x);
    bat = (slot / gridDim.x) * 8 + (lin & 7);
  }
  if (d.active && !d.active[bat]) return;
  int ti, tj;
  if (d.lower_only) {
    const int t = tx;
    int I = (int)((sqrtf(8.0f * t + 1.0f) - 1.0f) * 0.5f);
    while ((I + 1) * (I + 2) / 2 <= t) ++I;
    while (I * (I + 1) / 2 > t) --I;
    ti = I;
    tj = t - I * (I + 1) / 2;
  } else {
    const int ntn = (d.N + BN - 1) / BN;
    ti = tx / ntn;
    tj = tx % ntn;
  }
  const int i0 = ti * BM, j0 = tj * BN;
  const float* A = d.A + bat * d.sA + bat2 * d.sA2;
  const float* B = d.B + bat * d.sB + bat2 * d.sB2;
  float* C = d.C + bat * d.sC + bat2 * d.sC2;

  int klo = 0, khi = d.K;
  if (mask_upper(maskA)) klo = max(klo, i0 + d.offAr - d.offAc);
  if (mask_lower(maskA)) khi = min(khi, i0 + BM + d.offAr - d.offAc);
  if (mask_lower(maskB)) klo = max(klo, j0 + d.offBc - d.offBr);
  if (mask_upper(maskB)) khi = min(khi, j0 + BN + d.offBc - d.offBr);
  klo = max(0, (klo / GBK) * GBK);

  const bool interior = i0 + BM <= d.M && j0 + BN <= d.N;
  // a stage is plain for an operand when none of its elements meets the operand's
  // triangle diagonal (the K range is trimmed to the triangle per tile), and inside the
  // matrices when no element is past M, N or K
  auto plain_a = [&](int k0) {
    if (maskA == MASK_LOWER_UNIT) return i0 + d.offAr > k0 + GBK - 1 + d.offAc;
    if (maskA == MASK_UPPER) return i0 + BM - 1 + d.offAr <= k0 + d.offAc;
    if (maskA == MASK_UPPER_UNIT) return i0 + BM - 1 + d.offAr < k0 + d.offAc;
    return true;
  };
  auto plain_b = [&](int k0) {
    if (maskB == MASK_LOWER_UNIT) return k0 + d.offBr > j0 + BN - 1 + d.offBc;
    if (maskB == MASK_UPPER) return k0 + GBK - 1 + d.offBr <= j0 + d.offBc;
    if (maskB == MASK_UPPER_UNIT) return k0 + GBK - 1 + d.offBr < j0 + d.offBc;
    return true;
  };
  auto inside = [&](int k0) { return interior && k0 + GBK <= d.K; };
  auto plain_stage = [&](int k0) { return inside(k0) && plain_a(k0) && plain_b(k0); };

  // this thread's staging slots (two float4 of A, two of B per stage), 32-bit offsets
  // within a matrix (N * N < 2^31); rows / columns past the matrix clamped once here
  // A (not TA): rows ra + 64 e, columns k0 + ka .. +3;  A^T (TA): k rows k0 + ka + 8 e,
  // columns ia .. +3;  B: k rows k0 + kb + 8 e, columns jb .. +3
  const int ra = tid >> 2, ka = TA ? (tid >> 5) : 4 * (tid & 3);
  const int ia = min(i0 + 4 * (tid & 31), d.M - 4);
  const int kb = tid >> 5, jb = min(j0 + 4 * (tid & 31), d.N - 4);
  int aoff[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) aoff[e] = TA ? ia : min(i0 + ra + 64 * e, d.M - 1) * d.lda;
  float va[2][4], vb[2][4];  // plain floats: arrays of float4 are not kept in registers
  float bsv[2];              // B row scales (bscale), signed, loaded with the stage
  auto load_stage = [&](int k0) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float4 x = !TA ? *reinterpret_cast<const float4*>(A + aoff[e] + min(k0 + ka, d.K - 4))
                           : *reinterpret_cast<const float4*>(A + min(k0 + ka + 8 * e, d.K - 1) * d.lda + aoff[e]);
      const int kr = min(k0 + kb + 8 * e, d.K - 1);
      if (BS) bsv[e] = d.bscale[bat * (d.K / 2) + (kr >> 1)];
      const float4 y = *reinterpret_cast<const float4*>(B + (BS ? kr ^ 1 : kr) * d.ldb + jb);
      va[e][0] = x.x;
      va[e][1] = x.y;
      va[e][2] = x.z;
      va[e][3] = x.w;
      vb[e][0] = y.x;
      vb[e][1] = y.y;
      vb[e][2] = y.z;
      vb[e][3] = y.w;
    }
  };
  // registers -> LDS, K-major (As[k][i], Bs[k][j]); clamped columns land in the slots of
  // the columns past the matrix, which the fix pass zeroes
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      if (!TA) {
        float* p = &As[buf][ka * LDA_ + ra + 64 * e];
        p[0] = va[e][0];
        p[LDA_] = va[e][1];
        p[2 * LDA_] = va[e][2];
        p[3 * LDA_] = va[e][3];
      } else {
        *reinterpret_cast<float4*>(&As[buf][(ka + 8 * e) * LDA_ + 4 * (tid & 31)]) =
            make_float4(va[e][0], va[e][1], va[e][2], va[e][3]);
      }
      if (BS) {  // row k of op(B) = s_k B[k ^ 1]: the sign of odd rows (kb + 8 e = k mod 2)
        const float sg = (kb & 1) ? -bsv[e] : bsv[e];
        *reinterpret_cast<float4*>(&Bs[buf][(kb + 8 * e) * LDB_ + 4 * (tid & 31)]) =
            make_float4(sg * vb[e][0], sg * vb[e][1], sg * vb[e][2], sg * vb[e][3]);
      } else {
        *reinterpret_cast<float4*>(&Bs[buf][(kb + 8 * e) * LDB_ + 4 * (tid & 31)]) =
            make_float4(vb[e][0], vb[e][1], vb[e][2], vb[e][3]);
      }
    }
  };
  auto fix_stage = [&](int buf, int k0) {
    for (int e = tid; e < GBK * BM; e += 256) {
      const int k = e / BM, i = e % BM, gi = i0 + i, gk = k0 + k;
      float* p = &As[buf][k * LDA_ + i];
      *p = (gi >= d.M || gk >= d.K) ? 0.0f : (maskA ? mask_val(*p, maskA, gi + d.offAr, gk + d.offAc) : *p);
    }
    for (int e = tid; e < GBK * BN; e += 256) {
      const int k = e / BN, j = e % BN, gj = j0 + j, gk = k0 + k;
      float* p = &Bs[buf][k * LDB_ + j];
      *p = (gj >= d.N || gk >= d.K) ? 0.0f : (maskB ? mask_val(*p, maskB, gk + d.offBr, gj + d.offBc) : *p);
    }
  };

  // split-bf16x3 staging (X3): each thread holds two groups of four consecutive k -- of
  // rows ra, ra + 64 of A (one 16-byte load each), or of columns p, p + 64 (p = tid % 64)
  // of A^T / B (eight 4-byte loads along k, each a 256-byte row segment per wave) -- fixed
  // in registers when the stage is not plain, then split once into the planes. A wave's
  // planes stores of A^T / B then cover 64 consecutive operand rows (32 bytes apart):
  // with columns 2 p, 2 p + 1 per lane (one 8-byte load per k) they were 64 bytes apart,
  // and twice as many lanes met in each LDS bank (C3 5.72 -> 5.42 ms, C4 13.85 -> 13.61
  // ms). Four lanes per operand row (A's pattern, no bank met twice) lost more to the
  // 64-byte load segments it needs than it gained (C3 5.74, C4 14.12 ms).
  auto xA = [&](int b) { return reinterpret_cast<__bf16*>(smem) + b * 3 * (XPA + XPB); };
  auto xB = [&](int b) { return reinterpret_cast<__bf16*>(smem) + b * 3 * (XPA + XPB) + 3 * XPA; };
  const int xp = tid & 63, xk = 4 * (tid >> 6);
  int xia[2], xjb[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    xia[e] = min(i0 + xp + 64 * e, d.M - 1);
    xjb[e] = min(j0 + xp + 64 * e, d.N - 1);
  }
  // a stage's loaded values (a second set, with the loads two stages ahead, measured
  // 26 % slower on the n = 512 slogdet backward: 194 VGPRs leave two workgroups per CU
  // against three)
  struct X3Regs {
    float a[2][4], b[2][4], s[4];
  };
  X3Regs rg0;
  // The stage loads are raw buffer loads: each operand's base and extent in a descriptor
  // (scalar registers), the thread's fixed byte offset in a vector register and the
  // stage's row offset in a scalar one, so a load costs no address arithmetic and no
  // clamp. A read past the operand's last element returns 0 (the descriptor's range
  // check); whatever lies past M, N or K inside it, the edge path of put_x3 zeroes.
  const unsigned extA = (unsigned)(TA ? (d.K - 1) * d.lda + d.M : (d.M - 1) * d.lda + d.K) * 4u;
  const unsigned extB = (unsigned)((d.K - 1) * d.ldb + d.N) * 4u;
  const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, (int)extA, BUF_RSRC_WORD3);
  const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc((void*)B, 0, (int)extB, BUF_RSRC_WORD3);
  const int xkw = __builtin_amdgcn_readfirstlane(xk);  // wave-uniform
  int oa[2], ob[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    oa[e] = 4 * (TA ? xkw * d.lda + xia[e] : aoff[e] + ka);
    ob[e] = 4 * (xkw * d.ldb + xjb[e]);
  }
  auto load_x3 = [&](int k0, X3Regs& R) {
    if (!TA) {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const v4u x = __builtin_amdgcn_raw_buffer_load_b128(rA, oa[e], 4 * k0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) R.a[e][r] = __uint_as_float(x[r]);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int so = 4 * (k0 + r) * d.lda;
        R.a[0][r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rA, oa[0], so, 0));
        R.a[1][r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rA, oa[1], so, 0));
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int kr = min(k0 + xk + r, d.K - 1);
      if (BS) R.s[r] = d.bscale[bat * (d.K / 2) + (kr >> 1)];
      // row k0 + xk + r (BS: its pair partner, (xk + r) ^ 1 as k0 and xk are even)
      const int so = 4 * (k0 + (BS ? r ^ 1 : r)) * d.ldb;
      R.b[0][r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rB, ob[0], so, 0));
      R.b[1][r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rB, ob[1], so, 0));
    }
  };
  // the stage's masks: each operand's triangle only where its stage meets the diagonal,
  // the matrix edges only in edge tiles and a partial last stage (all uniform)
  auto put_x3 = [&](int b, int k0, const X3Regs& R, auto ma_c, auto mb_c, auto edge_c) {
    constexpr bool ma = decltype(ma_c)::value, mb = decltype(mb_c)::value, edge = decltype(edge_c)::value;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      // A: row gi, k from gk; B: column gj, k from k0 + xk
      const int gi = TA ? i0 + xp + 64 * e : i0 + ra + 64 * e, gk = TA ? k0 + xk : k0 + ka;
      const int gj = j0 + xp + 64 * e;
      float va4[4], vb4[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = R.a[e][r];
        if (ma) v = mask_val(v, maskA, gi + d.offAr, gk + r + d.offAc);
        if (edge) v = (gi >= d.M || gk + r >= d.K) ? 0.0f : v;
        va4[r] = v;
        const int k = k0 + xk + r;
        float w = R.b[e][r];
        if (BS) w *= (k & 1) ? -R.s[r] : R.s[r];
        if (mb) w = mask_val(w, maskB, k + d.offBr, gj + d.offBc);
        if (edge) w = (gj >= d.N || k >= d.K) ? 0.0f : w;
        vb4[r] = w;
      }
      x3_put<XPA>(xA(b), x3_off16(gi - i0, gk - k0), va4);
      x3_put<XPB>(xB(b), x3_off16(gj - j0, xk), vb4);
    }
  };
  auto store_x3 = [&](int b, int k0, const X3Regs& R) {
    using T = std::true_type;
    using F = std::false_type;
    const bool ma = !plain_a(k0), mb = !plain_b(k0), edge = !inside(k0);
    if (edge) put_x3(b, k0, R, T{}, T{}, T{});
    else if (ma && mb) put_x3(b, k0, R, T{}, T{}, F{});
    else if (ma) put_x3(b, k0, R, T{}, F{}, F{});
    else if (mb) put_x3(b, k0, R, F{}, T{}, F{});
    else put_x3(b, k0, R, F{}, F{}, F{});
  };

  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int l32 = lane & 31, lh = lane >> 5;
  v16f acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;
  if constexpr (X3) {
   if (klo < khi) {
    load_x3(klo, rg0);
    store_x3(0, klo, rg0);
    __syncthreads();
    int buf = 0;
    for (int k0 = klo; k0 < khi; k0 += GBK) {
      const bool more = k0 + GBK < khi;
      if (more) load_x3(k0 + GBK, rg0);
      // the stage's K = 16 in one bf16x3 product per accumulator; A's parts first, then
      // each B column block's, used by both A row blocks
      bf16x8 ap[2][3];
#pragma unroll
      for (int a = 0; a < 2; ++a) x3_get<XPA>(xA(buf), x3_off16(wm + 32 * a + l32, 8 * lh), ap[a]);
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        bf16x8 bp[3];
        x3_get<XPB>(xB(buf), x3_off16(wn + 32 * b + l32, 8 * lh), bp);
#pragma unroll
        for (int a = 0; a < 2; ++a) acc[a][b] = mfma_bf16x3(ap[a], bp, acc[a][b]);
      }
      if (more) {
        store_x3(buf ^ 1, k0 + GBK, rg0);
        __syncthreads();
        buf ^= 1;
      }
    }
   }
  } else if (klo < khi) {
    load_stage(klo);
    store_stage(0);
    if (!plain_stage(klo)) {
      __syncthreads();
      fix_stage(0, klo);
    }
    __syncthreads();
    int buf = 0;
    for (int k0 = klo; k0 < khi; k0 += GBK) {
      const bool more = k0 + GBK < khi;
      if (more) load_stage(k0 + GBK);
#pragma unroll
      for (int kp = 0; kp < GBK / 2; ++kp) {
        float av[2], bv[2];
#pragma unroll
        for (int a = 0; a < 2; ++a) av[a] = As[buf][(2 * kp + lh) * LDA_ + wm + 32 * a + l32];
#pragma unroll
        for (int b = 0; b < 2; ++b) bv[b] = Bs[buf][(2 * kp + lh) * LDB_ + wn + 32 * b + l32];
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
          for (int b = 0; b < 2; ++b)
            acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[a], bv[b], acc[a][b], 0, 0, 0);
      }
      if (more) {
        store_stage(buf ^ 1);
        if (!plain_stage(k0 + GBK)) {
          __syncthreads();
          fix_stage(buf ^ 1, k0 + GBK);
        }
        __syncthreads();
        buf ^= 1;
      }
    }
  }

  if (d.tout) {
    // transposed, row-permuted output as in gemm_kernel, in two passes of 64 tile columns
    // (a 64 x 128 transposed half fits the operand LDS): the two waves holding the pass's
    // columns stage them as Ts[c][r], then each of the 64 columns is stored as one
    // contiguous run of 128 rows (two per lane) of row g0[j] of tout
    constexpr int LDT = BM + 1;
    static_assert(64 * LDT * 4 <= SMEM, "half tile fits the operand stages");
    float* Ts = reinterpret_cast<float*>(smem);
    const int* gb = d.g0 + bat * d.N;
    const float sc = d.scale ? d.alpha * d.scale[bat] : d.alpha;
    float* ob = d.tout + bat * (int64_t)d.nout * d.nout;
    bool nf = false;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      __syncthreads();  // the operands (pass 0) / the previous pass's stores are done
      if ((wave & 1) == pass) {
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
          for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const int r = wm + 32 * a + 8 * (v >> 2) + 4 * lh + (v & 3), c = 32 * b + l32;
              Ts[c * LDT + r] = acc[a][b][v];
              nf = nf || (i0 + r < d.M && j0 + 64 * pass + c < d.N && !isfinite(acc[a][b][v]));
            }
      }
      __syncthreads();
      const int jc = j0 + 64 * pass;
      const int rl = jc + lane < d.N ? gb[jc + lane] : d.nout;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int cc = wave + 4 * u;
        const int r = __builtin_amdgcn_readlane(rl, cc);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int i = i0 + lane + 64 * h;
          if (i < d.nout && r < d.nout) ob[(int64_t)r * d.nout + i] = sc * Ts[cc * LDT + lane + 64 * h];
        }
      }
    }
    // one flag per 64 x 64 tile (the layout of gemm_kernel's flags): this tile's value
    // goes to the (up to four) 64-tiles it covers
    const int any = __syncthreads_or(nf ? 1 : 0);
    if (tid == 0) {
      const int ntm = (d.M + 63) / 64, ntn = (d.N + 63) / 64;
      int* fb = d.flags + bat * (int64_t)ntm * ntn;
      for (int a = 0; a < 2; ++a)
        for (int b = 0; b < 2; ++b)
          if (2 * ti + a < ntm && 2 * tj + b < ntn) fb[(2 * ti + a) * ntn + 2 * tj + b] = any;
    }
    return;
  }

  // epilogue as in gemm_kernel, with 32-bit offsets within the matrix: element v of an
  // accumulator is row r0 + dv, dv = 8 (v / 4) + v % 4, so its offsets step by the
  // uniform dv * ldc (and dv for the mirrored store)
  const bool diag_tile = d.lower_only && ti == tj;
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int c = j0 + wn + 32 * b + l32;
      const int r0 = i0 + wm + 32 * a + 4 * lh;
      const int o = r0 * d.ldc + c, om = c * d.ldc + r0;
      float cv[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int dv = 8 * (v >> 2) + (v & 3);
        cv[v] = (d.beta != 0.0f && r0 + dv < d.M && c < d.N) ? C[o + dv * d.ldc] : 0.0f;
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int dv = 8 * (v >> 2) + (v & 3), r = r0 + dv;
        if (r >= d.M || c >= d.N) continue;
        if (diag_tile && r < c) continue;
        float val = d.alpha * acc[a][b][v];
        if (d.beta != 0.0f) val = fmaf(d.beta, cv[v], val);
        if (d.lower_only && r == c && d.mirror < 0.0f) val = 0.0f;
        C[o + dv * d.ldc] = val;
        if (d.lower_only && r != c) C[om + dv] = d.mirror * val;
      }
    }
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <bool X3>
static int launch_gemm_t(const GemmDesc& d, int64_t batch, int nb2, hipStream_t s) {
  if (d.lower_only && d.M != d.N) return FX_ERR_INVALID_ARGUMENT;
  // 64 x 64 tiles throughout: with one 32x32 accumulator per wave many more workgroups
  // stay resident per CU than with 128 x 128 tiles, which hides the operand and C
  // latencies better on every product of this library (measured 11 % faster on the n =
  // 512 slogdet backward, 2 % on the n = 2048 slogpf backward). Square tiles: the
  // lower-only (skew) enumeration assumes BM == BN.
  constexpr int BM = 64, BN = 64;
  const int tm = (d.M + BM - 1) / BM, tn = (d.N + BN - 1) / BN;
  const int tiles = d.lower_only ? tm * (tm + 1) / 2 : tm * tn;
  // 16-byte loads need every contiguous extent, leading dimension, batch stride and base
  // pointer to be a multiple of 4 floats
  const bool vec = aligned16(d.A) && aligned16(d.B) && d.lda % 4 == 0 && d.ldb % 4 == 0 &&
                   d.sA % 4 == 0 && d.sB % 4 == 0 && d.sA2 % 4 == 0 && d.sB2 % 4 == 0 &&
                   d.K % 4 == 0 && (d.transA ? d.M % 4 == 0 : true) &&
                   (d.transB ? true : d.N % 4 == 0);
  // 128 x 128 tiles for the large products (measured at batch 64: the n = 2048 top
  // triangular-inverse level 18 % and the skew R product 15 % faster); at M = 512 and
  // below, and for short K, the coarser triangle trimming and the longer prologue /
  // epilogue per K stage make the 64 x 64 tiles faster
  const fx_tune& tu = tune();
  const int mn128 = X3 ? tu.gemm128_x3_min_mn : tu.gemm128_min_mn;
  const int k128 = X3 ? tu.gemm128_x3_min_k : tu.gemm128_min_k;
  const int tout128 = X3 ? tu.gemm128_x3_tout : tu.gemm128_tout;
  const bool big = vec && !d.transB && d.M >= mn128 && d.N >= mn128 && d.K >= k128 && (!d.tout || tout128);
  if (d.tout && (d.lower_only || nb2 != 1 || d.active)) return FX_ERR_INVALID_ARGUMENT;
  if (d.bscale && (d.maskB != MASK_NONE || d.transB || d.K % 2 || nb2 != 1 || !vec)) return FX_ERR_INVALID_ARGUMENT;
  const int tm2 = (d.M + 127) / 128, tn2 = (d.N + 127) / 128;
  const int tiles2 = d.lower_only ? tm2 * (tm2 + 1) / 2 : tm2 * tn2;
  for (int64_t b0 = 0; b0 < batch; b0 += 65535) {
    const int64_t nb = batch - b0 < 65535 ? batch - b0 : 65535;
    GemmDesc e = d;
    // XCD-aware tile order (all tiles of one matrix on one XCD, so its L2 fetches the
    // matrix's operands once): 14 % faster on the K = 64 LU trailing update, 6 % on a
    // plain 512^3 product, neutral on the masked ones
    e.xcd8 = nb % 8 == 0;
    e.A += b0 * d.sA;
    e.B += b0 * d.sB;
    if (d.C) e.C += b0 * d.sC;
    if (d.active) e.active += b0;
    if (d.tout) {
      e.tout += b0 * (int64_t)d.nout * d.nout;
      e.g0 += b0 * d.N;
      e.flags += b0 * tiles;
      if (d.scale) e.scale += b0;
    }
    if (d.bscale) e.bscale += b0 * (d.K / 2);
    if (d.bscale) {  // the B row transform: its own instantiations (A^T unit upper, or any mask)
      const bool ua = d.transA && d.maskA == MASK_UPPER_UNIT;
      if (big) {
        const dim3 grid2(tiles2, (unsigned)nb, nb2);
        if (ua) hipLaunchKernelGGL((gemm128_kernel<true, 4 * MASK_UPPER_UNIT, true, X3>), grid2, dim3(256), 0, s, e);
        else if (d.transA) hipLaunchKernelGGL((gemm128_kernel<true, -1, true, X3>), grid2, dim3(256), 0, s, e);
        else hipLaunchKernelGGL((gemm128_kernel<false, -1, true, X3>), grid2, dim3(256), 0, s, e);
      } else {
        const dim3 grid(tiles, (unsigned)nb, nb2);
        if (ua) hipLaunchKernelGGL((gemm_kernel<BM, BN, true, 4 * MASK_UPPER_UNIT, true, X3>), grid, dim3(256), 0, s, e);
        else hipLaunchKernelGGL((gemm_kernel<BM, BN, true, -1, true, X3>), grid, dim3(256), 0, s, e);
      }
      if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
      continue;
    }
    if (big) {
      const dim3 grid2(tiles2, (unsigned)nb, nb2);
#define FX_GEMM128(T, K) hipLaunchKernelGGL((gemm128_kernel<T, K, false, X3>), grid2, dim3(256), 0, s, e)
      const int mk = 4 * d.maskA + d.maskB;
      if (d.transA) {
        if (mk == 4 * MASK_UPPER_UNIT + MASK_NONE) FX_GEMM128(true, 4 * MASK_UPPER_UNIT + MASK_NONE);
        else if (mk == 0) FX_GEMM128(true, 0);
        else FX_GEMM128(true, -1);
      } else {
        switch (mk) {
          case 4 * MASK_NONE + MASK_NONE: FX_GEMM128(false, 4 * MASK_NONE + MASK_NONE); break;
          case 4 * MASK_NONE + MASK_LOWER_UNIT: FX_GEMM128(false, 4 * MASK_NONE + MASK_LOWER_UNIT); break;
          case 4 * MASK_NONE + MASK_UPPER: FX_GEMM128(false, 4 * MASK_NONE + MASK_UPPER); break;
          case 4 * MASK_LOWER_UNIT + MASK_NONE: FX_GEMM128(false, 4 * MASK_LOWER_UNIT + MASK_NONE); break;
          case 4 * MASK_UPPER + MASK_NONE: FX_GEMM128(false, 4 * MASK_UPPER + MASK_NONE); break;
          case 4 * MASK_UPPER + MASK_LOWER_UNIT: FX_GEMM128(false, 4 * MASK_UPPER + MASK_LOWER_UNIT); break;
          default: FX_GEMM128(false, -1); break;
        }
      }
#undef FX_GEMM128
      if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
      continue;
    }
    const dim3 grid(tiles, (unsigned)nb, nb2);
#define FX_GEMM_MK(K) hipLaunchKernelGGL((gemm_kernel<BM, BN, true, K, false, X3>), grid, dim3(256), 0, s, e)
    if (vec) {
      switch (4 * d.maskA + d.maskB) {
        case 4 * MASK_NONE + MASK_NONE: FX_GEMM_MK(4 * MASK_NONE + MASK_NONE); break;
        case 4 * MASK_NONE + MASK_LOWER_UNIT: FX_GEMM_MK(4 * MASK_NONE + MASK_LOWER_UNIT); break;
        case 4 * MASK_NONE + MASK_UPPER: FX_GEMM_MK(4 * MASK_NONE + MASK_UPPER); break;
        case 4 * MASK_LOWER_UNIT + MASK_NONE: FX_GEMM_MK(4 * MASK_LOWER_UNIT + MASK_NONE); break;
        case 4 * MASK_UPPER + MASK_NONE: FX_GEMM_MK(4 * MASK_UPPER + MASK_NONE); break;
        case 4 * MASK_UPPER + MASK_LOWER_UNIT: FX_GEMM_MK(4 * MASK_UPPER + MASK_LOWER_UNIT); break;
        case 4 * MASK_UPPER_UNIT + MASK_NONE: FX_GEMM_MK(4 * MASK_UPPER_UNIT + MASK_NONE); break;
        default: FX_GEMM_MK(-1); break;
      }
    } else {
      hipLaunchKernelGGL((gemm_kernel<BM, BN, false, -1, false, X3>), grid, dim3(256), 0, s, e);
    }
#undef FX_GEMM_MK
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  }
  return FX_OK;
}

int launch_gemm(const GemmDesc& d, int64_t batch, int nb2, hipStream_t s) {
  if (d.M <= 0 || d.N <= 0 || batch <= 0 || nb2 <= 0) return FX_OK;
  return d.x3 ? launch_gemm_t<true>(d, batch, nb2, s) : launch_gemm_t<false>(d, batch, nb2, s);
}

}  // namespace fx
