// Blocked LU with partial pivoting for 128 < n <= 8192 (any batch): per block of PW = 64
// columns at r0 three launches (blocks go in pairs, see run_blocks: the first block's
// trailing update is deferred and merged into the second's at K = 128),
//   1. the panel (one workgroup per matrix), factored in place in the work buffer; the
//      rows stay in place during the panel (virtual pivoting) and each column step finds
//      the pivot with a per-wave DPP max and one workgroup barrier (every wave posts its
//      best row, all waves pick the same winner):
//      - lu_panel_reg_kernel for m = N - r0 <= 1024: one row per lane (64..1024 threads,
//        the smallest count that covers m), the whole 64-column row in registers; after
//        each 16-column sub-panel the pivot rows publish their remaining columns in LDS,
//        U = X * A_piv is formed there and every unassigned row applies A_rest -= L U
//        with its own FMAs, so the panel is read once and written once;
//      - lu_panel_kernel for taller panels: 2-4 rows per lane, one 16-column sub-panel in
//        registers at a time, the trailing columns inside the panel updated on MFMA
//        (stores predicated to unassigned rows);
//      both write the panel back in the new row order, with the map
//      src[new position] = old row and X_s = L_ss^-1 of every sub-panel;
//   2. lu_urow_kernel   (matrix x 64-column strip): applies the row permutation to the
//      strip, touching only the rows that move, and for trailing strips forms the U rows
//      U12 = L11^-1 A12 by blocked forward substitution on MFMA (in a pair's second block
//      after subtracting the first block's deferred update from the pivot rows);
//   3. lu_update_kernel: the trailing update A22 -= L21 U12 on MFMA, one LDS stage of
//      K = 64 per 64 x 64 tile at a time: a pair's first block updates only the second
//      block's 64 columns, the second block the whole trailing matrix at K = 128.
// A final kernel turns the pivots and swap counts into (sign, logabs).
//
// Reference roles replaced (ChenAo-Phys/fermix): _lu_core's block loop (src/fermix/
// _lu.py:543-611) with its inner panel (_lu.py:54-224), inter-panel update (:228-296),
// U-row solve (:300-330) and trailing GEMM (:334-393).
#include "common.h"
#include "fermix_internal.h"

namespace fx {

template <int MR, int PW, int NT>
struct LuPanel {
  static constexpr int NW = NT / 64;
  static constexpr int R = MR / NT;  // rows per lane
  static constexpr int NSUB = PW / 16;
};

struct Cand {
  unsigned key;
  int row;
  int pos;
  int pad;
  float v[16];
};

// Copy A (B, n, n) into the work buffer W (B, N, N) with identity padding.
// 32-bit index math within a matrix (N * N < 2^31).
__global__ void copy_pad_kernel(const float* __restrict__ A, int n, float* __restrict__ W, int N) {
  const int64_t b = blockIdx.y;
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= N * N) return;
  const int r = e / N, c = e - r * N;
  W[b * N * N + e] = (r < n && c < n) ? A[b * n * n + r * n + c] : (r == c ? 1.0f : 0.0f);
}

// Panels taller than one row per lane (m > 1024): factored in place in the work buffer
// (rows in place until the final permutation), 16 columns at a time in registers -- the
// workgroup's own global accesses are ordered by its barriers (one CU, workgroup-scope
// fences).
template <int MR, int PW, int NT>
__global__ __launch_bounds__(NT) void lu_panel_kernel(float* __restrict__ W, int N, int r0, int blk,
                                                      float* __restrict__ piv_out,
                                                      int* __restrict__ nsw_out, int nblk,
                                                      int* __restrict__ src_out,
                                                      float* __restrict__ X_out,
                                                      int* __restrict__ g0, int lmove) {
  using C = LuPanel<MR, PW, NT>;
  constexpr int R = C::R, NSUB = C::NSUB, NW = C::NW;
  __shared__ Cand cand[2][NW];
  __shared__ float Ubuf[16 * PW];
  __shared__ int posL[MR];
  __shared__ int prowL[16];
  __shared__ float Xs[256];
  __shared__ float L11s[256];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int m = N - r0;
  float* Wb = W + b * (int64_t)N * N;
  float* const P = Wb + (int64_t)r0 * N + r0;
  const int LDP = N;

  int pos[R];
  bool valid[R];
#pragma unroll
  for (int s = 0; s < R; ++s) {
    const int i = R * (64 * wave + lane) + s;
    valid[s] = i < m;
    pos[s] = i;
  }
  int nsw = 0;
  __syncthreads();

  for (int sp = 0; sp < NSUB; ++sp) {
    const int c0 = 16 * sp;
    float a[R][16];
    // 16-byte loads (r0, c0 and N are multiples of 16); rows past m read row 0
#pragma unroll
    for (int s = 0; s < R; ++s) {
      const int i = R * tid + s;
      const float4* rp = reinterpret_cast<const float4*>(P + (int64_t)(valid[s] ? i : 0) * LDP + c0);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 v = rp[q];
        a[s][4 * q] = valid[s] ? v.x : 0.0f;
        a[s][4 * q + 1] = valid[s] ? v.y : 0.0f;
        a[s][4 * q + 2] = valid[s] ? v.z : 0.0f;
        a[s][4 * q + 3] = valid[s] ? v.w : 0.0f;
      }
    }
    static_for<0, 16>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      const int posc = c0 + j;
      unsigned kb = 0;
      int ib = 0;
#pragma unroll
      for (int s = 0; s < R; ++s) {
        const unsigned k = cand_key(a[s][j], valid[s] && pos[s] >= posc);
        if (k > kb) { kb = k; ib = s; }
      }
      const unsigned gk = wave_max_u32(kb);
      const int pl = first_lane(gk != 0u ? (kb == gk) : (lane == 0));
      Cand& my = cand[j & 1][wave];
      if (lane == pl) {
        my.key = gk;
        my.row = R * (64 * wave + lane) + ib;
#pragma unroll
        for (int s = 0; s < R; ++s) {
          if (ib == s) {
            my.pos = pos[s];
#pragma unroll
            for (int jj = 0; jj < 16; ++jj) my.v[jj] = opaque(a[s][jj]);
          }
        }
      }
      __syncthreads();
      unsigned best = cand[j & 1][0].key;
      int wb = 0;
#pragma unroll
      for (int w = 1; w < NW; ++w) {
        const unsigned kw = cand[j & 1][w].key;
        if (kw > best) { best = kw; wb = w; }
      }
      const Cand& win = cand[j & 1][wb];
      float u[16];
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) u[jj] = win.v[jj];
      const int pp = win.pos, prow = win.row;
      // the pivot row and its L entries (row j of L11) for X = L11^-1 after the steps
      if (tid == 0) prowL[j] = prow;
      if (tid < j) L11s[j * 16 + tid] = win.v[tid];
#pragma unroll
      for (int s = 0; s < R; ++s) {
        const int i = R * (64 * wave + lane) + s;
        if (valid[s] && pos[s] == posc) pos[s] = pp;
        if (i == prow) pos[s] = posc;
      }
      nsw += (pp != posc) ? 1 : 0;
      pin(nsw);
      const float pivv = u[j];
      if (wave == 0 && lane == 0) piv_out[b * N + r0 + posc] = pivv;
      const float rcp = safe_rcp(pivv);
#pragma unroll
      for (int s = 0; s < R; ++s) {
        if (valid[s] && pos[s] > posc) {
          const float l = a[s][j] * rcp;
          a[s][j] = l;
          static_for<j + 1, 16>([&](auto cc) { a[s][cc.value] = fmaf(-l, u[cc.value], a[s][cc.value]); });
        }
      }
    });
    // sub-panel back (rows stay in place), positions, pivot rows, X
#pragma unroll
    for (int s = 0; s < R; ++s) {
      const int i = R * (64 * wave + lane) + s;
      if (valid[s]) {
        float4* rp = reinterpret_cast<float4*>(P + (int64_t)i * LDP + c0);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          rp[q] = make_float4(a[s][4 * q], a[s][4 * q + 1], a[s][4 * q + 2], a[s][4 * q + 3]);
        posL[i] = pos[s];
      }
    }
    __syncthreads();
    // X = L11^-1 (unit lower): lane c < 16 of wave 0 forms column c,
    // X[j][c] = -sum_{k<j} L11[j][k] X[k][c], X[c][c] = 1, X[j][c] = 0 for j < c
    if (wave == 0 && lane < 16) {
      float xcol[16];
      static_for<0, 16>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        float x = 0.0f;
        static_for<0, j>([&](auto kc) { x = fmaf(-L11s[j * 16 + kc.value], xcol[kc.value], x); });
        xcol[j] = (lane == j) ? 1.0f : x;
      });
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        Xs[k * 16 + lane] = xcol[k];
        X_out[((b * NSUB + sp) * 16 + k) * 16 + lane] = xcol[k];
      }
    }
    __syncthreads();
    const int nss = NSUB - sp - 1;  // strips right of the sub-panel inside the panel
    if (nss > 0) {
      const int li = lane & 15, g = lane >> 4;
      // phase A: U = X * A[pivot rows, strip]
      if (wave < nss) {
        const int cs = c0 + 16 * (wave + 1);
        v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 4; ++t)
          acc = mfma16(Xs[li * 16 + 4 * t + g], P[(int64_t)prowL[4 * t + g] * LDP + cs + li], acc);
#pragma unroll
        for (int v = 0; v < 4; ++v) Ubuf[(4 * g + v) * PW + cs + li] = acc[v];
      }
      __syncthreads();
      // phase B: rest -= L * U on the unassigned rows
      const int nrt = (m + 15) / 16;
      for (int task = wave; task < nss * nrt; task += NW) {
        const int st = task % nss, rt = task / nss;
        const int cs = c0 + 16 * (st + 1);
        const int rb = 16 * rt;
        v4f acc;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int r = rb + 4 * g + v;
          acc[v] = r < m ? P[(int64_t)r * LDP + cs + li] : 0.0f;
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int r = rb + li;
          const float lv = r < m ? P[(int64_t)r * LDP + c0 + 4 * t + g] : 0.0f;
          acc = mfma16(-lv, Ubuf[(4 * t + g) * PW + cs + li], acc);
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int r = rb + 4 * g + v;
          if (r < m && posL[r] > c0 + 15) P[(int64_t)r * LDP + cs + li] = acc[v];
        }
      }
      __syncthreads();
      // phase C: the pivot rows take their U values
      const int ncols = 16 * nss;
      for (int e = tid; e < 16 * ncols; e += NT) {
        const int k = e / ncols, c = c0 + 16 + e % ncols;
        P[(int64_t)prowL[k] * LDP + c] = Ubuf[k * PW + c];
      }
      __syncthreads();
    }
  }
  // write the panel back in the new row order, in place, 16 columns at a time: every row
  // of a pass is read before any is written. With lmove the previous block's 64 L
  // columns (left of the panel) go along.
  for (int q = lmove ? -4 : 0; q < NSUB; ++q) {
    float v[R][16];  // plain floats: an array of float4 stays in scratch memory
#pragma unroll
    for (int s = 0; s < R; ++s) {
      const int i = R * tid + s;
      const float4* rp = reinterpret_cast<const float4*>(P + (int64_t)(i < m ? i : 0) * LDP + 16 * q);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float4 t = rp[k];
        v[s][4 * k] = t.x;
        v[s][4 * k + 1] = t.y;
        v[s][4 * k + 2] = t.z;
        v[s][4 * k + 3] = t.w;
      }
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < R; ++s) {
      const int i = R * tid + s;
      if (i < m) {
        float4* wp = reinterpret_cast<float4*>(P + (int64_t)posL[i] * LDP + 16 * q);
#pragma unroll
        for (int k = 0; k < 4; ++k) wp[k] = make_float4(v[s][4 * k], v[s][4 * k + 1], v[s][4 * k + 2], v[s][4 * k + 3]);
      }
    }
    __syncthreads();
  }
  for (int i = tid; i < m; i += NT) src_out[b * N + r0 + posL[i]] = r0 + i;
  if (g0) {
    // compose the row map: g0[r0 + p] <- g0[r0 + src(p)]
    int* gb = g0 + b * N;
    int tmp[(MR + NT - 1) / NT];
#pragma unroll
    for (int q = 0; q < (MR + NT - 1) / NT; ++q) {
      const int i = tid + NT * q;
      tmp[q] = i < m ? gb[r0 + i] : 0;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < (MR + NT - 1) / NT; ++q) {
      const int i = tid + NT * q;
      if (i < m) gb[r0 + posL[i]] = tmp[q];
    }
  }
  if (tid == 0) nsw_out[b * nblk + blk] = nsw;
}

// The same panel (PW = 64, in place in the work buffer) for m <= NT with one row per lane
// and the whole 64-column row in registers: the column steps are those of
// lu_panel_kernel, but after each sub-panel the 16 pivot rows publish their remaining
// columns in LDS, U = X * (those columns) is formed there, and every unassigned row
// applies A_rest -= L U with its own FMAs (pivot rows take their U row). The panel is
// read once and written once, in the new row order, with no global round trip between.
template <int NT>
__global__ __launch_bounds__(NT) void lu_panel_reg_kernel(float* __restrict__ W, int N, int r0, int blk,
                                                          float* __restrict__ piv_out,
                                                          int* __restrict__ nsw_out, int nblk,
                                                          int* __restrict__ src_out,
                                                          float* __restrict__ X_out,
                                                          int* __restrict__ g0,
                                                          const float* __restrict__ A0, int lmove) {
  constexpr int NW = NT / 64, PW = 64, NSUB = 4;
  __shared__ Cand cand[2][NW];
  __shared__ __align__(16) float Prow[16 * PW];  // pivot rows of the sub-panel, all columns
  __shared__ __align__(16) float Ubuf[16 * PW];
  __shared__ float Xs[256];
  __shared__ float L11s[256];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int m = N - r0;
  float* Wb = W + b * (int64_t)N * N;
  float* const P = Wb + (int64_t)r0 * N + r0;
  const bool valid = tid < m;
  int pos = tid;
  float a[PW];
  {
    // 16-byte loads (r0 and N are multiples of 64); lanes past m read row 0. A0 (first
    // block only, in place of the input copy): the panel is read from the input itself.
    const float* Ps = A0 ? A0 + b * (int64_t)N * N : P;
    const float4* rp = reinterpret_cast<const float4*>(Ps + (int64_t)(valid ? tid : 0) * N);
#pragma unroll
    for (int q = 0; q < PW / 4; ++q) {
      const float4 v = rp[q];
      a[4 * q] = valid ? v.x : 0.0f;
      a[4 * q + 1] = valid ? v.y : 0.0f;
      a[4 * q + 2] = valid ? v.z : 0.0f;
      a[4 * q + 3] = valid ? v.w : 0.0f;
    }
  }
  int nsw = 0;
  static_for<0, NSUB>([&](auto spc) {
    constexpr int c0 = 16 * decltype(spc)::value;
    static_for<0, 16>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      constexpr int col = c0 + j;
      const unsigned kb = cand_key(a[col], valid && pos >= col);
      const unsigned gk = wave_max_u32(kb);
      const int pl = first_lane(gk != 0u ? (kb == gk) : (lane == 0));
      Cand& my = cand[j & 1][wave];
      if (lane == pl) {
        my.key = gk;
        my.row = tid;
        my.pos = pos;
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) my.v[jj] = a[c0 + jj];
      }
      __syncthreads();
      unsigned best = cand[j & 1][0].key;
      int wb = 0;
#pragma unroll
      for (int w = 1; w < NW; ++w) {
        const unsigned kw = cand[j & 1][w].key;
        if (kw > best) { best = kw; wb = w; }
      }
      const Cand& win = cand[j & 1][wb];
      float u[16];
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) u[jj] = win.v[jj];
      const int pp = win.pos, prow = win.row;
      if (tid < j) L11s[j * 16 + tid] = win.v[tid];
      if (valid && pos == col) pos = pp;
      if (tid == prow) pos = col;
      nsw += (pp != col) ? 1 : 0;
      pin(nsw);
      const float pivv = u[j];
      if (tid == 0) piv_out[b * N + r0 + col] = pivv;
      const float rcp = safe_rcp(pivv);
      if (valid && pos > col) {
        const float l = a[col] * rcp;
        a[col] = l;
        static_for<j + 1, 16>([&](auto cc) { a[c0 + cc.value] = fmaf(-l, u[cc.value], a[c0 + cc.value]); });
      }
    });
    if constexpr (c0 + 16 < PW) {
      // the sub-panel's pivot rows publish their remaining columns
      if (valid && pos >= c0 && pos < c0 + 16) {
        float* pr = Prow + (pos - c0) * PW;
#pragma unroll
        for (int c = c0 + 16; c < PW; c += 4) *reinterpret_cast<float4*>(pr + c) = make_float4(a[c], a[c + 1], a[c + 2], a[c + 3]);
      }
    }
    __syncthreads();
    // X = L11^-1 (unit lower): lane c < 16 of wave 0 forms column c,
    // X[j][c] = -sum_{k<j} L11[j][k] X[k][c], X[c][c] = 1, X[j][c] = 0 for j < c
    if (wave == 0 && lane < 16) {
      float xcol[16];
      static_for<0, 16>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        float x = 0.0f;
        static_for<0, j>([&](auto kc) { x = fmaf(-L11s[j * 16 + kc.value], xcol[kc.value], x); });
        xcol[j] = (lane == j) ? 1.0f : x;
      });
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        Xs[k * 16 + lane] = xcol[k];
        X_out[((b * NSUB + c0 / 16) * 16 + k) * 16 + lane] = xcol[k];
      }
    }
    if constexpr (c0 + 16 < PW) {
      constexpr int NC = PW - c0 - 16;  // columns right of the sub-panel
      __syncthreads();
      // U = X * Prow[:, c0+16 ..] (X unit lower: terms t <= k)
      for (int e = tid; e < 16 * NC; e += NT) {
        const int k = e / NC, c = c0 + 16 + e % NC;
        float s = Prow[k * PW + c];
        for (int t = 0; t < k; ++t) s = fmaf(Xs[k * 16 + t], Prow[t * PW + c], s);
        Ubuf[k * PW + c] = s;
      }
      __syncthreads();
      if (valid && pos > c0 + 15) {
        // A_rest -= L U on the unassigned rows (U rows broadcast from LDS)
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const float l = a[c0 + k];
#pragma unroll
          for (int c = c0 + 16; c < PW; c += 4) {
            const float4 uv = *reinterpret_cast<const float4*>(Ubuf + k * PW + c);
            a[c] = fmaf(-l, uv.x, a[c]);
            a[c + 1] = fmaf(-l, uv.y, a[c + 1]);
            a[c + 2] = fmaf(-l, uv.z, a[c + 2]);
            a[c + 3] = fmaf(-l, uv.w, a[c + 3]);
          }
        }
      } else if (valid && pos >= c0) {
        // pivot rows take their U row
        const float* ur = Ubuf + (pos - c0) * PW;
#pragma unroll
        for (int c = c0 + 16; c < PW; c += 4) {
          const float4 uv = *reinterpret_cast<const float4*>(ur + c);
          a[c] = uv.x;
          a[c + 1] = uv.y;
          a[c + 2] = uv.z;
          a[c + 3] = uv.w;
        }
      }
    }
  });
  // the panel back in the new row order (every row was read at the start, many barriers
  // ago, so the in-place stores cannot overwrite an unread row)
  if (valid) {
    float4* wp = reinterpret_cast<float4*>(P + (int64_t)pos * N);
#pragma unroll
    for (int q = 0; q < PW / 4; ++q) wp[q] = make_float4(a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]);
    src_out[b * N + r0 + pos] = r0 + tid;
  }
  if (lmove) {
    // the previous block's 64 L columns (left of the panel) follow the rows that moved:
    // all read, one barrier, all written (a moved row's slot belongs to another moved row)
    const bool mv = valid && pos != tid;
    if (mv) {
      const float4* rp = reinterpret_cast<const float4*>(P - PW + (int64_t)tid * N);
#pragma unroll
      for (int q = 0; q < PW / 4; ++q) {
        const float4 t = rp[q];
        a[4 * q] = t.x;
        a[4 * q + 1] = t.y;
        a[4 * q + 2] = t.z;
        a[4 * q + 3] = t.w;
      }
    }
    __syncthreads();
    if (mv) {
      float4* wp = reinterpret_cast<float4*>(P - PW + (int64_t)pos * N);
#pragma unroll
      for (int q = 0; q < PW / 4; ++q) wp[q] = make_float4(a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]);
    }
  }
  if (g0) {
    // compose the row map: g0[r0 + p] <- g0[r0 + src(p)]
    int* gb = g0 + b * N;
    const int t0 = valid ? gb[r0 + tid] : 0;
    __syncthreads();
    if (valid) gb[r0 + pos] = t0;
  }
  if (tid == 0) nsw_out[b * nblk + blk] = nsw;
}

// Row permutation of one 64-column strip and, for a trailing strip, its U rows
// U12 = L11^-1 A12. Everything is read before anything is written (the moved rows into
// registers, 32 per thread; A12, L11 and the panel's X straight into MFMA operand
// layout), then the moved rows are stored and each wave solves for its 16 columns of U12
// in registers: U_s = X_s (A_s - sum_{t<s} L_st U_t), the right operands in accumulator
// layout (lane (g, c) holding rows 4g + v) taken as they stand, one MFMA per v over the
// K indices {4g + v}. About 1.3 KiB of LDS and (launch bound) at most 128 registers, so
// 4 waves per SIMD.
template <int PW, int MAXM>
__global__ __launch_bounds__(256, 4) void lu_urow_kernel(float* __restrict__ W, int N, int r0,
                                                      const int* __restrict__ src,
                                                      const float* __restrict__ Xg, int lfirst,
                                                      int nleft, const float* __restrict__ A0,
                                                      const int* __restrict__ rmap, int rc,
                                                      int* __restrict__ comp_out) {
  static_assert(PW == 64, "one 16-column slice of the strip per wave");
  constexpr int NSUB = PW / 16;
  __shared__ int list[2 * PW];
  __shared__ int srcv[2 * PW];
  __shared__ int srcU[PW];
  __shared__ int srcUr[PW];
  __shared__ int cnt;
  constexpr int LDL = PW + 4;
  __shared__ __align__(16) float Ls[PW * LDL];  // L21' of the pivot rows (deferred update)
  const int64_t b = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int strip = blockIdx.x;
  const bool left = strip < nleft;
  const int cstart = left ? 64 * (lfirst + strip) : r0 + PW + 64 * (strip - nleft);
  const int ncol = min(64, left ? r0 - cstart : N - cstart);
  float* Wb = W + b * (int64_t)N * N;
  // A0 (first block pair, in place of the input copy): the trailing rows are read from
  // the input (position p of the first block's order is input row rmap[p] when rmap is
  // given), and the trailing update writes every row below the block (from the input,
  // through the row maps), so only U12 is stored here
  const float* Rb = A0 && !left ? A0 + b * (int64_t)N * N : Wb;
  const int* rm = rmap && !left ? rmap + b * N : nullptr;
  const int* sb = src + b * N;
  const int m = N - r0;
  // pass 1 (indices): the moved rows (position, source row) and the source rows of
  // positions r0 .. r0+PW-1. srcv[0] starts as a valid row: the gathers below read
  // srcv[0] for every slot k >= nm, including when no row moved (nm = 0).
  if (tid == 0) {
    cnt = 0;
    srcv[0] = r0;
  }
  // deferred update (rc >= 0): the pivot rows' L21' (rows r0 .. r0+63 -- the panel moved
  // those columns along -- columns rc .. rc+63) is read once per workgroup, here, so its
  // latency overlaps the index pass; it reaches LDS before the read barrier below
  float lr[16];
  const bool corr = rc >= 0 && !left;
  if (corr) {
    const float4* lp = reinterpret_cast<const float4*>(Wb + (int64_t)(r0 + (tid >> 2)) * N + rc + 16 * (tid & 3));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 t = lp[q];
      lr[4 * q] = t.x;
      lr[4 * q + 1] = t.y;
      lr[4 * q + 2] = t.z;
      lr[4 * q + 3] = t.w;
    }
  }
  __syncthreads();
  constexpr int MQ = MAXM / 256;  // m <= N <= MAXM
  int sv[MQ];
#pragma unroll
  for (int q = 0; q < MQ; ++q) {
    const int p = tid + 256 * q;
    sv[q] = p < m ? sb[r0 + p] : r0 + p;
  }
#pragma unroll
  for (int q = 0; q < MQ; ++q) {
    const int p = tid + 256 * q;
    // srcv / srcUr index the rows of Rb (through rmap), srcU those of W
    const int sr = rm && p < m ? rm[sv[q]] : sv[q];
    if (p < m && sv[q] != r0 + p) {
      const int k = atomicAdd(&cnt, 1);
      if (k < 2 * PW) {
        list[k] = p;
        srcv[k] = sr;
      }
    }
    if (p < PW) {
      srcU[p] = sv[q];
      srcUr[p] = sr;
    }
  }
  // the composed map of the first block pair (position -> input row), for its update
  if (comp_out && rm && blockIdx.x == nleft) {  // the first trailing strip
#pragma unroll
    for (int q = 0; q < MQ; ++q) {
      const int p = tid + 256 * q;
      if (p < m) comp_out[b * N + r0 + p] = rm[sv[q]];
    }
  }
  __syncthreads();
  const int nm = min(cnt, 2 * PW);
  // pass 2: every read. Moved row k (< nm) column cl: thread (k % 4 = tid >> 6, cl).
  const int cl = tid & 63;
  const int cc = min(cl, ncol - 1);
  float mv[2 * PW / 4];
#pragma unroll
  for (int u = 0; u < 2 * PW / 4; ++u) {
    const int k = (tid >> 6) + 4 * u;
    mv[u] = Rb[(int64_t)srcv[k < nm ? k : 0] * N + cstart + cc];
  }
  // operands of the U12 solve (trailing strips): lane (g, li) of wave w, column 16w + li
  const int li = lane & 15, g = lane >> 4;
  const int col = min(16 * wave + li, ncol - 1);
  v4f a12[NSUB];
  float lv[NSUB * (NSUB - 1) / 2][4], xv[NSUB][4];
  if (!left) {
    const float* Xb = Xg + b * NSUB * 256;
#pragma unroll
    for (int s = 0; s < NSUB; ++s)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        a12[s][v] = Rb[(int64_t)srcUr[16 * s + 4 * g + v] * N + cstart + col];
        xv[s][v] = Xb[s * 256 + li * 16 + 4 * g + v];
      }
#pragma unroll
    for (int s = 1, q = 0; s < NSUB; ++s)
#pragma unroll
      for (int t = 0; t < s; ++t, ++q)
#pragma unroll
        for (int v = 0; v < 4; ++v) lv[q][v] = Wb[(int64_t)(r0 + 16 * s + li) * N + r0 + 16 * t + 4 * g + v];
  }
  if (corr) {
    float* lq = Ls + (tid >> 2) * LDL + 16 * (tid & 3);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<float4*>(lq + 4 * q) = make_float4(lr[4 * q], lr[4 * q + 1], lr[4 * q + 2], lr[4 * q + 3]);
  }
  __syncthreads();  // no row is written before every thread has read what it needs
  // the moved rows; rows r0 .. r0+PW-1 of a trailing strip are written below as U12
#pragma unroll
  for (int u = 0; u < 2 * PW / 4; ++u) {
    const int k = (tid >> 6) + 4 * u;
    if ((left || !A0) && k < nm && cl < ncol && (left || list[k] >= PW)) Wb[(int64_t)(r0 + list[k]) * N + cstart + cl] = mv[u];
  }
  if (left) return;
  if (corr) {
    // deferred update of the previous block (rows / columns rc .. rc+63, not yet applied
    // to these columns): A12 -= L21' U12' on the pivot rows, with L21' from LDS (staged
    // above) and U12' from rows rc .. rc+63. MFMA c takes k = 16 g + c on lane (g, li):
    // four 16-byte L21' reads per row block, one U12' row element per c.
    float uv[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) uv[c] = -Wb[(int64_t)(rc + 16 * g + c) * N + cstart + col];  // -U12
#pragma unroll
    for (int s = 0; s < NSUB; ++s) {
      const float* Lr = Ls + (16 * s + li) * LDL + 16 * g;
      float lw[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 t = *reinterpret_cast<const float4*>(Lr + 4 * q);
        lw[4 * q] = t.x;
        lw[4 * q + 1] = t.y;
        lw[4 * q + 2] = t.z;
        lw[4 * q + 3] = t.w;
      }
#pragma unroll
      for (int c = 0; c < 16; ++c) a12[s] = mfma16(lw[c], uv[c], a12[s]);
    }
  }
  v4f U[NSUB];
#pragma unroll
  for (int s = 0, q0 = 0; s < NSUB; q0 += s, ++s) {
    v4f acc = a12[s];
#pragma unroll
    for (int t = 0; t < s; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc = mfma16(-lv[q0 + t][v], U[t][v], acc);
    v4f u = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int v = 0; v < 4; ++v) u = mfma16(xv[s][v], acc[v], u);
    U[s] = u;
  }
  if (16 * wave + li < ncol) {
#pragma unroll
    for (int s = 0; s < NSUB; ++s)
#pragma unroll
      for (int v = 0; v < 4; ++v) Wb[(int64_t)(r0 + 16 * s + 4 * g + v) * N + cstart + 16 * wave + li] = U[s][v];
  }
}

// (sign, logabs) from the pivots (B, N) and the swap counts (B, nblk); one wave per
// matrix. Also flags matrices with an exactly zero pivot (zero_out, optional).
__global__ void lu_finish_kernel(const float* __restrict__ piv, const int* __restrict__ nsw, int N,
                                 int nblk, float* __restrict__ sign, float* __restrict__ logabs,
                                 int64_t batch) {
  const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (b >= batch) return;
  float lg = 0.0f;
  bool z = false, ng = false;
  for (int i = lane; i < N; i += 64) {
    const float v = piv[b * N + i];
    z = z || (v == 0.0f);
    ng = ng != (v < 0.0f);
    lg += (v != 0.0f) ? logf(fabsf(v)) : 0.0f;
  }
  lg = wave_sum_f32(lg);
  int sw = 0;
  for (int k = lane; k < nblk; k += 64) sw += nsw[b * nblk + k];
  sw = (int)wave_sum_f32((float)sw);
  const bool anyz = __ballot(z) != 0ull;
  const int negs = __popcll(__ballot(ng)) + sw;
  if (lane == 0) {
    sign[b] = anyz ? 0.0f : ((negs & 1) ? -1.0f : 1.0f);
    logabs[b] = anyz ? -INFINITY : lg;
  }
}

__global__ void iota_kernel(int* g0, int N, int64_t total) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < total) g0[e] = (int)(e % N);
}

int lu_large_padded(int n) { return ((n + 63) / 64) * 64; }

// Panel width: 64 columns (the trailing products run at K = 64).
static int lu_panel_width(int) { return 64; }

size_t lu_large_workspace(int64_t batch, int n, bool parts, bool external) {
  const int N = lu_large_padded(n);
  const int PW = lu_panel_width(N);
  const int nblk = N / PW;
  size_t bytes = 0;
  auto add = [&](size_t x) { bytes += (x + 255) / 256 * 256; };
  if (!external) add((size_t)batch * N * N * 4);  // W
  add((size_t)batch * N * 4);            // pivots
  add((size_t)batch * nblk * 4);         // swap counts
  add((size_t)batch * N * 4);            // src (even blocks)
  add((size_t)batch * N * 4);            // src (odd blocks)
  add((size_t)batch * N * 4);            // composed map of the first block pair
  add((size_t)batch * (PW / 16) * 1024); // X
  if (parts && !external) add((size_t)batch * N * 4);  // g0
  return bytes;
}

typedef float v16f __attribute__((ext_vector_type(16)));

// The trailing update A22 -= L21 U12 over K = 64 KC columns from r0 (KC = 1: one block,
// KC = 2: a block pair whose first update was deferred), on the 64 x 64 tiles of rows
// >= r1 = r0 + 64 KC and of ntc tile columns from r1. Every K chunk of 64 is one LDS
// stage; the first chunk's L21 rows and U12 columns are loaded up front, the next chunk's
// while the current chunk's MFMAs run, and the products -L21 U12 are summed in
// accumulators of their own, C read and added in fp32 at the end.
// A0 (first block pair, in place of the input copy): C of position p is input row
// rmapC[p].
// XCD-aware tile order when the batch is a multiple of 8 (one matrix's L21 / U12 fetched
// into one L2).
// X3 (split-bf16x3): each staged element is split once into three bf16 planes (48 KiB,
// three workgroups per CU) and each K = 16 slice is six bf16 MFMAs on 16-byte operand
// reads: measured 11 % faster than splitting at the point of use.
template <int KC, bool X3 = false>
__global__ __launch_bounds__(256, X3 ? 3 : 4) void lu_update_kernel(float* __restrict__ W, int N, int r0, int ntc,
                                                        const float* __restrict__ A0, const int* __restrict__ rmapC) {
  constexpr int LDA_ = 64 + 1, LDB_ = 64 + 4;
  // fp32: the L21 chunk (i, k) and the U12 chunk (k, j); X3: three split bf16 planes of
  // -L21 (rows i) and of U12 (rows j), 64 k per row
  constexpr int XP = 64 * 64;
  constexpr int SMEM = X3 ? 2 * 3 * XP * 2 : (64 * LDA_ + 64 * LDB_) * 4;
  __shared__ __align__(16) char smem[SMEM];
  float* const As = reinterpret_cast<float*>(smem);
  float* const Bs = As + 64 * LDA_;
  __bf16* const xA = reinterpret_cast<__bf16*>(smem);
  __bf16* const xB = xA + 3 * XP;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  int64_t b = blockIdx.y;
  int tx = blockIdx.x;
  if ((gridDim.y & 7) == 0) {
    const int64_t lin = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
    const int64_t slot = lin >> 3;
    tx = (int)(slot % gridDim.x);
    b = (slot / gridDim.x) * 8 + (lin & 7);
  }
  float* Wb = W + b * (int64_t)N * N;  // offsets below are 32-bit (N * N < 2^31)
  const int r1 = r0 + 64 * KC;
  const int i0 = r1 + 64 * (tx / ntc), j0 = r1 + 64 * (tx % ntc);
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  const int l32 = lane & 31, lh = lane >> 5;
  // staging of one chunk: thread (r = e / 16, q = 4 (e % 16)) of e = tid + 256 u holds
  // L21 (i0 + r, q .. q+3) and U12 (r, j0 + q .. q+3) of the chunk; float arrays stay in
  // registers. X3 takes U12 column-wise instead: thread (j = tid % 64, kq = tid / 64)
  // holds U12 (16 u + 4 kq .. +3, j0 + j), so that each staged group is four
  // consecutive k of one column.
  float av[16], bw[16];
  // the products' accumulators, added to C (in acc) at the end: the MFMAs truncate what
  // they add to an accumulator below about three bits under its last place, so products
  // summed on their own lose far less than products added to C one by one (measured at
  // n = 4160: logabs error 1.1e-4 -> 1.7e-5 for the bf16x3 mode). fp32 mode: xhh only;
  // X3: hi*hi in xhh, the smaller terms in xsm.
  v16f xhh, xsm;
#pragma unroll
  for (int v = 0; v < 16; ++v) xhh[v] = xsm[v] = 0.0f;
  auto load = [&](int c) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e = tid + 256 * u, r = e >> 4, q = 4 * (e & 15);
      const float4 x = *reinterpret_cast<const float4*>(Wb + (i0 + r) * N + r0 + 64 * c + q);
      av[4 * u] = x.x;
      av[4 * u + 1] = x.y;
      av[4 * u + 2] = x.z;
      av[4 * u + 3] = x.w;
      if constexpr (X3) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          bw[4 * u + t] = Wb[(r0 + 64 * c + 16 * u + 4 * (tid >> 6) + t) * N + j0 + (tid & 63)];
      } else {
        const float4 y = *reinterpret_cast<const float4*>(Wb + (r0 + 64 * c + r) * N + j0 + q);
        bw[4 * u] = y.x;
        bw[4 * u + 1] = y.y;
        bw[4 * u + 2] = y.z;
        bw[4 * u + 3] = y.w;
      }
    }
  };
  load(0);
#pragma unroll
  for (int c = 0; c < KC; ++c) {
    if (c > 0) __syncthreads();  // every wave is done with the previous chunk
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e = tid + 256 * u, r = e >> 4, q = 4 * (e & 15);
      if constexpr (X3) {
        const float na[4] = {-av[4 * u], -av[4 * u + 1], -av[4 * u + 2], -av[4 * u + 3]};
        const float nb[4] = {bw[4 * u], bw[4 * u + 1], bw[4 * u + 2], bw[4 * u + 3]};
        x3_put<XP>(xA, x3_off64(r, q), na);
        x3_put<XP>(xB, x3_off64(tid & 63, 16 * u + 4 * (tid >> 6)), nb);
      } else {
        float* pa = As + r * LDA_ + q;
        pa[0] = av[4 * u];
        pa[1] = av[4 * u + 1];
        pa[2] = av[4 * u + 2];
        pa[3] = av[4 * u + 3];
        *reinterpret_cast<float4*>(Bs + r * LDB_ + q) = make_float4(bw[4 * u], bw[4 * u + 1], bw[4 * u + 2], bw[4 * u + 3]);
      }
    }
    __syncthreads();
    if (c + 1 < KC) load(c + 1);
    if constexpr (X3) {
      // split-bf16x3: four K = 16 slices, lane operands the eight k = 16 q + 8 lh + u of
      // its row of -L21 and its column of U12, one 16-byte read per plane; the products
      // in their own accumulators (hi*hi and the smaller terms), added to C at the end
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        bf16x8 pa[3], pb[3];
        x3_get<XP>(xA, x3_off64(wm + l32, 16 * q + 8 * lh), pa);
        x3_get<XP>(xB, x3_off64(wn + l32, 16 * q + 8 * lh), pb);
        mfma_bf16x3_2(pa, pb, xhh, xsm);
      }
    } else {
#pragma unroll
      for (int kp = 0; kp < 32; ++kp)
        xhh = __builtin_amdgcn_mfma_f32_32x32x2f32(-As[(wm + l32) * LDA_ + 2 * kp + lh],
                                                   Bs[(2 * kp + lh) * LDB_ + wn + l32], xhh, 0, 0, 0);
    }
  }
  // C, read after the products (its registers are free during them)
  v16f acc;
  if (A0) {
    const float* Ab = A0 + b * (int64_t)N * N;
    const int* rb = rmapC + b * N;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = Ab[rb[i0 + wm + 8 * (v >> 2) + 4 * lh + (v & 3)] * N + j0 + wn + l32];
  } else {
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = Wb[(i0 + wm + 8 * (v >> 2) + 4 * lh + (v & 3)) * N + j0 + wn + l32];
  }
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] += X3 ? xhh[v] + xsm[v] : xhh[v];
#pragma unroll
  for (int v = 0; v < 16; ++v) Wb[(i0 + wm + 8 * (v >> 2) + 4 * lh + (v & 3)) * N + j0 + wn + l32] = acc[v];
}

// Grid of the trailing update: ntr x ntc tiles per matrix, batches of at most 65535.
template <int KC>
static int launch_update(float* W, int N, int64_t batch, int r0, int ntr, int ntc, const float* A0,
                         const int* rmapC, hipStream_t s, int x3) {
  const int64_t NN = (int64_t)N * N;
  for (int64_t b0 = 0; b0 < batch; b0 += 65535) {
    const int64_t nb = batch - b0 < 65535 ? batch - b0 : 65535;
    if (x3)
      hipLaunchKernelGGL((lu_update_kernel<KC, true>), dim3(ntr * ntc, (unsigned)nb), dim3(256), 0, s, W + b0 * NN, N,
                         r0, ntc, A0 ? A0 + b0 * NN : nullptr, rmapC ? rmapC + b0 * N : nullptr);
    else
      hipLaunchKernelGGL((lu_update_kernel<KC, false>), dim3(ntr * ntc, (unsigned)nb), dim3(256), 0, s, W + b0 * NN, N,
                         r0, ntc, A0 ? A0 + b0 * NN : nullptr, rmapC ? rmapC + b0 * N : nullptr);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  }
  return FX_OK;
}

// MR: the largest m of the matrix's panels; panels with m > 1024 (MR > 1024 only) use
// lu_panel_kernel with NT threads, the others lu_panel_reg_kernel.
//
// Blocks go in pairs (r0, r0 + 64): after the first block's U rows, only the next 64
// columns get its update (the second panel's columns); the second block's U rows take
// the first block's update themselves, and one K = 128 update then applies both blocks
// to the trailing matrix, at twice the arithmetic intensity of two K = 64 updates (the
// update is bound by reading and writing the trailing matrix at K = 64). The second
// panel moves the first block's L columns along with the rows it moves, so both blocks'
// L columns are in the final row order for the U-row correction and the K = 128 update.
// The panels' row maps alternate between srcs[0] (even blocks) and srcs[1] (odd); the
//
// The batch may be split over two streams (hv[0] on the caller's stream, hv[1] on the side
// stream, ordered after hv[0]'s first panel): the blocks are enqueued alternately, half by
// half, so a half's panel runs beside the other half's U rows and update.
struct LuHalf {
  float* W;
  float* piv;
  int* nsw;
  int* srcs[3];
  float* X;
  int* g0;
  const float* A_in;  // the input, read in place of a copy (direct), else nullptr
  int64_t batch;
  hipStream_t s;
};

template <int MR, int NT>
static int run_blocks(int N, const LuHalf* hv, int nh, bool fact, int x3, bool paired, SideStream* side) {
  constexpr int PW = 64;
  const int nblk = N / PW;
  constexpr int MAXM = MR < 1024 ? 1024 : MR;
  auto urow = [&](const LuHalf& H, int r0, const int* src, int lfirst, int nleft, int nright, const float* A0,
                  const int* rmap, int rc, int* comp) {
    if (nleft + nright == 0) return FX_OK;
    hipLaunchKernelGGL((lu_urow_kernel<PW, MAXM>), dim3(nleft + nright, (unsigned)H.batch), dim3(256), 0, H.s, H.W,
                       N, r0, src, H.X, lfirst, nleft, A0, rmap, rc, comp);
    return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
  };
  for (int blk = 0; blk < nblk; ++blk) {
    for (int h = 0; h < nh; ++h) {
      const LuHalf& H = hv[h];
      const hipStream_t s = H.s;
      const int r0 = blk * PW;
      const int m = N - r0;
      int* src = H.srcs[blk & 1];
      const float* A0 = blk == 0 ? H.A_in : nullptr;  // input read in place of a copy
      const int lmove = paired && (blk & 1);  // a pair's second panel moves the first block's L along
      if (m <= 1024) {
#define FX_PANEL_REG(T)                                                                                   \
  hipLaunchKernelGGL((lu_panel_reg_kernel<T>), dim3((unsigned)H.batch), dim3(T), 0, s, H.W, N, r0, blk, \
                     H.piv, H.nsw, nblk, src, H.X, H.g0, A0, lmove)
        if (m <= 64) FX_PANEL_REG(64);
        else if (m <= 128) FX_PANEL_REG(128);
        else if (m <= 256) FX_PANEL_REG(256);
        else if (m <= 512) FX_PANEL_REG(512);
        else FX_PANEL_REG(1024);
#undef FX_PANEL_REG
      } else if constexpr (MR > 1024) {
        hipLaunchKernelGGL((lu_panel_kernel<MR, PW, NT>), dim3((unsigned)H.batch), dim3(NT), 0, s, H.W, N, r0, blk,
                           H.piv, H.nsw, nblk, src, H.X, H.g0, lmove);
      }
      if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
      if (blk == 0 && h == 0 && nh == 2 && side->fork() != FX_OK) return FX_ERR_LAUNCH;
      const int nright = (N - r0 - PW) / 64;  // trailing strips / tile rows (N a multiple of 64)
      int st;
      if (!paired) {
        st = urow(H, r0, src, 0, fact ? r0 / 64 : 0, nright, A0, nullptr, -1, nullptr);
        if (st == FX_OK && nright > 0)
          st = launch_update<1>(H.W, N, H.batch, r0, nright, nright, A0, A0 ? src : nullptr, s, x3);
      } else if ((blk & 1) == 0) {
        // first block of a pair: U rows, then the update of the next panel's columns only
        st = urow(H, r0, src, 0, fact ? r0 / 64 : 0, nright, A0, nullptr, -1, nullptr);
        if (st == FX_OK && nright > 0)
          st = launch_update<1>(H.W, N, H.batch, r0, nright, 1, A0, A0 ? src : nullptr, s, x3);
      } else {
        // second block: U rows with the first block's deferred update, then both blocks'
        // update of the trailing matrix; the first pair reads the input through both maps
        const int rp = r0 - PW;
        const float* Ain = blk == 1 ? H.A_in : nullptr;
        st = urow(H, r0, src, 0, fact ? rp / 64 : 0, nright, Ain, Ain ? H.srcs[0] : nullptr, rp,
                  Ain && nright > 0 ? H.srcs[2] : nullptr);
        if (st == FX_OK && nright > 0)
          st = launch_update<2>(H.W, N, H.batch, rp, nright, nright, Ain, Ain ? H.srcs[2] : nullptr, s, x3);
      }
      if (st != FX_OK) return st;
    }
  }
  return FX_OK;
}

// Factor a (B, n, n) into the workspace; returns the packed LU (B, N, N) through *W_out
// and the composed row map g0 (parts only) through *g0_out.
int launch_lu_large(const float* A, int n, int64_t batch, float* sign, float* logabs, void* ws,
                    size_t ws_bytes, bool parts, float** W_out, int** g0_out, hipStream_t s, float* W_ext,
                    int* g0_ext, int x3, int lu_block, bool split) {
  const int N = lu_large_padded(n);
  const int PW = lu_panel_width(N);
  const int nblk = N / PW;
  if (N > LU_LARGE_MAXN) return FX_ERR_UNSUPPORTED;
  const bool external = W_ext != nullptr;
  if (external && parts && !g0_ext) return FX_ERR_INVALID_ARGUMENT;
  if (ws_bytes < lu_large_workspace(batch, n, parts, external) || !ws) return FX_ERR_WORKSPACE;
  char* p = (char*)ws;
  auto take = [&](size_t x) {
    char* q = p;
    p += (x + 255) / 256 * 256;
    return (void*)q;
  };
  float* W = external ? W_ext : (float*)take((size_t)batch * N * N * 4);
  float* piv = (float*)take((size_t)batch * N * 4);
  int* nsw = (int*)take((size_t)batch * nblk * 4);
  int* const srcs[3] = {(int*)take((size_t)batch * N * 4), (int*)take((size_t)batch * N * 4),
                        (int*)take((size_t)batch * N * 4)};
  float* X = (float*)take((size_t)batch * (PW / 16) * 1024);
  int* g0 = parts ? (external ? g0_ext : (int*)take((size_t)batch * N * 4)) : nullptr;
  // No padding and panels held in registers throughout (N <= 1024): the first block's
  // kernels read the input directly and together write all of W, so no copy is made.
  // Otherwise the input is copied (identity-padded) into W first.
  const fx_tune& tn = tune();
  const bool direct = n == N && N <= tn.lu_direct_max_n && N <= 1024 && ((uintptr_t)A & 15) == 0;
  // block pairs (one K = 128 update per pair) per the call's option, else the table (at
  // N <= 256 the pairs' extra launches and U-row correction cost more than they save)
  const bool paired = lu_block == FX_LU_BLOCK_128 || (lu_block != FX_LU_BLOCK_64 && N > tn.lu_pair_above_n);
  if (!direct) {
    if (n == N && ((uintptr_t)A & 15) == 0) {  // no padding: a straight streaming copy
      const int st = launch_copy(A, W, batch * (int64_t)N * N, s);
      if (st != FX_OK) return st;
    } else {
      const int64_t tot = (int64_t)N * N;
      hipLaunchKernelGGL(copy_pad_kernel, dim3((unsigned)((tot + 255) / 256), (unsigned)batch), dim3(256),
                         0, s, A, n, W, N);
      if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
    }
  }
  if (g0) {
    const int64_t tot = batch * N;
    hipLaunchKernelGGL(iota_kernel, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, g0, N, tot);
  }
  // Batches with batch N^2 >= fx_tune.lu_split_min_work 2^20 run as two halves side by side
  // (see run_blocks) for N <= 4096 (above, the halves' panels lose more than the overlap
  // gains); every kernel works per matrix, so the results are the same bits. The
  // no-allocation entry point passes split = false.
  const bool halves = split && batch >= 2 && N <= 4096 && tn.lu_split_min_work > 0 &&
                      (double)batch * N * N >= (double)tn.lu_split_min_work * (1 << 20);
  SideStream side(s, halves);
  const int nh = side.ok() ? 2 : 1;
  const int64_t hb = (batch + nh - 1) / nh;
  LuHalf hv[2];
  for (int h = 0; h < nh; ++h) {
    const int64_t b0 = h * hb;
    LuHalf& H = hv[h];
    H.W = W + b0 * (int64_t)N * N;
    H.piv = piv + b0 * N;
    H.nsw = nsw + b0 * nblk;
    for (int k = 0; k < 3; ++k) H.srcs[k] = srcs[k] + b0 * N;
    H.X = X + b0 * (PW / 16) * 256;
    H.g0 = g0 ? g0 + b0 * N : nullptr;
    H.A_in = direct ? A + b0 * (int64_t)N * N : nullptr;
    H.batch = h + 1 < nh ? hb : batch - b0;
    H.s = h == 0 ? s : side.side();
  }
  int st;
  if (N <= 1024)
    st = run_blocks<1024, 0>(N, hv, nh, parts, x3, paired, &side);
  else if (N <= 2048)
    st = run_blocks<2048, 512>(N, hv, nh, parts, x3, paired, &side);
  else if (N <= 4096)
    st = run_blocks<4096, 1024>(N, hv, nh, parts, x3, paired, &side);
  else
    st = run_blocks<8192, 1024>(N, hv, nh, parts, x3, paired, &side);
  if (st != FX_OK) return st;
  if (side.join() != FX_OK) return FX_ERR_LAUNCH;
  hipLaunchKernelGGL(lu_finish_kernel, dim3((unsigned)((batch + 3) / 4)), dim3(256), 0, s, piv, nsw, N,
                     nblk, sign, logabs, batch);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  if (W_out) *W_out = W;
  if (g0_out) *g0_out = g0;
  return FX_OK;
}

}  // namespace fx
