// Fused slogdet for 32 < n <= 128: one workgroup (4 waves) per matrix, blocked
// right-looking LU with partial pivoting in 16-column panels in LDS. Up to N = 64 the
// whole matrix is resident (lu_small_kernel); from N = 80 on, lu_split_kernel factors
// the left block in LDS, forms the Schur complement of the right block on MFMA straight
// from global memory and factors it in the same LDS, so a matrix needs about half the
// LDS (40,448 bytes at N = 128) and four workgroups share a CU instead of two.
//
// Reference roles replaced (ChenAo-Phys/fermix): the LU inner panel (src/fermix/_lu.py:
// 54-224), the inter-panel and U-row updates (_lu.py:228-330) and the trailing GEMM
// (_lu.py:334-393), which the reference issues as 26 separate launches at n = 128
// (_lu.py:543-611); here they are one launch.
//
// Per panel k (rows/cols from r0 = 16k):
//   * wave 0 factors the m x 16 panel in registers (lane l owns rows R*l .. R*l+R-1):
//     pivot = largest |a| among the unassigned rows (ties: lowest row), found with a
//     DPP max over order-preserving integer keys; rows are pivoted virtually inside
//     the panel and written back in the new order; it then forms X = L11^-1 from the
//     stored L11 (lane c holds column c) and the map src[new position] = old row;
//   * the trailing 16-column strips are gathered through src, U12 = X * A12 and
//     A22 -= L21 * U12 run on fp32 MFMA 16x16x4, and the strip is stored in the new row
//     order (each strip is read completely before it is written, and strips own
//     disjoint columns, so the permutation is applied in place);
//   * look-ahead: wave 0 updates strip 0 (the next panel's columns) itself and factors
//     the next panel while waves 1-3 update the remaining strips.
// With FACT the left (already factored) columns are permuted along, so the LDS holds
// the packed LU of P A in the final row order, and the composed permutation is kept.
//
// n < N is padded with the identity (exact: [[A,0],[0,I]] = [[L,0],[0,I]][[U,0],[0,I]]).
#include "common.h"
#include "fermix_internal.h"

namespace fx {

template <int N>
struct LuSmall {
  static constexpr int LDA = N + 4;        // row stride in LDS (floats)
  static constexpr int R = (N + 63) / 64;  // panel rows per lane
  static constexpr int NP = N / 16;        // panels
  static constexpr int NPV = (N + 63) / 64;  // pivot slots per lane
};

// Factor the 16-column panel at (r0, r0) of an NR-row matrix in LDS (row stride LDA;
// wave 0 only). Accumulates the pivot signs, log|pivot|, zero-pivot flag and swap count
// into the wave-uniform state; pivot positions are logged from pbase on.
template <int NR, int LDA, bool FACT, int NPV>
__device__ __forceinline__ void lu_panel(float* As, int r0, int* src, float* X, int* perm,
                                         int lane, PivotLog<NPV>& piv_log, int& nsw, int pbase = 0) {
  constexpr int R = (NR + 63) / 64;
  float a[R][16];
  int pos[R];
  bool valid[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int row = R * lane + i;
    valid[i] = (row >= r0) && (row < NR);
    pos[i] = row;
#pragma unroll
    for (int j = 0; j < 16; ++j) a[i][j] = valid[i] ? As[row * LDA + r0 + j] : 0.0f;
  }
  static_for<0, 16>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    const int posc = r0 + j;
    unsigned kb = 0;
    int ib = 0;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const unsigned k = cand_key(a[i][j], valid[i] && pos[i] >= posc);
      if (k > kb) { kb = k; ib = i; }
    }
    // each lane's best slot's row (columns j .. 15) and position, selected before the
    // reduction (off the dependency chain: the pivot lane's values are then one readlane
    // away); the row's columns < j (row j of L11) are read back from LDS for X after the
    // panel, so no scalar register holds them across the step
    float brow[16];
    int bpos = pos[0];
    static_for<j, 16>([&](auto cc) {
      float v = a[0][cc.value];
#pragma unroll
      for (int i = 1; i < R; ++i) v = (ib == i) ? a[i][cc.value] : v;
      brow[cc.value] = v;
    });
#pragma unroll
    for (int i = 1; i < R; ++i) bpos = (ib == i) ? pos[i] : bpos;
    const unsigned gk = wave_max_u32(kb);
    const int pl = first_lane(kb == gk);
    float u[16];
    static_for<j, 16>([&](auto cc) { u[cc.value] = readlane_f(brow[cc.value], pl); });
    const int pp = readlane_i(bpos, pl);
    // swap positions posc <-> pp (the pivot row is the pivot lane's best slot)
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (valid[i] && pos[i] == posc) pos[i] = pp;
      if (lane == pl && i == ib) pos[i] = posc;
    }
    nsw += (pp != posc) ? 1 : 0;
    const float piv = u[j];
    piv_log.put(pbase + posc, piv, lane);
    const float rcp = safe_rcp(piv);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (valid[i] && pos[i] > posc) {
        const float l = a[i][j] * rcp;
        a[i][j] = l;
        static_for<j + 1, 16>([&](auto cc) {
          a[i][cc.value] = fmaf(-l, u[cc.value], a[i][cc.value]);
        });
      }
    }
  });
  // write the panel back in the new row order and the position map
#pragma unroll
  for (int i = 0; i < R; ++i) {
    if (valid[i]) {
#pragma unroll
      for (int j = 0; j < 16; ++j) As[pos[i] * LDA + r0 + j] = a[i][j];
      src[pos[i]] = R * lane + i;
    }
  }
  wave_lds_fence();
  // X = L11^-1 from the unit lower L11 just stored (lane c holds column c):
  // X[j][c] = -sum_{k<j} L11[j][k] X[k][c] in order of k, X[j][j] = 1
  {
    const float* L11 = As + r0 * LDA + r0;
    float xcol[16];
    static_for<0, 16>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      float x = 0.0f;
      static_for<0, j>([&](auto kc) { x = fmaf(-L11[j * LDA + kc.value], xcol[kc.value], x); });
      xcol[j] = (lane == j) ? 1.0f : x;
    });
    if (lane < 16) {
#pragma unroll
      for (int k = 0; k < 16; ++k) X[k * 16 + lane] = xcol[k];
    }
  }
  if (FACT) {
    int pv[R];
#pragma unroll
    for (int i = 0; i < R; ++i) pv[i] = valid[i] ? perm[R * lane + i] : 0;
    wave_lds_fence();
#pragma unroll
    for (int i = 0; i < R; ++i)
      if (valid[i]) perm[pos[i]] = pv[i];
  }
  wave_lds_fence();
}

// Update one trailing strip (columns c0 .. c0+15, rows r0 .. NR-1) of an NR-row matrix
// in LDS (row stride LDA): gather the rows through src, U12 = X * A12,
// A22 -= L21 * U12 (fp32 MFMA), store in the new order.
template <int NR, int LDA>
__device__ __forceinline__ void lu_strip(float* As, int r0, int c0, const int* src, const float* X,
                                         int lane) {
  constexpr int MAXT = (NR / 16 > 1) ? NR / 16 - 1 : 1;
  const int nt = (NR - r0 - 16) / 16;
  const int li = lane & 15, g = lane >> 4;
  const int col = c0 + li;
  float tb[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) tb[t] = As[__umul24(src[r0 + 4 * t + g], LDA) + col];
  v4f ct[MAXT];
#pragma unroll
  for (int i = 0; i < MAXT; ++i) {
    if (i < nt) {
#pragma unroll
      for (int v = 0; v < 4; ++v) ct[i][v] = As[__umul24(src[r0 + 16 + 16 * i + 4 * g + v], LDA) + col];
    }
  }
  v4f u = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int t = 0; t < 4; ++t) u = mfma16(X[li * 16 + 4 * t + g], tb[t], u);
#pragma unroll
  for (int v = 0; v < 4; ++v) As[(r0 + 4 * g + v) * LDA + col] = u[v];
  wave_lds_fence();
  // -U12, negated once here rather than L21 in every product
  float ub[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) ub[t] = -As[(r0 + 4 * t + g) * LDA + col];
#pragma unroll
  for (int i = 0; i < MAXT; ++i) {
    if (i < nt) {
      const int rb = r0 + 16 + 16 * i;
#pragma unroll
      for (int t = 0; t < 4; ++t) ct[i] = mfma16(As[(rb + li) * LDA + r0 + 4 * t + g], ub[t], ct[i]);
#pragma unroll
      for (int v = 0; v < 4; ++v) As[(rb + 4 * g + v) * LDA + col] = ct[i][v];
    }
  }
}

// Apply the panel's row permutation to a strip of already factored columns (rows r0 ..
// NR-1, row stride LDA).
template <int NR, int LDA>
__device__ __forceinline__ void lu_permute_strip(float* As, int r0, int c0, const int* src, int lane) {
  // 8 columns per pass (lane & 7), rows r0 + g + 8 i: NR / 8 values per lane in flight
  constexpr int MAXR = NR / 8;
  const int g = lane >> 3;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int col = c0 + 8 * h + (lane & 7);
    float v[MAXR];
#pragma unroll
    for (int i = 0; i < MAXR; ++i) {
      const int p = r0 + g + 8 * i;
      if (p < NR) v[i] = As[__umul24(src[p], LDA) + col];
    }
    wave_lds_fence();
#pragma unroll
    for (int i = 0; i < MAXR; ++i) {
      const int p = r0 + g + 8 * i;
      if (p < NR) As[p * LDA + col] = v[i];
    }
    wave_lds_fence();
  }
}

template <int N, bool FACT>
__global__ __launch_bounds__(256) void lu_small_kernel(const float* __restrict__ A, int n,
                                                       float* __restrict__ sign_out,
                                                       float* __restrict__ logabs_out,
                                                       float* __restrict__ lu_out,
                                                       int* __restrict__ perm_out) {
  constexpr int LDA = LuSmall<N>::LDA, NP = LuSmall<N>::NP;
  __shared__ float As[N * LDA];
  __shared__ int srcs[2][N];
  __shared__ float Xs[2][256];
  __shared__ int perm[N];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const float* Ab = A + b * (int64_t)n * n;
  load_tile<N, LDA, 256>(As, Ab, n, tid, [](int r, int c) { return r == c ? 1.0f : 0.0f; });
  if (FACT)
    for (int r = tid; r < N; r += 256) perm[r] = r;
  __syncthreads();

  PivotLog<LuSmall<N>::NPV> piv_log;
  piv_log.init();
  int nsw = 0;
  if (wave == 0) lu_panel<N, LDA, FACT>(As, 0, srcs[0], Xs[0], perm, lane, piv_log, nsw);
  __syncthreads();
  for (int k = 0; k < NP; ++k) {
    const int r0 = 16 * k;
    const int S = NP - 1 - k;
    const int* src = srcs[k & 1];
    const float* X = Xs[k & 1];
    if (wave == 0) {
      if (S > 0) {
        lu_strip<N, LDA>(As, r0, r0 + 16, src, X, lane);
        lu_panel<N, LDA, FACT>(As, r0 + 16, srcs[(k + 1) & 1], Xs[(k + 1) & 1], perm, lane, piv_log,
                               nsw);
      }
    } else {
      for (int s = wave; s < S; s += 3) lu_strip<N, LDA>(As, r0, r0 + 16 + 16 * s, src, X, lane);
      if (FACT)
        for (int q = wave - 1; q < k; q += 3) lu_permute_strip<N, LDA>(As, r0, 16 * q, src, lane);
    }
    __syncthreads();
  }
  if (wave == 0) {
    float sg, la;
    piv_log.finish(nsw, sg, la);
    if (lane == 0) {
      sign_out[b] = sg;
      logabs_out[b] = la;
    }
  }
  if (FACT) {
    float* Lb = lu_out + b * (int64_t)N * N;
    for (int e = tid; e < N * N; e += 256) {
      const int r = e / N, c = e - r * N;
      Lb[e] = As[r * LDA + c];
    }
    for (int r = tid; r < N; r += 256) perm_out[b * N + r] = perm[r];
  }
}

// Forward-only slogdet with about half the LDS of lu_small_kernel (so twice the
// matrices per CU), in three phases over A = [[A1, A2]] split after column H:
//   1. the N x H left block is factored in LDS exactly as above (panels, strips,
//      look-ahead), its factored columns permuted along, so it ends as the packed
//      [[L11 \ U11], [L21]] of P A1 in the final row order, with perm = P;
//   2. the Schur complement S = (P A)22 - L21 U12 with U12 = L11^-1 (P A)12 is formed on
//      MFMA straight from global memory, one 16-column chunk per wave (the rows gathered
//      through perm), U12 by blocked forward substitution with the panels' X = L_ss^-1,
//      and kept in registers until every wave has read L;
//   3. S ((N-H) x (N-H)) goes to LDS in place of the left block's first rows and is
//      factored the same way; its pivots continue the log from position H.
// With FACT the packed LU of P A and P are written as by lu_small_kernel: L11 \ U11 after
// phase 1, U12 from phase 2's registers, and L21 -- which stays in the left block's last
// N - H rows, clear of S -- permuted along with S's rows in phase 3.
// Products whose right operand sits in accumulator layout (lane (g, c) holding rows
// 4g + v of a 16 x 16 tile) take it as it stands, one MFMA per v over the K indices
// {4g + v}, with the left operand read from LDS in that order.
// Four workgroups per CU: at most 128 registers per lane (the compiler fits 111 without
// scratch at N = 128) and 40,448 bytes of LDS.
template <int N, int H, bool FACT>
__global__ __launch_bounds__(256, 4) void lu_split_kernel(const float* __restrict__ A, int n,
                                                          float* __restrict__ sign_out,
                                                          float* __restrict__ logabs_out,
                                                          float* __restrict__ lu_out,
                                                          int* __restrict__ perm_out) {
  constexpr int LDH = H + 4;           // left block row stride
  constexpr int NS = N - H;            // Schur complement order
  constexpr int LDS_ = NS + 4;         // its row stride
  constexpr int NPH = H / 16, NPS = NS / 16;
  constexpr int NPV = (N + 63) / 64;
  static_assert(H % 16 == 0 && NS % 16 == 0 && NPS <= 4 && NS <= H, "split shape");
  static_assert(NS * LDS_ <= H * LDH, "S must not reach the rows of L21");
  __shared__ float As[N * LDH];        // N x H left block, later the NS x NS complement
  __shared__ int srcs[2][N];
  __shared__ float Xall[NPH][256];     // X = L_ss^-1 of every left panel (phase 2)
  __shared__ int perm[N];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const float* Ab = A + b * (int64_t)n * n;
  float* Lb = FACT ? lu_out + b * (int64_t)N * N : nullptr;

  // phase 1: the left block, identity-padded beyond n
  if (n == N) {
    constexpr int NV = N * H / 4, PER = (NV + 255) / 256;
    float4 v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = tid + 256 * i;
      if (NV % 256 == 0 || e < NV) v[i] = *reinterpret_cast<const float4*>(Ab + (e / (H / 4)) * N + 4 * (e % (H / 4)));
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = tid + 256 * i;
      if (NV % 256 == 0 || e < NV) {
        float* d = As + (e / (H / 4)) * LDH + 4 * (e % (H / 4));
        d[0] = v[i].x;
        d[1] = v[i].y;
        d[2] = v[i].z;
        d[3] = v[i].w;
      }
    }
  } else {
    for (int e = tid; e < N * H; e += 256) {
      const int r = e / H, c = e % H;
      As[r * LDH + c] = (r < n && c < n) ? Ab[r * n + c] : (r == c ? 1.0f : 0.0f);
    }
  }
  for (int r = tid; r < N; r += 256) perm[r] = r;
  __syncthreads();
  PivotLog<NPV> piv_log;
  piv_log.init();
  int nsw = 0;
  if (wave == 0) lu_panel<N, LDH, true>(As, 0, srcs[0], Xall[0], perm, lane, piv_log, nsw);
  __syncthreads();
  for (int k = 0; k < NPH; ++k) {
    const int r0 = 16 * k;
    const int S = NPH - 1 - k;
    const int* src = srcs[k & 1];
    const float* X = Xall[k];
    if (wave == 0) {
      if (S > 0) {
        lu_strip<N, LDH>(As, r0, r0 + 16, src, X, lane);
        lu_panel<N, LDH, true>(As, r0 + 16, srcs[(k + 1) & 1], Xall[k + 1], perm, lane, piv_log, nsw);
      }
    } else {
      for (int s = wave; s < S; s += 3) lu_strip<N, LDH>(As, r0, r0 + 16 + 16 * s, src, X, lane);
      for (int q = wave - 1; q < k; q += 3) lu_permute_strip<N, LDH>(As, r0, 16 * q, src, lane);
    }
    __syncthreads();
  }

  if (FACT) {
    // rows 0 .. H-1 of the left block are final: L11 \ U11
    for (int e = tid; e < H * H; e += 256) Lb[(e / H) * N + e % H] = As[(e / H) * LDH + e % H];
  }

  // phase 2: wave w forms columns H + 16w .. H + 16w + 15 of S
  const int li = lane & 15, g = lane >> 4;
  v4f Sc[NPS];
  if (wave < NPS) {
    const int c = H + 16 * wave + li;
    auto elem = [&](int p) {
      const int r = perm[p];
      return (r < n && c < n) ? Ab[__umul24(r, n) + c] : (r == c ? 1.0f : 0.0f);
    };
    v4f ap[NPH];
#pragma unroll
    for (int s = 0; s < NPH; ++s)
#pragma unroll
      for (int v = 0; v < 4; ++v) ap[s][v] = elem(16 * s + 4 * g + v);
#pragma unroll
    for (int q = 0; q < NPS; ++q)
#pragma unroll
      for (int v = 0; v < 4; ++v) Sc[q][v] = elem(H + 16 * q + 4 * g + v);
    // U12 = L11^-1 (P A)12 block by block: U_s = X_s (A_s - sum_{t<s} L_st U_t); the
    // products take -U (nU, negated once per block) rather than -L in every product
    v4f nU[NPH];
#pragma unroll
    for (int s = 0; s < NPH; ++s) {
      v4f acc = ap[s];
#pragma unroll
      for (int t = 0; t < s; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc = mfma16(As[(16 * s + li) * LDH + 16 * t + 4 * g + v], nU[t][v], acc);
      v4f u = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int v = 0; v < 4; ++v) u = mfma16(Xall[s][li * 16 + 4 * g + v], acc[v], u);
      nU[s] = -u;
      if (FACT) {
#pragma unroll
        for (int v = 0; v < 4; ++v) Lb[(16 * s + 4 * g + v) * N + c] = u[v];
      }
    }
    // S = (P A)22 - L21 U12
#pragma unroll
    for (int q = 0; q < NPS; ++q)
#pragma unroll
      for (int t = 0; t < NPH; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          Sc[q] = mfma16(As[(H + 16 * q + li) * LDH + 16 * t + 4 * g + v], nU[t][v], Sc[q]);
  }
  __syncthreads();  // every wave is done with L
  if (wave < NPS) {
#pragma unroll
    for (int q = 0; q < NPS; ++q)
#pragma unroll
      for (int v = 0; v < 4; ++v) As[(16 * q + 4 * g + v) * LDS_ + 16 * wave + li] = Sc[q][v];
  }
  __syncthreads();

  // phase 3: factor S, pivots logged from position H (with FACT, the rows of S and of
  // L21 keep one order and P composes over positions H .. N-1)
  float* const L21 = As + H * LDH;
  if (wave == 0) lu_panel<NS, LDS_, FACT>(As, 0, srcs[0], Xall[0], perm + H, lane, piv_log, nsw, H);
  __syncthreads();
  for (int k = 0; k < NPS; ++k) {
    const int r0 = 16 * k;
    const int S = NPS - 1 - k;
    const int* src = srcs[k & 1];
    const float* X = Xall[k & 1];
    if (wave == 0) {
      if (S > 0) {
        lu_strip<NS, LDS_>(As, r0, r0 + 16, src, X, lane);
        lu_panel<NS, LDS_, FACT>(As, r0 + 16, srcs[(k + 1) & 1], Xall[(k + 1) & 1], perm + H, lane, piv_log,
                                 nsw, H);
      }
    } else {
      for (int s = wave; s < S; s += 3) lu_strip<NS, LDS_>(As, r0, r0 + 16 + 16 * s, src, X, lane);
      if (FACT) {
        // S's factored strips and all of L21 follow the panel's row permutation
        for (int q = wave - 1; q < k + NPH; q += 3) {
          if (q < k) lu_permute_strip<NS, LDS_>(As, r0, 16 * q, src, lane);
          else lu_permute_strip<NS, LDH>(L21, r0, 16 * (q - k), src, lane);
        }
      }
    }
    __syncthreads();
  }
  if (wave == 0) {
    float sg, la;
    piv_log.finish(nsw, sg, la);
    if (lane == 0) {
      sign_out[b] = sg;
      logabs_out[b] = la;
    }
  }
  if (FACT) {
    // rows H .. N-1: L21 and the packed LU of S
    for (int e = tid; e < NS * N; e += 256) {
      const int r = e / N, c = e % N;
      Lb[(H + r) * N + c] = c < H ? L21[r * LDH + c] : As[r * LDS_ + c - H];
    }
    for (int r = tid; r < N; r += 256) perm_out[b * N + r] = perm[r];
  }
}

template <int N, bool FACT>
static int launch_n(const float* A, int n, int64_t batch, float* sign, float* logabs, float* lu,
                    int* perm, hipStream_t s) {
  hipLaunchKernelGGL((lu_small_kernel<N, FACT>), dim3((unsigned)batch), dim3(256), 0, s, A, n,
                     sign, logabs, lu, perm);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

int lu_small_padded(int n) { return ((n + 15) / 16) * 16; }

template <int N, int H, bool FACT>
static int launch_split(const float* A, int n, int64_t batch, float* sign, float* logabs, float* lu, int* perm,
                        hipStream_t s) {
  hipLaunchKernelGGL((lu_split_kernel<N, H, FACT>), dim3((unsigned)batch), dim3(256), 0, s, A, n, sign, logabs, lu,
                     perm);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

template <bool FACT>
static int dispatch(const float* A, int n, int64_t batch, float* sign, float* logabs, float* lu,
                    int* perm, hipStream_t s) {
  switch (lu_small_padded(n)) {
    case 80: return launch_split<80, 48, FACT>(A, n, batch, sign, logabs, lu, perm, s);
    case 96: return launch_split<96, 48, FACT>(A, n, batch, sign, logabs, lu, perm, s);
    case 112: return launch_split<112, 64, FACT>(A, n, batch, sign, logabs, lu, perm, s);
    case 128: return launch_split<128, 64, FACT>(A, n, batch, sign, logabs, lu, perm, s);
    default: break;
  }
  switch (lu_small_padded(n)) {
    case 48: return launch_n<48, FACT>(A, n, batch, sign, logabs, lu, perm, s);
    case 64: return launch_n<64, FACT>(A, n, batch, sign, logabs, lu, perm, s);
    default: return FX_ERR_UNSUPPORTED;
  }
}

int launch_lu_small(const float* A, int n, int64_t batch, float* sign, float* logabs, float* lu,
                    int* perm, hipStream_t s) {
  if (n <= TINY_MAXN) return launch_lu_tiny(A, n, batch, sign, logabs, lu, perm, s);
  if (lu) return dispatch<true>(A, n, batch, sign, logabs, lu, perm, s);
  return dispatch<false>(A, n, batch, sign, logabs, nullptr, nullptr, s);
}

}  // namespace fx
