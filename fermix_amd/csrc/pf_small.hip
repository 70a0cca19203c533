// Fused slogpf for even n <= 128: one workgroup (4 waves) per matrix, blocked Parlett-Reid
// with partial pivoting in blocks of 8 pair steps, the skew matrix resident in LDS as its
// strictly lower triangle.
//
// Reference roles replaced (ChenAo-Phys/fermix): the pair-step panel
// (src/fermix/_pf.py:59-284) and the rank-2b trailing update (_pf.py:287-382), issued by
// the reference as 7 launches at n = 128 (_pf.py:516-570); here one launch. The pivoting
// and sign conventions are those of the generic path (_fallback.py:266-300): in pair
// step c the pivot is the largest |entry| of column c among the unassigned rows (ties:
// lowest row), it is swapped into position c+1 (a non-trivial swap flips the sign),
// d = M[c, c+1], tau = -M[:, c] / d and w = M[:, c+1] on the rows after c+1, and the
// trailing matrix becomes M + tau w^T - w tau^T.
//
// LDS (N = 128: exactly 40 KiB, so four matrices share a CU):
//   * T: M[p][q] for p > q at T[p (p - 1) / 2 + q]; M[q][p] = -M[p][q], M[p][p] = 0;
//   * Gs (directly after T): the block's tau / w vectors, 16 per row, stored as four
//     column groups Gs[k / 4][row][k % 4], so one row's group is a 16-byte vector at a
//     constant offset from the row's first group and 16 consecutive rows' groups cover
//     all 64 banks;
//   * src (position -> row at block start) and orig (FACT: row -> original row), bytes.
//
// Per block (positions from r0; rows stored in block-start order):
//   * wave 0 runs 8 pair steps (lane l owns rows l + 64 s). Column a and column p of the
//     current matrix are the block-start matrix plus the G corrections
//     sum_u tau_u[i] w_u[q] - w_u[i] tau_u[q]; the G row of a / p is read back from Gs as
//     an LDS broadcast; the permutation stays virtual;
//   * all waves then form the trailing block M'' = M + G J G^T (J = diag of
//     [[0,1],[-1,0]]) on fp32 MFMA 16x16x4 over the lower-triangle tiles, gathered through
//     the block's permutation and stored in the new order.
// The load reads each matrix once in 4 x 4 block pairs and forms (A - A^T) / 2 in
// registers (n == N).
// With FACT every block's G is exported indexed by the original row index, with the
// pivots d and the final position -> original row map (the factors of P S P^T = L D L^T).
//
// Padding n < N uses the blocks [[0,1],[-1,0]] (Pfaffian exactly +1).
#include "common.h"
#include "fermix_internal.h"

namespace fx {

template <int N>
struct PfSmall {
  static constexpr int R = (N + 63) / 64;                        // panel rows per lane
  static constexpr int NTRI = N * (N - 1) / 2;                   // strictly lower triangle
  static constexpr int NB = N / 16;
  static constexpr int NPV = (N / 2 + 63) / 64;                  // pivot slots per lane
  static constexpr int LDS_BYTES = NTRI * 4 + N * 16 * 4 + 2 * N;
};
static_assert(PfSmall<128>::LDS_BYTES <= 40960, "four n = 128 workgroups per CU");

// Start of row p of the strictly lower triangle (a 24-bit multiply: one VALU
// instruction per lane).
__device__ __forceinline__ int tri_row(int p) { return (int)(__umul24((unsigned)p, (unsigned)(p - 1)) >> 1); }
// Byte offset of row p: 4 p (p - 1) / 2 = p (2 p - 2), formed as one shift-add and one 24-bit
// multiply (p (p - 1) is even, so no rounding or masking is involved).
__device__ __forceinline__ unsigned tri_row_b(int p) { return __umul24((unsigned)p, (unsigned)(2 * p - 2)); }

// Index of G element (row s, column k) in Gs.
template <int N>
__device__ __forceinline__ int g_idx(int s, int k) { return (k >> 2) * (4 * N) + 4 * s + (k & 3); }

// Lowest set row of a per-slot ballot pair: slot s holds rows l + 64 s.
// Slots below S0 hold no candidate.
template <int R, int S0>
__device__ __forceinline__ int first_row(const unsigned long long (&b)[R]) {
  if constexpr (R - S0 == 1) {
    return 64 * S0 + (int)__builtin_ctzll(b[S0]);
  } else {
    return b[0] ? (int)__builtin_ctzll(b[0]) : 64 + (int)__builtin_ctzll(b[1]);
  }
}

// S0: first slot with rows >= r0 (rows l + 64 s with s < S0 are all finished).
//
// The step is one wave's instruction stream (one instruction per four cycles at best), so
// it is written for few instructions: byte offsets precomputed per lane, the next row's
// column and G row read before the pivot search (independent of it, so their LDS latency
// overlaps the reduction), stores unpredicated where every lane row exists. Without FACT
// the finished rows' tau / w are left as computed: they only enter the corrections of
// finished rows, whose values nothing reads; FACT exports them, as zeros.
template <int N, bool FACT, int S0>
__device__ __forceinline__ void pf_panel(const float* T, float* Gs, int r0, unsigned char* src, int lane,
                                         PivotLog<PfSmall<N>::NPV>& piv_log, int& nsw,
                                         unsigned char* orig, float* gbuf_k, float* d_k) {
  constexpr int R = PfSmall<N>::R;
  constexpr bool ALL = N == 64 * R;  // every lane row exists
  // lane-derived addresses are recomputed per block instead of held across the loop
  asm volatile("" : "+v"(lane));
  const char* const Tb = reinterpret_cast<const char*>(T);
  float G[R][16];
  int pos[R], rop4[R], row4[R];
  bool valid[R];
#pragma unroll
  for (int i = S0; i < R; ++i) {
    const int row = lane + 64 * i;
    valid[i] = (row >= r0) && (ALL || row < N);
    pos[i] = valid[i] ? row : -1;  // finished / absent rows never match a position >= r0
    rop4[i] = (ALL || row < N) ? 4 * tri_row(row) : 0;
    row4[i] = 4 * row;
#pragma unroll
    for (int k = 0; k < 16; ++k) G[i][k] = 0.0f;
  }
  // M[row][q] of the block-start matrix for the lane's rows (value for row == q unused)
  auto column = [&](int q, float (&v)[R]) {
    const int q4 = 4 * q, roq4 = q * (2 * q - 2);  // 4 tri_row(q)
#pragma unroll
    for (int i = S0; i < R; ++i) {
      const bool below = row4[i] > q4;
      // row == q == N-1 addresses T[NTRI], the first entry of Gs (value unused)
      const float t = *reinterpret_cast<const float*>(Tb + (below ? rop4[i] + q4 : roq4 + row4[i]));
      v[i] = below ? t : -t;
    }
  };
  // the first 2t entries of Gs row q, broadcast to every lane
  auto grow = [&](int q, float (&g)[16], auto tc) {
    constexpr int t = decltype(tc)::value;
    static_for<0, (2 * t + 3) / 4>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      const float4 v = *reinterpret_cast<const float4*>(Gs + 4 * q + j * (4 * N));
      g[4 * j] = v.x;
      g[4 * j + 1] = v.y;
      g[4 * j + 2] = v.z;
      g[4 * j + 3] = v.w;
    });
  };
  // the row at position c (wave-uniform)
  auto row_at = [&](int c) {
    unsigned long long b[R];
#pragma unroll
    for (int i = S0; i < R; ++i) b[i] = __ballot(pos[i] == c);
    return first_row<R, S0>(b);
  };
  // v += sum_{u < U} G[.][2u] gq[2u+1] - G[.][2u+1] gq[2u], in order of u
  auto correct = [&](float (&v)[R], const float (&gq)[16], auto uc) {
    constexpr int U = decltype(uc)::value;
#pragma unroll
    for (int i = S0; i < R; ++i) {
      static_for<0, U>([&](auto wc) {
        constexpr int u = decltype(wc)::value;
        v[i] = fmaf(G[i][2 * u], gq[2 * u + 1], v[i]);
        v[i] = fmaf(G[i][2 * u + 1], -gq[2 * u], v[i]);
      });
    }
  };
  // Row a of step t and its current column x are carried from step t - 1: before step
  // t - 1 searches its pivot, the row at position c + 2 is read and corrected with the
  // finished G columns; unless the pivot swap moved that row, only step t - 1's own term
  // is added afterwards (from the owner lane's registers, same order of operations).
  int qa = row_at(r0);
  float x[R];
  column(qa, x);
  static_for<0, 8>([&](auto tc) {
    constexpr int t = decltype(tc)::value;
    const int c = r0 + 2 * t;
    // speculative next row a, its G row and column, read before the pivot search
    const int qn = t < 7 ? row_at(c + 2) : 0;
    float gn[16], xn[R];
    if constexpr (t < 7) {
      grow(qn, gn, tc);
      column(qn, xn);
    }
    unsigned key[R], kb = 0;
#pragma unroll
    for (int i = S0; i < R; ++i) {
      key[i] = cand_key(x[i], pos[i] > c);
      kb = max(kb, key[i]);
    }
    // the position of the lane's own candidate, selected before the reduction: on the
    // pivot lane the winning slot is the lowest one holding the lane's maximum (if any
    // row l < 64 holds the wave's maximum, the pivot is such a row; otherwise no slot-0
    // key reaches it), so the pivot's position is one readlane once the lane is known
    int bpos = pos[R - 1];
#pragma unroll
    for (int i = R - 2; i >= S0; --i) bpos = key[i] == kb ? pos[i] : bpos;
    const unsigned gk = wave_max_u32(kb);
    unsigned long long bp[R];
#pragma unroll
    for (int i = S0; i < R; ++i) bp[i] = __ballot(key[i] == gk);
    const int qp = first_row<R, S0>(bp);
    const int lp = qp & 63;
    const int pp = readlane_i(bpos, lp);
    float gp[16], y[R];
    grow(qp, gp, tc);
    column(qp, y);
    correct(y, gp, tc);
    const int la = qa & 63, sa = qa >> 6;
    float yv = y[S0];  // M[a][p] = y at row a
#pragma unroll
    for (int i = S0 + 1; i < R; ++i) yv = (sa == i) ? y[i] : yv;
    const float d = readlane_f(yv, la);
    piv_log.put(c >> 1, d, lane);
#pragma unroll
    for (int i = S0; i < R; ++i) {
      const int row = lane + 64 * i;
      if (pos[i] == c + 1) pos[i] = pp;
      if (row == qp) pos[i] = c + 1;
    }
    nsw += (pp != c + 1) ? 1 : 0;
    const float inv = safe_rcp(d);
#pragma unroll
    for (int i = S0; i < R; ++i) {
      const int row = lane + 64 * i;
      if constexpr (FACT) {
        const bool act = pos[i] > c + 1;
        G[i][2 * t] = act ? -x[i] * inv : 0.0f;
        G[i][2 * t + 1] = act ? y[i] : 0.0f;
      } else {
        G[i][2 * t] = -x[i] * inv;
        G[i][2 * t + 1] = y[i];
      }
      if (ALL || row < N)
        *reinterpret_cast<float2*>(Gs + g_idx<N>(row, 2 * t)) = make_float2(G[i][2 * t], G[i][2 * t + 1]);
    }
    wave_lds_fence();
    if (FACT && lane == 0) d_k[t] = d;
    if constexpr (t < 7) {
      correct(xn, gn, tc);
      if (pp != c + 2) {
        const int ln = qn & 63, sn = qn >> 6;
        float g0 = G[S0][2 * t], g1 = G[S0][2 * t + 1];
#pragma unroll
        for (int i = S0 + 1; i < R; ++i) {
          g0 = (sn == i) ? G[i][2 * t] : g0;
          g1 = (sn == i) ? G[i][2 * t + 1] : g1;
        }
        const float h0 = readlane_f(g0, ln), h1 = readlane_f(g1, ln);
#pragma unroll
        for (int i = S0; i < R; ++i) {
          x[i] = fmaf(G[i][2 * t], h1, xn[i]);
          x[i] = fmaf(G[i][2 * t + 1], -h0, x[i]);
        }
        qa = qn;
      } else {
        qa = row_at(c + 2);
        float ga[16];
        grow(qa, ga, ic<t + 1>{});
        column(qa, x);
        correct(x, ga, ic<t + 1>{});
      }
    }
  });
#pragma unroll
  for (int i = S0; i < R; ++i)
    if (valid[i]) src[pos[i]] = (unsigned char)(lane + 64 * i);
  if (FACT) {
    int ov[R];
#pragma unroll
    for (int i = S0; i < R; ++i) ov[i] = valid[i] ? orig[lane + 64 * i] : 0;
#pragma unroll
    for (int i = S0; i < R; ++i) {
      if (valid[i]) {
        float4* gr = reinterpret_cast<float4*>(gbuf_k + ov[i] * 16);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          gr[j] = make_float4(G[i][4 * j], G[i][4 * j + 1], G[i][4 * j + 2], G[i][4 * j + 3]);
      }
    }
    wave_lds_fence();
#pragma unroll
    for (int i = S0; i < R; ++i)
      if (valid[i]) orig[pos[i]] = (unsigned char)ov[i];
  }
  wave_lds_fence();
}

// Load of a full N x N matrix (n == N) into T in one pass over 4 x 4 block pairs: pair
// (I, J), I >= J, owns T(p, q) for p in rows 4I..4I+3, q in columns 4J..4J+3, p > q. A
// thread reads the block A[I][J] as four 16-byte rows and, with skew, the transposed block
// A[J][I] the same way, and forms every entry in registers: T(p, q) = A[p][q] / 2 -
// A[q][p] / 2 (fma(-A[q][p], 1/2, A[p][q] / 2): halving is exact, one rounding), or
// A[p][q] without skew. No LDS read-modify-write and no barrier. Pairs are numbered by
// folded block rows: rows f and NB4 - 1 - f together hold NB4 + 1 pairs, so consecutive
// threads read consecutive 16-byte pieces of the same rows of A[I][J].
template <int N>
__device__ __forceinline__ void pf_load_full(float* T, const float* __restrict__ g, int skew, int tid) {
  constexpr int NB4 = N / 4;
  static_assert(NB4 % 2 == 0, "folded block rows");
  constexpr int NPAIR = NB4 * (NB4 + 1) / 2;
  constexpr int ITER = (NPAIR + 255) / 256;
  float4 lo[ITER][4], up[ITER][4];
  int bi[ITER], bj[ITER];
#pragma unroll
  for (int it = 0; it < ITER; ++it) {
    const int t = tid + 256 * it;
    const int f = t / (NB4 + 1), x = t - f * (NB4 + 1);
    bi[it] = x <= f ? f : NB4 - 1 - f;
    bj[it] = x <= f ? x : x - f - 1;
    if (NPAIR % 256 == 0 || t < NPAIR) {
      const float4* a = reinterpret_cast<const float4*>(g + (4 * bi[it]) * N + 4 * bj[it]);
      const float4* u = reinterpret_cast<const float4*>(g + (4 * bj[it]) * N + 4 * bi[it]);
#pragma unroll
      for (int i = 0; i < 4; ++i) lo[it][i] = a[i * (N / 4)];
      if (skew && bi[it] != bj[it]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) up[it][i] = u[i * (N / 4)];
      }
    }
  }
#pragma unroll
  for (int it = 0; it < ITER; ++it) {
    const int t = tid + 256 * it;
    if (NPAIR % 256 == 0 || t < NPAIR) {
      const int p0 = 4 * bi[it], q0 = 4 * bj[it];
      float v[4][4];  // v[i][j] = T(p0 + i, q0 + j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float r[4] = {lo[it][i].x, lo[it][i].y, lo[it][i].z, lo[it][i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) v[i][j] = r[j];
      }
      if (bi[it] != bj[it]) {
        if (skew) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float c[4] = {up[it][j].x, up[it][j].y, up[it][j].z, up[it][j].w};  // A[q0 + j][p0 + i]
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i][j] = fmaf(-c[i], 0.5f, v[i][j] * 0.5f);
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float* d = T + tri_row(p0 + i) + q0;
#pragma unroll
          for (int j = 0; j < 4; ++j) d[j] = v[i][j];
        }
      } else {
        // diagonal block: T(p0 + i, p0 + j) for i > j; the transposed entries are this
        // block's own
#pragma unroll
        for (int i = 1; i < 4; ++i) {
          float* d = T + tri_row(p0 + i) + q0;
#pragma unroll
          for (int j = 0; j < i; ++j) d[j] = skew ? fmaf(-v[j][i], 0.5f, v[i][j] * 0.5f) : v[i][j];
        }
      }
    }
  }
}

// Load the matrix (row-major n x n, n even) into T, padded with [[0,1],[-1,0]] blocks;
// with skew, T holds (A - A^T) / 2 formed as A[p][q] / 2 - A[q][p] / 2 (halving is exact).
template <int N>
__device__ __forceinline__ void pf_load(float* T, const float* __restrict__ g, int n, int skew, int tid) {
  const float h = skew ? 0.5f : 1.0f;
  if (n == N) {
    pf_load_full<N>(T, g, skew, tid);
    return;
  }
  {
    // lower triangle (every entry written once), then the upper halves subtracted
    constexpr int CH = 8;
    for (int base = 0; base < N * N; base += 256 * CH) {
      float v[CH];
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int e = base + tid + 256 * u;
        const int r = e / N, c = e % N;
        v[u] = (e < N * N && r < n && c < r) ? g[r * n + c] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int e = base + tid + 256 * u;
        const int r = e / N, c = e % N;
        // padding: M[2m+1][2m] = -1 below the n x n block
        if (e < N * N && c < r)
          T[tri_row(r) + c] = (r < n) ? v[u] * h : ((c == r - 1 && (r & 1)) ? -1.0f : 0.0f);
      }
    }
    if (skew) {
      __syncthreads();
      for (int base = 0; base < N * N; base += 256 * CH) {
        float v[CH];
#pragma unroll
        for (int u = 0; u < CH; ++u) {
          const int e = base + tid + 256 * u;
          const int r = e / N, c = e % N;
          v[u] = (e < N * N && c < n && r < c) ? g[r * n + c] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < CH; ++u) {
          const int e = base + tid + 256 * u;
          const int r = e / N, c = e % N;
          if (e < N * N && c < n && r < c) {
            float* d = T + tri_row(c) + r;
            *d = *d - v[u] * 0.5f;
          }
        }
      }
    }
  }
}

// Trailing update of one block: M'' = M + G J G^T (J = diag of [[0,1],[-1,0]]) over the
// lower-triangle 16 x 16 tiles of the positions >= rb, fp32 MFMA 16x16x4. Entry (P, Q) of
// the new order is read as M_old(src[P], src[Q]) from the triangle (negated when stored
// transposed) and written in place at (P, Q); G is indexed by block-start row.
// No barrier separates the reads from the stores: an entry whose row and column both stay
// in place is read and rewritten by the same lane, and every other old entry lies in a row
// or column of the block just factored (positions r0..rb-1), which this update never
// writes. Tiles t = wv, wv + 4, ... (row-major over (I, J), I >= J) go to wave wv, two per
// iteration so the second tile's LDS reads overlap the first's; (I, J) advance in scalar
// registers.
template <int N>
__device__ __forceinline__ void pf_update(float* T, const float* Gs, const unsigned char* src, int rb, int nt, int wv,
                                          int li, int g) {
  const int ntiles = nt * (nt + 1) / 2;
  int I = wv == 0 ? 0 : (wv < 3 ? 1 : 2);
  int J = wv - I * (I + 1) / 2;
  auto advance = [&]() {
    J += 4;
    while (J > I) {
      J -= I + 1;
      ++I;
    }
  };
  struct Tile {
    int P0, Q0, sq, sr;
    unsigned sp4;
    float raw[4];
    float4 ga, gb;
  };
  auto read_src = [&](Tile& x) {
    x.sp4 = *reinterpret_cast<const unsigned*>(src + x.P0 + 4 * g);
    x.sq = src[x.Q0 + li];
    x.sr = src[x.P0 + li];
  };
  const char* const Tb = reinterpret_cast<const char*>(T);
  auto read_old = [&](Tile& x) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      // branch-free addressing: the entry lives in the row of the larger index
      const int sv = (x.sp4 >> (8 * v)) & 0xFF;
      const int hi = max(sv, x.sq), lo = min(sv, x.sq);
      // p == q (diagonal tiles; never stored) may address T[NTRI], the first entry of Gs
      x.raw[v] = *reinterpret_cast<const float*>(Tb + tri_row_b(hi) + 4 * lo);
    }
    x.ga = *reinterpret_cast<const float4*>(Gs + g_idx<N>(x.sr, 4 * g));
    x.gb = *reinterpret_cast<const float4*>(Gs + g_idx<N>(x.sq, 4 * g));
  };
  // MFMA step u contracts k = 4 g + u, so each lane's A and B operands are one 16-byte G
  // row group; (J G^T)[k] = G[k+1] (k even), -G[k-1] (k odd)
  auto finish = [&](const Tile& x) {
    // the entry is stored at (row, column) when its row index is the larger, else negated
    v4f acc;
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[v] = (int)((x.sp4 >> (8 * v)) & 0xFF) > x.sq ? x.raw[v] : -x.raw[v];
    acc = mfma16(x.ga.x, x.gb.y, acc);
    acc = mfma16(x.ga.y, -x.gb.x, acc);
    acc = mfma16(x.ga.z, x.gb.w, acc);
    acc = mfma16(x.ga.w, -x.gb.z, acc);
    const int q = x.Q0 + li;
    int p0 = x.P0 + 4 * g;
    asm volatile("" : "+v"(p0));  // no known-bits masking in front of the 24-bit multiply
    // tri_row(p0 + v) = tri_row(p0) + v p0 + v (v - 1) / 2, in bytes
    char* const e0 = reinterpret_cast<char*>(T) + tri_row_b(p0) + 4 * q;
    auto st = [&](int off, float val) { *reinterpret_cast<float*>(e0 + off) = val; };
    if (x.P0 != x.Q0) {
      st(0, acc[0]);
      st(4 * p0, acc[1]);
      st(8 * p0 + 4, acc[2]);
      st(12 * p0 + 12, acc[3]);
    } else {
      // entries on or above the diagonal go to T[0] instead (M[1][0]: position 1 is
      // finished before the first update, which starts at position 16, and never read
      // again), so the stores need no per-element branch
      char* const dead = reinterpret_cast<char*>(T);
      auto sd = [&](bool keep, int off, float val) { *reinterpret_cast<float*>(keep ? e0 + off : dead) = val; };
      sd(p0 > q, 0, acc[0]);
      sd(p0 + 1 > q, 4 * p0, acc[1]);
      sd(p0 + 2 > q, 8 * p0 + 4, acc[2]);
      sd(p0 + 3 > q, 12 * p0 + 12, acc[3]);
    }
  };
  for (int t = wv; t < ntiles; t += 8) {
    Tile a, b;
    a.P0 = rb + 16 * I;
    a.Q0 = rb + 16 * J;
    advance();
    const bool two = t + 4 < ntiles;
    b.P0 = rb + 16 * I;
    b.Q0 = rb + 16 * J;
    advance();
    read_src(a);
    if (two) read_src(b);
    read_old(a);
    if (two) read_old(b);
    finish(a);
    if (two) finish(b);
  }
}

template <int N, bool FACT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void pf_small_kernel(const float* __restrict__ A, int n, int skew,
                                                       float* __restrict__ sign_out,
                                                       float* __restrict__ logabs_out,
                                                       float* __restrict__ gbuf_out,
                                                       float* __restrict__ d_out,
                                                       int* __restrict__ perm_out) {
  using C = PfSmall<N>;
  constexpr int NB = C::NB;
  __shared__ __align__(16) float lds[C::NTRI + N * 16];  // T, then Gs (NTRI * 4 % 16 == 0)
  float* const T = lds;
  float* const Gs = lds + C::NTRI;
  __shared__ __align__(16) unsigned char src[N];
  __shared__ unsigned char orig[FACT ? N : 1];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  pf_load<N>(T, A + b * (int64_t)n * n, n, skew, tid);
  if (FACT)
    for (int r = tid; r < N; r += 256) orig[r] = (unsigned char)r;
  __syncthreads();

  PivotLog<C::NPV> piv_log;
  piv_log.init();
  int nsw = 0;
  for (int k = 0; k < NB; ++k) {
    const int r0 = 16 * k;
    if (wave == 0) {
      float* gk = FACT ? gbuf_out + (b * NB + k) * (int64_t)N * 16 : nullptr;
      float* dk = FACT ? d_out + b * (N / 2) + 8 * k : nullptr;
      if (C::R == 2 && r0 >= 64)
        pf_panel<N, FACT, C::R - 1>(T, Gs, r0, src, lane, piv_log, nsw, orig, gk, dk);
      else
        pf_panel<N, FACT, 0>(T, Gs, r0, src, lane, piv_log, nsw, orig, gk, dk);
    }
    const int nt = (N - r0 - 16) / 16;
    if (nt == 0) break;
    __syncthreads();
    const int rb = r0 + 16;
    int li = lane & 15, g = lane >> 4, wv = __builtin_amdgcn_readfirstlane(wave);
    asm volatile("" : "+v"(li), "+v"(g), "+s"(wv));
    pf_update<N>(T, Gs, src, rb, nt, wv, li, g);
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
    __syncthreads();
    for (int r = tid; r < N; r += 256) perm_out[b * N + r] = orig[r];
  }
}

template <int N, bool FACT>
static int launch_n(const float* A, int n, int skew, int64_t batch, float* sign, float* logabs,
                    float* gbuf, float* d, int* perm, hipStream_t s) {
  hipLaunchKernelGGL((pf_small_kernel<N, FACT>), dim3((unsigned)batch), dim3(256), 0, s, A, n, skew,
                     sign, logabs, gbuf, d, perm);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

int pf_small_padded(int n) { return ((n + 15) / 16) * 16; }

template <bool FACT>
static int dispatch(const float* A, int n, int skew, int64_t batch, float* sign, float* logabs,
                    float* gbuf, float* d, int* perm, hipStream_t s) {
  switch (pf_small_padded(n)) {
    case 32: return launch_n<32, FACT>(A, n, skew, batch, sign, logabs, gbuf, d, perm, s);
    case 48: return launch_n<48, FACT>(A, n, skew, batch, sign, logabs, gbuf, d, perm, s);
    case 64: return launch_n<64, FACT>(A, n, skew, batch, sign, logabs, gbuf, d, perm, s);
    case 80: return launch_n<80, FACT>(A, n, skew, batch, sign, logabs, gbuf, d, perm, s);
    case 96: return launch_n<96, FACT>(A, n, skew, batch, sign, logabs, gbuf, d, perm, s);
    case 112: return launch_n<112, FACT>(A, n, skew, batch, sign, logabs, gbuf, d, perm, s);
    case 128: return launch_n<128, FACT>(A, n, skew, batch, sign, logabs, gbuf, d, perm, s);
    default: return FX_ERR_UNSUPPORTED;
  }
}

int launch_pf_small(const float* A, int n, int skew, int64_t batch, float* sign, float* logabs,
                    float* gbuf, float* d, int* perm, hipStream_t s) {
  if (n <= PF_TINY_MAXN) return launch_pf_tiny(A, n, skew, batch, sign, logabs, gbuf, d, perm, s);
  if (gbuf) return dispatch<true>(A, n, skew, batch, sign, logabs, gbuf, d, perm, s);
  return dispatch<false>(A, n, skew, batch, sign, logabs, nullptr, nullptr, nullptr, s);
}

}  // namespace fx
