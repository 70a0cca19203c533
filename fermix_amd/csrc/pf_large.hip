// Blocked Parlett-Reid with partial pivoting for 128 < n <= 8192 (any batch). The skew
// matrix lives in one workspace buffer as its strictly lower triangle, in strips of four
// rows stored column-major (entry (p, q), p > q, at ((p / 4) N + q) 4 + p % 4): an MFMA
// accumulator's four consecutive rows of one column are one 16-byte store, and a row of
// the skew matrix is its stored part (columns q < p, 16-byte strided) and the negated
// column below the diagonal (whole 16-byte strip pieces). Per block of PB columns (PB / 2
// pair steps; PB = 64 once the trailing order m = N - r0 is at most 1024 for N >= 512 a
// multiple of 64, else 32; 16 above N = 2048, 8 above N = 4096) at r0:
//   1. pf_panel_kernel (one workgroup of NT = 256..1024 threads per matrix, each lane
//      owning R = 1, 2, 4 or 8 of the m = N - r0 rows): the pair steps with the tau / w vectors
//      kept in registers as G (m x PB); column a and column p of the current matrix are read
//      as rows of the block-start matrix (skew) plus the G corrections; each pair step
//      has two workgroup barriers (the row at position c, the pivot). The permutation is
//      virtual inside the block; the kernel writes G in the block's new row order and
//      the map src[new position] = old row;
//   2. pf_update_kernel (matrix x lower-triangle 64x64 tile, in place):
//      M'' = M[src, src] + G J G^T on fp32 MFMA (K = PB), the old entries read through the
//      permutation (from the stored triangle, negated where the pair is transposed), the
//      new lower entries stored in the new order, four rows of a column per 16-byte
//      store; the upper half is never formed. In place is safe: a row that moves into a
//      trailing position comes from the block just factored, whose columns the update
//      never writes, and every other old entry is read by the lane that rewrites it.
// Reference roles replaced (ChenAo-Phys/fermix): _pf_run / _pf_core (src/fermix/_pf.py:
// 497-570), the pair-step panel (:59-284) and the rank-2b update (:287-382).
#include "common.h"
#include "fermix_internal.h"

namespace fx {

// Trailing-update tile: 64 x 64 (one 32x32 accumulator per wave) keeps eight waves per
// SIMD resident, against two for 128 x 128 tiles, and the in-place update streams
// M about 10 % faster at n = 1200 .. 2048.
constexpr int PF_UPDATE_TILE = 64;
constexpr int PFB_L = 64;   // columns per block (32 pair steps) where m <= 1024 (see pf_block_width)
constexpr int PFB = 32;     // the other blocks of N <= 2048
constexpr int PFB_XL = 16;  // every block of 2048 < N <= 4096
constexpr int PFB_XXL = 8;  // every block of 4096 < N <= PF_LARGE_MAXN (R = 8 rows per lane)

// Columns per chunk of the exported factors gbuf (B, N / CW, N, CW) for padded order N:
// the 32 (16 above N = 2048, 8 above 4096) columns of a block, or one half of a 64-column
// block.
int pf_large_block_cols(int N) { return N > 4096 ? PFB_XXL : N > 2048 ? PFB_XL : PFB; }

// Columns of the block at r0: 64 once the trailing order m = N - r0 is at most
// fx_tune.pf_block64_max_m (1024 in the table, the register limit: G (m x 64) in the
// registers of 256 / 512 threads; the trailing updates' HBM traffic halves), for N >=
// fx_tune.pf_block64_min_n (512) a multiple of 64, else 32; 16 above N = 2048, 8 above
// N = 4096 (G (m x PB) in the registers of a 1024-thread workgroup).
static int pf_block_width(int N, int r0) {
  if (N > 4096) return PFB_XXL;
  if (N > 2048) return PFB_XL;
  const fx_tune& t = tune();
  const int max_m = t.pf_block64_max_m < 1024 ? t.pf_block64_max_m : 1024;
  return (N >= t.pf_block64_min_n && N % PFB_L == 0 && N - r0 <= max_m && r0 % PFB_L == 0) ? PFB_L : PFB;
}

struct PfCand {
  unsigned key;
  int row;
  int pos;
  float xv;  // x at the candidate row (d = -x[p])
  float g[PFB_L];
};

struct PfRowA {
  int row;    // at position c
  int next1;  // at position c + 1
  int next2;  // at position c + 2
  int pad;
  float g[PFB_L];
};

// Offset of the stored entry (p, q), p > q, in a matrix of the lower-triangle strip
// layout (32-bit: N * N < 2^31).
__device__ __forceinline__ unsigned l4(int p, int q, int N) {
  return ((unsigned)(p >> 2) * (unsigned)N + (unsigned)q) * 4u + (unsigned)(p & 3);
}

// Copy a (B, n, n) into M (B, N, N) in the strip layout: S = (a - a^T)/2 (or a) with
// [[0,1],[-1,0]] padding, the strictly lower entries (the rest of each strip is never
// read; the diagonal tiles' upper entries are written as zeros). One workgroup per 64 x 64
// tile pair (I, J), I >= J: the blocks A[I][J] and, with skew, A[J][I] are read once each
// along their rows into LDS (each wave a 256-byte row segment), the entries formed there
// (fma(-A[c][r], 1/2, A[r][c] / 2): halving is exact, one rounding), and the strips of the
// tile written as 16-byte vectors -- four rows of one column are one strip piece, so a
// strip of the tile is 1 KiB of consecutive memory.
constexpr int PCT = 64;  // tile of the copy
__global__ __launch_bounds__(256) void pf_copy_pad_kernel(const float* __restrict__ A, int n, int skew,
                                                         float* __restrict__ M, int N) {
  __shared__ float Tl[PCT][PCT + 1], Tu[PCT][PCT + 1];
  const int64_t b = blockIdx.y;
  const int t = blockIdx.x;
  int I = (int)((sqrtf(8.0f * t + 1.0f) - 1.0f) * 0.5f);
  while ((I + 1) * (I + 2) / 2 <= t) ++I;
  while (I * (I + 1) / 2 > t) --I;
  const int J = t - I * (I + 1) / 2;
  const int r0 = PCT * I, c0 = PCT * J;
  const float* Ab = A + b * (int64_t)n * n;
  const int tid = threadIdx.x;
  // Tl[i][j] = A[r0 + i][c0 + j], Tu[j][i] = A[c0 + j][r0 + i] (0 outside the n x n input):
  // thread t reads columns 4 (t % 16) .. + 3 of rows t / 16 + 16 k, one 16-byte load per
  // row piece when the rows are 16-byte aligned (n % 4 == 0) and the piece is inside the
  // input, so each wave reads four 256-byte row segments per load, all eight in flight
  const int c4 = 4 * (tid & 15), rr = tid >> 4;
  const bool vec = (n & 3) == 0;
  float4 lo[4], up[4];
  auto ld4 = [&](int gr, int gc) {
    if (gr >= n) return make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float* p = Ab + (int64_t)gr * n + gc;
    if (vec && gc + 3 < n) return *reinterpret_cast<const float4*>(p);
    return make_float4(gc < n ? p[0] : 0.0f, gc + 1 < n ? p[1] : 0.0f, gc + 2 < n ? p[2] : 0.0f,
                       gc + 3 < n ? p[3] : 0.0f);
  };
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    lo[k] = ld4(r0 + rr + 16 * k, c0 + c4);
    if (skew) up[k] = ld4(c0 + rr + 16 * k, r0 + c4);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float* d = &Tl[rr + 16 * k][c4];
    d[0] = lo[k].x;
    d[1] = lo[k].y;
    d[2] = lo[k].z;
    d[3] = lo[k].w;
    if (skew) {
      float* e = &Tu[rr + 16 * k][c4];
      e[0] = up[k].x;
      e[1] = up[k].y;
      e[2] = up[k].z;
      e[3] = up[k].w;
    }
  }
  __syncthreads();
  float* Mb = M + b * (int64_t)N * N;
  // (strip s of the tile, column q): rows r0 + 4 s .. + 3 of column c0 + q
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int e = tid + 256 * u, s = e >> 6, q = e & 63;
    const int gr = r0 + 4 * s, gc = c0 + q;
    if (gr >= N || gc >= N) continue;
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = gr + k, i = 4 * s + k;
      float x;
      if (r <= gc) {
        x = 0.0f;  // upper entries of a diagonal tile: never read
      } else if (r < n && gc < n) {
        x = skew ? fmaf(-Tu[q][i], 0.5f, Tl[i][q] * 0.5f) : Tl[i][q];
      } else {
        x = ((r ^ gc) == 1 && r >= n) ? -1.0f : 0.0f;  // r odd, c = r - 1: M[r][r-1] = -1
      }
      v[k] = x;
    }
    *reinterpret_cast<float4*>(Mb + l4(gr, gc, N)) = make_float4(v[0], v[1], v[2], v[3]);
  }
}

// The panel of matrix b (one workgroup of NT threads; pf_panel_kernel, pf_step_kernel).
template <int NT, int R, int PB>
__device__ __forceinline__ void pf_panel_body(const float* __restrict__ M, int N, int r0, int nch,
                                              float* __restrict__ d_out, int* __restrict__ nsw_out,
                                              int* __restrict__ src_out, float* __restrict__ Gn,
                                              int* __restrict__ orig, float* __restrict__ gbuf, int full,
                                              int64_t b) {
  constexpr int NW = NT / 64;
  constexpr int CW = PB < 32 ? PB : 32;  // factor chunk width
  static_assert(PB % CW == 0 && PB / CW <= 2, "a block spans one or two chunks");
  __shared__ __align__(16) PfRowA rowa;
  __shared__ __align__(16) PfCand cand[2][NW];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int m = N - r0;
  // M[r0 + q][r0 + i] of the block-start matrix: the input itself in full storage (full:
  // the first block reading it in place of a copy), else the strip layout's triangle
  const float* Mm = M + b * (int64_t)N * N;
  // The lane's R consecutive entries M[r0 + q][r0 + R tid + s] (zero beyond m). r0 and m
  // are multiples of 8, so a lane's rows are whole strip pieces (R <= 4: one, R = 8: two
  // strips): the part below the diagonal (rows > r0 + q) is one 8- or 16-byte load per
  // strip, the part right of it R loads 16 bytes apart.
  typedef float vR __attribute__((ext_vector_type(R)));
  typedef float vS __attribute__((ext_vector_type(R < 4 ? R : 4)));
  constexpr int SR = R < 4 ? R : 4;  // rows of one strip piece
  auto rowr = [&](int q, float (&v)[R]) {
    const int i0 = R * tid;
    const int gq = r0 + q, gi = r0 + i0;
    if (i0 >= m) {
#pragma unroll
      for (int s = 0; s < R; ++s) v[s] = 0.0f;
    } else if (full) {
      const vR y = *reinterpret_cast<const vR*>(Mm + (unsigned)(gq * N + gi));
#pragma unroll
      for (int s = 0; s < R; ++s) v[s] = y[s];
    } else if (gi > gq) {
#pragma unroll
      for (int h = 0; h < R / SR; ++h) {
        const vS y = *reinterpret_cast<const vS*>(Mm + l4(gi + SR * h, gq, N));
#pragma unroll
        for (int s = 0; s < SR; ++s) v[SR * h + s] = -y[s];
      }
    } else if (gi + R <= gq) {
#pragma unroll
      for (int s = 0; s < R; ++s) v[s] = Mm[l4(gq, gi + s, N)];
    } else {
#pragma unroll
      for (int s = 0; s < R; ++s) {
        const int g = gi + s;
        const float y = Mm[l4(max(gq, g), min(gq, g), N)];
        v[s] = g < gq ? y : (g > gq ? -y : 0.0f);
      }
    }
  };
  float G[R][PB];
  int pos[R];
  bool valid[R];
#pragma unroll
  for (int s = 0; s < R; ++s) {
    const int i = R * tid + s;
    valid[s] = i < m;
    pos[s] = i;
#pragma unroll
    for (int k = 0; k < PB; ++k) G[s][k] = 0.0f;
  }
  int nsw = 0;
  float mv_next[R];  // row a of the next pair step, loaded ahead (see below)
  static_for<0, PB / 2>([&](auto tc) {
    constexpr int t = decltype(tc)::value;
    const int c = 2 * t;  // local position of row a
    // 1. the row at position c publishes its index and G row; the rows at c + 1 and c + 2
    //    their indices (the next step's row a is one of them)
#pragma unroll
    for (int s = 0; s < R; ++s) {
      if (valid[s] && pos[s] == c) {
        rowa.row = R * tid + s;
        // 16-byte stores; the columns from 2 t on are still zero and never read
#pragma unroll
        for (int k = 0; k < 2 * t; k += 4)
          *reinterpret_cast<float4*>(rowa.g + k) = make_float4(opaque(G[s][k]), opaque(G[s][k + 1]), opaque(G[s][k + 2]), opaque(G[s][k + 3]));
      }
      if (valid[s] && pos[s] == c + 1) rowa.next1 = R * tid + s;
      if (valid[s] && pos[s] == c + 2) rowa.next2 = R * tid + s;
    }
    __syncthreads();
    const int qa = rowa.row, qn1 = rowa.next1, qn2 = rowa.next2;
    const float* ga = rowa.g;
    // x = column a of the current matrix on my rows: M[i][qa] = -M[qa][i] + corrections
    float x[R];
    {
      float mv[R];
      if constexpr (t == 0) {
        rowr(qa, mv);
      } else {
#pragma unroll
        for (int s = 0; s < R; ++s) mv[s] = mv_next[s];
      }
#pragma unroll
      for (int s = 0; s < R; ++s) {
        float v = -mv[s];
#pragma unroll
        for (int u = 0; u < t; ++u) {
          v = fmaf(G[s][2 * u], ga[2 * u + 1], v);
          v = fmaf(-G[s][2 * u + 1], ga[2 * u], v);
        }
        x[s] = v;
      }
    }
    // 2. pivot: largest |x| among the rows after position c (ties: lowest row)
    unsigned kb = 0;
    int ib = 0;
#pragma unroll
    for (int s = 0; s < R; ++s) {
      const unsigned k = cand_key(x[s], valid[s] && pos[s] > c);
      if (k > kb) { kb = k; ib = s; }
    }
    const unsigned gk = wave_max_u32(kb);
    const int pl = first_lane(gk != 0u ? (kb == gk) : (lane == 0));
    PfCand& my = cand[t & 1][wave];
    if (lane == pl) {
      my.key = gk;
      my.row = R * tid + ib;
      // the winning slot's x, position and G row, written straight from that slot
#pragma unroll
      for (int s = 0; s < R; ++s) {
        if (ib == s) {
          my.pos = pos[s];
          my.xv = x[s];
#pragma unroll
          for (int k = 0; k < 2 * t; k += 4)
            *reinterpret_cast<float4*>(my.g + k) = make_float4(opaque(G[s][k]), opaque(G[s][k + 1]), opaque(G[s][k + 2]), opaque(G[s][k + 3]));
        }
      }
    }
    __syncthreads();
    unsigned best = cand[t & 1][0].key;
    int wb = 0;
    for (int w = 1; w < NW; ++w) {
      const unsigned kw = cand[t & 1][w].key;
      if (kw > best) { best = kw; wb = w; }
    }
    const PfCand& win = cand[t & 1][wb];
    const int qp = win.row, pp = win.pos;
    const float d = -win.xv;  // M[a][p] = -M[p][a]
    const float* gp = win.g;
#pragma unroll
    for (int s = 0; s < R; ++s) {
      if (valid[s] && pos[s] == c + 1) pos[s] = pp;
      if (R * tid + s == qp) pos[s] = c + 1;
    }
    nsw += (pp != c + 1) ? 1 : 0;
    pin(nsw);
    if (tid == 0) d_out[b * (N / 2) + (r0 >> 1) + t] = d;
    // the next step's row a sits at position c + 2 after this step's swap: the old row
    // at c + 1 if the pivot came from c + 2, else the row at c + 2. Its load goes out
    // now, beside the pivot row's (the block-start matrix is read-only in the panel).
    if constexpr (t + 1 < PB / 2) {
      const int qn = pp == c + 2 ? qn1 : qn2;
      rowr(qn, mv_next);
    }
    // y = column p on my rows
    float y[R];
    {
      float mv[R];
      rowr(qp, mv);
#pragma unroll
      for (int s = 0; s < R; ++s) {
        float v = -mv[s];
#pragma unroll
        for (int u = 0; u < t; ++u) {
          v = fmaf(G[s][2 * u], gp[2 * u + 1], v);
          v = fmaf(-G[s][2 * u + 1], gp[2 * u], v);
        }
        y[s] = v;
      }
    }
    const float inv = safe_rcp(d);
#pragma unroll
    for (int s = 0; s < R; ++s) {
      const bool act = valid[s] && pos[s] > c + 1;
      G[s][2 * t] = act ? -x[s] * inv : 0.0f;
      G[s][2 * t + 1] = act ? y[s] : 0.0f;
    }
  });
  // outputs: G in the new row order, the position map, factors by original row
#pragma unroll
  for (int s = 0; s < R; ++s) {
    const int i = R * tid + s;
    if (valid[s]) {
      float* gr = Gn + (b * N + r0 + pos[s]) * (int64_t)PB;
#pragma unroll
      for (int k = 0; k < PB; k += 4) *reinterpret_cast<float4*>(gr + k) = make_float4(G[s][k], G[s][k + 1], G[s][k + 2], G[s][k + 3]);
      src_out[b * N + r0 + pos[s]] = r0 + i;
    }
  }
  if (gbuf) {
    int* ob = orig + b * N;
    int ov[R];
#pragma unroll
    for (int s = 0; s < R; ++s) ov[s] = valid[s] ? ob[r0 + R * tid + s] : 0;
#pragma unroll
    for (int s = 0; s < R; ++s) {
      if (valid[s]) {
        // chunks of CW columns: chunk r0 / CW + k / CW, column k % CW
#pragma unroll
        for (int k = 0; k < PB; ++k)
          gbuf[((b * nch + r0 / CW + k / CW) * N + ov[s]) * (int64_t)CW + k % CW] = G[s][k];
      }
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < R; ++s)
      if (valid[s]) ob[r0 + pos[s]] = ov[s];
  }
  // swap count per chunk: positions of this block are local, every wave counted the same
  // swaps (a 64-column block's second chunk counts none)
  if (tid == 0) {
    nsw_out[b * nch + r0 / CW] = nsw;
    if (PB > CW) nsw_out[b * nch + r0 / CW + 1] = 0;
  }
}

template <int NT, int R, int PB>
__global__ __launch_bounds__(NT) void pf_panel_kernel(const float* __restrict__ M, int N, int r0, int nch,
                                                      float* __restrict__ d_out,
                                                      int* __restrict__ nsw_out,
                                                      int* __restrict__ src_out,
                                                      float* __restrict__ Gn,
                                                      int* __restrict__ orig,
                                                      float* __restrict__ gbuf, int full) {
  pf_panel_body<NT, R, PB>(M, N, r0, nch, d_out, nsw_out, src_out, Gn, orig, gbuf, full, blockIdx.x);
}

// M_new[p][q] = M_old[src p][src q] + sum_k G[p][k] (J G^T)[k][q] for the trailing
// positions p > q >= r1 (lower tiles of T x T). Four waves, each owning a (T/2) x (T/2)
// quarter as AW x AW 32x32 MFMA accumulators (the rows 8 (v / 4) + 4 lh + v % 4 of
// accumulator elements v = 4 g .. 4 g + 3 form one strip of the layout). Old entries: for
// the first block read through src from the full-storage input Min; for the others from
// the strip layout: a strip of four rows none of which moved is one 16-byte load at
// column src q (a moved column's source is a block row, below every trailing row, so the
// entry is stored there), a strip with a moved row (at most PB per block) entry by entry.
// New entries: the strip layout, four rows of a column per 16-byte store.
// Here in three phases on tile t of matrix b by the 256 threads tid of a workgroup:
// stage (G rows and the permutation into LDS), a workgroup barrier, load (the old entries
// into the accumulators), finish (G J G^T added, the lower entries stored). A workgroup
// may hold several tiles (pf_step_kernel: each 256-thread group two, all staged before the
// one barrier and all loaded before the first finish, for more loads in flight); an
// inactive tile (act = false) takes part in the barrier only. lds: 2 PB (T + 4) floats.
template <int PB, int T>
struct PfTile {
  static constexpr int H = T / 2, AW = H / 32;  // quarter size, accumulators per side
  static constexpr int LDG = T + 4;
  typedef float v16f __attribute__((ext_vector_type(16)));
  int I, J, p0, q0;
  int64_t b;
  bool act;
  float* Ga;  // the G rows of the tile rows, K-major
  float* Hb;  // the (J G^T) columns of the tile columns, K-major
  int* sp;
  int* sq;
  int* smv;  // strip of the tile rows with a moved row
  v16f acc[AW][AW];

  PfTile() = default;
  __device__ __forceinline__ PfTile(int r1, int64_t b_, int t, bool act_, float* lds, int* sp_, int* sq_, int* smv_)
      : b(b_), act(act_), Ga(lds), Hb(lds + PB * LDG), sp(sp_), sq(sq_), smv(smv_) {
    I = (int)((sqrtf(8.0f * t + 1.0f) - 1.0f) * 0.5f);
    while ((I + 1) * (I + 2) / 2 <= t) ++I;
    while (I * (I + 1) / 2 > t) --I;
    J = t - I * (I + 1) / 2;
    p0 = r1 + T * I;
    q0 = r1 + T * J;
  }

  __device__ __forceinline__ void stage(int N, const int* __restrict__ src, const float* __restrict__ Gn, int tid);

  __device__ __forceinline__ void load(const float* __restrict__ M, int N, const float* __restrict__ Min, int tid) {
    if (!act) return;
    const int wave = tid >> 6, lane = tid & 63;
    const float* Mb = M + b * (int64_t)N * N;  // entries addressed by 32-bit offsets (N * N < 2^31)
    // wave (wr, wc) owns an H x H quarter: the old entries M[src p][src q] (zeros for rows
    // / columns beyond N and the upper half of a diagonal tile, which are never stored),
    // loaded first, and G J G^T in AW x AW 32x32 accumulators of its own, added in fp32:
    // the MFMAs truncate what they add below about three bits under the accumulator's
    // last place, so small products added to the old entries one by one would lose more
    const bool diag = I == J;
    const int wr = (wave >> 1) * H, wc = (wave & 1) * H;
    const int l32 = lane & 31, lh = lane >> 5;
#pragma unroll
    for (int a = 0; a < AW; ++a)
#pragma unroll
      for (int c = 0; c < AW; ++c) {
        const int cl = wc + 32 * c + l32, q = q0 + cl;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int rl = wr + 32 * a + 8 * g + 4 * lh, p = p0 + rl;  // p % 4 == 0
          float x[4] = {0.0f, 0.0f, 0.0f, 0.0f};
          if (Min) {
            // rows / columns beyond N hold index 0 in sp / sq: in-bounds reads
            const float* Ab = Min + b * (int64_t)N * N;
#pragma unroll
            for (int u = 0; u < 4; ++u) x[u] = Ab[(unsigned)(sp[rl + u] * N + sq[cl])];
          } else if (p < N && q < N) {
            const int scol = sq[cl];
            if (!diag && !smv[rl >> 2]) {  // uniform per half-wave
              const float4 y = *reinterpret_cast<const float4*>(Mb + l4(p, scol, N));
              x[0] = y.x;
              x[1] = y.y;
              x[2] = y.z;
              x[3] = y.w;
            } else {
#pragma unroll
              for (int u = 0; u < 4; ++u) {
                const int srow = sp[rl + u];
                const float y = Mb[l4(max(srow, scol), min(srow, scol), N)];
                x[u] = (diag && p + u <= q) ? 0.0f : (srow > scol ? y : -y);
              }
            }
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) acc[a][c][4 * g + u] = x[u];
        }
      }
  }

  __device__ __forceinline__ void finish(float* __restrict__ M, int N, int tid) {
    if (!act) return;
    const int wave = tid >> 6, lane = tid & 63;
    const bool diag = I == J;
    const int wr = (wave >> 1) * H, wc = (wave & 1) * H;
    const int l32 = lane & 31, lh = lane >> 5;
    float* Mb = M + b * (int64_t)N * N;
    v16f prod[AW][AW];
#pragma unroll
    for (int a = 0; a < AW; ++a)
#pragma unroll
      for (int c = 0; c < AW; ++c)
#pragma unroll
        for (int v = 0; v < 16; ++v) prod[a][c][v] = 0.0f;
#pragma unroll
    for (int kp = 0; kp < PB / 2; ++kp) {
      float av[AW], bv[AW];
#pragma unroll
      for (int a = 0; a < AW; ++a) av[a] = Ga[(2 * kp + lh) * LDG + wr + 32 * a + l32];
#pragma unroll
      for (int c = 0; c < AW; ++c) bv[c] = Hb[(2 * kp + lh) * LDG + wc + 32 * c + l32];
#pragma unroll
      for (int a = 0; a < AW; ++a)
#pragma unroll
        for (int c = 0; c < AW; ++c)
          prod[a][c] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[a], bv[c], prod[a][c], 0, 0, 0);
    }
#pragma unroll
    for (int a = 0; a < AW; ++a)
#pragma unroll
      for (int c = 0; c < AW; ++c)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[a][c][v] += prod[a][c][v];
    // the lower entries: whole strips off the diagonal tiles (N is a multiple of 4, so a
    // strip is inside the matrix or outside it), entry by entry below the diagonal of a
    // diagonal tile
#pragma unroll
    for (int a = 0; a < AW; ++a)
#pragma unroll
      for (int c = 0; c < AW; ++c) {
        const int q = q0 + wc + 32 * c + l32;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int p = p0 + wr + 32 * a + 8 * g + 4 * lh;  // a multiple of 4
          if (p >= N || q >= N) continue;
          float* dst = Mb + l4(p, q, N);
          if (!diag) {
            *reinterpret_cast<float4*>(dst) =
                make_float4(acc[a][c][4 * g], acc[a][c][4 * g + 1], acc[a][c][4 * g + 2], acc[a][c][4 * g + 3]);
          } else {
#pragma unroll
            for (int u = 0; u < 4; ++u)
              if (p + u > q) dst[u] = acc[a][c][4 * g + u];
          }
        }
      }
  }
};

// The staging registers of one tile: gload (its G rows and permutation entries, every
// load issued before the first use) then lwrite (into the tile's LDS); stage is both.
// pf_step_kernel issues a later tile's gload before finishing the current tile.
template <int PB, int T>
struct PfStage {
  static constexpr int GE = T * PB / 256, LDG = T + 4;
  float ga[GE], gb[GE];
  int gsp, gsq;
  bool gmv;

  __device__ __forceinline__ void gload(const PfTile<PB, T>& x, int N, const int* __restrict__ src,
                                        const float* __restrict__ Gn, int tid) {
    if (!x.act) return;
    const float* G = Gn + x.b * (int64_t)N * PB;
    const int* sb = src + x.b * N;
#pragma unroll
    for (int i = 0; i < GE; ++i) {
      const int e = tid + 256 * i;
      const int r = e / PB, k = e % PB;
      const int p = min(x.p0 + r, N - 1), q = min(x.q0 + r, N - 1);
      ga[i] = G[(unsigned)(p * PB + k)];
      gb[i] = G[(unsigned)(q * PB + (k ^ 1))];
    }
    if (tid < T) {
      gsp = x.p0 + tid < N ? sb[x.p0 + tid] : 0;
      gsq = x.q0 + tid < N ? sb[x.q0 + tid] : 0;
    } else if (tid < T + T / 4) {
      const int r = x.p0 + 4 * (tid - T);  // rows beyond N (whole strips: N % 4 == 0) count as unmoved
      bool mv = false;
#pragma unroll
      for (int u = 0; u < 4; ++u) mv = mv || (r < N && sb[r + u] != r + u);
      gmv = mv;
    }
  }

  __device__ __forceinline__ void lwrite(const PfTile<PB, T>& x, int N, int tid) const {
    if (!x.act) return;
#pragma unroll
    for (int i = 0; i < GE; ++i) {
      const int e = tid + 256 * i;
      const int r = e / PB, k = e % PB;
      x.Ga[k * LDG + r] = x.p0 + r < N ? ga[i] : 0.0f;
      const float gq = x.q0 + r < N ? gb[i] : 0.0f;
      x.Hb[k * LDG + r] = (k & 1) ? -gq : gq;
    }
    if (tid < T) {
      x.sp[tid] = gsp;
      x.sq[tid] = gsq;
    } else if (tid < T + T / 4) {
      x.smv[tid - T] = gmv;
    }
  }
};

template <int PB, int T>
__device__ __forceinline__ void PfTile<PB, T>::stage(int N, const int* __restrict__ src, const float* __restrict__ Gn,
                                                     int tid) {
  PfStage<PB, T> g;
  g.gload(*this, N, src, Gn, tid);
  g.lwrite(*this, N, tid);
}

template <int PB, int T>
__global__ __launch_bounds__(256) void pf_update_kernel(float* __restrict__ M, int N, int r1,
                                                        const int* __restrict__ src,
                                                        const float* __restrict__ Gn,
                                                        const float* __restrict__ Min) {
  __shared__ __align__(16) float lds[2 * PB * (T + 4)];
  __shared__ int sp[T], sq[T];
  __shared__ int smv[T / 4];  // strip of the tile rows with a moved row
  int64_t b = blockIdx.y;
  int t = blockIdx.x;
  if (PB >= 64 && (gridDim.y & 7) == 0) {
    // workgroups go to the 8 XCDs round-robin by linear id: renumber so that all tiles
    // of one matrix run on one XCD and its G block is fetched into one L2 (measured at
    // n = 2048: 10 % faster with 64-column blocks, 8 % slower with 32-column ones)
    const int64_t lin = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
    const int64_t slot = lin >> 3;
    t = (int)(slot % gridDim.x);
    b = (slot / gridDim.x) * 8 + (lin & 7);
  }
  PfTile<PB, T> x(r1, b, t, true, lds, sp, sq, smv);
  x.stage(N, src, Gn, threadIdx.x);
  __syncthreads();
  x.load(M, N, Min, threadIdx.x);
  x.finish(M, N, threadIdx.x);
}

// One launch of two independent pieces of work on two halves of a batch: the panels of one
// half (workgroups 0 .. pa.batch - 1, one matrix each, pf_panel_body) and the trailing
// update of the other half (the later workgroups, persistent, one per CU left over). The panel
// workgroups come first in the dispatch order, so each finds an empty CU (a 1024-thread
// panel needs one to itself) before the update tiles fill the GPU beside them; as
// separate kernels on two streams the update's small workgroups keep every CU partly busy
// and the panel waits for the whole update.
struct PfPanelArgs {
  const float* M;
  int N, r0, nch, full;
  float* d;
  int* nsw;
  int* src;
  float* Gn;
  int* orig;
  float* gbuf;
  int64_t batch;
};
struct PfUpdateArgs {
  float* M;
  int r1, ntiles;
  const int* src;
  const float* Gn;
  const float* Min;
  int64_t batch;
};

template <int NT, int R, int PBp, int PBu>
__global__ __launch_bounds__(NT) void pf_step_kernel(PfPanelArgs pa, PfUpdateArgs ua) {
  if ((int64_t)blockIdx.x < pa.batch) {
    pf_panel_body<NT, R, PBp>(pa.M, pa.N, pa.r0, pa.nch, pa.d, pa.nsw, pa.src, pa.Gn, pa.orig, pa.gbuf, pa.full,
                              blockIdx.x);
    return;
  }
  // The update workgroups (the ids from pa.batch on, each holding a CU) are persistent: in
  // iteration k, group sub of the w-th of the nU update workgroups of one XCD updates the
  // NL tiles ((k nU + w) NS + sub) NL + l of that XCD's matrices. The loop keeps two stages per group in flight: stage k + 1's old entries (and,
  // where the registers hold them, stage k + 2's G rows) are loaded while stage k is
  // finished (LDS double-buffered; two barriers per iteration, the trip count uniform
  // over the workgroup). In the 128 registers of a 1024-thread workgroup: NL = 1, the G
  // rows ahead for PB <= 16 only (at PB = 32 they would spill). (Measured: 512-thread
  // workgroups, whose panels hold 4 rows per lane and whose update groups then have the
  // registers for two tiles per stage, ran the update part slower still: 8 waves per CU
  // hide less latency than 16.)
  constexpr int NS = NT / 256, NL = 1, T = PF_UPDATE_TILE;
  constexpr bool GAHEAD = PBu <= 16;
  __shared__ __align__(16) float lds[2][NS * NL][2 * PBu * (T + 4)];
  __shared__ int sp[2][NS * NL][T], sq[2][NS * NL][T], smv[2][NS * NL][T / 4];
  const int sub = threadIdx.x >> 8, tid = threadIdx.x & 255;
  // Workgroups go to the XCDs round-robin by id, so the update workgroups with id = x mod
  // 8 take the matrices b = x mod 8: a matrix's tiles then meet in one XCD's L2, which
  // fetches its G rows once (spread over the XCDs, every L2 fetched them: 1.48x the
  // matrix's read traffic at 32-column blocks).
  const int x8 = (int)(blockIdx.x & 7);
  const int64_t g_first = pa.batch + ((x8 - pa.batch % 8) + 8) % 8;  // first update id on XCD x8
  const int64_t nU = ((int64_t)gridDim.x - g_first + 7) / 8, w = ((int64_t)blockIdx.x - g_first) / 8;
  const int64_t nbx = (ua.batch - x8 + 7) / 8;  // matrices x8, x8 + 8, ...
  const int64_t tot = nbx * ua.ntiles;
  const int64_t iters = (tot + nU * NS * NL - 1) / (nU * NS * NL);
  auto tile = [&](int64_t k, int l) {
    const int64_t f = ((k * nU + w) * NS + sub) * NL + l;
    const bool act = k < iters && f < tot;
    const int64_t bx = act ? f / ua.ntiles : 0;
    const int64_t b = x8 + 8 * bx;
    const int buf = (int)(k & 1), slot = sub * NL + l;
    return PfTile<PBu, T>(ua.r1, act ? b : 0, act ? (int)(f - bx * ua.ntiles) : 0, act, lds[buf][slot], sp[buf][slot],
                          sq[buf][slot], smv[buf][slot]);
  };
  if (iters == 0) return;
  const int N = pa.N;
  typedef PfTile<PBu, T> Tile;
  // stage slots A (even iterations) and B (odd); g holds stage k + 2's staging registers
  // (the loops over l are unrolled, so the arrays stay in registers)
  Tile ta[NL], tb[NL];
#pragma unroll
  for (int l = 0; l < NL; ++l) {
    ta[l] = tile(0, l);
    tb[l] = tile(1, l);
    ta[l].stage(N, ua.src, ua.Gn, tid);
    tb[l].stage(N, ua.src, ua.Gn, tid);
  }
  __syncthreads();
#pragma unroll
  for (int l = 0; l < NL; ++l) ta[l].load(ua.M, N, ua.Min, tid);
  PfStage<PBu, T> g[NL];
  // stage k in cur, k + 1 in nxt (loaded here); cur then takes stage k + 2
  auto step = [&](Tile (&cur)[NL], Tile (&nxt)[NL], int64_t k) {
    Tile nn[NL];
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      nxt[l].load(ua.M, N, ua.Min, tid);
      nn[l] = tile(k + 2, l);
      if constexpr (GAHEAD) g[l].gload(nn[l], N, ua.src, ua.Gn, tid);
    }
#pragma unroll
    for (int l = 0; l < NL; ++l) cur[l].finish(ua.M, N, tid);
    __syncthreads();  // cur's buffers are free
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      cur[l] = nn[l];
      if constexpr (!GAHEAD) g[l].gload(cur[l], N, ua.src, ua.Gn, tid);
      g[l].lwrite(cur[l], N, tid);
    }
    __syncthreads();  // their rows visible
  };
  for (int64_t k = 0; k < iters; k += 2) {
    step(ta, tb, k);
    if (k + 1 < iters) step(tb, ta, k + 1);
  }
}

__global__ void pf_finish_kernel(const float* __restrict__ d, const int* __restrict__ nsw, int H, int nch,
                                 float* __restrict__ sign, float* __restrict__ logabs, int64_t batch) {
  const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (b >= batch) return;
  float lg = 0.0f;
  bool z = false, ng = false;
  for (int i = lane; i < H; i += 64) {
    const float v = d[b * H + i];
    z = z || (v == 0.0f);
    ng = ng != (v < 0.0f);
    lg += (v != 0.0f) ? logf(fabsf(v)) : 0.0f;
  }
  lg = wave_sum_f32(lg);
  int sw = 0;
  for (int k = lane; k < nch; k += 64) sw += nsw[b * nch + k];
  sw = (int)wave_sum_f32((float)sw);
  const bool anyz = __ballot(z) != 0ull;
  const int negs = __popcll(__ballot(ng)) + sw;
  if (lane == 0) {
    sign[b] = anyz ? 0.0f : ((negs & 1) ? -1.0f : 1.0f);
    logabs[b] = anyz ? -INFINITY : lg;
  }
}

static __global__ void pf_iota_kernel(int* g, int N, int64_t total) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < total) g[e] = (int)(e % N);
}

int pf_large_padded(int n) { return ((n + 31) / 32) * 32; }

// Widest block of padded order N, over the block sequence launch_pf_large runs.
static int pf_max_width(int N) {
  int w = 0;
  for (int r0 = 0; r0 < N;) {
    const int pb = pf_block_width(N, r0);
    w = pb > w ? pb : w;
    r0 += pb;
  }
  return w;
}

size_t pf_large_workspace(int64_t batch, int n, bool fact) {
  const int N = pf_large_padded(n);
  const int nch = N / pf_large_block_cols(N);
  size_t bytes = 0;
  auto add = [&](size_t x) { bytes += (x + 255) / 256 * 256; };
  add((size_t)batch * N * N * 4);  // M (updated in place)
  add((size_t)batch * N * pf_max_width(N) * 4);  // G (new order) of the current block
  add((size_t)batch * N * 4);      // src
  add((size_t)batch * nch * 4);    // swap counts per chunk
  add((size_t)batch * N / 2 * 4);  // d (forward only; parts uses its own)
  if (fact) add((size_t)batch * N * 4);  // orig
  return bytes;
}

// One block of PB columns at r0: the panel (NT = 256, 512 or 1024 threads, R rows per
// lane) and, unless it is the last block, the in-place trailing update.
template <int PB, int R>
static int pf_block(float* M, int N, int r0, int nch, int64_t batch, float* d, int* nsw, int* src, float* Gn,
                    int* orig, float* gbuf, const float* A0, hipStream_t s) {
  const int m = N - r0;
  const float* Mp = A0 ? A0 : M;  // A0 (first block): the input itself, full storage
  const int full = A0 != nullptr;
  const int r1 = r0 + PB;
  if (m <= 256 * R)
    hipLaunchKernelGGL((pf_panel_kernel<256, R, PB>), dim3((unsigned)batch), dim3(256), 0, s, Mp, N, r0, nch, d,
                       nsw, src, Gn, orig, gbuf, full);
  else if (m <= 512 * R)
    hipLaunchKernelGGL((pf_panel_kernel<512, R, PB>), dim3((unsigned)batch), dim3(512), 0, s, Mp, N, r0, nch, d,
                       nsw, src, Gn, orig, gbuf, full);
  else if constexpr (PB * R <= 64)  // G[R][PB] fits the 128 VGPRs of a 1024-thread workgroup
    hipLaunchKernelGGL((pf_panel_kernel<1024, R, PB>), dim3((unsigned)batch), dim3(1024), 0, s, Mp, N, r0, nch,
                       d, nsw, src, Gn, orig, gbuf, full);
  else
    return FX_ERR_UNSUPPORTED;
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  if (r1 >= N) return FX_OK;
  constexpr int TU = PF_UPDATE_TILE;
  const int nt = (N - r1 + TU - 1) / TU;
  const int64_t NN = (int64_t)N * N;
  for (int64_t b0 = 0; b0 < batch; b0 += 65535) {
    const int64_t nb = batch - b0 < 65535 ? batch - b0 : 65535;
    hipLaunchKernelGGL((pf_update_kernel<PB, TU>), dim3(nt * (nt + 1) / 2, (unsigned)nb), dim3(256), 0, s,
                       M + b0 * NN, N, r1, src + b0 * N, Gn + b0 * N * PB, A0 ? A0 + b0 * NN : nullptr);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  }
  return FX_OK;
}

// Rows per lane of the panels of PB-column blocks.
static constexpr int pf_rows(int PB) { return PB == PFB_XXL ? 8 : PB == PFB_XL ? 4 : 2; }

// One launch of pf_step_kernel: the panels of pa (1024 threads, their trailing order
// m > 512 R) and the update of ua.
template <int R, int PB>
static int step_launch(const PfPanelArgs& pa, const PfUpdateArgs& ua, hipStream_t s) {
  constexpr int NT = 1024;
  static_assert(PB * R <= 64, "G[R][PB] fits the 128 VGPRs of a 1024-thread workgroup");
  if (pa.batch > 0 && pa.N - pa.r0 <= 512 * R) return FX_ERR_UNSUPPORTED;
  // update workgroups: one per CU the panels leave (at least a quarter of the device)
  const int cus = device_cus();
  int64_t nu = 0;
  if (ua.batch * ua.ntiles > 0) nu = cus - pa.batch > cus / 4 ? cus - pa.batch : cus / 4;
  const int64_t grid = pa.batch + nu;
  if (grid > 0x7fffffff || grid == 0) return FX_ERR_UNSUPPORTED;
  hipLaunchKernelGGL((pf_step_kernel<NT, R, PB, PB>), dim3((unsigned)grid), dim3(NT), 0, s, pa, ua);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

// The buffers of the matrices b0 .. b0 + batch - 1 of a run.
struct PfPart {
  float* M;
  float* d;
  int* nsw;
  int* src;
  float* G;  // this part's G region (widest block)
  int* orig;
  float* gbuf;
  const float* A;  // the input, read in place by the first block (direct), else nullptr
  int64_t batch;
};

// Panels of block (rp, PB) of part P (nullptr: none) and the update after block (ru, PB)
// of part U (nullptr: none), in one launch of pf_step_kernel; both blocks PB columns wide
// with 1024-thread panels.
static int pf_pair(int N, int nch, const PfPart* P, int rp, const PfPart* U, int ru, int PB, hipStream_t s) {
  if (U && ru + PB >= N) U = nullptr;  // the last block has no update
  if (!P && !U) return FX_OK;
  PfPanelArgs pa{};
  PfUpdateArgs ua{};
  pa.N = N;
  if (P) {
    pa.M = rp == 0 && P->A ? P->A : P->M;
    pa.r0 = rp;
    pa.nch = nch;
    pa.full = rp == 0 && P->A;
    pa.d = P->d;
    pa.nsw = P->nsw;
    pa.src = P->src;
    pa.Gn = P->G;
    pa.orig = P->orig;
    pa.gbuf = P->gbuf;
    pa.batch = P->batch;
  }
  if (U) {
    constexpr int TU = PF_UPDATE_TILE;
    const int nt = (N - ru - PB + TU - 1) / TU;
    ua.M = U->M;
    ua.r1 = ru + PB;
    ua.ntiles = nt * (nt + 1) / 2;
    ua.src = U->src;
    ua.Gn = U->G;
    ua.Min = ru == 0 ? U->A : nullptr;
    ua.batch = U->batch;
  }
  if (PB == PFB) return step_launch<2, PFB>(pa, ua, s);
  if (PB == PFB_XL) return step_launch<4, PFB_XL>(pa, ua, s);
  if (PB == PFB_XXL) return step_launch<8, PFB_XXL>(pa, ua, s);
  return FX_ERR_UNSUPPORTED;
}

// Forward (and, with gbuf/dout/perm, the factors: gbuf (B, N/PB, N, PB) by original row,
// d (B, N/2), perm (B, N) final position -> original row).
int launch_pf_large(const float* A, int n, int skew, int64_t batch, float* sign, float* logabs,
                    float* gbuf, float* dout, int* perm, void* ws, size_t ws_bytes, hipStream_t s) {
  const int N = pf_large_padded(n);
  if (N > PF_LARGE_MAXN) return FX_ERR_UNSUPPORTED;
  const bool fact = gbuf != nullptr;
  if (!ws || ws_bytes < pf_large_workspace(batch, n, fact)) return FX_ERR_WORKSPACE;
  const int nch = N / pf_large_block_cols(N);
  char* p = (char*)ws;
  auto take = [&](size_t x) {
    char* q = p;
    p += (x + 255) / 256 * 256;
    return (void*)q;
  };
  float* M0 = (float*)take((size_t)batch * N * N * 4);
  float* Gn = (float*)take((size_t)batch * N * pf_max_width(N) * 4);
  int* src = (int*)take((size_t)batch * N * 4);
  int* nsw = (int*)take((size_t)batch * nch * 4);
  float* dbuf = (float*)take((size_t)batch * N / 2 * 4);
  int* orig = fact ? (int*)take((size_t)batch * N * 4) : nullptr;
  float* d = dout ? dout : dbuf;
  const int64_t NN = (int64_t)N * N;
  // No padding and no symmetrisation: the first block's panel and update read the input
  // itself, and the update writes every trailing entry of M (later blocks never read the
  // first block's rows), so no copy is made. Otherwise the padded copy comes first.
  const bool direct = n == N && !skew && ((uintptr_t)A & 15) == 0;
  if (!direct) {
    const int ntc = (N + PCT - 1) / PCT;
    hipLaunchKernelGGL(pf_copy_pad_kernel, dim3((unsigned)(ntc * (ntc + 1) / 2), (unsigned)batch), dim3(256), 0, s,
                       A, n, skew, M0, N);
    if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  }
  if (fact) {
    const int64_t tot = batch * N;
    hipLaunchKernelGGL(pf_iota_kernel, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, orig, N, tot);
  }
  const int maxw = pf_max_width(N);
  const fx_tune& tn = tune();
  // 64-column blocks (m <= 1024): one row per lane (up to 1024 threads, G[1][64]) where the
  // batch leaves CUs idle, two (half the threads, G[2][64]) where it fills the device:
  // slogpf B = 16, n = 1024 1.455 -> 1.375 ms, B = 256, n = 1024 3.70 -> 3.57 ms, B = 64,
  // n = 2048 8.37 -> 8.28 ms; B = 1024, n = 512 2.57 -> 2.84 ms (the same bits)
  const bool rows1 = batch <= device_cus();
  const int64_t hb = (batch + 1) / 2;
  const bool overlap = batch >= 2 && hb <= tn.pf_overlap_max_half &&
                       (double)batch * N * N >= (double)tn.pf_overlap_min_work * (1 << 20);
  if (!overlap) {
    for (int r0 = 0; r0 < N;) {
      const float* A0 = direct && r0 == 0 ? A : nullptr;
      const int PB = pf_block_width(N, r0);
      const int st =
          PB == PFB_L ? (rows1 ? pf_block<PFB_L, 1>(M0, N, r0, nch, batch, d, nsw, src, Gn, orig, gbuf, A0, s)
                               : pf_block<PFB_L, 2>(M0, N, r0, nch, batch, d, nsw, src, Gn, orig, gbuf, A0, s))
                     : PB == PFB ? pf_block<PFB, 2>(M0, N, r0, nch, batch, d, nsw, src, Gn, orig, gbuf, A0, s)
                     : PB == PFB_XL ? pf_block<PFB_XL, 4>(M0, N, r0, nch, batch, d, nsw, src, Gn, orig, gbuf, A0, s)
                                    : pf_block<PFB_XXL, 8>(M0, N, r0, nch, batch, d, nsw, src, Gn, orig, gbuf, A0, s);
      if (st != FX_OK) return st;
      r0 += PB;
    }
  } else {
    // Small batches of large matrices (fx_tune.pf_overlap_*) run as two halves a and b, b
    // one panel behind: each launch holds one half's panels and the other half's update
    // (pf_step_kernel), so the panels (one latency-bound workgroup per matrix, on few
    // CUs) run beside the updates (HBM-bound) where the whole batch would alternate
    // between the two:
    //   P(a, 0); P(b, 0) + U(a, 0); P(a, 1) + U(b, 0); P(b, 1) + U(a, 1); ...
    // Every kernel works per matrix, so the results are the same bits. The update part
    // runs in the panel's workgroup shape (1024 threads, 128 registers, one workgroup
    // per CU), about 70 % as fast as pf_update_kernel, so the overlap pays where half an
    // update takes about as long as a panel: measured B = 64, n = 2048 9.06 -> 8.76 ms,
    // B = 16, n = 4096 28.5 -> 27.0 ms, B = 4, n = 8192 102.5 -> 94.6 ms; B = 8 or 128,
    // n = 2048 lose (panels or updates alone dominate).
    PfPart part[2];
    for (int h = 0; h < 2; ++h) {
      const int64_t b0 = h * hb;
      part[h] = PfPart{M0 + b0 * NN, d + b0 * (N / 2), nsw + b0 * nch, src + b0 * N, Gn + b0 * N * maxw,
                       orig ? orig + b0 * N : nullptr, gbuf ? gbuf + b0 * NN : nullptr,
                       direct ? A + b0 * NN : nullptr, h ? batch - b0 : hb};
    }
    // the pipeline covers the blocks whose panels run 1024 threads (a CU each) and whose
    // next block does too; the later blocks, whose panels take longer than half an
    // update, run whole-batch
    auto wide = [&](int r0) {
      const int PB = pf_block_width(N, r0);
      return r0 < N && N - r0 > 512 * pf_rows(PB) && PB * pf_rows(PB) <= 64 && pf_block_width(N, r0 + PB) == PB;
    };
    int st = FX_OK, r0 = 0;
    if (wide(0)) {
      const int PB = pf_block_width(N, 0);
      st = pf_pair(N, nch, &part[0], 0, nullptr, 0, PB, s);
      for (; st == FX_OK;) {
        const int r1 = r0 + PB;
        st = pf_pair(N, nch, &part[1], r0, &part[0], r0, PB, s);
        if (st != FX_OK) break;
        if (!wide(r1)) {
          st = pf_pair(N, nch, nullptr, 0, &part[1], r0, PB, s);
          r0 = r1;
          break;
        }
        st = pf_pair(N, nch, &part[0], r1, &part[1], r0, PB, s);
        r0 = r1;
      }
    }
    for (; r0 < N && st == FX_OK;) {
      const float* A0 = direct && r0 == 0 ? A : nullptr;
      const int PB = pf_block_width(N, r0);
      st = PB == PFB_L ? (rows1 ? pf_block<PFB_L, 1>(M0, N, r0, nch, batch, d, nsw, src, Gn, orig, gbuf, A0, s)
                                : pf_block<PFB_L, 2>(M0, N, r0, nch, batch, d, nsw, src, Gn, orig, gbuf, A0, s))
           : PB == PFB ? pf_block<PFB, 2>(M0, N, r0, nch, batch, d, nsw, src, Gn, orig, gbuf, A0, s)
           : PB == PFB_XL ? pf_block<PFB_XL, 4>(M0, N, r0, nch, batch, d, nsw, src, Gn, orig, gbuf, A0, s)
                          : pf_block<PFB_XXL, 8>(M0, N, r0, nch, batch, d, nsw, src, Gn, orig, gbuf, A0, s);
      r0 += PB;
    }
    if (st != FX_OK) return st;
  }
  hipLaunchKernelGGL(pf_finish_kernel, dim3((unsigned)((batch + 3) / 4)), dim3(256), 0, s, d, nsw, N / 2, nch,
                     sign, logabs, batch);
  if (hipGetLastError() != hipSuccess) return FX_ERR_LAUNCH;
  if (perm && fact)
    if (hipMemcpyAsync(perm, orig, (size_t)batch * N * 4, hipMemcpyDeviceToDevice, s) != hipSuccess)
      return FX_ERR_LAUNCH;
  return FX_OK;
}

}  // namespace fx
