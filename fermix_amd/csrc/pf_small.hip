// Fused slogpf for even n <= 128: one workgroup (4 waves) per matrix, the skew matrix
// resident in LDS, blocked Parlett-Reid with partial pivoting in blocks of 8 pair steps.
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
// Per block (positions from r0):
//   * wave 0 runs 8 pair steps on the block's rows (lane l owns rows R*l ..), keeping
//     the tau / w vectors as the columns of G (m x 16); column a and column p of the
//     current matrix are the block-start matrix plus the G corrections
//     sum_u tau_u[i] w_u[q] - w_u[i] tau_u[q]; the permutation stays virtual;
//   * all waves then form the trailing block M'' = M + G J G^T (J = diag of
//     [[0,1],[-1,0]]) on fp32 MFMA 16x16x4, lower-triangle tiles only, gathered through
//     the block's permutation, stored in the new order together with the mirrored
//     (negated) upper triangle, so the LDS matrix stays exactly skew.
// With FACT every block's G is exported indexed by the original row index, with the
// pivots d and the final position -> original row map (the factors of P S P^T = L D L^T).
//
// Padding n < N uses the blocks [[0,1],[-1,0]] (Pfaffian exactly +1).
#include "common.h"
#include "fermix_internal.h"

namespace fx {

template <int N>
struct PfSmall {
  static constexpr int LDA = N + 1;
  static constexpr int LDG = 17;
  static constexpr int R = (N + 63) / 64;
  static constexpr int NB = N / 16;
  static constexpr int NPV = (N / 2 + 63) / 64;  // pivot slots per lane
  static constexpr int MAXNT = N / 16 - 1;                       // trailing tiles per side
  static constexpr int MAXTILES = MAXNT * (MAXNT + 1) / 2;       // lower-triangle tiles
  static constexpr int TPW = MAXTILES > 0 ? (MAXTILES + 3) / 4 : 1;  // tiles per wave
};

template <int N, bool FACT>
__device__ __forceinline__ void pf_panel(const float* As, float* Gs, int r0, int* src, int lane,
                                         PivotLog<PfSmall<N>::NPV>& piv_log, int& nsw, int* orig,
                                         float* gbuf_k, float* d_k) {
  constexpr int LDA = PfSmall<N>::LDA, LDG = PfSmall<N>::LDG, R = PfSmall<N>::R;
  float G[R][16];
  int pos[R];
  bool valid[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int row = R * lane + i;
    valid[i] = (row >= r0) && (row < N);
    pos[i] = row;
#pragma unroll
    for (int k = 0; k < 16; ++k) G[i][k] = 0.0f;
  }
  static_for<0, 8>([&](auto tc) {
    constexpr int t = decltype(tc)::value;
    const int c = r0 + 2 * t;
    // row a: the row at position c (wave-uniform lane la, slot sa)
    bool hit = false;
    int hs = 0;
#pragma unroll
    for (int i = 0; i < R; ++i)
      if (valid[i] && pos[i] == c) { hit = true; hs = i; }
    const int la = first_lane(hit);
    const int sa = readlane_i(hs, la);
    const int qa = R * la + sa;
    float ga[16];
    static_for<0, 2 * t>([&](auto kc) {
      float v = G[0][kc.value];
#pragma unroll
      for (int i = 1; i < R; ++i) v = (sa == i) ? G[i][kc.value] : v;
      ga[kc.value] = readlane_f(v, la);
    });
    // column a of the current matrix: M[i][qa] = -M[qa][i] plus the G corrections
    float x[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int row = R * lane + i;
      float v = valid[i] ? -As[qa * LDA + row] : 0.0f;
      static_for<0, t>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        v = fmaf(G[i][2 * u], ga[2 * u + 1], v);
        v = fmaf(-G[i][2 * u + 1], ga[2 * u], v);
      });
      x[i] = v;
    }
    unsigned kb = 0;
    int ib = 0;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const unsigned k = cand_key(x[i], valid[i] && pos[i] > c);
      if (k > kb) { kb = k; ib = i; }
    }
    const unsigned gk = wave_max_u32(kb);
    const int lp = first_lane(kb == gk);
    const int sp = readlane_i(ib, lp);
    const int qp = R * lp + sp;
    float gp[16];
    static_for<0, 2 * t>([&](auto kc) {
      float v = G[0][kc.value];
#pragma unroll
      for (int i = 1; i < R; ++i) v = (sp == i) ? G[i][kc.value] : v;
      gp[kc.value] = readlane_f(v, lp);
    });
    int pv = pos[0];
#pragma unroll
    for (int i = 1; i < R; ++i) pv = (sp == i) ? pos[i] : pv;
    const int pp = readlane_i(pv, lp);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (valid[i] && pos[i] == c + 1) pos[i] = pp;
      if (lane == lp && i == sp) pos[i] = c + 1;
    }
    nsw += (pp != c + 1) ? 1 : 0;
    float y[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int row = R * lane + i;
      float v = valid[i] ? -As[qp * LDA + row] : 0.0f;
      static_for<0, t>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        v = fmaf(G[i][2 * u], gp[2 * u + 1], v);
        v = fmaf(-G[i][2 * u + 1], gp[2 * u], v);
      });
      y[i] = v;
    }
    float yv = y[0];  // M[a][p] = y at row a
#pragma unroll
    for (int i = 1; i < R; ++i) yv = (sa == i) ? y[i] : yv;
    const float d = readlane_f(yv, la);
    piv_log.put(c >> 1, d, lane);
    const float inv = safe_rcp(d);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const bool act = valid[i] && pos[i] > c + 1;
      G[i][2 * t] = act ? -x[i] * inv : 0.0f;
      G[i][2 * t + 1] = act ? y[i] : 0.0f;
    }
    if (FACT && lane == 0) d_k[t] = d;
  });
#pragma unroll
  for (int i = 0; i < R; ++i) {
    if (valid[i]) {
      const int row = R * lane + i;
#pragma unroll
      for (int k = 0; k < 16; ++k) Gs[row * LDG + k] = G[i][k];
      src[pos[i]] = row;
    }
  }
  if (FACT) {
    int ov[R];
#pragma unroll
    for (int i = 0; i < R; ++i) ov[i] = valid[i] ? orig[R * lane + i] : 0;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (valid[i]) {
#pragma unroll
        for (int k = 0; k < 16; ++k) gbuf_k[ov[i] * 16 + k] = G[i][k];
      }
    }
    wave_lds_fence();
#pragma unroll
    for (int i = 0; i < R; ++i)
      if (valid[i]) orig[pos[i]] = ov[i];
  }
  wave_lds_fence();
}

template <int N, bool FACT>
__global__ __launch_bounds__(256) void pf_small_kernel(const float* __restrict__ A, int n, int skew,
                                                       float* __restrict__ sign_out,
                                                       float* __restrict__ logabs_out,
                                                       float* __restrict__ gbuf_out,
                                                       float* __restrict__ d_out,
                                                       int* __restrict__ perm_out) {
  using C = PfSmall<N>;
  constexpr int LDA = C::LDA, LDG = C::LDG, NB = C::NB, TPW = C::TPW;
  __shared__ float As[N * LDA];
  __shared__ float Gs[N * LDG];
  __shared__ int src[N];
  __shared__ int orig[N];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const float* Ab = A + b * (int64_t)n * n;
  // [[0,1],[-1,0]] padding blocks (n is even)
  load_tile<N, LDA, 256>(As, Ab, n, tid, [](int r, int c) {
    return ((r ^ c) == 1) ? ((r & 1) ? -1.0f : 1.0f) : 0.0f;
  });
  if (skew) {
    __syncthreads();
    // S = (A - A^T) / 2 in place: thread pairs (r, c) with r < c
    for (int e = tid; e < n * n; e += 256) {
      const int r = e / n, c = e - r * n;
      if (r < c) {
        const float x = As[r * LDA + c], y = As[c * LDA + r];
        As[r * LDA + c] = (x - y) * 0.5f;
        As[c * LDA + r] = (y - x) * 0.5f;
      } else if (r == c) {
        As[r * LDA + c] = 0.0f;
      }
    }
  }
  if (FACT)
    for (int r = tid; r < N; r += 256) orig[r] = r;
  __syncthreads();

  PivotLog<C::NPV> piv_log;
  piv_log.init();
  int nsw = 0;
  const int li = lane & 15, g = lane >> 4;
  for (int k = 0; k < NB; ++k) {
    const int r0 = 16 * k;
    if (wave == 0) {
      float* gk = FACT ? gbuf_out + (b * NB + k) * (int64_t)N * 16 : nullptr;
      float* dk = FACT ? d_out + b * (N / 2) + 8 * k : nullptr;
      pf_panel<N, FACT>(As, Gs, r0, src, lane, piv_log, nsw, orig, gk, dk);
    }
    __syncthreads();
    const int nt = (N - r0 - 16) / 16;
    const int ntiles = nt * (nt + 1) / 2;
    const int rb = r0 + 16;
    v4f acc[TPW];
    int ti[TPW], tj[TPW];
#pragma unroll
    for (int s = 0; s < TPW; ++s) {
      const int t = wave + 4 * s;
      ti[s] = 0;
      tj[s] = 0;
      if (t < ntiles) {
        // tile t -> (I, J), I >= J, row-major over the lower triangle
        int I = 0;
        while ((I + 1) * (I + 2) / 2 <= t) ++I;
        const int J = t - I * (I + 1) / 2;
        ti[s] = I;
        tj[s] = J;
        const int q = rb + 16 * J + li;
        const int sq = src[q];
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[s][v] = As[src[rb + 16 * I + 4 * g + v] * LDA + sq];
      }
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < TPW; ++s) {
      const int t = wave + 4 * s;
      if (t < ntiles) {
        const int I = ti[s], J = tj[s];
        const int sr = src[rb + 16 * I + li];
        const int sq = src[rb + 16 * J + li];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int k = 4 * u + g;
          const float av = Gs[sr * LDG + k];
          const float bv = (k & 1) ? -Gs[sq * LDG + k - 1] : Gs[sq * LDG + k + 1];
          acc[s] = mfma16(av, bv, acc[s]);
        }
        const int q = rb + 16 * J + li;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int p = rb + 16 * I + 4 * g + v;
          if (p > q) {
            As[p * LDA + q] = acc[s][v];
            As[q * LDA + p] = -acc[s][v];
          } else if (p == q) {
            As[p * LDA + q] = 0.0f;
          }
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
  if (FACT)
    for (int r = tid; r < N; r += 256) perm_out[b * N + r] = orig[r];
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
    case 16: return launch_n<16, FACT>(A, n, skew, batch, sign, logabs, gbuf, d, perm, s);
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
  if (gbuf) return dispatch<true>(A, n, skew, batch, sign, logabs, gbuf, d, perm, s);
  return dispatch<false>(A, n, skew, batch, sign, logabs, nullptr, nullptr, nullptr, s);
}

}  // namespace fx
