// The gfx950 tuning table and its override (fx_tune_table / fx_tune_override /
// fx_tune_active): the launch choices the host code makes from n alone. Counterpart of
// the reference's Tune / TUNES[arch][kind] / OVERRIDE / _tune (src/fermix/_common.py:
// 17-378), whose per-architecture values are Triton tiles and warps; the values here
// are the size thresholds of this library's own dispatch decisions, each measured on
// MI355X:
//  - fused_max_n 128: the one-workgroup-per-matrix kernels hold an n <= 128 matrix in
//    LDS (40 KiB at n = 128, four matrices per CU) and beat the blocked kernels there;
//  - lu_pair_above_n 256: LU blocks in pairs (one K = 128 trailing update per pair)
//    lost 1.6 % at N = 256 (their extra U-row correction and launches) and win above
//    (slogdet B = 1024, n = 512 2.54 -> 2.46 ms; B = 64, n = 2048 11.48 -> 10.40 ms);
//  - lu_direct_max_n 1024: the largest order whose panels are held in registers, so the
//    first block pair can read the input in place of a copy;
//  - pf_block64_min_n 512 / pf_block64_max_m 1024: 64-column Parlett-Reid blocks halve
//    the trailing updates' traffic (B = 256, n = 1024 5.33 -> 3.97 ms) but at N = 256 the
//    panel's halved occupancy loses (2.44 -> 3.20 ms); m <= 1024 is the register limit
//    of the 64-column panel;
//  - gemm128_min_mn 1024 / gemm128_min_k 512 / gemm128_tout 0 (fp32 MFMA): 128 x 128
//    GEMM tiles won on the n = 2048 products (triangular-inverse top level -18 %,
//    R = Y^T D Y -15 %) and lost at M = 512 and for short K (coarser triangle trimming,
//    longer prologue per stage); for the A^-T product they lose at n = 512 / 1024
//    (slogdet fwd + grad B = 1024, n = 512: 6.23 -> 6.56 ms) and tie at 2048;
//  - gemm128_x3_*: 128 / 128 / 1 (bf16x3): there the 128 x 128 kernel, which splits each
//    operand once into LDS planes, wins on every product from 128 on: slogdet fwd + grad
//    n = 512 6.32 -> 5.78 ms, n = 1024 9.74 -> 8.64, n = 2048 19.68 -> 17.64, n = 256
//    4.56 -> 4.41; slogpf fwd + grad 1-4 %;
//  - f64_reg_max_n 128 / f64_strip16_max_n 64: float64 matrices in registers for
//    n <= 128 (slogdet n = 128 8.66 -> 3.16 ms against the LDS kernel), in 16-column strips
//    for n <= 64 (n = 64 1.37 ms; at n = 128 they lose, 3.97 against 3.16 ms);
//  - pf_overlap_max_half 32 / pf_overlap_min_work 256: the Parlett-Reid halves with one
//    half's panels beside the other's update gain where half an update takes about as
//    long as a panel (slogpf B = 64, n = 2048 9.06 -> 8.76 ms; B = 16, n = 4096 28.5 ->
//    27.0; B = 4, n = 8192 102.5 -> 94.6) and lose where either dominates (B = 8 or 128,
//    n = 2048: 3.79 -> 4.88, 15.2 -> 17.4 ms);
//  - lu_split_min_work 128: the LU's halves on two streams (tails of one half's kernels
//    beside the other's) gain from batch * N^2 >= 2^27 (slogdet + A^-T B = 1024, n = 512
//    5.54 -> 5.37 ms; B = 16, n = 4096 38.9 -> 36.7) and lose below (B = 256, n = 512
//    slogdet 0.88 -> 0.92 ms; B = 16, n = 2048 6.30 -> 6.54) and above N = 4096 (B = 4,
//    n = 8192 153.3 -> 154.7);
//  - lu_generic_above_n 4096: above it the float32 LU's panels of more than 4096 rows
//    spill their registers, and the field-generic kernels' multi-workgroup panels win:
//    slogdet n = 6144 83.5 -> 55.2 ms, n = 8192 138 -> 83 ms, slogdet + A^-T 90.0 -> 82.9 /
//    146 -> 142 ms; at n = 4160 the forward wins (43.5 -> 35.6) and the gradient is even
//    (52.8 / 54.0). The Parlett-Reid keeps its own kernels to 8192 (its generic path is
//    1.7-4x slower there).
#include <atomic>
#include <deque>
#include <mutex>
#include <string.h>

#include "common.h"
#include "fermix_internal.h"

namespace fx {
namespace {

constexpr fx_tune GFX950 = {
    /* fused_max_n */ 128,
    /* lu_pair_above_n */ 256,
    /* lu_direct_max_n */ 1024,
    /* pf_block64_min_n */ 512,
    /* pf_block64_max_m */ 1024,
    /* gemm128_min_mn */ 1024,
    /* gemm128_min_k */ 512,
    /* gemm128_tout */ 0,
    /* gemm128_x3_min_mn */ 128,
    /* gemm128_x3_min_k */ 128,
    /* gemm128_x3_tout */ 1,
    /* f64_reg_max_n */ 128,
    /* f64_strip16_max_n */ 64,
    /* pf_overlap_max_half */ 32,
    /* pf_overlap_min_work */ 256,
    /* lu_split_min_work */ 128,
    /* lu_generic_above_n */ 4096,
    /* reserved */ {0, 0, 0},
};

// Every table an override publishes is kept, unchanged, until the process ends (a few
// dozen bytes each; an identical table is published once), so a pointer to the active
// table stays valid for as long as any call holds it.
std::mutex g_store_mu;
std::deque<fx_tune> g_store;
std::atomic<const fx_tune*> g_active{&GFX950};
thread_local const fx_tune* t_pinned = nullptr;

const fx_tune* publish(const fx_tune& t) {
  std::lock_guard<std::mutex> lock(g_store_mu);
  for (const fx_tune& x : g_store)
    if (memcmp(&x, &t, sizeof t) == 0) return &x;
  g_store.push_back(t);
  return &g_store.back();
}

bool valid(const fx_tune& t) {
  auto in = [](int32_t v, int32_t lo, int32_t hi) { return v >= lo && v <= hi; };
  for (int32_t r : t.reserved)
    if (r != 0) return false;
  return in(t.fused_max_n, TINY_MAXN, 128) && in(t.lu_pair_above_n, 0, 1 << 30) &&
         in(t.lu_direct_max_n, 0, 1024) && in(t.pf_block64_min_n, 128, 1 << 30) &&
         in(t.pf_block64_max_m, 0, 1024) && in(t.gemm128_min_mn, 128, 1 << 30) &&
         in(t.gemm128_min_k, 64, 1 << 30) && in(t.gemm128_tout, 0, 1) &&
         in(t.gemm128_x3_min_mn, 128, 1 << 30) && in(t.gemm128_x3_min_k, 64, 1 << 30) && in(t.gemm128_x3_tout, 0, 1) && in(t.f64_reg_max_n, 0, 128) &&
         in(t.f64_strip16_max_n, 0, 64) && in(t.pf_overlap_max_half, 0, 1 << 30) &&
         in(t.pf_overlap_min_work, 0, 1 << 30) && in(t.lu_split_min_work, 0, 1 << 30) &&
         in(t.lu_generic_above_n, 128, LU_LARGE_MAXN);
}

}  // namespace

// The table of the current call: the one pinned when the outermost entry point on this
// thread began, so every decision of one call (workspace layout, block widths, tile
// shapes) reads the same table even while another thread publishes an override.
const fx_tune& tune() { return t_pinned ? *t_pinned : *g_active.load(std::memory_order_acquire); }

TunePin::TunePin() : own_(t_pinned == nullptr) {
  if (own_) t_pinned = g_active.load(std::memory_order_acquire);
}

TunePin::~TunePin() {
  if (own_) t_pinned = nullptr;
}

}  // namespace fx

using namespace fx;

extern "C" {

int fx_tune_table(const char* arch, fx_tune* out) {
  if (!arch || !out) return FX_ERR_INVALID_ARGUMENT;
  // a full device name may carry target features ("gfx950:sramecc+:xnack-")
  const size_t len = strcspn(arch, ":");
  if (len != 6 || strncmp(arch, "gfx950", 6) != 0) return FX_ERR_UNSUPPORTED;
  *out = GFX950;
  return FX_OK;
}

int fx_tune_override(const fx_tune* t) {
  if (!t) {
    g_active.store(&GFX950, std::memory_order_release);
    return FX_OK;
  }
  if (!valid(*t)) return FX_ERR_INVALID_ARGUMENT;
  g_active.store(publish(*t), std::memory_order_release);
  return FX_OK;
}

int fx_tune_active(fx_tune* out) {
  if (!out) return FX_ERR_INVALID_ARGUMENT;
  *out = tune();
  return FX_OK;
}

}  // extern "C"
