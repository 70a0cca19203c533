// fx_slogdet_f32_noalloc: fx_slogdet_f32 for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
// The blocked kernels' workspace (n > 128) comes from a device array of this library,
// `scratch`, of FX_NOALLOC_SCRATCH_BYTES; a batch whose workspace exceeds it runs in
// consecutive sub-batches that each fit (every kernel is per matrix, so the results are
// those of fx_slogdet_f32 bitwise). n <= 128 needs no workspace and runs fx_slogdet_f32
// directly. The plan (sub-batch size) is fixed and every argument checked before the
// first sub-batch is enqueued.
//
// Each GPU the library runs on holds its own copy of the array until the process ends;
// its address on a device is looked up once, with that device current
// (hipGetSymbolAddress), and kept. Every call on one GPU shares that GPU's array: calls
// that overlap on one GPU (different streams, or threads) race. The array keeps the last
// call's contents; the blocked kernels write every workspace entry they read, so nothing
// needs clearing between calls.
#include <mutex>

#include "common.h"
#include "fermix_internal.h"

static_assert(FX_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size is a multiple of 256 bytes");
// In host code `scratch` names a host-side stand-in, not device memory: only the
// address from scratch_address() may be handed to kernels, copies or fills.
static __device__ __align__(256) unsigned char scratch[FX_NOALLOC_SCRATCH_BYTES];

namespace fx {
namespace {

constexpr int MAX_DEVICES = 64;
void* scratch_dev[MAX_DEVICES];
hipError_t scratch_rc[MAX_DEVICES];
std::once_flag scratch_once[MAX_DEVICES];

// Device address of `scratch` on the current device (looked up once per device).
int scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return FX_ERR_LAUNCH;
  std::call_once(scratch_once[dev], [dev] {
    void* p = nullptr;
    scratch_rc[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    scratch_dev[dev] = p;
  });
  if (scratch_rc[dev] != hipSuccess || !scratch_dev[dev]) return FX_ERR_LAUNCH;
  *out = scratch_dev[dev];
  return FX_OK;
}

// Largest sub-batch (a multiple of 8 when at least 8, which keeps the XCD-aware tile
// order) whose workspace fits the scratch array; 0 if not even one member fits.
int64_t fitting_batch(int64_t batch, int n) {
  if (fx_slogdet_f32_workspace(1, n) > FX_NOALLOC_SCRATCH_BYTES) return 0;
  int64_t lo = 1, hi = batch;  // workspace is monotone in the batch
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo + 1) / 2;
    if (fx_slogdet_f32_workspace(mid, n) <= FX_NOALLOC_SCRATCH_BYTES)
      lo = mid;
    else
      hi = mid - 1;
  }
  if (lo >= batch) return batch;
  return lo >= 8 ? lo / 8 * 8 : lo;
}

}  // namespace
}  // namespace fx

using namespace fx;

extern "C" int64_t fx_slogdet_f32_noalloc_batch(int64_t batch, int32_t n) {
  fx::TunePin pin_;
  if (batch <= 0 || n < 0) return 0;
  if (fx_slogdet_f32_workspace(batch, n) == 0) return batch;
  return fitting_batch(batch, n);
}

extern "C" int fx_slogdet_f32_noalloc(const float* a, int64_t batch, int32_t n, float* sign, float* logabs,
                                      fx_stream_t stream) {
  fx::TunePin pin_;
  if (batch < 0 || n < 0) return FX_ERR_INVALID_ARGUMENT;
  if (batch == 0) return FX_OK;
  if (!sign || !logabs || (n > 0 && !a)) return FX_ERR_INVALID_ARGUMENT;
  if (fx_slogdet_f32_workspace(batch, n) == 0)  // no workspace needed (or n unsupported)
    return fx_slogdet_f32(a, batch, n, sign, logabs, FX_PREC_IEEE, nullptr, 0, stream);
  // the whole plan is checked before the first sub-batch is enqueued
  if (((uintptr_t)a & 15) || ((uintptr_t)sign & 3) || ((uintptr_t)logabs & 3)) return FX_ERR_INVALID_ARGUMENT;
  const int64_t m = fitting_batch(batch, n);
  if (m == 0) return FX_ERR_UNSUPPORTED;  // the workspace of one sub-batch exceeds the array
  void* ws = nullptr;
  const int st = scratch_address(&ws);
  if (st != FX_OK) return st;
  // Sub-batches go straight to the blocked LU, which reads each member's rows with
  // 4-byte loads whenever the matrices are not 16-byte aligned: for odd n a sub-batch
  // starts at a + b0 n^2 floats, 4-byte aligned only (n^2 = 1 mod 4). Same arguments as
  // fx_slogdet_f32 with FX_PREC_IEEE and the table's block choice, so bit-identical; all on
  // the caller's stream (the side stream of a split batch is created on first use).
  for (int64_t b0 = 0; b0 < batch; b0 += m) {
    const int64_t nb = batch - b0 < m ? batch - b0 : m;
    const int r = launch_lu_large(a + b0 * n * n, n, nb, sign + b0, logabs + b0, ws, FX_NOALLOC_SCRATCH_BYTES,
                                  false, nullptr, nullptr, (hipStream_t)stream, nullptr, nullptr, FX_PREC_IEEE, 0,
                                  false);
    if (r != FX_OK) return r;
  }
  return FX_OK;
}
