// C ABI entry points of the fermix_amd library: argument validation, size dispatch
// (by n only, never by the batch, so a batched call and a vmapped one run the same
// arithmetic), workspace accounting and kernel sequencing on the caller's stream.
#include "common.h"
#include "fermix_internal.h"

namespace fx {

__global__ void fill2_kernel(float* a, float va, float* b, float vb, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) {
    a[i] = va;
    b[i] = vb;
  }
}

static int fill2(float* a, float va, float* b, float vb, int64_t count, hipStream_t s) {
  if (count <= 0) return FX_OK;
  const unsigned blocks = (unsigned)((count + 255) / 256);
  hipLaunchKernelGGL(fill2_kernel, dim3(blocks), dim3(256), 0, s, a, va, b, vb, count);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

static constexpr int SMALL_MAX = 128;
static constexpr int LARGE_MAX = 1024;

}  // namespace fx

using namespace fx;

extern "C" {

const char* fx_status_string(int status) {
  switch (status) {
    case FX_OK: return "ok";
    case FX_ERR_INVALID_ARGUMENT: return "invalid argument";
    case FX_ERR_WORKSPACE: return "workspace missing or too small";
    case FX_ERR_LAUNCH: return "HIP kernel launch failed";
    case FX_ERR_UNSUPPORTED: return "matrix size not supported by the compiled kernels";
    default: return "unknown status";
  }
}

int fx_abi_version(void) { return 100; }

int32_t fx_lu_padded_size(int32_t n) {
  if (n <= 0) return 0;
  if (n <= SMALL_MAX) return lu_small_padded(n);
  return n <= LARGE_MAX ? lu_large_padded(n) : -1;
}

int32_t fx_pf_padded_size(int32_t n) {
  if (n <= 0) return 0;
  return n <= SMALL_MAX ? pf_small_padded(n) : -1;
}

size_t fx_slogdet_f32_workspace(int64_t batch, int32_t n) {
  if (batch <= 0 || n <= SMALL_MAX || n > LARGE_MAX) return 0;
  return lu_large_workspace(batch, n, false);
}

int fx_slogdet_f32(const float* a, int64_t batch, int32_t n, float* sign, float* logabs,
                   void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  if (batch < 0 || n < 0) return FX_ERR_INVALID_ARGUMENT;
  if (batch == 0) return FX_OK;
  if (!sign || !logabs || (n > 0 && !a)) return FX_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (n == 0) return fill2(sign, 1.0f, logabs, 0.0f, batch, s);
  if (n <= SMALL_MAX) return launch_lu_small(a, n, batch, sign, logabs, nullptr, nullptr, s);
  if (n <= LARGE_MAX)
    return launch_lu_large(a, n, batch, sign, logabs, workspace, workspace_bytes, false, nullptr,
                           nullptr, s);
  return FX_ERR_UNSUPPORTED;
}

size_t fx_slogdet_parts_f32_workspace(int64_t batch, int32_t n) {
  (void)batch;
  (void)n;
  return 0;
}

int fx_slogdet_parts_f32(const float* a, int64_t batch, int32_t n, int32_t zero_singular,
                         float* sign, float* logabs, float* inv_t, float* lu, int32_t* perm,
                         void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  (void)zero_singular;
  (void)workspace;
  (void)workspace_bytes;
  if (batch < 0 || n < 0) return FX_ERR_INVALID_ARGUMENT;
  if (batch == 0) return FX_OK;
  if (!sign || !logabs || (n > 0 && !a)) return FX_ERR_INVALID_ARGUMENT;
  if ((lu == nullptr) != (perm == nullptr)) return FX_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (n == 0) return fill2(sign, 1.0f, logabs, 0.0f, batch, s);
  if (inv_t) return FX_ERR_UNSUPPORTED;
  if (n <= SMALL_MAX)
    return launch_lu_small(a, n, batch, sign, logabs, lu, (int*)perm, s);
  return FX_ERR_UNSUPPORTED;
}

size_t fx_slogpf_f32_workspace(int64_t batch, int32_t n) {
  (void)batch;
  (void)n;
  return 0;
}

int fx_slogpf_f32(const float* a, int64_t batch, int32_t n, int32_t skew_symmetrize, float* sign,
                  float* logabs, void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  (void)workspace;
  (void)workspace_bytes;
  if (batch < 0 || n < 0) return FX_ERR_INVALID_ARGUMENT;
  if (batch == 0) return FX_OK;
  if (!sign || !logabs || (n > 0 && !a)) return FX_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (n == 0) return fill2(sign, 1.0f, logabs, 0.0f, batch, s);
  if (n % 2 == 1) return fill2(sign, 0.0f, logabs, -INFINITY, batch, s);
  if (n <= SMALL_MAX)
    return launch_pf_small(a, n, skew_symmetrize ? 1 : 0, batch, sign, logabs, nullptr, nullptr,
                           nullptr, s);
  return FX_ERR_UNSUPPORTED;
}

int fx_slogpf_factors_f32(const float* a, int64_t batch, int32_t n, int32_t skew_symmetrize,
                          float* sign, float* logabs, float* gbuf, float* d, int32_t* perm,
                          fx_stream_t stream) {
  if (batch < 0 || n < 0) return FX_ERR_INVALID_ARGUMENT;
  if (batch == 0) return FX_OK;
  if (!sign || !logabs || !gbuf || !d || !perm || (n > 0 && !a)) return FX_ERR_INVALID_ARGUMENT;
  if (n == 0 || n % 2 == 1) return FX_ERR_UNSUPPORTED;
  hipStream_t s = (hipStream_t)stream;
  if (n <= SMALL_MAX)
    return launch_pf_small(a, n, skew_symmetrize ? 1 : 0, batch, sign, logabs, gbuf, d, (int*)perm,
                           s);
  return FX_ERR_UNSUPPORTED;
}

}  // extern "C"
