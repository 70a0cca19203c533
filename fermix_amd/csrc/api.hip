// C ABI entry points of the fermix_amd library: argument validation, size dispatch
// (by n only, never by the batch, so a batched call and a vmapped one run the same
// arithmetic), workspace accounting and kernel sequencing on the caller's stream.
#include <stdlib.h>
#include <string.h>

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

__global__ void fill_kernel(float* a, float v, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) a[i] = v;
}

// Streaming copy: four 16-byte loads in flight per thread (indices clamped so the loads
// are unconditional; only in-range stores happen).
__global__ __launch_bounds__(256) void copy4_kernel(const float4* __restrict__ src, float4* __restrict__ dst,
                                                    int64_t n4) {
  const int64_t base = (int64_t)blockIdx.x * 1024 + threadIdx.x;
  float4 v[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t i = base + 256 * u;
    v[u] = src[i < n4 ? i : n4 - 1];
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t i = base + 256 * u;
    if (i < n4) dst[i] = v[u];
  }
}

int launch_copy(const float* src, float* dst, int64_t count, hipStream_t s) {
  const int64_t n4 = count / 4;
  if (n4 <= 0) return FX_OK;
  hipLaunchKernelGGL(copy4_kernel, dim3((unsigned)((n4 + 1023) / 1024)), dim3(256), 0, s,
                     reinterpret_cast<const float4*>(src), reinterpret_cast<float4*>(dst), n4);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

// A fill kernel rather than hipMemsetAsync, so the call stays safe under graph capture.
static int fill(float* a, float v, int64_t count, hipStream_t s) {
  if (count <= 0) return FX_OK;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, a, v, count);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

static int fill2(float* a, float va, float* b, float vb, int64_t count, hipStream_t s) {
  if (count <= 0) return FX_OK;
  const unsigned blocks = (unsigned)((count + 255) / 256);
  hipLaunchKernelGGL(fill2_kernel, dim3(blocks), dim3(256), 0, s, a, va, b, vb, count);
  return hipGetLastError() == hipSuccess ? FX_OK : FX_ERR_LAUNCH;
}

static constexpr int SMALL_MAX = 128;
static constexpr int LARGE_MAX = LU_LARGE_MAXN;
static constexpr int PF_LARGE_MAX = PF_LARGE_MAXN;

// Kernel families. The choice depends on n only (never on the batch), so a batched call
// and a vmapped one run the same arithmetic: several matrices per wave (n <= 32 for the
// LU, 16 for Parlett-Reid), one fused workgroup per matrix (n <= 128), blocked kernels
// with workspace (n <= 8192), and above them the field-generic blocked kernels of the
// float64 path on float storage (n <= GEN32_MAXN: values and the gradients' parts runs,
// no packed factors). The environment variable FERMIX_AMD_KERNELS = tiny | fused |
// blocked forces a family where it covers n (for cross-checks and tuning sweeps; an
// uncovered n then reports FX_ERR_UNSUPPORTED; "blocked" keeps the generic family above
// 8192). It is read on every call and the library keeps no state of its own.
enum { FAM_NONE = -1, FAM_TINY = 0, FAM_FUSED = 1, FAM_BLOCKED = 2, FAM_GENERIC = 3 };

static int family_override() {
  const char* e = getenv("FERMIX_AMD_KERNELS");
  if (!e || !*e) return FAM_NONE;
  if (!strcmp(e, "tiny")) return FAM_TINY;
  if (!strcmp(e, "fused")) return FAM_FUSED;
  if (!strcmp(e, "blocked")) return FAM_BLOCKED;
  if (!strcmp(e, "generic")) return FAM_GENERIC;
  return FAM_NONE;
}

// tiny_max: largest n of the tiny family for this factorisation; large_max: of the blocked.
static int family(int n, int tiny_max, int large_max) {
  if (n <= 0 || n > GEN32_MAXN) return FAM_NONE;
  if (n > large_max) {
    const int o = family_override();
    return o == FAM_NONE || o == FAM_BLOCKED || o == FAM_GENERIC ? FAM_GENERIC : FAM_NONE;
  }
  switch (family_override()) {
    case FAM_TINY: return n <= tiny_max ? FAM_TINY : FAM_NONE;
    case FAM_FUSED: return (n > tiny_max && n <= SMALL_MAX) ? FAM_FUSED : FAM_NONE;
    case FAM_BLOCKED: return FAM_BLOCKED;
    case FAM_GENERIC: return n > SMALL_MAX ? FAM_GENERIC : FAM_NONE;
    default: break;
  }
  if (n <= tiny_max) return FAM_TINY;
  const int fused_max = tune().fused_max_n < SMALL_MAX ? tune().fused_max_n : SMALL_MAX;
  return n <= fused_max ? FAM_FUSED : FAM_BLOCKED;
}

// The LU's own blocked kernels stop at fx_tune.lu_generic_above_n unless a family is forced.
static int lu_family(int n) {
  const int f = family(n, TINY_MAXN, LARGE_MAX);
  return f == FAM_BLOCKED && n > tune().lu_generic_above_n && family_override() == FAM_NONE ? FAM_GENERIC : f;
}
static int pf_family(int n) { return family(n, PF_TINY_MAXN, PF_LARGE_MAX); }

// Alignment contract of the ABI: every matrix-shaped or workspace pointer is 16-byte
// aligned (the kernels move rows as 16-byte vectors), per-member scalars (sign, logabs,
// scale) 4-byte aligned. Checked before any work is enqueued.
static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }
static bool al4(const void* p) { return ((uintptr_t)p & 3) == 0; }

// Batch chunking: several kernels put the batch on gridDim.y (at most 65535), so the
// entry points that reach them run the batch in chunks of BATCH_CHUNK members (a multiple
// of 8, which keeps the XCD-aware tile order and 16-byte alignment of every chunk's
// slices), one after another on the stream, each reusing the same workspace. Workspace
// sizes are those of one chunk.
static constexpr int64_t BATCH_CHUNK = 65528;
static int64_t chunk_batch(int64_t batch) { return batch < BATCH_CHUNK ? batch : BATCH_CHUNK; }

// prec argument of the entry points: FX_PREC_IEEE (fp32 MFMA) or FX_PREC_BF16X3; the
// LU factorisations also take an FX_LU_BLOCK_* option in the same word.
static bool bad_prec(int32_t prec) { return prec != FX_PREC_IEEE && prec != FX_PREC_BF16X3; }
static bool bad_lu_prec(int32_t prec) {
  return (prec & ~(FX_PREC_MASK | FX_LU_BLOCK_MASK)) != 0 || bad_prec(prec & FX_PREC_MASK) ||
         (prec & FX_LU_BLOCK_MASK) == FX_LU_BLOCK_MASK;
}
static int x3_of(int32_t prec) { return prec & FX_PREC_MASK; }
static int block_of(int32_t prec) { return prec & FX_LU_BLOCK_MASK; }

template <class F>
static int for_chunks(int64_t batch, F&& f) {
  for (int64_t b0 = 0; b0 < batch; b0 += BATCH_CHUNK) {
    const int st = f(b0, chunk_batch(batch - b0));
    if (st != FX_OK) return st;
  }
  return FX_OK;
}

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

int fx_abi_version(void) { return 203; }

int32_t fx_lu_padded_size(int32_t n) {
  fx::TunePin pin_;
  if (n <= 0) return 0;
  const int f = lu_family(n);
  if (f == FAM_NONE || f == FAM_GENERIC) return -1;
  return f == FAM_BLOCKED ? lu_large_padded(n) : lu_small_padded(n);
}

int32_t fx_pf_padded_size(int32_t n) {
  fx::TunePin pin_;
  if (n <= 0) return 0;
  const int f = pf_family(n);
  if (f == FAM_NONE || f == FAM_GENERIC) return -1;
  return f == FAM_BLOCKED ? pf_large_padded(n) : pf_small_padded(n);
}

int32_t fx_pf_block_columns(int32_t n) {
  fx::TunePin pin_;
  return pf_family(n) != FAM_BLOCKED ? 16 : pf_large_block_cols(pf_large_padded(n));
}

size_t fx_slogdet_f32_workspace(int64_t batch, int32_t n) {
  fx::TunePin pin_;
  if (batch > 0 && lu_family(n) == FAM_GENERIC) return gen32_slogdet_ws(batch, n);
  if (batch <= 0 || lu_family(n) != FAM_BLOCKED) return 0;
  return lu_large_workspace(chunk_batch(batch), n, false);
}

int fx_slogdet_f32(const float* a, int64_t batch, int32_t n, float* sign, float* logabs, int32_t prec,
                   void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  if (batch < 0 || n < 0 || bad_lu_prec(prec)) return FX_ERR_INVALID_ARGUMENT;
  if (batch == 0) return FX_OK;
  if (!sign || !logabs || (n > 0 && !a)) return FX_ERR_INVALID_ARGUMENT;
  if (!al16(a) || !al4(sign) || !al4(logabs) || !al16(workspace)) return FX_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (n == 0) return fill2(sign, 1.0f, logabs, 0.0f, batch, s);
  switch (lu_family(n)) {
    case FAM_TINY: return launch_lu_tiny(a, n, batch, sign, logabs, nullptr, nullptr, s);
    case FAM_FUSED: return launch_lu_small(a, n, batch, sign, logabs, nullptr, nullptr, s);
    case FAM_BLOCKED:
      return for_chunks(batch, [&](int64_t b0, int64_t nb) {
        return launch_lu_large(a + b0 * n * n, n, nb, sign + b0, logabs + b0, workspace, workspace_bytes, false,
                               nullptr, nullptr, s, nullptr, nullptr, x3_of(prec), block_of(prec));
      });
    case FAM_GENERIC: return gen32_slogdet(a, batch, n, sign, logabs, workspace, workspace_bytes, s);
    default: return FX_ERR_UNSUPPORTED;
  }
}

// The packed LU and row map of the tiny / fused families (no workspace; N = lu_small_padded).
static int lu_fused_factors(int fam, const float* a, int n, int64_t batch, float* sign, float* logabs, float* lu,
                            int* perm, hipStream_t s) {
  return fam == FAM_TINY ? launch_lu_tiny(a, n, batch, sign, logabs, lu, perm, s)
                         : launch_lu_small(a, n, batch, sign, logabs, lu, perm, s);
}

static size_t align256(size_t x) { return (x + 255) / 256 * 256; }

// Workspace of one chunk of nb members of fx_slogdet_parts_f32.
static size_t slogdet_parts_ws(int64_t nb, int n, int fam) {
  const int N = fx_lu_padded_size(n);
  const bool copy = inv_padded(N) != N;
  size_t bytes = 0;
  if (fam != FAM_BLOCKED) {
    bytes += align256((size_t)nb * N * N * 4) + align256((size_t)nb * N * 4);
  } else {
    bytes += align256(lu_large_workspace(nb, n, true));
  }
  return bytes + lu_inverse_workspace(nb, N, copy);
}

size_t fx_slogdet_parts_f32_workspace(int64_t batch, int32_t n) {
  fx::TunePin pin_;
  const int fam = lu_family(n);
  if (batch <= 0 || fam == FAM_NONE) return 0;
  if (fam == FAM_GENERIC) return gen32_slogdet_parts_ws(batch, n);
  return slogdet_parts_ws(chunk_batch(batch), n, fam);
}

int fx_slogdet_parts_f32(const float* a, int64_t batch, int32_t n, int32_t zero_singular,
                         float* sign, float* logabs, float* inv_t, float* lu, int32_t* perm, int32_t prec,
                         void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  if (batch < 0 || n < 0 || bad_lu_prec(prec)) return FX_ERR_INVALID_ARGUMENT;
  if (batch == 0) return FX_OK;
  if (!sign || !logabs || (n > 0 && !a)) return FX_ERR_INVALID_ARGUMENT;
  if ((lu == nullptr) != (perm == nullptr)) return FX_ERR_INVALID_ARGUMENT;
  if (!al16(a) || !al4(sign) || !al4(logabs) || !al16(inv_t) || !al16(lu) || !al16(perm) || !al16(workspace))
    return FX_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (n == 0) return fill2(sign, 1.0f, logabs, 0.0f, batch, s);
  const int fam = lu_family(n);
  if (fam == FAM_NONE) return FX_ERR_UNSUPPORTED;
  if (fam == FAM_GENERIC) {  // no packed factors, no unguarded inverse there
    if (lu || !zero_singular) return FX_ERR_UNSUPPORTED;
    return gen32_slogdet_parts(a, batch, n, sign, logabs, inv_t, workspace, workspace_bytes, s);
  }
  if (!inv_t && fam != FAM_BLOCKED && lu)  // factors only: straight into the caller's buffers
    return lu_fused_factors(fam, a, n, batch, sign, logabs, lu, (int*)perm, s);
  if (inv_t && !lu && fam == FAM_TINY)  // one Gauss-Jordan pass, no workspace
    return launch_lu_tiny_inv(a, n, batch, zero_singular ? 1 : 0, sign, logabs, inv_t, s);
  const size_t need = fx_slogdet_parts_f32_workspace(batch, n);
  if (!workspace || workspace_bytes < need) return FX_ERR_WORKSPACE;
  const int N = fx_lu_padded_size(n);
  return for_chunks(batch, [&](int64_t b0, int64_t nb) {
    const float* ab = a + b0 * n * n;
    float* sg = sign + b0;
    float* lg = logabs + b0;
    char* p = (char*)workspace;
    float* LU = nullptr;
    int* g0 = nullptr;
    int st;
    if (fam != FAM_BLOCKED) {
      LU = (float*)p;
      p += align256((size_t)nb * N * N * 4);
      g0 = (int*)p;
      p += align256((size_t)nb * N * 4);
      st = lu_fused_factors(fam, ab, n, nb, sg, lg, LU, g0, s);
    } else {
      const size_t wl = lu_large_workspace(nb, n, true);
      st = launch_lu_large(ab, n, nb, sg, lg, p, wl, true, &LU, &g0, s, nullptr, nullptr, x3_of(prec),
                           block_of(prec));
      p += align256(wl);
    }
    if (st != FX_OK) return st;
    if (lu) {
      if (hipMemcpyAsync(lu + b0 * N * N, LU, (size_t)nb * N * N * 4, hipMemcpyDeviceToDevice, s) != hipSuccess ||
          hipMemcpyAsync(perm + b0 * N, g0, (size_t)nb * N * 4, hipMemcpyDeviceToDevice, s) != hipSuccess)
        return FX_ERR_LAUNCH;
    }
    if (!inv_t) return FX_OK;
    const size_t rest = workspace_bytes - (size_t)(p - (char*)workspace);
    return launch_lu_inverse(LU, g0, N, n, nb, sg, zero_singular, inv_t + b0 * n * n, true, p, rest, s, nullptr,
                             x3_of(prec));
  });
}

size_t fx_slogdet_factors_f32_workspace(int64_t batch, int32_t n) {
  fx::TunePin pin_;
  if (batch <= 0 || lu_family(n) != FAM_BLOCKED) return 0;
  return lu_large_workspace(chunk_batch(batch), n, true, true);
}

int fx_slogdet_factors_f32(const float* a, int64_t batch, int32_t n, float* sign, float* logabs, float* lu,
                           int32_t* perm, int32_t prec, void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  if (batch < 0 || n < 0 || bad_lu_prec(prec)) return FX_ERR_INVALID_ARGUMENT;
  if (batch == 0) return FX_OK;
  if (!sign || !logabs || (n > 0 && (!a || !lu || !perm))) return FX_ERR_INVALID_ARGUMENT;
  if (!al16(a) || !al4(sign) || !al4(logabs) || !al16(lu) || !al16(perm) || !al16(workspace))
    return FX_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (n == 0) return fill2(sign, 1.0f, logabs, 0.0f, batch, s);
  const int fam = lu_family(n);
  if (fam == FAM_NONE || fam == FAM_GENERIC) return FX_ERR_UNSUPPORTED;
  if (fam != FAM_BLOCKED) return lu_fused_factors(fam, a, n, batch, sign, logabs, lu, (int*)perm, s);
  const int N = fx_lu_padded_size(n);
  return for_chunks(batch, [&](int64_t b0, int64_t nb) {
    return launch_lu_large(a + b0 * n * n, n, nb, sign + b0, logabs + b0, workspace, workspace_bytes, true, nullptr,
                           nullptr, s, lu + b0 * N * N, (int*)perm + b0 * N, x3_of(prec), block_of(prec));
  });
}

size_t fx_slogdet_inverse_f32_workspace(int64_t batch, int32_t n) {
  fx::TunePin pin_;
  if (batch <= 0 || n <= 0 || lu_family(n) == FAM_NONE || lu_family(n) == FAM_GENERIC) return 0;
  const int N = fx_lu_padded_size(n);
  return lu_inverse_workspace(chunk_batch(batch), N, inv_padded(N) != N);
}

int fx_slogdet_inverse_f32(float* lu, const int32_t* perm, const float* sign, const float* scale, int64_t batch,
                           int32_t n, int32_t zero_singular, float* inv_t, int32_t prec, void* workspace,
                           size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  if (batch < 0 || n < 0 || bad_prec(prec)) return FX_ERR_INVALID_ARGUMENT;
  if (batch == 0 || n == 0) return FX_OK;
  if (!lu || !perm || !sign || !inv_t) return FX_ERR_INVALID_ARGUMENT;
  if (!al16(lu) || !al16(perm) || !al4(sign) || !al4(scale) || !al16(inv_t) || !al16(workspace))
    return FX_ERR_INVALID_ARGUMENT;
  if (lu_family(n) == FAM_NONE || lu_family(n) == FAM_GENERIC) return FX_ERR_UNSUPPORTED;
  const size_t need = fx_slogdet_inverse_f32_workspace(batch, n);
  if (!workspace || workspace_bytes < need) return FX_ERR_WORKSPACE;
  const int N = fx_lu_padded_size(n);
  return for_chunks(batch, [&](int64_t b0, int64_t nb) {
    return launch_lu_inverse(lu + b0 * N * N, (const int*)perm + b0 * N, N, n, nb, sign + b0, zero_singular ? 1 : 0,
                             inv_t + b0 * n * n, true, workspace, workspace_bytes, (hipStream_t)stream,
                             scale ? scale + b0 : nullptr, prec);
  });
}

size_t fx_det_parts_f32_workspace(int64_t batch, int32_t n) {
  fx::TunePin pin_;
  if (batch <= 0 || lu_family(n) == FAM_NONE) return 0;
  if (lu_family(n) == FAM_GENERIC) return gen32_det_parts_ws(batch, n);
  return fx_slogdet_parts_f32_workspace(batch, n) + align256(det_adjugate_workspace(chunk_batch(batch), n));
}

int fx_det_parts_f32(const float* a, int64_t batch, int32_t n, float* sign, float* logabs, float* adj_t,
                     int32_t prec, void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  if (batch < 0 || n < 0 || bad_lu_prec(prec)) return FX_ERR_INVALID_ARGUMENT;
  if (batch == 0) return FX_OK;
  if (!sign || !logabs || (n > 0 && (!a || !adj_t))) return FX_ERR_INVALID_ARGUMENT;
  if (!al16(a) || !al4(sign) || !al4(logabs) || !al16(adj_t) || !al16(workspace)) return FX_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (n == 0) return fill2(sign, 1.0f, logabs, 0.0f, batch, s);
  const int fam = lu_family(n);
  if (fam == FAM_NONE) return FX_ERR_UNSUPPORTED;
  if (fam == FAM_GENERIC) return gen32_det_parts(a, batch, n, sign, logabs, adj_t, workspace, workspace_bytes, s);
  const size_t need = fx_det_parts_f32_workspace(batch, n);
  if (!workspace || workspace_bytes < need) return FX_ERR_WORKSPACE;
  const int N = fx_lu_padded_size(n);
  return for_chunks(batch, [&](int64_t b0, int64_t nb) {
    const float* ab = a + b0 * n * n;
    float* sg = sign + b0;
    float* lg = logabs + b0;
    float* adj = adj_t + b0 * n * n;
    char* p = (char*)workspace;
    float* LU = nullptr;
    int* g0 = nullptr;
    int st;
    if (fam != FAM_BLOCKED) {
      LU = (float*)p;
      p += align256((size_t)nb * N * N * 4);
      g0 = (int*)p;
      p += align256((size_t)nb * N * 4);
      st = lu_fused_factors(fam, ab, n, nb, sg, lg, LU, g0, s);
    } else {
      const size_t wl = lu_large_workspace(nb, n, true);
      st = launch_lu_large(ab, n, nb, sg, lg, p, wl, true, &LU, &g0, s, nullptr, nullptr, x3_of(prec),
                           block_of(prec));
      p += align256(wl);
    }
    if (st != FX_OK) return st;
    // the adjugate's scalars and vectors come from the LU before the inverse overwrites it
    void* dws = p;
    p += align256(det_adjugate_workspace(nb, n));
    float* scale = nullptr;
    st = launch_det_adjugate_prep(LU, g0, N, n, nb, dws, &scale, s);
    if (st != FX_OK) return st;
    const size_t rest = workspace_bytes - (size_t)(p - (char*)workspace);
    st = launch_lu_inverse(LU, g0, N, n, nb, sg, 0, adj, true, p, rest, s, scale, x3_of(prec));
    if (st != FX_OK) return st;
    return launch_det_adjugate_finish(n, nb, dws, adj, s);
  });
}

size_t fx_slogpf_f32_workspace(int64_t batch, int32_t n) {
  fx::TunePin pin_;
  if (batch > 0 && n % 2 == 0 && pf_family(n) == FAM_GENERIC) return gen32_slogpf_ws(batch, n);
  if (batch <= 0 || n % 2 || pf_family(n) != FAM_BLOCKED) return 0;
  return pf_large_workspace(chunk_batch(batch), n, false);
}

static int pf_fused(int fam, const float* a, int n, int sk, int64_t batch, float* sign, float* logabs, float* gbuf,
                    float* d, int* perm, hipStream_t s) {
  return fam == FAM_TINY ? launch_pf_tiny(a, n, sk, batch, sign, logabs, gbuf, d, perm, s)
                         : launch_pf_small(a, n, sk, batch, sign, logabs, gbuf, d, perm, s);
}

int fx_slogpf_f32(const float* a, int64_t batch, int32_t n, int32_t skew_symmetrize, float* sign,
                  float* logabs, void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  if (batch < 0 || n < 0) return FX_ERR_INVALID_ARGUMENT;
  if (batch == 0) return FX_OK;
  if (!sign || !logabs || (n > 0 && !a)) return FX_ERR_INVALID_ARGUMENT;
  if (!al16(a) || !al4(sign) || !al4(logabs) || !al16(workspace)) return FX_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (n == 0) return fill2(sign, 1.0f, logabs, 0.0f, batch, s);
  if (n % 2 == 1) return fill2(sign, 0.0f, logabs, -INFINITY, batch, s);
  const int sk = skew_symmetrize ? 1 : 0;
  const int fam = pf_family(n);
  if (fam == FAM_NONE) return FX_ERR_UNSUPPORTED;
  if (fam == FAM_GENERIC) return gen32_slogpf(a, batch, n, sk, sign, logabs, workspace, workspace_bytes, s);
  if (fam != FAM_BLOCKED) return pf_fused(fam, a, n, sk, batch, sign, logabs, nullptr, nullptr, nullptr, s);
  return for_chunks(batch, [&](int64_t b0, int64_t nb) {
    return launch_pf_large(a + b0 * n * n, n, sk, nb, sign + b0, logabs + b0, nullptr, nullptr, nullptr, workspace,
                           workspace_bytes, s);
  });
}

size_t fx_slogpf_factors_f32_workspace(int64_t batch, int32_t n) {
  fx::TunePin pin_;
  if (batch <= 0 || n % 2 || pf_family(n) != FAM_BLOCKED) return 0;
  return pf_large_workspace(chunk_batch(batch), n, true);
}

int fx_slogpf_factors_f32(const float* a, int64_t batch, int32_t n, int32_t skew_symmetrize,
                          float* sign, float* logabs, float* gbuf, float* d, int32_t* perm,
                          void* workspace, size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  if (batch < 0 || n < 0) return FX_ERR_INVALID_ARGUMENT;
  if (batch == 0) return FX_OK;
  if (!sign || !logabs || !gbuf || !d || !perm || (n > 0 && !a)) return FX_ERR_INVALID_ARGUMENT;
  if (!al16(a) || !al4(sign) || !al4(logabs) || !al16(gbuf) || !al16(d) || !al16(perm) || !al16(workspace))
    return FX_ERR_INVALID_ARGUMENT;
  if (n == 0 || n % 2 == 1) return FX_ERR_UNSUPPORTED;
  hipStream_t s = (hipStream_t)stream;
  const int sk = skew_symmetrize ? 1 : 0;
  const int fam = pf_family(n);
  if (fam == FAM_NONE || fam == FAM_GENERIC) return FX_ERR_UNSUPPORTED;
  if (fam != FAM_BLOCKED) return pf_fused(fam, a, n, sk, batch, sign, logabs, gbuf, d, (int*)perm, s);
  const int N = fx_pf_padded_size(n);
  return for_chunks(batch, [&](int64_t b0, int64_t nb) {
    return launch_pf_large(a + b0 * n * n, n, sk, nb, sign + b0, logabs + b0, gbuf + b0 * N * N, d + b0 * (N / 2),
                           (int*)perm + b0 * N, workspace, workspace_bytes, s);
  });
}

size_t fx_slogpf_inverse_f32_workspace(int64_t batch, int32_t n) {
  fx::TunePin pin_;
  if (batch <= 0 || n <= 0 || n % 2 || pf_family(n) == FAM_NONE || pf_family(n) == FAM_GENERIC) return 0;
  return pf_inverse_workspace(chunk_batch(batch), fx_pf_padded_size(n));
}

int fx_slogpf_inverse_f32(const float* gbuf, const float* d, const int32_t* perm, const float* scale,
                          int64_t batch, int32_t n, int32_t adjugate, float* g, int32_t prec, void* workspace,
                          size_t workspace_bytes, fx_stream_t stream) {
  fx::TunePin pin_;
  if (batch < 0 || n < 0 || bad_prec(prec)) return FX_ERR_INVALID_ARGUMENT;
  if (batch == 0 || n == 0) return FX_OK;
  if (!g) return FX_ERR_INVALID_ARGUMENT;
  if (!al16(gbuf) || !al16(d) || !al16(perm) || !al4(scale) || !al16(g) || !al16(workspace))
    return FX_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (n % 2 == 1) return fill(g, 0.0f, batch * (int64_t)n * n, s);
  if (!gbuf || !d || !perm) return FX_ERR_INVALID_ARGUMENT;
  if (pf_family(n) == FAM_NONE || pf_family(n) == FAM_GENERIC) return FX_ERR_UNSUPPORTED;
  const size_t need = fx_slogpf_inverse_f32_workspace(batch, n);
  if (!workspace || workspace_bytes < need) return FX_ERR_WORKSPACE;
  const int N = fx_pf_padded_size(n);
  return for_chunks(batch, [&](int64_t b0, int64_t nb) {
    return launch_pf_inverse(gbuf + b0 * N * N, fx_pf_block_columns(n), d + b0 * (N / 2), (const int*)perm + b0 * N,
                             N, n, nb, adjugate ? 1 : 0, g + b0 * n * n, workspace, workspace_bytes, s,
                             scale ? scale + b0 : nullptr, prec);
  });
}

// Workspace of one chunk of nb members of fx_slogpf_parts_f32.
static size_t slogpf_parts_ws(int64_t nb, int n, int fam) {
  const int N = fx_pf_padded_size(n);
  size_t bytes = align256((size_t)nb * N * N * 4) + align256((size_t)nb * N / 2 * 4) + align256((size_t)nb * N * 4);
  if (fam == FAM_BLOCKED) bytes += align256(pf_large_workspace(nb, n, true));
  return bytes + pf_inverse_workspace(nb, N);
}

size_t fx_slogpf_parts_f32_workspace(int64_t batch, int32_t n) {
  fx::TunePin pin_;
  const int fam = pf_family(n);
  if (batch <= 0 || n % 2 || fam == FAM_NONE) return 0;
  if (fam == FAM_GENERIC) return gen32_slogpf_parts_ws(batch, n);
  return slogpf_parts_ws(chunk_batch(batch), n, fam);
}

int fx_slogpf_parts_f32(const float* a, int64_t batch, int32_t n, int32_t skew_symmetrize, int32_t adjugate,
                        float* sign, float* logabs, float* g, int32_t prec, void* workspace, size_t workspace_bytes,
                        fx_stream_t stream) {
  fx::TunePin pin_;
  if (batch < 0 || n < 0 || bad_prec(prec)) return FX_ERR_INVALID_ARGUMENT;
  if (batch == 0) return FX_OK;
  if (!sign || !logabs || !g || (n > 0 && !a)) return FX_ERR_INVALID_ARGUMENT;
  if (!al16(a) || !al4(sign) || !al4(logabs) || !al16(g) || !al16(workspace)) return FX_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (n == 0) return fill2(sign, 1.0f, logabs, 0.0f, batch, s);
  if (n % 2 == 1) {
    int st = fill2(sign, 0.0f, logabs, -INFINITY, batch, s);
    if (st != FX_OK) return st;
    return fill(g, 0.0f, batch * (int64_t)n * n, s);
  }
  const int fam = pf_family(n);
  if (fam == FAM_NONE) return FX_ERR_UNSUPPORTED;
  if (fam == FAM_GENERIC)
    return gen32_slogpf_parts(a, batch, n, skew_symmetrize ? 1 : 0, adjugate ? 1 : 0, sign, logabs, g, workspace,
                              workspace_bytes, s);
  const size_t need = fx_slogpf_parts_f32_workspace(batch, n);
  if (!workspace || workspace_bytes < need) return FX_ERR_WORKSPACE;
  const int N = fx_pf_padded_size(n);
  const int sk = skew_symmetrize ? 1 : 0;
  return for_chunks(batch, [&](int64_t b0, int64_t nb) {
    const float* ab = a + b0 * n * n;
    float* sg = sign + b0;
    float* lg = logabs + b0;
    char* p = (char*)workspace;
    float* gbuf = (float*)p;
    p += align256((size_t)nb * N * N * 4);
    float* d = (float*)p;
    p += align256((size_t)nb * N / 2 * 4);
    int* perm = (int*)p;
    p += align256((size_t)nb * N * 4);
    int st;
    if (fam != FAM_BLOCKED) {
      st = pf_fused(fam, ab, n, sk, nb, sg, lg, gbuf, d, perm, s);
    } else {
      const size_t wl = pf_large_workspace(nb, n, true);
      st = launch_pf_large(ab, n, sk, nb, sg, lg, gbuf, d, perm, p, wl, s);
      p += align256(wl);
    }
    if (st != FX_OK) return st;
    const size_t rest = workspace_bytes - (size_t)(p - (char*)workspace);
    return launch_pf_inverse(gbuf, fx_pf_block_columns(n), d, perm, N, n, nb, adjugate ? 1 : 0, g + b0 * n * n, p,
                             rest, s, nullptr, prec);
  });
}

}  // extern "C"
