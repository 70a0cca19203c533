// Internal launcher declarations of the fermix_amd HIP library (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/fermix.h"

namespace fx {

// n <= 128 fused kernels (one workgroup per matrix).
int lu_small_padded(int n);
int pf_small_padded(int n);
// slogdet; with lu != nullptr also the packed LU of P A (B, N, N) in the final row order
// and perm (B, N) with (P A)[c] = A[perm[c]], N = lu_small_padded(n).
int launch_lu_small(const float* A, int n, int64_t batch, float* sign, float* logabs, float* lu,
                    int* perm, hipStream_t s);
// slogpf; with gbuf != nullptr also the Parlett-Reid factors: gbuf (B, N/16, N, 16) with
// block k's tau_t / w_t in columns 2t / 2t+1 indexed by original row, d (B, N/2) the pair
// pivots, perm (B, N) final position -> original row. N = pf_small_padded(n).
int launch_pf_small(const float* A, int n, int skew, int64_t batch, float* sign, float* logabs,
                    float* gbuf, float* d, int* perm, hipStream_t s);

}  // namespace fx
