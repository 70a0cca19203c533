// The blocked LU / solves / Parlett-Reid of lu64_impl.inc instantiated for float64
// (one translation unit per field, compiled in parallel).
#include "lu64_impl.inc"

namespace fx {

FX_BLK_INST(double)

// the float64 names used by f64.hip and cplx.hip
size_t lu64_workspace(int64_t batch, int n) { return blk_lu_workspace<double>(batch, n); }
int launch_lu64(const double* A, int n, int64_t batch, double* sign, double* logabs, void* ws, size_t ws_bytes,
                hipStream_t s) {
  return blk_lu<double>(A, n, batch, sign, logabs, ws, ws_bytes, s);
}
size_t lu64_inverse_workspace(int64_t batch, int n) { return blk_lu_inverse_workspace<double>(batch, n); }
int launch_lu64_inverse(const double* A, int n, int skew, int64_t batch, double* sign, double* logabs,
                        const double* gate, const double* ssign, const double* slog, double* out, int out_t,
                        void* ws, size_t ws_bytes, hipStream_t s) {
  return blk_lu_inverse<double>(A, n, skew, batch, sign, logabs, gate, ssign, slog, out, out_t, ws, ws_bytes, s);
}
size_t pr64_workspace(int64_t batch, int n) { return blk_pr_workspace<double>(batch, n); }
int launch_pr64_blocked(const double* A, int n, int skew, int64_t batch, double* sign, double* logabs, void* ws,
                        size_t ws_bytes, hipStream_t s, double* spread) {
  return blk_pr<double>(A, n, skew, batch, sign, logabs, ws, ws_bytes, s, spread);
}

}  // namespace fx
