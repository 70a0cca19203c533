// The blocked LU / solves / Parlett-Reid of lu64_impl.inc instantiated for float32 above
// its own blocked kernels' orders (one translation unit per field, compiled in parallel).
#include "lu64_impl.inc"

namespace fx {

FX_BLK_INST(float)

}  // namespace fx
