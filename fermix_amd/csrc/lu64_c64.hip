// The blocked LU / solves / Parlett-Reid of lu64_impl.inc instantiated for complex64
// (one translation unit per field, compiled in parallel).
#include "lu64_impl.inc"

namespace fx {

FX_BLK_INST(cx<float>)

}  // namespace fx
