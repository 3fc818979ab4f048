// dK/dV and dQ kernels (placeholders until the MFMA backward lands).
#include "g4_kernels.h"

namespace g4 {
hipError_t launch_bwd_dkdv(const BwdParams&, hipStream_t) { return hipErrorNotSupported; }
hipError_t launch_bwd_dq(const BwdParams&, hipStream_t) { return hipErrorNotSupported; }
}  // namespace g4
