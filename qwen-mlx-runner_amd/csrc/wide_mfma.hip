// Wide block (chunked prefill) on MFMA: Q4/g64 weights times up to 256 RHS.
// Not built yet: every wide request runs through the small-block kernel in
// groups of four RHS (runtime.cpp) until this kernel lands.
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace qmr {

bool wide_mfma_supported(const AffineArgs &) { return false; }

hipError_t launch_wide_mfma(const AffineArgs &, const DeviceLimits &, hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace qmr
