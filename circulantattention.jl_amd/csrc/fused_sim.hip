// Instantiations of the windowed-tile kernels for MODE_SIM (fused_impl.h).
#include "fused_impl.h"

namespace circatt {

hipError_t launch_fused_sim(const FusedPlan &pl, int nsp, bool dist, hipStream_t s) {
    return launch_mode_all<MODE_SIM>(pl, nsp, dist, s);
}

}  // namespace circatt
