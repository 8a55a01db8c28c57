// Instantiations of the split-half kernels for one-dimensional signals,
// forward, 16 real components per head (fused2h_impl.h).
#include "fused2h_impl.h"

namespace circatt {

hipError_t launch_f1h_fwd(int p, bool cplx, bool dist, const f2d::Args &a, int cus,
                          hipStream_t s) {
    return f2h::dispatch1<f2h::FWD, 1>(p, cplx, dist, a, cus, s);
}

}  // namespace circatt
