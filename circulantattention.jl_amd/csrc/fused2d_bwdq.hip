// Instantiations of the compile-time-window 2D kernels for one mode (fused2d_impl.h).
#include "fused2d_impl.h"

namespace circatt {

hipError_t launch_f2d_bwdq(int p, int nt, bool cplx, bool dist, const f2d::Args &a, int cus,
                          hipStream_t s) {
    return f2d::dispatch<f2d::BWDQ>(p, nt, cplx, dist, a, cus, s);
}

}  // namespace circatt
