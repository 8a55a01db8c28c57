// Instantiations of the split-half backward kernel, one mode (fused2h_impl.h).
#include "fused2h_impl.h"

namespace circatt {

hipError_t launch_f2h_bwdkv(int p, bool cplx, bool dist, const f2d::Args &a, int cus,
                          hipStream_t s) {
    return f2h::dispatch<f2h::BWDKV, 1>(p, cplx, dist, a, cus, s);
}

}  // namespace circatt
