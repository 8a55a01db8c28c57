// Instantiations of the split-half kernels for one-dimensional signals,
// forward, 32 real components per head (fused2h_impl.h).
#include "fused2h_impl.h"

namespace circatt {

hipError_t launch_f1h2_fwd(int p, bool cplx, bool dist, const f2d::Args &a, int cus,
                           hipStream_t s) {
    return f2h::dispatch1<f2h::FWD, 2>(p, cplx, dist, a, cus, s);
}

#if CIRCATT_F2H_PHASE
// phase-timing builds of these kernels only (microbench/phase_timing.py
// --config cfg4b): the buffer of 512 floats the waves write to
float *&phase_buffer() {
    static float *p = nullptr;
    return p;
}
#endif

}  // namespace circatt

#if CIRCATT_F2H_PHASE
extern "C" void circatt_debug_set_phase_buffer(float *p) { circatt::phase_buffer() = p; }
#endif
