// Instantiations of the channel-chunked fused kernels (fused_wide_impl.h).
#include "fused_wide_impl.h"

namespace circatt {

namespace {

template <int NSP, bool DIST, int MODE>
hipError_t launch_one(const FArgs &a, size_t lds, dim3 grid, hipStream_t s) {
    auto kern = wide::wide_kernel<NSP, DIST, MODE>;
    // set once per instantiation (a function-local static is initialised
    // exactly once, also when several host threads launch at the same time)
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)wide::kLdsBudget);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(kern, grid, dim3(wide::THREADS), lds, s, a);
    return hipGetLastError();
}

template <int MODE>
hipError_t launch_mode(int nsp, bool dist, const FArgs &a, size_t lds, dim3 grid, hipStream_t s) {
    if (nsp == 1)
        return dist ? launch_one<1, true, MODE>(a, lds, grid, s)
                    : launch_one<1, false, MODE>(a, lds, grid, s);
    return dist ? launch_one<2, true, MODE>(a, lds, grid, s)
                : launch_one<2, false, MODE>(a, lds, grid, s);
}

}  // namespace

hipError_t launch_wide(FusedMode mode, int nsp, bool dist, const FArgs &a, size_t lds_bytes,
                       dim3 grid, hipStream_t s) {
    switch (mode) {
    case MODE_FWD: return launch_mode<MODE_FWD>(nsp, dist, a, lds_bytes, grid, s);
    case MODE_BWDQ: return launch_mode<MODE_BWDQ>(nsp, dist, a, lds_bytes, grid, s);
    case MODE_BWDKV: return launch_mode<MODE_BWDKV>(nsp, dist, a, lds_bytes, grid, s);
    default: return hipErrorNotSupported;
    }
}

}  // namespace circatt
