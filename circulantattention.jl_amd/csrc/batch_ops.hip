// Batch-dimension operations of the Circulant type on the device: fill,
// strided block copies (repeat and cat over batch dims, broadcasts of
// per-slice factors), sums over one batch dim, and element comparison.
//
// They replace the array-library kernels the reference gets from CUDA.jl on
// a Circulant's CSR arrays (CUDA.ones, repeat, cat, sum over dims, ==:
// src/circulant.jl:68,90, src/array.jl:9,49-64,87-101,132-154,179-186), so
// that a host binding launches nothing outside libcircatt.  None is on the
// attention's hot path: each is one memory-bound grid-stride pass.
#include "circatt_kernels.h"

namespace circatt {
namespace {

constexpr int kThreads = 256;

unsigned grid_of(int64_t units) {
    int64_t b = (units + kThreads - 1) / kThreads;
    b = b < 1 ? 1 : b;
    return (unsigned)(b < (1 << 16) ? b : (1 << 16));
}

__global__ __launch_bounds__(kThreads) void fill_kernel(uint32_t *__restrict__ dst, int64_t n,
                                                        uint32_t bits) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) dst[i] = bits;
}

// Unit of U bytes: 16, 8, 4 or 1.
template <int U>
struct Unit;
template <>
struct Unit<16> {
    typedef uint32_t T __attribute__((ext_vector_type(4)));
};
template <>
struct Unit<8> {
    typedef uint32_t T __attribute__((ext_vector_type(2)));
};
template <>
struct Unit<4> {
    typedef uint32_t T;
};
template <>
struct Unit<1> {
    typedef uint8_t T;
};

// dst[o*dso + i*dsi + e] = src[o*sso + i*ssi + e] for e < upb units, i <
// ninner, o < nouter (all in units of U bytes).  IDX is the index type
// (32-bit when the unit count fits, whose divisions are cheaper).
template <int U, typename IDX>
__global__ __launch_bounds__(kThreads) void copy_blocks_kernel(
    typename Unit<U>::T *__restrict__ dst, const typename Unit<U>::T *__restrict__ src, IDX upb,
    IDX ninner, IDX nouter, int64_t dsi, int64_t ssi, int64_t dso, int64_t sso) {
    const IDX total = upb * ninner * nouter;
    const IDX stride = (IDX)gridDim.x * kThreads;
    for (IDX u = (IDX)blockIdx.x * kThreads + threadIdx.x; u < total; u += stride) {
        const IDX t = u / upb, e = u - t * upb;
        const IDX o = t / ninner, i = t - o * ninner;
        dst[(int64_t)o * dso + (int64_t)i * dsi + e] = src[(int64_t)o * sso + (int64_t)i * ssi + e];
    }
}

template <int U>
hipError_t copy_blocks_u(void *dst, const void *src, int64_t block, int64_t ninner, int64_t dsi,
                         int64_t ssi, int64_t nouter, int64_t dso, int64_t sso, hipStream_t s) {
    using T = typename Unit<U>::T;
    const int64_t upb = block / U;
    const int64_t total = upb * ninner * nouter;
    T *d = static_cast<T *>(dst);
    const T *c = static_cast<const T *>(src);
    const unsigned grid = grid_of(total);
    if (total < ((int64_t)1 << 31))
        hipLaunchKernelGGL((copy_blocks_kernel<U, uint32_t>), dim3(grid), dim3(kThreads), 0, s, d, c,
                           (uint32_t)upb, (uint32_t)ninner, (uint32_t)nouter, dsi / U, ssi / U,
                           dso / U, sso / U);
    else
        hipLaunchKernelGGL((copy_blocks_kernel<U, uint64_t>), dim3(grid), dim3(kThreads), 0, s, d, c,
                           (uint64_t)upb, (uint64_t)ninner, (uint64_t)nouter, dsi / U, ssi / U,
                           dso / U, sso / U);
    return hipGetLastError();
}

// dst[i + inner*o] = sum_s src[i + inner*(s + nsum*o)], summed in double in
// order of s (reproducible)
__global__ __launch_bounds__(kThreads) void sum_middle_kernel(const float *__restrict__ src,
                                                              float *__restrict__ dst, int64_t inner,
                                                              int64_t nsum, int64_t outer) {
    const int64_t n = inner * outer;
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x; j < n; j += stride) {
        const int64_t o = j / inner, i = j - o * inner;
        const float *p = src + i + inner * nsum * o;
        double acc = 0.0;
        for (int64_t s = 0; s < nsum; ++s) acc += (double)p[inner * s];
        dst[j] = (float)acc;
    }
}

__global__ void zero_count_kernel(unsigned long long *count) { *count = 0ull; }

// number of positions i < n where a[i] != b[i]: 32-bit words (FLOATS false)
// or Float32 values compared as floats (-0 == 0, NaN != NaN); one atomic add
// per wavefront
template <bool FLOATS>
__global__ __launch_bounds__(kThreads) void count_unequal_kernel(const uint32_t *__restrict__ a,
                                                                 const uint32_t *__restrict__ b,
                                                                 int64_t n,
                                                                 unsigned long long *count) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    unsigned long long c = 0;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        const uint32_t x = a[i], y = b[i];
        const bool ne = FLOATS ? !(__uint_as_float(x) == __uint_as_float(y)) : x != y;
        c += ne ? 1ull : 0ull;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o);
    if ((threadIdx.x & 63) == 0 && c != 0) atomicAdd(count, c);
}

}  // namespace

hipError_t launch_fill(uint32_t *dst, int64_t n, uint32_t bits, hipStream_t s) {
    hipLaunchKernelGGL(fill_kernel, dim3(grid_of(n)), dim3(kThreads), 0, s, dst, n, bits);
    return hipGetLastError();
}

hipError_t launch_copy_blocks(void *dst, const void *src, int64_t block, int64_t ninner,
                              int64_t dsi, int64_t ssi, int64_t nouter, int64_t dso, int64_t sso,
                              hipStream_t s) {
    // widest unit that divides both addresses, the block and every stride
    const uint64_t bits = (uint64_t)(uintptr_t)dst | (uint64_t)(uintptr_t)src | (uint64_t)block |
                          (uint64_t)dsi | (uint64_t)ssi | (uint64_t)dso | (uint64_t)sso;
    if ((bits & 15) == 0) return copy_blocks_u<16>(dst, src, block, ninner, dsi, ssi, nouter, dso, sso, s);
    if ((bits & 7) == 0) return copy_blocks_u<8>(dst, src, block, ninner, dsi, ssi, nouter, dso, sso, s);
    if ((bits & 3) == 0) return copy_blocks_u<4>(dst, src, block, ninner, dsi, ssi, nouter, dso, sso, s);
    return copy_blocks_u<1>(dst, src, block, ninner, dsi, ssi, nouter, dso, sso, s);
}

hipError_t launch_sum_middle(const float *src, float *dst, int64_t inner, int64_t nsum,
                             int64_t outer, hipStream_t s) {
    hipLaunchKernelGGL(sum_middle_kernel, dim3(grid_of(inner * outer)), dim3(kThreads), 0, s, src,
                       dst, inner, nsum, outer);
    return hipGetLastError();
}

hipError_t launch_count_unequal(bool floats, int64_t n, const uint32_t *a, const uint32_t *b,
                                int64_t *count, hipStream_t s) {
    auto *c = reinterpret_cast<unsigned long long *>(count);
    hipLaunchKernelGGL(zero_count_kernel, dim3(1), dim3(1), 0, s, c);
    if (n == 0) return hipGetLastError();
    if (floats)
        hipLaunchKernelGGL(count_unequal_kernel<true>, dim3(grid_of(n)), dim3(kThreads), 0, s, a, b,
                           n, c);
    else
        hipLaunchKernelGGL(count_unequal_kernel<false>, dim3(grid_of(n)), dim3(kThreads), 0, s, a,
                           b, n, c);
    return hipGetLastError();
}

}  // namespace circatt
