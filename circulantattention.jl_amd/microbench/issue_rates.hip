// Issue cost of single gfx950 instructions and of mixed streams, in cycles of
// one SIMD shared by four wavefronts (256 workgroups of 1024 threads: one per
// CU, four waves per SIMD).  Each wave runs R iterations of a fixed
// instruction group on its own registers; the slowest wave's s_memtime span
// divided by (R x 4 waves) is the SIMD's cost of one group.
//
// Build and run (one MI355X):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       circulantattention.jl_amd/microbench/issue_rates.hip -o /tmp/issue_rates && /tmp/issue_rates
//
// The groups are written in inline assembly so that the instruction stream is
// exactly the one named; the fused kernels' cost model (which instructions run
// at full, half or quarter rate, and that matrix-core and vector instructions
// of one SIMD do not overlap) comes from these numbers.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int R = 256;
constexpr int WAVES_PER_SIMD = 4;

#define OPS8 "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7)

// A group of vector instructions on the eight registers a0..a7; %8 is an SGPR
// holding a float, %9 an SGPR pair holding a lane mask.
#define VEC_KERNEL(NAME, BODY)                                                              \
    __global__ void NAME(float *out, uint64_t *cyc, float seed) {                          \
        float a0 = seed + threadIdx.x, a1 = a0 + 1, a2 = a0 + 2, a3 = a0 + 3;              \
        float a4 = a0 + 4, a5 = a0 + 5, a6 = a0 + 6, a7 = a0 + 7;                          \
        const float sc = seed;                                                            \
        const uint64_t sm = 0x5555aaaa3333ccccull;                                        \
        __syncthreads();                                                                  \
        const uint64_t t0 = __builtin_readcyclecounter();                                 \
        for (int r = 0; r < R; ++r) asm volatile(BODY : OPS8 : "s"(sc), "s"(sm) : "vcc"); \
        const uint64_t t1 = __builtin_readcyclecounter();                                 \
        out[blockIdx.x * blockDim.x + threadIdx.x] = a0 + a1 + a2 + a3 + a4 + a5 + a6 + a7; \
        if ((threadIdx.x & 63) == 0) cyc[blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64] = t1 - t0; \
    }

#define X8(I) I(0, 3) I(1, 4) I(2, 5) I(3, 6) I(4, 7) I(5, 0) I(6, 1) I(7, 2)
#define ADD(d, a) "v_add_f32 %" #d ", %" #a ", %" #d "\n"
#define MULS(d, a) "v_mul_f32 %" #d ", %8, %" #d "\n"
#define MAX(d, a) "v_max_f32 %" #d ", %" #a ", %" #d "\n"
#define CND(d, a) "v_cndmask_b32_e64 %" #d ", %" #d ", %" #a ", %9\n"
#define CVTPK(d, a) "v_cvt_pk_f16_f32 %" #d ", %" #a ", %" #d "\n"
#define MIXF32(d, a) "v_fma_mix_f32 %" #d ", %" #a ", %8, %" #d " op_sel_hi:[1,0,0]\n"
#define MIXLO(d, a) "v_fma_mixlo_f16 %" #d ", %" #a ", %8, %" #d " op_sel_hi:[1,0,0]\n"
#define EXP(d, a) "v_exp_f32 %" #d ", %" #a "\n"
#define LDEXP(d, a) "v_ldexp_f32 %" #d ", %" #d ", 3\n"
// a half-rate instruction followed by three independent adds
#define CND_ADD3(d, a) CND(d, a) "v_add_f32 %" #a ", 1.0, %" #a "\n" ADD(d, d) ADD(d, d)
#define ADD4(d, a) ADD(d, a) "v_add_f32 %" #a ", 1.0, %" #a "\n" ADD(d, d) ADD(d, d)

VEC_KERNEL(k_add, X8(ADD) X8(ADD))
VEC_KERNEL(k_mul_sgpr, X8(MULS) X8(MULS))
VEC_KERNEL(k_max, X8(MAX) X8(MAX))
VEC_KERNEL(k_cndmask, X8(CND) X8(CND))
VEC_KERNEL(k_cvt_pk, X8(CVTPK) X8(CVTPK))
VEC_KERNEL(k_mix_f32, X8(MIXF32) X8(MIXF32))
VEC_KERNEL(k_mixlo, X8(MIXLO) X8(MIXLO))
VEC_KERNEL(k_exp, X8(EXP) X8(EXP))
VEC_KERNEL(k_ldexp, X8(LDEXP) X8(LDEXP))
VEC_KERNEL(k_cnd_add3, X8(CND_ADD3))
VEC_KERNEL(k_add4, X8(ADD4))

// MFMA v_mfma_f32_16x16x32_f16 with N independent v_add_f32 after each one.
template <int N>
__global__ void k_mfma_valu(float *out, uint64_t *cyc, float seed) {
    float a0 = seed + threadIdx.x, a1 = a0 + 1, a2 = a0 + 2, a3 = a0 + 3;
    float a4 = a0 + 4, a5 = a0 + 5, a6 = a0 + 6, a7 = a0 + 7;
    const h8 x = (h8)(_Float16)(seed * 0.001f), y = (h8)(_Float16)(seed * 0.002f);
    f4 c0 = {a0, a1, a2, a3}, c1 = c0 + 1.f;
    __syncthreads();
    const uint64_t t0 = __builtin_readcyclecounter();
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(x, y, c0, 0, 0, 0);
            if constexpr (N >= 4)
                asm volatile("v_add_f32 %0, 1.0, %0\n v_add_f32 %1, 1.0, %1\n v_add_f32 %2, 1.0, %2\n"
                             " v_add_f32 %3, 1.0, %3" : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3));
            if constexpr (N >= 8)
                asm volatile("v_add_f32 %0, 1.0, %0\n v_add_f32 %1, 1.0, %1\n v_add_f32 %2, 1.0, %2\n"
                             " v_add_f32 %3, 1.0, %3" : "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7));
            c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(x, y, c1, 0, 0, 0);
            if constexpr (N >= 4)
                asm volatile("v_add_f32 %0, 1.0, %0\n v_add_f32 %1, 1.0, %1\n v_add_f32 %2, 1.0, %2\n"
                             " v_add_f32 %3, 1.0, %3" : "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7));
            if constexpr (N >= 8)
                asm volatile("v_add_f32 %0, 1.0, %0\n v_add_f32 %1, 1.0, %1\n v_add_f32 %2, 1.0, %2\n"
                             " v_add_f32 %3, 1.0, %3" : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3));
        }
    }
    const uint64_t t1 = __builtin_readcyclecounter();
    out[blockIdx.x * blockDim.x + threadIdx.x] =
        a0 + a1 + a2 + a3 + a4 + a5 + a6 + a7 + c0[0] + c1[1];
    if ((threadIdx.x & 63) == 0) cyc[blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64] = t1 - t0;
}

template <typename K>
static void run(K kern, const char *name, int groups_per_iter, float *out, uint64_t *cyc) {
    const int threads = 256 * WAVES_PER_SIMD;
    for (int rep = 0; rep < 2; ++rep)
        hipLaunchKernelGGL(kern, dim3(256), dim3(threads), 0, 0, out, cyc, 0.5f);
    if (hipDeviceSynchronize() != hipSuccess) {
        printf("%s: launch failed\n", name);
        return;
    }
    const int nw = 256 * threads / 64;
    static uint64_t h[256 * 16];
    if (hipMemcpy(h, cyc, nw * 8, hipMemcpyDeviceToHost) != hipSuccess) return;
    uint64_t mx = 0;
    for (int i = 0; i < nw; ++i) mx = h[i] > mx ? h[i] : mx;
    printf("%-44s %6.2f cycles per group\n", name,
           (double)mx / ((double)R * groups_per_iter * WAVES_PER_SIMD));
}

int main() {
    float *out = nullptr;
    uint64_t *cyc = nullptr;
    if (hipMalloc(&out, 256 * 1024 * 4) != hipSuccess || hipMalloc(&cyc, 256 * 16 * 8) != hipSuccess)
        return 1;
    printf("SIMD cycles, 4 waves per SIMD (gfx950)\n");
    run(k_add, "v_add_f32 (VGPR operands)", 16, out, cyc);
    run(k_mul_sgpr, "v_mul_f32 with an SGPR operand", 16, out, cyc);
    run(k_max, "v_max_f32", 16, out, cyc);
    run(k_cndmask, "v_cndmask_b32 (SGPR-pair mask)", 16, out, cyc);
    run(k_cvt_pk, "v_cvt_pk_f16_f32", 16, out, cyc);
    run(k_mix_f32, "v_fma_mix_f32", 16, out, cyc);
    run(k_mixlo, "v_fma_mixlo_f16", 16, out, cyc);
    run(k_exp, "v_exp_f32", 16, out, cyc);
    run(k_ldexp, "v_ldexp_f32", 16, out, cyc);
    run(k_add4, "group: 4 v_add_f32", 8, out, cyc);
    run(k_cnd_add3, "group: v_cndmask_b32 + 3 v_add_f32", 8, out, cyc);
    run(k_mfma_valu<0>, "group: mfma 16x16x32 f16", 8, out, cyc);
    run(k_mfma_valu<4>, "group: mfma + 4 independent v_add_f32", 8, out, cyc);
    run(k_mfma_valu<8>, "group: mfma + 8 independent v_add_f32", 8, out, cyc);
    return 0;
}
