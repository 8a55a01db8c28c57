// Kernel launchers shared between the kernel sources and the C-ABI layer.
#pragma once

#include "circatt.h"
#include "circatt_common.h"

namespace circatt {

hipError_t launch_pattern(const Geom &g, int64_t nb, int32_t *rowptr, int32_t *colval,
                          hipStream_t s);
hipError_t launch_softmax(int K, int64_t rows, const float *in, float *out, hipStream_t s);
hipError_t launch_softmax_bwd(int K, int64_t rows, const float *A, const float *dA, float *dS,
                              hipStream_t s);
// y = scale * (op(A) ⊗ x - [corr] sums(A) .* z), op = identity or transpose
hipError_t launch_apply(bool trans, bool corr, int ncomp, const Geom &g, int C, int64_t nb,
                        float scale, const float *nz, const float *x, const float *z, float *y,
                        hipStream_t s);
// Register-blocked form of launch_apply for windows 3 .. 15 (apply_rb.hip);
// launch_apply routes there when apply_rb_supported holds.
bool apply_rb_supported(const Geom &g, int C, int ncomp, int64_t nb);
hipError_t launch_apply_rb(bool trans, bool corr, int ncomp, const Geom &g, int C, int64_t nb,
                           float scale, const float *nz, const float *x, const float *z, float *y,
                           hipStream_t s);
// nzVal = scale * similarity for 2D windows 3 .. 15 (apply_rb.hip)
bool sim_rows_supported(const Geom &g, int C, int ncomp, int64_t nb);
hipError_t launch_sim_rows(bool dist, int ncomp, const Geom &g, int C, int64_t nb, float scale,
                           const float *x, const float *y, float *nz, hipStream_t s);
// colsum (sum(A; dims=1)) through the transposed product's offset tables
hipError_t launch_colsum_rb(const Geom &g, int64_t nb, const float *nz, float *out, hipStream_t s);
// Windows of any odd width in 1D and 2D (sub-rows of 16 window columns);
// launch_apply / launch_sum route there for windows wider than 15.
bool apply_wide_supported(const Geom &g, int C, int ncomp, int64_t nb);
hipError_t launch_apply_wide(bool trans, bool corr, int ncomp, const Geom &g, int C, int64_t nb,
                             float scale, const float *nz, const float *x, const float *z, float *y,
                             hipStream_t s);
hipError_t launch_colsum_wide(const Geom &g, int64_t nb, const float *nz, float *out,
                              hipStream_t s);
// The similarity pullback's two products in one grid (2D windows up to 15,
// and windows past 15 in 1D and 2D):
// dx = A ⊗ y, dy = Aᵀ ⊗ x, with the Distance terms when corr.
bool apply_pair_supported(const Geom &g, int C, int ncomp, int64_t nb);
hipError_t launch_apply_pair(bool corr, int ncomp, const Geom &g, int C, int64_t nb, float scale,
                             const float *nz, const float *x, const float *y, float *dx,
                             float *dy, hipStream_t s);
// Similarity for windows of any odd width in 1D and 2D (sub-row tasks).
bool sim_wide_supported(const Geom &g, int C, int ncomp, int64_t nb);
hipError_t launch_sim_wide(bool dist, int ncomp, const Geom &g, int C, int64_t nb, float scale,
                           const float *x, const float *y, float *nz, hipStream_t s);
hipError_t launch_similarity(bool dist, int ncomp, const Geom &g, int C, int64_t nb, float scale,
                             const float *x, const float *y, float *nz, hipStream_t s);
hipError_t launch_sum(bool col, const Geom &g, int64_t nb, const float *nz, float *out,
                      hipStream_t s);
// out[b] = sum_i X[i, b] * Y[i, b] (Y == nullptr: sum_i X[i, b]); work holds
// nb * batch_dot_chunks(nnz) doubles
int batch_dot_chunks(int64_t nnz);
hipError_t launch_batch_dot(int64_t nnz, int64_t nb, const float *X, const float *Y, float *out,
                            void *work, hipStream_t s);
hipError_t launch_axpby(int64_t nnz, int64_t nb, const float *alpha, float alpha0,
                        const float *X, const float *beta, float beta0, const float *Y, float *Z,
                        hipStream_t s);

// Batch-dimension operations (batch_ops.hip): fill with a 32-bit pattern;
// strided block copy dst[o*dso + i*dsi + e] = src[o*sso + i*ssi + e] (bytes,
// e < block); dst[i + inner*o] = sum_s src[i + inner*(s + nsum*o)]; count of
// unequal 32-bit words (floats: as Float32 values) into one device int64.
hipError_t launch_fill(uint32_t *dst, int64_t n, uint32_t bits, hipStream_t s);
hipError_t launch_copy_blocks(void *dst, const void *src, int64_t block, int64_t ninner,
                              int64_t dsi, int64_t ssi, int64_t nouter, int64_t dso, int64_t sso,
                              hipStream_t s);
hipError_t launch_sum_middle(const float *src, float *dst, int64_t inner, int64_t nsum,
                             int64_t outer, hipStream_t s);
hipError_t launch_count_unequal(bool floats, int64_t n, const uint32_t *a, const uint32_t *b,
                                int64_t *count, hipStream_t s);

// Arithmetic of the fused kernels' matrix products (circatt_set_math):
// CIRCATT_MATH_SPLIT_F16 or CIRCATT_MATH_F32.
int math_mode();

// Fused (MFMA) kernels.  Modes of the windowed-tile kernel family:
enum FusedMode {
    MODE_FWD = 0,   // y, lse                         (flash forward)
    MODE_SIM = 1,   // nzval = scale * sim, CSR order (unfused similarity)
    MODE_BWDQ = 2,  // dq and D = <dy, y>             (query-centric backward)
    MODE_BWDKV = 3  // dk, dv                         (key-centric backward)
};

struct FusedProblem {
    Geom g;
    int kind;     // CIRCATT_DOT / CIRCATT_DISTANCE
    int ncomp;    // 1 real, 2 complex
    int dh;       // channels per head (per unit)
    int64_t nunits;
    float scale;  // similarity scale
    int cl;       // 1: channels-last tensors (C, spatial..., B)
    int nheads;   // heads per image (units = nheads * B, head fastest)
    const float *q, *k, *v, *y, *dy, *lse;
    float *yout, *lse_out, *dq, *dk, *dv, *dbuf, *nz;
};

// Returns hipErrorNotSupported (never launching) if the shape is outside the
// supported range: dh*ncomp > 64 or a 1D halo that exceeds LDS.
hipError_t launch_fused(FusedMode mode, const FusedProblem &pr, hipStream_t s);
bool fused_supported(FusedMode mode, const FusedProblem &pr);

}  // namespace circatt
