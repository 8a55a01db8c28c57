// C-ABI layer of libcircatt: host-side validation (the reference's @assert
// checks, src/circulant.jl:65,87, src/similarity.jl:43-44,
// src/attention.jl:54,73, src/array.jl:133,142,180) and kernel dispatch.
// No entry point allocates device memory.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "circatt.h"
#include "circatt_kernels.h"

using namespace circatt;

namespace circatt {
namespace {
std::atomic<int> g_math{CIRCATT_MATH_SPLIT_F16};
}
int math_mode() { return g_math.load(std::memory_order_relaxed); }
}  // namespace circatt

namespace {

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int ok() {
    g_last_error.clear();
    return CIRCATT_OK;
}

int hip_result(hipError_t e, const char *what) {
    if (e == hipSuccess) return ok();
    if (e == hipErrorNotSupported)
        return fail(CIRCATT_ERR_UNSUPPORTED, "%s: shape not supported by the HIP kernels", what);
    return fail(CIRCATT_ERR_HIP, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
}

hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// Validates (nsp, n1, n2, ws) and fills g.  Returns 0 or an error code.
int check_geom(int nsp, int64_t n1, int64_t n2, int32_t ws, Geom &g) {
    if (nsp != 1 && nsp != 2) return fail(CIRCATT_ERR_INVALID, "nsp=%d must be 1 or 2", nsp);
    if (ws < 1 || ws % 2 != 1) return fail(CIRCATT_ERR_INVALID, "filter size M=%d must be odd.", ws);
    if (n1 < 1 || n1 > INT32_MAX) return fail(CIRCATT_ERR_INVALID, "invalid spatial size n1=%lld", (long long)n1);
    if (nsp == 2 && (n2 < 1 || n2 > INT32_MAX))
        return fail(CIRCATT_ERR_INVALID, "invalid spatial size n2=%lld", (long long)n2);
    if (nsp == 2 && (int64_t)ws * ws > INT32_MAX)
        return fail(CIRCATT_ERR_INVALID, "window %d too large", ws);
    g = make_geom(nsp, (int)n1, nsp == 2 ? (int)n2 : 1, ws);
    // colVal / rowPtr are Int32 (src/circulant.jl:64,86): P*K+1 must fit.
    if (g.P * (int64_t)g.K + 1 > INT32_MAX)
        return fail(CIRCATT_ERR_INVALID, "P*K = %lld exceeds the Int32 index range",
                    (long long)(g.P * (int64_t)g.K));
    return CIRCATT_OK;
}

int check_dtype(int dtype) {
    if (dtype != CIRCATT_F32 && dtype != CIRCATT_C32)
        return fail(CIRCATT_ERR_UNSUPPORTED, "dtype %d not supported (Float32 or ComplexF32)", dtype);
    return CIRCATT_OK;
}

int check_kind(int kind) {
    if (kind != CIRCATT_DOT && kind != CIRCATT_DISTANCE)
        return fail(CIRCATT_ERR_INVALID, "unknown similarity kind %d", kind);
    return CIRCATT_OK;
}

#define CIRCATT_TRY(expr)            \
    do {                             \
        int _rc = (expr);            \
        if (_rc != CIRCATT_OK) return _rc; \
    } while (0)

#define CIRCATT_NONNULL(p)                                                  \
    do {                                                                    \
        if ((p) == nullptr) return fail(CIRCATT_ERR_INVALID, "%s is NULL", #p); \
    } while (0)

}  // namespace

extern "C" {

int circatt_version(void) { return 10000; }

int circatt_set_math(int mode) {
    if (mode != CIRCATT_MATH_SPLIT_F16 && mode != CIRCATT_MATH_F32)
        return fail(CIRCATT_ERR_INVALID, "unknown math mode %d", mode);
    g_math.store(mode, std::memory_order_relaxed);
    return ok();
}

int circatt_get_math(void) { return math_mode(); }

const char *circatt_last_error(void) { return g_last_error.c_str(); }

int circatt_pattern(int nsp, int64_t n1, int64_t n2, int32_t ws, int64_t nb, int32_t *rowptr,
                    int32_t *colval, void *stream) {
    Geom g;
    CIRCATT_TRY(check_geom(nsp, n1, n2, ws, g));
    if (nb < 1) return fail(CIRCATT_ERR_INVALID, "nb=%lld must be >= 1", (long long)nb);
    CIRCATT_NONNULL(rowptr);
    CIRCATT_NONNULL(colval);
    return hip_result(launch_pattern(g, nb, rowptr, colval, as_stream(stream)), "circatt_pattern");
}

int circatt_similarity(int kind, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws,
                       int64_t C, int64_t nb, float scale, const void *x, const void *y,
                       float *nzval, void *stream) {
    Geom g;
    CIRCATT_TRY(check_kind(kind));
    CIRCATT_TRY(check_dtype(dtype));
    CIRCATT_TRY(check_geom(nsp, n1, n2, ws, g));
    if (C < 1 || C > INT32_MAX) return fail(CIRCATT_ERR_INVALID, "invalid channel count %lld", (long long)C);
    if (nb < 1) return fail(CIRCATT_ERR_INVALID, "nb=%lld must be >= 1", (long long)nb);
    CIRCATT_NONNULL(x);
    CIRCATT_NONNULL(y);
    CIRCATT_NONNULL(nzval);
    const int ncomp = dtype == CIRCATT_C32 ? 2 : 1;
    FusedProblem pr{};
    pr.g = g;
    pr.kind = kind;
    pr.ncomp = ncomp;
    pr.dh = (int)C;
    pr.nunits = nb;
    pr.scale = scale;
    pr.q = static_cast<const float *>(x);
    pr.k = static_cast<const float *>(y);
    pr.nz = nzval;
    // 2D windows up to 15 wide: the row kernel (faster than the matrix-core
    // kernel at every measured size); wider windows, 1D or 2D, and every
    // Distance similarity the row kernel does not take: the sub-row kernel
    // (both form -|x - y|^2 / 2 from the differences, as the reference does,
    // where the matrix-core kernel expands it); otherwise the matrix-core
    // kernel
    const bool rows_ok = sim_rows_supported(g, (int)C, ncomp, nb);
    const bool mfma_ok = fused_supported(MODE_SIM, pr);
    if (!rows_ok && (g.ws > 15 || kind == CIRCATT_DISTANCE) &&
        sim_wide_supported(g, (int)C, ncomp, nb))
        return hip_result(launch_sim_wide(kind == CIRCATT_DISTANCE, ncomp, g, (int)C, nb, scale,
                                          pr.q, pr.k, nzval, as_stream(stream)),
                          "circatt_similarity");
    if (rows_ok)
        return hip_result(launch_sim_rows(kind == CIRCATT_DISTANCE, ncomp, g, (int)C, nb, scale,
                                          pr.q, pr.k, nzval, as_stream(stream)),
                          "circatt_similarity");
    if (mfma_ok)
        return hip_result(launch_fused(MODE_SIM, pr, as_stream(stream)), "circatt_similarity");
    return hip_result(launch_similarity(kind == CIRCATT_DISTANCE, ncomp, g, (int)C, nb, scale,
                                        pr.q, pr.k, nzval, as_stream(stream)),
                      "circatt_similarity");
}

int circatt_softmax(int64_t K, int64_t rows, const float *in, float *out, void *stream) {
    if (K < 1 || K > INT32_MAX) return fail(CIRCATT_ERR_INVALID, "invalid K=%lld", (long long)K);
    if (rows < 0) return fail(CIRCATT_ERR_INVALID, "invalid rows=%lld", (long long)rows);
    if (rows == 0) return ok();
    CIRCATT_NONNULL(in);
    CIRCATT_NONNULL(out);
    return hip_result(launch_softmax((int)K, rows, in, out, as_stream(stream)), "circatt_softmax");
}

int circatt_softmax_bwd(int64_t K, int64_t rows, const float *A, const float *dA, float *dS,
                        void *stream) {
    if (K < 1 || K > INT32_MAX) return fail(CIRCATT_ERR_INVALID, "invalid K=%lld", (long long)K);
    if (rows < 0) return fail(CIRCATT_ERR_INVALID, "invalid rows=%lld", (long long)rows);
    if (rows == 0) return ok();
    CIRCATT_NONNULL(A);
    CIRCATT_NONNULL(dA);
    CIRCATT_NONNULL(dS);
    return hip_result(launch_softmax_bwd((int)K, rows, A, dA, dS, as_stream(stream)),
                      "circatt_softmax_bwd");
}

int circatt_apply(int trans, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws, int64_t C,
                  int64_t nb, const float *nzval, const void *x, void *y, void *stream) {
    Geom g;
    CIRCATT_TRY(check_dtype(dtype));
    CIRCATT_TRY(check_geom(nsp, n1, n2, ws, g));
    if (trans != 0 && trans != 1) return fail(CIRCATT_ERR_INVALID, "trans=%d must be 0 or 1", trans);
    if (C < 1 || C > INT32_MAX) return fail(CIRCATT_ERR_INVALID, "invalid channel count %lld", (long long)C);
    if (nb < 1) return fail(CIRCATT_ERR_INVALID, "nb=%lld must be >= 1", (long long)nb);
    CIRCATT_NONNULL(nzval);
    CIRCATT_NONNULL(x);
    CIRCATT_NONNULL(y);
    if (x == y) return fail(CIRCATT_ERR_INVALID, "x and y must not alias");
    return hip_result(launch_apply(trans == 1, false, dtype == CIRCATT_C32 ? 2 : 1, g, (int)C, nb,
                                   1.f, nzval, static_cast<const float *>(x), nullptr,
                                   static_cast<float *>(y), as_stream(stream)),
                      "circatt_apply");
}

int circatt_similarity_bwd(int kind, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws,
                           int64_t C, int64_t nb, float scale, const float *dS, const void *x,
                           const void *y, void *dx, void *dy, void *stream) {
    Geom g;
    CIRCATT_TRY(check_kind(kind));
    CIRCATT_TRY(check_dtype(dtype));
    CIRCATT_TRY(check_geom(nsp, n1, n2, ws, g));
    if (C < 1 || C > INT32_MAX) return fail(CIRCATT_ERR_INVALID, "invalid channel count %lld", (long long)C);
    if (nb < 1) return fail(CIRCATT_ERR_INVALID, "nb=%lld must be >= 1", (long long)nb);
    CIRCATT_NONNULL(dS);
    CIRCATT_NONNULL(x);
    CIRCATT_NONNULL(y);
    const int ncomp = dtype == CIRCATT_C32 ? 2 : 1;
    const bool dist = kind == CIRCATT_DISTANCE;
    const float *xf = static_cast<const float *>(x);
    const float *yf = static_cast<const float *>(y);
    if (dx && dy && apply_pair_supported(g, (int)C, ncomp, nb)) {
        // both products in one grid
        if (dx == x || dx == y) return fail(CIRCATT_ERR_INVALID, "dx must not alias x or y");
        if (dy == x || dy == y) return fail(CIRCATT_ERR_INVALID, "dy must not alias x or y");
        return hip_result(launch_apply_pair(dist, ncomp, g, (int)C, nb, scale, dS, xf, yf,
                                            static_cast<float *>(dx), static_cast<float *>(dy),
                                            as_stream(stream)),
                          "circatt_similarity_bwd");
    }
    if (dx) {
        if (dx == x || dx == y) return fail(CIRCATT_ERR_INVALID, "dx must not alias x or y");
        hipError_t e = launch_apply(false, dist, ncomp, g, (int)C, nb, scale, dS, yf, xf,
                                    static_cast<float *>(dx), as_stream(stream));
        if (e != hipSuccess) return hip_result(e, "circatt_similarity_bwd");
    }
    if (dy) {
        if (dy == x || dy == y) return fail(CIRCATT_ERR_INVALID, "dy must not alias x or y");
        hipError_t e = launch_apply(true, dist, ncomp, g, (int)C, nb, scale, dS, xf, yf,
                                    static_cast<float *>(dy), as_stream(stream));
        if (e != hipSuccess) return hip_result(e, "circatt_similarity_bwd");
    }
    return ok();
}

static int sum_impl(bool col, int nsp, int64_t n1, int64_t n2, int32_t ws, int64_t nb,
                    const float *nzval, float *out, void *stream, const char *name) {
    Geom g;
    CIRCATT_TRY(check_geom(nsp, n1, n2, ws, g));
    if (nb < 1) return fail(CIRCATT_ERR_INVALID, "nb=%lld must be >= 1", (long long)nb);
    CIRCATT_NONNULL(nzval);
    CIRCATT_NONNULL(out);
    return hip_result(launch_sum(col, g, nb, nzval, out, as_stream(stream)), name);
}

int circatt_rowsum(int nsp, int64_t n1, int64_t n2, int32_t ws, int64_t nb, const float *nzval,
                   float *out, void *stream) {
    return sum_impl(false, nsp, n1, n2, ws, nb, nzval, out, stream, "circatt_rowsum");
}

int circatt_colsum(int nsp, int64_t n1, int64_t n2, int32_t ws, int64_t nb, const float *nzval,
                   float *out, void *stream) {
    return sum_impl(true, nsp, n1, n2, ws, nb, nzval, out, stream, "circatt_colsum");
}

int circatt_axpby(int64_t nnz, int64_t nb, const float *alpha, float alpha0, const float *X,
                  const float *beta, float beta0, const float *Y, float *Z, void *stream) {
    if (nnz < 0 || nb < 1) return fail(CIRCATT_ERR_INVALID, "invalid nnz=%lld / nb=%lld", (long long)nnz, (long long)nb);
    if (nnz == 0) return ok();
    CIRCATT_NONNULL(X);
    CIRCATT_NONNULL(Z);
    return hip_result(launch_axpby(nnz, nb, alpha, alpha0, X, beta, beta0, Y, Z, as_stream(stream)),
                      "circatt_axpby");
}

int64_t circatt_batch_dot_workspace_bytes(int64_t nnz, int64_t nb) {
    if (nnz < 0 || nb < 1) return -1;
    return nb * (int64_t)batch_dot_chunks(nnz) * (int64_t)sizeof(double);
}

int circatt_batch_dot(int64_t nnz, int64_t nb, const float *X, const float *Y, float *out,
                      void *workspace, int64_t workspace_bytes, void *stream) {
    if (nnz < 0 || nb < 1)
        return fail(CIRCATT_ERR_INVALID, "invalid nnz=%lld / nb=%lld", (long long)nnz, (long long)nb);
    CIRCATT_NONNULL(X);
    CIRCATT_NONNULL(out);
    CIRCATT_NONNULL(workspace);
    const int64_t need = circatt_batch_dot_workspace_bytes(nnz, nb);
    if (workspace_bytes < need)
        return fail(CIRCATT_ERR_INVALID, "workspace of %lld bytes, %lld needed",
                    (long long)workspace_bytes, (long long)need);
    if (out == X || out == Y || workspace == X || workspace == Y || workspace == out)
        return fail(CIRCATT_ERR_INVALID, "out and workspace must not alias X or Y");
    return hip_result(launch_batch_dot(nnz, nb, X, Y, out, workspace, as_stream(stream)),
                      "circatt_batch_dot");
}

static int fused_problem(int kind, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws,
                         int64_t C, int64_t nheads, int64_t B, FusedProblem &pr) {
    Geom g;
    const int cl = (dtype & CIRCATT_CHANNELS_LAST) ? 1 : 0;
    dtype &= ~CIRCATT_CHANNELS_LAST;
    CIRCATT_TRY(check_kind(kind));
    CIRCATT_TRY(check_dtype(dtype));
    CIRCATT_TRY(check_geom(nsp, n1, n2, ws, g));
    if (nheads < 1 || C < 1 || C % nheads != 0)
        return fail(CIRCATT_ERR_INVALID, "channels (%lld) must be divisible by nheads (%lld)",
                    (long long)C, (long long)nheads);
    if (B < 1) return fail(CIRCATT_ERR_INVALID, "batch B=%lld must be >= 1", (long long)B);
    pr = FusedProblem{};
    pr.g = g;
    pr.kind = kind;
    pr.ncomp = dtype == CIRCATT_C32 ? 2 : 1;
    pr.dh = (int)(C / nheads);
    pr.nunits = nheads * B;
    pr.cl = cl;
    pr.nheads = (int)nheads;
    if (cl && g.P * C * pr.ncomp * 4 >= (int64_t)INT32_MAX)
        return fail(CIRCATT_ERR_UNSUPPORTED,
                    "channels-last image of %lld floats exceeds the kernels' 32-bit offsets",
                    (long long)(g.P * C * pr.ncomp));
    // q ./ sqrt(tau), k ./ sqrt(tau), tau = sqrt(channels per head)
    // (src/attention.jl:20-21) scale the similarity by 1/sqrt(dh).
    pr.scale = (float)(1.0 / std::sqrt((double)pr.dh));
    return CIRCATT_OK;
}

int circatt_fused_fwd(int kind, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws,
                      int64_t C, int64_t nheads, int64_t B, const void *q, const void *k,
                      const void *v, void *y, float *lse, void *stream) {
    FusedProblem pr;
    CIRCATT_TRY(fused_problem(kind, dtype, nsp, n1, n2, ws, C, nheads, B, pr));
    CIRCATT_NONNULL(q);
    CIRCATT_NONNULL(k);
    CIRCATT_NONNULL(v);
    CIRCATT_NONNULL(y);
    CIRCATT_NONNULL(lse);
    if (y == q || y == k || y == v) return fail(CIRCATT_ERR_INVALID, "y must not alias q, k or v");
    pr.q = static_cast<const float *>(q);
    pr.k = static_cast<const float *>(k);
    pr.v = static_cast<const float *>(v);
    pr.yout = static_cast<float *>(y);
    pr.lse_out = lse;
    if (!fused_supported(MODE_FWD, pr))
        return fail(CIRCATT_ERR_UNSUPPORTED,
                    "circatt_fused_fwd: window ws=%d with %d real components per head is outside "
                    "the fused kernels' range", pr.g.ws, pr.dh * pr.ncomp);
    return hip_result(launch_fused(MODE_FWD, pr, as_stream(stream)), "circatt_fused_fwd");
}

int64_t circatt_fused_bwd_workspace_bytes(int nsp, int64_t n1, int64_t n2, int64_t nheads,
                                          int64_t B) {
    if ((nsp != 1 && nsp != 2) || n1 < 1 || (nsp == 2 && n2 < 1) || nheads < 1 || B < 1) return -1;
    const int64_t P = nsp == 1 ? n1 : n1 * n2;
    return P * nheads * B * (int64_t)sizeof(float);
}

namespace {

enum BwdParts { BWD_DQ = 1, BWD_DKDV = 2 };

int fused_bwd_impl(int parts, int kind, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws,
                   int64_t C, int64_t nheads, int64_t B, const void *q, const void *k,
                   const void *v, const void *y, const void *dy, const float *lse, void *dq,
                   void *dk, void *dv, const void *workspace, int64_t workspace_bytes,
                   void *stream, const char *name) {
    FusedProblem pr;
    CIRCATT_TRY(fused_problem(kind, dtype, nsp, n1, n2, ws, C, nheads, B, pr));
    CIRCATT_NONNULL(q);
    CIRCATT_NONNULL(k);
    CIRCATT_NONNULL(v);
    CIRCATT_NONNULL(dy);
    CIRCATT_NONNULL(lse);
    CIRCATT_NONNULL(workspace);
    if (parts & BWD_DQ) {
        CIRCATT_NONNULL(y);
        CIRCATT_NONNULL(dq);
    }
    if (parts & BWD_DKDV) {
        CIRCATT_NONNULL(dk);
        CIRCATT_NONNULL(dv);
    }
    const int64_t need = circatt_fused_bwd_workspace_bytes(nsp, n1, n2, nheads, B);
    if (workspace_bytes < need)
        return fail(CIRCATT_ERR_INVALID, "workspace of %lld bytes, %lld needed",
                    (long long)workspace_bytes, (long long)need);
    for (const void *out : {dq, dk, dv}) {
        if (out == nullptr) continue;
        for (const void *in : {q, k, v, y, dy, static_cast<const void *>(lse), workspace})
            if (out == in) return fail(CIRCATT_ERR_INVALID, "gradient outputs must not alias inputs");
    }
    pr.q = static_cast<const float *>(q);
    pr.k = static_cast<const float *>(k);
    pr.v = static_cast<const float *>(v);
    pr.y = static_cast<const float *>(y);
    pr.dy = static_cast<const float *>(dy);
    pr.lse = lse;
    pr.dq = static_cast<float *>(dq);
    pr.dk = static_cast<float *>(dk);
    pr.dv = static_cast<float *>(dv);
    pr.dbuf = static_cast<float *>(const_cast<void *>(workspace));
    if (!fused_supported(MODE_BWDQ, pr) || !fused_supported(MODE_BWDKV, pr))
        return fail(CIRCATT_ERR_UNSUPPORTED,
                    "%s: window ws=%d with %d real components per head is outside the fused "
                    "kernels' range", name, pr.g.ws, pr.dh * pr.ncomp);
    if (parts & BWD_DQ) {
        hipError_t e = launch_fused(MODE_BWDQ, pr, as_stream(stream));
        if (e != hipSuccess) return hip_result(e, name);
    }
    if (parts & BWD_DKDV) {
        hipError_t e = launch_fused(MODE_BWDKV, pr, as_stream(stream));
        if (e != hipSuccess) return hip_result(e, name);
    }
    return ok();
}

}  // namespace

int circatt_fused_bwd(int kind, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws,
                      int64_t C, int64_t nheads, int64_t B, const void *q, const void *k,
                      const void *v, const void *y, const void *dy, const float *lse, void *dq,
                      void *dk, void *dv, void *workspace, int64_t workspace_bytes,
                      void *stream) {
    return fused_bwd_impl(BWD_DQ | BWD_DKDV, kind, dtype, nsp, n1, n2, ws, C, nheads, B, q, k,
                          v, y, dy, lse, dq, dk, dv, workspace, workspace_bytes, stream,
                          "circatt_fused_bwd");
}

int circatt_fused_bwd_dq(int kind, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws,
                         int64_t C, int64_t nheads, int64_t B, const void *q, const void *k,
                         const void *v, const void *y, const void *dy, const float *lse,
                         void *dq, void *workspace, int64_t workspace_bytes, void *stream) {
    return fused_bwd_impl(BWD_DQ, kind, dtype, nsp, n1, n2, ws, C, nheads, B, q, k, v, y, dy,
                          lse, dq, nullptr, nullptr, workspace, workspace_bytes, stream,
                          "circatt_fused_bwd_dq");
}

int circatt_fused_bwd_dkdv(int kind, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws,
                           int64_t C, int64_t nheads, int64_t B, const void *q, const void *k,
                           const void *v, const void *dy, const float *lse, void *dk, void *dv,
                           const void *workspace, int64_t workspace_bytes, void *stream) {
    return fused_bwd_impl(BWD_DKDV, kind, dtype, nsp, n1, n2, ws, C, nheads, B, q, k, v,
                          nullptr, dy, lse, nullptr, dk, dv, workspace, workspace_bytes, stream,
                          "circatt_fused_bwd_dkdv");
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Fused backward without a workspace argument: the per-row D = <dy, y> lives
// in `scratch`, a file-scope device array of fixed size.  Each GPU the
// library runs on holds its own copy until the process ends; its device
// address is looked up once per device (hipGetSymbolAddress) and kept.
// ---------------------------------------------------------------------------
namespace {

constexpr int64_t kScratchBytes = int64_t(16) << 20;  // 4M rows of D
constexpr int kMaxDevices = 64;

static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's `scratch` (looked up on its first use).
int scratch_address(void **out, const char *name) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_result(e, name);
    if (dev < 0 || dev >= kMaxDevices)
        return fail(CIRCATT_ERR_UNSUPPORTED, "%s: device %d beyond the %d supported", name, dev,
                    kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_result(e, name);
        if (p == nullptr) return fail(CIRCATT_ERR_HIP, "%s: no device address for scratch", name);
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return CIRCATT_OK;
}

}  // namespace

extern "C" {

int64_t circatt_fused_bwd_noalloc_max_rows(void) {
    return kScratchBytes / (int64_t)sizeof(float);
}

int circatt_fused_bwd_noalloc(int kind, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws,
                              int64_t C, int64_t nheads, int64_t B, const void *q,
                              const void *k, const void *v, const void *y, const void *dy,
                              const float *lse, void *dq, void *dk, void *dv, void *stream) {
    const char *name = "circatt_fused_bwd_noalloc";
    const int64_t need = circatt_fused_bwd_workspace_bytes(nsp, n1, n2, nheads, B);
    if (need < 0) return fail(CIRCATT_ERR_INVALID, "%s: invalid shape", name);
    if (need > kScratchBytes)
        return fail(CIRCATT_ERR_INVALID,
                    "%s: %lld rows of D (P*nheads*B) exceed the static scratch of %lld rows; "
                    "use circatt_fused_bwd with a workspace",
                    name, (long long)(need / 4), (long long)(kScratchBytes / 4));
    FusedProblem pr;
    CIRCATT_TRY(fused_problem(kind, dtype, nsp, n1, n2, ws, C, nheads, B, pr));
    CIRCATT_NONNULL(q);
    CIRCATT_NONNULL(k);
    CIRCATT_NONNULL(v);
    CIRCATT_NONNULL(y);
    CIRCATT_NONNULL(dy);
    CIRCATT_NONNULL(lse);
    CIRCATT_NONNULL(dq);
    CIRCATT_NONNULL(dk);
    CIRCATT_NONNULL(dv);
    void *work = nullptr;
    CIRCATT_TRY(scratch_address(&work, name));
    return fused_bwd_impl(BWD_DQ | BWD_DKDV, kind, dtype, nsp, n1, n2, ws, C, nheads, B, q, k,
                          v, y, dy, lse, dq, dk, dv, work, need, stream, name);
}

int circatt_malloc(void **ptr, int64_t bytes) {
    CIRCATT_NONNULL(ptr);
    if (bytes < 0) return fail(CIRCATT_ERR_INVALID, "negative size");
    return hip_result(hipMalloc(ptr, (size_t)bytes), "circatt_malloc");
}

int circatt_free(void *ptr) { return hip_result(hipFree(ptr), "circatt_free"); }

int circatt_fill(float *dst, int64_t n, float value, void *stream) {
    if (n < 0) return fail(CIRCATT_ERR_INVALID, "n=%lld must be >= 0", (long long)n);
    if (n == 0) return ok();
    CIRCATT_NONNULL(dst);
    uint32_t bits;
    std::memcpy(&bits, &value, 4);
    return hip_result(launch_fill(reinterpret_cast<uint32_t *>(dst), n, bits, as_stream(stream)),
                      "circatt_fill");
}

int circatt_copy_blocks(void *dst, const void *src, int64_t block_bytes, int64_t ninner,
                        int64_t dst_stride_inner, int64_t src_stride_inner, int64_t nouter,
                        int64_t dst_stride_outer, int64_t src_stride_outer, void *stream) {
    if (block_bytes < 0 || ninner < 0 || nouter < 0)
        return fail(CIRCATT_ERR_INVALID, "negative block size or count");
    if (dst_stride_inner < 0 || src_stride_inner < 0 || dst_stride_outer < 0 || src_stride_outer < 0)
        return fail(CIRCATT_ERR_INVALID, "negative stride");
    if (block_bytes == 0 || ninner == 0 || nouter == 0) return ok();
    CIRCATT_NONNULL(dst);
    CIRCATT_NONNULL(src);
    // the destination blocks must not overlap (a destination byte written
    // twice would depend on the order of the writes)
    if ((ninner > 1 && dst_stride_inner < block_bytes) ||
        (nouter > 1 && dst_stride_outer < (ninner - 1) * dst_stride_inner + block_bytes))
        return fail(CIRCATT_ERR_INVALID, "destination blocks overlap");
    const int64_t dst_end = (nouter - 1) * dst_stride_outer + (ninner - 1) * dst_stride_inner + block_bytes;
    const int64_t src_end = (nouter - 1) * src_stride_outer + (ninner - 1) * src_stride_inner + block_bytes;
    const char *d0 = static_cast<const char *>(dst), *s0 = static_cast<const char *>(src);
    if (d0 < s0 + src_end && s0 < d0 + dst_end)
        return fail(CIRCATT_ERR_INVALID, "source and destination ranges overlap");
    return hip_result(launch_copy_blocks(dst, src, block_bytes, ninner, dst_stride_inner,
                                         src_stride_inner, nouter, dst_stride_outer,
                                         src_stride_outer, as_stream(stream)),
                      "circatt_copy_blocks");
}

int circatt_sum_middle(const float *src, float *dst, int64_t inner, int64_t nsum, int64_t outer,
                       void *stream) {
    if (inner < 0 || nsum < 0 || outer < 0) return fail(CIRCATT_ERR_INVALID, "negative size");
    if (inner == 0 || outer == 0) return ok();
    if (nsum == 0) return circatt_fill(dst, inner * outer, 0.f, stream);
    CIRCATT_NONNULL(src);
    CIRCATT_NONNULL(dst);
    if (dst < src + inner * nsum * outer && src < dst + inner * outer)
        return fail(CIRCATT_ERR_INVALID, "src and dst overlap");
    return hip_result(launch_sum_middle(src, dst, inner, nsum, outer, as_stream(stream)),
                      "circatt_sum_middle");
}

int circatt_count_unequal(int kind, int64_t n, const void *a, const void *b, int64_t *count,
                          void *stream) {
    if (kind != 0 && kind != 1) return fail(CIRCATT_ERR_INVALID, "kind=%d must be 0 or 1", kind);
    if (n < 0) return fail(CIRCATT_ERR_INVALID, "n=%lld must be >= 0", (long long)n);
    CIRCATT_NONNULL(count);
    if (n > 0) {
        CIRCATT_NONNULL(a);
        CIRCATT_NONNULL(b);
    }
    return hip_result(launch_count_unequal(kind == 1, n, static_cast<const uint32_t *>(a),
                                           static_cast<const uint32_t *>(b), count,
                                           as_stream(stream)),
                      "circatt_count_unequal");
}

int circatt_memcpy(void *dst, const void *src, int64_t bytes, int kind) {
    static const hipMemcpyKind kinds[] = {hipMemcpyHostToDevice, hipMemcpyDeviceToHost,
                                          hipMemcpyDeviceToDevice};
    if (kind < 0 || kind > 2) return fail(CIRCATT_ERR_INVALID, "memcpy kind %d", kind);
    if (bytes < 0) return fail(CIRCATT_ERR_INVALID, "negative size");
    if (bytes == 0) return ok();
    CIRCATT_NONNULL(dst);
    CIRCATT_NONNULL(src);
    return hip_result(hipMemcpy(dst, src, (size_t)bytes, kinds[kind]), "circatt_memcpy");
}

int circatt_stream_synchronize(void *stream) {
    return hip_result(hipStreamSynchronize(as_stream(stream)), "circatt_stream_synchronize");
}

}  // extern "C"
