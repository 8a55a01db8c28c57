/*
 * CPU restatement of CirculantAttention.jl's circulant attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP library is
 * compared against (tests/, __graft_entry__.smoke) and the CPU baseline that
 * bench.py times beside the GPU.  Nothing in the product links or calls it.
 *
 * The same source is compiled twice (see oracle/Makefile):
 *   OC_REAL=double -> liboracle_f64.so : parity oracle (float64 accumulation)
 *   OC_REAL=float  -> liboracle_f32.so : CPU baseline, the reference's
 *                                         unfused algorithm in Float32
 *
 * Layout follows Julia's column-major arrays.  A signal x of Julia size
 * (N1[,N2], C, nb) holds element (pixel r, channel c, batch b) at
 * r + P*(c + C*b), P = N1*N2; ComplexF32 data is interleaved (re, im), so the
 * element is two consecutive reals (ncomp = 2).  Pixel r = i1 + N1*i2
 * (0-based here, 1-based in Julia).
 *
 * Each function cites the reference lines it restates (paths relative to the
 * reference repository root).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifndef OC_REAL
#define OC_REAL double
#endif
typedef OC_REAL real_t;

static inline int64_t oc_mod(int64_t a, int64_t n) {
    int64_t r = a % n;
    return r < 0 ? r + n : r;
}
static inline int64_t oc_cld(int64_t a, int64_t b) { /* ceil(a/b), a>=0, b>0 */
    return (a + b - 1) / b;
}

/* src/circulant.jl:4 circshift_index(m, s, M) = mod(m - 1 - s, M) + 1 */
static inline int64_t circshift_index(int64_t m, int64_t s, int64_t M) {
    return oc_mod(m - 1 - s, M) + 1;
}

/* src/circulant.jl:6-19, literal (1-based n, returns 1-based (i, j)). */
void oc_cartesian_circulant_1d(int64_t n, int64_t N, int64_t M, int64_t *i, int64_t *j) {
    int64_t p = (M - 1) / 2;
    int64_t jj = oc_cld(n, M);
    int64_t m = oc_mod(n - 1, M) + 1;
    if (jj <= p)
        m = circshift_index(m, jj - p - 1, M);
    else if (jj > N - p)
        m = circshift_index(m, p - N + jj, M);
    *i = oc_mod((m - 1) + (jj - 1) - p, N) + 1;
    *j = jj;
}

/* src/circulant.jl:21-43, literal (1-based n, returns 1-based (i, j)). */
void oc_cartesian_circulant_2d(int64_t n, int64_t N1, int64_t N2, int64_t M, int64_t *i,
                               int64_t *j) {
    int64_t p = (M - 1) / 2;
    int64_t jg = oc_cld(n, M * M);                          /* global col num */
    int64_t jj = oc_cld(jg, N1);                            /* block col num */
    int64_t j0 = oc_mod(jg - 1, N1) + 1;                    /* intra block col num */
    int64_t nn = oc_mod(oc_cld(n, M) - 1, M) + 1 + M * (jj - 1); /* block num */
    int64_t mm = oc_mod(nn - 1, M) + 1;                     /* block filter coeff num */
    int64_t m0 = n - M * (mm - 1) - (jg - 1) * M * M;       /* intra block coeff num */
    if (jj <= p)
        mm = circshift_index(mm, jj - p - 1, M);
    else if (jj > N2 - p)
        mm = circshift_index(mm, p - N2 + jj, M);
    if (j0 <= p)
        m0 = circshift_index(m0, j0 - p - 1, M);
    else if (j0 > N1 - p)
        m0 = circshift_index(m0, p - N1 + j0, M);
    int64_t ii = oc_mod((mm - 1) + (jj - 1) - p, N2) + 1;
    *i = N1 * (ii - 1) + oc_mod((m0 - 1) + (j0 - 1) - p, N1) + 1;
    *j = jg;
}

/*
 * Pattern of one Circulant, replicated over nb batches:
 * src/circulant.jl:64-106 (cucirculant: rowptr = 1 + K*r, colval from
 * cartesian_circulant) and src/array.jl:9 (repeat over the batch dims).
 * rowptr: (P+1, nb) Int32 1-based, colval: (P*K, nb) Int32 1-based.
 * Returns 0, or -1 for an even window / unsupported nsp.
 */
int oc_pattern(int nsp, int64_t n1, int64_t n2, int64_t ws, int64_t nb, int32_t *rowptr,
               int32_t *colval) {
    if (ws % 2 != 1 || ws < 1) return -1; /* circulant.jl:65,87 */
    if (nsp != 1 && nsp != 2) return -1;
    int64_t P = (nsp == 1) ? n1 : n1 * n2;
    int64_t K = (nsp == 1) ? ws : ws * ws;
    for (int64_t r = 0; r <= P; ++r) rowptr[r] = (int32_t)(1 + K * r);
    for (int64_t n = 1; n <= P * K; ++n) {
        int64_t i, j;
        if (nsp == 1)
            oc_cartesian_circulant_1d(n, n1, ws, &i, &j);
        else
            oc_cartesian_circulant_2d(n, n1, n2, ws, &i, &j);
        colval[n - 1] = (int32_t)i;
    }
    for (int64_t b = 1; b < nb; ++b) {
        memcpy(rowptr + b * (P + 1), rowptr, sizeof(int32_t) * (size_t)(P + 1));
        memcpy(colval + b * P * K, colval, sizeof(int32_t) * (size_t)(P * K));
    }
    return 0;
}

/*
 * Similarity on the pattern: src/similarity.jl:55-103.
 * Row r of the CSR is the pixel of the FIRST argument x (query), colval is
 * the pixel of the second argument y (key).
 *   kind 0 (Dot):      S = sum_m Re(x[r,m] * conj(y[c,m]))     (:96-100)
 *   kind 1 (Distance): S = -(sum_m |x[r,m] - y[c,m]|^2) / 2     (:71-75)
 * `scale` multiplies S; src/attention.jl:20-21 feeds q/sqrt(tau), k/sqrt(tau)
 * with tau = sqrt(C), which is S(q,k) * C^(-1/2) for both kinds.
 * colval is one batch's pattern (P*K, 1-based); nz is (P*K, nb).
 */
void oc_similarity(int kind, int ncomp, int64_t P, int64_t C, int64_t nb, int64_t K,
                   const int32_t *colval, real_t scale, const real_t *x, const real_t *y,
                   real_t *nz) {
    const int64_t PK = P * K;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < nb; ++b) {
        for (int64_t n = 0; n < PK; ++n) {
            int64_t r = n / K;
            int64_t col = (int64_t)colval[n] - 1;
            real_t s = 0;
            for (int64_t c = 0; c < C; ++c) {
                const real_t *xr = x + ncomp * (r + P * (c + C * b));
                const real_t *yc = y + ncomp * (col + P * (c + C * b));
                for (int e = 0; e < ncomp; ++e) {
                    if (kind == 0)
                        s += xr[e] * yc[e];
                    else {
                        real_t d = xr[e] - yc[e];
                        s -= d * d;
                    }
                }
            }
            if (kind == 1) s = s / 2;
            nz[n + PK * b] = s * scale;
        }
    }
}

/* Row softmax over the K slots of each row: src/similarity.jl:105-110
 * (NNlib.softmax! with dims=1 on nzVal viewed as (K, rows)), max-subtracted. */
void oc_softmax(int64_t K, int64_t rows, const real_t *in, real_t *out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const real_t *a = in + r * K;
        real_t *o = out + r * K;
        real_t m = -INFINITY;
        for (int64_t t = 0; t < K; ++t) m = a[t] > m ? a[t] : m;
        real_t s = 0;
        for (int64_t t = 0; t < K; ++t) {
            o[t] = exp(a[t] - m);
            s += o[t];
        }
        for (int64_t t = 0; t < K; ++t) o[t] /= s;
    }
}

/* Softmax pullback: src/rrules.jl:42-56 (NNlib.∇softmax_data):
 * dS = A .* (dA .- sum(A .* dA; dims=1)). */
void oc_softmax_bwd(int64_t K, int64_t rows, const real_t *A, const real_t *dA, real_t *dS) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const real_t *a = A + r * K, *da = dA + r * K;
        real_t s = 0;
        for (int64_t t = 0; t < K; ++t) s += a[t] * da[t];
        for (int64_t t = 0; t < K; ++t) dS[r * K + t] = a[t] * (da[t] - s);
    }
}

/*
 * Sparse apply, the CSR x dense product that CUSPARSE.bmm! computes in
 * src/batchedmul.jl:82-110 with alpha=1, beta=0:
 *   trans 0 ('N'): y[r,:,b] = sum_t nz[r,t,b] * x[col(r,t),:,b]   (A ⊗ x,
 *                  src/attention.jl:53-70)
 *   trans 1 ('T'): y[c,:,b] = sum_{col(r,t)=c} nz[r,t,b] * x[r,:,b]
 *                  (src/attention.jl:72-80, batchedmul.jl:102-110)
 * nz is real; x, y may be complex (ncomp = 2), the real-A x complex-x
 * promotion of src/batchedmul.jl:72-75.  x, y: (P, C, nb).
 */
void oc_apply(int trans, int ncomp, int64_t P, int64_t C, int64_t nb, int64_t K,
              const int32_t *colval, const real_t *nz, const real_t *x, real_t *y) {
    const int64_t PK = P * K;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < nb; ++b) {
        for (int64_t c = 0; c < C; ++c) {
            const real_t *xb = x + ncomp * P * (c + C * b);
            real_t *yb = y + ncomp * P * (c + C * b);
            for (int64_t i = 0; i < ncomp * P; ++i) yb[i] = 0;
            for (int64_t n = 0; n < PK; ++n) {
                int64_t r = n / K;
                int64_t col = (int64_t)colval[n] - 1;
                real_t a = nz[n + PK * b];
                for (int e = 0; e < ncomp; ++e) {
                    if (trans == 0)
                        yb[ncomp * r + e] += a * xb[ncomp * col + e];
                    else
                        yb[ncomp * col + e] += a * xb[ncomp * r + e];
                }
            }
        }
    }
}

/* sum(A; dims=2) -> (P, 1, nb): src/array.jl:126-130 (reduce nzVal over K). */
void oc_rowsum(int64_t P, int64_t K, int64_t nb, const real_t *nz, real_t *out) {
    for (int64_t b = 0; b < nb; ++b)
        for (int64_t r = 0; r < P; ++r) {
            real_t s = 0;
            for (int64_t t = 0; t < K; ++t) s += nz[(r * K + t) + P * K * b];
            out[r + P * b] = s;
        }
}

/* sum(A; dims=1) -> (1, P, nb): src/array.jl:119-124 (Aᵀ ⊠ ones). */
void oc_colsum(int64_t P, int64_t K, int64_t nb, const int32_t *colval, const real_t *nz,
               real_t *out) {
    for (int64_t b = 0; b < nb; ++b) {
        for (int64_t c = 0; c < P; ++c) out[c + P * b] = 0;
        for (int64_t n = 0; n < P * K; ++n)
            out[(int64_t)colval[n] - 1 + P * b] += nz[n + P * K * b];
    }
}
