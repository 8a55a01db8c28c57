/*
 * Address- and undefined-behaviour-sanitized run of the CPU restatement.
 *
 * TEST INFRASTRUCTURE ONLY.  Built by `make -C oracle sanitize` together with
 * circatt_oracle.c under -fsanitize=address,undefined (no recovery), and run
 * by tests/test_oracle_sanitized.py.  It calls every function of the
 * restatement on small shapes, windows wider than the signal included, and
 * checks invariants that hold for any input:
 *   pattern   rowptr[r] = 1 + K r, every column a pixel of the signal, and the
 *             K columns of a row are distinct when the window fits the signal
 *   similarity  Distance(x, x) is 0 where the column is the row's own pixel;
 *             Dot(x, y) at (r, c) equals Dot(y, x) at (c, r)
 *   softmax   rows sum to 1; its pullback's rows sum to 0
 *   apply     A ⊗ 1 = rowsum(A), Aᵀ ⊗ 1 = colsum(A)
 * Exit status 0 when every check passes; the sanitizers abort on a fault.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

typedef double real_t;

int oc_pattern(int nsp, int64_t n1, int64_t n2, int64_t ws, int64_t nb, int32_t *rowptr,
               int32_t *colval);
void oc_similarity(int kind, int ncomp, int64_t P, int64_t C, int64_t nb, int64_t K,
                   const int32_t *colval, real_t scale, const real_t *x, const real_t *y,
                   real_t *nz);
void oc_softmax(int64_t K, int64_t rows, const real_t *in, real_t *out);
void oc_softmax_bwd(int64_t K, int64_t rows, const real_t *A, const real_t *dA, real_t *dS);
void oc_apply(int trans, int ncomp, int64_t P, int64_t C, int64_t nb, int64_t K,
              const int32_t *colval, const real_t *nz, const real_t *x, real_t *y);
void oc_rowsum(int64_t P, int64_t K, int64_t nb, const real_t *nz, real_t *out);
void oc_colsum(int64_t P, int64_t K, int64_t nb, const int32_t *colval, const real_t *nz,
               real_t *out);

static int failures = 0;

static void check(int ok, const char *what, int nsp, long n1, long n2, long ws) {
    if (!ok) {
        fprintf(stderr, "FAIL %s nsp=%d n1=%ld n2=%ld ws=%ld\n", what, nsp, n1, n2, ws);
        ++failures;
    }
}

static uint64_t rng = 88172645463325252ull;
static real_t uniform(void) { /* xorshift64, in [-1, 1) */
    rng ^= rng << 13;
    rng ^= rng >> 7;
    rng ^= rng << 17;
    return (real_t)(rng >> 11) / (real_t)(1ull << 52) - 1.0;
}

static void *alloc(size_t n) {
    void *p = malloc(n ? n : 1);
    if (!p) {
        fprintf(stderr, "out of memory\n");
        exit(2);
    }
    return p;
}

static void run_case(int nsp, int64_t n1, int64_t n2, int64_t ws, int ncomp, int64_t C,
                     int64_t nb) {
    const int64_t P = nsp == 1 ? n1 : n1 * n2;
    const int64_t K = nsp == 1 ? ws : ws * ws;
    const int64_t PK = P * K, X = ncomp * P * C * nb;
    int32_t *rowptr = alloc(sizeof(int32_t) * (size_t)((P + 1) * nb));
    int32_t *colval = alloc(sizeof(int32_t) * (size_t)(PK * nb));
    real_t *x = alloc(sizeof(real_t) * (size_t)X), *y = alloc(sizeof(real_t) * (size_t)X);
    real_t *ones = alloc(sizeof(real_t) * (size_t)(P * nb));
    real_t *S = alloc(sizeof(real_t) * (size_t)(PK * nb)), *T = alloc(sizeof(real_t) * (size_t)(PK * nb));
    real_t *A = alloc(sizeof(real_t) * (size_t)(PK * nb)), *dS = alloc(sizeof(real_t) * (size_t)(PK * nb));
    real_t *u = alloc(sizeof(real_t) * (size_t)(P * nb)), *v = alloc(sizeof(real_t) * (size_t)(P * nb));
    for (int64_t i = 0; i < X; ++i) {
        x[i] = uniform();
        y[i] = uniform();
    }
    for (int64_t i = 0; i < P * nb; ++i) ones[i] = 1.0;

    check(oc_pattern(nsp, n1, n2, ws, nb, rowptr, colval) == 0, "pattern status", nsp, n1, n2, ws);
    const int fits = nsp == 1 ? ws <= n1 : ws <= n1 && ws <= n2;
    for (int64_t b = 0; b < nb; ++b)
        for (int64_t r = 0; r < P; ++r) {
            check(rowptr[b * (P + 1) + r] == 1 + K * r, "rowptr", nsp, n1, n2, ws);
            for (int64_t t = 0; t < K; ++t) {
                const int32_t c = colval[b * PK + r * K + t];
                check(c >= 1 && c <= P, "column in range", nsp, n1, n2, ws);
                if (fits)
                    for (int64_t s = 0; s < t; ++s)
                        check(colval[b * PK + r * K + s] != c, "distinct columns", nsp, n1, n2, ws);
            }
        }

    /* Distance(x, x): zero on the row's own pixel */
    oc_similarity(1, ncomp, P, C, nb, K, colval, 1.0, x, x, S);
    for (int64_t b = 0; b < nb; ++b)
        for (int64_t n = 0; n < PK; ++n)
            if (colval[n] - 1 == n / K)
                check(S[b * PK + n] == 0.0, "distance to itself", nsp, n1, n2, ws);
    /* Dot(x, y) at (r, c) against Dot(y, x) at (c, r), where the window fits
     * (then (c, r) is an entry of the pattern, the window being symmetric) */
    oc_similarity(0, ncomp, P, C, nb, K, colval, 0.5, x, y, S);
    oc_similarity(0, ncomp, P, C, nb, K, colval, 0.5, y, x, T);
    if (fits)
        for (int64_t b = 0; b < nb; ++b)
            for (int64_t n = 0; n < PK; ++n) {
                const int64_t r = n / K, c = colval[n] - 1;
                int64_t m = -1;
                for (int64_t t = 0; t < K; ++t)
                    if (colval[c * K + t] - 1 == r) m = c * K + t;
                check(m >= 0, "transposed entry", nsp, n1, n2, ws);
                if (m >= 0)
                    check(fabs(S[b * PK + n] - T[b * PK + m]) <= 1e-12 * (1 + fabs(S[b * PK + n])),
                          "dot symmetry", nsp, n1, n2, ws);
            }

    oc_softmax(K, P * nb, S, A);
    for (int64_t r = 0; r < P * nb; ++r) {
        real_t s = 0;
        for (int64_t t = 0; t < K; ++t) s += A[r * K + t];
        check(fabs(s - 1) <= 1e-12, "softmax row sum", nsp, n1, n2, ws);
    }
    oc_softmax_bwd(K, P * nb, A, T, dS);
    for (int64_t r = 0; r < P * nb; ++r) {
        real_t s = 0, m = 0;
        for (int64_t t = 0; t < K; ++t) {
            s += dS[r * K + t];
            m += fabs(T[r * K + t]);
        }
        check(fabs(s) <= 1e-12 * (1 + m), "softmax pullback row sum", nsp, n1, n2, ws);
    }

    /* products with x = 1 (one real channel) against the sums */
    oc_apply(0, 1, P, 1, nb, K, colval, A, ones, u);
    oc_rowsum(P, K, nb, A, v);
    for (int64_t i = 0; i < P * nb; ++i) check(fabs(u[i] - v[i]) <= 1e-12, "A x 1 = rowsum", nsp, n1, n2, ws);
    oc_apply(1, 1, P, 1, nb, K, colval, A, ones, u);
    oc_colsum(P, K, nb, colval, A, v);
    for (int64_t i = 0; i < P * nb; ++i)
        check(fabs(u[i] - v[i]) <= 1e-12 * (1 + fabs(v[i])), "At x 1 = colsum", nsp, n1, n2, ws);
    /* the full-width products (complex or several channels), for the sanitizers */
    oc_apply(0, ncomp, P, C, nb, K, colval, A, x, y);
    oc_apply(1, ncomp, P, C, nb, K, colval, A, y, x);

    free(rowptr);
    free(colval);
    free(x);
    free(y);
    free(ones);
    free(S);
    free(T);
    free(A);
    free(dS);
    free(u);
    free(v);
}

int main(void) {
    /* nsp, n1, n2, ws, ncomp, C, nb */
    run_case(1, 1, 1, 1, 1, 1, 1);
    run_case(1, 3, 1, 5, 2, 2, 2);   /* window wider than the signal */
    run_case(1, 16, 1, 7, 1, 3, 2);
    run_case(1, 40, 1, 15, 2, 2, 1);
    run_case(2, 4, 3, 5, 1, 2, 2);   /* window wider than both dimensions */
    run_case(2, 5, 7, 3, 2, 3, 1);
    run_case(2, 9, 6, 5, 1, 4, 2);
    run_case(2, 8, 8, 7, 2, 1, 1);
    check(oc_pattern(1, 4, 1, 4, 1, NULL, NULL) == -1, "even window rejected", 1, 4, 1, 4);
    check(oc_pattern(3, 4, 4, 3, 1, NULL, NULL) == -1, "three dimensions rejected", 3, 4, 4, 3);
    if (failures) {
        fprintf(stderr, "%d checks failed\n", failures);
        return 1;
    }
    printf("sanitized oracle run: all checks passed\n");
    return 0;
}
