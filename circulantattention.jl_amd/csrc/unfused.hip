// Unfused kernels: pattern, softmax (+ pullback), sparse apply (N and T),
// similarity pullback, row/column sums, nzVal algebra.
//
// Every kernel walks window offsets rather than colVal, using the slot <->
// offset bijection of circatt_common.h, so the transposed products gather
// without atomics.  These kernels are memory/latency bound; the fused
// MFMA kernels (fused.hip) carry the north-star path.
#include <algorithm>

#include "circatt_common.h"
#include "circatt_kernels.h"

namespace circatt {

// ---------------------------------------------------------------------------
// Pattern: src/circulant.jl:46-106 + repeat over batches (src/array.jl:9)
// ---------------------------------------------------------------------------
__global__ void pattern_kernel(Geom g, int64_t nb, int32_t *__restrict__ rowptr,
                               int32_t *__restrict__ colval) {
    const int64_t PK = g.P * g.K;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t n = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; n < PK; n += stride) {
        const int64_t r = n / g.K;
        const int t = (int)(n - r * g.K);
        int d1, d2;
        slot_offsets(g, r, t, d1, d2);
        const int32_t col = (int32_t)(offset_pixel(g, r, d1, d2) + 1);
        for (int64_t b = 0; b < nb; ++b) colval[n + b * PK] = col;
    }
    for (int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; r <= g.P; r += stride) {
        const int32_t v = (int32_t)(1 + (int64_t)g.K * r);
        for (int64_t b = 0; b < nb; ++b) rowptr[r + b * (g.P + 1)] = v;
    }
}

// Same pattern with 32-bit index arithmetic (P * K < 2^31): 16 lanes per CSR
// row, the row's border shifts computed once per lane, each slot's window
// offsets from t = mm * ws + m0 (quotient by a float reciprocal, exact for
// t < 2^22), all batch copies written from the same column.
typedef int i4u __attribute__((ext_vector_type(4), aligned(4)));  // 4-byte aligned
// v folded into [0, n) for -n <= v < 2n
__device__ __forceinline__ int fold_n(int v, int n) { return v < 0 ? v + n : (v >= n ? v - n : v); }

__global__ __launch_bounds__(256) void pattern32_kernel(int nsp, int n1, int n2, int ws, int nb,
                                                        int32_t *__restrict__ rowptr,
                                                        int32_t *__restrict__ colval) {
    const int p = (ws - 1) / 2;
    const int K = nsp == 1 ? ws : ws * ws;
    const int P = n1 * n2;
    const int PK = P * K;
    const float inv_ws = 1.f / (float)ws;
    const int gl = threadIdx.x & 15;
    // every offset is within one period of the image (p < n1, n2): wrapped
    // indices by one compare each instead of a remainder
    const bool near = p < n1 && (nsp == 1 || p < n2);
    for (int r = blockIdx.x * 16 + (threadIdx.x >> 4); r < P; r += gridDim.x * 16) {
        const int i1 = r % n1, i2 = r / n1;
        const int s1 = slot_shift(i1 + 1, n1, p);
        const int s2 = nsp == 2 ? slot_shift(i2 + 1, n2, p) : 0;
        // 16 lanes per row, 4 consecutive slots per lane and store
        for (int t0 = 4 * gl; t0 < K; t0 += 64) {
            int v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = min(t0 + e, K - 1);
                const int mm = nsp == 2 ? (int)(((float)t + 0.5f) * inv_ws) : 0;
                const int m0 = t - mm * ws;
                int col;
                if (near) {
                    col = fold_n(i1 + fold_n(m0 - s1, ws) - p, n1);
                    if (nsp == 2) col += n1 * fold_n(i2 + fold_n(mm - s2, ws) - p, n2);
                } else {
                    col = pmod(i1 + slot_to_offset(m0, s1, ws, p), n1);
                    if (nsp == 2) col += n1 * pmod(i2 + slot_to_offset(mm, s2, ws, p), n2);
                }
                v[e] = col + 1;
            }
            const int n = r * K + t0;
            for (int b = 0; b < nb; ++b) {
                int32_t *dst = colval + n + (int64_t)b * PK;
                if (t0 + 4 <= K) {
                    *(i4u *)dst = i4u{v[0], v[1], v[2], v[3]};
                } else {
#pragma unroll
                    for (int e = 0; e < 3; ++e)
                        if (t0 + e < K) dst[e] = v[e];
                }
            }
        }
    }
    for (int r = blockIdx.x * blockDim.x + threadIdx.x; r <= P; r += gridDim.x * blockDim.x)
        for (int b = 0; b < nb; ++b) rowptr[r + (int64_t)b * (P + 1)] = 1 + K * r;
}

// ---------------------------------------------------------------------------
// Row softmax and its pullback: one wavefront per row of K slots.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__global__ __launch_bounds__(256) void softmax_kernel(int K, int64_t rows,
                                                      const float *__restrict__ in,
                                                      float *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *a = in + row * K;
    float *o = out + row * K;
    float m = -INFINITY;
    for (int t = lane; t < K; t += 64) m = fmaxf(m, a[t]);
    m = wave_max(m);
    float s = 0.f;
    for (int t = lane; t < K; t += 64) s += __expf(a[t] - m);
    s = wave_sum(s);
    const float inv = 1.f / s;
    for (int t = lane; t < K; t += 64) o[t] = __expf(a[t] - m) * inv;
}

__global__ __launch_bounds__(256) void softmax_bwd_kernel(int K, int64_t rows,
                                                          const float *__restrict__ A,
                                                          const float *dA, float *dS) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *a = A + row * K;
    const float *da = dA + row * K;
    float s = 0.f;
    for (int t = lane; t < K; t += 64) s += a[t] * da[t];
    s = wave_sum(s);
    for (int t = lane; t < K; t += 64) dS[row * K + t] = a[t] * (da[t] - s);
}

// Rows held in registers: a group of L lanes owns one row of K <= L * V
// slots, reads it once, reduces with cross-lane shuffles inside the group and
// writes it once.
template <int L>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int o = L / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
template <int L>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = L / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Lane gl of a row's group holds slots 4 gl + 4 L v + e (v < V / 4, e < 4):
// one 16-byte access per v (rows start at any 4-byte boundary: K is odd for
// the circulant patterns), single floats only where a vector crosses the
// row's end.  V = 1 (K <= 16) uses single floats.
typedef float f4u __attribute__((ext_vector_type(4), aligned(4)));

template <int L, int V>
__device__ __forceinline__ void load_row(const float *a, int K, int gl, bool live, float fill,
                                         float (&v)[V]) {
    if constexpr (V < 4) {
#pragma unroll
        for (int u = 0; u < V; ++u) {
            const int t = gl + L * u;
            v[u] = live && t < K ? a[t] : fill;
        }
    } else {
#pragma unroll
        for (int u = 0; u < V / 4; ++u) {
            const int t0 = 4 * gl + 4 * L * u;
            if (live && t0 + 3 < K) {
                const f4u x = *(const f4u *)(a + t0);
                v[4 * u] = x[0];
                v[4 * u + 1] = x[1];
                v[4 * u + 2] = x[2];
                v[4 * u + 3] = x[3];
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) v[4 * u + q] = live && t0 + q < K ? a[t0 + q] : fill;
            }
        }
    }
}
template <int L, int V>
__device__ __forceinline__ int slot_of(int gl, int u) {
    return V < 4 ? gl + L * u : 4 * gl + 4 * L * (u / 4) + (u & 3);
}
template <int L, int V>
__device__ __forceinline__ void store_row(float *o, int K, int gl, const float (&v)[V]) {
    if constexpr (V < 4) {
#pragma unroll
        for (int u = 0; u < V; ++u) {
            const int t = gl + L * u;
            if (t < K) o[t] = v[u];
        }
    } else {
#pragma unroll
        for (int u = 0; u < V / 4; ++u) {
            const int t0 = 4 * gl + 4 * L * u;
            if (t0 + 3 < K) {
                *(f4u *)(o + t0) = f4u{v[4 * u], v[4 * u + 1], v[4 * u + 2], v[4 * u + 3]};
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (t0 + q < K) o[t0 + q] = v[4 * u + q];
            }
        }
    }
}

template <int L, int V>
__global__ __launch_bounds__(256) void softmax_rows_kernel(int K, int64_t rows,
                                                           const float *__restrict__ in,
                                                           float *__restrict__ out) {
    const int gl = threadIdx.x % L;
    const int64_t row = (int64_t)blockIdx.x * (256 / L) + threadIdx.x / L;
    const bool live = row < rows;
    float v[V];
    load_row<L, V>(in + (live ? row : 0) * K, K, gl, live, -INFINITY, v);
    float m = -INFINITY;
#pragma unroll
    for (int u = 0; u < V; ++u) m = fmaxf(m, v[u]);
    m = group_max<L>(m);
    float s = 0.f;
#pragma unroll
    for (int u = 0; u < V; ++u) {
        v[u] = live && slot_of<L, V>(gl, u) < K ? __expf(v[u] - m) : 0.f;
        s += v[u];
    }
    s = group_sum<L>(s);
    const float inv = 1.f / s;
    if (!live) return;
#pragma unroll
    for (int u = 0; u < V; ++u) v[u] *= inv;
    store_row<L, V>(out + row * K, K, gl, v);
}

template <int L, int V>
__global__ __launch_bounds__(256) void softmax_bwd_rows_kernel(int K, int64_t rows,
                                                               const float *__restrict__ A,
                                                               const float *dA, float *dS) {
    const int gl = threadIdx.x % L;
    const int64_t row = (int64_t)blockIdx.x * (256 / L) + threadIdx.x / L;
    const bool live = row < rows;
    const int64_t base = (live ? row : 0) * K;
    float av[V], dv[V];
    load_row<L, V>(A + base, K, gl, live, 0.f, av);
    load_row<L, V>(dA + base, K, gl, live, 0.f, dv);
    float s = 0.f;
#pragma unroll
    for (int u = 0; u < V; ++u) s += av[u] * dv[u];
    s = group_sum<L>(s);  // every read of the row precedes this, so dS may alias dA
    if (!live) return;
#pragma unroll
    for (int u = 0; u < V; ++u) av[u] *= dv[u] - s;
    store_row<L, V>(dS + base, K, gl, av);
}

// sum over a row's K contiguous slots, 16 lanes per row
__global__ __launch_bounds__(256) void rowsum_kernel(int K, int64_t rows,
                                                     const float *__restrict__ nz,
                                                     float *__restrict__ out) {
    const int gl = threadIdx.x & 15;
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const bool live = row < rows;
    const float *a = nz + (live ? row : 0) * K;
    float s = 0.f;
    if (live) {
#pragma unroll 4
        for (int t = gl; t < K; t += 16) s += a[t];
    }
    s = group_sum<16>(s);
    if (live && gl == 0) out[row] = s;
}

// ---------------------------------------------------------------------------
// Sparse apply.  One thread per (row, batch, chunk of CH channels).
//   TRANS = false: y[r] = sum_t A[r,t] x[col(r,t)]          (A ⊗ x)
//   TRANS = true : y[c] = sum_d A[r=c-d, slot(r,d)] x[r]     (Aᵀ ⊗ x)
//   CORR        : y -= (sum of the A entries used) .* z     (Distance rrule)
// Result is multiplied by `scale`.
// ---------------------------------------------------------------------------
template <int NCOMP, bool TRANS, bool CORR, int CH>
__global__ __launch_bounds__(256) void apply_kernel(Geom g, int C, int64_t nb, float scale,
                                                    const float *__restrict__ nz,
                                                    const float *__restrict__ x,
                                                    const float *__restrict__ z,
                                                    float *__restrict__ y) {
    const int nchunk = (C + CH - 1) / CH;
    const int64_t total = g.P * nb * nchunk;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (tid >= total) return;
    const int64_t r = tid % g.P;
    const int64_t rest = tid / g.P;
    const int64_t b = rest % nb;
    const int c0 = (int)(rest / nb) * CH;
    const int cn = min(CH, C - c0);
    const float *nzb = nz + b * g.P * g.K;
    const float *xb = x + (int64_t)NCOMP * g.P * ((int64_t)C * b + c0);
    float acc[CH * NCOMP];
#pragma unroll
    for (int i = 0; i < CH * NCOMP; ++i) acc[i] = 0.f;
    float asum = 0.f;
    const int p = g.p;
    const int p2 = g.nsp == 1 ? 0 : p;
    for (int d2 = -p2; d2 <= p2; ++d2) {
        for (int d1 = -p; d1 <= p; ++d1) {
            int64_t src;
            float a;
            if (!TRANS) {
                src = offset_pixel(g, r, d1, d2);
                a = nzb[r * g.K + offset_slot(g, r, d1, d2)];
            } else {
                src = offset_pixel(g, r, -d1, -d2);
                a = nzb[src * g.K + offset_slot(g, src, d1, d2)];
            }
            asum += a;
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                if (c < cn) {
#pragma unroll
                    for (int e = 0; e < NCOMP; ++e)
                        acc[c * NCOMP + e] += a * xb[NCOMP * (src + g.P * c) + e];
                }
            }
        }
    }
    const float *zb = z ? z + (int64_t)NCOMP * g.P * ((int64_t)C * b + c0) : nullptr;
    float *yb = y + (int64_t)NCOMP * g.P * ((int64_t)C * b + c0);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        if (c < cn) {
#pragma unroll
            for (int e = 0; e < NCOMP; ++e) {
                float v = acc[c * NCOMP + e];
                if (CORR) v -= asum * zb[NCOMP * (r + g.P * c) + e];
                yb[NCOMP * (r + g.P * c) + e] = v * scale;
            }
        }
    }
}

// Similarity for shapes outside the fused kernels' range (more than 64 real
// components per pixel): one thread per (nz, batch), sequential channel sum
// in the order of src/similarity.jl:96-100.
template <int NCOMP, bool DIST>
__global__ __launch_bounds__(256) void similarity_kernel(Geom g, int C, int64_t nb, float scale,
                                                         const float *__restrict__ x,
                                                         const float *__restrict__ y,
                                                         float *__restrict__ nz) {
    const int64_t PK = g.P * g.K;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (tid >= PK * nb) return;
    const int64_t n = tid % PK, b = tid / PK;
    const int64_t r = n / g.K;
    int d1, d2;
    slot_offsets(g, r, (int)(n - r * g.K), d1, d2);
    const int64_t col = offset_pixel(g, r, d1, d2);
    const float *xb = x + (int64_t)NCOMP * g.P * C * b;
    const float *yb = y + (int64_t)NCOMP * g.P * C * b;
    float s = 0.f;
    for (int c = 0; c < C; ++c) {
#pragma unroll
        for (int e = 0; e < NCOMP; ++e) {
            const float xv = xb[NCOMP * (r + g.P * c) + e];
            const float yv = yb[NCOMP * (col + g.P * c) + e];
            if (DIST) {
                const float d = xv - yv;
                s -= d * d;
            } else {
                s += xv * yv;
            }
        }
    }
    if (DIST) s *= 0.5f;
    nz[tid] = s * scale;
}

// sum over a row's slots (dims=2) or a column's entries (dims=1)
template <bool COL>
__global__ void sum_kernel(Geom g, int64_t nb, const float *__restrict__ nz,
                           float *__restrict__ out) {
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (tid >= g.P * nb) return;
    const int64_t r = tid % g.P, b = tid / g.P;
    const float *nzb = nz + b * g.P * g.K;
    float s = 0.f;
    if (!COL) {
        for (int t = 0; t < g.K; ++t) s += nzb[r * g.K + t];
    } else {
        const int p = g.p, p2 = g.nsp == 1 ? 0 : g.p;
        for (int d2 = -p2; d2 <= p2; ++d2)
            for (int d1 = -p; d1 <= p; ++d1) {
                int64_t src = offset_pixel(g, r, -d1, -d2);
                s += nzb[src * g.K + offset_slot(g, src, d1, d2)];
            }
    }
    out[tid] = s;
}

__global__ void axpby_kernel(int64_t nnz, int64_t nb, const float *__restrict__ alpha,
                             float alpha0, const float *X, const float *__restrict__ beta,
                             float beta0, const float *Y, float *Z) {
    const int64_t total = nnz * nb;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t b = i / nnz;
        const float a = alpha ? alpha[b] : alpha0;
        float v = a * X[i];
        if (Y) v += (beta ? beta[b] : beta0) * Y[i];
        Z[i] = v;
    }
}

// Z[:, b] = alpha_b X[:, b] + beta_b Y[:, b]: batch b = blockIdx.y, float4
// accesses when every slice is 16-byte aligned (VEC), no per-element division.
template <bool VEC>
__global__ __launch_bounds__(256) void axpby2_kernel(int64_t nnz, const float *__restrict__ alpha,
                                                     float alpha0, const float *X,
                                                     const float *__restrict__ beta, float beta0,
                                                     const float *Y, float *Z) {
    const int64_t b = blockIdx.y;
    const float al = alpha ? alpha[b] : alpha0;
    const float be = Y ? (beta ? beta[b] : beta0) : 0.f;
    const int64_t off = b * nnz;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t i0 = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (VEC) {
        typedef float f4 __attribute__((ext_vector_type(4)));
        const f4 *x4 = (const f4 *)(X + off);
        const f4 *y4 = (const f4 *)(Y ? Y + off : nullptr);
        f4 *z4 = (f4 *)(Z + off);
        for (int64_t i = i0; i < nnz / 4; i += stride) {
            f4 v = al * x4[i];
            if (Y) v += be * y4[i];
            z4[i] = v;
        }
    } else {
        for (int64_t i = i0; i < nnz; i += stride) {
            float v = al * X[off + i];
            if (Y) v += be * Y[off + i];
            Z[off + i] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// out[b] = sum_i X[i, b] Y[i, b] (sum_i X[i, b] without Y) over nnz entries per
// batch, deterministic: workgroup (c, b) reduces chunk c of batch b in double
// into part[b * nchunk + c], then one workgroup per batch adds its chunks in
// order.  HBM-bound: each element is read once.
// ---------------------------------------------------------------------------
constexpr int kDotThreads = 256;

__device__ __forceinline__ double block_sum_d(double v) {
    __shared__ double wsum[kDotThreads / 64];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < kDotThreads / 64; ++w) t += wsum[w];
    return t;
}

// chunk: entries per workgroup (a multiple of 4 when VEC)
template <bool VEC, bool HASY>
__global__ __launch_bounds__(kDotThreads) void batch_dot_part_kernel(int64_t nnz, int64_t chunk,
                                                                     const float *__restrict__ X,
                                                                     const float *__restrict__ Y,
                                                                     double *__restrict__ part) {
    const int64_t b = blockIdx.y, c = blockIdx.x;
    const int64_t lo = c * chunk, hi = min(nnz, lo + chunk);
    const float *x = X + b * nnz;
    const float *y = HASY ? Y + b * nnz : nullptr;
    double acc = 0.0;
    if (VEC) {
        typedef float f4 __attribute__((ext_vector_type(4)));
        const f4 *x4 = reinterpret_cast<const f4 *>(x);
        const f4 *y4 = reinterpret_cast<const f4 *>(y);
        for (int64_t i = lo / 4 + threadIdx.x; i < hi / 4; i += kDotThreads) {
            const f4 a = x4[i];
            if (HASY) {
                const f4 e = y4[i];
                acc += ((double)a[0] * e[0] + (double)a[1] * e[1]) +
                       ((double)a[2] * e[2] + (double)a[3] * e[3]);
            } else {
                acc += ((double)a[0] + a[1]) + ((double)a[2] + a[3]);
            }
        }
    } else {
        for (int64_t i = lo + threadIdx.x; i < hi; i += kDotThreads)
            acc += HASY ? (double)x[i] * y[i] : (double)x[i];
    }
    acc = block_sum_d(acc);
    if (threadIdx.x == 0) part[b * gridDim.x + c] = acc;
}

__global__ __launch_bounds__(kDotThreads) void batch_dot_final_kernel(int nchunk,
                                                                      const double *__restrict__ part,
                                                                      float *__restrict__ out) {
    const int64_t b = blockIdx.x;
    double acc = 0.0;
    for (int c = threadIdx.x; c < nchunk; c += kDotThreads) acc += part[b * nchunk + c];
    acc = block_sum_d(acc);
    if (threadIdx.x == 0) out[b] = (float)acc;
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
static inline unsigned grid_for(int64_t n, int threads, int64_t cap = 1 << 20) {
    int64_t b = (n + threads - 1) / threads;
    if (b > cap) b = cap;
    if (b < 1) b = 1;
    return (unsigned)b;
}

hipError_t launch_pattern(const Geom &g, int64_t nb, int32_t *rowptr, int32_t *colval,
                          hipStream_t s) {
    // the float quotient t / ws of pattern32_kernel is exact for ws < 1024
    if (g.P * g.K < ((int64_t)1 << 31) - 1 && nb <= INT32_MAX && g.ws < 1024) {
        hipLaunchKernelGGL(pattern32_kernel, dim3(grid_for(g.P * 16, 256, 1 << 16)), dim3(256), 0,
                           s, g.nsp, g.n1, g.n2, g.ws, (int)nb, rowptr, colval);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(pattern_kernel, dim3(grid_for(g.P * g.K, 256)), dim3(256), 0, s, g, nb,
                       rowptr, colval);
    return hipGetLastError();
}

#define CIRCATT_ROWS_DISPATCH(KERNEL, ...)                                                   \
    do {                                                                                     \
        const int64_t rows16 = (rows + 15) / 16, rows4 = (rows + 3) / 4;                     \
        if (K <= 16 && rows16 < (1LL << 31)) {                                               \
            hipLaunchKernelGGL((KERNEL<16, 1>), dim3((unsigned)rows16), dim3(256), 0, s, __VA_ARGS__); \
            return hipGetLastError();                                                        \
        }                                                                                    \
        if (K <= 64 && rows16 < (1LL << 31)) {                                               \
            hipLaunchKernelGGL((KERNEL<16, 4>), dim3((unsigned)rows16), dim3(256), 0, s, __VA_ARGS__); \
            return hipGetLastError();                                                        \
        }                                                                                    \
        if (K <= 128 && rows16 < (1LL << 31)) {                                              \
            hipLaunchKernelGGL((KERNEL<16, 8>), dim3((unsigned)rows16), dim3(256), 0, s, __VA_ARGS__); \
            return hipGetLastError();                                                        \
        }                                                                                    \
        if (K <= 256 && rows16 < (1LL << 31)) {                                              \
            hipLaunchKernelGGL((KERNEL<16, 16>), dim3((unsigned)rows16), dim3(256), 0, s, __VA_ARGS__); \
            return hipGetLastError();                                                        \
        }                                                                                    \
        if (K <= 1024 && rows4 < (1LL << 31)) {                                              \
            hipLaunchKernelGGL((KERNEL<64, 16>), dim3((unsigned)rows4), dim3(256), 0, s, __VA_ARGS__); \
            return hipGetLastError();                                                        \
        }                                                                                    \
    } while (0)

hipError_t launch_softmax(int K, int64_t rows, const float *in, float *out, hipStream_t s) {
    CIRCATT_ROWS_DISPATCH(softmax_rows_kernel, K, rows, in, out);
    hipLaunchKernelGGL(softmax_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, K,
                       rows, in, out);
    return hipGetLastError();
}

hipError_t launch_softmax_bwd(int K, int64_t rows, const float *A, const float *dA, float *dS,
                              hipStream_t s) {
    CIRCATT_ROWS_DISPATCH(softmax_bwd_rows_kernel, K, rows, A, dA, dS);
    hipLaunchKernelGGL(softmax_bwd_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s,
                       K, rows, A, dA, dS);
    return hipGetLastError();
}

template <int NCOMP, bool TRANS, bool CORR>
static hipError_t launch_apply_t(const Geom &g, int C, int64_t nb, float scale, const float *nz,
                                 const float *x, const float *z, float *y, hipStream_t s) {
    constexpr int CH = 8;
    const int64_t total = g.P * nb * ((C + CH - 1) / CH);
    hipLaunchKernelGGL((apply_kernel<NCOMP, TRANS, CORR, CH>), dim3(grid_for(total, 256, 1LL << 31)),
                       dim3(256), 0, s, g, C, nb, scale, nz, x, z, y);
    return hipGetLastError();
}

hipError_t launch_apply(bool trans, bool corr, int ncomp, const Geom &g, int C, int64_t nb,
                        float scale, const float *nz, const float *x, const float *z, float *y,
                        hipStream_t s) {
    if (apply_rb_supported(g, C, ncomp, nb))
        return launch_apply_rb(trans, corr, ncomp, g, C, nb, scale, nz, x, z, y, s);
    if (apply_wide_supported(g, C, ncomp, nb))
        return launch_apply_wide(trans, corr, ncomp, g, C, nb, scale, nz, x, z, y, s);
#define CIRCATT_APPLY_CASE(NC, T, CR)                                       \
    if (ncomp == NC && trans == T && corr == CR)                            \
        return launch_apply_t<NC, T, CR>(g, C, nb, scale, nz, x, z, y, s);
    CIRCATT_APPLY_CASE(1, false, false)
    CIRCATT_APPLY_CASE(1, true, false)
    CIRCATT_APPLY_CASE(1, false, true)
    CIRCATT_APPLY_CASE(1, true, true)
    CIRCATT_APPLY_CASE(2, false, false)
    CIRCATT_APPLY_CASE(2, true, false)
    CIRCATT_APPLY_CASE(2, false, true)
    CIRCATT_APPLY_CASE(2, true, true)
#undef CIRCATT_APPLY_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_similarity(bool dist, int ncomp, const Geom &g, int C, int64_t nb, float scale,
                             const float *x, const float *y, float *nz, hipStream_t s) {
    const unsigned grid = grid_for(g.P * g.K * nb, 256, 1LL << 31);
    if (ncomp == 1 && !dist)
        hipLaunchKernelGGL((similarity_kernel<1, false>), dim3(grid), dim3(256), 0, s, g, C, nb, scale, x, y, nz);
    else if (ncomp == 1 && dist)
        hipLaunchKernelGGL((similarity_kernel<1, true>), dim3(grid), dim3(256), 0, s, g, C, nb, scale, x, y, nz);
    else if (!dist)
        hipLaunchKernelGGL((similarity_kernel<2, false>), dim3(grid), dim3(256), 0, s, g, C, nb, scale, x, y, nz);
    else
        hipLaunchKernelGGL((similarity_kernel<2, true>), dim3(grid), dim3(256), 0, s, g, C, nb, scale, x, y, nz);
    return hipGetLastError();
}

hipError_t launch_sum(bool col, const Geom &g, int64_t nb, const float *nz, float *out,
                      hipStream_t s) {
    if (!col && (g.P * nb + 15) / 16 < (1LL << 31)) {
        hipLaunchKernelGGL(rowsum_kernel, dim3((unsigned)((g.P * nb + 15) / 16)), dim3(256), 0, s,
                           g.K, g.P * nb, nz, out);
        return hipGetLastError();
    }
    if (col && apply_rb_supported(g, 1, 1, nb)) return launch_colsum_rb(g, nb, nz, out, s);
    if (col && apply_wide_supported(g, 1, 1, nb)) return launch_colsum_wide(g, nb, nz, out, s);
    const unsigned grid = grid_for(g.P * nb, 256, 1LL << 31);
    if (col)
        hipLaunchKernelGGL(sum_kernel<true>, dim3(grid), dim3(256), 0, s, g, nb, nz, out);
    else
        hipLaunchKernelGGL(sum_kernel<false>, dim3(grid), dim3(256), 0, s, g, nb, nz, out);
    return hipGetLastError();
}

hipError_t launch_axpby(int64_t nnz, int64_t nb, const float *alpha, float alpha0,
                        const float *X, const float *beta, float beta0, const float *Y, float *Z,
                        hipStream_t s) {
    if (nb <= 65535) {
        const bool vec = nnz % 4 == 0 && ((uintptr_t)X | (uintptr_t)Z | (uintptr_t)Y) % 16 == 0;
        const int64_t n = vec ? nnz / 4 : nnz;
        const unsigned gx = grid_for(n, 256, std::max<int64_t>(1, 4096 / nb));
        if (vec)
            hipLaunchKernelGGL(axpby2_kernel<true>, dim3(gx, (unsigned)nb), dim3(256), 0, s, nnz,
                               alpha, alpha0, X, beta, beta0, Y, Z);
        else
            hipLaunchKernelGGL(axpby2_kernel<false>, dim3(gx, (unsigned)nb), dim3(256), 0, s, nnz,
                               alpha, alpha0, X, beta, beta0, Y, Z);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(axpby_kernel, dim3(grid_for(nnz * nb, 256, 1 << 16)), dim3(256), 0, s,
                       nnz, nb, alpha, alpha0, X, beta, beta0, Y, Z);
    return hipGetLastError();
}

int batch_dot_chunks(int64_t nnz) {
    const int64_t n = (nnz + 65535) / 65536;  // 64 Ki entries per workgroup
    return (int)std::max<int64_t>(1, std::min<int64_t>(1024, n));
}

hipError_t launch_batch_dot(int64_t nnz, int64_t nb, const float *X, const float *Y, float *out,
                            void *work, hipStream_t s) {
    const int nchunk = batch_dot_chunks(nnz);
    const bool vec = nnz % 4 == 0 && ((uintptr_t)X | (uintptr_t)Y) % 16 == 0;
    int64_t chunk = (nnz + nchunk - 1) / nchunk;
    chunk = (chunk + 3) / 4 * 4;
    double *part = static_cast<double *>(work);
    // batches in slices of at most 65535 (grid y)
    for (int64_t b0 = 0; b0 < nb; b0 += 65535) {
        const unsigned nbs = (unsigned)std::min<int64_t>(65535, nb - b0);
        const float *xs = X + b0 * nnz;
        const float *ys = Y ? Y + b0 * nnz : nullptr;
        double *ps = part + b0 * nchunk;
        const dim3 grid((unsigned)nchunk, nbs);
        if (vec && Y)
            hipLaunchKernelGGL((batch_dot_part_kernel<true, true>), grid, dim3(kDotThreads), 0, s,
                               nnz, chunk, xs, ys, ps);
        else if (vec)
            hipLaunchKernelGGL((batch_dot_part_kernel<true, false>), grid, dim3(kDotThreads), 0, s,
                               nnz, chunk, xs, ys, ps);
        else if (Y)
            hipLaunchKernelGGL((batch_dot_part_kernel<false, true>), grid, dim3(kDotThreads), 0, s,
                               nnz, chunk, xs, ys, ps);
        else
            hipLaunchKernelGGL((batch_dot_part_kernel<false, false>), grid, dim3(kDotThreads), 0, s,
                               nnz, chunk, xs, ys, ps);
        hipLaunchKernelGGL(batch_dot_final_kernel, dim3(nbs), dim3(kDotThreads), 0, s, nchunk, ps,
                           out + b0);
    }
    return hipGetLastError();
}

}  // namespace circatt
