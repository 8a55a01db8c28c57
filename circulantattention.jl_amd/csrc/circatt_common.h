// Shared definitions for the circulant attention HIP library (gfx950).
//
// Index conventions (identical to the reference's Julia arrays):
//   * a signal of Julia size (N1[,N2], C, nb) stores element (pixel r,
//     channel c, batch b) at r + P*(c + C*b), P = N1*N2, pixel r = i1 + N1*i2;
//     ComplexF32 elements are interleaved (re, im) float pairs;
//   * a Circulant's CSR row r (the query pixel) owns nz slots r*K .. r*K+K-1
//     (K = ws^nsp) of each batch; nzVal is (P*K, nb) Float32, colVal/rowPtr
//     are Int32 1-based (src/circulant.jl:64-106, src/array.jl:6-11).
//
// Slot <-> window offset.  src/circulant.jl:6-44 orders the K slots of a row
// by window offset, dim 1 fastest, circularly shifting the order of a
// dimension when the row's position j (1-based) lies within p of a border.
// Per dimension of size N with window M = 2p+1:
//   shift s(j) = j-p-1 if j <= p;  p-N+j if j > N-p;  0 otherwise
//   slot m (0-based) -> offset d = mod(m - s, M) - p   (circshift_index)
//   offset d         -> slot m   = mod(d + p + s, M)
//   column position  = mod(j-1 + d, N)
// The map slot <-> offset is a bijection per row, so every row holds each
// offset of [-p, p]^nsp exactly once, also when ws > N (then several offsets
// hit the same column).  All kernels here enumerate offsets, which is what
// makes the key-centric (transposed) passes possible without atomics.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace circatt {

__host__ __device__ __forceinline__ int64_t pmod64(int64_t a, int64_t n) {
    int64_t r = a % n;
    return r < 0 ? r + n : r;
}
__host__ __device__ __forceinline__ int pmod(int a, int n) {
    int r = a % n;
    return r < 0 ? r + n : r;
}

// Division by a run-time constant d >= 1 as a multiply-high and a shift (the
// round-up method of Granlund and Montgomery, "Division by invariant integers
// using multiplication", PLDI 1994): l = ceil(log2 d),
// m = floor(2^32 (2^l - d) / d) + 1, and n / d = (mulhi(n, m) + n) >> l for
// 0 <= n < 2^31 (the sum stays below 2^32).  Kernels divide wave-uniform
// indices this way in scalar instructions instead of the vector expansion of
// an integer division.
struct FastDiv {
    uint32_t m, l;
};
inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    return FastDiv{(uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1), l};
}
__device__ __forceinline__ int fdiv(int n, FastDiv d) {
    return (int)((__umulhi((uint32_t)n, d.m) + (uint32_t)n) >> d.l);
}

// shift s(j) of one dimension, j is 1-based (src/circulant.jl:10-14, 30-39)
__host__ __device__ __forceinline__ int slot_shift(int j1, int N, int p) {
    if (j1 <= p) return j1 - p - 1;
    if (j1 > N - p) return p - N + j1;
    return 0;
}
__host__ __device__ __forceinline__ int slot_to_offset(int m, int s, int M, int p) {
    return pmod(m - s, M) - p;
}
__host__ __device__ __forceinline__ int offset_to_slot(int d, int s, int M, int p) {
    return pmod(d + p + s, M);
}

// Tile (th, tw) of tile number t on a tiles_h x tiles_w grid, in bands of 8
// tile rows, column by column within a band (the last band may be shorter):
// consecutive tile numbers form compact 8-row blocks, so the tiles a GPU
// region runs at once share their halos in its cache.  A bijection.
__host__ __device__ __forceinline__ void banded_tile(int t, int tiles_h, int tiles_w, int &th, int &tw) {
    const int full = (tiles_h >> 3) * 8 * tiles_w;  // tiles in full bands
    if (t < full) {
        const int band = t / (8 * tiles_w), r = t - band * 8 * tiles_w;
        th = 8 * band + (r & 7);
        tw = r >> 3;
    } else {
        const int bh = tiles_h & 7, r = t - full;
        th = (tiles_h & ~7) + r % bh;
        tw = r / bh;
    }
}

// Geometry of one problem: nsp spatial dims, N1 (fastest) and N2 (1 for 1D),
// window ws along each spatial dim.
struct Geom {
    int nsp;
    int n1, n2;
    int ws, p;
    int64_t P;  // pixels
    int K;      // slots per row = ws^nsp
};

__host__ __device__ __forceinline__ Geom make_geom(int nsp, int n1, int n2, int ws) {
    Geom g;
    g.nsp = nsp;
    g.n1 = n1;
    g.n2 = nsp == 1 ? 1 : n2;
    g.ws = ws;
    g.p = (ws - 1) / 2;
    g.P = (int64_t)g.n1 * g.n2;
    g.K = nsp == 1 ? ws : ws * ws;
    return g;
}

// Offsets (d1, d2) of slot t of row r.  d2 = 0 in 1D.
__host__ __device__ __forceinline__ void slot_offsets(const Geom &g, int64_t r, int t, int &d1,
                                                      int &d2) {
    int i1 = (int)(r % g.n1);
    if (g.nsp == 1) {
        d1 = slot_to_offset(t, slot_shift(i1 + 1, g.n1, g.p), g.ws, g.p);
        d2 = 0;
    } else {
        int i2 = (int)(r / g.n1);
        int m0 = t % g.ws, mm = t / g.ws;
        d1 = slot_to_offset(m0, slot_shift(i1 + 1, g.n1, g.p), g.ws, g.p);
        d2 = slot_to_offset(mm, slot_shift(i2 + 1, g.n2, g.p), g.ws, g.p);
    }
}

// Slot of row r that holds offset (d1, d2).
__host__ __device__ __forceinline__ int offset_slot(const Geom &g, int64_t r, int d1, int d2) {
    int i1 = (int)(r % g.n1);
    int m0 = offset_to_slot(d1, slot_shift(i1 + 1, g.n1, g.p), g.ws, g.p);
    if (g.nsp == 1) return m0;
    int i2 = (int)(r / g.n1);
    int mm = offset_to_slot(d2, slot_shift(i2 + 1, g.n2, g.p), g.ws, g.p);
    return mm * g.ws + m0;
}

// Pixel at offset (d1, d2) from pixel r, circular in both dims.
__host__ __device__ __forceinline__ int64_t offset_pixel(const Geom &g, int64_t r, int d1,
                                                         int d2) {
    int i1 = (int)(r % g.n1);
    int j1 = pmod(i1 + d1, g.n1);
    if (g.nsp == 1) return j1;
    int i2 = (int)(r / g.n1);
    int j2 = pmod(i2 + d2, g.n2);
    return (int64_t)j1 + (int64_t)g.n1 * j2;
}

}  // namespace circatt
