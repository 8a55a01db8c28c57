// Compile-time-window fused kernels for 2D circulant attention on gfx950.
//
// Specialisation of the windowed-tile scheme (fused_impl.h) for 2D windows of
// half width P <= 7 with exactly 16 or 32 real components per head (Float32
// dh = 16, 32; ComplexF32 dh = 8, 16).  It serves the forward, the
// query-centric backward (dq, D) and the key-centric backward (dk, dv).
//
// Measured on MI355X, FP32 VALU instructions do not overlap FP32 MFMA work
// of the same SIMD (a VALU fma costs ~2.4 cycles per wave, one
// v_mfma_f32_16x16x4f32 32 cycles, and the two add up), so these kernels are
// built to spend as few VALU instructions per MFMA as possible:
//   * the whole window geometry is a template constant: every LDS address is
//     a lane base plus an immediate offset, and every window mask is a 64-bit
//     lane mask constant applied with one v_cndmask per masked value (values
//     of a block that are valid in every lane take no mask at all);
//   * the register-side operand of the score product is pre-scaled by
//     scale * log2(e), and the per-row softmax terms enter the score product
//     as its initial accumulator (the -lse row term of the backward, the -D
//     term of dP - D, the Distance key bias), so P = exp2(acc) and
//     dS = P * acc2 cost one exp and one multiply per value;
//   * the forward keeps the scores of its 16 queries in registers, one or two
//     chunks of blocks at a time, and takes each chunk's exact maximum (one
//     rescale between the two chunks);
//   * global loads are buffer loads whose channel stride is a scalar offset,
//     so staging a pixel costs no vector address arithmetic.
//
// Work decomposition (as in fused_impl.h): persistent workgroups walk
// XCD-contiguous runs of (tile, unit) items; the circularly wrapped halo of
// the other side is staged in LDS, with the next item's global loads issued
// into registers before the current item is computed.  A workgroup is a
// WH x WW grid of wavefronts over a (8 WH) x (2 WW) tile; wavefront (wh, ww)
// holds the 8 (dim 1) x 2 (dim 2) register pixels at tile rows 8 wh ..
// 8 wh + 7, columns 2 ww, 2 ww + 1 (lane j -> (j % 8, j / 8)) and walks the
// 2 x 8 LDS blocks covering their windows (element e -> (e % 2, e / 2)).
// The wave grid is the largest of 2x8, 1x8 and 1x4 whose halo fits LDS
// (2x8, four waves per SIMD, for 16 components per pixel).
#pragma once
#include <stdint.h>

#include <algorithm>
#include <type_traits>

#include "circatt_common.h"
#include "circatt_kernels.h"

extern __shared__ __attribute__((aligned(16))) float circatt_lds2[];

namespace circatt {
namespace f2d {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr size_t kLdsCap = 160 * 1024;
constexpr unsigned kRsrcWord3 = 0x00020000;  // raw buffer, 32-bit data

__device__ __forceinline__ f4 mfma(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// compile-time loop: f(std::integral_constant<int, I>) for I in [B, E)
template <int I, int E>
struct SFor {
    template <typename F>
    __device__ __forceinline__ static void run(F &f) {
        f(std::integral_constant<int, I>{});
        SFor<I + 1, E>::run(f);
    }
};
template <int E>
struct SFor<E, E> {
    template <typename F>
    __device__ __forceinline__ static void run(F &) {}
};
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    SFor<B, E>::run(f);
}

// Geometry of a (P, NT) window on a WH x WW wave grid.
template <int P_, int NT_, int WH_, int WW_>
struct Geo {
    static constexpr int P = P_;
    static constexpr int NT = NT_;          // 16-component tiles per pixel
    static constexpr int WH = WH_, WW = WW_;
    static constexpr int THREADS = 64 * WH * WW;
    static constexpr int NC = 16 * NT;      // real components per pixel
    static constexpr int NS = 4 * NT;       // MFMA k-steps per product
    static constexpr int PS = NC + 4;       // LDS floats per staged pixel
    static constexpr int TH = 8 * WH, TW = 2 * WW;   // register tile of a workgroup
    static constexpr int NKH = 4 + P;       // 2-row LDS blocks per wave along dim 1
    static constexpr int NKW = (2 + 2 * P + 7) / 8;  // 8-column LDS blocks per wave along dim 2
    static constexpr int NBLK = NKH * NKW;
    static constexpr int HH = TH + 2 * P;   // staged rows
    static constexpr int HWD = 2 * (WW - 1) + 8 * NKW;  // staged columns (>= TW + 2P)
    static constexpr int CR = HH + ((2 - HH % 4) + 4) % 4;  // LDS column stride, 2 mod 4
    static constexpr int NPX = HH * HWD;    // staged pixels
    static constexpr int LPX = CR * HWD;    // LDS pixel slots per tensor
    static constexpr int PPT = (NPX + THREADS - 1) / THREADS;  // staged pixels per thread
};

enum { FWD = 0, BWDQ = 1, BWDKV = 2 };

template <int MODE, bool DIST>
struct ModeCfg {
    static constexpr int NSCAL = MODE == BWDKV ? 2 : (DIST ? 1 : 0);  // staged scalars
};

template <int P, int NT, int WH, int WW, bool DIST, int MODE>
constexpr size_t lds_bytes() {
    using G = Geo<P, NT, WH, WW>;
    return (size_t)(2 * G::LPX * G::PS + ModeCfg<MODE, DIST>::NSCAL * G::LPX) * 4;
}

#ifndef CIRCATT_F2D_NCH
#define CIRCATT_F2D_NCH 2
#endif
#ifndef CIRCATT_F2D_BIG_WW
#define CIRCATT_F2D_BIG_WW 8
#endif
// Wave grid of an instantiation: 2xBIG, else 1x8, else 1x4 (the first whose LDS fits).
template <int P, int NT, bool DIST, int MODE>
struct Grid {
    static constexpr int BW = CIRCATT_F2D_BIG_WW;
#ifdef CIRCATT_F2D_NO_BIG
    static constexpr bool big = false;
#else
    static constexpr bool big = lds_bytes<P, NT, 2, BW, DIST, MODE>() <= kLdsCap;
#endif
    static constexpr bool mid = lds_bytes<P, NT, 1, 8, DIST, MODE>() <= kLdsCap;
    static constexpr int WH = big ? 2 : 1;
    static constexpr int WW = big ? BW : mid ? 8 : 4;
    static constexpr size_t bytes = lds_bytes<P, NT, WH, WW, DIST, MODE>();
    static constexpr int THREADS = 64 * WH * WW;
    static constexpr int MINWG = bytes <= 80 * 1024 ? 2 : 1;
};

// Lane mask of valid (query, key) pairs for element r of block (bi, bj):
// lane j + 16 g holds query (j % 8, j / 8) and key element 4 g + r at
// (2 bi + r % 2, 8 bj + 2 g + r / 2) in wave-relative halo coordinates.
__host__ __device__ constexpr uint64_t lane_mask(int P, int bi, int bj, int r) {
    uint64_t m = 0;
    for (int lane = 0; lane < 64; ++lane) {
        const int j = lane & 15, g = lane >> 4;
        const int u1 = 2 * bi + (r & 1) - (j & 7);
        const int u2 = 8 * bj + 2 * g + (r >> 1) - (j >> 3);
        if (u1 >= 0 && u1 <= 2 * P && u2 >= 0 && u2 <= 2 * P) m |= 1ull << lane;
    }
    return m;
}

// v (mask bit of this lane set) or alt: one v_cndmask with the constant as
// its SGPR lane mask.  (Written with inverse_ballot rather than inline asm so
// that the compiler sees the read and inserts the wait states gfx950 needs
// after an MFMA or a transcendental result.)
template <uint64_t M>
__device__ __forceinline__ float mask_sel(float v, float alt) {
    if constexpr (M == ~0ull) {
        return v;
    } else if constexpr (M == 0) {
        return alt;
    } else {
        return __builtin_amdgcn_inverse_ballot_w64(M) ? v : alt;
    }
}
// As mask_sel, with the lane mask written into SGPRs at the point of use:
// `dep` is any wave-uniform value that changes from one loop iteration to the
// next, so the two s_mov_b32 stay inside the loop instead of being hoisted
// out of it, where dozens of live mask constants overflow the SGPR file.
template <uint64_t M>
__device__ __forceinline__ float mask_sel_d(float v, float alt, int dep) {
    if constexpr (M == ~0ull) {
        return v;
    } else if constexpr (M == 0) {
        return alt;
    } else {
        uint32_t lo, hi;
        asm("s_mov_b32 %0, %2" : "=s"(lo) : "s"(dep), "i"((int)(uint32_t)M));
        asm("s_mov_b32 %0, %2" : "=s"(hi) : "s"(dep), "i"((int)(uint32_t)(M >> 32)));
        return __builtin_amdgcn_inverse_ballot_w64(((uint64_t)hi << 32) | lo) ? v : alt;
    }
}

// Scheduling fence between the blocks of a walk: keeps the compiler from
// hoisting later blocks' LDS reads (and their registers) into earlier blocks.
#ifndef CIRCATT_F2D_FENCE
#define CIRCATT_F2D_FENCE 1
#endif
#if CIRCATT_F2D_FENCE
#define BLOCK_FENCE() __builtin_amdgcn_sched_barrier(0)
#else
#define BLOCK_FENCE() ((void)0)
#endif

// Sum / max over the four lane groups holding the same register pixel
// (lanes j, j^16, j^32, j^48).
__device__ __forceinline__ float gsum(float v) {
    unsigned u = __float_as_uint(v);
    auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    v = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    u = __float_as_uint(v);
    auto r32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}
__device__ __forceinline__ float gmax(float v) {
    unsigned u = __float_as_uint(v);
    auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    v = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
    u = __float_as_uint(v);
    auto r32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}

struct Args {
    const float *q, *k, *v, *y, *dy, *lse;
    float *yout, *lse_out, *dq, *dk, *dv, *dbuf;
    int n1, n2;
    int P;                // pixels per image
    int unit_stride;      // floats per (head, batch) unit = P * NC
    float scale, c2;      // similarity scale, scale * log2(e)
    int nunits;           // (head, batch) units
    int tiles_h, tiles_w, nitems, per_xcd;  // set by launch()
    FastDiv div_tiles, div_th;  // by tiles_h * tiles_w and by tiles_h (split-half launch)
    // channels-last tensors (C, spatial..., B): cl = 1, nheads heads per
    // image (div_nh divides by it), ncrall = floats per pixel (C *
    // components); planar when cl = 0.  The kernels take the layout as a
    // template argument; cl selects the instantiation.
    int cl, nheads, ncrall;
    FastDiv div_nh;
    // per-wave phase sums of the split-half kernels in phase-timing builds
    // (CIRCATT_F2H_PHASE); unused otherwise
    float *phase;
};

// Layout of q, k, v, y, dy and the gradients.  Planar (CL = false, the
// reference's column-major (spatial..., C, B)): unit u = (batch, head) starts
// at float u * P * ncr, pixel p sits p floats in (complex: 2p) and real
// component k P k floats further (complex: 2 P (k >> 1) + (k & 1)).
// Channels-last (CL = true, (C, spatial..., B)): unit (b, h) starts at
// b * P * ncrall + h * ncr, pixel p at p * ncrall, component k at k.  Both
// offsets separate into a pixel part (per lane) and a component part
// (constant or wave-uniform).
template <bool CL>
__device__ __forceinline__ int64_t unit_base(const Args &a, int unit) {
    if constexpr (CL) {
        const int b = fdiv(unit, a.div_nh);
        return (int64_t)b * a.P * a.ncrall + (int64_t)(unit - b * a.nheads) * (a.unit_stride / a.P);
    }
    return (int64_t)unit * a.unit_stride;
}
// bytes from the unit's base to the end of its data (the buffer range)
template <bool CL>
__device__ __forceinline__ int unit_bytes(const Args &a, int unit) {
    if constexpr (CL) {
        const int h = unit - fdiv(unit, a.div_nh) * a.nheads;
        return (a.P * a.ncrall - h * (a.unit_stride / a.P)) * 4;
    }
    return a.unit_stride * 4;
}
template <bool CPLX, bool CL>
__device__ __forceinline__ int pix_off(const Args &a, int pix) {
    if constexpr (CL) return pix * a.ncrall;
    return CPLX ? 2 * pix : pix;
}
template <bool CPLX, bool CL>
__device__ __forceinline__ int comp_soff(const Args &a, int comp) {
    if constexpr (CL) return comp;
    return CPLX ? 2 * a.P * (comp >> 1) + (comp & 1) : a.P * comp;
}

// Buffer resource over `bytes` bytes at p (loads beyond it return 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const float *p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p), (short)0, bytes, kRsrcWord3);
}
__device__ __forceinline__ float bload(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ f2 bload2(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(f2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}

// Real component `comp` of pixel `pix` in a unit (float index from the
// unit's base).
template <bool CPLX, bool CL>
__device__ __forceinline__ int comp_off(const Args &a, int pix, int comp) {
    return pix_off<CPLX, CL>(a, pix) + comp_soff<CPLX, CL>(a, comp);
}

// Work item k of this workgroup: XCD x = blockIdx % 8 owns items
// [x * per_xcd, (x + 1) * per_xcd), walked by its workgroups in turn.
__device__ __forceinline__ int item_of(const Args &a, int k) {
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, nslot = gridDim.x >> 3;
    const int it = xcd * a.per_xcd + slot + k * nslot;
    return it < min(a.nitems, (xcd + 1) * a.per_xcd) ? it : a.nitems;
}

template <int P, int NT, bool CPLX, bool DIST, int MODE, bool CL>
__global__ __launch_bounds__((Grid<P, NT, DIST, MODE>::THREADS), (Grid<P, NT, DIST, MODE>::MINWG))
void kernel2d(Args a) {
    constexpr int WH = Grid<P, NT, DIST, MODE>::WH, WW = Grid<P, NT, DIST, MODE>::WW;
    using G = Geo<P, NT, WH, WW>;
    constexpr int NC = G::NC, NS = G::NS, PS = G::PS, CR = G::CR, HH = G::HH, NKW = G::NKW;
    constexpr int NBLK = G::NBLK, PPT = G::PPT, NPX = G::NPX, LPX = G::LPX;
    constexpr int THREADS = G::THREADS;
    // forward: chunks of blocks whose scores are held in registers at once
    // (three when the wave grid leaves <= 128 VGPRs per lane)
    constexpr int NCH = MODE != FWD ? 1 : (THREADS >= 768 && NBLK > 12) ? CIRCATT_F2D_NCH : (NBLK > 12 ? 2 : 1);
    constexpr int CHB = (NBLK + NCH - 1) / NCH;
    // block at which the next item's loads are issued: the start of the
    // forward's last chunk, the middle of the backward walks
    constexpr int PFB = MODE == FWD ? (NCH - 1) * CHB : NBLK / 2;
    // LDS layout (floats): tensor 0, tensor 1 ([slot][PS]), then scalars ([slot])
    constexpr int OT1 = LPX * PS;
    constexpr int OS0 = 2 * LPX * PS;
    constexpr int OS1 = OS0 + LPX;
    float *const lds = circatt_lds2;

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int wh = wv % WH, ww = wv / WH;
    const int j = lane & 15, g = lane >> 4;
    const int jh = j & 7, jw = j >> 3;

    // lane bases (LDS pixel slots): block (bi, bj) of this wave starts at
    // slot 8 wh + 2 bi + CR (2 ww + 8 bj); element e sits (e % 2) + CR (e / 2)
    // further
    const int slotA = 8 * wh + (j & 1) + CR * (2 * ww + (j >> 1));  // element j
    const int slotE = 8 * wh + CR * (2 * ww + 2 * g);               // element 4g
    const int baseA = slotA * PS + 4 * g;
    const int baseT = slotE * PS + j;
    // Per-lane region bases, hidden from constant folding so that every
    // block offset stays a ds_read immediate (the regions lie up to 150 KB
    // apart, beyond the 64 KB immediate range).
    auto opaque = [](int v) {
        asm volatile("" : "+v"(v));
        return v;
    };
    const float *const pA0 = lds + opaque(baseA);            // product-1 rows, tensor 0
    const float *const pA1 = lds + opaque(OT1 + baseA);      // product-1 rows, tensor 1
    const float *const pT0 = lds + opaque(baseT);            // product-2 rows, tensor 0
    const float *const pT1 = lds + opaque(OT1 + baseT);      // product-2 rows, tensor 1
    const float *const pS0 = lds + opaque(OS0 + slotE);      // scalars 0 of element 4g
    const float *const pS1 = lds + opaque(OS1 + slotE);      // scalars 1 of element 4g

    // ---- prefetch registers ----
    float hv[PPT][2][NC];
    float hs[PPT][2];
    int hslot[PPT];
    float nr0[NS], nr1[NS], nry[NS];
    float nlse = 0.f;
    // Distance: lane c of the wave holds component c (mod NC) of the item's
    // centre, k at the tile's first pixel
    float nmu = 0.f;

    auto decode = [&](int item, int &unit, int &h0, int &w0) {
        const int ntiles = a.tiles_h * a.tiles_w;
        unit = item / ntiles;
        const int tile = item - unit * ntiles;
        const int th = tile % a.tiles_h;
        h0 = th * G::TH;
        w0 = (tile - th) / a.tiles_h * G::TW;
    };

    const bool big = a.n1 >= HH && a.n2 >= G::HWD;
    auto load_stage = [&](int item) {
        int unit, h0, w0;
        decode(item, unit, h0, w0);
        const int hs0 = pmod(h0 - P, a.n1), ws0 = pmod(w0 - P, a.n2);  // uniform
        const int64_t uoff = unit_base<CL>(a, unit);
        const int ubytes = unit_bytes<CL>(a, unit);
        const auto r0 = rsrc((MODE == BWDKV ? a.q : a.k) + uoff, ubytes);
        const auto r1 = rsrc((MODE == BWDKV ? a.dy : a.v) + uoff, ubytes);
#pragma unroll
        for (int pp = 0; pp < PPT; ++pp) {
            const int px0 = threadIdx.x + THREADS * pp;
            const bool pv = px0 < NPX;
            const int px = pv ? px0 : 0;
            const int kw = px / HH, kh = px - kw * HH;
            hslot[pp] = pv ? kh + CR * kw : -1;
            // wrapped halo position; one conditional subtraction when the
            // image is at least as large as the halo, a modulo otherwise
            int gh = hs0 + kh, gw = ws0 + kw;
            if (big) {
                gh -= gh >= a.n1 ? a.n1 : 0;
                gw -= gw >= a.n2 ? a.n2 : 0;
            } else {
                gh %= a.n1;
                gw %= a.n2;
            }
            const int gp = gh + a.n1 * gw;
            if constexpr (CPLX) {
#pragma unroll
                for (int c = 0; c < NC / 2; ++c) {
                    const f2 x0 = bload2(r0, pix_off<true, CL>(a, gp) * 4, comp_soff<true, CL>(a, 2 * c) * 4);
                    const f2 x1 = bload2(r1, pix_off<true, CL>(a, gp) * 4, comp_soff<true, CL>(a, 2 * c) * 4);
                    hv[pp][0][2 * c] = x0[0];
                    hv[pp][0][2 * c + 1] = x0[1];
                    hv[pp][1][2 * c] = x1[0];
                    hv[pp][1][2 * c + 1] = x1[1];
                }
            } else {
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    hv[pp][0][c] = bload(r0, pix_off<false, CL>(a, gp) * 4, comp_soff<false, CL>(a, c) * 4);
                    hv[pp][1][c] = bload(r1, pix_off<false, CL>(a, gp) * 4, comp_soff<false, CL>(a, c) * 4);
                }
            }
            if constexpr (MODE == BWDKV) {
                const int64_t soff = (int64_t)unit * a.P;
                const auto rl = rsrc(a.lse + soff, a.P * 4);
                const auto rd = rsrc(a.dbuf + soff, a.P * 4);
                hs[pp][0] = bload(rl, gp * 4, 0);
                hs[pp][1] = bload(rd, gp * 4, 0);
            }
        }
    };

    auto load_regs = [&](int item) {
        int unit, h0, w0;
        decode(item, unit, h0, w0);
        const int rh = h0 + 8 * wh + jh, rw = w0 + 2 * ww + jw;
        const bool rvalid = rh < a.n1 && rw < a.n2;
        const int rpix = rvalid ? rh + a.n1 * rw : 0;
        const int64_t uoff = unit_base<CL>(a, unit);
        const int ubytes = unit_bytes<CL>(a, unit);
        const auto r0 = rsrc((MODE == BWDKV ? a.k : a.q) + uoff, ubytes);
        const auto r1 = rsrc((MODE == BWDKV ? a.v : a.dy) + uoff, ubytes);
        // component 16 t + 4 g + c of the lane's pixel: lane part 4 g,
        // scalar part 16 t + c
        const int vo = comp_off<CPLX, CL>(a, rpix, 4 * g) * 4;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int sc = 16 * (s >> 2) + (s & 3);
            const int so = comp_soff<CPLX, CL>(a, sc) * 4;
            nr0[s] = bload(r0, vo, so);
            if constexpr (MODE != FWD) nr1[s] = bload(r1, vo, so);
            if constexpr (MODE == BWDQ) nry[s] = bload(rsrc(a.y + uoff, ubytes), vo, so);
        }
        if constexpr (MODE == BWDQ) nlse = bload(rsrc(a.lse + (int64_t)unit * a.P, a.P * 4), rpix * 4, 0);
        if constexpr (DIST)
            nmu = bload(rsrc(a.k + uoff, ubytes), comp_off<CPLX, CL>(a, h0 + a.n1 * w0, lane & (NC - 1)) * 4, 0);
    };

    int k = 0;
    int item = item_of(a, 0);
    if (item >= a.nitems) return;  // uniform over the workgroup
    load_stage(item);
    load_regs(item);

    while (true) {
        int unit, h0, w0;
        decode(item, unit, h0, w0);
        const int rh = h0 + 8 * wh + jh, rw = w0 + 2 * ww + jw;
        const bool rvalid = rh < a.n1 && rw < a.n2;
        const int rpix = rvalid ? rh + a.n1 * rw : 0;
        const int64_t uoff = unit_base<CL>(a, unit);
        const int64_t soff = (int64_t)unit * a.P;
        const float c2 = a.c2;

        // Distance: both sides of the score product centred on mu (the
        // expansion q.k - |k|^2 / 2 - |q|^2 / 2 of -|q - k|^2 / 2 then scales
        // with the spread of the data, not its offset)
        if constexpr (DIST) {
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const float mc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(nmu), c));
#pragma unroll
                for (int pp = 0; pp < PPT; ++pp) hv[pp][0][c] -= mc;
            }
#pragma unroll
            for (int s = 0; s < NS; ++s) nr0[s] -= __shfl(nmu, 16 * (s >> 2) + 4 * g + (s & 3));
        }
        __syncthreads();  // the previous item's LDS reads are done
#pragma unroll
        for (int pp = 0; pp < PPT; ++pp) {
            if (hslot[pp] >= 0) {
                const int o0 = hslot[pp] * PS;
                float n2 = 0.f;
#pragma unroll
                for (int c = 0; c < NC; c += 4) {
                    *reinterpret_cast<f4 *>(&lds[o0 + c]) =
                        f4{hv[pp][0][c], hv[pp][0][c + 1], hv[pp][0][c + 2], hv[pp][0][c + 3]};
                    *reinterpret_cast<f4 *>(&lds[OT1 + o0 + c]) =
                        f4{hv[pp][1][c], hv[pp][1][c + 1], hv[pp][1][c + 2], hv[pp][1][c + 3]};
                    if constexpr (DIST)
                        n2 += hv[pp][0][c] * hv[pp][0][c] + hv[pp][0][c + 1] * hv[pp][0][c + 1] +
                              hv[pp][0][c + 2] * hv[pp][0][c + 2] +
                              hv[pp][0][c + 3] * hv[pp][0][c + 3];
                }
                if constexpr (MODE == BWDKV) {
                    // staged queries: A_q = -lse log2(e) [- c2 |q|^2 / 2], and -D
                    lds[OS0 + hslot[pp]] = -hs[pp][0] * kLog2e - (DIST ? 0.5f * c2 * n2 : 0.f);
                    lds[OS1 + hslot[pp]] = -hs[pp][1];
                } else if constexpr (DIST) {
                    lds[OS0 + hslot[pp]] = -0.5f * c2 * n2;  // staged keys: -c2 |k|^2 / 2
                }
            }
        }
        // this item's register operands; the side that enters the score
        // product is pre-scaled by c2
        float reg0[NS], reg1[NS];
        float raw2 = 0.f;  // |x|^2 of the (unscaled) register pixel
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            if constexpr (DIST) raw2 += nr0[s] * nr0[s];
            reg0[s] = nr0[s] * c2;
            if constexpr (MODE != FWD) reg1[s] = nr1[s];
        }
        float rowD = 0.f, rowL = 0.f;
        if constexpr (MODE == BWDQ) {
            float dd = 0.f;
#pragma unroll
            for (int s = 0; s < NS; ++s) dd += nr1[s] * nry[s];
            rowD = gsum(dd);
            rowL = nlse;
        }
        const float sq = DIST ? gsum(raw2) : 0.f;
        __syncthreads();  // halo staged

        // The next item's global loads are issued part-way through this
        // item's block walk (at block PFB), which keeps their destination
        // registers out of the first blocks' register budget.
        const int nitem = item_of(a, k + 1);
        const bool has_next = nitem < a.nitems;
        auto prefetch = [&]() {
            if (has_next) {
                load_stage(nitem);
                load_regs(nitem);
            }
        };

        if constexpr (MODE == FWD) {
            // running maximum starts finite: a chunk may hold no valid key of
            // a query (then its scores are all -inf and exp2 gives 0, not NaN)
            float m = -1e30f, lsum = 0.f;
            f4 acc[2][NT];
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[u][t] = f4{0.f, 0.f, 0.f, 0.f};
            auto chunk = [&](auto CH) {
                constexpr int ci = decltype(CH)::value;
                constexpr int cb = ci * CHB;
                constexpr int ce = cb + CHB < NBLK ? cb + CHB : NBLK;
                if constexpr (cb == PFB) prefetch();
                // scores of the chunk: S[b][r] = c2 q.k (+ Distance key bias)
                f4 S[CHB];
                static_for<cb, ce>([&](auto B) {
                    constexpr int b = decltype(B)::value;
                    constexpr int bi = b / NKW, bj = b % NKW;
                    constexpr int boff = 2 * bi + CR * 8 * bj;  // block slot offset
                    BLOCK_FENCE();
                    f4 acc0 = f4{0.f, 0.f, 0.f, 0.f};
                    if constexpr (DIST) {
                        const f2 lo = *reinterpret_cast<const f2 *>(&pS0[boff]);
                        const f2 hi = *reinterpret_cast<const f2 *>(&pS0[boff + CR]);
                        acc0 = f4{lo[0], lo[1], hi[0], hi[1]};
                    }
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const f4 x = *reinterpret_cast<const f4 *>(&pA0[boff * PS + 16 * t]);
                        acc0 = mfma(x[0], reg0[4 * t + 0], acc0);
                        acc0 = mfma(x[1], reg0[4 * t + 1], acc0);
                        acc0 = mfma(x[2], reg0[4 * t + 2], acc0);
                        acc0 = mfma(x[3], reg0[4 * t + 3], acc0);
                    }
                    S[b - cb] = acc0;
                });
                // window mask and the chunk's exact row maximum
                float mx = m;
                static_for<cb, ce>([&](auto B) {
                    constexpr int b = decltype(B)::value;
                    constexpr int bi = b / NKW, bj = b % NKW;
                    f4 &s = S[b - cb];
                    s[0] = mask_sel<lane_mask(P, bi, bj, 0)>(s[0], -INFINITY);
                    s[1] = mask_sel<lane_mask(P, bi, bj, 1)>(s[1], -INFINITY);
                    s[2] = mask_sel<lane_mask(P, bi, bj, 2)>(s[2], -INFINITY);
                    s[3] = mask_sel<lane_mask(P, bi, bj, 3)>(s[3], -INFINITY);
                    mx = fmaxf(fmaxf(mx, s[0]), s[1]);
                    mx = fmaxf(fmaxf(mx, s[2]), s[3]);
                });
                const float mn = gmax(mx);
                if constexpr (ci > 0) {
                    const float alpha = __builtin_amdgcn_exp2f(m - mn);
                    lsum *= alpha;
#pragma unroll
                    for (int u = 0; u < 2; ++u)
#pragma unroll
                        for (int t = 0; t < NT; ++t) acc[u][t] *= alpha;
                }
                m = mn;
                static_for<cb, ce>([&](auto B) {
                    constexpr int b = decltype(B)::value;
                    constexpr int bi = b / NKW, bj = b % NKW;
                    constexpr int boff = 2 * bi + CR * 8 * bj;
                    BLOCK_FENCE();
                    float p[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        p[r] = __builtin_amdgcn_exp2f(S[b - cb][r] - m);
                        lsum += p[r];
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int roff = ((r & 1) + CR * (r >> 1)) * PS;
#pragma unroll
                        for (int t = 0; t < NT; ++t)
                            acc[b & 1][t] = mfma(pT1[boff * PS + roff + 16 * t],
                                                 p[r], acc[b & 1][t]);
                    }
                });
            };
            static_for<0, NCH>(chunk);
            const float l = gsum(lsum);
            const float inv = 1.f / l;
            if (rvalid) {
                float *yb = a.yout + uoff;
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        yb[comp_off<CPLX, CL>(a, rpix, 16 * t + 4 * g + r)] =
                            (acc[0][t][r] + acc[1][t][r]) * inv;
                if (g == 0)
                    a.lse_out[soff + rpix] =
                        (m + __log2f(l)) * kLn2 - (DIST ? 0.5f * sq * a.scale : 0.f);
            }
        } else if constexpr (MODE == BWDQ) {
            // initial accumulators: -lse log2(e) [- c2 |q|^2 / 2] and -D
            const float nl = -rowL * kLog2e - (DIST ? 0.5f * c2 * sq : 0.f);
            const f4 cS = f4{nl, nl, nl, nl};
            const f4 cD = f4{-rowD, -rowD, -rowD, -rowD};
            f4 acc[2][NT];
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[u][t] = f4{0.f, 0.f, 0.f, 0.f};
            float corr = 0.f;
            static_for<0, NBLK>([&](auto B) {
                constexpr int b = decltype(B)::value;
                constexpr int bi = b / NKW, bj = b % NKW;
                constexpr int boff = 2 * bi + CR * 8 * bj;
                BLOCK_FENCE();
                if constexpr (b == PFB) prefetch();
                f4 s = cS, dp = cD;
                if constexpr (DIST) {
                    const f2 lo = *reinterpret_cast<const f2 *>(&pS0[boff]);
                    const f2 hi = *reinterpret_cast<const f2 *>(&pS0[boff + CR]);
                    s = s + f4{lo[0], lo[1], hi[0], hi[1]};
                }
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const f4 x = *reinterpret_cast<const f4 *>(&pA0[boff * PS + 16 * t]);
                    const f4 w =
                        *reinterpret_cast<const f4 *>(&pA1[boff * PS + 16 * t]);
                    s = mfma(x[0], reg0[4 * t + 0], s);
                    dp = mfma(w[0], reg1[4 * t + 0], dp);
                    s = mfma(x[1], reg0[4 * t + 1], s);
                    dp = mfma(w[1], reg1[4 * t + 1], dp);
                    s = mfma(x[2], reg0[4 * t + 2], s);
                    dp = mfma(w[2], reg1[4 * t + 2], dp);
                    s = mfma(x[3], reg0[4 * t + 3], s);
                    dp = mfma(w[3], reg1[4 * t + 3], dp);
                }
                float ds[4];
                ds[0] = mask_sel<lane_mask(P, bi, bj, 0)>(__builtin_amdgcn_exp2f(s[0]), 0.f) * dp[0];
                ds[1] = mask_sel<lane_mask(P, bi, bj, 1)>(__builtin_amdgcn_exp2f(s[1]), 0.f) * dp[1];
                ds[2] = mask_sel<lane_mask(P, bi, bj, 2)>(__builtin_amdgcn_exp2f(s[2]), 0.f) * dp[2];
                ds[3] = mask_sel<lane_mask(P, bi, bj, 3)>(__builtin_amdgcn_exp2f(s[3]), 0.f) * dp[3];
                if constexpr (DIST) corr += (ds[0] + ds[1]) + (ds[2] + ds[3]);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int roff = ((r & 1) + CR * (r >> 1)) * PS;
#pragma unroll
                    for (int t = 0; t < NT; ++t)
                        acc[b & 1][t] =
                            mfma(pT0[boff * PS + roff + 16 * t], ds[r], acc[b & 1][t]);
                }
            });
            const float rs = DIST ? gsum(corr) : 0.f;
            if (rvalid) {
                float *ob = a.dq + uoff;
                const float invc2 = 1.f / c2;
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float val = acc[0][t][r] + acc[1][t][r];
                        if constexpr (DIST) val -= rs * reg0[4 * t + r] * invc2;
                        ob[comp_off<CPLX, CL>(a, rpix, 16 * t + 4 * g + r)] = val * a.scale;
                    }
                if (g == 0) a.dbuf[soff + rpix] = rowD;
            }
        } else {  // BWDKV: register pixels are keys, LDS pixels are queries
            const float kb = DIST ? -0.5f * c2 * sq : 0.f;  // key bias
            f4 accv[2][NT], acck[2][NT];
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    accv[u][t] = f4{0.f, 0.f, 0.f, 0.f};
                    acck[u][t] = f4{0.f, 0.f, 0.f, 0.f};
                }
            float corr = 0.f;
            static_for<0, NBLK>([&](auto B) {
                constexpr int b = decltype(B)::value;
                constexpr int bi = b / NKW, bj = b % NKW;
                constexpr int boff = 2 * bi + CR * 8 * bj;
                BLOCK_FENCE();
                if constexpr (b == PFB) prefetch();
                const f2 alo = *reinterpret_cast<const f2 *>(&pS0[boff]);
                const f2 ahi = *reinterpret_cast<const f2 *>(&pS0[boff + CR]);
                const f2 dlo = *reinterpret_cast<const f2 *>(&pS1[boff]);
                const f2 dhi = *reinterpret_cast<const f2 *>(&pS1[boff + CR]);
                f4 s = f4{alo[0], alo[1], ahi[0], ahi[1]};
                if constexpr (DIST) s = s + f4{kb, kb, kb, kb};
                f4 dp = f4{dlo[0], dlo[1], dhi[0], dhi[1]};
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const f4 x = *reinterpret_cast<const f4 *>(&pA0[boff * PS + 16 * t]);
                    const f4 w =
                        *reinterpret_cast<const f4 *>(&pA1[boff * PS + 16 * t]);
                    s = mfma(x[0], reg0[4 * t + 0], s);
                    dp = mfma(w[0], reg1[4 * t + 0], dp);
                    s = mfma(x[1], reg0[4 * t + 1], s);
                    dp = mfma(w[1], reg1[4 * t + 1], dp);
                    s = mfma(x[2], reg0[4 * t + 2], s);
                    dp = mfma(w[2], reg1[4 * t + 2], dp);
                    s = mfma(x[3], reg0[4 * t + 3], s);
                    dp = mfma(w[3], reg1[4 * t + 3], dp);
                }
                float p[4], ds[4];
                p[0] = mask_sel<lane_mask(P, bi, bj, 0)>(__builtin_amdgcn_exp2f(s[0]), 0.f);
                p[1] = mask_sel<lane_mask(P, bi, bj, 1)>(__builtin_amdgcn_exp2f(s[1]), 0.f);
                p[2] = mask_sel<lane_mask(P, bi, bj, 2)>(__builtin_amdgcn_exp2f(s[2]), 0.f);
                p[3] = mask_sel<lane_mask(P, bi, bj, 3)>(__builtin_amdgcn_exp2f(s[3]), 0.f);
#pragma unroll
                for (int r = 0; r < 4; ++r) ds[r] = p[r] * dp[r];
                if constexpr (DIST) corr += (ds[0] + ds[1]) + (ds[2] + ds[3]);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int roff = ((r & 1) + CR * (r >> 1)) * PS;
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        accv[b & 1][t] = mfma(pT1[boff * PS + roff + 16 * t], p[r],
                                              accv[b & 1][t]);
                        acck[b & 1][t] =
                            mfma(pT0[boff * PS + roff + 16 * t], ds[r], acck[b & 1][t]);
                    }
                }
            });
            const float cs = DIST ? gsum(corr) : 0.f;
            if (rvalid) {
                float *vb = a.dv + uoff;
                float *kbp = a.dk + uoff;
                const float invc2 = 1.f / c2;
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int o = comp_off<CPLX, CL>(a, rpix, 16 * t + 4 * g + r);
                        vb[o] = accv[0][t][r] + accv[1][t][r];
                        float val = acck[0][t][r] + acck[1][t][r];
                        if constexpr (DIST) val -= cs * reg0[4 * t + r] * invc2;
                        kbp[o] = val * a.scale;
                    }
            }
        }

        if (!has_next) break;
        ++k;
        item = nitem;
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
template <int P, int NT, bool CPLX, bool DIST, int MODE, bool CL>
hipError_t launch(const Args &a0, int cus, hipStream_t s) {
    using GR = Grid<P, NT, DIST, MODE>;
    using G = Geo<P, NT, GR::WH, GR::WW>;
    static_assert(GR::bytes <= kLdsCap, "halo does not fit LDS");
    auto kern = kernel2d<P, NT, CPLX, DIST, MODE, CL>;
    // set once per instantiation (a function-local static is initialised
    // exactly once, also when several host threads launch at the same time)
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)GR::bytes);
    if (attr != hipSuccess) return attr;
    Args a = a0;
    a.tiles_h = (a.n1 + G::TH - 1) / G::TH;
    a.tiles_w = (a.n2 + G::TW - 1) / G::TW;
    const int64_t nitems = (int64_t)a.tiles_h * a.tiles_w * a.nunits;
    if (nitems <= 0 || nitems > INT32_MAX / 2) return hipErrorNotSupported;
    a.nitems = (int)nitems;
    a.per_xcd = (int)((nitems + 7) / 8);
    if (CL) a.div_nh = make_fastdiv((uint32_t)a.nheads);
    int64_t grid = (int64_t)cus * GR::MINWG;
    grid = std::min<int64_t>(grid, 8LL * a.per_xcd);
    grid = std::max<int64_t>(8, grid / 8 * 8);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(G::THREADS), GR::bytes, s, a);
    return hipGetLastError();
}

// Launch of one mode for the compiled-in shapes: half widths P in
// {1, 2, 3, 5, 7}, 16 or 32 real components per pixel, Float32 or
// ComplexF32, Dot or Distance.  Other shapes return hipErrorNotSupported
// without launching.
template <int MODE>
hipError_t dispatch(int p, int nt, bool cplx, bool dist, const Args &a, int cus, hipStream_t s) {
#define CIRCATT_F2D_CL(PP, NTT, CLL)                                                   \
    {                                                                                  \
        if (cplx) return dist ? launch<PP, NTT, true, true, MODE, CLL>(a, cus, s)      \
                              : launch<PP, NTT, true, false, MODE, CLL>(a, cus, s);    \
        return dist ? launch<PP, NTT, false, true, MODE, CLL>(a, cus, s)               \
                    : launch<PP, NTT, false, false, MODE, CLL>(a, cus, s);             \
    }
#define CIRCATT_F2D_CASE(PP, NTT)                                                      \
    if (p == PP && nt == NTT) {                                                        \
        if (a.cl) CIRCATT_F2D_CL(PP, NTT, true)                                        \
        CIRCATT_F2D_CL(PP, NTT, false)                                                 \
    }
    CIRCATT_F2D_CASE(1, 1)
    CIRCATT_F2D_CASE(2, 1)
    CIRCATT_F2D_CASE(3, 1)
    CIRCATT_F2D_CASE(5, 1)
    CIRCATT_F2D_CASE(7, 1)
    CIRCATT_F2D_CASE(1, 2)
    CIRCATT_F2D_CASE(2, 2)
    CIRCATT_F2D_CASE(3, 2)
    CIRCATT_F2D_CASE(5, 2)
    CIRCATT_F2D_CASE(7, 2)
#undef CIRCATT_F2D_CASE
#undef CIRCATT_F2D_CL
    return hipErrorNotSupported;
}

// Shapes the compile-time-window kernels cover.  Offsets are 32-bit: a unit
// of P * 16 NT floats must stay below 2^31 bytes.
inline bool supported(int nsp, int p, int ncr, int64_t P) {
    return nsp == 2 && (p == 1 || p == 2 || p == 3 || p == 5 || p == 7) &&
           (ncr == 16 || ncr == 32) && P * ncr * 4 < (int64_t)INT32_MAX;
}

}  // namespace f2d

// One translation unit per mode (fused2d_<mode>.hip).
hipError_t launch_f2d_fwd(int p, int nt, bool cplx, bool dist, const f2d::Args &a, int cus,
                          hipStream_t s);
hipError_t launch_f2d_bwdq(int p, int nt, bool cplx, bool dist, const f2d::Args &a, int cus,
                           hipStream_t s);
hipError_t launch_f2d_bwdkv(int p, int nt, bool cplx, bool dist, const f2d::Args &a, int cus,
                            hipStream_t s);

}  // namespace circatt
