// Split-half kernels for 2D circulant attention on gfx950.
//
// Same work decomposition and window geometry as the Float32 kernels of
// fused2d_impl.h (16x16 tiles, 16 wavefronts, 8x2 register blocks, 2x8 LDS
// blocks), but every product runs on the f16 matrix cores
// (v_mfma_f32_16x16x32_f16: 16 cycles for a 16x16 block over 32 terms,
// against 32 cycles over 4 terms for v_mfma_f32_16x16x4f32).  Each Float32
// operand x is carried as two halves, x = hi + lo with hi = f16(x) and
// lo = f16(x - hi), and a product a.b is taken as hi.hi + lo.hi + hi.lo
// (+ lo.lo where it is free) with Float32 accumulation: the relative error
// stays near 2^-21 per operand, the order of Float32 rounding.  On gfx950
// Float32 MFMA and vector instructions do not overlap, so the cheaper
// products leave the softmax vector work as the larger part of a block.
//
// Contraction layouts (lane j + 16 g; the 32 terms of one MFMA are the
// 8 g .. 8 g + 7 of every lane):
//   * score-type products (contraction over the 16 channels): terms 0..15
//     are hi channels, 16..31 lo channels of the LDS pixel, against the
//     register pixel's hi (first MFMA) or lo (second MFMA) channels
//     8 (g & 1) .. 8 (g & 1) + 7;
//   * apply-type products (contraction over the keys of two blocks b, b+1):
//     terms 8 g .. 8 g + 3 are elements 4 g .. 4 g + 3 of block b, terms
//     8 g + 4 .. 8 g + 7 the same elements of block b+1, which is where the
//     score accumulators of the two blocks already sit in the lane.
//
// LDS per staged pixel: [16 hi | 16 lo | pad] halves.  Score-type rows are
// 16-byte reads of a slot; apply-type rows (one channel of four elements)
// come from the same slots through the transposing read ds_read_b64_tr_b16.
//
// The halves alone would lose Float32's range (lo turns subnormal below
// 2^-3, every half overflows at 65520), so each item scales its operands by
// powers of two before the split and undoes the scale on the Float32 results
// (see shift_of below); waves whose scores could overflow the halves take a
// slower walk that unscales every score after its product.
#pragma once
#include "fused2d_impl.h"

// Scheduling fences of the forward walk.  The backward passes keep
// BLOCK_FENCE between block pairs (without it the key-centric pass
// interleaves blocks and runs out of registers); the forward fences its apply
// pairs but lets the score products of a chunk schedule freely (measured best
// on gfx950: fences everywhere cost 4%, none at all 7%).
#ifndef CIRCATT_F2H_SGB
#define CIRCATT_F2H_SGB 0
#endif
#ifndef CIRCATT_F2H_FWD_FENCE
#define CIRCATT_F2H_FWD_FENCE 2
#endif
// Per-wave phase timing, off by default (microbench/phase_timing.py builds a
// library with it on).  Every wave sums s_memtime spans of four phases over
// its items: staging (without the barriers), the barrier after the maxima, the
// barrier after the staging, and the walk with its epilogue.  Wave w of
// workgroup b < 8 writes the four sums (as 32-bit integers) to floats
// 4 (16 b + w) .. + 3 of a dedicated buffer of 512 floats, which such a build
// takes through circatt_debug_set_phase_buffer (defined in fused2h_fwd.hip
// only when CIRCATT_F2H_PHASE is set; a null buffer writes nothing).
#ifndef CIRCATT_F2H_PHASE
#define CIRCATT_F2H_PHASE 0
#endif
#if CIRCATT_F2H_PHASE
#define F2H_PHASE(...) __VA_ARGS__
namespace circatt {
float *&phase_buffer();
}
#else
#define F2H_PHASE(...)
#endif
// bit 0: between score blocks, bit 1: between apply pairs
#if CIRCATT_F2H_FWD_FENCE & 1
#define FWD_FENCE_S() __builtin_amdgcn_sched_barrier(0)
#else
#define FWD_FENCE_S() ((void)0)
#endif
#if CIRCATT_F2H_FWD_FENCE & 2
#define FWD_FENCE_A() __builtin_amdgcn_sched_barrier(0)
#else
#define FWD_FENCE_A() ((void)0)
#endif

namespace circatt {
namespace f2h {

using f2d::Args;
using f2d::f4;
using f2d::gmax;
using f2d::gsum;
using f2d::kLn2;
using f2d::kLog2e;
using f2d::mask_sel;
using f2d::mask_sel_d;
using f2d::static_for;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f4 mfmah(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// -1.0f the compiler cannot see: fma(h, -1, x) with a literal -1 folds to
// x - h, which loses the mixed-precision form below (the SALU move is hoisted
// to one SGPR).
__device__ __forceinline__ float opaque_neg_one() {
    float c;
    asm("s_mov_b32 %0, -1.0" : "=s"(c));
    return c;
}
// hi = f16(x), lo = f16(x - hi): one packed conversion for hi, then
// v_fma_mix_f32 takes x - hi exactly in Float32 from each packed half (the
// difference is representable), and a second packed conversion rounds the two
// differences once into lo.  On gfx950 the packed conversions and
// v_fma_mix_f32 issue at half rate, v_fma_mixlo_f16 / v_fma_mixhi_f16 (which
// would round into the halves of lo directly) at quarter rate: 8.4 against
// 10.2 cycles per value of a SIMD shared by four waves, with the same halves.
// Only empty asm statements steer the instruction selection (the first keeps
// hi one packed value, the second keeps the Float32 differences), so these
// are ordinary compiler instructions and the compiler inserts the wait states
// they need next to matrix-core operations.
__device__ __forceinline__ void split2(float x0, float x1, h2 &hi, h2 &lo) {
    const float m1 = opaque_neg_one();
    h2 h = h2{(_Float16)x0, (_Float16)x1};
    asm("" : "+v"(h));
    float d0 = __builtin_fmaf((float)h[0], m1, x0);
    float d1 = __builtin_fmaf((float)h[1], m1, x1);
    asm("" : "+v"(d0), "+v"(d1));
    hi = h;
    lo = h2{(_Float16)d0, (_Float16)d1};
}
// 4 values -> hi, lo as one half of a pair operand
__device__ __forceinline__ void split4(const float (&x)[4], h4 &hi, h4 &lo) {
    h2 a0, a1, b0, b1;
    split2(x[0], x[1], a0, b0);
    split2(x[2], x[3], a1, b1);
    hi = h4{a0[0], a0[1], a1[0], a1[1]};
    lo = h4{b0[0], b0[1], b1[0], b1[1]};
}
// transposing LDS read (ds_read_b64_tr_b16): within each group of 16 lanes,
// lane 4 t + a supplies the address of 4 consecutive halves x[t][4a .. 4a+3]
// and lane i receives x[0..3][i]
typedef short s4v __attribute__((vector_size(8)));
__device__ __forceinline__ h4 ldtr(const char *p) {
    const s4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s4v *)(p));
    return __builtin_bit_cast(h4, v);
}
// 16-byte LDS-DMA load: each active lane's 16 bytes from byte voff of the
// buffer rs to LDS byte m0 + 16 lane (m0 wave-uniform).  Inline assembly
// rather than __builtin_amdgcn_raw_ptr_buffer_load_lds: after the builtin the
// compiler waits for every load in flight before the next LDS read, as it
// cannot tell the DMA rows from the slots the walk reads, which would expose
// the whole prefetch at the start of each walk.  The callers wait for the rows
// (vmcnt(0) and a barrier) before reading them.  (The compiler writes M0 for
// the asm; one wait state then separates that write from the load.)
typedef int i4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i4v dma_rsrc(const float *p, int bytes) {
    const uint64_t b = reinterpret_cast<uint64_t>(p);
    return i4v{(int)(uint32_t)b, (int)((b >> 32) & 0xffffu), bytes, (int)f2d::kRsrcWord3};
}
__device__ __forceinline__ void dma16(i4v rs, unsigned m0, int voff) {
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :
                 : "v"(voff), "s"(rs), "{m0}"(m0)
                 : "memory");
}
__device__ __forceinline__ h8 cat(h4 a, h4 b) {
    return h8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Wave priority over the N pair steps of an item's walk: 3 for the first
// quarter, then 2, 1, 0.  A SIMD's arbiter issues for the oldest of its
// highest-priority waves; with equal priorities the four waves of a SIMD end
// an item's walk in age order (forward at cfg3 on gfx950: the four slot
// groups after 128k, 184k, 235k and 277k cycles of walk) and the last runs
// its tail alone, with no latency hidden, while the others wait at the
// barrier.  Lowering a wave's priority as it advances lets the waves behind
// it issue (164k .. 260k), which cuts the cycles per launch (forward 331k ->
// 317k per wave, query-centric pass 346k -> 324k); the clock drops with the
// higher utilisation, so the gain in time is smaller.  The key-centric pass
// uses walk_prio_tail instead (below).
// (CIRCATT_F2H_PRIO=0 keeps equal priorities, for the comparison)
#ifndef CIRCATT_F2H_PRIO
#define CIRCATT_F2H_PRIO 1
#endif
template <int I, int N>
__device__ __forceinline__ void walk_prio() {
    if constexpr (CIRCATT_F2H_PRIO && I * 4 % N < 4) __builtin_amdgcn_s_setprio(3 - I * 4 / N);
}
// Key-centric pass: priority 1 over the first three quarters of the walk, 0
// over the last, so that a wave in its last quarter yields to the waves
// behind it.  Measured at cfg3 on gfx950 (interleaved A/B, two boxes): key-
// centric pass 233.5 -> 227.6 us; the quarter steps of walk_prio gave 0.7%,
// two steps (at one half and three quarters) 1%, a single drop at one half
// was slower (+3%).
template <int I, int N>
__device__ __forceinline__ void walk_prio_tail() {
    if constexpr (CIRCATT_F2H_PRIO && I == 0) __builtin_amdgcn_s_setprio(1);
    if constexpr (CIRCATT_F2H_PRIO && I == (3 * N) / 4) __builtin_amdgcn_s_setprio(0);
}

// LDS pixel slot: NT sub-pixels of 16 channels, each [16 hi | 16 lo] halves
// (64 bytes), then 8 halves of pad: 80 bytes for 16 real components, 144 for
// 32 (both strides keep the 16-byte row reads free of bank conflicts)
template <int NT>
constexpr int slot_bytes() { return (32 * NT + 8) * 2; }
// Workgroup grid: 2 x 8 wavefronts (16x16 tiles) for 16 real components per
// pixel; 1 x 8 (8x16 tiles) for 32, whose two staged tensors would not fit
// LDS on the larger tile
template <int NT>
constexpr int grid_wh() { return NT == 1 ? 2 : 1; }

// ---- power-of-two operand scaling ----
// f16 halves lose Float32's range: lo turns subnormal (spacing 2^-24) once
// |x| < 2^-3 and every half overflows at 65520.  Operands are therefore
// scaled by powers of two (exact) before the split, chosen from the largest
// magnitude m over what is staged for an item (or over a register pixel),
// and the scale is undone on the Float32 results.  With b the biased
// exponent of m (m < 2^(b - 126)), shift_of(b) is 0 when m lies in
// [2^-2, 2^5) and otherwise the shift that brings m into [4, 8).
__device__ __forceinline__ int shift_of(unsigned b) {
    return (b >= 125u && b <= 131u) ? 0 : 129 - (int)b;
}
// biased exponent of a non-negative float (its bits >> 23; 255 for inf/NaN)
__device__ __forceinline__ unsigned bexp(float m) { return __float_as_uint(m) >> 23; }
// exponent e with |x * 2^shift_of(b)| < 2^e for every x of the set
__device__ __forceinline__ int scaled_exp(unsigned b) { return (int)b - 126 + shift_of(b); }

template <int N>
__device__ __forceinline__ float maxabs(const float (&x)[N]) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < N; ++i) m = fmaxf(m, fabsf(x[i]));
    return m;
}
// maximum of a non-negative value (as bits) over the wave, in lane 63
template <int CTRL, int ROWS>
__device__ __forceinline__ unsigned dpp_umax(unsigned u) {
    const unsigned o = (unsigned)__builtin_amdgcn_update_dpp(0, (int)u, CTRL, ROWS, 0xf, false);
    return u > o ? u : o;
}
__device__ __forceinline__ unsigned wave_umax63(unsigned u) {
    u = dpp_umax<0x111, 0xf>(u);  // row_shr:1
    u = dpp_umax<0x112, 0xf>(u);  // row_shr:2
    u = dpp_umax<0x114, 0xf>(u);  // row_shr:4
    u = dpp_umax<0x118, 0xf>(u);  // row_shr:8  (lane 15 of each row: the row's maximum)
    u = dpp_umax<0x142, 0xa>(u);  // row_bcast:15 into rows 1, 3
    u = dpp_umax<0x143, 0xc>(u);  // row_bcast:31 into rows 2, 3
    return u;
}

// slot store of 16 Float32 values as [16 hi | 16 lo] halves, each scaled by
// 2^s first when SC
template <bool SC = false>
__device__ __forceinline__ void store_slot(char *sp, const float (&xin)[16], int s = 0) {
    float x[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) x[c] = SC ? __builtin_amdgcn_ldexpf(xin[c], s) : xin[c];
    h2 hi[8], lo[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) split2(x[2 * c], x[2 * c + 1], hi[c], lo[c]);
#pragma unroll
    for (int c = 0; c < 8; c += 4) {
        *reinterpret_cast<f4 *>(sp + 4 * c) =
            f4{__builtin_bit_cast(float, hi[c]), __builtin_bit_cast(float, hi[c + 1]),
               __builtin_bit_cast(float, hi[c + 2]), __builtin_bit_cast(float, hi[c + 3])};
        *reinterpret_cast<f4 *>(sp + 32 + 4 * c) =
            f4{__builtin_bit_cast(float, lo[c]), __builtin_bit_cast(float, lo[c + 1]),
               __builtin_bit_cast(float, lo[c + 2]), __builtin_bit_cast(float, lo[c + 3])};
    }
}

// register operand: channels 8 (g & 1) .. + 7 of the lane's pixel, scaled, split
__device__ __forceinline__ void reg_split(const float (&x)[8], float sc, h8 &hi, h8 &lo) {
    h2 a[4], b[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) split2(x[2 * c] * sc, x[2 * c + 1] * sc, a[c], b[c]);
    hi = h8{a[0][0], a[0][1], a[1][0], a[1][1], a[2][0], a[2][1], a[3][0], a[3][1]};
    lo = h8{b[0][0], b[0][1], b[1][0], b[1][1], b[2][0], b[2][1], b[3][0], b[3][1]};
}

enum { FWD = f2d::FWD, BWDQ = f2d::BWDQ, BWDKV = f2d::BWDKV };

// Tile and block geometry.  A wavefront holds an 8x2 block of register
// pixels (queries in the forward) and walks LDS blocks of 16 pixels covering
// their (8 + 2P) x (2 + 2P) window region: 2x8 blocks, or at windows 3 and
// 11 4x4 blocks, which cover that region with fewer pixels (ws 11: 15
// blocks, 240 pixels, against 18 blocks, 288).
// Element e = 4 g + r of a block (the score accumulator's row) sits at block
// row e / 8, column e % 8 (2x8 blocks, row-major), or at row r, column g
// (4x4).  LDS slots are column-major with CR slots per column: CR = 2 mod 4
// for 2x8 blocks and CR = 4 mod 16 for 4x4 blocks, which keeps the 16-byte
// reads of a block's rows (slot stride 80 or 144 bytes) free of bank
// conflicts.  With 2x8 blocks the row-major element order also keeps the
// transposing reads free of them: the 16 lanes of a lane group read 32-byte
// runs of four slots CR apart, and the 32 lanes of two groups eight slots of
// one block row, which fall on distinct banks of the 64 (4 bytes each): the
// slot stride is an odd number of 16-byte units and CR is even.  2x2 element
// groups put two of a group's four runs on the same banks.  Per-slot Float32
// scalars are stored row-major for 2x8 blocks (so that a lane group's four
// elements are adjacent) and column-major, like the slots, for 4x4 blocks.
// 4x4 blocks reach
// BR * NKH - (8 + 2P) rows past the staged ones, into the pad rows of the
// column; those rows, and staged-region columns past the last staged one,
// hold zeros written once per launch and are read only under the mask.
//
// One-dimensional signals (ONE): a wavefront holds 16 consecutive register
// pixels and walks 16x1 LDS blocks (BR = 16) of the 16 + 2P keys around them;
// the workgroup's wavefronts are stacked along the line (TH = 16 per
// wavefront, TW = 1) and the staged halo is one slot column of TH + 2P pixels,
// padded with zero slots to the end of the last wavefront's last block.
template <int P, int NT, bool ONE = false>
struct HGeo {
    static constexpr int WH = ONE ? 8 * grid_wh<NT>() : grid_wh<NT>(), WW = ONE ? 1 : 8;
    static constexpr int THREADS = 64 * WH * WW;
    static constexpr int TH = ONE ? 16 * WH : 8 * WH, TW = ONE ? 1 : 2 * WW;
    static constexpr int BR = ONE ? 16 : (P == 1 || P == 5) ? 4 : 2;  // block rows
    static constexpr int BC = 16 / BR;                                   // block columns
    static constexpr int NKH = ONE ? (16 + 2 * P + 15) / 16 : (8 + 2 * P + BR - 1) / BR;
    static constexpr int NKW = ONE ? 1 : (2 + 2 * P + BC - 1) / BC;
    static constexpr int NBLK = NKH * NKW;
    static constexpr int HH = TH + 2 * P;
    static constexpr int HWD = ONE ? 1 : 2 * (WW - 1) + BC * NKW;
    static constexpr int CR = ONE     ? 16 * (WH - 1) + 16 * NKH   // LDS column stride
                              : BR == 2 ? HH + ((2 - HH % 4) + 4) % 4
                                        : HH + ((4 - HH % 16) + 16) % 16;
    static constexpr int LPX = CR * HWD;                    // LDS pixel slots per tensor
    // slot offset of block b within a wavefront's region
    static constexpr int bslot(int b) { return BR * (b / NKW) + CR * BC * (b % NKW); }
    // index of the scalar of the pixel at slot row `row`, column `col`, and
    // the scalar offset of block b within a wavefront's region
    static constexpr int sidx(int row, int col) { return BR == 2 ? col + HWD * row : row + CR * col; }
    // first slot row of wavefront row wh's region
    static constexpr int wrow(int wh) { return ONE ? 16 * wh : 8 * wh; }
    static constexpr int sbslot(int b) { return sidx(BR * (b / NKW), BC * (b % NKW)); }
    // central pair of the streamed forward: two blocks of the block row that
    // holds key rows 8, 9 (in every query's window when 2P >= 9); for smaller
    // windows the two block rows that hold key row 7 (4..7 with 2x8 blocks,
    // 0..7 with 4x4); ONE: the pair of keys 32 PCENT .. 32 PCENT + 31 of the
    // 16 + 2P key region
    static constexpr int PCENT = ONE ? (8 + P) / 32 : P >= 5 ? (8 / BR) * NKW / 2 : 7 / (2 * BR);
    static_assert(wrow(WH - 1) + BR * NKH <= CR, "a wavefront's blocks stay within their column's slots");
    static_assert(HH <= CR, "the staged rows fit the column");
    static_assert((8 / BR) * NKW % 2 == 0, "the central pair lies in one block row");
    // (ONE) query j of a wavefront has region keys j .. j + 2P in its window:
    // the central pair's keys meet every one of those windows
    static_assert(!ONE || (32 * PCENT <= 2 * P && 32 * PCENT + 31 >= 15 && 2 * PCENT < NBLK),
                  "the central pair holds a key of every query's window");
    // (2D) query (i, j) of a wavefront's 8x2 block has region rows i .. i + 2P
    // and columns j .. j + 2P in its window: the central pair's rows and
    // columns (one rectangle) meet every one of them
    static constexpr bool central_ok() {
        const int b0 = 2 * PCENT, b1 = 2 * PCENT + 1 < NBLK ? 2 * PCENT + 1 : 2 * PCENT;
        const int ra = BR * (b0 / NKW), rb = BR * (b1 / NKW), ca = BC * (b0 % NKW), cb = BC * (b1 % NKW);
        const int r0 = ra < rb ? ra : rb, r1 = (ra < rb ? rb : ra) + BR - 1;
        const int c0 = ca < cb ? ca : cb, c1 = (ca < cb ? cb : ca) + BC - 1;
        const bool rect = ra == rb || ca == cb;
        return rect && 2 * PCENT < NBLK && r0 <= 2 * P && r1 >= 7 && c0 <= 2 * P && c1 >= 1;
    }
    static_assert(ONE || central_ok(), "the central pair holds a key of every query's window");
};
static_assert(HGeo<5, 2>::LPX == 520 && HGeo<5, 2>::NBLK == 15, "4x4 blocks at ws 11");
static_assert(HGeo<7, 1>::LPX == f2d::Geo<7, 1, 2, 8>::LPX && HGeo<7, 1>::NBLK == f2d::Geo<7, 1, 2, 8>::NBLK,
              "2x8 geometry as the Float32 kernels'");

// lane j + 16 g holds query (j % 8, j / 8) and key element 4 g + r of block
// (bi, bj); bit set where the key lies in the query's window
// (BR = 16: 16x1 register and LDS blocks of a one-dimensional signal, element
// 4 g + r of block bi at row 16 bi + 4 g + r, query j at row j)
template <int BR>
__host__ __device__ constexpr uint64_t hmask(int P, int bi, int bj, int r) {
    uint64_t m = 0;
    for (int lane = 0; lane < 64; ++lane) {
        const int j = lane & 15, g = lane >> 4;
        const int kr = BR == 16 ? 16 * bi + 4 * g + r : BR == 2 ? 2 * bi + (g >> 1) : 4 * bi + r;
        const int kc = BR == 16 ? 0 : BR == 2 ? 8 * bj + 4 * (g & 1) + r : 4 * bj + g;
        const int u1 = kr - (BR == 16 ? j : j & 7), u2 = kc - (BR == 16 ? 0 : j >> 3);
        if (u1 >= 0 && u1 <= 2 * P && u2 >= 0 && u2 <= 2 * P) m |= 1ull << lane;
    }
    return m;
}
// the Float32 kernels (f2d::lane_mask) keep the 2x2 element groups
static_assert(hmask<2>(7, 3, 1, 2) != f2d::lane_mask(7, 3, 1, 2), "row-major 2x8 elements");

// WIDE (one-dimensional planar Float32 signals whose length is a multiple of
// 4): the next item's halo and register pixels arrive by 16-byte LDS-DMA
// loads (4 pixels of one channel per lane) into planar buffers, XS (staged
// tensors: channel-major rows of NXS pixels from the halo origin rounded down
// to a multiple of 4, XA pixels earlier) and XR (register tensors: rows of the
// tile's TH pixels), which the staging and the register set-up read.  A lane
// of a dword load moves 4 bytes, and a wavefront can keep only so many loads
// in flight: with the short walks of a one-dimensional window the dword loads
// of the staged and register pixels bounded the passes.
template <int P, int NT, int MODE, bool DIST, bool ONE = false, bool WIDE = false>
struct LGeo {
    using G = HGeo<P, NT, ONE>;
    static constexpr int NCH = 16 * NT;                                // real components per pixel
    static constexpr int XA = (4 - P % 4) % 4;                         // halo origin - XS origin
    static constexpr int NXS = (G::HH + XA + 3) / 4 * 4;               // XS pixels per row
    static constexpr int NRT = MODE == FWD ? 1 : MODE == BWDQ ? 3 : 2;  // register tensors
    static constexpr int SB = slot_bytes<NT>();
    static constexpr int OT0 = 0;                  // tensor 0 slots (K, or Q in BWDKV)
    static constexpr int OT1 = G::LPX * SB;        // tensor 1 slots (V, or dY in BWDKV)
    static constexpr int OS0 = 2 * OT1;            // Float32 scalars per slot
    static constexpr int OS1 = OS0 + G::LPX * 4;
    static constexpr int NSCAL = MODE == BWDKV ? 2 : (DIST ? 1 : 0);
    // per-item exchange of maxima: 4 words of (item << 9 | biased exponent)
    static constexpr int OX = OS0 + NSCAL * G::LPX * 4;
    static constexpr int OXS = OX + 16;                         // (WIDE) staged tensors, planar
    static constexpr int OXR = OXS + (WIDE ? 2 * NCH * NXS * 4 : 0);  // (WIDE) register tensors
    static constexpr int bytes = OXR + (WIDE ? NRT * NCH * G::TH * 4 : 0);
    static_assert(!WIDE || (ONE && G::TH <= 256), "register rows: one DMA instruction per channel");
};

// NT: 16-channel sub-pixels per pixel (1 or 2, i.e. 16 or 32 real components);
// ONE: one-dimensional signal (n2 = 1)
template <int P, int NT, bool CPLX, bool DIST, int MODE, bool CL, bool ONE = false, bool WIDE = false>
__global__ __launch_bounds__((HGeo<P, NT, ONE>::THREADS), 1) void kernel2h(Args a) {
    using G = HGeo<P, NT, ONE>;
    using L = LGeo<P, NT, MODE, DIST, ONE, WIDE>;
    static_assert(!WIDE || (ONE && !CPLX && !CL), "planar DMA rows: one-dimensional planar Float32");
    constexpr int WH = G::WH;
    constexpr int BR = G::BR;
    constexpr int SB = L::SB;
    constexpr int CR = G::CR, HH = G::HH, HWD = G::HWD, NKW = G::NKW, NBLK = G::NBLK;
    // staged columns: all HWD slot columns on the 16x16 tile; on the 8x16
    // tile only the TW + 2P that lie in some query's window (the slot columns
    // past them are read by the last LDS blocks under the window mask and
    // hold zeros, written once)
    constexpr int SWC = ONE ? 1 : NT == 1 ? HWD : G::TW + 2 * P;
    constexpr int NPX = HH * SWC;
    constexpr int NPAIR = (NBLK + 1) / 2;
    constexpr bool KV = MODE == BWDKV;
    // forward: pair chunks whose scores are held in registers at once
    constexpr int NCH = (MODE == FWD && NPAIR > 6) ? 2 : 1;
    constexpr int CHP = (NPAIR + NCH - 1) / NCH;
    // pair at which the next item's loads are issued (the streamed forward
    // issues them before its walk; otherwise the forward issues them in its
    // apply walk, with two chunks at the last pair of the first, so that the
    // loads are in flight over the whole second chunk).  Backward:
    // pair NPAIR / PFD; measured on gfx950, the query-centric pass is fastest
    // with its loads issued at a quarter of the walk (200 against 205 us at
    // cfg3), the key-centric pass at half of it
#ifndef CIRCATT_F2H_BWD_PFD
#define CIRCATT_F2H_BWD_PFD 2
#endif
#ifndef CIRCATT_F2H_BWDQ_PFD
#define CIRCATT_F2H_BWDQ_PFD 4
#endif
#ifndef CIRCATT_F2H_BWD_FSTEP
#define CIRCATT_F2H_BWD_FSTEP 1
#endif
    // Backward passes of 32-component 2D kernels (two wavefronts per SIMD,
    // 64 staged values per thread): the next item's loads start at the
    // second pair and spread over three (cfg5: query-centric pass 144 -> 140
    // us, key-centric 170 -> 160 us against all loads at one pair, a quarter
    // and half way through the walk); 16-component kernels keep one pair
    // (spreading was 2% slower in their query-centric pass at cfg3)
    constexpr bool SPREAD = !ONE && MODE != FWD && NT == 2;
    // every forward takes its reference maximum from the central block pair
    // PCENT, which holds a key of every query's window
    constexpr bool STREAM = MODE == FWD;
    constexpr int PFP = STREAM                      ? 0
                        : (MODE == FWD && NCH == 2)   ? CHP - 1
                        : (SPREAD && NPAIR > 3)       ? 1
                        : MODE == BWDQ                ? NPAIR / CIRCATT_F2H_BWDQ_PFD
                                                      : NPAIR / CIRCATT_F2H_BWD_PFD;
    static_assert(PFP >= 0 && PFP < NPAIR, "the next item's loads must be issued in the walk");
    static_assert(NPX <= G::THREADS, "one staged pixel per thread");
    // HALF: two threads per staged pixel of 32 components, one sub-pixel of
    // 16 each (where the halo has at most half as many pixels as the
    // workgroup has threads: one-dimensional signals), so that the staging
    // loads spread over more wavefronts; NCS components staged per thread
    constexpr bool HALF = NT == 2 && 2 * NPX <= G::THREADS;
    constexpr int NCS = HALF ? 16 : 16 * NT;
    static_assert(NT == 1 || NT == 2, "16 or 32 real components per head");
    static_assert(HH % 2 == 0, "row pairs");
    char *const lds = reinterpret_cast<char *>(circatt_lds2);
    // LDS byte address of the array (the DMA loads' M0 base)
    typedef __attribute__((address_space(3))) const char *lcp;
    const unsigned lds0 = __builtin_amdgcn_readfirstlane((unsigned)reinterpret_cast<uintptr_t>((lcp)lds));

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int wh = wv % WH, ww = wv / WH;
    const int j = lane & 15, g = lane >> 4;
    const int jh = ONE ? j : j & 7, jw = ONE ? 0 : j >> 3;

    auto opaque = [](int v) {
        asm volatile("" : "+v"(v));
        return v;
    };
    // score-type rows: element j of a block, halves 8 g .. 8 g + 7 of its slot
    const int slotA = ONE       ? G::wrow(wh) + j
                      : BR == 2 ? 8 * wh + (j >> 3) + CR * (2 * ww + (j & 7))
                                : 8 * wh + (j & 3) + CR * (2 * ww + (j >> 2));
    const char *const pA0 = lds + opaque(L::OT0 + slotA * SB + 16 * g);
    const char *const pA1 = lds + opaque(L::OT1 + slotA * SB + 16 * g);
    // apply-type rows from slots by transposing reads: lane (j, g) receives
    // channel j (hi; lo 16 halves further) of elements 4g + t, t = 0..3, so
    // lane j of group g addresses channels 4 (j & 3) .. + 3 of element
    // 4g + (j >> 2), which sits at row g / 2, column 4 (g % 2) + (j >> 2)
    // (2x8), at row j >> 2, column g (4x4) or at row 4g + (j >> 2) (16x1)
    const int slotE = ONE       ? G::wrow(wh) + 4 * g
                      : BR == 2 ? 8 * wh + (g >> 1) + CR * (2 * ww + 4 * (g & 1))
                                : 8 * wh + CR * (2 * ww + g);
    const int slotT = BR == 2 ? slotE + CR * (j >> 2) : slotE + (j >> 2);
    const char *const pR0 = lds + opaque(L::OT0 + slotT * SB + 8 * (j & 3));
    const char *const pR1 = lds + opaque(L::OT1 + slotT * SB + 8 * (j & 3));
    // per-slot Float32 scalars of elements 4g .. 4g+3 (adjacent)
    const int sidxE = ONE       ? G::wrow(wh) + 4 * g
                      : BR == 2 ? G::sidx(8 * wh + (g >> 1), 2 * ww + 4 * (g & 1))
                                : G::sidx(8 * wh, 2 * ww + g);
    const float *const pS0 = reinterpret_cast<const float *>(lds + opaque(L::OS0 + sidxE * 4));
    const float *const pS1 = reinterpret_cast<const float *>(lds + opaque(L::OS1 + sidxE * 4));

    // ---- prefetch registers ----
    float h0v[NCS], h1v[NCS], hs0 = 0.f, hs1 = 0.f;
    int hslot;
    // register operands: lane groups g and g ^ 2 (lanes l, l ^ 32) share a
    // pixel and its channels 8 (g & 1) .. + 7 of each sub-pixel h; each loads
    // half of them, components 16 h + 8 (g & 1) + 4 (g >> 1) + t, and a lane
    // swap joins the halves
    float nh0[NT][4], nh1[NT][4], nry[NT][4];
    float nlse = 0.f;
    // Distance: lane c of the wave holds component c (mod 16 NT) of the
    // item's centre, k at the tile's first pixel
    float nmu = 0.f;

    // register pixel of this lane in the tile at (h0, w0)
    auto regpix = [&](int h0, int w0, bool &rvalid, int &rpix) {
        const int rh = h0 + G::wrow(wh) + jh, rw = w0 + 2 * ww + jw;
        rvalid = rh < a.n1 && rw < a.n2;
        rpix = rvalid ? rh + a.n1 * rw : 0;
    };
    // item -> (head, batch) unit and tile origin; wave-uniform, so scalar
    // instructions with the launch's precomputed divisors
    auto decode = [&](int item, int &unit, int &h0, int &w0) {
        unit = fdiv(item, a.div_tiles);
        const int tile = item - unit * (a.tiles_h * a.tiles_w);
        const int tw = fdiv(tile, a.div_th);
        h0 = (tile - tw * a.tiles_h) * G::TH;
        w0 = tw * G::TW;
    };
    const bool big = a.n1 >= HH && a.n2 >= HWD;
    const int px = HALF ? threadIdx.x >> 1 : threadIdx.x;
    const int hsub = HALF ? threadIdx.x & 1 : 0;  // staged sub-pixel (HALF)
    const int kw = px / HH, kh = px - kw * HH;
    const int hsid = G::sidx(kh, kw);  // scalar index of the staged pixel
    // wavefronts with no staged pixel issue no staging loads (one-dimensional
    // halos only: in 2D every wavefront or all but one stage pixels, and the
    // branch would split the walk's basic block around the prefetch)
    const bool stw = !ONE || (HALF ? 32 * wv : 64 * wv) < NPX;
    // HP: -1 all of the staged loads, 0 / 1 the first / second half of the
    // components (with the scalars in the first)
    auto load_stage = [&](int unit, int h0, int w0, auto HP) __attribute__((always_inline)) {
        constexpr int hp = decltype(HP)::value;
        // halo origin (h0 - P, w0 - P) mod (n1, n2), uniform
        int hsh = h0 - P, wsh = ONE ? 0 : w0 - P;
        while (hsh < 0) hsh += a.n1;
        while (wsh < 0) wsh += a.n2;
        const int64_t uoff = f2d::unit_base<CL>(a, unit);
        const int ubytes = f2d::unit_bytes<CL>(a, unit);
        const auto r0 = f2d::rsrc((KV ? a.q : a.k) + uoff, ubytes);
        const auto r1 = f2d::rsrc((KV ? a.dy : a.v) + uoff, ubytes);
        hslot = px < NPX ? kh + CR * kw : -1;
        if constexpr (WIDE && hp != 1) {
            // XS rows: wavefront wv loads channels wv + NW cg of both tensors
            // (every operand but the lane offset a per-wavefront base plus a
            // constant: few scalar instructions per load); in part m of a row
            // (256 pixels) lane l loads pixels o4 + 4 (64 m + l) .. + 3 (mod
            // n1: o4 and n1 are multiples of 4, so no chunk straddles the wrap)
            constexpr int NPART = (L::NXS + 255) / 256;
            constexpr int NW = G::THREADS / 64, KC = L::NCH / NW;
            static_assert(L::NCH % NW == 0, "whole channel groups per wavefront");
            const int o4 = hsh >= L::XA ? hsh - L::XA : hsh - L::XA + a.n1;
            const bool bigx = a.n1 >= L::NXS;
            const i4v d0 = dma_rsrc((KV ? a.q : a.k) + uoff, ubytes);
            const i4v d1 = dma_rsrc((KV ? a.dy : a.v) + uoff, ubytes);
            const int wvu = __builtin_amdgcn_readfirstlane(wv);
            const unsigned m0w = lds0 + L::OXS + wvu * L::NXS * 4;
            const int cstep = NW * a.P * 4;  // bytes between the channels of one wavefront
#pragma unroll
            for (int part = 0; part < NPART; ++part) {
                const int l4 = 64 * part + lane;
                int p4 = o4 + 4 * l4;
                p4 = bigx ? (p4 >= a.n1 ? p4 - a.n1 : p4) : p4 % a.n1;
                const int vo = (p4 + wvu * a.P) * 4;
                // (only the last part has idle lanes)
                if (part + 1 < NPART || l4 < L::NXS / 4) {
#pragma unroll
                    for (int t = 0; t < 2; ++t)
#pragma unroll
                        for (int cg = 0; cg < KC; ++cg)
                            dma16(t ? d1 : d0, m0w + ((t * L::NCH + NW * cg) * L::NXS + 256 * part) * 4,
                                  vo + cg * cstep);
                }
            }
        }
        if (!stw) {
            // (zeros rather than an early return, which would keep the
            // previous item's values live across the walk)
#pragma unroll
            for (int c = 0; c < NCS; ++c) h0v[c] = h1v[c] = 0.f;
            hs0 = hs1 = 0.f;
            return;
        }
        int gh = hsh + kh, gw = wsh + kw;
        if (big) {
            gh -= gh >= a.n1 ? a.n1 : 0;
            gw -= gw >= a.n2 ? a.n2 : 0;
        } else {
            gh %= a.n1;
            gw %= a.n2;
        }
        const int gp = gh + a.n1 * gw;
        // (component offsets are linear in the component, so the sub-pixel's
        // first one joins the per-lane offset)
        if constexpr (WIDE) {
            // (read from the XS rows at the item's start)
        } else if constexpr (CPLX) {
            const int vb = (f2d::pix_off<true, CL>(a, gp) + f2d::comp_soff<true, CL>(a, 16 * hsub)) * 4;
#pragma unroll
            for (int c = hp == 1 ? NCS / 4 : 0; c < (hp == 0 ? NCS / 4 : NCS / 2); ++c) {
                const int vo = vb, so = f2d::comp_soff<true, CL>(a, 2 * c) * 4;
                const f2d::f2 x0 = f2d::bload2(r0, vo, so);
                const f2d::f2 x1 = f2d::bload2(r1, vo, so);
                h0v[2 * c] = x0[0];
                h0v[2 * c + 1] = x0[1];
                h1v[2 * c] = x1[0];
                h1v[2 * c + 1] = x1[1];
            }
        } else {
            const int vb = (f2d::pix_off<false, CL>(a, gp) + f2d::comp_soff<false, CL>(a, 16 * hsub)) * 4;
#pragma unroll
            for (int c = hp == 1 ? NCS / 2 : 0; c < (hp == 0 ? NCS / 2 : NCS); ++c) {
                const int vo = vb, so = f2d::comp_soff<false, CL>(a, c) * 4;
                h0v[c] = f2d::bload(r0, vo, so);
                h1v[c] = f2d::bload(r1, vo, so);
            }
        }
        if constexpr (KV && hp != 1) {
            const int64_t soff = (int64_t)unit * a.P;
            hs0 = f2d::bload(f2d::rsrc(a.lse + soff, a.P * 4), gp * 4, 0);
            hs1 = f2d::bload(f2d::rsrc(a.dbuf + soff, a.P * 4), gp * 4, 0);
        }
    };
    auto load_regs = [&](int unit, int h0, int w0) __attribute__((always_inline)) {
        bool rvalid;
        int rpix;
        regpix(h0, w0, rvalid, rpix);
        const int64_t uoff = f2d::unit_base<CL>(a, unit);
        const int ubytes = f2d::unit_bytes<CL>(a, unit);
        const auto r0 = f2d::rsrc((KV ? a.k : a.q) + uoff, ubytes);
        const auto r1 = f2d::rsrc((KV ? a.v : a.dy) + uoff, ubytes);
        if constexpr (WIDE) {
            // XR rows: wavefront wv loads channels wv + NW cg of each register
            // tensor; lane l the tile's pixels h0 + 4l .. + 3 (those past n1
            // belong to no register pixel)
            constexpr int NW = G::THREADS / 64, KC = L::NCH / NW;
            const i4v d0 = dma_rsrc((KV ? a.k : a.q) + uoff, ubytes);
            const i4v d1 = dma_rsrc((KV ? a.v : a.dy) + uoff, ubytes);
            const i4v dy = dma_rsrc(a.y + uoff, ubytes);
            const int wvu = __builtin_amdgcn_readfirstlane(wv);
            const unsigned m0r = lds0 + L::OXR + wvu * G::TH * 4;
            const int vr = (h0 + 4 * lane + wvu * a.P) * 4;
            const int cstep = NW * a.P * 4;
            if (lane < G::TH / 4) {
#pragma unroll
                for (int rt = 0; rt < L::NRT; ++rt)
#pragma unroll
                    for (int cg = 0; cg < KC; ++cg)
                        dma16(rt == 0 ? d0 : rt == 1 ? d1 : dy, m0r + ((rt * L::NCH + NW * cg) * G::TH) * 4,
                              vr + cg * cstep);
            }
        }
#pragma unroll
        for (int h = 0; h < NT && !WIDE; ++h) {
            const int vo = f2d::comp_off<CPLX, CL>(a, rpix, 16 * h + 8 * (g & 1) + 4 * (g >> 1)) * 4;
            if constexpr (CPLX || CL) {
                // components t, t + 1 adjacent (real and imaginary part, or
                // channels-last): one 8-byte load per pair
#pragma unroll
                for (int t = 0; t < 4; t += 2) {
                    const int so = f2d::comp_soff<CPLX, CL>(a, t) * 4;
                    const f2d::f2 x0 = f2d::bload2(r0, vo, so);
                    nh0[h][t] = x0[0];
                    nh0[h][t + 1] = x0[1];
                    if constexpr (MODE != FWD) {
                        const f2d::f2 x1 = f2d::bload2(r1, vo, so);
                        nh1[h][t] = x1[0];
                        nh1[h][t + 1] = x1[1];
                    }
                    if constexpr (MODE == BWDQ) {
                        const f2d::f2 xy = f2d::bload2(f2d::rsrc(a.y + uoff, ubytes), vo, so);
                        nry[h][t] = xy[0];
                        nry[h][t + 1] = xy[1];
                    }
                }
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int so = f2d::comp_soff<CPLX, CL>(a, t) * 4;
                    nh0[h][t] = f2d::bload(r0, vo, so);
                    if constexpr (MODE != FWD) nh1[h][t] = f2d::bload(r1, vo, so);
                    // y beside dy, for D = <dy, y>
                    if constexpr (MODE == BWDQ) nry[h][t] = f2d::bload(f2d::rsrc(a.y + uoff, ubytes), vo, so);
                }
            }
        }
        if constexpr (MODE == BWDQ)
            nlse = f2d::bload(f2d::rsrc(a.lse + (int64_t)unit * a.P, a.P * 4), rpix * 4, 0);
        if constexpr (DIST && !WIDE)
            nmu = f2d::bload(f2d::rsrc(a.k + uoff, ubytes),
                             f2d::comp_off<CPLX, CL>(a, h0 + a.n1 * w0, lane & (16 * NT - 1)) * 4, 0);
    };

    int k = 0;
    int item = f2d::item_of(a, 0);
    if (item >= a.nitems) return;
    F2H_PHASE(uint64_t phase[4] = {0, 0, 0, 0};)
    unsigned *const xwords = reinterpret_cast<unsigned *>(lds + L::OX);
    if (threadIdx.x < 4) xwords[threadIdx.x] = 0u;
    if constexpr (NT == 2 || BR == 4 || ONE) {
        // slots never staged (pad rows, columns past the staged ones): zero
        // halves and scalars, so that the masked products over them stay
        // finite
        for (int i = threadIdx.x; i < G::LPX; i += G::THREADS) {
            if (i % CR < HH && i / CR < SWC) continue;
            f4 *const z0 = reinterpret_cast<f4 *>(lds + L::OT0 + i * SB);
            f4 *const z1 = reinterpret_cast<f4 *>(lds + L::OT1 + i * SB);
#pragma unroll
            for (int q = 0; q < SB / 16; ++q) z0[q] = z1[q] = f4{0.f, 0.f, 0.f, 0.f};
            if constexpr (L::NSCAL >= 1) reinterpret_cast<float *>(lds + L::OS0)[G::sidx(i % CR, i / CR)] = 0.f;
            if constexpr (L::NSCAL >= 2) reinterpret_cast<float *>(lds + L::OS1)[G::sidx(i % CR, i / CR)] = 0.f;
        }
    }
    int unit, h0, w0;
    decode(item, unit, h0, w0);
    load_stage(unit, h0, w0, std::integral_constant<int, -1>{});
    load_regs(unit, h0, w0);
    __syncthreads();  // exchange words cleared before any item's maxima

    while (true) {
        F2H_PHASE(const uint64_t pt0 = __builtin_readcyclecounter();)
        bool rvalid;
        int rpix;
        regpix(h0, w0, rvalid, rpix);
        // output channels 16 h + 4 g + r, r = 0..3, of the register pixel;
        // adjacent pairs (real and imaginary part, or channels-last) as one
        // 8-byte store
        auto put4 = [&](float *base, int h, const float (&x)[4]) {
            if constexpr (CPLX || CL) {
#pragma unroll
                for (int r = 0; r < 4; r += 2)
                    *reinterpret_cast<f2 *>(base + f2d::comp_off<CPLX, CL>(a, rpix, 16 * h + 4 * g + r)) =
                        f2{x[r], x[r + 1]};
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) base[f2d::comp_off<CPLX, CL>(a, rpix, 16 * h + 4 * g + r)] = x[r];
            }
        };
        if constexpr (WIDE) {
            // the item's rows are in LDS once every wavefront's loads are
            // (vmcnt(0): the DMA writes count as this wavefront's loads)
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            const float *const xs = reinterpret_cast<const float *>(lds + L::OXS);
            const float *const xr = reinterpret_cast<const float *>(lds + L::OXR);
            const int xp = min(px, NPX - 1) + L::XA;
#pragma unroll
            for (int c = 0; c < NCS; ++c) {
                h0v[c] = xs[(16 * hsub + c) * L::NXS + xp];
                h1v[c] = xs[(L::NCH + 16 * hsub + c) * L::NXS + xp];
            }
            // register pixels past n1 read zeros
            const int rp = G::wrow(wh) + j;
#pragma unroll
            for (int h = 0; h < NT; ++h)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int comp = 16 * h + 8 * (g & 1) + 4 * (g >> 1) + t;
                    nh0[h][t] = rvalid ? xr[comp * G::TH + rp] : 0.f;
                    if constexpr (MODE != FWD) nh1[h][t] = rvalid ? xr[(L::NCH + comp) * G::TH + rp] : 0.f;
                    if constexpr (MODE == BWDQ) nry[h][t] = rvalid ? xr[(2 * L::NCH + comp) * G::TH + rp] : 0.f;
                }
        }
        const int64_t uoff = f2d::unit_base<CL>(a, unit);
        const int64_t soff = (int64_t)unit * a.P;
        const float c2 = a.c2;

        // Distance: both sides of the score product centred on mu.  The
        // expansion -|q - k|^2 / 2 = q.k - |k|^2 / 2 - |q|^2 / 2 (key bias
        // and row term) is then formed from q - mu and k - mu, whose terms
        // scale with the spread of the data rather than its offset; |q - k|
        // and the gradient terms dS (k - q) are unchanged.
        if constexpr (DIST && WIDE) {
            // mu from the rows in LDS: k at the tile's first pixel, position
            // P + XA of the staged k rows, or position 0 of the register k
            // rows (key-centric pass)
            constexpr int MS = MODE == BWDKV ? G::TH : L::NXS;
            const float *const mu = reinterpret_cast<const float *>(lds + (MODE == BWDKV ? L::OXR : L::OXS)) +
                                    (MODE == BWDKV ? 0 : P + L::XA);
#pragma unroll
            for (int c = 0; c < NCS; ++c) h0v[c] -= mu[(16 * hsub + c) * MS];
#pragma unroll
            for (int h = 0; h < NT; ++h)
#pragma unroll
                for (int t = 0; t < 4; ++t) nh0[h][t] -= mu[(16 * h + 8 * (g & 1) + 4 * (g >> 1) + t) * MS];
        } else if constexpr (DIST) {
#pragma unroll
            for (int c = 0; c < NCS; ++c) {
                const float m0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(nmu), c));
                if constexpr (HALF) {
                    const float m1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(nmu), 16 + c));
                    h0v[c] -= hsub ? m1 : m0;
                } else {
                    h0v[c] -= m0;
                }
            }
#pragma unroll
            for (int h = 0; h < NT; ++h)
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    nh0[h][t] -= __shfl(nmu, 16 * h + 8 * (g & 1) + 4 * (g >> 1) + t);
        }

        // Largest magnitudes of what this item stages (tensors 0, 1) and, in
        // the key-centric pass, of the register v (the staged -D carries its
        // scale): a wave maximum, then one LDS atomic per wave.  Keys
        // (k << 9 | exponent) rise from item to item, so the words need no
        // clearing between items.
        {
            unsigned u0 = 0u, u1 = 0u, u2 = 0u;
            if (hslot >= 0) {
                u0 = __float_as_uint(maxabs(h0v));
                u1 = __float_as_uint(maxabs(h1v));
            }
            if constexpr (KV) {
                float m2 = maxabs(nh1[0]);
                if constexpr (NT == 2) m2 = fmaxf(m2, maxabs(nh1[1]));
                u2 = __float_as_uint(m2);
            }
            u0 = wave_umax63(u0);
            u1 = wave_umax63(u1);
            if constexpr (KV) u2 = wave_umax63(u2);
            if (lane == 63) {
                const unsigned key = (unsigned)k << 9;
                __hip_atomic_fetch_max(xwords + 0, key | (u0 >> 23), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_WORKGROUP);
                __hip_atomic_fetch_max(xwords + 1, key | (u1 >> 23), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_WORKGROUP);
                if constexpr (KV)
                    __hip_atomic_fetch_max(xwords + 2, key | (u2 >> 23), __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        }
        F2H_PHASE(const uint64_t pta = __builtin_readcyclecounter();)
        __syncthreads();  // the previous item's LDS reads are done; maxima in
        F2H_PHASE(const uint64_t ptb = __builtin_readcyclecounter(); phase[1] += ptb - pta;)
        const unsigned b0 = __builtin_amdgcn_readfirstlane(xwords[0]) & 255u;
        const unsigned b1 = __builtin_amdgcn_readfirstlane(xwords[1]) & 255u;
        const unsigned b2 = KV ? __builtin_amdgcn_readfirstlane(xwords[2]) & 255u : 127u;
        // shifts of the staged tensors (k or q; v or dy) and of the register v
        const int s0 = shift_of(b0), s1 = shift_of(b1), s2 = KV ? shift_of(b2) : 0;
        // |k - mu|^2 of the staged pixel (HALF: the two sub-pixel threads of
        // a pixel are adjacent lanes)
        float n2 = 0.f;
        if constexpr (DIST) {
#pragma unroll
            for (int c = 0; c < NCS; ++c) n2 += h0v[c] * h0v[c];
            if constexpr (HALF) n2 += __shfl_xor(n2, 1);
        }
        if (hslot >= 0) {
            char *const sl0 = lds + L::OT0 + hslot * SB;
            char *const sl1 = lds + L::OT1 + hslot * SB;
            if constexpr (HALF) {
                // this thread's sub-pixel at byte 64 hsub of the slot
                if (s0 == 0) store_slot(sl0 + 64 * hsub, h0v); else store_slot<true>(sl0 + 64 * hsub, h0v, s0);
                if (s1 == 0) store_slot(sl1 + 64 * hsub, h1v); else store_slot<true>(sl1 + 64 * hsub, h1v, s1);
            } else if constexpr (NT == 1) {
                if (s0 == 0) store_slot(sl0, h0v); else store_slot<true>(sl0, h0v, s0);
                if (s1 == 0) store_slot(sl1, h1v); else store_slot<true>(sl1, h1v, s1);
            } else {
                // sub-pixel h of the slot at byte 64 h
                float x0[2][16], x1[2][16];
#pragma unroll
                for (int c = 0; c < 32; ++c) {
                    x0[c >> 4][c & 15] = h0v[c];
                    x1[c >> 4][c & 15] = h1v[c];
                }
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    if (s0 == 0) store_slot(sl0 + 64 * h, x0[h]); else store_slot<true>(sl0 + 64 * h, x0[h], s0);
                    if (s1 == 0) store_slot(sl1 + 64 * h, x1[h]); else store_slot<true>(sl1 + 64 * h, x1[h], s1);
                }
            }
            if (hsub == 0) {
                if constexpr (KV) {
                    // staged queries: A_q = -lse log2(e) [- c2 |q|^2 / 2], and
                    // -D in the scale of the dP product
                    reinterpret_cast<float *>(lds + L::OS0)[hsid] =
                        -hs0 * kLog2e - (DIST ? 0.5f * c2 * n2 : 0.f);
                    reinterpret_cast<float *>(lds + L::OS1)[hsid] =
                        -__builtin_amdgcn_ldexpf(hs1, s1 + s2);
                } else if constexpr (DIST) {
                    reinterpret_cast<float *>(lds + L::OS0)[hsid] = -0.5f * c2 * n2;  // key bias
                }
            }
        }
        // register operands (the score product's side pre-scaled by c2):
        // channels 8 (g & 1) + t from the lower half of the wave, + 4 + t
        // from the upper half, for each sub-pixel h
        float nr0[NT][8], nr1[NT][8];
        auto join = [](const float (&h)[4], float (&x)[8]) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const unsigned u = __float_as_uint(h[t]);
                const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
                x[t] = __uint_as_float(r[0]);
                x[4 + t] = __uint_as_float(r[1]);
            }
        };
#pragma unroll
        for (int h = 0; h < NT; ++h) join(nh0[h], nr0[h]);
        // The score product's register operand absorbs the staged tensor's
        // shift (q' = q c2 2^-s0 against k' = k 2^s0), so scores keep their
        // scale.  A wave whose |q'| reaches 2^15 (the halves would overflow)
        // or, in the backward, whose scores could pass 2^20 (where the
        // recomputed probabilities exp2(s - lse) lose all precision and could
        // overflow the dS halves) takes the slow walk: q normalised per pixel
        // and each score unscaled after its product.
        const float c2s = __builtin_amdgcn_ldexpf(c2, -s0);
        float mr0 = maxabs(nr0[0]);
        if constexpr (NT == 2) mr0 = fmaxf(mr0, maxabs(nr0[1]));
        const float lim = MODE == FWD ? 32768.f
                                      : fminf(32768.f, __builtin_amdgcn_ldexpf(1.f, 16 - scaled_exp(b0)));
        const bool slow = __builtin_amdgcn_ballot_w64(!(mr0 * c2s < lim)) != 0;
        // slow walk: q c2 shifted per pixel to [4, 8), products scaled by 2^eu
        int eu = 0;
        h8 r0h[NT], r0l[NT], r1h[NT], r1l[NT];
        if (slow) {
            const int sp = min(120, max(-120, 129 - (int)bexp(gmax(mr0) * c2)));
            eu = sp + s0;
#pragma unroll
            for (int h = 0; h < NT; ++h) reg_split(nr0[h], __builtin_amdgcn_ldexpf(c2, sp), r0h[h], r0l[h]);
        } else {
#pragma unroll
            for (int h = 0; h < NT; ++h) reg_split(nr0[h], c2s, r0h[h], r0l[h]);
        }
        // dy (query-centric pass) is shifted per register pixel; v
        // (key-centric pass) by the block-wide s2
        int sd = 0;
        if constexpr (MODE != FWD) {
#pragma unroll
            for (int h = 0; h < NT; ++h) join(nh1[h], nr1[h]);
        }
        auto split_r1 = [&](float sc) {
#pragma unroll
            for (int h = 0; h < NT; ++h) reg_split(nr1[h], sc, r1h[h], r1l[h]);
        };
        if constexpr (MODE == BWDQ) {
            float mr1 = maxabs(nr1[0]);
            if constexpr (NT == 2) mr1 = fmaxf(mr1, maxabs(nr1[1]));
            sd = shift_of(bexp(gmax(mr1)));
            if (__builtin_amdgcn_ballot_w64(sd != 0) != 0)
                split_r1(__builtin_amdgcn_ldexpf(1.f, sd));
            else
                split_r1(1.f);
        } else if constexpr (MODE == BWDKV) {
            if (s2 != 0)
                split_r1(__builtin_amdgcn_ldexpf(1.f, s2));
            else
                split_r1(1.f);
        }
        // sums of the loaded halves over the four lane groups count every
        // channel once
        float raw2 = 0.f, rowD = 0.f, rowL = 0.f;
        if constexpr (DIST) {
#pragma unroll
            for (int h = 0; h < NT; ++h)
#pragma unroll
                for (int t = 0; t < 4; ++t) raw2 += nh0[h][t] * nh0[h][t];
        }
        if constexpr (MODE == BWDQ) {
            float dd = 0.f;
#pragma unroll
            for (int h = 0; h < NT; ++h)
#pragma unroll
                for (int t = 0; t < 4; ++t) dd += nh1[h][t] * nry[h][t];
            rowD = gsum(dd);
            rowL = nlse;
        }
        const float sq = DIST ? gsum(raw2) : 0.f;
        // Distance correction of the outputs needs the register pixel's
        // channels 16 h + 4 g + r (the output layout): channel 4 g + r of a
        // sub-pixel sits at index 4 (g & 1) + r in lane group
        // g' = (g >> 1) + 2 (g & 1), whose groups >= 2 offer indices 4..7 and
        // groups < 2 indices 0..3.
        float reg0[NT][4] = {};
        if constexpr (DIST && MODE != FWD) {
            const int srcl = j + 16 * ((g >> 1) | ((g & 1) << 1));
#pragma unroll
            for (int h = 0; h < NT; ++h)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    // (the two values pass through registers first: a select
                    // of two array elements would become a load at a
                    // lane-dependent index, putting nr0 in scratch memory)
                    float lo = nr0[h][r], hi = nr0[h][4 + r];
                    asm volatile("" : "+v"(lo), "+v"(hi));
                    reg0[h][r] = __shfl((g & 2) ? hi : lo, srcl);
                }
        }
        F2H_PHASE(const uint64_t ptc = __builtin_readcyclecounter();)
        __syncthreads();  // halo staged
        F2H_PHASE(const uint64_t pt1 = __builtin_readcyclecounter(); phase[2] += pt1 - ptc;
                  phase[0] += (ptc - pt0) - (ptb - pta);)

        const int nitem = f2d::item_of(a, k + 1);
        const bool has_next = nitem < a.nitems;
        // unconditional (the last item loads itself again), so that the
        // prefetch registers are dead between the staging and this point
        int xunit = unit, xh0 = h0, xw0 = w0;
        if (has_next) decode(nitem, xunit, xh0, xw0);
        auto prefetch = [&]() __attribute__((always_inline)) {
            load_stage(xunit, xh0, xw0, std::integral_constant<int, -1>{});
            load_regs(xunit, xh0, xw0);
        };
        // the same loads over three consecutive pairs from PFP: halves of the
        // staged components, then the register operands (SPREAD)
        auto prefetch_at = [&](auto PI) __attribute__((always_inline)) {
            constexpr int pi = decltype(PI)::value;
            if constexpr (!SPREAD) {
                if (pi == PFP) prefetch();
            } else {
                constexpr int p1 = PFP + 1 < NPAIR ? PFP + 1 : PFP;
                constexpr int p2 = p1 + 1 < NPAIR ? p1 + 1 : p1;
                if constexpr (pi == PFP) load_stage(xunit, xh0, xw0, std::integral_constant<int, 0>{});
                if constexpr (pi == p1) load_stage(xunit, xh0, xw0, std::integral_constant<int, 1>{});
                if constexpr (pi == p2) load_regs(xunit, xh0, xw0);
            }
        };

        // score-type product of block b (16 elements x 16 register pixels),
        // summed over the sub-pixels
        auto score = [&](auto B, const char *pA, const h8 (&rh)[NT], const h8 (&rl)[NT], f4 init) {
            constexpr int b = decltype(B)::value;
            constexpr int aoff = G::bslot(b) * SB;
#pragma unroll
            for (int h = 0; h < NT; ++h) {
                const h8 x = *reinterpret_cast<const h8 *>(pA + aoff + 64 * h);
                init = mfmah(x, rh[h], init);
                init = mfmah(x, rl[h], init);
            }
            return init;
        };
        // apply-type rows of block b: channel 16 h + j of elements 4g + t
        auto trows = [&](auto B, const char *pR, h4 (&hi)[NT], h4 (&lo)[NT]) {
            constexpr int b = decltype(B)::value;
            constexpr int boff = G::bslot(b) * SB;
#pragma unroll
            for (int h = 0; h < NT; ++h) {
                hi[h] = ldtr(pR + boff + 64 * h);
                lo[h] = ldtr(pR + boff + 64 * h + 32);
            }
        };
        // per-slot scalars of elements 4g + r of block b (4 adjacent floats)
        auto scal = [&](auto B, const float *pS) {
            constexpr int b = decltype(B)::value;
            constexpr int boff = G::sbslot(b);
            const f2 lo = *reinterpret_cast<const f2 *>(pS + boff);
            const f2 hi = *reinterpret_cast<const f2 *>(pS + boff + 2);
            return f4{lo[0], lo[1], hi[0], hi[1]};
        };

        if constexpr (MODE == FWD) {
            float m = 0.f, lsum = 0.f;
            f4 acc[NT];
#pragma unroll
            for (int h = 0; h < NT; ++h) acc[h] = f4{0.f, 0.f, 0.f, 0.f};
            // LDS operands of a pair: score rows of its two blocks, apply rows
            // (values), and the Distance key biases
            struct POps {
                h8 a[2][NT];
                h4 vh[2][NT], vl[2][NT];
                f4 kb[2];
            };
            auto load_a = [&](auto PI, POps &o) {
                constexpr int pi = decltype(PI)::value;
                constexpr int b0 = 2 * pi;
                constexpr int b1 = b0 + 1 < NBLK ? b0 + 1 : b0;
                constexpr int a0 = G::bslot(b0) * SB;
                constexpr int a1 = G::bslot(b1) * SB;
#pragma unroll
                for (int h = 0; h < NT; ++h) o.a[0][h] = *reinterpret_cast<const h8 *>(pA0 + a0 + 64 * h);
#pragma unroll
                for (int h = 0; h < NT; ++h) o.a[1][h] = *reinterpret_cast<const h8 *>(pA0 + a1 + 64 * h);
                if constexpr (DIST) {
                    o.kb[0] = scal(std::integral_constant<int, b0>{}, pS0);
                    o.kb[1] = scal(std::integral_constant<int, b1>{}, pS0);
                }
            };
            auto load_v = [&](auto PI, POps &o) {
                constexpr int pi = decltype(PI)::value;
                constexpr int b0 = 2 * pi;
                constexpr int b1 = b0 + 1 < NBLK ? b0 + 1 : b0;
                trows(std::integral_constant<int, b0>{}, pR1, o.vh[0], o.vl[0]);
                trows(std::integral_constant<int, b1>{}, pR1, o.vh[1], o.vl[1]);
            };
            auto load_ops = [&](auto PI) {
                POps o;
                load_a(PI, o);
                load_v(PI, o);
                return o;
            };
            // scores of the pair's blocks relative to m, masked to -inf outside
            // the window (dep: a per-walk value for the lane masks, so that
            // walks do not share, and keep live, each other's masks)
            // (SLOW: the product of the per-pixel normalised q is unscaled by
            // 2^-eu and the row terms are added after it)
            auto scores_ops = [&](auto PI, auto REL, const POps &o, f4 (&sv)[2], int dep,
                                  auto SLOW) {
                constexpr int pi = decltype(PI)::value;
                constexpr bool rel = decltype(REL)::value;
                constexpr bool slw = decltype(SLOW)::value;
                constexpr int b0 = 2 * pi;
                constexpr bool has1 = b0 + 1 < NBLK;
                auto sc = [&](auto B, int u) {
                    constexpr int b = decltype(B)::value;
                    constexpr int bi = b / NKW, bj = b % NKW;
                    f4 x;
                    if constexpr (slw) {
                        // the relative score is the maximised value minus m,
                        // rounded as in the pass that took the maximum
                        f4 z = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int h = 0; h < NT; ++h) {
                            z = mfmah(o.a[u][h], r0h[h], z);
                            z = mfmah(o.a[u][h], r0l[h], z);
                        }
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            x[r] = __builtin_amdgcn_ldexpf(z[r], -eu);
                            if constexpr (DIST) x[r] += o.kb[u][r];
                            if constexpr (rel) x[r] -= m;
                        }
                    } else {
                        f4 init = f4{0.f, 0.f, 0.f, 0.f};
                        if constexpr (DIST) init = o.kb[u];
                        if constexpr (rel) init = init - f4{m, m, m, m};
#pragma unroll
                        for (int h = 0; h < NT; ++h) {
                            init = mfmah(o.a[u][h], r0h[h], init);
                            init = mfmah(o.a[u][h], r0l[h], init);
                        }
                        x = init;
                    }
                    x[0] = mask_sel_d<hmask<BR>(P, bi, bj, 0)>(x[0], -INFINITY, dep);
                    x[1] = mask_sel_d<hmask<BR>(P, bi, bj, 1)>(x[1], -INFINITY, dep);
                    x[2] = mask_sel_d<hmask<BR>(P, bi, bj, 2)>(x[2], -INFINITY, dep);
                    x[3] = mask_sel_d<hmask<BR>(P, bi, bj, 3)>(x[3], -INFINITY, dep);
                    sv[u] = x;
                };
                sc(std::integral_constant<int, b0>{}, 0);
                if constexpr (has1) {
                    sc(std::integral_constant<int, b0 + 1>{}, 1);
                } else {
                    sv[1] = f4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
                }
            };
            auto pair_max = [](const f4 (&sv)[2]) {
                const float a0 = fmaxf(fmaxf(sv[0][0], sv[0][1]), sv[0][2]);
                const float a1 = fmaxf(fmaxf(sv[0][3], sv[1][0]), sv[1][1]);
                return fmaxf(fmaxf(a0, a1), fmaxf(sv[1][2], sv[1][3]));
            };
            // probabilities exp2(sv) of a pair into the sums and the output
            auto apply_ops = [&](const POps &o, const f4 (&sv)[2]) {
                float p[2][4];
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int r = 0; r < 4; ++r) p[u][r] = __builtin_amdgcn_exp2f(sv[u][r]);
                const float ps = ((p[0][0] + p[0][1]) + (p[0][2] + p[0][3])) +
                                 ((p[1][0] + p[1][1]) + (p[1][2] + p[1][3]));
                lsum += ps;
                h4 ph0, pl0, ph1, pl1;
                split4(p[0], ph0, pl0);
                split4(p[1], ph1, pl1);
                const h8 ph = cat(ph0, ph1), pl = cat(pl0, pl1);
#pragma unroll
                for (int h = 0; h < NT; ++h) {
                    const h8 vh = cat(o.vh[0][h], o.vh[1][h]), vl = cat(o.vl[0][h], o.vl[1][h]);
                    acc[h] = mfmah(vh, ph, acc[h]);
                    acc[h] = mfmah(vh, pl, acc[h]);
                    acc[h] = mfmah(vl, ph, acc[h]);
                }
                return ps;
            };
            auto scores = [&](auto PI, auto REL, f4 (&sv)[2], int dep, auto SLOW) {
                scores_ops(PI, REL, load_ops(PI), sv, dep, SLOW);
            };
            auto apply = [&](auto PI, const f4 (&sv)[2]) { return apply_ops(load_ops(PI), sv); };
            // Scores relative to a reference maximum m, folded into the MFMA's
            // initial accumulator.  The first walk takes m from the central
            // pair PC (it holds a key of every query's window, so m is
            // finite) and has no branch;
            // if a pair's probabilities sum past 2^8 in some lane (a score
            // more than 8 above m, in log2 units, where the halves could
            // overflow), the item is redone with m the exact row maximum from
            // a scores-only pass.  On typical data the redo never runs.
            constexpr int PC = STREAM ? G::PCENT : 0;
            uint64_t over = 1;
            // streamed configurations issue the next item's loads before the
            // walk, on both of its paths alike (loads issued inside each path
            // make the compiler copy the 36 prefetch registers at the merge)
            if constexpr (STREAM) prefetch();
            if constexpr (STREAM) {
              if (!slow) {
                // Walk order: PC, then the other pairs.  Skewed by one pair:
                // an iteration takes the scores of the next pair (MFMA) beside
                // the softmax of the current one (vector ALU), so that the two
                // units have independent work; the score rows of the pair
                // after next and the value rows of the next pair are read from
                // LDS one iteration ahead.
                constexpr auto ord = [](int i) { return i == 0 ? PC : (i - 1 < PC ? i - 1 : i); };
                f4 sv[2];
                POps ca, cv;  // score rows of the next pair, value rows of the current
                load_a(std::integral_constant<int, PC>{}, ca);
                load_v(std::integral_constant<int, PC>{}, cv);
                scores_ops(std::integral_constant<int, PC>{}, std::false_type{}, ca, sv, k,
                           std::false_type{});
                m = gmax(pair_max(sv));
                sv[0] = sv[0] - f4{m, m, m, m};
                sv[1] = sv[1] - f4{m, m, m, m};
                load_a(std::integral_constant<int, ord(1)>{}, ca);
                over = 0;
                static_for<0, NPAIR>([&](auto I) {
                    constexpr int i = decltype(I)::value;
                    FWD_FENCE_A();
                    walk_prio<i, NPAIR>();
                    POps na, nv;
                    if constexpr (i + 2 < NPAIR) load_a(std::integral_constant<int, ord(i + 2)>{}, na);
                    if constexpr (i + 1 < NPAIR) load_v(std::integral_constant<int, ord(i + 1)>{}, nv);
                    f4 svn[2];
                    if constexpr (i + 1 < NPAIR)
                        scores_ops(std::integral_constant<int, ord(i + 1)>{}, std::true_type{}, ca, svn, k,
                                   std::false_type{});
                    const float ps = apply_ops(cv, sv);
                    if constexpr (i > 0) over |= __builtin_amdgcn_ballot_w64(!(ps <= 256.f));
                    if constexpr (i + 1 < NPAIR) {
                        sv[0] = svn[0];
                        sv[1] = svn[1];
                        cv = nv;
                    }
                    if constexpr (i + 2 < NPAIR) ca = na;
#if CIRCATT_F2H_SGB
                    // issue order: LDS reads, then MFMAs one at a time with
                    // vector instructions between them
                    __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
                    static_for<0, 7>([&](auto) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, CIRCATT_F2H_SGB, 0);
                    });
#endif
                });
              }
            }
            // exact row maximum, then one walk with every score <= m (the slow
            // walk always takes this form)
            auto twopass = [&](auto SLOW) {
                float mx = -INFINITY;
                static_for<0, NPAIR>([&](auto PI) {
                    FWD_FENCE_A();
                    if constexpr (!STREAM && decltype(PI)::value == PFP) prefetch();
                    f4 sv[2];
                    scores(PI, std::false_type{}, sv, k + 1, SLOW);
                    mx = fmaxf(mx, pair_max(sv));
                });
                m = gmax(mx);
                lsum = 0.f;
#pragma unroll
                for (int h = 0; h < NT; ++h) acc[h] = f4{0.f, 0.f, 0.f, 0.f};
                static_for<0, NPAIR>([&](auto PI) {
                    FWD_FENCE_A();
                    f4 sv[2];
                    scores(PI, std::true_type{}, sv, k + 2, SLOW);
                    apply(PI, sv);
                });
            };
            if (slow) {
                twopass(std::true_type{});
            } else if (over != 0) {
                twopass(std::false_type{});
            }
            // l >= 1 (the element at m contributes exp2(0)); v_rcp_f32 is
            // within 1 ulp, where an IEEE division would add a dozen vector
            // instructions per item
            const float l = gsum(lsum);
            const float inv = __builtin_amdgcn_rcpf(l);
            if (rvalid) {
                float *yb = a.yout + uoff;
#pragma unroll
                for (int h = 0; h < NT; ++h) {
                    float x[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) x[r] = __builtin_amdgcn_ldexpf(acc[h][r] * inv, -s1);
                    put4(yb, h, x);
                }
                if (g == 0)
                    a.lse_out[soff + rpix] =
                        (m + __log2f(l)) * kLn2 - (DIST ? 0.5f * sq * a.scale : 0.f);
            }
        } else {
            // BWDQ: score row term -lse log2(e) [- c2 |q|^2 / 2], dP row term
            // -D in the scale of the dP product (2^(sd + s1): dy' against v')
            const float nl = -rowL * kLog2e - (DIST ? 0.5f * c2 * sq : 0.f);
            const float nD = -__builtin_amdgcn_ldexpf(rowD, sd + s1);
            const float kb = DIST ? -0.5f * c2 * sq : 0.f;  // BWDKV key bias
            f4 acc0[NT], acc1[NT];  // dQ (BWDQ) or dK (BWDKV); dV (BWDKV)
#pragma unroll
            for (int h = 0; h < NT; ++h) acc0[h] = acc1[h] = f4{0.f, 0.f, 0.f, 0.f};
            float corr = 0.f;
            // SLOW: scores of the per-pixel normalised register operand,
            // unscaled by 2^-eu after the product, the row terms added, and
            // clamped at 0 (a probability recomputed from lse is at most 1)
            auto walk = [&](auto SLOW) {
            constexpr bool slw = decltype(SLOW)::value;
            static_for<0, NPAIR>([&](auto PI) {
                constexpr int pi = decltype(PI)::value;
                constexpr int b0 = 2 * pi;
                constexpr bool has1 = b0 + 1 < NBLK;
                constexpr int b1 = has1 ? b0 + 1 : b0;
                if constexpr (pi % CIRCATT_F2H_BWD_FSTEP == 0) BLOCK_FENCE();
                if constexpr (MODE == BWDQ) walk_prio<pi, NPAIR>();
                if constexpr (MODE == BWDKV) walk_prio_tail<pi, NPAIR>();
                prefetch_at(PI);
                float p[2][4], ds[2][4];
                auto blk = [&](auto B, int u) {
                    constexpr int b = decltype(B)::value;
                    constexpr int bi = b / NKW, bj = b % NKW;
                    f4 s, dp;
                    if constexpr (KV) {
                        s = scal(B, pS0);
                        if constexpr (DIST) s = s + f4{kb, kb, kb, kb};
                        dp = scal(B, pS1);
                    } else {
                        s = f4{nl, nl, nl, nl};
                        if constexpr (DIST) s = s + scal(B, pS0);
                        dp = f4{nD, nD, nD, nD};
                    }
                    if constexpr (slw) {
                        const f4 z = score(B, pA0, r0h, r0l, f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            s[r] = fminf(__builtin_amdgcn_ldexpf(z[r], -eu) + s[r], 0.f);
                    } else {
                        s = score(B, pA0, r0h, r0l, s);
                    }
                    dp = score(B, pA1, r1h, r1l, dp);
                    p[u][0] = mask_sel_d<hmask<BR>(P, bi, bj, 0)>(__builtin_amdgcn_exp2f(s[0]), 0.f, k);
                    p[u][1] = mask_sel_d<hmask<BR>(P, bi, bj, 1)>(__builtin_amdgcn_exp2f(s[1]), 0.f, k);
                    p[u][2] = mask_sel_d<hmask<BR>(P, bi, bj, 2)>(__builtin_amdgcn_exp2f(s[2]), 0.f, k);
                    p[u][3] = mask_sel_d<hmask<BR>(P, bi, bj, 3)>(__builtin_amdgcn_exp2f(s[3]), 0.f, k);
#pragma unroll
                    for (int r = 0; r < 4; ++r) ds[u][r] = p[u][r] * dp[r];
                    if constexpr (DIST) corr += (ds[u][0] + ds[u][1]) + (ds[u][2] + ds[u][3]);
                };
                blk(std::integral_constant<int, b0>{}, 0);
                if constexpr (has1) {
                    blk(std::integral_constant<int, b1>{}, 1);
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) p[1][r] = ds[1][r] = 0.f;
                }
                h4 dh0, dl0, dh1, dl1;
                split4(ds[0], dh0, dl0);
                split4(ds[1], dh1, dl1);
                const h8 dsh = cat(dh0, dh1), dsl = cat(dl0, dl1);
                h4 t0h[NT], t0l[NT], t1h[NT], t1l[NT];
                trows(std::integral_constant<int, b0>{}, pR0, t0h, t0l);
                trows(std::integral_constant<int, b1>{}, pR0, t1h, t1l);
#pragma unroll
                for (int h = 0; h < NT; ++h) {
                    const h8 yh = cat(t0h[h], t1h[h]), yl = cat(t0l[h], t1l[h]);
                    acc0[h] = mfmah(yh, dsh, acc0[h]);
                    acc0[h] = mfmah(yl, dsh, acc0[h]);
                    acc0[h] = mfmah(yh, dsl, acc0[h]);
                }
                if constexpr (KV) {
                    h4 ph0, pl0, ph1, pl1;
                    split4(p[0], ph0, pl0);
                    split4(p[1], ph1, pl1);
                    const h8 ph = cat(ph0, ph1), pl = cat(pl0, pl1);
                    trows(std::integral_constant<int, b0>{}, pR1, t0h, t0l);
                    trows(std::integral_constant<int, b1>{}, pR1, t1h, t1l);
#pragma unroll
                    for (int h = 0; h < NT; ++h) {
                        const h8 zh = cat(t0h[h], t1h[h]), zl = cat(t0l[h], t1l[h]);
                        acc1[h] = mfmah(zh, ph, acc1[h]);
                        acc1[h] = mfmah(zl, ph, acc1[h]);
                        acc1[h] = mfmah(zh, pl, acc1[h]);
                    }
                }
            });
            };
            if (slow) {
                walk(std::true_type{});
            } else {
                walk(std::false_type{});
            }
            const float cs = DIST ? gsum(corr) : 0.f;
            if (rvalid) {
                if constexpr (!KV) {
                    float *ob = a.dq + uoff;
#pragma unroll
                    for (int h = 0; h < NT; ++h) {
                        float x[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            // dS' = 2^(sd + s1) dS, k' = 2^s0 k
                            float val = __builtin_amdgcn_ldexpf(acc0[h][r], -(sd + s1 + s0));
                            if constexpr (DIST) val -= __builtin_amdgcn_ldexpf(cs, -(sd + s1)) * reg0[h][r];
                            x[r] = val * a.scale;
                        }
                        put4(ob, h, x);
                    }
                    if (g == 0) a.dbuf[soff + rpix] = rowD;
                } else {
                    float *vb = a.dv + uoff;
                    float *kbp = a.dk + uoff;
#pragma unroll
                    for (int h = 0; h < NT; ++h) {
                        float xv[4], xk[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            // dy' = 2^s1 dy, dS' = 2^(s2 + s1) dS, q' = 2^s0 q
                            xv[r] = __builtin_amdgcn_ldexpf(acc1[h][r], -s1);
                            float val = __builtin_amdgcn_ldexpf(acc0[h][r], -(s2 + s1 + s0));
                            if constexpr (DIST) val -= __builtin_amdgcn_ldexpf(cs, -(s2 + s1)) * reg0[h][r];
                            xk[r] = val * a.scale;
                        }
                        put4(vb, h, xv);
                        put4(kbp, h, xk);
                    }
                }
            }
        }

        F2H_PHASE(phase[3] += __builtin_readcyclecounter() - pt1;)
        if (!has_next) break;
        ++k;
        item = nitem;
        unit = xunit;
        h0 = xh0;
        w0 = xw0;
    }
#if CIRCATT_F2H_PHASE
    if (blockIdx.x < 8 && lane == 0 && a.phase) {
        float *o = a.phase + 4 * (16 * blockIdx.x + wv);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = __uint_as_float((unsigned)phase[i]);
    }
#endif
}

template <int P, int NT, bool CPLX, bool DIST, int MODE, bool CL, bool ONE = false, bool WIDE = false>
hipError_t launch2h(const Args &a0, int cus, hipStream_t s) {
    using G = HGeo<P, NT, ONE>;
    static_assert(ONE || (G::TH == f2d::Geo<P, 1, grid_wh<NT>(), 8>::TH &&
                          G::TW == f2d::Geo<P, 1, grid_wh<NT>(), 8>::TW),
                  "2D tiles as the Float32 kernels'");
    constexpr int bytes = LGeo<P, NT, MODE, DIST, ONE, WIDE>::bytes;
    static_assert(bytes <= (int)f2d::kLdsCap, "halo does not fit LDS");
    auto kern = kernel2h<P, NT, CPLX, DIST, MODE, CL, ONE, WIDE>;
    // set once per instantiation (a function-local static is initialised
    // exactly once, also when several host threads launch at the same time)
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (attr != hipSuccess) return attr;
    Args a = a0;
    F2H_PHASE(a.phase = phase_buffer();)
    a.tiles_h = (a.n1 + G::TH - 1) / G::TH;
    a.tiles_w = (a.n2 + G::TW - 1) / G::TW;
    const int64_t nitems = (int64_t)a.tiles_h * a.tiles_w * a.nunits;
    if (nitems <= 0 || nitems > INT32_MAX / 2) return hipErrorNotSupported;
    a.div_tiles = make_fastdiv((uint32_t)(a.tiles_h * a.tiles_w));
    a.div_th = make_fastdiv((uint32_t)a.tiles_h);
    if (CL) a.div_nh = make_fastdiv((uint32_t)a.nheads);
    a.nitems = (int)nitems;
    a.per_xcd = (int)((nitems + 7) / 8);
    int64_t grid = std::min<int64_t>(cus, 8LL * a.per_xcd);
    grid = std::max<int64_t>(8, grid / 8 * 8);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(G::THREADS), bytes, s, a);
    return hipGetLastError();
}

// NT = 1 covers windows 3, 5, 7, 11 and 15; NT = 2 (32 real components per
// head) windows up to 11, beyond which its halo would not fit LDS
template <int MODE, int NT>
hipError_t dispatch(int p, bool cplx, bool dist, const Args &a, int cus, hipStream_t s) {
#define CIRCATT_F2H_CL(PP, CLL)                                                          \
    {                                                                                    \
        if (cplx) return dist ? launch2h<PP, NT, true, true, MODE, CLL>(a, cus, s)         \
                              : launch2h<PP, NT, true, false, MODE, CLL>(a, cus, s);       \
        return dist ? launch2h<PP, NT, false, true, MODE, CLL>(a, cus, s)                  \
                    : launch2h<PP, NT, false, false, MODE, CLL>(a, cus, s);                \
    }
#define CIRCATT_F2H_CASE(PP)                                                             \
    if (p == PP) {                                                                       \
        if (a.cl) CIRCATT_F2H_CL(PP, true)                                               \
        CIRCATT_F2H_CL(PP, false)                                                        \
    }
    CIRCATT_F2H_CASE(1)
    CIRCATT_F2H_CASE(2)
    CIRCATT_F2H_CASE(3)
    CIRCATT_F2H_CASE(5)
    if constexpr (NT == 1) CIRCATT_F2H_CASE(7)
#undef CIRCATT_F2H_CASE
#undef CIRCATT_F2H_CL
    return hipErrorNotSupported;
}

// Planar real signals whose length is a multiple of 4, on 16-byte aligned
// tensors: staged and register rows loaded by 16-byte DMA into LDS
inline bool wide_rows(const Args &a, bool cplx) {
    if (cplx || a.cl || a.n1 % 4 != 0) return false;
    uintptr_t bits = 0;
    for (const float *p : {a.q, a.k, a.v, a.dy, a.y}) bits |= reinterpret_cast<uintptr_t>(p);
    return (bits & 15) == 0;
}

// One-dimensional signals: windows 15 and 63, 16 or 32 real components per
// head (the run-time-window kernel covers the others)
template <int MODE, int NT>
hipError_t dispatch1(int p, bool cplx, bool dist, const Args &a, int cus, hipStream_t s) {
#define CIRCATT_F1H_CL(PP, CLL)                                                          \
    {                                                                                    \
        if (!CLL && wide_rows(a, cplx))                                                 \
            return dist ? launch2h<PP, NT, false, true, MODE, false, true, true>(a, cus, s) \
                        : launch2h<PP, NT, false, false, MODE, false, true, true>(a, cus, s); \
        if (cplx) return dist ? launch2h<PP, NT, true, true, MODE, CLL, true>(a, cus, s)   \
                              : launch2h<PP, NT, true, false, MODE, CLL, true>(a, cus, s); \
        return dist ? launch2h<PP, NT, false, true, MODE, CLL, true>(a, cus, s)            \
                    : launch2h<PP, NT, false, false, MODE, CLL, true>(a, cus, s);          \
    }
#define CIRCATT_F1H_CASE(PP)                                                             \
    if (p == PP) {                                                                       \
        if (a.cl) CIRCATT_F1H_CL(PP, true)                                               \
        CIRCATT_F1H_CL(PP, false)                                                        \
    }
    CIRCATT_F1H_CASE(7)
    CIRCATT_F1H_CASE(31)
#undef CIRCATT_F1H_CASE
#undef CIRCATT_F1H_CL
    return hipErrorNotSupported;
}
inline bool supported1(int p, int ncr) { return (p == 7 || p == 31) && (ncr == 16 || ncr == 32); }

}  // namespace f2h

// 16 real components per head (fused2h_*.hip) and 32 (fused2h2_*.hip)
hipError_t launch_f2h_fwd(int p, bool cplx, bool dist, const f2d::Args &a, int cus, hipStream_t s);
hipError_t launch_f2h_bwdq(int p, bool cplx, bool dist, const f2d::Args &a, int cus, hipStream_t s);
hipError_t launch_f2h_bwdkv(int p, bool cplx, bool dist, const f2d::Args &a, int cus, hipStream_t s);
hipError_t launch_f2h2_fwd(int p, bool cplx, bool dist, const f2d::Args &a, int cus, hipStream_t s);
hipError_t launch_f2h2_bwdq(int p, bool cplx, bool dist, const f2d::Args &a, int cus, hipStream_t s);
hipError_t launch_f2h2_bwdkv(int p, bool cplx, bool dist, const f2d::Args &a, int cus, hipStream_t s);
// one-dimensional signals (fused1h_*.hip: 16 real components per head,
// fused1h2_*.hip: 32)
hipError_t launch_f1h_fwd(int p, bool cplx, bool dist, const f2d::Args &a, int cus, hipStream_t s);
hipError_t launch_f1h_bwdq(int p, bool cplx, bool dist, const f2d::Args &a, int cus, hipStream_t s);
hipError_t launch_f1h_bwdkv(int p, bool cplx, bool dist, const f2d::Args &a, int cus, hipStream_t s);
hipError_t launch_f1h2_fwd(int p, bool cplx, bool dist, const f2d::Args &a, int cus, hipStream_t s);
hipError_t launch_f1h2_bwdq(int p, bool cplx, bool dist, const f2d::Args &a, int cus, hipStream_t s);
hipError_t launch_f1h2_bwdkv(int p, bool cplx, bool dist, const f2d::Args &a, int cus, hipStream_t s);

}  // namespace circatt
