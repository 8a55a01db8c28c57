// Windowed-tile MFMA kernels for circulant attention on gfx950.
//
// One kernel template serves four modes (circatt_kernels.h, FusedMode):
//   FWD   : flash forward, y = softmax(scale*S) ⊗ v and lse, A never formed
//   SIM   : scale*S written into nzVal in the reference's CSR slot order
//   BWDQ  : query-centric backward, dq and D = <dy, y>
//   BWDKV : key-centric backward, dk and dv (no atomics: the window is
//           symmetric, so key c's contributing queries are exactly the
//           pixels at offsets [-p, p] from c)
//
// Work decomposition.  Work items are (tile, unit) pairs: a tile of "register
// pixels" (queries, or keys in BWDKV) of one (head, batch) unit.  Workgroups
// (4 wavefronts) are persistent: each walks its own run of items, and the
// runs of the workgroups resident on one XCD are adjacent tiles, so halo
// re-reads hit that XCD's L2.  For each item the circularly wrapped halo of
// the other side (K/V, or Q/dY) is staged in LDS, row chunk by row chunk; the
// global loads of the next chunk (or item) are issued into registers before
// the current chunk is computed, which hides their latency.
//
// Each wavefront holds a block of 16 register pixels and walks blocks of 16
// LDS pixels covering its window, two blocks at a time (independent MFMA
// chains), with v_mfma_f32_16x16x4f32 for every contraction:
//   S^T[key][q]   = sum_c K[key][c] Q[q][c]     A = K (LDS),  B = Q (regs)
//   y^T[c][q]    += sum_k V[k][c] P^T[k][q]     A = V (LDS),  B = P (regs)
// The S^T accumulator layout (lane j+16g, item r = key 4g+r, query j) is
// exactly the B-operand layout of the next product, so probabilities never
// leave registers.  Pairs outside the window are masked to zero weight; with
// 2D register blocks 8x2 and LDS blocks 2x8 the dense 16x16 products are
// 64% useful at ws = 15 (1D: 16-pixel runs).
//
// On gfx950 VALU work does not overlap MFMA work of the same SIMD, so the
// kernel minimises VALU instructions per MFMA: the windows of the benchmark
// configurations are compiled with their geometry as constants (block walk
// fully unrolled, LDS addresses as immediate offsets, window masks as lane
// masks shared across blocks), the scale folds into one FMA before each
// exp2, and the forward's online softmax rescales only when a row maximum
// grows by more than 2^8.  Other windows use the same code with run-time
// geometry.
//
// Layouts.  Global signals are the reference's planar (P, C) per unit
// (complex: interleaved pairs, treated as 2 real components per channel).
// LDS holds [pixel][component] rows padded to NC+4 floats so that both the
// 4-wide row reads (ds_read_b128) and the transposed single reads are free of
// bank conflicts.
#pragma once
#include <algorithm>

#include "circatt_common.h"
#include "circatt_kernels.h"

extern __shared__ __attribute__((aligned(16))) float circatt_lds[];

namespace circatt {

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma4(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescaleLog2 = 8.f;  // forward: rescale when a max grows by > 2^8

// Block geometry.  Register block: lane j -> (j % QH, j / QH).  LDS block:
// element kk -> (kk % KH, kk / KH).  Workgroup tile TH x TW.
template <int NSP>
struct FGeo;
template <>
struct FGeo<2> {
    static constexpr int QH = 8, QW = 2, KH = 2, KW = 8, TH = 8, TW = 8;
    __device__ static int wave_h(int) { return 0; }
    __device__ static int wave_w(int wv) { return 2 * wv; }
};
template <>
struct FGeo<1> {
    static constexpr int QH = 16, QW = 1, KH = 16, KW = 1, TH = 64, TW = 1;
    __device__ static int wave_h(int wv) { return 16 * wv; }
    __device__ static int wave_w(int) { return 0; }
};

constexpr size_t kLdsBudget = 80 * 1024;  // two workgroups per CU

// Halo / chunk geometry of one launch.  Computed on the host for every launch
// and, for the compiled-in windows, at compile time inside the kernel.
struct HaloGeo {
    int p1, p2;          // half windows along dims 1 and 2 (p2 = 0 in 1D)
    int nkh, nkw;        // LDS blocks per wavefront along dims 1 and 2
    int halo_h, halo_w;  // staged halo box: rows along dim 1, columns along dim 2
    int chunk_rows, cr;  // halo rows per LDS chunk, LDS row stride in pixels
    int nchunks;
    int lds_floats;      // per chunk
    bool ok;
};

// ntensor staged [pixel][NC+4] tensors and nscalar staged per-pixel scalars;
// ppt halo pixels per thread and stage (register staging capacity); extra
// floats after them (the Distance centre).
__host__ __device__ constexpr HaloGeo plan_halo(int nsp, int p, int nc, int ntensor,
                                                int nscalar, int ppt, int extra = 0) {
    HaloGeo h{};
    const int PS = nc + 4;
    const int bpp = ntensor * PS + nscalar;  // floats per staged pixel
    const int cap_px = 256 * ppt;
    if (nsp == 2) {
        h.p1 = h.p2 = p;
        h.nkh = (8 + 2 * p + 1) / 2;
        h.nkw = (2 + 2 * p + 7) / 8;
        h.halo_h = 2 * h.nkh;
        h.halo_w = 6 + 8 * h.nkw;
        // largest even chunk whose padded stride (cr % 4 == 2) fits
        int rows = h.halo_h;
        int cr = 0;
        for (; rows >= 2; rows -= 2) {
            cr = rows + ((2 - rows % 4) + 4) % 4;
            if ((size_t)(cr * h.halo_w * bpp + extra) * 4 <= kLdsBudget && rows * h.halo_w <= cap_px) break;
        }
        if (rows < 2) return h;
        h.chunk_rows = rows;
        h.cr = cr;
    } else {
        h.p1 = p;
        h.p2 = 0;
        h.nkh = (16 + 2 * p + 15) / 16;
        h.nkw = 1;
        h.halo_h = 48 + 16 * h.nkh;
        h.halo_w = 1;
        int rows = h.halo_h;  // chunks are whole 16-row LDS blocks
        for (; rows >= 16; rows -= 16)
            if ((size_t)(rows * bpp + extra) * 4 <= kLdsBudget && rows <= cap_px) break;
        if (rows < 16) return h;
        h.chunk_rows = rows;
        h.cr = rows;
    }
    h.nchunks = (h.halo_h + h.chunk_rows - 1) / h.chunk_rows;
    h.lds_floats = h.cr * h.halo_w * bpp + extra;
    h.ok = true;
    return h;
}

struct FArgs {
    const float *q, *k, *v, *y, *dy, *lse;
    float *yout, *lse_out, *dq, *dk, *dv, *dbuf, *nz;
    Geom g;
    HaloGeo hg;
    int dh, ncomp, ncr;   // channels per unit, components per channel, dh*ncomp
    int64_t unit_stride;  // floats per unit (P*dh*ncomp)
    float scale, c2;      // similarity scale and scale*log2(e)
    int tiles_h, tiles_w;
    int nitems;           // tiles * units
    int per_xcd;          // items per XCD run
    // channels-last tensors (C, spatial..., B): cl = 1, nheads heads per
    // image, ncrall = floats per pixel (C * components); planar when cl = 0
    int cl, nheads, ncrall;
    // channel-chunked kernels (fused_wide_impl.h): block rows per stage, LDS
    // column stride, stages per pass, score chunks, output passes
    int rb, cr, nst, ncc, noc;
};

template <int NC, int MODE, bool DIST>
struct Cfg {
    static constexpr int PS = NC + 4;
    static constexpr int NT = NC / 16;  // 16-component tiles
    static constexpr int NS = NC / 4;   // MFMA k-steps
    static constexpr int NTEN = MODE == MODE_SIM ? 1 : 2;      // staged tensors
    static constexpr int NSCAL = MODE == MODE_BWDKV ? 2 : 0;   // staged scalars (lse, D)
    static constexpr bool BIAS = DIST && MODE != MODE_BWDKV;   // per-pixel -|k|^2/2
    static constexpr int NLDS_SCAL = NSCAL + (BIAS ? 1 : 0);   // LDS scalars per pixel
    static constexpr int PPT = NC * NTEN <= 32 ? 2 : 1;        // halo pixels per thread
};

// Layout of q, k, v, y, dy and the gradients.  Planar (the reference's
// column-major (spatial..., C, B)): unit u = (batch, head) starts at float
// u * P * ncr and real component comp of pixel pix sits at pix + P comp
// (complex: 2 (pix + P (comp >> 1)) + (comp & 1)).  Channels-last
// ((C, spatial..., B)): unit (b, h) starts at b * P * ncrall + h * ncr, and
// the component at pix * ncrall + comp.
__device__ __forceinline__ int64_t unit_base(const FArgs &a, int unit) {
    if (a.cl) {
        const int b = unit / a.nheads;
        return (int64_t)b * a.g.P * a.ncrall + (int64_t)(unit - b * a.nheads) * a.ncr;
    }
    return (int64_t)unit * a.unit_stride;
}
__device__ __forceinline__ int64_t comp_index(const FArgs &a, int64_t pix, int comp) {
    if (a.cl) return pix * a.ncrall + comp;
    if (a.ncomp == 1) return pix + a.g.P * comp;
    return 2 * (pix + a.g.P * (comp >> 1)) + (comp & 1);
}

// All NC components of one pixel (padded components re-read the last real
// channel and are zeroed by a select, so no load is predicated).
template <int NC>
__device__ __forceinline__ void load_pixel(float (&v)[NC], const float *base, const FArgs &a,
                                           int64_t gp) {
    const int64_t P = a.g.P;
    const bool full = a.ncr == NC;
    if (a.cl) {
        const float *src = base + gp * a.ncrall;
#pragma unroll
        for (int c = 0; c < NC; ++c) v[c] = src[full ? c : min(c, a.ncr - 1)];
    } else if (a.ncomp == 1) {
        const float *src = base + gp;
#pragma unroll
        for (int c = 0; c < NC; ++c) v[c] = src[(int64_t)(full ? c : min(c, a.dh - 1)) * P];
    } else {
        const float2 *src = reinterpret_cast<const float2 *>(base) + gp;
#pragma unroll
        for (int c = 0; c < NC / 2; ++c) {
            const float2 x = src[(int64_t)(full ? c : min(c, a.dh - 1)) * P];
            v[2 * c] = x.x;
            v[2 * c + 1] = x.y;
        }
    }
    if (!full) {
#pragma unroll
        for (int c = 0; c < NC; ++c) v[c] = c < a.ncr ? v[c] : 0.f;
    }
}

// Reductions over the four lane groups (rows of 16) that hold the same
// register-block pixel: lanes j, j^16, j^32, j^48.  v_permlane16_swap and
// v_permlane32_swap (gfx950) exchange rows inside the VALU.
__device__ __forceinline__ float xsum16_32(float v) {
    unsigned u = __float_as_uint(v);
    auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    v = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    u = __float_as_uint(v);
    auto r32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}
__device__ __forceinline__ float xmax16_32(float v) {
    unsigned u = __float_as_uint(v);
    auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    v = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
    u = __float_as_uint(v);
    auto r32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}

// First products of a block: rows = the 16 LDS pixels (A operand, 4-wide row
// reads at LDS float offset `off`), columns = the 16 register pixels (B).
template <int NT>
__device__ __forceinline__ f4 block_product(int off, const float *reg) {
    f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const f4 x = *reinterpret_cast<const f4 *>(&circatt_lds[off + 16 * t]);
        acc = mfma4(x[0], reg[4 * t + 0], acc);
        acc = mfma4(x[1], reg[4 * t + 1], acc);
        acc = mfma4(x[2], reg[4 * t + 2], acc);
        acc = mfma4(x[3], reg[4 * t + 3], acc);
    }
    return acc;
}

// acc[t] += sum_r LDS[off + roff[r] + 16t] * w[r]: second products (A =
// transposed single reads of the LDS block, B = per-pixel weights).
template <int NT>
__device__ __forceinline__ void block_accumulate(f4 (&acc)[NT], int off, const int (&roff)[4],
                                                 const float (&w)[4]) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int t = 0; t < NT; ++t)
            acc[t] = mfma4(circatt_lds[off + roff[r] + 16 * t], w[r], acc[t]);
}

// Work item k of this workgroup (persistent, XCD-aware); >= nitems when done.
__device__ __forceinline__ int item_of(const FArgs &a, int k) {
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, nslot = gridDim.x >> 3;
    const int begin = xcd * a.per_xcd;
    const int end = min(a.nitems, begin + a.per_xcd);
    const int it = begin + slot + k * nslot;
    return it < end ? it : a.nitems;
}

// PC >= 0: half window compiled in (geometry constants); PC < 0: run-time.
template <int NSP, int NC, bool DIST, int MODE, int PC>
__global__ __launch_bounds__(256, 2) void fused_kernel(FArgs a) {
    using G = FGeo<NSP>;
    using CF = Cfg<NC, MODE, DIST>;
    constexpr int PS = CF::PS, NT = CF::NT, NS = CF::NS, NTEN = CF::NTEN, NSCAL = CF::NSCAL;
    constexpr int PPT = CF::PPT;
    constexpr bool BIAS = CF::BIAS;
    constexpr bool TWO = MODE == MODE_BWDQ || MODE == MODE_BWDKV;
    constexpr bool CT = PC >= 0;
    constexpr HaloGeo GC = plan_halo(NSP, CT ? PC : 0, NC, NTEN, CF::NLDS_SCAL, PPT, DIST ? NC : 0);
    static_assert(!CT || GC.ok, "compiled-in window does not fit");
    // geometry: constants when compiled in
    const int p1 = CT ? GC.p1 : a.hg.p1;
    const int p2 = CT ? GC.p2 : a.hg.p2;
    const int nkh = CT ? GC.nkh : a.hg.nkh;
    const int nkw = CT ? GC.nkw : a.hg.nkw;
    const int halo_h = CT ? GC.halo_h : a.hg.halo_h;
    const int halo_w = CT ? GC.halo_w : a.hg.halo_w;
    const int chunk_rows = CT ? GC.chunk_rows : a.hg.chunk_rows;
    const int CR = CT ? GC.cr : a.hg.cr;
    const int nchunks = CT ? GC.nchunks : a.hg.nchunks;
    constexpr bool ONECHUNK = CT && GC.nchunks == 1;

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int wh = G::wave_h(wv), ww = G::wave_w(wv);
    const int jh = j % G::QH, jw = j / G::QH;

    // LDS layout of a chunk (float offsets into circatt_lds)
    const int chunk_px = CR * halo_w;
    const int oT1 = chunk_px * PS;
    const int oS0 = NTEN * chunk_px * PS;
    const int oS1 = oS0 + chunk_px;
    const int oMU = oS0 + CF::NLDS_SCAL * chunk_px;  // Distance: the item's centre (NC floats)

    // Per-lane LDS bases.  LDS block (i, jb) of this wavefront starts at
    // pixel (wh + KH*i - cr0) + CR*(ww + KW*jb); its element kk = 4g + r sits
    // kk % KH + CR*(kk / KH) pixels further, the A-operand row j at
    // j % KH + CR*(j / KH).  Relative to element r = 0 the elements are
    // r % KH' + CR*(...) apart independently of the lane (rdel).
    const int wbase = wh + CR * ww;
    const int kk0 = 4 * g;
    const int laneA = (wbase + j % G::KH + CR * (j / G::KH)) * PS + 4 * g;
    const int laneE = wbase + kk0 % G::KH + CR * (kk0 / G::KH);  // pixel of element r = 0
    // (kk0 = 4g is a multiple of KH = 2, and KH = 16 is a multiple of 4)
    int rdel[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) rdel[r] = G::KH >= 4 ? r : r % G::KH + CR * (r / G::KH);
    int rdelPS[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) rdelPS[r] = rdel[r] * PS;
    // window tests: element r of block (i, jb) is inside the window of this
    // lane's pixel iff (KH*i + hoff[r]) in [0, 2 p1] and (KW*jb + woff[r]) in
    // [0, 2 p2] (unsigned compares)
    int hoff[4], woff[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        hoff[r] = (kk0 + r) % G::KH - jh;
        woff[r] = (kk0 + r) / G::KH - jw;
    }
    const unsigned span1 = 2 * p1, span2 = 2 * p2;

    // ---- prefetch registers: the next stage's halo and the next item's
    //      register operands (component 16*(s/4) + 4g + s%4 at k-step s) ----
    float hv[PPT][NTEN][NC];
    float hs[PPT][NSCAL > 0 ? NSCAL : 1];
    int hpx[PPT];
    float nr0[NS], nr1[NS], nry[NS];
    float nlse = 0.f;
    // Distance: lane c of the wave holds component c (mod NC) of the item's
    // centre, k at the tile's first pixel (0 past the real components); it
    // is replaced by the next item's only after the item's last chunk is staged
    float nmu = 0.f;

    // 2D tiles in bands of 8 tile rows, column by column within a band, so
    // that the items an XCD runs at once (consecutive item numbers) form a
    // compact block whose halos share that XCD's L2 (a column-major order
    // puts them in one tall strip, whose halos at large windows overflow it)
    auto decode = [&](int item, int &unit, int &h0, int &w0) {
        const int ntiles = a.tiles_h * a.tiles_w;
        unit = item / ntiles;
        const int tile = item - unit * ntiles;
        if constexpr (NSP == 2) {
            int th, tw;
            banded_tile(tile, a.tiles_h, a.tiles_w, th, tw);
            h0 = th * G::TH;
            w0 = tw * G::TW;
        } else {
            h0 = (tile % a.tiles_h) * G::TH;
            w0 = (tile / a.tiles_h) * G::TW;
        }
    };

    auto load_stage = [&](int item, int chunk) {
        int unit, h0, w0;
        decode(item, unit, h0, w0);
        const int cr0 = chunk * chunk_rows;
        const int crn = min(chunk_rows, halo_h - cr0);
        const int npx = crn * halo_w;
        const int64_t uoff = unit_base(a, unit);
        const int64_t soff = (int64_t)unit * a.g.P;
        const float *src0 = (MODE == MODE_BWDKV ? a.q : a.k) + uoff;
        const float *src1 = (MODE == MODE_BWDKV ? a.dy : a.v) + uoff;
#pragma unroll
        for (int pp = 0; pp < PPT; ++pp) {
            const int px0 = threadIdx.x + pp * 256;
            const bool pv = px0 < npx;
            const int px = pv ? px0 : 0;
            const int wl = px / crn, hl = px - wl * crn;
            hpx[pp] = pv ? hl + CR * wl : -1;
            const int64_t gp = pmod(h0 - p1 + cr0 + hl, a.g.n1) +
                               (int64_t)a.g.n1 * pmod(w0 - p2 + wl, a.g.n2);
            load_pixel<NC>(hv[pp][0], src0, a, gp);
            if (NTEN > 1) load_pixel<NC>(hv[pp][NTEN - 1], src1, a, gp);
            if (NSCAL > 0) {
                hs[pp][0] = a.lse[soff + gp];
                hs[pp][NSCAL - 1] = a.dbuf[soff + gp];
            }
        }
    };

    auto load_regs = [&](int item) {
        int unit, h0, w0;
        decode(item, unit, h0, w0);
        const int rh = h0 + wh + jh, rw = w0 + ww + jw;
        const bool rvalid = rh < a.g.n1 && rw < a.g.n2;
        const int64_t rpix = rvalid ? (int64_t)rh + (int64_t)a.g.n1 * rw : 0;
        const int64_t uoff = unit_base(a, unit);
        const float *b0 = (MODE == MODE_BWDKV ? a.k : a.q) + uoff;
        const float *b1 = (MODE == MODE_BWDKV ? a.v : a.dy) + uoff;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int comp = 16 * (s >> 2) + 4 * g + (s & 3);
            const int cc = min(comp, a.ncr - 1);
            const bool cv = comp < a.ncr;
            nr0[s] = cv ? b0[comp_index(a, rpix, cc)] : 0.f;
            if (TWO) nr1[s] = cv ? b1[comp_index(a, rpix, cc)] : 0.f;
            if (MODE == MODE_BWDQ) nry[s] = cv ? a.y[uoff + comp_index(a, rpix, cc)] : 0.f;
        }
        if (MODE == MODE_BWDQ) nlse = a.lse[(int64_t)unit * a.g.P + rpix];
        if constexpr (DIST) {
            const int c = lane & (NC - 1);
            const int64_t p0 = (int64_t)h0 + (int64_t)a.g.n1 * w0;
            nmu = c < a.ncr ? a.k[uoff + comp_index(a, p0, c)] : 0.f;
        }
    };

    // ---- per-item state ----
    float reg0[NS], reg1[NS];
    float sq = 0.f, dq_d = 0.f, lseb = 0.f, rbias = 0.f;
    float m = -1e30f, lsum = 0.f, corr = 0.f;
    f4 acc[2][NT], acc2[2][NT];

    int k = 0;
    int item = item_of(a, 0);
    if (item >= a.nitems) return;  // uniform over the workgroup
    int chunk = 0;
    load_stage(item, 0);
    load_regs(item);

    while (true) {
        if (ONECHUNK) chunk = 0;
        int unit, h0, w0;
        decode(item, unit, h0, w0);
        const int rh = h0 + wh + jh, rw = w0 + ww + jw;
        const bool rvalid = rh < a.g.n1 && rw < a.g.n2;
        const int64_t rpix = rvalid ? (int64_t)rh + (int64_t)a.g.n1 * rw : 0;
        const int64_t uoff = unit_base(a, unit);
        const int64_t soff = (int64_t)unit * a.g.P;
        const int cr0 = chunk * chunk_rows;
        const int crn = min(chunk_rows, halo_h - cr0);

        // Distance: both sides of the score product centred on mu (the
        // expansion q.k - |k|^2 / 2 - |q|^2 / 2 of -|q - k|^2 / 2 then scales
        // with the spread of the data, not its offset).  Lane c of wave 0
        // publishes component c of the item's centre in LDS; every chunk's
        // staged tensor-0 pixels and the register pixel subtract it as they
        // are written (broadcast reads: no per-component registers are held).
        // The previous item's centre was last read before its last chunk's
        // "chunk staged" barrier, which every wave has passed.
        if (DIST && chunk == 0 && threadIdx.x < NC) circatt_lds[oMU + threadIdx.x] = nmu;
        __syncthreads();  // the previous chunk's LDS reads are done
#pragma unroll
        for (int pp = 0; pp < PPT; ++pp) {
            if (hpx[pp] >= 0) {
                const int o0 = hpx[pp] * PS;
                float n2 = 0.f;
#pragma unroll
                for (int c = 0; c < NC; c += 4) {
                    f4 x = f4{hv[pp][0][c], hv[pp][0][c + 1], hv[pp][0][c + 2], hv[pp][0][c + 3]};
                    if constexpr (DIST) x = x - *reinterpret_cast<const f4 *>(&circatt_lds[oMU + c]);
                    *reinterpret_cast<f4 *>(&circatt_lds[o0 + c]) = x;
                    n2 += x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
                }
                if (NTEN > 1) {
#pragma unroll
                    for (int c = 0; c < NC; c += 4)
                        *reinterpret_cast<f4 *>(&circatt_lds[oT1 + o0 + c]) =
                            f4{hv[pp][NTEN - 1][c], hv[pp][NTEN - 1][c + 1],
                               hv[pp][NTEN - 1][c + 2], hv[pp][NTEN - 1][c + 3]};
                }
                if (BIAS) circatt_lds[oS0 + hpx[pp]] = -0.5f * n2;
                if (NSCAL > 0) {
                    // log2-domain subtrahend of the softmax (with the Distance
                    // |q|^2/2 term of the staged query) and D
                    circatt_lds[oS0 + hpx[pp]] =
                        hs[pp][0] * kLog2e + (DIST ? 0.5f * a.c2 * n2 : 0.f);
                    circatt_lds[oS1 + hpx[pp]] = hs[pp][NSCAL - 1];
                }
            }
        }
        if (chunk == 0) {
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                reg0[s] = nr0[s];
                if constexpr (DIST) reg0[s] -= circatt_lds[oMU + 16 * (s >> 2) + 4 * g + (s & 3)];
                if (TWO) reg1[s] = nr1[s];
            }
            float qq = 0.f, dd = 0.f;
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                qq += reg0[s] * reg0[s];
                if (MODE == MODE_BWDQ) dd += reg1[s] * nry[s];
            }
            sq = DIST ? xsum16_32(qq) : 0.f;
            if (MODE == MODE_BWDQ) {
                dq_d = xsum16_32(dd);
                lseb = nlse * kLog2e + (DIST ? 0.5f * sq * a.c2 : 0.f);
            }
            rbias = DIST ? -0.5f * sq : 0.f;  // SIM: -|q|^2/2 ; BWDKV: key bias -|k|^2/2
            m = -1e30f;
            lsum = 0.f;
            corr = 0.f;
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    acc[u][t] = f4{0.f, 0.f, 0.f, 0.f};
                    acc2[u][t] = f4{0.f, 0.f, 0.f, 0.f};
                }
        }
        __syncthreads();  // chunk staged

        // ---- issue the next stage's global loads (consumed next iteration) ----
        int nitem = item, nchunk = chunk + 1;
        if (nchunk == nchunks) {
            nchunk = 0;
            nitem = item_of(a, k + 1);
        }
        const bool has_next = nitem < a.nitems;
        if (has_next) {
            load_stage(nitem, nchunk);
            if (nchunk == 0) load_regs(nitem);
        }

        // ---- this wavefront's LDS blocks inside the chunk: rows i in
        //      [ib, ie), columns jb in [0, nkw), walked two at a time ----
        const int lo = cr0 - wh, hi = cr0 + crn - wh;
        const int ib = lo > 0 ? (lo + G::KH - 1) / G::KH : 0;
        const int ie = hi > 0 ? min(nkh, (hi + G::KH - 1) / G::KH) : 0;
        const int nblk = ie > ib ? (ie - ib) * nkw : 0;
        const float c2 = a.c2;
        const float mlseb = -lseb;

        int bi = ib, bj = 0;  // first block of the pair
        // the key-centric pass keeps four accumulator sets; unrolling its
        // walk would spill, the other modes unroll completely
        constexpr int UNROLL = MODE == MODE_BWDKV ? 1 : 64;
#pragma unroll UNROLL
        for (int qb = 0; qb < (CT ? GC.nkh * GC.nkw : nblk); qb += 2) {
            if (!ONECHUNK && qb >= nblk) break;
            // 2D: wave priority 1 over the first three quarters of a chunk's
            // block walk, 0 over the last, so that a wave near its end yields
            // to the waves behind it (cfg4a on gfx950, interleaved A/B on two
            // boxes: step 2838 -> 2702 and 2913 -> 2843 us; drops at two
            // thirds or seven eighths no better; in 1D, cfg4b, 1.4% slower,
            // so not there)
            if constexpr (NSP == 2) {
                if (qb == 0) __builtin_amdgcn_s_setprio(1);
                if (qb == ((3 * nblk / 4) & ~1)) __builtin_amdgcn_s_setprio(0);
            }
            const bool hasb = qb + 1 < nblk;
            int bi2 = bi, bj2 = bj + 1;
            if (bj2 == nkw) {
                bj2 = 0;
                ++bi2;
            }
            // uniform block offsets (pixels) and window tests
            int bo[2], hrow[2], wcol[2];
            hrow[0] = G::KH * bi;
            wcol[0] = G::KW * bj;
            hrow[1] = hasb ? G::KH * bi2 : hrow[0];
            wcol[1] = hasb ? G::KW * bj2 : wcol[0];
#pragma unroll
            for (int u = 0; u < 2; ++u) bo[u] = (hrow[u] - cr0) + CR * wcol[u];
            bool val[2][4];
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    val[u][r] = (u == 0 || hasb) && (unsigned)(hrow[u] + hoff[r]) <= span1 &&
                                (unsigned)(wcol[u] + woff[r]) <= span2;
            bi = bi2;
            bj = bj2 + 1;
            if (bj == nkw) {
                bj = 0;
                ++bi;
            }

            f4 s[2], dp[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                s[u] = block_product<NT>(laneA + bo[u] * PS, reg0);
                if (TWO) dp[u] = block_product<NT>(oT1 + laneA + bo[u] * PS, reg1);
            }
            // LDS pixel of element r of block u: laneE + bo[u] + rdel[r]

            if constexpr (MODE == MODE_SIM) {
                if (rvalid) {
                    float *nzu = a.nz + (int64_t)unit * a.g.P * a.g.K + rpix * a.g.K;
#pragma unroll
                    for (int u = 0; u < 2; ++u)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if (val[u][r]) {
                                float sv = s[u][r];
                                if (DIST) sv += circatt_lds[oS0 + laneE + bo[u] + rdel[r]] + rbias;
                                const int d1 = hrow[u] + hoff[r] - p1;
                                const int d2 = wcol[u] + woff[r] - p2;
                                nzu[offset_slot(a.g, rpix, d1, d2)] = sv * a.scale;
                            }
                        }
                }
            } else if constexpr (MODE == MODE_FWD) {
                float tt[2][4];
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float sv = s[u][r];
                        if (DIST) sv += circatt_lds[oS0 + laneE + bo[u] + rdel[r]];
                        tt[u][r] = val[u][r] ? sv : -INFINITY;
                    }
                const float lm = fmaxf(fmaxf(fmaxf(tt[0][0], tt[0][1]), fmaxf(tt[0][2], tt[0][3])),
                                       fmaxf(fmaxf(tt[1][0], tt[1][1]), fmaxf(tt[1][2], tt[1][3]))) *
                                 c2;
                if (__any(lm > m + kRescaleLog2)) {
                    const float mn = fmaxf(m, xmax16_32(lm));
                    const float alpha = fast_exp2(m - mn);
                    m = mn;
                    lsum *= alpha;
#pragma unroll
                    for (int u = 0; u < 2; ++u)
#pragma unroll
                        for (int t = 0; t < NT; ++t) acc[u][t] *= alpha;
                }
                const float mm = -m;
                float pr[2][4];
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        pr[u][r] = fast_exp2(fmaf(tt[u][r], c2, mm));
                        lsum += pr[u][r];
                    }
#pragma unroll
                for (int u = 0; u < 2; ++u)
                    block_accumulate<NT>(acc[u], oT1 + (laneE + bo[u]) * PS + j, rdelPS, pr[u]);
            } else if constexpr (MODE == MODE_BWDQ) {
                float ds[2][4];
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float sv = s[u][r];
                        if (DIST) sv += circatt_lds[oS0 + laneE + bo[u] + rdel[r]];
                        const float pr = val[u][r] ? fast_exp2(fmaf(sv, c2, mlseb)) : 0.f;
                        ds[u][r] = pr * (dp[u][r] - dq_d);
                        if (DIST) corr += ds[u][r];
                    }
#pragma unroll
                for (int u = 0; u < 2; ++u)
                    block_accumulate<NT>(acc[u], (laneE + bo[u]) * PS + j, rdelPS, ds[u]);
            } else {  // MODE_BWDKV
                float pr[2][4], ds[2][4];
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int e = laneE + bo[u] + rdel[r];
                        pr[u][r] = val[u][r]
                                       ? fast_exp2(fmaf(s[u][r] + rbias, c2, -circatt_lds[oS0 + e]))
                                       : 0.f;
                        ds[u][r] = pr[u][r] * (dp[u][r] - circatt_lds[oS1 + e]);
                        if (DIST) corr += ds[u][r];
                    }
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    block_accumulate<NT>(acc[u], oT1 + (laneE + bo[u]) * PS + j, rdelPS,
                                         pr[u]);  // dv
                    block_accumulate<NT>(acc2[u], (laneE + bo[u]) * PS + j, rdelPS,
                                         ds[u]);  // dk
                }
            }
        }

        // ---- epilogue after the item's last chunk: lane (j, g) holds
        //      component 16t + 4g + r of pixel j ----
        if (chunk == nchunks - 1) {
            if constexpr (MODE == MODE_FWD) {
                const float l = xsum16_32(lsum);
                const float inv = 1.f / l;
                if (rvalid) {
                    float *yb = a.yout + uoff;
#pragma unroll
                    for (int t = 0; t < NT; ++t)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int comp = 16 * t + 4 * g + r;
                            if (comp < a.ncr)
                                yb[comp_index(a, rpix, comp)] = (acc[0][t][r] + acc[1][t][r]) * inv;
                        }
                    if (g == 0)
                        a.lse_out[soff + rpix] =
                            (m + log2f(l)) * kLn2 - (DIST ? 0.5f * sq * a.scale : 0.f);
                }
            } else if constexpr (MODE == MODE_BWDQ) {
                const float rs = DIST ? xsum16_32(corr) : 0.f;
                if (rvalid) {
                    float *ob = a.dq + uoff;
#pragma unroll
                    for (int t = 0; t < NT; ++t)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int comp = 16 * t + 4 * g + r;
                            float val = acc[0][t][r] + acc[1][t][r];
                            if (DIST) val -= rs * reg0[4 * t + r];
                            if (comp < a.ncr) ob[comp_index(a, rpix, comp)] = val * a.scale;
                        }
                    if (g == 0) a.dbuf[soff + rpix] = dq_d;
                }
            } else if constexpr (MODE == MODE_BWDKV) {
                const float cs = DIST ? xsum16_32(corr) : 0.f;
                if (rvalid) {
                    float *vb = a.dv + uoff;
                    float *kb = a.dk + uoff;
#pragma unroll
                    for (int t = 0; t < NT; ++t)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int comp = 16 * t + 4 * g + r;
                            if (comp < a.ncr) {
                                const int64_t idx = comp_index(a, rpix, comp);
                                vb[idx] = acc[0][t][r] + acc[1][t][r];
                                float val = acc2[0][t][r] + acc2[1][t][r];
                                if (DIST) val -= cs * reg0[4 * t + r];
                                kb[idx] = val * a.scale;
                            }
                        }
                }
            }
        }

        if (!has_next) break;
        if (nchunk == 0) ++k;
        item = nitem;
        chunk = nchunk;
    }
}

// ---------------------------------------------------------------------------
// per-mode launch (one translation unit per mode: fused_<mode>.hip)
// ---------------------------------------------------------------------------
struct FusedPlan {
    FArgs a;
    int nc;
    size_t lds_bytes;
    dim3 grid;
    bool ok;
};

constexpr size_t kLdsMax = 160 * 1024;

template <int NSP, int NC, bool DIST, int MODE, int PC>
hipError_t launch_inst(const FusedPlan &pl, hipStream_t s) {
    auto kern = fused_kernel<NSP, NC, DIST, MODE, PC>;
    // set once per instantiation (a function-local static is initialised
    // exactly once, also when several host threads launch at the same time)
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsMax);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(kern, pl.grid, dim3(256), pl.lds_bytes, s, pl.a);
    return hipGetLastError();
}

// Windows compiled in with constant geometry: the benchmark configurations
// (2D ws = 15 and 11 and 31, 1D ws = 63) at the component counts they use.
template <int NSP, int NC, bool DIST, int MODE>
hipError_t launch_window(const FusedPlan &pl, hipStream_t s) {
    const int p = pl.a.hg.p1;
    if constexpr (NSP == 2 && NC == 16) {
        if (p == 7) return launch_inst<NSP, NC, DIST, MODE, 7>(pl, s);
    }
    if constexpr (NSP == 2 && NC == 32) {
        if (p == 5) return launch_inst<NSP, NC, DIST, MODE, 5>(pl, s);
        if (p == 15) return launch_inst<NSP, NC, DIST, MODE, 15>(pl, s);
    }
    if constexpr (NSP == 1 && NC == 32) {
        if (p == 31) return launch_inst<NSP, NC, DIST, MODE, 31>(pl, s);
    }
    return launch_inst<NSP, NC, DIST, MODE, -1>(pl, s);
}

template <int MODE>
hipError_t launch_mode_all(const FusedPlan &pl, int nsp, bool dist, hipStream_t s) {
#define CIRCATT_LAUNCH_NC(NSP)                                                             \
    switch (pl.nc) {                                                                       \
    case 16: return dist ? launch_window<NSP, 16, true, MODE>(pl, s)                       \
                         : launch_window<NSP, 16, false, MODE>(pl, s);                     \
    case 32: return dist ? launch_window<NSP, 32, true, MODE>(pl, s)                       \
                         : launch_window<NSP, 32, false, MODE>(pl, s);                     \
    case 64: return dist ? launch_window<NSP, 64, true, MODE>(pl, s)                       \
                         : launch_window<NSP, 64, false, MODE>(pl, s);                     \
    }
    if (nsp == 1) {
        CIRCATT_LAUNCH_NC(1)
    } else {
        CIRCATT_LAUNCH_NC(2)
    }
#undef CIRCATT_LAUNCH_NC
    return hipErrorNotSupported;
}

hipError_t launch_fused_fwd(const FusedPlan &pl, int nsp, bool dist, hipStream_t s);
hipError_t launch_fused_sim(const FusedPlan &pl, int nsp, bool dist, hipStream_t s);
hipError_t launch_fused_bwdq(const FusedPlan &pl, int nsp, bool dist, hipStream_t s);
hipError_t launch_fused_bwdkv(const FusedPlan &pl, int nsp, bool dist, hipStream_t s);

}  // namespace circatt
