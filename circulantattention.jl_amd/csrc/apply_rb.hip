// Row-blocked kernels of the unfused (Circulant-materialising) path for
// windows of width 3 .. 15:
//   apply  y[c] = sum_d A[c, slot(c, d)] x[c + d]             (A ⊗ x)
//   trans  y[c] = sum_d A[c - d, slot(c - d, d)] x[c - d]     (Aᵀ ⊗ x)
//          optionally minus (sum of the A entries used) .* z (Distance
//          rrule), times scale; replaces the CUSPARSE.bmm! products of
//          src/batchedmul.jl:82-110;
//   colsum sum(A; dims=1) (src/array.jl:119-130);
//   sim    nzVal = scale * similarity(x, y) (src/similarity.jl:31-103).
//
// nzVal (K floats per pixel) dominates the bytes, so it is read or written
// with wide, coalesced accesses and everything else is arranged around that.
// Every lane owns 4 consecutive pixels along dim 1, so one run of 4 + 2p
// values of x per component serves 4 x ws products.
//   * 2D apply, both directions, and 2D column sums (apply2_kernel): a
//     wavefront owns 64 output pixels of one image row; its four lane groups
//     split the components.  Per window row the slot chunk that row needs of
//     every pixel involved is staged into LDS by 16-byte LDS-DMA pieces, and
//     x one channel per group and step; both are staged by rings of LDS
//     buffers two steps ahead.
//   * similarity (sim_rows_kernel): the same row ownership, lane groups
//     split the window rows; per channel the key rows and queries are staged
//     into LDS with 16-byte loads, and results leave through LDS as runs of
//     each pixel's row.
//   * 1D apply and column sums (apply_rb_kernel, colsum_rb_kernel): a
//     wavefront owns 256 pixels of the line in 4 lane rows; per iteration the
//     slot chunks it needs are DMA-loaded, 16 lanes per chunk, into a
//     wave-private LDS buffer and read back by the owning lanes.
// Wavefronts are dealt to XCDs in bands of consecutive image rows, so that
// rows shared by neighbouring wavefronts stay in one L2.  Near the borders
// of dim 1 the reference's circular shift of the slot order
// (src/circulant.jl:6-44) is applied by border bodies with wrapped columns;
// interior wavefronts use immediate offsets.
#include <algorithm>

#include "circatt_common.h"
#include "circatt_kernels.h"

extern __shared__ __attribute__((aligned(16))) float circatt_lds_apply[];

namespace circatt {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f4u __attribute__((ext_vector_type(4), aligned(4)));  // 4-byte aligned

constexpr int kR = 4;     // pixels per lane along dim 1
constexpr int kCP = 8;    // real components per staging pass of the chunked kernel
constexpr unsigned kRsrcWord3 = 0x00020000;  // raw buffer, 32-bit data

struct ApplyArgs {
    Geom g;
    int C;           // channels per unit
    int corr;        // subtract sums(A) .* z
    int tiles1;      // 64-pixel (2D) or 256-pixel (1D) segments per row
    int fa, fb;      // tile columns [fa, fb) are interior
    int gchunk;      // chunk groups on the grid
    int ichunk;      // chunks per wavefront
    int nrg, brg;    // band kernel: row groups of all units, row groups per XCD band
    float scale;
    const float *nz, *x, *z;
    float *y;
};

__host__ __device__ constexpr int tile_w(int nsp) { return nsp == 2 ? 64 : 256; }
__host__ __device__ constexpr int tile_h(int nsp) { return nsp == 2 ? 4 : 1; }
// staged source pixels per lane row and LDS floats per wavefront
__host__ __device__ constexpr int nsrc(int ws, bool trans) { return trans ? 64 + ws - 1 : 64; }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const float *p, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p), (short)0, (int)bytes,
                                             kRsrcWord3);
}
__device__ __forceinline__ float bload(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ f4 bload4(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// ---------------------------------------------------------------------------
// 1D products and column sums for windows up to 15 (apply_rb_kernel,
// colsum_rb_kernel; 2D and wider windows have the kernels further below).
// A wavefront owns 256 pixels of the line in 4 lane rows of 64 (lane row
// rho = lane >> 4, pixels f1 = 256 t1 + 64 rho ..).
// ---------------------------------------------------------------------------
template <int WS>
struct Lane {
    static constexpr int P = (WS - 1) / 2;
    int l16, rho;   // lane within its lane row, lane row
    int f1;         // first column of the lane row
    __device__ explicit Lane(int t1) {
        const int lane = threadIdx.x & 63;
        l16 = lane & 15;
        rho = lane >> 4;
        f1 = t1 * 256 + 64 * rho;
    }
    __device__ int col(int i) const { return f1 + 4 * l16 + i; }
};

// Stages the slot chunks of the line into the wavefront's LDS buffer with
// LDS-DMA buffer loads (no registers): chunk u (0 <= u < NS) of source column
// f1 - off + u (wrapped) of each lane row.  A load instruction covers chunk u
// of all 4 lane rows; lane 4 e + r loads element e of lane row r, and the
// instruction's 64 dwords land at u * kPU, so element e of chunk u of lane
// row r sits at u * kPU + 4 e + r.  With kPU = 65 the owners' reads
// (u = 4 l16 + i, lane row r) fall in 64 different banks.
constexpr int kPU = 65;
__host__ __device__ constexpr int lds_floats(int ws, bool trans) { return nsrc(ws, trans) * kPU; }

template <int WS, int NS, bool FAST>
__device__ __forceinline__ void stage_dma(float *lw, const Geom &g, __amdgpu_buffer_rsrc_t rs,
                                          int t1, int off, int k4) {
    const int e = min((int)(threadIdx.x & 63) >> 2, WS - 1);
    const int f1r = t1 * 256 + 64 * (threadIdx.x & 3);  // first column of lane row lane & 3
    typedef __attribute__((address_space(3))) void *lptr;
    // each load's offset is formed right before it (fences keep the
    // scheduler from computing all of them up front into registers)
    if (FAST) {
        const int vo = (f1r - off) * k4 + e * 4;
        int so = 0;
#pragma unroll
        for (int u = 0; u < NS; ++u) {
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lptr)(lw + u * kPU), 4, vo,
                                                    __builtin_amdgcn_readfirstlane(so), 0, 0);
            so += k4;
        }
    } else {
        const int vo = e * 4;
        int c = pmod(f1r - off, g.n1);
#pragma unroll
        for (int u = 0; u < NS; ++u) {
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lptr)(lw + u * kPU), 4, vo + c * k4, 0,
                                                    0, 0);
            c = c + 1 == g.n1 ? 0 : c + 1;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
}

// s_waitcnt encodings (gfx9): all counters, LDS/scalar counter only
constexpr int kWaitAll = 0;
constexpr int kWaitLgkm = 0x0070 | 0xC000 | 0x000F;  // lgkmcnt(0), vmcnt and expcnt at max

// slot_shift of 0-based column c (same case order as slot_shift)
__device__ __forceinline__ int shift0(int c, int n, int p) {
    return c + 1 <= p ? c - p : (c + 1 > n - p ? p - n + c + 1 : 0);
}
// j + s folded into [0, ws) for |s| <= p < ws
__device__ __forceinline__ int fold(int v, int ws) {
    return v < 0 ? v + ws : (v >= ws ? v - ws : v);
}

template <int WS, int NCOMP, bool TRANS, bool FAST>
__device__ __forceinline__ void apply_body(const ApplyArgs &a, int gc, int t1, int b) {
    using L_ = Lane<WS>;
    constexpr int P = L_::P;
    constexpr int XW = kR + 2 * P;                 // x run per lane
    constexpr int XN = NCOMP * XW;                 // floats of one run
    constexpr int XN4 = (XN + 3) / 4;
    constexpr int NS = nsrc(WS, TRANS);
    constexpr int CCH = kCP / NCOMP;               // channels per staging pass
    const Geom &g = a.g;
    const int n1 = g.n1, K = g.K;
    const int64_t Pp = g.P;
    const L_ L(t1);
    float *lw = circatt_lds_apply;
    const auto rs = rsrc(a.nz + (int64_t)b * Pp * K, Pp * K * 4);
    const auto rx = rsrc(a.x + (int64_t)b * Pp * NCOMP * a.C, Pp * NCOMP * a.C * 4);

    // x run of channel c: columns f1 + 4 l16 - p .. (wrapped in the border body)
    auto load_x = [&](float (&xw)[4 * XN4], int c, int f1) {
        const int cw = c < a.C ? c : a.C - 1;
        const int rowoff = (int)(NCOMP * Pp * cw) * 4;
        if (FAST) {
            const int vo = rowoff + NCOMP * (f1 + 4 * L.l16 - P) * 4;
#pragma unroll
            for (int q = 0; q < XN4; ++q) {
                const f4 v = bload4(rx, vo, 16 * q);
                xw[4 * q] = v[0];
                xw[4 * q + 1] = v[1];
                xw[4 * q + 2] = v[2];
                xw[4 * q + 3] = v[3];
            }
        } else {
            int xc = pmod(f1 + 4 * L.l16 - P, n1);
#pragma unroll
            for (int w = 0; w < XW; ++w) {
#pragma unroll
                for (int e = 0; e < NCOMP; ++e)
                    xw[NCOMP * w + e] = bload(rx, rowoff + (NCOMP * xc + e) * 4, 0);
                xc = xc + 1 == n1 ? 0 : xc + 1;
            }
        }
    };

    for (int ci = 0; ci < a.ichunk; ++ci) {
        const int k0 = (gc * a.ichunk + ci) * kCP;
        if (k0 >= NCOMP * a.C) break;
        float acc[kR][kCP];
        float asum[kR];
#pragma unroll
        for (int i = 0; i < kR; ++i) {
            asum[i] = 0.f;
#pragma unroll
            for (int kk = 0; kk < kCP; ++kk) acc[i][kk] = 0.f;
        }
        // the buffer is free: the previous chunk's reads completed before
        // its last products
        stage_dma<WS, NS, FAST>(lw, g, rs, t1, TRANS ? P : 0, 4 * K);
        // f1 is redefined here so that per-column offsets are recomputed
        // instead of being hoisted out of the chunk loop as register tables
        int f1 = L.f1;
        asm volatile("" : "+v"(f1));
        __builtin_amdgcn_s_waitcnt(kWaitAll);  // the chunks are in LDS
        float av[kR][WS];
#pragma unroll
        for (int i = 0; i < kR; ++i) {
            // border body: wrapped source column of offset j, stepped from
            // one modulo per pixel
            int c1 = 0, s1 = 0;
            if (!FAST) {
                c1 = pmod(f1 + 4 * L.l16 + i + (TRANS ? P : 0), n1);
                if (!TRANS) s1 = shift0(c1, n1, P);
            }
#pragma unroll
            for (int j = 0; j < WS; ++j) {
                const int u = TRANS ? 4 * L.l16 + i - j + 2 * P : 4 * L.l16 + i;
                int pos = j;
                if (!FAST) {
                    if (TRANS) {
                        pos = fold(j + shift0(c1, n1, P), WS);
                        c1 = c1 == 0 ? n1 - 1 : c1 - 1;
                    } else {
                        pos = fold(j + s1, WS);
                    }
                }
                av[i][j] = lw[u * kPU + 4 * pos + L.rho];
            }
        }
        if (a.corr) {
#pragma unroll
            for (int i = 0; i < kR; ++i)
#pragma unroll
                for (int j = 0; j < WS; ++j) asum[i] += av[i][j];
        }
        // products, one channel (NCOMP components) at a time; channels past C
        // are computed on a clamped channel and not stored
#pragma unroll
        for (int cl = 0; cl < CCH; ++cl) {
            float xc[4 * XN4];
            // nothing crosses these fences, so the loads of later channels are
            // not hoisted over the products into registers
            __builtin_amdgcn_sched_barrier(0);
            load_x(xc, k0 / NCOMP + cl, f1);
#pragma unroll
            for (int i = 0; i < kR; ++i)
#pragma unroll
                for (int j = 0; j < WS; ++j)
#pragma unroll
                    for (int e = 0; e < NCOMP; ++e)
                        acc[i][NCOMP * cl + e] =
                            __builtin_fmaf(av[i][j], xc[NCOMP * (TRANS ? i - j + 2 * P : i + j) + e],
                                           acc[i][NCOMP * cl + e]);
        }
        // every read of the buffer has returned before the next chunk's
        // loads refill it
        __builtin_amdgcn_s_waitcnt(kWaitLgkm);
        // store the chunk
        float *yb = a.y + (int64_t)b * Pp * NCOMP * a.C;
        const float *zb = a.z ? a.z + (int64_t)b * Pp * NCOMP * a.C : nullptr;
#pragma unroll
        for (int i = 0; i < kR; ++i) {
            if (L.col(i) >= n1) continue;
            const int64_t pix = L.col(i);
#pragma unroll
            for (int kk = 0; kk < kCP; ++kk) {
                const int k = k0 + kk;
                if (k >= NCOMP * a.C) break;
                const int c = k / NCOMP, e = k - c * NCOMP;
                const int64_t idx = NCOMP * (pix + Pp * c) + e;
                float v = acc[i][kk];
                if (a.corr) v -= asum[i] * zb[idx];
                yb[idx] = v * a.scale;
            }
        }
    }
}

// One wavefront per (chunk group, 256 pixels, unit).  Tiles [fa, fb) lie 2p
// or more inside the line (no wrap of x, no slot shift) and take the interior
// body, whose offsets are immediates; the others take the border body, which
// computes wrapped columns and shifted slots per value.
template <int WS, int NCOMP, bool TRANS>
__global__ __launch_bounds__(64, 2) void apply_rb_kernel(ApplyArgs a) {
    // item indices (integer division runs on the vector unit: bring the
    // results back to scalar registers, or every buffer load whose descriptor
    // derives from them is wrapped in a readfirstlane loop)
    int it = blockIdx.x;
    const int gc = __builtin_amdgcn_readfirstlane(it % a.gchunk);
    it /= a.gchunk;
    const int t1 = __builtin_amdgcn_readfirstlane(it % a.tiles1);
    const int b = __builtin_amdgcn_readfirstlane(it / a.tiles1);
    if (t1 >= a.fa && t1 < a.fb)
        apply_body<WS, NCOMP, TRANS, true>(a, gc, t1, b);
    else
        apply_body<WS, NCOMP, TRANS, false>(a, gc, t1, b);
}

// sum(A; dims=1): out[c] = sum over window offsets d of A[c - d, slot(c - d, d)]
template <int WS, bool FAST>
__device__ __forceinline__ void colsum_body(const Geom &g, int t1, int b, const float *nz,
                                            float *out) {
    using L_ = Lane<WS>;
    constexpr int P = L_::P;
    constexpr int NS = nsrc(WS, true);
    const int n1 = g.n1, K = g.K;
    const L_ L(t1);
    float *lw = circatt_lds_apply;
    const auto rs = rsrc(nz + (int64_t)b * g.P * K, g.P * K * 4);
    float s[kR] = {0.f, 0.f, 0.f, 0.f};
    stage_dma<WS, NS, FAST>(lw, g, rs, t1, P, 4 * K);
    int f1 = L.f1;
    asm volatile("" : "+v"(f1));
    __builtin_amdgcn_s_waitcnt(kWaitAll);
#pragma unroll
    for (int i = 0; i < kR; ++i)
#pragma unroll
        for (int j = 0; j < WS; ++j) {
            const int u = 4 * L.l16 + i - j + 2 * P;
            int pos = j;
            if (!FAST) pos = fold(j + shift0(pmod(f1 - P + u, n1), n1, P), WS);
            s[i] += lw[u * kPU + 4 * pos + L.rho];
        }
#pragma unroll
    for (int i = 0; i < kR; ++i)
        if (L.col(i) < n1) out[(int64_t)b * g.P + L.col(i)] = s[i];
}

template <int WS>
__global__ __launch_bounds__(64, 2) void colsum_rb_kernel(Geom g, int tiles1, int fa, int fb,
                                                          const float *nz, float *out) {
    const int t1 = __builtin_amdgcn_readfirstlane((int)blockIdx.x % tiles1);
    const int b = __builtin_amdgcn_readfirstlane((int)blockIdx.x / tiles1);
    if (t1 >= fa && t1 < fb)
        colsum_body<WS, true>(g, t1, b, nz, out);
    else
        colsum_body<WS, false>(g, t1, b, nz, out);
}

// s_waitcnt vmcnt(N) (gfx9 encoding, expcnt and lgkmcnt at their maximum)
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt has 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// vmcnt(C0 + n XI) for n in 0 .. K (n wave-uniform; constant after unrolling)
template <int C0, int XI, int K>
__device__ __forceinline__ void wait_vm_steps(int n) {
    if constexpr (K == 0) {
        wait_vm<C0>();
    } else {
        if (n >= K)
            wait_vm<C0 + K * XI>();
        else
            wait_vm_steps<C0, XI, K - 1>(n);
    }
}

// ---------------------------------------------------------------------------
// nzVal = scale * similarity(x, y) in 2D (src/similarity.jl:31-103): a
// wavefront owns 64 consecutive pixels of one image row; lane group r takes
// window rows r, r + 4, ...; for one window row a lane accumulates the ws
// slots of its 4 pixels over the channels (sequentially, as the reference
// does), then stores each pixel's chunk of ws slots (contiguous in the row,
// rotated near borders).
//
// Per channel the 4 key rows' columns f1 - kHalo .. f1 + 63 + kHalo and the
// 64 query pixels are staged into LDS by LDS-DMA, in 16-byte pieces (3 + 1
// loads for complex data instead of one overlapping run of 4 + 2p pixels per
// lane), into a ring of NR buffers NR - 1 channels ahead; the lanes read
// their runs back from LDS.  Loads return in issue order, and each channel
// waits with a vmcnt that counts the loads of the channels staged after it.
// ---------------------------------------------------------------------------
constexpr int kHalo = 8;  // staged key columns beyond each side (>= p)
constexpr int kJC = 16;   // window columns per sub-row (windows wider than 15)
template <int NCOMP, int CP = 1>
struct SimStage {
    // CP channels per step (the row kernel pairs real channels, so that a
    // step stages and multiplies as much as one complex channel)
    static constexpr int RW = 64 + 2 * kHalo;  // staged key columns per row
    static constexpr int CR = NCOMP * RW;      // floats per key row and channel
    static constexpr int RF = CP * CR;         // floats per key row
    static constexpr int KF = 4 * RF;          // key floats
    static constexpr int KS = KF / 4;          // key pieces
    static constexpr int KL = (KS + 63) / 64;  // 16-byte key loads per lane
    static constexpr int QC = NCOMP * 64;      // query floats per channel
    static constexpr int QF = CP * QC;         // query floats
    static constexpr int QS = QF / 4;          // query pieces (<= 64)
    static constexpr int QOFF = KL * 256;      // query area (floats)
    static constexpr int SB = QOFF + 256;      // floats per ring buffer
    static constexpr int KL1 = KF / 64, QL1 = QF / 64;  // 4-byte loads (border)
    // ring buffers: complex data three steps ahead (cfg5 on gfx950,
    // interleaved A/B: 142.4 -> 137.9 us, five buffers 148.9 us); real data
    // two (three ahead was within noise or slower at cfg2, cfg4a and 512x96)
    static constexpr int NR = NCOMP == 2 ? 4 : 3;
};

// XV: pieces of 16 bytes (interior segments, and border segments when n1 is
// a multiple of the 4 / NCOMP pixels of a piece); otherwise float by float.
template <int WS, int NCOMP, bool DIST, bool FAST, bool XV = FAST>
__device__ __forceinline__ void sim_body(const ApplyArgs &a, int gc, int t1, int c2, int b) {
    constexpr int CP = NCOMP == 1 ? 2 : 1;  // channels per step
    using S = SimStage<NCOMP, CP>;
    constexpr int P = (WS - 1) / 2;
    constexpr int K = WS * WS;
    constexpr int XW = kR + 2 * P;
    constexpr int NIT = (WS + 3) / 4;
    // a lane's key run starts at staged column 4 l16 + kHalo - P; it is read
    // from the 16-byte boundary AL floats before
    constexpr int AL = (NCOMP * (kHalo - P)) % 4;
    constexpr int KW4 = (NCOMP * XW + AL + 3) / 4;
    constexpr int NK = XV ? S::KL : S::KL1;  // key loads per lane and channel
    constexpr int NQ = XV ? 1 : S::QL1;      // query loads
    constexpr int NI = NK + NQ;
    static_assert(P <= kHalo, "window wider than the staged halo");
    static_assert(NI < 64, "vmcnt");
    typedef __attribute__((address_space(3))) void *lptr;
    const Geom &g = a.g;
    const int n1 = g.n1, n2 = g.n2;
    const int64_t Pp = g.P;
    const int lane = threadIdx.x & 63;
    const int l16 = lane & 15, rho = lane >> 4;
    const int f1 = t1 * 64;
    const int ubytes = (int)(Pp * NCOMP * a.C * 4);
    const auto rq = rsrc(a.x + (int64_t)b * Pp * NCOMP * a.C, ubytes);  // rows (queries)
    const auto rk = rsrc(a.z + (int64_t)b * Pp * NCOMP * a.C, ubytes);  // columns (keys)
    float *nzb = a.y + (int64_t)b * Pp * K;
    float *lw = circatt_lds_apply;
    int s1[kR];
#pragma unroll
    for (int i = 0; i < kR; ++i) s1[i] = FAST ? 0 : shift0(pmod(f1 + 4 * l16 + i, n1), n1, P);
    const int s2 = slot_shift(c2 + 1, n2, P);
    const int plane = (int)(NCOMP * Pp * 4);  // bytes per channel
    // query offsets (the lane's piece, or float, of the 64 query pixels of
    // channel h of the step)
    int qo[NQ];
#pragma unroll
    for (int m = 0; m < NQ; ++m) {
        const int f = XV ? 4 * min(lane, S::QS - 1) : lane + 64 * m;
        const int h = f / S::QC, w = f - h * S::QC;
        const int u = w / NCOMP, e = w - u * NCOMP;  // (e = 0 for a piece)
        const int col = FAST ? f1 + u : pmod(f1 + u, n1);
        qo[m] = h * plane + (NCOMP * (n1 * c2 + col) + e) * 4;
    }
    // steps of CP channels; a second channel past C lies past the unit's
    // bytes and reads as zeros, which add nothing to either similarity
    const int nst = (a.C + CP - 1) / CP;

    // window-row iterations [gc * ichunk, ...) of this wavefront
    const int it1 = min(NIT, (gc + 1) * a.ichunk);
    for (int itr = gc * a.ichunk; itr < it1; ++itr) {
        const int dd = 4 * itr + rho;
        const bool live = dd < WS;
        const int mm = pmod(min(dd, WS - 1) + s2, WS);
        // key offsets of this iteration: the lane's piece (or float) of key
        // row rr = window row 4 itr + rr (clamped)
        int ko[NK];
#pragma unroll
        for (int m = 0; m < NK; ++m) {
            const int f = XV ? 4 * min(lane + 64 * m, S::KS - 1) : lane + 64 * m;
            const int rr = f / S::RF, rf = f - rr * S::RF;
            const int h = rf / S::CR, w = rf - h * S::CR;
            const int kr2 = pmod(c2 + min(4 * itr + rr, WS - 1) - P, n2);
            const int u = w / NCOMP, e = w - u * NCOMP;  // (e = 0 for a piece)
            const int col = FAST ? f1 - kHalo + u : pmod(f1 - kHalo + u, n1);
            ko[m] = h * plane + (NCOMP * (n1 * kr2 + col) + e) * 4;
        }
        // step c: channels c CP ..; the whole offset is in the vector
        // operand, which the range check sees
        auto stage = [&](int c, int buf) {
            const int cb = __builtin_amdgcn_readfirstlane(c * CP * plane);
            float *dst = lw + buf * S::SB;
#pragma unroll
            for (int m = 0; m < NK; ++m) {
                __builtin_amdgcn_sched_barrier(0);
                if (XV) {
                    // (lanes past the last piece load nothing; some lane of
                    // every instruction is active, so each is issued)
                    if (lane + 64 * m < S::KS)
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lptr)(dst + 256 * m), 16,
                                                                ko[m] + cb, 0, 0, 0);
                } else {
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lptr)(dst + 64 * m), 4,
                                                            ko[m] + cb, 0, 0, 0);
                }
            }
#pragma unroll
            for (int m = 0; m < NQ; ++m) {
                __builtin_amdgcn_sched_barrier(0);
                if (XV) {
                    if (lane < S::QS)
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lptr)(dst + S::QOFF), 16,
                                                                qo[m] + cb, 0, 0, 0);
                } else {
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lptr)(dst + S::QOFF + 64 * m), 4,
                                                            qo[m] + cb, 0, 0, 0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        };

        float acc[kR][WS];
#pragma unroll
        for (int i = 0; i < kR; ++i)
#pragma unroll
            for (int j = 0; j < WS; ++j) acc[i][j] = 0.f;
        // the previous iteration's reads of the LDS area are complete
        __builtin_amdgcn_s_waitcnt(kWaitLgkm);
        constexpr int SD = S::NR - 1;  // steps staged ahead
        static_assert((SD - 1) * NI < 64, "waits exceed vmcnt");
#pragma unroll
        for (int u = 0; u < SD; ++u)
            if (u < nst) stage(u, u);
        int cur = 0;
#pragma unroll 1
        for (int c = 0; c < nst; ++c) {
            // priority 1 over the first three quarters of the steps, 0 over
            // the last (cfg5 on gfx950, interleaved A/B: 145.6 -> 143.7 us)
            if (c == 0) __builtin_amdgcn_s_setprio(1);
            if (c == (3 * nst) / 4) __builtin_amdgcn_s_setprio(0);
            // loads issued after step c's: those of steps c + 1 .. c + SD - 1
            wait_vm_steps<0, NI, SD - 1>(min(SD - 1, nst - 1 - c));
            // the buffer refilled here was read for step c - 1
            __builtin_amdgcn_s_waitcnt(kWaitLgkm);
            if (c + SD < nst) stage(c + SD, cur == 0 ? S::NR - 1 : cur - 1);
            const float *sb = lw + cur * S::SB;
#pragma unroll
            for (int hc = 0; hc < CP; ++hc) {
                float q[4 * NCOMP], kw[4 * KW4];
#pragma unroll
                for (int h = 0; h < NCOMP; ++h) {
                    const f4 v = *(const f4 *)(sb + S::QOFF + hc * S::QC + NCOMP * 4 * l16 + 4 * h);
                    q[4 * h] = v[0];
                    q[4 * h + 1] = v[1];
                    q[4 * h + 2] = v[2];
                    q[4 * h + 3] = v[3];
                }
                const float *kr =
                    sb + rho * S::RF + hc * S::CR + NCOMP * (4 * l16 + kHalo - P) - AL;
#pragma unroll
                for (int h = 0; h < KW4; ++h) {
                    const f4 v = *(const f4 *)(kr + 4 * h);
                    kw[4 * h] = v[0];
                    kw[4 * h + 1] = v[1];
                    kw[4 * h + 2] = v[2];
                    kw[4 * h + 3] = v[3];
                }
#pragma unroll
                for (int i = 0; i < kR; ++i)
#pragma unroll
                    for (int j = 0; j < WS; ++j)
#pragma unroll
                        for (int e = 0; e < NCOMP; ++e) {
                            const float xv = q[NCOMP * i + e], yv = kw[AL + NCOMP * (i + j) + e];
                            if (DIST) {
                                const float d = xv - yv;
                                acc[i][j] = __builtin_fmaf(d, d, acc[i][j]);
                            } else {
                                acc[i][j] = __builtin_fmaf(xv, yv, acc[i][j]);
                            }
                        }
            }
            cur = cur == S::NR - 1 ? 0 : cur + 1;
        }
        // (the ring area is rewritten below: its last reads are complete, as
        // LDS operations of a wavefront complete in order, and no load is in
        // flight.)  The slot shifts are redefined here, so that the store
        // addresses are not computed before the channel loop and held
#pragma unroll
        for (int i = 0; i < kR; ++i) asm volatile("" : "+v"(s1[i]));
        const float sc = DIST ? -0.5f * a.scale : a.scale;
        // the live window rows of this iteration, mm0 .. mm0 + nlive - 1,
        // are one run of each pixel's nzVal row unless the slot order wraps
        const int nlive = min(4, WS - 4 * itr);
        const int mm0 = pmod(4 * itr + s2, WS);
        if (mm0 + nlive <= WS) {
            // through LDS, then 16 lanes per pixel store its run of nlive * ws
            // floats with 16-byte stores, 4 pixels per instruction.  Pixel px
            // sits at px PS + 4 (px / 4): the writing lanes (pixels 4 apart)
            // then fall in different banks
            constexpr int PS = 4 * WS;  // LDS floats per pixel
            if (live) {
#pragma unroll
                for (int i = 0; i < kR; ++i)
#pragma unroll
                    for (int j = 0; j < WS; ++j)
                        lw[(4 * l16 + i) * PS + 4 * l16 + rho * WS +
                           (FAST ? j : fold(j + s1[i], WS))] = acc[i][j] * sc;
            }
            const int run = nlive * WS, tq = lane & 15, g4 = lane >> 4;
#pragma unroll 4
            for (int m = 0; m < 16; ++m) {
                const int px = 4 * m + g4, col = f1 + px;
                const f4 v = *(const f4 *)(lw + px * PS + 4 * m + 4 * tq);
                float *dst = nzb + (col + (int64_t)n1 * c2) * K + mm0 * WS + 4 * tq;
                if (col >= n1 || 4 * tq >= run) continue;
                if (4 * tq + 4 <= run) {
                    *(f4u *)dst = v;
                } else {
#pragma unroll
                    for (int e = 0; e < 3; ++e)
                        if (4 * tq + e < run) dst[e] = v[e];
                }
            }
        } else if (live) {
#pragma unroll
            for (int i = 0; i < kR; ++i) {
                const int col = f1 + 4 * l16 + i;
                if (col >= n1) continue;
                float *row = nzb + (col + (int64_t)n1 * c2) * K + mm * WS;
#pragma unroll
                for (int j = 0; j < WS; ++j) row[FAST ? j : fold(j + s1[i], WS)] = acc[i][j] * sc;
            }
        }
    }
}

// One wavefront per (64 pixels of an image row, unit).  Fields of ApplyArgs:
// x = rows (queries), z = columns (keys), y = nzVal.  The dispatcher deals
// workgroups round robin over the 8 XCDs; work item (bid % 8) * nper + bid / 8
// gives each XCD a contiguous band of image rows, whose key rows stay in its
// L2 for the wavefronts of the neighbouring rows.
template <int WS, int NCOMP, bool DIST>
__global__ __launch_bounds__(64, 2) void sim_rows_kernel(ApplyArgs a, int nwork) {
    const int nper = (nwork + 7) >> 3;
    int it = (int)(blockIdx.x & 7) * nper + (int)(blockIdx.x >> 3);
    if (it >= nwork) return;
    const int gc = __builtin_amdgcn_readfirstlane(it % a.gchunk);
    it /= a.gchunk;
    const int t1 = __builtin_amdgcn_readfirstlane(it % a.tiles1);
    it /= a.tiles1;
    const int c2 = __builtin_amdgcn_readfirstlane(it % a.g.n2);
    const int b = __builtin_amdgcn_readfirstlane(it / a.g.n2);
    if (t1 >= a.fa && t1 < a.fb)
        sim_body<WS, NCOMP, DIST, true>(a, gc, t1, c2, b);
    else if (a.g.n1 % (4 / NCOMP) == 0)
        sim_body<WS, NCOMP, DIST, false, true>(a, gc, t1, c2, b);
    else
        sim_body<WS, NCOMP, DIST, false, false>(a, gc, t1, c2, b);
}

// ---------------------------------------------------------------------------
// Similarity for wide windows (any odd ws, 1D or 2D; sim_wide_kernel): tasks
// are sub-rows (window row dd, columns j0 = 16 jc .. j0 + 15), and lane group
// r takes task 4 itr + r, so that 1D windows (one window row) use all four
// groups.  Per channel the four tasks' key rows (80 columns from
// f1 + j0 - p) and the 64 queries are staged by LDS-DMA (a ring of 3, two
// channels ahead).  Interior segments store through LDS, 4 lanes per
// (pixel, task) run of 16 slots; border segments, whose slots are rotated,
// store directly.
// ---------------------------------------------------------------------------
template <int NCOMP, bool DIST, bool FAST>
__device__ __forceinline__ void sim_wide_body(const ApplyArgs &a, int t1, int c2, int b) {
    using S = SimStage<NCOMP>;  // key rows of 80 columns, queries, ring
    constexpr int KW4 = (NCOMP * (kR + kJC - 1) + 3) / 4;
    constexpr int NK = FAST ? S::KL : S::KL1;
    constexpr int NQ = FAST ? 1 : S::QL1;
    constexpr int NI = NK + NQ;
    static_assert(NI < 64, "vmcnt");
    typedef __attribute__((address_space(3))) void *lptr;
    const Geom &g = a.g;
    const int WS = g.ws, P = g.p, K = g.K;
    const bool two = g.nsp == 2;
    const int n1 = g.n1, n2 = two ? g.n2 : 1;
    const int WR = two ? WS : 1;
    const int NJC = (WS + kJC - 1) / kJC;
    const int NT = WR * NJC;                 // tasks
    const int64_t Pp = g.P;
    const int lane = threadIdx.x & 63;
    const int l16 = lane & 15, rho = lane >> 4;
    const int f1 = t1 * 64;
    const int ubytes = (int)(Pp * NCOMP * a.C * 4);
    const auto rq = rsrc(a.x + (int64_t)b * Pp * NCOMP * a.C, ubytes);
    const auto rk = rsrc(a.z + (int64_t)b * Pp * NCOMP * a.C, ubytes);
    float *nzb = a.y + (int64_t)b * Pp * K;
    float *lw = circatt_lds_apply;
    const int s2 = two ? slot_shift(c2 + 1, n2, P) : 0;
    const int plane = (int)(NCOMP * Pp * 4);
    int qo[NQ];
#pragma unroll
    for (int m = 0; m < NQ; ++m) {
        if (FAST) {
            const int u = 4 * min(lane, S::QS - 1) / NCOMP;
            qo[m] = NCOMP * (n1 * c2 + f1 + u) * 4;
        } else {
            const int f = lane + 64 * m, u = f / NCOMP, e = f - u * NCOMP;
            qo[m] = (NCOMP * (n1 * c2 + pmod(f1 + u, n1)) + e) * 4;
        }
    }
    // task -> window row, sub-row
    auto task = [&](int tau, int &dd, int &jc) {
        const int tc = min(tau, NT - 1);
        dd = tc / NJC;
        jc = tc - dd * NJC;
    };

    const int nit = (NT + 3) / 4;
#pragma unroll 1
    for (int itr = 0; itr < nit; ++itr) {
        // priority 1 over the first three quarters, 0 over the last (cfg4a on
        // gfx950, interleaved A/B: 926 -> 909 us)
        if (itr == 0) __builtin_amdgcn_s_setprio(1);
        if (itr == (3 * nit) / 4) __builtin_amdgcn_s_setprio(0);
        int ko[NK];
#pragma unroll
        for (int m = 0; m < NK; ++m) {
            const int f = FAST ? 4 * min(lane + 64 * m, S::KS - 1) : lane + 64 * m;
            const int rr = f / S::RF, w = f - rr * S::RF;
            int dd, jc;
            task(4 * itr + rr, dd, jc);
            const int kr2 = two ? pmod(c2 + dd - P, n2) : 0;
            const int u = w / NCOMP, e = w - u * NCOMP;
            const int c0 = f1 + kJC * jc - P;
            const int col = FAST ? c0 + u : pmod(c0 + u, n1);
            ko[m] = (NCOMP * (n1 * kr2 + col) + e) * 4;
        }
        auto stage = [&](int c, int buf) {
            const int cb = __builtin_amdgcn_readfirstlane(c * plane);
            float *dst = lw + buf * S::SB;
#pragma unroll
            for (int m = 0; m < NK; ++m) {
                __builtin_amdgcn_sched_barrier(0);
                if (FAST) {
                    if (lane + 64 * m < S::KS)
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lptr)(dst + 256 * m), 16,
                                                                ko[m], cb, 0, 0);
                } else {
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lptr)(dst + 64 * m), 4, ko[m],
                                                            cb, 0, 0);
                }
            }
#pragma unroll
            for (int m = 0; m < NQ; ++m) {
                __builtin_amdgcn_sched_barrier(0);
                if (FAST) {
                    if (lane < S::QS)
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lptr)(dst + S::QOFF), 16,
                                                                qo[m], cb, 0, 0);
                } else {
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lptr)(dst + S::QOFF + 64 * m), 4,
                                                            qo[m], cb, 0, 0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        float acc[kR][kJC];
#pragma unroll
        for (int i = 0; i < kR; ++i)
#pragma unroll
            for (int j = 0; j < kJC; ++j) acc[i][j] = 0.f;
        __builtin_amdgcn_s_waitcnt(kWaitLgkm);
        constexpr int SD = S::NR - 1;  // channels staged ahead
        static_assert((SD - 1) * NI < 64, "waits exceed vmcnt");
#pragma unroll
        for (int u = 0; u < SD; ++u)
            if (u < a.C) stage(u, u);
        int cur = 0;
#pragma unroll 1
        for (int c = 0; c < a.C; ++c) {
            wait_vm_steps<0, NI, SD - 1>(min(SD - 1, a.C - 1 - c));
            __builtin_amdgcn_s_waitcnt(kWaitLgkm);
            if (c + SD < a.C) stage(c + SD, cur == 0 ? S::NR - 1 : cur - 1);
            const float *sb = lw + cur * S::SB;
            float q[4 * NCOMP], kw[4 * KW4];
#pragma unroll
            for (int h = 0; h < NCOMP; ++h) {
                const f4 v = *(const f4 *)(sb + S::QOFF + NCOMP * 4 * l16 + 4 * h);
                q[4 * h] = v[0];
                q[4 * h + 1] = v[1];
                q[4 * h + 2] = v[2];
                q[4 * h + 3] = v[3];
            }
            const float *kr = sb + rho * S::RF + NCOMP * 4 * l16;
#pragma unroll
            for (int h = 0; h < KW4; ++h) {
                const f4 v = *(const f4 *)(kr + 4 * h);
                kw[4 * h] = v[0];
                kw[4 * h + 1] = v[1];
                kw[4 * h + 2] = v[2];
                kw[4 * h + 3] = v[3];
            }
#pragma unroll
            for (int i = 0; i < kR; ++i)
#pragma unroll
                for (int j = 0; j < kJC; ++j)
#pragma unroll
                    for (int e = 0; e < NCOMP; ++e) {
                        const float xv = q[NCOMP * i + e], yv = kw[NCOMP * (i + j) + e];
                        if (DIST) {
                            const float d = xv - yv;
                            acc[i][j] = __builtin_fmaf(d, d, acc[i][j]);
                        } else {
                            acc[i][j] = __builtin_fmaf(xv, yv, acc[i][j]);
                        }
                    }
            cur = cur == S::NR - 1 ? 0 : cur + 1;
        }
        // this group's task; slots past the window are not stored
        const float sc = DIST ? -0.5f * a.scale : a.scale;
        const int tau = 4 * itr + rho;
        int dd, jc;
        task(tau, dd, jc);
        const bool live = tau < NT;
        const int mm = two ? pmod(dd + s2, WS) : 0;
        const int j0 = kJC * jc, jn = min(kJC, WS - j0);
        if (FAST) {
            // through LDS (the ring area is free: its last reads are complete
            // and no load is in flight): pixel px, task r at
            // px 64 + 4 (px / 4) + 16 r
            if (live) {
#pragma unroll
                for (int i = 0; i < kR; ++i)
#pragma unroll
                    for (int j = 0; j < kJC; ++j)
                        lw[(4 * l16 + i) * 64 + 4 * l16 + 16 * rho + j] = acc[i][j] * sc;
            }
            // 16 lanes per pixel: lane tq stores piece tq % 4 of task tq / 4
            const int tq = lane & 15, g4 = lane >> 4, tr = tq >> 2, pc = tq & 3;
            int ddt, jct;
            task(4 * itr + tr, ddt, jct);
            const bool livet = 4 * itr + tr < NT;
            const int mmt = two ? pmod(ddt + s2, WS) : 0;
            const int j0t = kJC * jct, jnt = min(kJC, WS - j0t);
#pragma unroll 4
            for (int m = 0; m < 16; ++m) {
                const int px = 4 * m + g4, col = f1 + px;
                const f4 v = *(const f4 *)(lw + px * 64 + 4 * m + 16 * tr + 4 * pc);
                float *dst = nzb + (col + (int64_t)n1 * c2) * K + mmt * WS + j0t + 4 * pc;
                if (!livet || col >= n1 || 4 * pc >= jnt) continue;
                if (4 * pc + 4 <= jnt) {
                    *(f4u *)dst = v;
                } else {
#pragma unroll
                    for (int e = 0; e < 3; ++e)
                        if (4 * pc + e < jnt) dst[e] = v[e];
                }
            }
        } else if (live) {
#pragma unroll
            for (int i = 0; i < kR; ++i) {
                const int col = f1 + 4 * l16 + i;
                if (col >= n1) continue;
                const int s1 = shift0(pmod(col, n1), n1, P);
                float *row = nzb + (col + (int64_t)n1 * c2) * K + mm * WS;
#pragma unroll
                for (int j = 0; j < kJC; ++j)
                    if (j < jn) row[fold(j0 + j + s1, WS)] = acc[i][j] * sc;
            }
        }
    }
}

template <int NCOMP, bool DIST>
__global__ __launch_bounds__(64, 2) void sim_wide_kernel(ApplyArgs a, int nwork) {
    const int nper = (nwork + 7) >> 3;
    int it = (int)(blockIdx.x & 7) * nper + (int)(blockIdx.x >> 3);
    if (it >= nwork) return;
    const int t1 = __builtin_amdgcn_readfirstlane(it % a.tiles1);
    it /= a.tiles1;
    const int n2 = a.g.nsp == 2 ? a.g.n2 : 1;
    const int c2 = __builtin_amdgcn_readfirstlane(it % n2);
    const int b = __builtin_amdgcn_readfirstlane(it / n2);
    if (t1 >= a.fa && t1 < a.fb)
        sim_wide_body<NCOMP, DIST, true>(a, t1, c2, b);
    else
        sim_wide_body<NCOMP, DIST, false>(a, t1, c2, b);
}

template <int NCOMP, bool DIST>
hipError_t launch_sim_wide_t(ApplyArgs a, int64_t nb, hipStream_t s) {
    using S = SimStage<NCOMP>;
    const int n1 = a.g.n1, n2 = a.g.nsp == 2 ? a.g.n2 : 1;
    a.tiles1 = (n1 + 63) / 64;
    // interior: staged key columns f1 - p .. f1 + p + 79 in range, own
    // columns free of slot shifts
    const int edge = a.g.p + kJC;
    a.fa = (edge + 63) / 64;
    a.fb = n1 - 64 - edge >= 0 ? (n1 - 64 - edge) / 64 + 1 : 0;
    if (a.fb > a.tiles1) a.fb = a.tiles1;
    if (a.fb < a.fa) a.fb = a.fa;
    const int64_t nwork = (int64_t)a.tiles1 * n2 * nb;
    const size_t lds = (size_t)std::max(S::NR * S::SB, 64 * 64 + 64 + 64) * sizeof(float);
    hipLaunchKernelGGL((sim_wide_kernel<NCOMP, DIST>), dim3((unsigned)(8 * ((nwork + 7) / 8))),
                       dim3(64), lds, s, a, (int)nwork);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// 2D apply, both directions (apply2_kernel): a wavefront owns 64 output
// pixels of one image row and a pass of 4 x kCG components; lane group g
// (lane >> 4) owns components g kCG .. g kCG + kCG - 1 of the pass, so no
// partial sums are exchanged.  Per window row dd the wavefront needs one slot
// chunk of every pixel involved (the 64 own pixels for A ⊗ x, the 64 + 2p
// source pixels for Aᵀ ⊗ x); per step (window row, channel of each group) it
// needs the x row's columns f1 - kHalo .. f1 + 63 + kHalo.  Both are staged
// by LDS-DMA into rings (2 chunk buffers, 3 x buffers), x two steps ahead
// and the chunks of row dd + 1 during row dd, so that the loads' latency is
// covered by two steps of products.  Loads return in issue order: each step
// waits with a vmcnt that counts exactly the loads issued after the ones it
// needs.
//   forward:    y[o] += A[o, slot(o, (j - p, dd - p))] x[o + (j - p, dd - p)]
//   transposed: y[o] += A[s, slot(s, (p - j, dd - p))] x[s], s = o - (p - j, dd - p)
// ---------------------------------------------------------------------------
constexpr int kCG = 8;          // components per lane group and pass
constexpr int kCPass = 4 * kCG; // components per pass
// x ring sizes (x loads in flight kNX - 1 steps ahead of a step).  Four
// buffers against three, interleaved A/B on gfx950 (identical outputs):
// cfg5 apply 130 -> 125 us, transposed 140 -> 130 us, similarity pullback
// (pair kernel) 263 -> 233 us; 1D ws = 63 (wide kernel) apply 104 -> 98 us,
// pullback 198 -> 185 us.  Five were slower than four.  Grids of fewer
// wavefronts than SIMDs (passes of 16 components) keep three: deeper rings
// did not help there (cfg2 34.6 -> 36.9 us with five).
constexpr int kNX = 4;
constexpr int kNXSmall = 3;

// CG: components per lane group and pass (4 CG per pass); NX: x buffers in
// the ring, so that NX - 1 steps' x loads are in flight ahead of a step
template <int WS, int NCOMP, bool TRANS, int CG = kCG, int NX = 3>
struct A2 {
    static constexpr int P = (WS - 1) / 2;
    static constexpr int NSRC = TRANS ? 64 + 2 * P : 64;  // staged chunks per row
    static constexpr int WSP = (WS + 3) & ~3;             // LDS floats per chunk
    static constexpr int Q = WSP / 4;                     // 16-byte pieces per chunk
    // chunks in blocks of 4, each block followed by one free 16-byte slot:
    // piece q of chunk w is slot w Q + q + w / 4, so chunks 4 apart (the
    // lanes of one read) lie an odd number 4 Q + 1 of slots apart and their
    // reads fall in different banks
    static constexpr int BLK = 4 * Q + 1;                 // slots per block
    static constexpr int NSLOT = (NSRC + 3) / 4 * BLK;
    static constexpr int NZ4 = (NSLOT + 63) / 64;         // interior: 16-byte DMA loads per lane
    static constexpr int NZ1 = (4 * NSLOT + 63) / 64;     // border: 4-byte DMA loads per lane
    static constexpr int NZB = NZ4 * 256 > NZ1 * 64 ? NZ4 * 256 : NZ1 * 64;  // chunk buffer floats
    // border tiles, mixed form: single-slot loads per lane over the LDS span
    // of a run of 2p chunks
    static constexpr int ND = (2 * P * WSP + 4 * ((2 * P + 3) / 4) + 63) / 64;
    static_assert(64 * ND <= NZB, "the single-slot window fits a chunk buffer");
    static constexpr int RF = NCOMP * (64 + 2 * kHalo);   // x floats per group
    static constexpr int XF = 4 * RF;
    static constexpr int XL = (XF / 4 + 63) / 64;         // interior: 16-byte DMA loads per lane
    static constexpr int XBF = XL * 256;                  // x buffer floats (border: 4 XL dword loads)
    static constexpr int CHS = CG / NCOMP;                // channels per group and pass
    static constexpr int NZR = 2, NXB = NX;               // ring sizes
    static constexpr int XD = NX - 1;                     // x prefetch distance in steps
    static constexpr int NZR_SUMS = 4;                    // column sums: chunks 3 rows ahead
    // a lane's last x read may pass its row by 3 floats
    static constexpr int LDS = NZR * NZB + NXB * XBF + 4;
    static constexpr int LDS_SUMS = NZR_SUMS * NZB;
    static constexpr int EDGE = kHalo > 2 * P ? kHalo : 2 * P;  // interior margin
    static_assert(CHS >= 2, "the step waits assume two or more steps per window row");
    // a row's chunks are issued CHS steps ahead, at least as far as x, so the
    // wait for x(t) also covers the chunks read at step t
    static_assert(XD >= 2 && XD <= CHS, "x prefetch distance out of range");
};

// SUMS: column sums only (x = 1, no products): out[o] = sum of the staged
// coefficients, written to a.y (one float per pixel).  XV: x is staged in
// 16-byte pieces (interior tiles, and border tiles when n1 is a multiple of
// the 4 / NCOMP pixels of a piece, so that no piece straddles the wrap);
// otherwise float by float.  ZM (border tiles whose rotated chunks form one
// run): chunks in 16-byte pieces as in the interior, except the rotated ones
// (columns within p of the image border, whose slot order the reference
// shifts), which a window of single-slot loads over that run writes.
template <int WS, int NCOMP, bool TRANS, bool FAST, bool SUMS = false, bool XV = FAST, int CG = kCG,
          int NX = 3, bool ZM = false>
__device__ __forceinline__ void apply2_body(const ApplyArgs &a, int pass, int t1, int c2, int b) {
    using S = A2<WS, NCOMP, TRANS, CG, NX>;
    constexpr int P = S::P;
    constexpr int K = WS * WS;
    constexpr int XW = kR + 2 * P;
    constexpr int AL = (NCOMP * (kHalo - P)) % 4;
    constexpr int KW4 = (NCOMP * XW + AL + 3) / 4;
    static_assert(!ZM || (!FAST && (XV || SUMS)), "mixed chunk loads are a border form");
    constexpr int ND = ZM ? S::ND : 0;              // single-slot loads per lane (mixed form)
    constexpr int ZI = FAST ? S::NZ4 : ZM ? S::NZ4 + ND : S::NZ1;  // chunk loads per lane and row
    constexpr int XI = XV ? S::XL : 4 * S::XL;      // x loads per lane and step
    // (column sums: one row fewer ahead where three rows of loads would
    // exceed the vmcnt field)
    constexpr int NZR = !SUMS ? S::NZR : ((S::NZR_SUMS - 1) * ZI < 64 ? S::NZR_SUMS : 3);
    constexpr int T = WS * S::CHS;                  // steps
    static_assert(ZI + (S::XD - 1) * XI < 64 && (NZR - 1) * ZI < 64, "waits exceed vmcnt");
    typedef __attribute__((address_space(3))) void *lptr;
    const Geom &g = a.g;
    const int n1 = g.n1, n2 = g.n2;
    const int64_t Pp = g.P;
    const int lane = threadIdx.x & 63;
    const int l16 = lane & 15, grp = lane >> 4;
    const int f1 = t1 * 64;
    float *lz = circatt_lds_apply;   // chunk ring
    float *lx = lz + NZR * S::NZB;   // x ring
    const auto rs = rsrc(a.nz + (int64_t)b * Pp * K, Pp * K * 4);
    const int ubytes = (int)(Pp * NCOMP * a.C * 4);
    const auto rx = rsrc(a.x + (int64_t)b * Pp * NCOMP * a.C, ubytes);
    const int plane = (int)(NCOMP * Pp * 4);  // bytes per channel
    const int s2own = slot_shift(c2 + 1, n2, P);

    // Chunk DMA into lz[w * WSP + 4 (w / 4) + j] = slot j of chunk w (source
    // column f1 - off + w, wrapped), in the order of window offsets: near the border
    // of dim 1 the reference's circular shift of the slot order is undone
    // here, by the element each lane loads, so the reads below use constant
    // offsets in both bodies.  The interior body loads 16-byte pieces (the
    // last piece of a chunk reads past it into the next chunk, or past the
    // unit, where the range check returns zeros); the border body loads
    // single slots.  A lane's byte offset within an image row of nzVal does
    // not depend on the window row.
    int zo[ZI];
    bool zon[ZM ? S::NZ4 : 1];  // mixed form: the piece's chunk is not rotated (or the lane's slot is a gap)
#pragma unroll
    for (int m = 0; m < (ZM ? S::NZ4 : ZI); ++m) {
        const int off = TRANS ? P : 0;
        // LDS slot of this lane's piece -> (chunk w, piece q); free slots and
        // pieces past the last chunk load chunk 0 / the last chunk (unused)
        const int f = FAST || ZM ? lane + 64 * m : (lane + 64 * m) >> 2;
        const int kb = f / S::BLK, r = f - kb * S::BLK;
        const int rq = r < 4 * S::Q ? r : 0;
        const int w = min(4 * kb + rq / S::Q, S::NSRC - 1), q = rq - (rq / S::Q) * S::Q;
        if (FAST) {
            zo[m] = ((f1 - off + w) * K + 4 * q) * 4;
        } else if (ZM) {
            const int col = pmod(f1 - off + w, n1);
            zo[m] = (col * K + 4 * q) * 4;
            zon[m] = r >= 4 * S::Q || shift0(col, n1, P) == 0;
        } else {
            const int j = 4 * q + ((lane + 64 * m) & 3);
            const int col = pmod(f1 - off + w, n1);
            const int e = fold((j < WS ? j : 0) + shift0(col, n1, P), WS);
            zo[m] = (col * K + e) * 4;
        }
    }
    // Mixed form: the rotated chunks are those of columns n1 - p .. n1 + p - 1
    // (mod n1), one run [a0, a0 + 2p) of chunk indices clipped to the staged
    // ones (n1 >= NSRC + 2p, so the run does not wrap).  The single-slot
    // window covers ND x 64 floats from the run's first slot (moved back to
    // stay inside the buffer); each of its lanes loads the element its LDS
    // float holds in either form (the rotation of a chunk not in the run is
    // zero, so there it writes what the piece loads write).
    int zbase = 0;
    if constexpr (ZM) {
        const int off = TRANS ? P : 0;
        const int c0 = pmod(f1 - off, n1);
        const int d = pmod(n1 - P - c0, n1);
        const int a0 = d < S::NSRC ? d : 0;
        zbase = __builtin_amdgcn_readfirstlane(min(a0 * S::WSP + 4 * (a0 >> 2), S::NZB - 64 * ND));
#pragma unroll
        for (int i = 0; i < ND; ++i) {
            const int ps = zbase + 64 * i + lane;     // LDS float
            const int sl = ps >> 2, kb = sl / S::BLK, r = sl - kb * S::BLK;
            const int w = 4 * kb + r / S::Q;
            const int j = 4 * (r - (r / S::Q) * S::Q) + (ps & 3);
            int e = 0, col = 0;
            if (r < 4 * S::Q && w < S::NSRC) {
                col = pmod(f1 - off + w, n1);
                e = j < WS ? fold(j + shift0(col, n1, P), WS) : 0;
            }
            zo[S::NZ4 + i] = (col * K + e) * 4;
        }
    }
    // image row and chunk index of window row dd
    auto zrow = [&](int dd, int &r2, int &mm) {
        if (TRANS) {
            const int d2 = dd - P;  // output row - source row
            r2 = pmod(c2 - d2, n2);
            mm = pmod(dd + slot_shift(r2 + 1, n2, P), WS);
        } else {
            r2 = c2;
            mm = pmod(dd + s2own, WS);
        }
    };
    auto stage_z = [&](int dd, int buf) {
        int r2, mm;
        zrow(dd, r2, mm);
        // the whole offset is in the vector operand, which the range check sees
        const int so = __builtin_amdgcn_readfirstlane((n1 * r2 * K + mm * WS) * 4);
        float *dst = lz + buf * S::NZB;
        if constexpr (ZM) {
            // pieces of the chunks not rotated (every instruction has gap
            // lanes, which stay active, so each is issued), then the window
#pragma unroll
            for (int m = 0; m < S::NZ4; ++m) {
                __builtin_amdgcn_sched_barrier(0);
                if (zon[m])
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lptr)(dst + 256 * m), 16,
                                                            zo[m] + so, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < ND; ++i) {
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lptr)(dst + zbase + 64 * i), 4,
                                                        zo[S::NZ4 + i] + so, 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            return;
        }
#pragma unroll
        for (int m = 0; m < ZI; ++m) {
            __builtin_amdgcn_sched_barrier(0);
            if (FAST)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lptr)(dst + 256 * m), 16, zo[m] + so,
                                                        0, 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lptr)(dst + 64 * m), 4, zo[m] + so, 0,
                                                        0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // x DMA into lx[grp * RF + NCOMP * w + e] (column f1 - kHalo + w of the
    // step's channel of group grp): lane value (16-byte piece, or float in
    // the border body) f of group gs = f / RF.  A group's channels past C lie
    // past the unit's bytes: the range check makes their reads zero (they
    // are never stored).
    const int ch0 = pass * (4 * CG / NCOMP);  // first channel of the pass
    int xo[XI];
#pragma unroll
    for (int m = 0; m < XI; ++m) {
        const int f = XV ? 4 * (lane + 64 * m) : lane + 64 * m;
        const int fr = f < S::XF ? f : 0;
        const int gs = fr / S::RF, w = fr - gs * S::RF;
        const int chan = (ch0 + gs * S::CHS) * plane;
        if (FAST) {
            xo[m] = chan + (NCOMP * (f1 - kHalo) + w) * 4;
        } else {
            // (with XV, w is the first float of a piece: e = 0 and the piece's
            // pixels are consecutive columns)
            const int u = w / NCOMP, e = w - u * NCOMP;
            xo[m] = chan + (NCOMP * pmod(f1 - kHalo + u, n1) + e) * 4;
        }
    }
    auto stage_x = [&](int t, int buf) {
        const int dd = t / S::CHS, cl = t - dd * S::CHS;
        int r2, mm;
        if (TRANS)
            zrow(dd, r2, mm);
        else
            r2 = pmod(c2 + dd - P, n2);
        const int so = __builtin_amdgcn_readfirstlane(NCOMP * n1 * r2 * 4 + cl * plane);
        float *dst = lx + buf * S::XBF;
#pragma unroll
        for (int m = 0; m < XI; ++m) {
            __builtin_amdgcn_sched_barrier(0);
            if (XV)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lptr)(dst + 256 * m), 16, xo[m] + so,
                                                        0, 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lptr)(dst + 64 * m), 4, xo[m] + so, 0,
                                                        0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    float acc[kR][CG];
    float asum[kR];
#pragma unroll
    for (int i = 0; i < kR; ++i) {
        asum[i] = 0.f;
#pragma unroll
        for (int k = 0; k < CG; ++k) acc[i][k] = 0.f;
    }
    // the lane's 4 x ws coefficients of window row dd, from chunk buffer zb
    auto read_av = [&](float (&av)[kR][WS], int zb) {
        const float *src = lz + zb * S::NZB;
#pragma unroll
        for (int i = 0; i < kR; ++i)
#pragma unroll
            for (int j = 0; j < WS; ++j) {
                // chunk u = 4 l16 + c (c >= 0): block l16 + c / 4
                const int c = TRANS ? i - j + 2 * P : i;
                av[i][j] = src[(4 * l16 + c) * S::WSP + 4 * (l16 + c / 4) + j];
            }
    };

    if (SUMS) {
        // chunks NZR - 1 rows ahead; at row dd the loads of rows
        // dd + 1 .. min(WS - 1, dd + NZR - 1) may stay in flight
#pragma unroll
        for (int r = 0; r < NZR - 1; ++r)
            if (r < WS) stage_z(r, r);
#pragma unroll 1
        for (int dd = 0; dd < WS; ++dd) {
            __builtin_amdgcn_s_waitcnt(kWaitLgkm);  // row dd - 1's reads are done
            if (dd + NZR - 1 < WS) stage_z(dd + NZR - 1, (dd + NZR - 1) % NZR);
            const int younger = min(NZR - 1, WS - 1 - dd);
            if (younger >= 3)
                wait_vm<(NZR > 3 ? 3 : 2) * ZI>();  // only reached when NZR > 3
            else if (younger == 2)
                wait_vm<2 * ZI>();
            else if (younger == 1)
                wait_vm<ZI>();
            else
                wait_vm<0>();
            float av[kR][WS];
            read_av(av, dd % NZR);
#pragma unroll
            for (int i = 0; i < kR; ++i)
#pragma unroll
                for (int j = 0; j < WS; ++j) asum[i] += av[i][j];
        }
        // every lane group holds the same sums; group 0 stores them
        float *ob = a.y + (int64_t)b * Pp;
        const int col0 = f1 + 4 * l16;
        float *dst = ob + col0 + (int64_t)n1 * c2;
        if (grp == 0) {
            if (col0 + kR <= n1) {
                *(f4u *)dst = f4{asum[0], asum[1], asum[2], asum[3]};
            } else {
#pragma unroll
                for (int i = 0; i < kR; ++i)
                    if (col0 + i < n1) dst[i] = asum[i];
            }
        }
        return;
    }

    // issue order: chunks(0), x(0) .. x(XD - 1); step t issues
    // [chunks(dd + 1) if cl == 0] then x(t + XD).  Loads issued after x(t):
    // chunks(dd + 1) when 1 <= cl < XD, and x(t + 1) .. x(t + XD - 1) (those
    // before T).  chunks(dd), issued CHS >= XD steps before row dd, precede
    // x(t) at cl == 0.
    constexpr int XD = S::XD;
    stage_z(0, 0);
#pragma unroll
    for (int u = 0; u < XD; ++u)
        if (u < T) stage_x(u, u);
    int xb = 0;  // x buffer of step t (t % NXB)
    float av[kR][WS];
#pragma unroll 1
    for (int dd = 0; dd < WS; ++dd) {
        // priority 1 over the first three quarters of the window rows, 0 over
        // the last (cfg5 on gfx950, interleaved A/B: transposed apply 142 ->
        // 139 us, pullback 270 -> 264 us; the forward apply unchanged)
        if (dd == 0) __builtin_amdgcn_s_setprio(1);
        if (dd == (3 * WS) / 4) __builtin_amdgcn_s_setprio(0);
#pragma unroll
        for (int cl = 0; cl < S::CHS; ++cl) {
            const int t = dd * S::CHS + cl;
            __builtin_amdgcn_sched_barrier(0);
            const bool zy = cl >= 1 && cl < XD && dd + 1 < WS;
            const int nx = min(XD - 1, T - 1 - t);  // x loads issued after x(t)
            if (zy)
                wait_vm_steps<ZI, XI, XD - 1>(nx);
            else
                wait_vm_steps<0, XI, XD - 1>(nx);
            if (cl == 0) {
                // chunks(dd) arrived before x(t), which was issued after them
                read_av(av, dd & 1);
                if (a.corr) {
#pragma unroll
                    for (int i = 0; i < kR; ++i)
#pragma unroll
                        for (int j = 0; j < WS; ++j) asum[i] += av[i][j];
                }
            }
            // the buffers refilled below were last read one step (x) or one
            // row (chunks) ago; those reads are complete
            __builtin_amdgcn_s_waitcnt(kWaitLgkm);
            if (cl == 0 && dd + 1 < WS) stage_z(dd + 1, (dd + 1) & 1);
            if (t + XD < T) stage_x(t + XD, xb == 0 ? S::NXB - 1 : xb - 1);
            float xw[4 * KW4];
            const float *xr = lx + xb * S::XBF + grp * S::RF + NCOMP * (4 * l16 + kHalo - P) - AL;
#pragma unroll
            for (int h = 0; h < KW4; ++h) {
                const f4 v = *(const f4 *)(xr + 4 * h);
                xw[4 * h] = v[0];
                xw[4 * h + 1] = v[1];
                xw[4 * h + 2] = v[2];
                xw[4 * h + 3] = v[3];
            }
#pragma unroll
            for (int i = 0; i < kR; ++i)
#pragma unroll
                for (int j = 0; j < WS; ++j)
#pragma unroll
                    for (int e = 0; e < NCOMP; ++e)
                        acc[i][NCOMP * cl + e] = __builtin_fmaf(
                            av[i][j], xw[AL + NCOMP * (TRANS ? i - j + 2 * P : i + j) + e],
                            acc[i][NCOMP * cl + e]);
            // the step's products complete here, before the next step's loads
            // and reads (otherwise every step's run is read up front and held)
#pragma unroll
            for (int i = 0; i < kR; ++i)
#pragma unroll
                for (int e = 0; e < NCOMP; ++e) asm volatile("" : "+v"(acc[i][NCOMP * cl + e]));
            xb = xb == S::NXB - 1 ? 0 : xb + 1;
        }
    }
    // group grp stores channels ch0 + grp CHS + cl: 4 pixels x NCOMP
    // consecutive floats per lane, 16 lanes per contiguous run
    float *yb = a.y + (int64_t)b * Pp * NCOMP * a.C;
    const float *zb = a.z ? a.z + (int64_t)b * Pp * NCOMP * a.C : nullptr;
    const int col0 = f1 + 4 * l16;
    const int64_t pix0 = col0 + (int64_t)n1 * c2;
#pragma unroll
    for (int cl = 0; cl < S::CHS; ++cl) {
        const int ch = ch0 + grp * S::CHS + cl;
        if (ch >= a.C) break;
        float v[kR * NCOMP];
#pragma unroll
        for (int i = 0; i < kR; ++i)
#pragma unroll
            for (int e = 0; e < NCOMP; ++e) v[NCOMP * i + e] = acc[i][NCOMP * cl + e];
        float *dst = yb + NCOMP * (pix0 + Pp * ch);
        const float *zs = a.corr ? zb + NCOMP * (pix0 + Pp * ch) : nullptr;
        if (col0 + kR <= n1) {
#pragma unroll
            for (int h = 0; h < NCOMP; ++h) {
                f4 r = f4{v[4 * h], v[4 * h + 1], v[4 * h + 2], v[4 * h + 3]};
                if (a.corr) {
                    const f4u z = *(const f4u *)(zs + 4 * h);
#pragma unroll
                    for (int q = 0; q < 4; ++q) r[q] -= asum[(4 * h + q) / NCOMP] * z[q];
                }
                *(f4u *)(dst + 4 * h) = r * a.scale;
            }
        } else {
#pragma unroll
            for (int i = 0; i < kR; ++i) {
                if (col0 + i >= n1) break;
#pragma unroll
                for (int e = 0; e < NCOMP; ++e) {
                    float r = v[NCOMP * i + e];
                    if (a.corr) r -= asum[i] * zs[NCOMP * i + e];
                    dst[NCOMP * i + e] = r * a.scale;
                }
            }
        }
    }
}

// the body for tile column t1: interior, border with 16-byte x pieces, or
// border float by float
template <int WS, int NCOMP, bool TRANS, bool SUMS, int CG = kCG, int NX = 3>
__device__ __forceinline__ void apply2_tile(const ApplyArgs &a, int pass, int t1, int c2, int b) {
    using S = A2<WS, NCOMP, TRANS, CG, NX>;
    const bool xv = !SUMS && a.g.n1 % (4 / NCOMP) == 0;
    if (t1 >= a.fa && t1 < a.fb) {
        apply2_body<WS, NCOMP, TRANS, true, SUMS, true, CG, NX>(a, pass, t1, c2, b);
        return;
    }
    if (a.g.n1 >= S::NSRC + 2 * S::P) {
        // (column sums stage no x)
        if constexpr (SUMS) {
            apply2_body<WS, NCOMP, TRANS, false, SUMS, false, CG, NX, true>(a, pass, t1, c2, b);
            return;
        } else if (xv) {
            apply2_body<WS, NCOMP, TRANS, false, SUMS, true, CG, NX, true>(a, pass, t1, c2, b);
            return;
        }
    }
    if (xv)
        apply2_body<WS, NCOMP, TRANS, false, SUMS, true, CG, NX>(a, pass, t1, c2, b);
    else
        apply2_body<WS, NCOMP, TRANS, false, SUMS, false, CG, NX>(a, pass, t1, c2, b);
}

// One wavefront per (64 output pixels of an image row, component pass, unit);
// work items in XCD bands as in sim_rows_kernel.
template <int WS, int NCOMP, bool TRANS, bool SUMS = false, int CG = kCG, int NX = 3>
__global__ __launch_bounds__(64, 2) void apply2_kernel(ApplyArgs a, int nwork) {
    const int nper = (nwork + 7) >> 3;
    int it = (int)(blockIdx.x & 7) * nper + (int)(blockIdx.x >> 3);
    if (it >= nwork) return;
    const int pass = __builtin_amdgcn_readfirstlane(it % a.gchunk);
    it /= a.gchunk;
    const int t1 = __builtin_amdgcn_readfirstlane(it % a.tiles1);
    it /= a.tiles1;
    const int c2 = __builtin_amdgcn_readfirstlane(it % a.g.n2);
    const int b = __builtin_amdgcn_readfirstlane(it / a.g.n2);
    apply2_tile<WS, NCOMP, TRANS, SUMS, CG, NX>(a, pass, t1, c2, b);
}

// The similarity pullback's two products in one grid: work items
// [0, nwork) are A ⊗ y (args af), [nwork, 2 nwork) are Aᵀ ⊗ x (args at), each
// half in XCD bands, so that the two share the GPU instead of running one
// after the other.
template <int WS, int NCOMP, int NX = 3>
__global__ __launch_bounds__(64, 2) void apply2_pair_kernel(ApplyArgs af, ApplyArgs at, int nwork) {
    const int nall = 2 * nwork;
    const int nper = (nall + 7) >> 3;
    int it = (int)(blockIdx.x & 7) * nper + (int)(blockIdx.x >> 3);
    if (it >= nall) return;
    const bool trans = it >= nwork;
    if (trans) it -= nwork;
    const ApplyArgs &a = trans ? at : af;
    const int pass = __builtin_amdgcn_readfirstlane(it % a.gchunk);
    it /= a.gchunk;
    const int t1 = __builtin_amdgcn_readfirstlane(it % a.tiles1);
    it /= a.tiles1;
    const int c2 = __builtin_amdgcn_readfirstlane(it % a.g.n2);
    const int b = __builtin_amdgcn_readfirstlane(it / a.g.n2);
    if (trans)
        apply2_tile<WS, NCOMP, true, false, kCG, NX>(at, pass, t1, c2, b);
    else
        apply2_tile<WS, NCOMP, false, false, kCG, NX>(af, pass, t1, c2, b);
}

// ---------------------------------------------------------------------------
// Wide windows (any odd ws, 1D or 2D; apply_wide_kernel): as apply2_kernel,
// with every window row (the whole window in 1D) split into sub-rows of kJC
// window columns.  Sub-row (dd, jc) covers slots j0 = kJC jc .. j0 + kJC - 1
// of window row dd (horizontal offsets h = j0 + j - p) and is processed like
// a window row of width kJC: per sub-row the wavefront stages one 16-float
// sub-chunk of every pixel involved (64, or 64 + kJC - 1 source pixels for
// the transposed product), and per step the x row's 80 columns that its
// lanes' runs of 4 + kJC - 1 pixels cover.  Slots past the window (the last
// sub-row of a row) are read as zeros.  ws and the dimension are run-time
// values.
// ---------------------------------------------------------------------------

template <int NCOMP, bool TRANS>
struct AW {
    static constexpr int NSRC = TRANS ? 64 + kJC - 1 : 64;  // staged sub-chunks
    static constexpr int Q = kJC / 4;                       // 16-byte pieces per sub-chunk
    static constexpr int BLK = 4 * Q + 1;                   // slots per block of 4 (skewed)
    static constexpr int NSLOT = (NSRC + 3) / 4 * BLK;
    static constexpr int NZ4 = (NSLOT + 63) / 64;
    static constexpr int NZ1 = (4 * NSLOT + 63) / 64;
    static constexpr int NZB = NZ4 * 256 > NZ1 * 64 ? NZ4 * 256 : NZ1 * 64;
    static constexpr int RW = 64 + kJC;                     // staged x columns
    static constexpr int RF = NCOMP * RW;
    static constexpr int XF = 4 * RF;
    static constexpr int XL = (XF / 4 + 63) / 64;
    static constexpr int XBF = XL * 256;
    static constexpr int CHS = kCG / NCOMP;
    static constexpr int NZR = 2, NXB = kNX;
    static constexpr int XD = NXB - 1;
    static constexpr int LDS = NZR * NZB + NXB * XBF + 4;
    static constexpr int LDS_SUMS = 4 * NZB;
    static_assert(CHS >= 2, "the step waits assume two or more steps per sub-row");
    static_assert(XD >= 2 && XD <= CHS, "x prefetch distance out of range");
};

// single-slot loads per lane of the wide kernel's mixed border form: the LDS
// span of a run of 30 sub-chunks (windows up to 31)
constexpr int kWideMixP = 15;
constexpr int kNDW = (2 * kWideMixP * kJC + 4 * ((2 * kWideMixP + 3) / 4) + 63) / 64;

// ZM: border tiles in the mixed form of apply2_body (sub-chunks of columns
// whose slot order is not rotated in 16-byte pieces, a window of single-slot
// loads over the run of rotated ones); p <= kWideMixP and n1 >= NSRC + 2p
template <int NCOMP, bool TRANS, bool FAST, bool SUMS, bool ZM = false>
__device__ __forceinline__ void apply_wide_body(const ApplyArgs &a, int pass, int t1, int c2,
                                                int b) {
    using S = AW<NCOMP, TRANS>;
    constexpr int KW4 = (NCOMP * (kR + kJC - 1) + 3) / 4;
    static_assert(!ZM || !FAST, "mixed chunk loads are a border form");
    static_assert(64 * kNDW <= S::NZB, "the single-slot window fits a chunk buffer");
    constexpr int ZI = FAST ? S::NZ4 : ZM ? S::NZ4 + kNDW : S::NZ1;
    constexpr int XI = FAST ? S::XL : 4 * S::XL;
    constexpr int NZR = !SUMS ? S::NZR : (3 * ZI < 64 ? 4 : 3);
    static_assert(ZI + (S::XD - 1) * XI < 64 && (NZR - 1) * ZI < 64, "waits exceed vmcnt");
    typedef __attribute__((address_space(3))) void *lptr;
    const Geom &g = a.g;
    const int WS = g.ws, P = g.p, K = g.K;
    const bool two = g.nsp == 2;
    const int n1 = g.n1, n2 = two ? g.n2 : 1;
    const int WR = two ? WS : 1;              // window rows
    const int NJC = (WS + kJC - 1) / kJC;     // sub-rows per window row
    const int NSR = WR * NJC;                 // sub-rows
    const int64_t Pp = g.P;
    const int lane = threadIdx.x & 63;
    const int l16 = lane & 15, grp = lane >> 4;
    const int f1 = t1 * 64;
    float *lz = circatt_lds_apply;
    float *lx = lz + NZR * S::NZB;
    const auto rs = rsrc(a.nz + (int64_t)b * Pp * K, Pp * K * 4);
    const int ubytes = (int)(Pp * NCOMP * a.C * 4);
    const auto rx = rsrc(a.x + (int64_t)b * Pp * NCOMP * a.C, ubytes);
    const int plane = (int)(NCOMP * Pp * 4);
    const int s2own = two ? slot_shift(c2 + 1, n2, P) : 0;

    // first horizontal offset and first staged column (sub-chunks, x) of a
    // sub-row
    auto h0_of = [&](int jc) { return kJC * jc - P; };
    auto col0 = [&](int jc) { return TRANS ? f1 - h0_of(jc) - (kJC - 1) : f1; };
    auto xcol0 = [&](int jc) { return TRANS ? f1 - h0_of(jc) - (kJC - 1) : f1 + h0_of(jc); };
    // image row and chunk index of window row dd
    auto zrow = [&](int dd, int &r2, int &mm) {
        if (!two) {
            r2 = 0;
            mm = 0;
        } else if (TRANS) {
            r2 = pmod(c2 - (dd - P), n2);
            mm = pmod(dd + slot_shift(r2 + 1, n2, P), WS);
        } else {
            r2 = c2;
            mm = pmod(dd + s2own, WS);
        }
    };
    // interior body: the lane's piece of sub-chunk w (LDS slot layout as in
    // apply2_kernel), relative to the sub-row's first column and slot
    int zo[ZI];
    if (FAST) {
#pragma unroll
        for (int m = 0; m < ZI; ++m) {
            const int f = lane + 64 * m;
            const int kb = f / S::BLK, r = f - kb * S::BLK;
            const int rq = r < 4 * S::Q ? r : 0;
            const int w = min(4 * kb + rq / S::Q, S::NSRC - 1), q = rq - (rq / S::Q) * S::Q;
            zo[m] = (w * K + 4 * q) * 4;
        }
    }
    // border body: single slots, rotated by the column's slot shift; the
    // offsets depend on the sub-row and are formed when it is staged
    auto zo_border = [&](int m, int jc) {
        const int f = (lane + 64 * m) >> 2;
        const int kb = f / S::BLK, r = f - kb * S::BLK;
        const int rq = r < 4 * S::Q ? r : 0;
        const int w = min(4 * kb + rq / S::Q, S::NSRC - 1), q = rq - (rq / S::Q) * S::Q;
        const int j = kJC * jc + 4 * q + ((lane + 64 * m) & 3);
        const int col = pmod(col0(jc) + w, n1);
        const int e = j < WS ? fold(j + shift0(col, n1, P), WS) : 0;
        return (col * K + e) * 4;
    };
    // mixed form: offsets of sub-row column jc (relative to the row's first
    // slot), the window's first LDS float and the piece lanes' enable bits.
    // The rotated columns n1 - p .. n1 + p - 1 (mod n1) form one run of
    // sub-chunks; each window lane loads what its LDS float holds in either
    // form.  With n1 >= NSRC + 2p every column lies in [-n1, 2 n1), so one
    // conditional step wraps it.
    auto wrap1 = [&](int x) { return x < 0 ? x + n1 : (x >= n1 ? x - n1 : x); };
    auto zm_make = [&](int jc, int (&zm)[ZI], int &zb, int &on) {
        const int c0 = col0(jc);
        on = 0;
#pragma unroll
        for (int m = 0; m < S::NZ4; ++m) {
            const int f = lane + 64 * m;
            const int kb = f / S::BLK, r = f - kb * S::BLK;
            const int rq = r < 4 * S::Q ? r : 0;
            const int w = min(4 * kb + rq / S::Q, S::NSRC - 1), q = rq - (rq / S::Q) * S::Q;
            const int col = wrap1(c0 + w);
            zm[m] = (col * K + kJC * jc + 4 * q) * 4;
            if (r >= 4 * S::Q || shift0(col, n1, P) == 0) on |= 1 << m;
        }
        const int d = wrap1(n1 - P - wrap1(c0));
        const int a0 = d < S::NSRC ? d : 0;
        zb = __builtin_amdgcn_readfirstlane(min(a0 * kJC + 4 * (a0 >> 2), S::NZB - 64 * kNDW));
#pragma unroll
        for (int i = 0; i < kNDW; ++i) {
            const int ps = zb + 64 * i + lane;
            const int sl = ps >> 2, kb = sl / S::BLK, r = sl - kb * S::BLK;
            const int w = 4 * kb + r / S::Q;
            const int j = kJC * jc + 4 * (r - (r / S::Q) * S::Q) + (ps & 3);
            int e = 0, col = 0;
            if (r < 4 * S::Q && w < S::NSRC) {
                col = wrap1(c0 + w);
                e = j < WS ? fold(j + shift0(col, n1, P), WS) : 0;
            }
            zm[S::NZ4 + i] = (col * K + e) * 4;
        }
    };
    int zmo[ZM && SUMS ? 2 : 1][ZM && SUMS ? ZI : 1], zmb[2] = {0, 0}, zmon[2] = {0, 0};
    if constexpr (ZM && SUMS) {
        zm_make(0, zmo[0], zmb[0], zmon[0]);
        if (NJC > 1) zm_make(1, zmo[1], zmb[1], zmon[1]);
    }
    auto stage_z = [&](int sr, int buf) {
        const int dd = sr / NJC, jc = sr - dd * NJC;
        int r2, mm;
        zrow(dd, r2, mm);
        float *dst = lz + buf * S::NZB;
        if (FAST) {
            const int so = __builtin_amdgcn_readfirstlane(
                ((n1 * r2 + col0(jc)) * K + mm * WS + kJC * jc) * 4);
#pragma unroll
            for (int m = 0; m < ZI; ++m) {
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lptr)(dst + 256 * m), 16, zo[m] + so,
                                                        0, 0, 0);
            }
        } else if constexpr (ZM) {
            const int so = __builtin_amdgcn_readfirstlane((n1 * r2 * K + mm * WS) * 4);
            int zm[ZI], zb, on;
            if constexpr (SUMS) {
                // formed once per item (windows up to 31 have two sub-rows)
                zb = jc == 0 ? zmb[0] : zmb[1];
                on = jc == 0 ? zmon[0] : zmon[1];
#pragma unroll
                for (int m = 0; m < ZI; ++m) zm[m] = jc == 0 ? zmo[0][m] : zmo[1][m];
            } else {
                zm_make(jc, zm, zb, on);
            }
            // pieces of the sub-chunks whose columns are not rotated (gap
            // lanes stay active, so every instruction is issued), then the
            // window over the run of rotated ones
#pragma unroll
            for (int m = 0; m < S::NZ4; ++m) {
                __builtin_amdgcn_sched_barrier(0);
                if ((on >> m) & 1)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lptr)(dst + 256 * m), 16, zm[m] + so,
                                                            0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < kNDW; ++i) {
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lptr)(dst + zb + 64 * i), 4,
                                                        zm[S::NZ4 + i] + so, 0, 0, 0);
            }
        } else {
            const int so = __builtin_amdgcn_readfirstlane((n1 * r2 * K + mm * WS) * 4);
#pragma unroll
            for (int m = 0; m < ZI; ++m) {
                const int vo = zo_border(m, jc) + so;
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lptr)(dst + 64 * m), 4, vo, 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // x: group gs's channel ch0 + gs CHS + cl, columns xcol0 .. xcol0 + RW - 1
    const int ch0 = pass * (kCPass / NCOMP);
    int xo[XI];
#pragma unroll
    for (int m = 0; m < XI; ++m) {
        const int f = FAST ? 4 * (lane + 64 * m) : lane + 64 * m;
        const int fr = f < S::XF ? f : 0;
        const int gs = fr / S::RF, w = fr - gs * S::RF;
        xo[m] = (ch0 + gs * S::CHS) * plane + (FAST ? w * 4 : 0);
    }
    auto stage_x = [&](int t, int buf) {
        const int sr = t / S::CHS, cl = t - sr * S::CHS;
        const int dd = sr / NJC, jc = sr - dd * NJC;
        int r2, mm;
        if (TRANS)
            zrow(dd, r2, mm);
        else
            r2 = two ? pmod(c2 + dd - P, n2) : 0;
        float *dst = lx + buf * S::XBF;
        if (FAST) {
            const int so = __builtin_amdgcn_readfirstlane(NCOMP * (n1 * r2 + xcol0(jc)) * 4 +
                                                          cl * plane);
#pragma unroll
            for (int m = 0; m < XI; ++m) {
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lptr)(dst + 256 * m), 16, xo[m] + so,
                                                        0, 0, 0);
            }
        } else {
            const int so = __builtin_amdgcn_readfirstlane(NCOMP * n1 * r2 * 4 + cl * plane);
            const int xc = xcol0(jc);
#pragma unroll
            for (int m = 0; m < XI; ++m) {
                const int f = lane + 64 * m;
                const int fr = f < S::XF ? f : 0;
                const int w = fr - (fr / S::RF) * S::RF, u = w / NCOMP, e = w - u * NCOMP;
                const int vo = xo[m] + (NCOMP * pmod(xc + u, n1) + e) * 4 + so;
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lptr)(dst + 64 * m), 4, vo, 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    float acc[kR][kCG];
    float asum[kR];
#pragma unroll
    for (int i = 0; i < kR; ++i) {
        asum[i] = 0.f;
#pragma unroll
        for (int k = 0; k < kCG; ++k) acc[i][k] = 0.f;
    }
    // the lane's 4 x kJC coefficients of sub-row sr (zero past the window)
    auto read_av = [&](float (&av)[kR][kJC], int zb, int sr) {
        const int jn = WS - kJC * (sr % NJC);
        const float *src = lz + zb * S::NZB;
#pragma unroll
        for (int i = 0; i < kR; ++i)
#pragma unroll
            for (int j = 0; j < kJC; ++j) {
                const int c = TRANS ? i - j + kJC - 1 : i;
                const float v = src[(4 * l16 + c) * kJC + 4 * (l16 + c / 4) + j];
                av[i][j] = j < jn ? v : 0.f;
            }
    };

    if (SUMS) {
#pragma unroll
        for (int r = 0; r < NZR - 1; ++r)
            if (r < NSR) stage_z(r, r);
#pragma unroll 1
        for (int sr = 0; sr < NSR; ++sr) {
            __builtin_amdgcn_s_waitcnt(kWaitLgkm);
            if (sr + NZR - 1 < NSR) stage_z(sr + NZR - 1, (sr + NZR - 1) % NZR);
            const int younger = min(NZR - 1, NSR - 1 - sr);
            if (younger >= 3)
                wait_vm<(NZR > 3 ? 3 : 2) * ZI>();
            else if (younger == 2)
                wait_vm<2 * ZI>();
            else if (younger == 1)
                wait_vm<ZI>();
            else
                wait_vm<0>();
            float av[kR][kJC];
            read_av(av, sr % NZR, sr);
#pragma unroll
            for (int i = 0; i < kR; ++i)
#pragma unroll
                for (int j = 0; j < kJC; ++j) asum[i] += av[i][j];
        }
        float *dst = a.y + (int64_t)b * Pp + f1 + 4 * l16 + (int64_t)n1 * c2;
        const int col0l = f1 + 4 * l16;
        if (grp == 0) {
            if (col0l + kR <= n1) {
                *(f4u *)dst = f4{asum[0], asum[1], asum[2], asum[3]};
            } else {
#pragma unroll
                for (int i = 0; i < kR; ++i)
                    if (col0l + i < n1) dst[i] = asum[i];
            }
        }
        return;
    }

    // issue order and waits as in apply2_body, over T = NSR x CHS steps
    const int T = NSR * S::CHS;
    constexpr int XD = S::XD;
    stage_z(0, 0);
#pragma unroll
    for (int u = 0; u < XD; ++u)
        if (u < T) stage_x(u, u);
    int xb = 0;
    float av[kR][kJC];
#pragma unroll 1
    for (int sr = 0; sr < NSR; ++sr) {
#pragma unroll
        for (int cl = 0; cl < S::CHS; ++cl) {
            const int t = sr * S::CHS + cl;
            __builtin_amdgcn_sched_barrier(0);
            const bool zy = cl >= 1 && cl < XD && sr + 1 < NSR;
            const int nx = min(XD - 1, T - 1 - t);  // x loads issued after x(t)
            if (zy)
                wait_vm_steps<ZI, XI, XD - 1>(nx);
            else
                wait_vm_steps<0, XI, XD - 1>(nx);
            if (cl == 0) {
                read_av(av, sr & 1, sr);
                if (a.corr) {
#pragma unroll
                    for (int i = 0; i < kR; ++i)
#pragma unroll
                        for (int j = 0; j < kJC; ++j) asum[i] += av[i][j];
                }
            }
            __builtin_amdgcn_s_waitcnt(kWaitLgkm);
            if (cl == 0 && sr + 1 < NSR) stage_z(sr + 1, (sr + 1) & 1);
            if (t + XD < T) stage_x(t + XD, xb == 0 ? S::NXB - 1 : xb - 1);
            float xw[4 * KW4];
            const float *xr = lx + xb * S::XBF + grp * S::RF + NCOMP * 4 * l16;
#pragma unroll
            for (int h = 0; h < KW4; ++h) {
                const f4 v = *(const f4 *)(xr + 4 * h);
                xw[4 * h] = v[0];
                xw[4 * h + 1] = v[1];
                xw[4 * h + 2] = v[2];
                xw[4 * h + 3] = v[3];
            }
#pragma unroll
            for (int i = 0; i < kR; ++i)
#pragma unroll
                for (int j = 0; j < kJC; ++j)
#pragma unroll
                    for (int e = 0; e < NCOMP; ++e)
                        acc[i][NCOMP * cl + e] = __builtin_fmaf(
                            av[i][j], xw[NCOMP * (TRANS ? i - j + kJC - 1 : i + j) + e],
                            acc[i][NCOMP * cl + e]);
#pragma unroll
            for (int i = 0; i < kR; ++i)
#pragma unroll
                for (int e = 0; e < NCOMP; ++e) asm volatile("" : "+v"(acc[i][NCOMP * cl + e]));
            xb = xb == S::NXB - 1 ? 0 : xb + 1;
        }
    }
    float *yb = a.y + (int64_t)b * Pp * NCOMP * a.C;
    const float *zb = a.z ? a.z + (int64_t)b * Pp * NCOMP * a.C : nullptr;
    const int colf = f1 + 4 * l16;
    const int64_t pix0 = colf + (int64_t)n1 * c2;
#pragma unroll
    for (int cl = 0; cl < S::CHS; ++cl) {
        const int ch = ch0 + grp * S::CHS + cl;
        if (ch >= a.C) break;
        float v[kR * NCOMP];
#pragma unroll
        for (int i = 0; i < kR; ++i)
#pragma unroll
            for (int e = 0; e < NCOMP; ++e) v[NCOMP * i + e] = acc[i][NCOMP * cl + e];
        float *dst = yb + NCOMP * (pix0 + Pp * ch);
        const float *zs = a.corr ? zb + NCOMP * (pix0 + Pp * ch) : nullptr;
        if (colf + kR <= n1) {
#pragma unroll
            for (int h = 0; h < NCOMP; ++h) {
                f4 r = f4{v[4 * h], v[4 * h + 1], v[4 * h + 2], v[4 * h + 3]};
                if (a.corr) {
                    const f4u z = *(const f4u *)(zs + 4 * h);
#pragma unroll
                    for (int q = 0; q < 4; ++q) r[q] -= asum[(4 * h + q) / NCOMP] * z[q];
                }
                *(f4u *)(dst + 4 * h) = r * a.scale;
            }
        } else {
#pragma unroll
            for (int i = 0; i < kR; ++i) {
                if (colf + i >= n1) break;
#pragma unroll
                for (int e = 0; e < NCOMP; ++e) {
                    float r = v[NCOMP * i + e];
                    if (a.corr) r -= asum[i] * zs[NCOMP * i + e];
                    dst[NCOMP * i + e] = r * a.scale;
                }
            }
        }
    }
}

// work item it (XCD-banded) -> (pass, tile column, image row, unit)
__device__ __forceinline__ void wide_item(const ApplyArgs &a, int it, int &pass, int &t1, int &c2,
                                          int &b) {
    pass = __builtin_amdgcn_readfirstlane(it % a.gchunk);
    it /= a.gchunk;
    t1 = __builtin_amdgcn_readfirstlane(it % a.tiles1);
    it /= a.tiles1;
    const int n2 = a.g.nsp == 2 ? a.g.n2 : 1;
    c2 = __builtin_amdgcn_readfirstlane(it % n2);
    b = __builtin_amdgcn_readfirstlane(it / n2);
}
template <int NCOMP, bool TRANS, bool SUMS>
__device__ __forceinline__ void apply_wide_tile(const ApplyArgs &a, int pass, int t1, int c2,
                                                int b) {
    if (t1 >= a.fa && t1 < a.fb)
        apply_wide_body<NCOMP, TRANS, true, SUMS>(a, pass, t1, c2, b);
    else if (a.g.p <= kWideMixP && a.g.n1 >= AW<NCOMP, TRANS>::NSRC + 2 * a.g.p)
        apply_wide_body<NCOMP, TRANS, false, SUMS, true>(a, pass, t1, c2, b);
    else
        apply_wide_body<NCOMP, TRANS, false, SUMS>(a, pass, t1, c2, b);
}

// One wavefront per (64 output pixels of an image row or of the line,
// component pass, unit); work items in XCD bands.
template <int NCOMP, bool TRANS, bool SUMS>
__global__ __launch_bounds__(64, 2) void apply_wide_kernel(ApplyArgs a, int nwork) {
    const int nper = (nwork + 7) >> 3;
    const int it = (int)(blockIdx.x & 7) * nper + (int)(blockIdx.x >> 3);
    if (it >= nwork) return;
    int pass, t1, c2, b;
    wide_item(a, it, pass, t1, c2, b);
    apply_wide_tile<NCOMP, TRANS, SUMS>(a, pass, t1, c2, b);
}

// The similarity pullback's two products in one grid (as apply2_pair_kernel)
template <int NCOMP>
__global__ __launch_bounds__(64, 2) void apply_wide_pair_kernel(ApplyArgs af, ApplyArgs at,
                                                                int nwork) {
    const int nall = 2 * nwork;
    const int nper = (nall + 7) >> 3;
    int it = (int)(blockIdx.x & 7) * nper + (int)(blockIdx.x >> 3);
    if (it >= nall) return;
    const bool trans = it >= nwork;
    if (trans) it -= nwork;
    int pass, t1, c2, b;
    wide_item(trans ? at : af, it, pass, t1, c2, b);
    if (trans)
        apply_wide_tile<NCOMP, true, false>(at, pass, t1, c2, b);
    else
        apply_wide_tile<NCOMP, false, false>(af, pass, t1, c2, b);
}

// geometry fields of the wide kernel (segments, interior range, passes)
template <int NCOMP, bool SUMS>
void set_wide(ApplyArgs &a) {
    const int n1 = a.g.n1;
    a.tiles1 = (n1 + 63) / 64;
    // interior segments: staged sub-chunk and x columns in range, no slot
    // shift (2p + kJC columns of margin on either side)
    const int edge = 2 * a.g.p + kJC;
    a.fa = (edge + 63) / 64;
    a.fb = n1 - 64 - edge >= 0 ? (n1 - 64 - edge) / 64 + 1 : 0;
    if (a.fb > a.tiles1) a.fb = a.tiles1;
    if (a.fb < a.fa) a.fb = a.fa;
    a.gchunk = SUMS ? 1 : (NCOMP * a.C + kCPass - 1) / kCPass;
}

template <int NCOMP>
hipError_t launch_wide_pair(ApplyArgs af, ApplyArgs at, int64_t nb, hipStream_t s) {
    set_wide<NCOMP, false>(af);
    set_wide<NCOMP, false>(at);
    const int64_t nwork = (int64_t)af.tiles1 * (af.g.nsp == 2 ? af.g.n2 : 1) * nb * af.gchunk;
    const size_t lds =
        (size_t)std::max(AW<NCOMP, false>::LDS, AW<NCOMP, true>::LDS) * sizeof(float);
    hipLaunchKernelGGL((apply_wide_pair_kernel<NCOMP>), dim3((unsigned)(8 * ((2 * nwork + 7) / 8))),
                       dim3(64), lds, s, af, at, (int)nwork);
    return hipGetLastError();
}

template <int NCOMP, bool TRANS, bool SUMS>
hipError_t launch_wide(ApplyArgs a, int64_t nb, hipStream_t s) {
    using S = AW<NCOMP, TRANS>;
    const int n2 = a.g.nsp == 2 ? a.g.n2 : 1;
    set_wide<NCOMP, SUMS>(a);
    const int64_t nwork = (int64_t)a.tiles1 * n2 * nb * a.gchunk;
    const size_t lds = (size_t)(SUMS ? S::LDS_SUMS : S::LDS) * sizeof(float);
    hipLaunchKernelGGL((apply_wide_kernel<NCOMP, TRANS, SUMS>), dim3((unsigned)(8 * ((nwork + 7) / 8))),
                       dim3(64), lds, s, a, (int)nwork);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Wide windows in 2D, workgroup form (apply_band_kernel).  Four wavefronts
// own four consecutive image rows c2 = kBR c2g + w of the same 64 columns and
// component pass, with the per-wavefront arithmetic of apply_wide_kernel
// (sub-rows of kJC window columns, lane groups splitting the components).
// The workgroup walks the kBR + 2p source rows its windows cover once: per
// source row the x row's columns for every component of the pass are staged
// by the four wavefronts together into a shared buffer (kBX columns, the
// union of every sub-row's runs), and each wavefront whose window covers that
// row runs its window row against its own staged coefficient chunks.  x thus
// crosses the vector memory path (kBR + 2p) / kBR times per output row
// instead of once per sub-row and component step, and the per-step staging
// arithmetic disappears; one barrier per source row hands the x buffers over.
//   forward:    source row u (0 .. kBR + 2p - 1) = kBR c2g - p + u serves
//               window row dd = u - w of wavefront w
//   transposed: the same source row serves window row dd = w + 2p - u (the
//               coefficients are the source row's pixels')
// ---------------------------------------------------------------------------
constexpr int kBR = 4;   // image rows (wavefronts) per workgroup
constexpr int kBX = 96;  // staged x columns per source row (16 NJC + 63 <= 96 for NJC <= 2)
constexpr int kBG = 8;   // real components per lane group and pass
constexpr int kBPass = 4 * kBG;
constexpr int kBZ = 1;   // chunk buffers per wavefront (chunks staged kBZ sub-rows ahead;
                         // two halve the workgroups per CU, which costs more)

template <int NCOMP, bool TRANS>
struct AB {
    using W = AW<NCOMP, TRANS>;
    static constexpr int XROW = NCOMP * kBX;            // floats per channel row
    static constexpr int CHS = kBG / NCOMP;             // channels per lane group and pass
    static constexpr int XF = kBPass / NCOMP * XROW;    // floats per source row
    static constexpr int PPW = XF / 4 / kBR;            // 16-byte pieces per wavefront
    static constexpr int XP = (PPW + 63) / 64;          // 16-byte loads per lane and wavefront
    static constexpr int XPL = PPW - 64 * (XP - 1);     // lanes of the last one
    static constexpr int X1 = XF / (64 * kBR);          // 4-byte loads per lane and wavefront
    // kBZ chunk buffers per wavefront: sub-row s's chunk goes to buffer
    // s % kBZ once sub-row s - kBZ's coefficients are in registers
    static constexpr int LDS = 2 * XF + kBR * kBZ * W::NZB;
    static_assert(XF % (64 * kBR) == 0 && XF % (16 * kBR) == 0,
                  "x floats and pieces split evenly over the wavefronts");
};

// first staged x column of a source row (the reads of every sub-row start at
// a multiple of 4 floats from it)
__host__ __device__ __forceinline__ int band_x0(bool trans, int f1, int p, int njc) {
    return trans ? f1 + p - kJC * (njc - 1) - (kJC - 1) : f1 - p;
}

template <int NCOMP, bool TRANS, bool FAST>
__device__ __forceinline__ void apply_band_body(const ApplyArgs &a, int pass, int t1, int c2g,
                                                int b) {
    using S = AW<NCOMP, TRANS>;
    using BB = AB<NCOMP, TRANS>;
    constexpr int KW4 = (NCOMP * (kR + kJC - 1) + 3) / 4;
    // chunk loads: NZ4 in the interior, NZ4 .. 4 NZ4 at the border (the
    // waits below allow NZ4 of them in flight, which waits for more than
    // needed when there are more)
    constexpr int ZI = S::NZ4;
    constexpr int XI = FAST ? BB::XP : BB::X1;
    static_assert(4 * ZI < 64 && XI < 64, "waits exceed vmcnt");
    typedef __attribute__((address_space(3))) void *lptr;
    const Geom &g = a.g;
    const int WS = g.ws, P = g.p, K = g.K;
    const int n1 = g.n1, n2 = g.n2;
    const int NJC = (WS + kJC - 1) / kJC;
    const int NSR = WS * NJC;           // own sub-rows
    const int NU = kBR + 2 * P;         // source rows of the workgroup
    const int64_t Pp = g.P;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int l16 = lane & 15, grp = lane >> 4;
    const int f1 = t1 * 64;
    const int c2 = c2g * kBR + w;
    const bool live = c2 < n2;
    float *lxs = circatt_lds_apply;                        // 2 shared x buffers
    float *lz = lxs + 2 * BB::XF + w * kBZ * S::NZB;       // own chunk buffers
    const auto rs = rsrc(a.nz + (int64_t)b * Pp * K, Pp * K * 4);
    const int ubytes = (int)(Pp * NCOMP * a.C * 4);
    const auto rx = rsrc(a.x + (int64_t)b * Pp * NCOMP * a.C, ubytes);
    const int plane = (int)(NCOMP * Pp * 4);
    const int s2own = slot_shift(c2 + 1, n2, P);
    const int r0 = kBR * c2g - P;   // source row of u = 0 (before wrapping)
    const int ch0 = pass * (kBPass / NCOMP);
    const int X0 = band_x0(TRANS, f1, P, NJC);

    // ---- coefficient chunks (as apply_wide_body) ----
    auto h0_of = [&](int jc) { return kJC * jc - P; };
    auto col0 = [&](int jc) { return TRANS ? f1 - h0_of(jc) - (kJC - 1) : f1; };
    // own sub-row s -> window row (in processing order: source rows ascend)
    auto dd_of = [&](int s) {
        const int q = s / NJC;
        return TRANS ? WS - 1 - q : q;
    };
    auto zrow = [&](int dd, int &r2, int &mm) {
        if (TRANS) {
            r2 = pmod(c2 - (dd - P), n2);
            mm = pmod(dd + slot_shift(r2 + 1, n2, P), WS);
        } else {
            r2 = c2;
            mm = pmod(dd + s2own, WS);
        }
    };
    int zo[FAST ? ZI : 1];
    if (FAST) {
#pragma unroll
        for (int m = 0; m < ZI; ++m) {
            const int f = lane + 64 * m;
            const int kb = f / S::BLK, r = f - kb * S::BLK;
            const int rq = r < 4 * S::Q ? r : 0;
            const int wc = min(4 * kb + rq / S::Q, S::NSRC - 1), q = rq - (rq / S::Q) * S::Q;
            zo[m] = (wc * K + 4 * q) * 4;
        }
    }
    // Border body.  Chunk pixels may wrap along dim 1 and, within p of the
    // image border, carry the reference's rotated slot order.  The chunk
    // keeps the interior body's LDS layout: a DMA instruction's 64 16-byte
    // slots whose pixels all have unrotated slots load as 16-byte pieces from
    // their (wrapped) pixels; an instruction with a rotated pixel is issued
    // as four 4-byte DMAs that place each slot.  Offsets are formed per
    // sub-row (held across the walk they would not fit the register budget).
    // The columns of a chunk or of a staged x row lie within [-n1, 2 n1)
    // when n1 >= 2p + 80: one conditional step wraps them, except in narrow
    // images.
    const bool narrow = n1 < 2 * P + 80;
    auto wrapc = [&](int x) {
        return narrow ? pmod(x, n1) : (x < 0 ? x + n1 : (x >= n1 ? x - n1 : x));
    };
    // chunk pixel wc and piece q of LDS 16-byte slot f
    auto slot_of = [&](int f, int &wc, int &q) {
        const int kb = f / S::BLK, r = f - kb * S::BLK;
        const int rq = r < 4 * S::Q ? r : 0;
        wc = min(4 * kb + rq / S::Q, S::NSRC - 1);
        q = rq - (rq / S::Q) * S::Q;
    };
    auto stage_z = [&](int s) {
        const int dd = dd_of(s), jc = s - (s / NJC) * NJC;
        int r2, mm;
        zrow(dd, r2, mm);
        float *dst = lz + (s % kBZ) * S::NZB;
        if (FAST) {
            const int so = __builtin_amdgcn_readfirstlane(
                ((n1 * r2 + col0(jc)) * K + mm * WS + kJC * jc) * 4);
#pragma unroll
            for (int m = 0; m < ZI; ++m) {
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lptr)(dst + 256 * m), 16, zo[m] + so,
                                                        0, 0, 0);
            }
        } else {
            // (loops kept rolled: the border code stays small in the
            // instruction cache next to the interior body)
            const int so = __builtin_amdgcn_readfirstlane((n1 * r2 * K + mm * WS) * 4);
            const int c0 = col0(jc);
#pragma unroll 1
            for (int m = 0; m < S::NZ4; ++m) {
                int wc, q;
                slot_of(lane + 64 * m, wc, q);
                const int col = wrapc(c0 + wc);
                if (__builtin_amdgcn_ballot_w64(shift0(col, n1, P) != 0) == 0) {
                    const int vo = (col * K + kJC * jc + 4 * q) * 4 + so;
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lptr)(dst + 256 * m), 16, vo, 0,
                                                            0, 0);
                } else {
#pragma unroll 1
                    for (int t = 0; t < 4; ++t) {
                        int wt, qt;
                        slot_of(64 * m + 16 * t + (lane >> 2), wt, qt);
                        const int ct = wrapc(c0 + wt);
                        const int j = kJC * jc + 4 * qt + (lane & 3);
                        const int e = j < WS ? fold(j + shift0(ct, n1, P), WS) : 0;
                        const int vo = (ct * K + e) * 4 + so;
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lptr)(dst + 256 * m + 64 * t),
                                                                4, vo, 0, 0, 0);
                    }
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // ---- shared x rows: this wavefront's share of source row u ----
    // interior: 16-byte piece pc = (w XP + m) 64 + lane of the buffer, i.e.
    // channel pc / (XROW / 4), floats 4 (pc % (XROW / 4)) ..; border: float
    // f = (w X1 + m) 64 + lane at its wrapped column.  Channels past C lie
    // past the unit's bytes and read as zeros.
    int xo[FAST ? XI : 1];
    if (FAST) {
#pragma unroll
        for (int m = 0; m < XI; ++m) {
            const int pc = w * BB::PPW + 64 * m + lane;
            const int c = pc / (BB::XROW / 4), q = pc - c * (BB::XROW / 4);
            xo[m] = (ch0 + c) * plane + (NCOMP * X0 + 4 * q) * 4;
        }
    }
    // border float f's offset, formed per source row (12 offsets held across
    // the walk would not fit the register budget)
    auto xo_border = [&](int m) {
        const int f = (w * XI + m) * 64 + lane;
        const int c = f / BB::XROW, e = f - c * BB::XROW;
        const int u = e / NCOMP, comp = e - u * NCOMP;
        return (ch0 + c) * plane + (NCOMP * wrapc(X0 + u) + comp) * 4;
    };
    auto stage_x = [&](int u, int buf) {
        const int so = __builtin_amdgcn_readfirstlane(NCOMP * n1 * pmod(r0 + u, n2) * 4);
        float *dst = lxs + buf * BB::XF + (FAST ? 4 * w * BB::PPW : w * XI * 64);
        if (FAST) {
#pragma unroll
            for (int m = 0; m < XI; ++m) {
                __builtin_amdgcn_sched_barrier(0);
                if (m + 1 < XI || BB::XPL == 64 || lane < BB::XPL)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lptr)(dst + 256 * m), 16,
                                                            xo[m] + so, 0, 0, 0);
            }
        } else {
#pragma unroll 1
            for (int m = 0; m < XI; ++m)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lptr)(dst + 64 * m), 4,
                                                        xo_border(m) + so, 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    float acc[kR][kBG];
    float asum[kR];
#pragma unroll
    for (int i = 0; i < kR; ++i) {
        asum[i] = 0.f;
#pragma unroll
        for (int k = 0; k < kBG; ++k) acc[i][k] = 0.f;
    }
    // slots jn .. kJC - 1 of a window row's last sub-row lie past the window:
    // once the chunk has landed they are cleared in LDS, so that the reads
    // below need no mask (chunk pixel wc, slot j at 16 wc + 4 (wc / 4) + j)
    auto clear_tail = [&](int jc, float *zb) {
        const int jn = WS - kJC * jc;
#pragma unroll 1
        for (int j = jn; j < kJC; ++j) {
#pragma unroll
            for (int h = 0; h < (S::NSRC + 63) / 64; ++h) {
                const int wc = lane + 64 * h;
                if (wc < S::NSRC) zb[16 * wc + 4 * (wc >> 2) + j] = 0.f;
            }
        }
    };
    auto read_av = [&](float (&av)[kR][kJC], const float *src) {
#pragma unroll
        for (int i = 0; i < kR; ++i)
#pragma unroll
            for (int j = 0; j < kJC; ++j) {
                const int c = TRANS ? i - j + kJC - 1 : i;
                av[i][j] = src[(4 * l16 + c) * kJC + 4 * (l16 + c / 4) + j];
            }
    };

    // Issue order per source row u: x(u + 1), then per own sub-row s the
    // chunk of sub-row s + kBZ.  The first kBZ chunks are staged before the
    // walk (a wavefront whose window starts at a later source row waits with
    // them in LDS).  The waits count the loads issued after the ones needed:
    // chunks s + 1 .. s + kBZ - 1 (ZI each, fewer at the end), and x(u + 1)
    // when chunk s was issued before source row u began (jc < kBZ).
    auto wait_after = [&](int nz, bool nx) {
        if (nx) {
            if (nz >= 2) wait_vm<2 * ZI + XI>();
            else if (nz == 1) wait_vm<ZI + XI>();
            else wait_vm<XI>();
        } else {
            if (nz >= 2) wait_vm<2 * ZI>();
            else if (nz == 1) wait_vm<ZI>();
            else wait_vm<0>();
        }
    };
    static_assert(kBZ <= 3, "wait_after covers up to two younger chunks");
    stage_x(0, 0);
    if (live) {
#pragma unroll
        for (int k = 0; k < kBZ; ++k)
            if (k < NSR) stage_z(k);
    }
    wait_vm<0>();
    __syncthreads();
    int s = 0;   // next own sub-row
    float av[kR][kJC];
#pragma unroll 1
    for (int u = 0; u < NU; ++u) {
        // priority 1 over the first three quarters of the source rows, 0 over
        // the last, so that a workgroup near its end yields to those behind it
        // (cfg4a similarity pullback on gfx950, interleaved A/B: 790 -> 738
        // us; the single applies unchanged)
        if (u == 0) __builtin_amdgcn_s_setprio(1);
        if (u == (3 * NU) / 4) __builtin_amdgcn_s_setprio(0);
        const bool more = u + 1 < NU;
        if (more) stage_x(u + 1, (u + 1) & 1);
        const int dd = TRANS ? w + 2 * P - u : u - w;
        const bool act = live && dd >= 0 && dd < WS;
        if (act) {
            const float *xbase = lxs + (u & 1) * BB::XF + grp * BB::CHS * BB::XROW;
#pragma unroll 1
            for (int jc = 0; jc < NJC; ++jc, ++s) {
                wait_after(min(kBZ - 1, NSR - 1 - s), more && jc < kBZ);
                float *zb = lz + (s % kBZ) * S::NZB;
                clear_tail(jc, zb);
                read_av(av, zb);
                if (a.corr) {
#pragma unroll
                    for (int i = 0; i < kR; ++i)
#pragma unroll
                        for (int j = 0; j < kJC; ++j) asum[i] += av[i][j];
                }
                // the lane's runs start kJC jc (forward) or kJC (NJC - 1 - jc)
                // columns into the staged row
                const float *xr = xbase + NCOMP * (kJC * (TRANS ? NJC - 1 - jc : jc) + 4 * l16);
                // real components: step cl + 1's runs are read while step
                // cl's products run (two register sets); complex runs are
                // twice as long and are read per step
                constexpr bool PIPE = NCOMP == 1;
                f4 xq[PIPE ? 2 : 1][KW4];
                if (PIPE) {
#pragma unroll
                    for (int h = 0; h < KW4; ++h) xq[0][h] = *(const f4 *)(xr + 4 * h);
                }
#pragma unroll
                for (int cl = 0; cl < BB::CHS; ++cl) {
                    const int cur = PIPE ? cl & 1 : 0;
                    if (PIPE && cl + 1 < BB::CHS) {
#pragma unroll
                        for (int h = 0; h < KW4; ++h)
                            xq[(cl + 1) & 1][h] = *(const f4 *)(xr + (cl + 1) * BB::XROW + 4 * h);
                    } else if (!PIPE) {
#pragma unroll
                        for (int h = 0; h < KW4; ++h)
                            xq[0][h] = *(const f4 *)(xr + cl * BB::XROW + 4 * h);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    float xw[4 * KW4];
#pragma unroll
                    for (int h = 0; h < KW4; ++h) {
                        xw[4 * h] = xq[cur][h][0];
                        xw[4 * h + 1] = xq[cur][h][1];
                        xw[4 * h + 2] = xq[cur][h][2];
                        xw[4 * h + 3] = xq[cur][h][3];
                    }
#pragma unroll
                    for (int i = 0; i < kR; ++i)
#pragma unroll
                        for (int j = 0; j < kJC; ++j)
#pragma unroll
                            for (int e = 0; e < NCOMP; ++e)
                                acc[i][NCOMP * cl + e] = __builtin_fmaf(
                                    av[i][j], xw[NCOMP * (TRANS ? i - j + kJC - 1 : i + j) + e],
                                    acc[i][NCOMP * cl + e]);
#pragma unroll
                    for (int i = 0; i < kR; ++i)
#pragma unroll
                        for (int e = 0; e < NCOMP; ++e)
                            asm volatile("" : "+v"(acc[i][NCOMP * cl + e]));
                    __builtin_amdgcn_sched_barrier(0);
                    if (cl == 0) {
                        // step 0 has consumed every coefficient, so the
                        // chunk's reads are complete: stage the next one over
                        // it (the reads' latency was covered by step 0)
                        __builtin_amdgcn_s_waitcnt(kWaitLgkm);
                        if (s + kBZ < NSR) stage_z(s + kBZ);
                    }
                }
            }
        }
        if (more) {
            // x(u + 1) landed; the chunks issued during this source row (if
            // any) may remain
            wait_after(act ? min(NJC, max(0, NSR - kBZ - (s - NJC))) : 0, false);
            __syncthreads();
        }
    }
    if (!live) return;
    float *yb = a.y + (int64_t)b * Pp * NCOMP * a.C;
    const float *zb = a.z ? a.z + (int64_t)b * Pp * NCOMP * a.C : nullptr;
    const int colf = f1 + 4 * l16;
    const int64_t pix0 = colf + (int64_t)n1 * c2;
#pragma unroll
    for (int cl = 0; cl < BB::CHS; ++cl) {
        const int ch = ch0 + grp * BB::CHS + cl;
        if (ch >= a.C) break;
        float v[kR * NCOMP];
#pragma unroll
        for (int i = 0; i < kR; ++i)
#pragma unroll
            for (int e = 0; e < NCOMP; ++e) v[NCOMP * i + e] = acc[i][NCOMP * cl + e];
        float *dst = yb + NCOMP * (pix0 + Pp * ch);
        const float *zs = a.corr ? zb + NCOMP * (pix0 + Pp * ch) : nullptr;
        if (colf + kR <= n1) {
#pragma unroll
            for (int h = 0; h < NCOMP; ++h) {
                f4 r = f4{v[4 * h], v[4 * h + 1], v[4 * h + 2], v[4 * h + 3]};
                if (a.corr) {
                    const f4u z = *(const f4u *)(zs + 4 * h);
#pragma unroll
                    for (int q = 0; q < 4; ++q) r[q] -= asum[(4 * h + q) / NCOMP] * z[q];
                }
                *(f4u *)(dst + 4 * h) = r * a.scale;
            }
        } else {
#pragma unroll
            for (int i = 0; i < kR; ++i) {
                if (colf + i >= n1) break;
#pragma unroll
                for (int e = 0; e < NCOMP; ++e) {
                    float r = v[NCOMP * i + e];
                    if (a.corr) r -= asum[i] * zs[NCOMP * i + e];
                    dst[NCOMP * i + e] = r * a.scale;
                }
            }
        }
    }
}

// Work items of one product: XCD band `band` holds row groups [band brg,
// (band + 1) brg) of all units, every tile column and pass; within a band the
// border segments come first, so that the slower border workgroups start in
// the first round rather than in the grid's tail.  idx < brg tiles1 gchunk;
// returns false past the last row group.
__device__ __forceinline__ bool band_item(const ApplyArgs &a, int band, int idx, int &pass,
                                          int &t1, int &c2g, int &b) {
    const int ngr = (a.g.n2 + kBR - 1) / kBR;
    const int nit = a.fb - a.fa, nbt = a.tiles1 - nit;
    const int nborder = a.brg * nbt * a.gchunk;
    const bool border = idx < nborder;
    const int per = (border ? nbt : nit) * a.gchunk;  // items per row group
    if (!border) idx -= nborder;
    const int rgl = idx / per, rem = idx - rgl * per;
    const int k = rem / a.gchunk;
    pass = rem - k * a.gchunk;
    t1 = border ? (k < a.fa ? k : a.fb + (k - a.fa)) : a.fa + k;
    const int rg = band * a.brg + rgl;
    c2g = rg % ngr;
    b = rg / ngr;
    return rg < a.nrg;
}
template <int NCOMP, bool TRANS>
__device__ __forceinline__ void apply_band_tile(const ApplyArgs &a, int pass, int t1, int c2g,
                                                int b) {
    if (t1 >= a.fa && t1 < a.fb)
        apply_band_body<NCOMP, TRANS, true>(a, pass, t1, c2g, b);
    else
        apply_band_body<NCOMP, TRANS, false>(a, pass, t1, c2g, b);
}
// One workgroup of kBR wavefronts per (64 columns of kBR image rows,
// component pass, unit); work items in XCD bands.
// (the grid is 8 x brg x tiles1 x gchunk workgroups; blockIdx & 7 is the
// XCD the dispatcher deals the workgroup to)
template <int NCOMP, bool TRANS>
__global__ __launch_bounds__(64 * kBR, 3) void apply_band_kernel(ApplyArgs a) {
    int pass, t1, c2g, b;
    const int band = (int)(blockIdx.x & 7), idx = (int)(blockIdx.x >> 3);
    if (!band_item(a, band, idx, pass, t1, c2g, b)) return;
    apply_band_tile<NCOMP, TRANS>(a, pass, t1, c2g, b);
}
// the similarity pullback's two products in one grid: per band, the border
// items of both products, then the interior ones
template <int NCOMP>
__global__ __launch_bounds__(64 * kBR, 3) void apply_band_pair_kernel(ApplyArgs af, ApplyArgs at) {
    const int band = (int)(blockIdx.x & 7);
    int idx = (int)(blockIdx.x >> 3);
    const int per = af.brg * af.tiles1 * af.gchunk;            // items per band and product
    const int bf = af.brg * (af.tiles1 - (af.fb - af.fa)) * af.gchunk;  // border items
    const int bt = at.brg * (at.tiles1 - (at.fb - at.fa)) * at.gchunk;
    bool trans;
    if (idx < bf) {
        trans = false;
    } else if (idx < bf + bt) {
        trans = true;
        idx -= bf;
    } else {
        idx -= bf + bt;
        trans = idx >= per - bf;
        idx = trans ? bt + idx - (per - bf) : bf + idx;
    }
    int pass, t1, c2g, b;
    if (!band_item(trans ? at : af, band, idx, pass, t1, c2g, b)) return;
    if (trans)
        apply_band_tile<NCOMP, true>(at, pass, t1, c2g, b);
    else
        apply_band_tile<NCOMP, false>(af, pass, t1, c2g, b);
}

// geometry fields of the band kernel: segments, passes, and the interior
// segments [fa, fb), whose staged x columns, chunk pixels and coefficient
// slots need no wrapping and no slot shift
template <bool TRANS>
void set_band(ApplyArgs &a, int ncomp, int64_t nb) {
    const Geom &g = a.g;
    const int n1 = g.n1, p = g.p, njc = (g.ws + kJC - 1) / kJC;
    a.tiles1 = (n1 + 63) / 64;
    a.gchunk = (ncomp * a.C + kBPass - 1) / kBPass;
    a.nrg = (int)(((g.n2 + kBR - 1) / kBR) * nb);
    a.brg = (a.nrg + 7) / 8;
    auto interior = [&](int t1) {
        const int f1 = 64 * t1, x0 = band_x0(TRANS, f1, p, njc);
        if (x0 < 0 || x0 + kBX > n1) return false;
        // chunk pixels: own 64 (forward) or the sub-rows' sources (transposed)
        const int lo = TRANS ? f1 + p - kJC * (njc - 1) - (kJC - 1) : f1;
        const int hi = TRANS ? f1 + p + 64 : f1 + 64;  // exclusive
        return lo >= p && hi <= n1 - p;
    };
    a.fa = a.tiles1;
    a.fb = a.tiles1;
    for (int t = 0; t < a.tiles1; ++t)
        if (interior(t)) {
            if (a.fa == a.tiles1) a.fa = t;
            a.fb = t + 1;
        }
    if (a.fa == a.tiles1) a.fa = a.fb = 0;
}

bool band_supported(const Geom &g) { return g.nsp == 2 && g.ws > 15 && (g.ws + kJC - 1) / kJC <= 2; }

// the band kernels' LDS passes 64 KiB: raise the kernel's dynamic limit once
// per instantiation (the callers keep the result in a function-local static,
// initialised exactly once, also when several host threads launch at once)
template <typename Kern>
hipError_t band_lds_attr(Kern kern, size_t bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}
template <int NCOMP, bool TRANS>
hipError_t launch_band(ApplyArgs a, int64_t nb, hipStream_t s) {
    set_band<TRANS>(a, NCOMP, nb);
    const int64_t grid = 8LL * a.brg * a.tiles1 * a.gchunk;
    const size_t lds = (size_t)AB<NCOMP, TRANS>::LDS * sizeof(float);
    static const hipError_t e = band_lds_attr(apply_band_kernel<NCOMP, TRANS>, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((apply_band_kernel<NCOMP, TRANS>), dim3((unsigned)grid), dim3(64 * kBR), lds,
                       s, a);
    return hipGetLastError();
}
template <int NCOMP>
hipError_t launch_band_pair(ApplyArgs af, ApplyArgs at, int64_t nb, hipStream_t s) {
    set_band<false>(af, NCOMP, nb);
    set_band<true>(at, NCOMP, nb);
    const int64_t grid = 16LL * af.brg * af.tiles1 * af.gchunk;
    const size_t lds =
        (size_t)std::max(AB<NCOMP, false>::LDS, AB<NCOMP, true>::LDS) * sizeof(float);
    static const hipError_t e = band_lds_attr(apply_band_pair_kernel<NCOMP>, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((apply_band_pair_kernel<NCOMP>), dim3((unsigned)grid), dim3(64 * kBR), lds,
                       s, af, at);
    return hipGetLastError();
}

// Interior tile columns [fa, fb): every lane row 2p or more inside dim 1.
inline void interior_cols(const Geom &g, int &fa, int &fb) {
    const int tw = tile_w(g.nsp), tiles1 = (g.n1 + tw - 1) / tw;
    const int two_p = g.ws - 1;
    fa = (two_p + tw - 1) / tw;                 // first t1 with t1 * tw >= 2p
    fb = (g.n1 - two_p - tw) >= 0 ? (g.n1 - two_p - tw) / tw + 1 : 0;  // t1 * tw + tw - 1 + 2p < n1
    if (fb > tiles1) fb = tiles1;
    if (fb < fa) fb = fa;
}

template <int WS, int NCOMP, bool TRANS>
hipError_t launch_rb(ApplyArgs a, int64_t nb, hipStream_t s) {
    if (a.g.nsp == 2) {
        constexpr int NXL = kNX;
        constexpr int NXS = kNXSmall;
        using S = A2<WS, NCOMP, TRANS, kCG, NXL>;
        const int tiles1 = (a.g.n1 + 63) / 64;
        a.tiles1 = tiles1;
        a.fa = (S::EDGE + 63) / 64;
        a.fb = a.g.n1 - 64 - S::EDGE >= 0 ? (a.g.n1 - 64 - S::EDGE) / 64 + 1 : 0;
        if (a.fb > tiles1) a.fb = tiles1;
        if (a.fb < a.fa) a.fb = a.fa;
        a.gchunk = (NCOMP * a.C + kCPass - 1) / kCPass;  // component passes
        int64_t nwork = (int64_t)tiles1 * a.g.n2 * nb * a.gchunk;
        // Grids of fewer wavefronts than SIMDs are bound by each wavefront's
        // chain of component steps: passes of 16 components there (twice the
        // wavefronts, chains half as long; cfg2 on gfx950: forward 37.9 ->
        // 34.1 us, transposed 42.9 -> 40.3 us).  Larger grids keep passes of
        // 32 (cfg5's forward apply took 150 against 126 us with 16).
        if (nwork < 1024 && NCOMP * a.C > kCPass / 2) {
            using S4 = A2<WS, NCOMP, TRANS, kCG / 2, NXS>;
            a.gchunk = (NCOMP * a.C + kCPass / 2 - 1) / (kCPass / 2);
            nwork = (int64_t)tiles1 * a.g.n2 * nb * a.gchunk;
            const int64_t grid = 8 * ((nwork + 7) / 8);
            hipLaunchKernelGGL((apply2_kernel<WS, NCOMP, TRANS, false, kCG / 2, NXS>), dim3((unsigned)grid),
                               dim3(64), (size_t)S4::LDS * sizeof(float), s, a, (int)nwork);
            return hipGetLastError();
        }
        const int64_t grid = 8 * ((nwork + 7) / 8);
        hipLaunchKernelGGL((apply2_kernel<WS, NCOMP, TRANS, false, kCG, NXL>), dim3((unsigned)grid), dim3(64),
                           (size_t)S::LDS * sizeof(float), s, a, (int)nwork);
        return hipGetLastError();
    }
    const size_t lds = (size_t)lds_floats(WS, TRANS) * sizeof(float);
    interior_cols(a.g, a.fa, a.fb);
    const int64_t grid = (int64_t)a.gchunk * a.tiles1 * nb;
    hipLaunchKernelGGL((apply_rb_kernel<WS, NCOMP, TRANS>), dim3((unsigned)grid), dim3(64), lds, s,
                       a);
    return hipGetLastError();
}

// geometry fields of the 2D row kernel (segments, interior range, passes)
template <int WS, int NCOMP, bool TRANS>
void set_rows2(ApplyArgs &a) {
    using S = A2<WS, NCOMP, TRANS>;
    a.tiles1 = (a.g.n1 + 63) / 64;
    a.fa = (S::EDGE + 63) / 64;
    a.fb = a.g.n1 - 64 - S::EDGE >= 0 ? (a.g.n1 - 64 - S::EDGE) / 64 + 1 : 0;
    if (a.fb > a.tiles1) a.fb = a.tiles1;
    if (a.fb < a.fa) a.fb = a.fa;
    a.gchunk = (NCOMP * a.C + kCPass - 1) / kCPass;
}

template <int WS, int NCOMP>
hipError_t launch_pair_t(ApplyArgs f, ApplyArgs t, int64_t nb, hipStream_t s) {
    set_rows2<WS, NCOMP, false>(f);
    set_rows2<WS, NCOMP, true>(t);
    const int64_t nwork = (int64_t)f.tiles1 * f.g.n2 * nb * f.gchunk;
    const int64_t grid = 8 * ((2 * nwork + 7) / 8);
    constexpr int NX = kNX;
    const size_t lds = (size_t)std::max(A2<WS, NCOMP, false, kCG, NX>::LDS,
                                        A2<WS, NCOMP, true, kCG, NX>::LDS) *
                       sizeof(float);
    hipLaunchKernelGGL((apply2_pair_kernel<WS, NCOMP, NX>), dim3((unsigned)grid), dim3(64), lds, s, f,
                       t, (int)nwork);
    return hipGetLastError();
}

template <int NCOMP>
hipError_t dispatch_pair(const ApplyArgs &f, const ApplyArgs &t, int64_t nb, hipStream_t s) {
    switch (f.g.ws) {
        case 3: return launch_pair_t<3, NCOMP>(f, t, nb, s);
        case 5: return launch_pair_t<5, NCOMP>(f, t, nb, s);
        case 7: return launch_pair_t<7, NCOMP>(f, t, nb, s);
        case 9: return launch_pair_t<9, NCOMP>(f, t, nb, s);
        case 11: return launch_pair_t<11, NCOMP>(f, t, nb, s);
        case 13: return launch_pair_t<13, NCOMP>(f, t, nb, s);
        case 15: return launch_pair_t<15, NCOMP>(f, t, nb, s);
        default: return hipErrorNotSupported;
    }
}

template <int NCOMP, bool TRANS>
hipError_t dispatch_ws(const ApplyArgs &a, int64_t nb, hipStream_t s) {
    switch (a.g.ws) {
        case 3: return launch_rb<3, NCOMP, TRANS>(a, nb, s);
        case 5: return launch_rb<5, NCOMP, TRANS>(a, nb, s);
        case 7: return launch_rb<7, NCOMP, TRANS>(a, nb, s);
        case 9: return launch_rb<9, NCOMP, TRANS>(a, nb, s);
        case 11: return launch_rb<11, NCOMP, TRANS>(a, nb, s);
        case 13: return launch_rb<13, NCOMP, TRANS>(a, nb, s);
        case 15: return launch_rb<15, NCOMP, TRANS>(a, nb, s);
        default: return hipErrorNotSupported;
    }
}

template <int WS>
hipError_t launch_colsum_t(const Geom &g, int64_t nb, const float *nz, float *out, hipStream_t s) {
    if (g.nsp == 2) {
        using S = A2<WS, 1, true>;
        ApplyArgs a{};
        a.g = g;
        a.C = 1;
        a.nz = nz;
        a.y = out;
        a.tiles1 = (g.n1 + 63) / 64;
        a.fa = (S::EDGE + 63) / 64;
        a.fb = g.n1 - 64 - S::EDGE >= 0 ? (g.n1 - 64 - S::EDGE) / 64 + 1 : 0;
        if (a.fb > a.tiles1) a.fb = a.tiles1;
        if (a.fb < a.fa) a.fb = a.fa;
        a.gchunk = 1;
        const int64_t nwork = (int64_t)a.tiles1 * g.n2 * nb;
        hipLaunchKernelGGL((apply2_kernel<WS, 1, true, true>), dim3((unsigned)(8 * ((nwork + 7) / 8))),
                           dim3(64), (size_t)S::LDS_SUMS * sizeof(float), s, a, (int)nwork);
        return hipGetLastError();
    }
    const int tiles1 = (g.n1 + tile_w(g.nsp) - 1) / tile_w(g.nsp);
    int fa, fb;
    interior_cols(g, fa, fb);
    hipLaunchKernelGGL(colsum_rb_kernel<WS>, dim3((unsigned)((int64_t)tiles1 * nb)), dim3(64),
                       (size_t)lds_floats(WS, true) * sizeof(float), s, g, tiles1, fa, fb, nz,
                       out);
    return hipGetLastError();
}

int64_t tiles_of(const Geom &g) {
    return (int64_t)((g.n1 + tile_w(g.nsp) - 1) / tile_w(g.nsp)) *
           ((g.n2 + tile_h(g.nsp) - 1) / tile_h(g.nsp));
}

template <int WS, int NCOMP, bool DIST>
hipError_t launch_sim_t(ApplyArgs a, int64_t nb, hipStream_t s) {
    const int tiles1 = (a.g.n1 + 63) / 64;
    a.tiles1 = tiles1;
    // interior tiles: staged key columns f1 - kHalo .. f1 + 63 + kHalo in range
    a.fa = (kHalo + 63) / 64;
    a.fb = a.g.n1 - 64 - kHalo >= 0 ? (a.g.n1 - 64 - kHalo) / 64 + 1 : 0;
    if (a.fb > tiles1) a.fb = tiles1;
    if (a.fb < a.fa) a.fb = a.fa;
    // window-row iterations split over wavefronts when the grid is small
    constexpr int NIT = (WS + 3) / 4;
    const int64_t waves = (int64_t)tiles1 * a.g.n2 * nb;
    a.ichunk = waves >= 2048 ? NIT : std::max(1, (int)((int64_t)NIT * waves / 2048));
    a.gchunk = (NIT + a.ichunk - 1) / a.ichunk;
    const int64_t nwork = waves * a.gchunk;
    const int64_t grid = 8 * ((nwork + 7) / 8);
    // LDS: the staging ring, which also holds 64 pixels x 4 window rows of
    // results before they are stored (skewed by 4 floats per 4 pixels, plus
    // the 16 floats that the last pixel's 16 lanes read past its 4 ws)
    const size_t lds =
        (size_t)std::max(SimStage<NCOMP, NCOMP == 1 ? 2 : 1>::NR * SimStage<NCOMP, NCOMP == 1 ? 2 : 1>::SB,
                         64 * 4 * WS + 64 + 64) *
        sizeof(float);
    hipLaunchKernelGGL((sim_rows_kernel<WS, NCOMP, DIST>), dim3((unsigned)grid), dim3(64), lds, s,
                       a, (int)nwork);
    return hipGetLastError();
}

template <int NCOMP, bool DIST>
hipError_t sim_ws(const ApplyArgs &a, int64_t nb, hipStream_t s) {
    switch (a.g.ws) {
        case 3: return launch_sim_t<3, NCOMP, DIST>(a, nb, s);
        case 5: return launch_sim_t<5, NCOMP, DIST>(a, nb, s);
        case 7: return launch_sim_t<7, NCOMP, DIST>(a, nb, s);
        case 9: return launch_sim_t<9, NCOMP, DIST>(a, nb, s);
        case 11: return launch_sim_t<11, NCOMP, DIST>(a, nb, s);
        case 13: return launch_sim_t<13, NCOMP, DIST>(a, nb, s);
        case 15: return launch_sim_t<15, NCOMP, DIST>(a, nb, s);
        default: return hipErrorNotSupported;
    }
}

}  // namespace

bool sim_rows_supported(const Geom &g, int C, int ncomp, int64_t nb) {
    if (g.nsp != 2 || g.ws < 3 || g.ws > 15 || (g.ws & 1) == 0) return false;
    if (g.P * g.K * 4 >= (int64_t)1 << 31) return false;
    if (g.P * ncomp * C * 4 >= (int64_t)1 << 31) return false;
    const int64_t grid = (int64_t)((g.n1 + 63) / 64) * g.n2 * nb * ((g.ws + 3) / 4) + 8;
    return grid > 0 && grid < ((int64_t)1 << 31);
}
hipError_t launch_sim_rows(bool dist, int ncomp, const Geom &g, int C, int64_t nb, float scale,
                           const float *x, const float *y, float *nz, hipStream_t s) {
    ApplyArgs a{};
    a.g = g;
    a.C = C;
    a.scale = scale;
    a.x = x;
    a.z = y;
    a.y = nz;
    if (ncomp == 1) return dist ? sim_ws<1, true>(a, nb, s) : sim_ws<1, false>(a, nb, s);
    return dist ? sim_ws<2, true>(a, nb, s) : sim_ws<2, false>(a, nb, s);
}

bool sim_wide_supported(const Geom &g, int C, int ncomp, int64_t nb) {
    if (g.ws < 3 || (g.ws & 1) == 0 || (g.nsp != 1 && g.nsp != 2)) return false;
    if (g.P * g.K * 4 >= (int64_t)1 << 31) return false;
    if (g.P * ncomp * (int64_t)C * 4 >= (int64_t)1 << 31) return false;
    const int64_t n2 = g.nsp == 2 ? g.n2 : 1;
    const int64_t grid = 8 + (int64_t)((g.n1 + 63) / 64) * n2 * nb;
    return grid > 0 && grid < ((int64_t)1 << 31);
}

hipError_t launch_sim_wide(bool dist, int ncomp, const Geom &g, int C, int64_t nb, float scale,
                           const float *x, const float *y, float *nz, hipStream_t s) {
    ApplyArgs a{};
    a.g = g;
    a.C = C;
    a.scale = scale;
    a.x = x;
    a.z = y;
    a.y = nz;
    if (ncomp == 1)
        return dist ? launch_sim_wide_t<1, true>(a, nb, s) : launch_sim_wide_t<1, false>(a, nb, s);
    return dist ? launch_sim_wide_t<2, true>(a, nb, s) : launch_sim_wide_t<2, false>(a, nb, s);
}

bool apply_rb_supported(const Geom &g, int C, int ncomp, int64_t nb) {
    if (g.ws < 3 || g.ws > 15 || (g.ws & 1) == 0) return false;
    // 32-bit byte offsets into one unit's nzVal and x, grid in one dimension
    if (g.P * g.K * 4 >= (int64_t)1 << 31) return false;
    // (the 2D kernel forms offsets of up to kCPass channels past C)
    if (g.P * ncomp * ((int64_t)C + kCPass) * 4 >= (int64_t)1 << 31) return false;
    const int64_t grid = tiles_of(g) * ((ncomp * C + kCP - 1) / kCP) * nb;  // upper bound
    return grid > 0 && grid < ((int64_t)1 << 31);
}

hipError_t launch_apply_rb(bool trans, bool corr, int ncomp, const Geom &g, int C, int64_t nb,
                           float scale, const float *nz, const float *x, const float *z, float *y,
                           hipStream_t s) {
    ApplyArgs a;
    a.g = g;
    a.C = C;
    a.corr = corr ? 1 : 0;
    a.tiles1 = (g.n1 + tile_w(g.nsp) - 1) / tile_w(g.nsp);
    // staging passes of one tile run in one wavefront (nzVal re-read from L2)
    // unless the grid would be too small to fill the GPU
    const int npass = (ncomp * C + kCP - 1) / kCP;
    const int64_t waves = tiles_of(g) * nb;
    a.ichunk = waves >= 1024 ? npass : 1;
    a.gchunk = (npass + a.ichunk - 1) / a.ichunk;
    a.scale = scale;
    a.nz = nz;
    a.x = x;
    a.z = z;
    a.y = y;
    if (ncomp == 1) return trans ? dispatch_ws<1, true>(a, nb, s) : dispatch_ws<1, false>(a, nb, s);
    return trans ? dispatch_ws<2, true>(a, nb, s) : dispatch_ws<2, false>(a, nb, s);
}

bool apply_wide_supported(const Geom &g, int C, int ncomp, int64_t nb) {
    if (g.ws < 3 || (g.ws & 1) == 0 || (g.nsp != 1 && g.nsp != 2)) return false;
    // 32-bit byte offsets (reads reach kJC slots past a window row and up to
    // kCPass channels past C), grid in one dimension
    if ((g.P * g.K + kJC) * 4 >= (int64_t)1 << 31) return false;
    if (g.P * ncomp * ((int64_t)C + kCPass) * 4 >= (int64_t)1 << 31) return false;
    const int64_t n2 = g.nsp == 2 ? g.n2 : 1;
    const int64_t grid = 8 + (int64_t)((g.n1 + 63) / 64) * n2 * nb * ((ncomp * C + kCPass - 1) / kCPass);
    return grid > 0 && grid < ((int64_t)1 << 31);
}

hipError_t launch_apply_wide(bool trans, bool corr, int ncomp, const Geom &g, int C, int64_t nb,
                             float scale, const float *nz, const float *x, const float *z, float *y,
                             hipStream_t s) {
    ApplyArgs a{};
    a.g = g;
    a.C = C;
    a.corr = corr ? 1 : 0;
    a.scale = scale;
    a.nz = nz;
    a.x = x;
    a.z = z;
    a.y = y;
    if (band_supported(g)) {
        if (ncomp == 1)
            return trans ? launch_band<1, true>(a, nb, s) : launch_band<1, false>(a, nb, s);
        return trans ? launch_band<2, true>(a, nb, s) : launch_band<2, false>(a, nb, s);
    }
    if (ncomp == 1)
        return trans ? launch_wide<1, true, false>(a, nb, s) : launch_wide<1, false, false>(a, nb, s);
    return trans ? launch_wide<2, true, false>(a, nb, s) : launch_wide<2, false, false>(a, nb, s);
}

// the pair goes to the 2D row kernel (ws <= 15) or the wide kernel (ws > 15)
static bool pair_rows(const Geom &g, int C, int ncomp, int64_t nb) {
    return g.nsp == 2 && apply_rb_supported(g, C, ncomp, nb);
}
static bool pair_wide(const Geom &g, int C, int ncomp, int64_t nb) {
    return !apply_rb_supported(g, C, ncomp, nb) && apply_wide_supported(g, C, ncomp, nb);
}
bool apply_pair_supported(const Geom &g, int C, int ncomp, int64_t nb) {
    if (!pair_rows(g, C, ncomp, nb) && !pair_wide(g, C, ncomp, nb)) return false;
    const int64_t n2 = g.nsp == 2 ? g.n2 : 1;
    const int64_t nwork = (int64_t)((g.n1 + 63) / 64) * n2 * nb *
                          ((ncomp * C + kCPass - 1) / kCPass);
    return 2 * nwork + 8 < ((int64_t)1 << 31);
}

hipError_t launch_apply_pair(bool corr, int ncomp, const Geom &g, int C, int64_t nb, float scale,
                             const float *nz, const float *x, const float *y, float *dx,
                             float *dy, hipStream_t s) {
    // dx = A ⊗ y (- rowsum(A) .* x), dy = Aᵀ ⊗ x (- colsum(A) .* y)
    ApplyArgs f{}, t{};
    f.g = t.g = g;
    f.C = t.C = C;
    f.corr = t.corr = corr ? 1 : 0;
    f.scale = t.scale = scale;
    f.nz = t.nz = nz;
    f.x = y;
    f.z = x;
    f.y = dx;
    t.x = x;
    t.z = y;
    t.y = dy;
    if (pair_rows(g, C, ncomp, nb))
        return ncomp == 1 ? dispatch_pair<1>(f, t, nb, s) : dispatch_pair<2>(f, t, nb, s);
    if (band_supported(g))
        return ncomp == 1 ? launch_band_pair<1>(f, t, nb, s) : launch_band_pair<2>(f, t, nb, s);
    return ncomp == 1 ? launch_wide_pair<1>(f, t, nb, s) : launch_wide_pair<2>(f, t, nb, s);
}

hipError_t launch_colsum_wide(const Geom &g, int64_t nb, const float *nz, float *out,
                              hipStream_t s) {
    ApplyArgs a{};
    a.g = g;
    a.C = 1;
    a.nz = nz;
    a.y = out;
    return launch_wide<1, true, true>(a, nb, s);
}

hipError_t launch_colsum_rb(const Geom &g, int64_t nb, const float *nz, float *out, hipStream_t s) {
    switch (g.ws) {
        case 3: return launch_colsum_t<3>(g, nb, nz, out, s);
        case 5: return launch_colsum_t<5>(g, nb, nz, out, s);
        case 7: return launch_colsum_t<7>(g, nb, nz, out, s);
        case 9: return launch_colsum_t<9>(g, nb, nz, out, s);
        case 11: return launch_colsum_t<11>(g, nb, nz, out, s);
        case 13: return launch_colsum_t<13>(g, nb, nz, out, s);
        case 15: return launch_colsum_t<15>(g, nb, nz, out, s);
        default: return hipErrorNotSupported;
    }
}

}  // namespace circatt
