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
// Work decomposition.  A workgroup (4 wavefronts) owns a tile of "register
// pixels" (queries, or keys in BWDKV) of one (head, batch) unit and stages the
// circularly wrapped halo of the other side (K/V, or Q/dY) in LDS, row chunk
// by row chunk.  Each wavefront holds a block of 16 register pixels and walks
// blocks of 16 LDS pixels covering its window, using
// v_mfma_f32_16x16x4f32 for every contraction:
//   S^T[key][q]   = sum_c K[key][c] Q[q][c]     A = K (LDS),  B = Q (regs)
//   y^T[c][q]    += sum_k V[k][c] P^T[k][q]     A = V (LDS),  B = P (regs)
// The S^T accumulator layout (lane j+16g, item r = key 4g+r, query j) is
// exactly the B-operand layout of the next product, so probabilities never
// leave registers.  Pairs outside the window are masked to zero weight; with
// 2D register blocks 8x2 and LDS blocks 2x8 the dense 16x16 products are
// 64% useful at ws = 15 (1D: 16-pixel runs).
//
// Layouts.  Global signals are the reference's planar (P, C) per unit
// (complex: interleaved pairs, treated as 2 real components per channel).
// LDS holds [pixel][component] rows padded to NC+4 floats so that both the
// 4-wide row reads (ds_read_b128) and the transposed single reads are free of
// bank conflicts.
#include "circatt_common.h"
#include "circatt_kernels.h"

namespace circatt {

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma4(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

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

struct FArgs {
    const float *q, *k, *v, *y, *dy, *lse;
    float *yout, *lse_out, *dq, *dk, *dv, *dbuf, *nz;
    Geom g;
    int p1, p2;           // half windows along dims 1 and 2 (p2 = 0 in 1D)
    int dh, ncomp, ncr;   // channels per unit, components per channel, dh*ncomp
    int64_t unit_stride;  // floats per unit (P*dh*ncomp)
    float scale, c2;      // similarity scale and scale*log2(e)
    int tiles_h, tiles_w;
    int halo_h, halo_w;   // staged halo box: rows along dim 1, columns along dim 2
    int chunk_rows, cr;   // halo rows per LDS chunk, LDS row stride in pixels
    int nkh, nkw;         // LDS blocks per wavefront along dims 1 and 2
};

__device__ __forceinline__ int64_t comp_index(const FArgs &a, int64_t pix, int comp) {
    if (a.ncomp == 1) return pix + a.g.P * comp;
    return 2 * (pix + a.g.P * (comp >> 1)) + (comp & 1);
}

// Stage halo rows [cr0, cr0+crn) x columns [0, halo_w) of one unit's signal
// into LDS as [pixel][NC+4] (zero padding beyond the real components).
template <int NC>
__device__ void stage_tensor(float *lds, const float *base, const FArgs &a, int h0, int w0,
                             int cr0, int crn) {
    constexpr int PS = NC + 4;
    const int nch = NC / a.ncomp;
    const int items = crn * a.halo_w * nch;
    for (int i = threadIdx.x; i < items; i += blockDim.x) {
        const int hl = i % crn;
        const int rest = i / crn;
        const int wl = rest % a.halo_w;
        const int c = rest / a.halo_w;
        const int gh = pmod(h0 - a.p1 + cr0 + hl, a.g.n1);
        const int gw = pmod(w0 - a.p2 + wl, a.g.n2);
        const int64_t pix = gh + (int64_t)a.g.n1 * gw;
        float *dst = lds + (hl + a.cr * wl) * PS;
        if (a.ncomp == 1) {
            dst[c] = c < a.dh ? base[pix + a.g.P * c] : 0.f;
        } else {
            float2 val = make_float2(0.f, 0.f);
            if (c < a.dh) val = *reinterpret_cast<const float2 *>(base + 2 * (pix + a.g.P * c));
            dst[2 * c] = val.x;
            dst[2 * c + 1] = val.y;
        }
    }
}

__device__ void stage_scalar(float *lds, const float *src, const FArgs &a, int h0, int w0,
                             int cr0, int crn) {
    const int items = crn * a.halo_w;
    for (int i = threadIdx.x; i < items; i += blockDim.x) {
        const int hl = i % crn;
        const int wl = i / crn;
        const int gh = pmod(h0 - a.p1 + cr0 + hl, a.g.n1);
        const int gw = pmod(w0 - a.p2 + wl, a.g.n2);
        lds[hl + a.cr * wl] = src[gh + (int64_t)a.g.n1 * gw];
    }
}

// out[px] = mul * out[px] + add * sum_c T[px][c]^2 over the staged chunk
template <int NC>
__device__ void chunk_sqnorm(float *out, const float *T, const FArgs &a, int crn, float mul,
                             float add) {
    constexpr int PS = NC + 4;
    const int items = crn * a.halo_w;
    for (int i = threadIdx.x; i < items; i += blockDim.x) {
        const int px = (i % crn) + a.cr * (i / crn);
        const float *t = T + px * PS;
        float s = 0.f;
#pragma unroll
        for (int c = 0; c < NC; ++c) s += t[c] * t[c];
        out[px] = (mul != 0.f ? mul * out[px] : 0.f) + add * s;
    }
}

__device__ __forceinline__ float xsum16_32(float v) {
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}
__device__ __forceinline__ float xmax16_32(float v) {
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}

template <int NSP, int NC, bool DIST, int MODE>
__global__ __launch_bounds__(256) void fused_kernel(FArgs a) {
    using G = FGeo<NSP>;
    constexpr int PS = NC + 4;
    constexpr int NT = NC / 16;  // 16-component tiles
    constexpr int NS = NC / 4;   // MFMA k-steps
    constexpr bool TWO = MODE != MODE_SIM;
    extern __shared__ float smem[];

    // ---- tile of this workgroup; consecutive tiles stay on one XCD ----
    const int ntiles = a.tiles_h * a.tiles_w;
    int tile = blockIdx.x;
    if ((ntiles & 7) == 0) tile = (tile & 7) * (ntiles >> 3) + (tile >> 3);
    const int unit = blockIdx.y;
    const int h0 = (tile % a.tiles_h) * G::TH;
    const int w0 = (tile / a.tiles_h) * G::TW;

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int wh = G::wave_h(wv), ww = G::wave_w(wv);
    const int jh = j % G::QH, jw = j / G::QH;
    const int rh = h0 + wh + jh, rw = w0 + ww + jw;
    const bool rvalid = rh < a.g.n1 && rw < a.g.n2;
    const int64_t rpix = rvalid ? (int64_t)rh + (int64_t)a.g.n1 * rw : 0;
    const int64_t uoff = (int64_t)unit * a.unit_stride;
    const int64_t soff = (int64_t)unit * a.g.P;  // per-row scalars (lse, D)

    // LDS layout of the current chunk
    const int chunk_px = a.cr * a.halo_w;
    float *T0 = smem;
    float *T1 = smem + (TWO ? chunk_px * PS : 0);
    float *S0 = smem + (TWO ? 2 : 1) * chunk_px * PS;
    float *S1 = S0 + chunk_px;

    // per-lane constants: element kk = 4g + r of an LDS block at (bh, bw)
    // has offset (bh + offh[r], bw + offw[r]) from this lane's pixel and LDS
    // position blockpix + eoff[r]; the lane's A-operand row j sits at aoff.
    int offh[4], offw[4], eoff[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int kk = 4 * g + r;
        offh[r] = kk % G::KH - wh - jh - a.p1;
        offw[r] = kk / G::KH - ww - jw - a.p2;
        eoff[r] = kk % G::KH + a.cr * (kk / G::KH);
    }
    const int aoff = j % G::KH + a.cr * (j / G::KH);
    const unsigned span1 = 2 * a.p1, span2 = 2 * a.p2;

    // ---- register operands: component 16*(s/4) + 4g + s%4 at k-step s ----
    const float *rbase0 = (MODE == MODE_BWDKV ? a.k : a.q) + uoff;
    float reg0[NS], reg1[NS];
    float sq = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const int comp = 16 * (s >> 2) + 4 * g + (s & 3);
        reg0[s] = comp < a.ncr ? rbase0[comp_index(a, rpix, comp)] : 0.f;
        sq += reg0[s] * reg0[s];
    }
    float dsum = 0.f;  // BWDQ: <dy, y> partial
    if (MODE == MODE_BWDQ || MODE == MODE_BWDKV) {
        const float *rbase1 = (MODE == MODE_BWDKV ? a.v : a.dy) + uoff;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int comp = 16 * (s >> 2) + 4 * g + (s & 3);
            reg1[s] = comp < a.ncr ? rbase1[comp_index(a, rpix, comp)] : 0.f;
            if (MODE == MODE_BWDQ && comp < a.ncr)
                dsum += reg1[s] * a.y[uoff + comp_index(a, rpix, comp)];
        }
    }
    if (DIST) sq = xsum16_32(sq);
    float dq_d = 0.f;
    if (MODE == MODE_BWDQ) dq_d = xsum16_32(dsum);

    // per-row quantities
    float m = -1e30f, lsum = 0.f;  // FWD online softmax (log2 domain)
    float lseb = 0.f;              // BWDQ: log2-domain subtrahend for P
    if (MODE == MODE_BWDQ) lseb = a.lse[soff + rpix] * kLog2e + (DIST ? 0.5f * sq * a.c2 : 0.f);
    const float rbias = DIST ? -0.5f * sq : 0.f;  // SIM: -|q|^2/2 ; BWDKV: key bias -|k|^2/2
    float corr = 0.f;                              // Distance row/col sum of dS

    f4 acc0[NT], acc1[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        acc0[t] = f4{0.f, 0.f, 0.f, 0.f};
        acc1[t] = f4{0.f, 0.f, 0.f, 0.f};
    }

    for (int cr0 = 0; cr0 < a.halo_h; cr0 += a.chunk_rows) {
        const int crn = min(a.chunk_rows, a.halo_h - cr0);
        __syncthreads();
        if (MODE == MODE_BWDKV) {
            stage_tensor<NC>(T0, a.q + uoff, a, h0, w0, cr0, crn);
            stage_tensor<NC>(T1, a.dy + uoff, a, h0, w0, cr0, crn);
            stage_scalar(S0, a.lse + soff, a, h0, w0, cr0, crn);
            stage_scalar(S1, a.dbuf + soff, a, h0, w0, cr0, crn);
        } else {
            stage_tensor<NC>(T0, a.k + uoff, a, h0, w0, cr0, crn);
            if (TWO) stage_tensor<NC>(T1, a.v + uoff, a, h0, w0, cr0, crn);
        }
        __syncthreads();
        if (MODE == MODE_BWDKV) {
            // lse -> log2-domain subtrahend including the Distance |q|^2/2 term
            chunk_sqnorm<NC>(S0, T0, a, crn, kLog2e, DIST ? 0.5f * a.c2 : 0.f);
            __syncthreads();
        } else if (DIST) {
            chunk_sqnorm<NC>(S0, T0, a, crn, 0.f, -0.5f);
            __syncthreads();
        }

        // this wavefront's LDS-block rows inside the chunk
        const int lo = cr0 - wh, hi = cr0 + crn - wh;
        const int ib = lo > 0 ? (lo + G::KH - 1) / G::KH : 0;
        const int ie = hi > 0 ? min(a.nkh, (hi + G::KH - 1) / G::KH) : 0;
        for (int i = ib; i < ie; ++i) {
            const int bh = wh + G::KH * i;
            for (int jb = 0; jb < a.nkw; ++jb) {
                const int bw = ww + G::KW * jb;
                const int bpix = (bh - cr0) + a.cr * bw;
                bool val[4];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    val[r] = (unsigned)(bh + offh[r] + a.p1) <= span1 &&
                             (unsigned)(bw + offw[r] + a.p2) <= span2;

                // first product: rows = LDS pixels (A), columns = register pixels (B)
                f4 s = f4{0.f, 0.f, 0.f, 0.f};
                f4 dp = f4{0.f, 0.f, 0.f, 0.f};
                {
                    const float *ap = T0 + (bpix + aoff) * PS + 4 * g;
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const f4 x = *reinterpret_cast<const f4 *>(ap + 16 * t);
                        s = mfma4(x[0], reg0[4 * t + 0], s);
                        s = mfma4(x[1], reg0[4 * t + 1], s);
                        s = mfma4(x[2], reg0[4 * t + 2], s);
                        s = mfma4(x[3], reg0[4 * t + 3], s);
                    }
                }
                if (MODE == MODE_BWDQ || MODE == MODE_BWDKV) {
                    const float *ap = T1 + (bpix + aoff) * PS + 4 * g;
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const f4 x = *reinterpret_cast<const f4 *>(ap + 16 * t);
                        dp = mfma4(x[0], reg1[4 * t + 0], dp);
                        dp = mfma4(x[1], reg1[4 * t + 1], dp);
                        dp = mfma4(x[2], reg1[4 * t + 2], dp);
                        dp = mfma4(x[3], reg1[4 * t + 3], dp);
                    }
                }

                if constexpr (MODE == MODE_SIM) {
                    if (rvalid) {
                        float *nzu = a.nz + (int64_t)unit * a.g.P * a.g.K + rpix * a.g.K;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if (val[r]) {
                                float sv = s[r];
                                if (DIST) sv += S0[bpix + eoff[r]] + rbias;
                                nzu[offset_slot(a.g, rpix, bh + offh[r], bw + offw[r])] =
                                    sv * a.scale;
                            }
                        }
                    }
                } else if constexpr (MODE == MODE_FWD) {
                    float tt[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float sv = s[r];
                        if (DIST) sv += S0[bpix + eoff[r]];
                        tt[r] = val[r] ? sv * a.c2 : -INFINITY;
                    }
                    const float mb =
                        xmax16_32(fmaxf(fmaxf(tt[0], tt[1]), fmaxf(tt[2], tt[3])));
                    const float mn = fmaxf(m, mb);
                    const float alpha = fast_exp2(m - mn);
                    m = mn;
                    float pr[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) pr[r] = fast_exp2(tt[r] - mn);
                    lsum = lsum * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
#pragma unroll
                    for (int t = 0; t < NT; ++t) acc0[t] *= alpha;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float *vp = T1 + (bpix + eoff[r]) * PS + j;
#pragma unroll
                        for (int t = 0; t < NT; ++t) acc0[t] = mfma4(vp[16 * t], pr[r], acc0[t]);
                    }
                } else if constexpr (MODE == MODE_BWDQ) {
                    float ds[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float sv = s[r];
                        if (DIST) sv += S0[bpix + eoff[r]];
                        const float pr = val[r] ? fast_exp2(sv * a.c2 - lseb) : 0.f;
                        ds[r] = pr * (dp[r] - dq_d);
                        if (DIST) corr += ds[r];
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float *kp = T0 + (bpix + eoff[r]) * PS + j;
#pragma unroll
                        for (int t = 0; t < NT; ++t) acc0[t] = mfma4(kp[16 * t], ds[r], acc0[t]);
                    }
                } else {  // MODE_BWDKV
                    float pr[4], ds[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int e = bpix + eoff[r];
                        pr[r] = val[r] ? fast_exp2((s[r] + rbias) * a.c2 - S0[e]) : 0.f;
                        ds[r] = pr[r] * (dp[r] - S1[e]);
                        if (DIST) corr += ds[r];
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float *yp = T1 + (bpix + eoff[r]) * PS + j;
                        const float *qp = T0 + (bpix + eoff[r]) * PS + j;
#pragma unroll
                        for (int t = 0; t < NT; ++t) {
                            acc0[t] = mfma4(yp[16 * t], pr[r], acc0[t]);  // dv
                            acc1[t] = mfma4(qp[16 * t], ds[r], acc1[t]);  // dk
                        }
                    }
                }
            }
        }
    }

    // ---- epilogues: lane (j, g) holds component 16t + 4g + r of pixel j ----
    if constexpr (MODE == MODE_FWD) {
        lsum = xsum16_32(lsum);
        const float inv = 1.f / lsum;
        if (rvalid) {
            float *yb = a.yout + uoff;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int comp = 16 * t + 4 * g + r;
                    if (comp < a.ncr) yb[comp_index(a, rpix, comp)] = acc0[t][r] * inv;
                }
            if (g == 0)
                a.lse_out[soff + rpix] =
                    (m + log2f(lsum)) * kLn2 - (DIST ? 0.5f * sq * a.scale : 0.f);
        }
    } else if constexpr (MODE == MODE_BWDQ) {
        if (DIST) corr = xsum16_32(corr);
        if (rvalid) {
            float *ob = a.dq + uoff;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int comp = 16 * t + 4 * g + r;
                    float val = acc0[t][r];
                    if (DIST) val -= corr * reg0[4 * t + r];
                    if (comp < a.ncr) ob[comp_index(a, rpix, comp)] = val * a.scale;
                }
            if (g == 0) a.dbuf[soff + rpix] = dq_d;
        }
    } else if constexpr (MODE == MODE_BWDKV) {
        if (DIST) corr = xsum16_32(corr);
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
                        vb[idx] = acc0[t][r];
                        float val = acc1[t][r];
                        if (DIST) val -= corr * reg0[4 * t + r];
                        kb[idx] = val * a.scale;
                    }
                }
        }
    }
}

// ---------------------------------------------------------------------------
// host planning and dispatch
// ---------------------------------------------------------------------------
namespace {

struct Plan {
    FArgs a;
    int nc;
    size_t lds_bytes;
    dim3 grid;
    bool ok;
};

constexpr size_t kLdsBudget = 80 * 1024;  // two workgroups per CU
constexpr size_t kLdsMax = 160 * 1024;

Plan make_plan(FusedMode mode, const FusedProblem &pr) {
    Plan pl{};
    FArgs &a = pl.a;
    a.q = pr.q; a.k = pr.k; a.v = pr.v; a.y = pr.y; a.dy = pr.dy; a.lse = pr.lse;
    a.yout = pr.yout; a.lse_out = pr.lse_out; a.dq = pr.dq; a.dk = pr.dk; a.dv = pr.dv;
    a.dbuf = pr.dbuf; a.nz = pr.nz;
    a.g = pr.g;
    a.dh = pr.dh;
    a.ncomp = pr.ncomp;
    a.ncr = pr.dh * pr.ncomp;
    a.unit_stride = pr.g.P * pr.dh * pr.ncomp;
    a.scale = pr.scale;
    a.c2 = pr.scale * kLog2e;
    pl.nc = a.ncr <= 16 ? 16 : a.ncr <= 32 ? 32 : a.ncr <= 64 ? 64 : 0;
    if (pl.nc == 0) return pl;
    const int PS = pl.nc + 4;
    const int p = pr.g.p;
    const bool dist = pr.kind == 1;
    const int ntensor = mode == MODE_SIM ? 1 : 2;
    const int nscalar = mode == MODE_BWDKV ? 2 : (dist ? 1 : 0);
    const size_t bpp = (size_t)(ntensor * PS + nscalar) * sizeof(float);
    if (pr.g.nsp == 2) {
        a.p1 = a.p2 = p;
        a.nkh = (8 + 2 * p + 1) / 2;
        a.nkw = (2 + 2 * p + 7) / 8;
        a.halo_h = 2 * a.nkh;
        a.halo_w = 6 + 8 * a.nkw;
        a.tiles_h = (pr.g.n1 + 7) / 8;
        a.tiles_w = (pr.g.n2 + 7) / 8;
        // largest even chunk whose padded stride (cr % 4 == 2) fits the budget
        auto stride_of = [](int rows) { return rows + ((2 - rows % 4) + 4) % 4; };
        int rows = a.halo_h;
        for (size_t budget : {kLdsBudget, kLdsMax}) {
            rows = a.halo_h;
            while (rows >= 2 && (size_t)stride_of(rows) * a.halo_w * bpp > budget) rows -= 2;
            if (rows >= 2) break;
        }
        if (rows < 2) return pl;
        a.chunk_rows = rows;
        a.cr = stride_of(rows);
    } else {
        a.p1 = p;
        a.p2 = 0;
        a.nkh = (16 + 2 * p + 15) / 16;
        a.nkw = 1;
        a.halo_h = 48 + 16 * a.nkh;
        a.halo_w = 1;
        a.tiles_h = (pr.g.n1 + 63) / 64;
        a.tiles_w = 1;
        a.chunk_rows = a.halo_h;
        a.cr = a.halo_h;
        if ((size_t)a.cr * bpp > kLdsMax) return pl;
    }
    pl.lds_bytes = (size_t)a.cr * a.halo_w * bpp;
    pl.grid = dim3((unsigned)(a.tiles_h * a.tiles_w), (unsigned)pr.nunits);
    pl.ok = pr.nunits <= 65535;
    return pl;
}

template <int NSP, int NC, bool DIST, int MODE>
hipError_t launch_inst(const Plan &pl, hipStream_t s) {
    auto kern = fused_kernel<NSP, NC, DIST, MODE>;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)kLdsMax);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL(kern, pl.grid, dim3(256), pl.lds_bytes, s, pl.a);
    return hipGetLastError();
}

template <int NSP, int NC, bool DIST>
hipError_t launch_mode(FusedMode mode, const Plan &pl, hipStream_t s) {
    switch (mode) {
    case MODE_FWD: return launch_inst<NSP, NC, DIST, MODE_FWD>(pl, s);
    case MODE_SIM: return launch_inst<NSP, NC, DIST, MODE_SIM>(pl, s);
    case MODE_BWDQ: return launch_inst<NSP, NC, DIST, MODE_BWDQ>(pl, s);
    case MODE_BWDKV: return launch_inst<NSP, NC, DIST, MODE_BWDKV>(pl, s);
    }
    return hipErrorInvalidValue;
}

template <int NSP, int NC>
hipError_t launch_kind(FusedMode mode, bool dist, const Plan &pl, hipStream_t s) {
    return dist ? launch_mode<NSP, NC, true>(mode, pl, s) : launch_mode<NSP, NC, false>(mode, pl, s);
}

template <int NSP>
hipError_t launch_nc(FusedMode mode, bool dist, const Plan &pl, hipStream_t s) {
    switch (pl.nc) {
    case 16: return launch_kind<NSP, 16>(mode, dist, pl, s);
    case 32: return launch_kind<NSP, 32>(mode, dist, pl, s);
    case 64: return launch_kind<NSP, 64>(mode, dist, pl, s);
    }
    return hipErrorNotSupported;
}

}  // namespace

bool fused_supported(FusedMode mode, const FusedProblem &pr) {
    Plan pl = make_plan(mode, pr);
    return pl.ok;
}

hipError_t launch_fused(FusedMode mode, const FusedProblem &pr, hipStream_t s) {
    Plan pl = make_plan(mode, pr);
    if (!pl.ok) return hipErrorNotSupported;
    if (pl.grid.x == 0 || pl.grid.y == 0) return hipSuccess;
    return pr.g.nsp == 1 ? launch_nc<1>(mode, pr.kind == 1, pl, s)
                         : launch_nc<2>(mode, pr.kind == 1, pl, s);
}

}  // namespace circatt
