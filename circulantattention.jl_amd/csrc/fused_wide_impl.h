// Fused circulant attention for heads wider than 64 real components: a
// channel-chunked walk.
//
// The other fused kernels hold a whole pixel's components in LDS and in
// registers (at most 64).  Here the window's score products are summed over
// chunks of CC = 32 components: for each stage of a few LDS block rows the
// staged tensor is loaded chunk by chunk and every chunk's products are added
// into the stage's score registers (at most MAXB blocks per wavefront).  The
// outputs are formed in passes of OC = 64 components (y; dq; dk and dv), each
// pass walking the window again, so registers stay bounded for any head
// width at the price of recomputing the scores per pass.
//
// Work decomposition, window geometry, masks, softmax and the backward's two
// passes (query-centric: dq and D; key-centric: dk and dv, no atomics) are
// those of fused_impl.h; its helpers (block_product, block_accumulate, the
// lane layouts) are reused.  Products run on v_mfma_f32_16x16x4f32 (Float32).
#pragma once
#include "fused_impl.h"

namespace circatt {
namespace wide {

constexpr int CC = 32;       // components per score chunk
constexpr int OC = 64;       // components per output pass
constexpr int PS = OC + 4;   // LDS floats per staged pixel
constexpr int MAXB = 8;      // LDS blocks per wavefront and stage
constexpr int THREADS = 256;
constexpr size_t kLdsBudget = 80 * 1024;  // two workgroups per CU

// Stage geometry on the host: rb block rows per stage, LDS column stride cr
// (pixels), nst stages per pass.  ntensor staged tensors, nscal scalars.
struct Plan {
    HaloGeo hg;
    int rb, cr, nst, lds_floats;
    bool ok;
};
inline Plan plan(int nsp, int p, int ntensor, int nscal) {
    Plan w{};
    HaloGeo &h = w.hg;
    int kh;
    if (nsp == 2) {
        h.p1 = h.p2 = p;
        h.nkh = (8 + 2 * p + 1) / 2;
        h.nkw = (2 + 2 * p + 7) / 8;
        h.halo_h = 2 * h.nkh;
        h.halo_w = 6 + 8 * h.nkw;
        kh = 2;
    } else {
        h.p1 = p;
        h.p2 = 0;
        h.nkh = (16 + 2 * p + 15) / 16;
        h.nkw = 1;
        h.halo_h = 48 + 16 * h.nkh;
        h.halo_w = 1;
        kh = 16;
    }
    if (h.nkw > MAXB) return w;
    for (w.rb = std::min(h.nkh, MAXB / h.nkw); w.rb >= 1; --w.rb) {
        const int rows = w.rb * kh;
        w.cr = nsp == 2 ? rows + ((2 - rows % 4) + 4) % 4 : rows;
        const int px = w.cr * h.halo_w;
        w.lds_floats = px * (PS * ntensor + nscal);
        if ((size_t)w.lds_floats * 4 <= kLdsBudget) break;
    }
    if (w.rb < 1) return w;
    w.nst = (h.halo_h + w.rb * kh - 1) / (w.rb * kh);
    h.ok = w.ok = true;
    return w;
}

template <int NSP, bool DIST, int MODE>
__global__ __launch_bounds__(THREADS, 2) void wide_kernel(FArgs a) {
    using G = FGeo<NSP>;
    constexpr int KH = G::KH, KW = G::KW;
    constexpr bool TWO = MODE == MODE_BWDQ || MODE == MODE_BWDKV;
    constexpr int NTC = CC / 16, NTO = OC / 16;
    const int p1 = a.hg.p1, p2 = a.hg.p2, nkh = a.hg.nkh, nkw = a.hg.nkw;
    const int halo_h = a.hg.halo_h, halo_w = a.hg.halo_w;
    const int RB = a.rb, CR = a.cr, NST = a.nst, NCC = a.ncc, NOC = a.noc;

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int wh = G::wave_h(wv), ww = G::wave_w(wv);
    const int jh = j % G::QH, jw = j / G::QH;

    // LDS: tensor slots [pixel][PS] (T0, T1), then per-pixel scalars S0, S1
    const int spx = CR * halo_w;
    const int oT1 = spx * PS;
    const int oS0 = (TWO ? 2 : 1) * spx * PS;
    const int oS1 = oS0 + spx;

    // per-lane LDS geometry (as fused_kernel): A-operand row, element 0 pixel,
    // element offsets and window tests
    const int wbase = wh + CR * ww;
    const int kk0 = 4 * g;
    const int laneA = (wbase + j % KH + CR * (j / KH)) * PS + 4 * g;
    const int laneE = wbase + kk0 % KH + CR * (kk0 / KH);
    int rdel[4], rdelPS[4], hoff[4], woff[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        rdel[r] = KH >= 4 ? r : r % KH + CR * (r / KH);
        rdelPS[r] = rdel[r] * PS;
        hoff[r] = (kk0 + r) % KH - jh;
        woff[r] = (kk0 + r) / KH - jw;
    }
    const unsigned span1 = 2 * p1, span2 = 2 * p2;
    const float c2 = a.c2;

    // components 16 t + 4 g + i (t < NT) from base c0 of the lane's pixel,
    // minus those of mu when mu is given
    auto load_reg = [&](auto NT_, auto &dst, const float *base, int64_t rpix, int c0,
                        const float *mu = nullptr, int64_t p0 = 0) {
        constexpr int NT = decltype(NT_)::value;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int comp = c0 + 16 * t + 4 * g + i;
                const int64_t ci = comp_index(a, 0, min(comp, a.ncr - 1));
                const bool ok = comp < a.ncr;
                dst[4 * t + i] = ok ? base[comp_index(a, rpix, 0) + ci] : 0.f;
                if (mu) dst[4 * t + i] -= ok ? mu[comp_index(a, p0, 0) + ci] : 0.f;
            }
    };
    using NTc = std::integral_constant<int, NTC>;
    using NTo = std::integral_constant<int, NTO>;

    for (int k = 0;; ++k) {
        const int item = item_of(a, k);
        if (item >= a.nitems) break;  // uniform over the workgroup
        const int ntiles = a.tiles_h * a.tiles_w;
        const int unit = item / ntiles;
        const int tile = item - unit * ntiles;
        const int h0 = (tile % a.tiles_h) * G::TH, w0 = (tile / a.tiles_h) * G::TW;
        const int rh = h0 + wh + jh, rw = w0 + ww + jw;
        const bool rvalid = rh < a.g.n1 && rw < a.g.n2;
        const int64_t rpix = rvalid ? (int64_t)rh + (int64_t)a.g.n1 * rw : 0;
        const int64_t uoff = unit_base(a, unit);
        const int64_t soff = (int64_t)unit * a.g.P;
        const float *R0 = (MODE == MODE_BWDKV ? a.k : a.q) + uoff;  // register side
        const float *R1 = (MODE == MODE_BWDKV ? a.v : a.dy) + uoff;
        const float *T0 = (MODE == MODE_BWDKV ? a.q : a.k) + uoff;  // staged side
        const float *T1 = (MODE == MODE_BWDKV ? a.dy : a.v) + uoff;
        // Distance: q and k centred on mu = k at the tile's first pixel p0
        // wherever they are loaded (the expansion q.k - |k|^2 / 2 - |q|^2 / 2
        // of -|q - k|^2 / 2 then scales with the spread of the data, not its
        // offset; |q - k| and the gradient terms dS (k - q) are unchanged)
        const float *MU = DIST ? a.k + uoff : nullptr;
        const int64_t p0 = (int64_t)h0 + (int64_t)a.g.n1 * w0;

        // per register pixel, over all components: |r0|^2 and, in the
        // query-centric pass, D = <dy, y>
        float qq = 0.f, dd = 0.f;
        for (int c0 = 0; c0 < a.ncr; c0 += CC) {
            float x[4 * NTC], y[4 * NTC];
            load_reg(NTc{}, x, R0, rpix, c0, MU, p0);
#pragma unroll
            for (int i = 0; i < 4 * NTC; ++i) qq += x[i] * x[i];
            if constexpr (MODE == MODE_BWDQ) {
                float yy[4 * NTC];
                load_reg(NTc{}, y, R1, rpix, c0);
                load_reg(NTc{}, yy, a.y + uoff, rpix, c0);
#pragma unroll
                for (int i = 0; i < 4 * NTC; ++i) dd += y[i] * yy[i];
            }
        }
        const float sq = DIST ? xsum16_32(qq) : 0.f;
        const float dq_d = MODE == MODE_BWDQ ? xsum16_32(dd) : 0.f;
        const float lseb = MODE == MODE_BWDQ
                               ? a.lse[soff + rpix] * kLog2e + (DIST ? 0.5f * sq * c2 : 0.f)
                               : 0.f;
        const float rbias = DIST ? -0.5f * sq : 0.f;  // key-centric: register key's -|k|^2/2
        if (MODE == MODE_BWDQ && rvalid && g == 0) a.dbuf[soff + rpix] = dq_d;

        // stage components [c0, c0 + nc) of X (and Y) for halo rows
        // [r0, r0 + nrows) into T0 (T1); the scalars as the mode needs them
        auto stage = [&](int r0, int nrows, int c0, int nc, const float *X, const float *Y,
                         int cc_scal) {
            const int npx = nrows * halo_w;
            for (int px = threadIdx.x; px < npx; px += THREADS) {
                const int wl = px / nrows, hl = px - wl * nrows;
                const int slot = hl + CR * wl;
                const int64_t gp = pmod(h0 - p1 + r0 + hl, a.g.n1) +
                                   (int64_t)a.g.n1 * pmod(w0 - p2 + wl, a.g.n2);
                float n2 = 0.f;
                for (int c = 0; c < nc; c += 4) {
                    f4 xv, yv;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int comp = c0 + c + i;
                        const bool ok = comp < a.ncr;
                        const int64_t idx = comp_index(a, gp, min(comp, a.ncr - 1));
                        const float mu = ok && MU ? MU[comp_index(a, p0, comp)] : 0.f;
                        xv[i] = ok ? X[idx] - (X == T0 ? mu : 0.f) : 0.f;
                        if (Y) yv[i] = ok ? Y[idx] - (Y == T0 ? mu : 0.f) : 0.f;
                        n2 += xv[i] * xv[i];
                    }
                    *reinterpret_cast<f4 *>(&circatt_lds[slot * PS + c]) = xv;
                    if (Y) *reinterpret_cast<f4 *>(&circatt_lds[oT1 + slot * PS + c]) = yv;
                }
                if (cc_scal >= 0) {
                    // scalars of the score chunks: cc_scal = chunk index
                    float *s0 = &circatt_lds[oS0 + slot];
                    if constexpr (MODE == MODE_BWDKV) {
                        // log2-domain subtrahend lse log2(e) [+ c2 |q|^2 / 2], and D
                        if (cc_scal == 0) {
                            s0[0] = a.lse[soff + gp] * kLog2e;
                            circatt_lds[oS1 + slot] = a.dbuf[soff + gp];
                        }
                        if (DIST) s0[0] += 0.5f * c2 * n2;
                    } else if (DIST) {
                        // key bias -|k|^2 / 2, summed over the chunks
                        s0[0] = (cc_scal == 0 ? 0.f : s0[0]) - 0.5f * n2;
                    }
                }
            }
        };

        for (int oc = 0; oc < NOC; ++oc) {
            const int oc0 = oc * OC;
            float m = -1e30f, lsum = 0.f, corr = 0.f;
            f4 acc[NTO], acc2[NTO];
#pragma unroll
            for (int t = 0; t < NTO; ++t) {
                acc[t] = f4{0.f, 0.f, 0.f, 0.f};
                acc2[t] = f4{0.f, 0.f, 0.f, 0.f};
            }
            for (int st = 0; st < NST; ++st) {
                const int r0 = st * RB * KH;
                const int nrows = min(RB * KH, halo_h - r0);
                const int lo = r0 - wh, hi = r0 + nrows - wh;
                const int ib = lo > 0 ? (lo + KH - 1) / KH : 0;
                const int ie = hi > 0 ? min(nkh, (hi + KH - 1) / KH) : 0;
                const int nb = ie > ib ? (ie - ib) * nkw : 0;

                f4 S[MAXB], DP[MAXB];
#pragma unroll
                for (int b = 0; b < MAXB; ++b) {
                    S[b] = f4{0.f, 0.f, 0.f, 0.f};
                    DP[b] = f4{0.f, 0.f, 0.f, 0.f};
                }
                for (int cc = 0; cc < NCC; ++cc) {
                    __syncthreads();  // the previous stage's LDS reads are done
                    stage(r0, nrows, cc * CC, CC, T0, TWO ? T1 : nullptr, cc);
                    __syncthreads();
                    float x0[4 * NTC], x1[4 * NTC];
                    load_reg(NTc{}, x0, R0, rpix, cc * CC, MU, p0);
                    if (TWO) load_reg(NTc{}, x1, R1, rpix, cc * CC);
                    int bi = ib, bj = 0;
#pragma unroll
                    for (int b = 0; b < MAXB; ++b) {
                        if (b < nb) {
                            const int bo = (KH * bi - r0) + CR * (KW * bj);
                            S[b] += block_product<NTC>(laneA + bo * PS, x0);
                            if (TWO) DP[b] += block_product<NTC>(oT1 + laneA + bo * PS, x1);
                        }
                        if (++bj == nkw) {
                            bj = 0;
                            ++bi;
                        }
                    }
                }

                // probabilities (FWD) or p and dS (backward) of the stage's blocks
                float pr[MAXB][4], ds[MAXB][4];
                {
                    float lm = -INFINITY;
                    int bi = ib, bj = 0;
#pragma unroll
                    for (int b = 0; b < MAXB; ++b) {
                        const int bo = (KH * bi - r0) + CR * (KW * bj);
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const bool val = b < nb &&
                                             (unsigned)(KH * bi + hoff[r]) <= span1 &&
                                             (unsigned)(KW * bj + woff[r]) <= span2;
                            const int e = laneE + bo + rdel[r];
                            float sv = S[b][r];
                            if constexpr (MODE == MODE_FWD) {
                                if (DIST) sv += val ? circatt_lds[oS0 + e] : 0.f;
                                pr[b][r] = val ? sv : -INFINITY;
                                lm = fmaxf(lm, pr[b][r]);
                            } else if constexpr (MODE == MODE_BWDQ) {
                                if (DIST) sv += val ? circatt_lds[oS0 + e] : 0.f;
                                const float p = val ? fast_exp2(fmaf(sv, c2, -lseb)) : 0.f;
                                pr[b][r] = p;
                                ds[b][r] = p * (DP[b][r] - dq_d);
                                if (DIST) corr += ds[b][r];
                            } else {
                                const float p =
                                    val ? fast_exp2(fmaf(sv + rbias, c2, -circatt_lds[oS0 + e])) : 0.f;
                                pr[b][r] = p;
                                ds[b][r] = val ? p * (DP[b][r] - circatt_lds[oS1 + e]) : 0.f;
                                if (DIST) corr += ds[b][r];
                            }
                        }
                        if (++bj == nkw) {
                            bj = 0;
                            ++bi;
                        }
                    }
                    if constexpr (MODE == MODE_FWD) {
                        lm *= c2;
                        if (__any(lm > m + kRescaleLog2)) {
                            const float mn = fmaxf(m, xmax16_32(lm));
                            const float alpha = fast_exp2(m - mn);
                            m = mn;
                            lsum *= alpha;
#pragma unroll
                            for (int t = 0; t < NTO; ++t) acc[t] *= alpha;
                        }
#pragma unroll
                        for (int b = 0; b < MAXB; ++b)
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                pr[b][r] = fast_exp2(fmaf(pr[b][r], c2, -m));
                                lsum += pr[b][r];
                            }
                    }
                }

                // output products over this pass's components
                __syncthreads();  // the score chunks' LDS reads are done
                if constexpr (MODE == MODE_FWD) stage(r0, nrows, oc0, OC, T1, nullptr, -1);
                if constexpr (MODE == MODE_BWDQ) stage(r0, nrows, oc0, OC, T0, nullptr, -1);
                if constexpr (MODE == MODE_BWDKV) stage(r0, nrows, oc0, OC, T1, T0, -1);
                __syncthreads();
                {
                    int bi = ib, bj = 0;
#pragma unroll
                    for (int b = 0; b < MAXB; ++b) {
                        if (b < nb) {
                            const int bo = (KH * bi - r0) + CR * (KW * bj);
                            const int off = (laneE + bo) * PS + j;
                            if constexpr (MODE == MODE_FWD) block_accumulate<NTO>(acc, off, rdelPS, pr[b]);
                            if constexpr (MODE == MODE_BWDQ) block_accumulate<NTO>(acc, off, rdelPS, ds[b]);
                            if constexpr (MODE == MODE_BWDKV) {
                                block_accumulate<NTO>(acc, off, rdelPS, pr[b]);         // dv (dY)
                                block_accumulate<NTO>(acc2, oT1 + off, rdelPS, ds[b]);  // dk (Q)
                            }
                        }
                        if (++bj == nkw) {
                            bj = 0;
                            ++bi;
                        }
                    }
                }
            }

            // ---- pass epilogue: lane (j, g) holds component oc0 + 16t + 4g + r ----
            if constexpr (MODE == MODE_FWD) {
                const float l = xsum16_32(lsum);
                const float inv = 1.f / l;
                if (rvalid) {
                    float *yb = a.yout + uoff;
#pragma unroll
                    for (int t = 0; t < NTO; ++t)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int comp = oc0 + 16 * t + 4 * g + r;
                            if (comp < a.ncr) yb[comp_index(a, rpix, comp)] = acc[t][r] * inv;
                        }
                    if (oc == 0 && g == 0)
                        a.lse_out[soff + rpix] =
                            (m + log2f(l)) * kLn2 - (DIST ? 0.5f * sq * a.scale : 0.f);
                }
            } else {
                const float cs = DIST ? xsum16_32(corr) : 0.f;
                float xr[4 * NTO];
#pragma unroll
                for (int i = 0; i < 4 * NTO; ++i) xr[i] = 0.f;
                if (DIST) load_reg(NTo{}, xr, R0, rpix, oc0, MU, p0);
                if (rvalid) {
                    float *ob = MODE == MODE_BWDQ ? a.dq + uoff : a.dk + uoff;
#pragma unroll
                    for (int t = 0; t < NTO; ++t)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int comp = oc0 + 16 * t + 4 * g + r;
                            if (comp < a.ncr) {
                                const int64_t idx = comp_index(a, rpix, comp);
                                float val = MODE == MODE_BWDQ ? acc[t][r] : acc2[t][r];
                                if (DIST) val -= cs * xr[4 * t + r];
                                ob[idx] = val * a.scale;
                                if (MODE == MODE_BWDKV) a.dv[uoff + idx] = acc[t][r];
                            }
                        }
                }
            }
        }
    }
}

}  // namespace wide

// Launch of the channel-chunked kernels for a prepared argument block
// (fused_wide.hip; planned in fused.hip).
hipError_t launch_wide(FusedMode mode, int nsp, bool dist, const FArgs &a, size_t lds_bytes,
                       dim3 grid, hipStream_t s);

}  // namespace circatt
