// Split-half forward kernel for 2D circulant attention on gfx950.
//
// Same work decomposition and window geometry as the Float32 kernels of
// fused2d_impl.h (16x16 tiles, 16 wavefronts, 8x2 register blocks, 2x8 LDS
// blocks), but both products run on the f16 matrix cores
// (v_mfma_f32_16x16x16_f16, 8 cycles, against 32 cycles for
// v_mfma_f32_16x16x4f32 per 16x16 block and 4 channels): every Float32
// operand x is carried as two halves, x = hi + lo with hi = x truncated to
// 11 significant bits and lo = f16(x - hi), and a product a.b is taken as
// hi.hi + lo.hi + hi.lo with Float32 accumulation.  The dropped lo.lo term
// and the rounding of lo leave a relative error near 2^-21 per operand, the
// order of Float32 accumulation itself.  (On gfx950 Float32 MFMA and vector
// instructions do not overlap, so the 4x cheaper products leave the softmax
// vector work as the larger part of a block.)
//
// LDS per staged pixel: keys as [16 hi | 16 lo | pad] halves (the score
// product's rows), values in channel planes of row-pair-major order so that
// the four keys 4g .. 4g+3 of a block are four consecutive halves (the
// apply product's rows), both split once at staging.
//
// Operands stay in the Float32 range of f16: |x| < 65504 after the scale
// (queries are multiplied by scale * log2(e) before splitting).  The host
// falls back to the Float32 kernels when a caller asks for exact Float32
// products (circatt_set_math).
#pragma once
#include "fused2d_impl.h"

namespace circatt {
namespace f2h {

using f2d::Args;
using f2d::f4;
using f2d::gmax;
using f2d::gsum;
using f2d::kLn2;
using f2d::kLog2e;
using f2d::lane_mask;
using f2d::mask_sel;
using f2d::static_for;

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f4 mfmah(h4 a, h4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// hi = x with the low 13 mantissa bits cleared (exact in f16 inside its
// normal range), lo = x - hi (exact in Float32, rounded once to f16)
__device__ __forceinline__ void split2(float x0, float x1, h2 &hi, h2 &lo) {
    const float t0 = __uint_as_float(__float_as_uint(x0) & 0xffffe000u);
    const float t1 = __uint_as_float(__float_as_uint(x1) & 0xffffe000u);
    hi = h2{(_Float16)t0, (_Float16)t1};
    lo = h2{(_Float16)(x0 - t0), (_Float16)(x1 - t1)};
}

template <int P>
struct HGeo {
    using G = f2d::Geo<P, 1, 2, 8>;
    static constexpr int KS = 40;                    // halves per key slot (16 hi, 16 lo, 8 pad)
    static constexpr int VPS = G::HH * G::HWD;       // halves per value channel plane
    static constexpr int OK = 0;                     // byte offsets of the regions
    static constexpr int OVH = G::LPX * KS * 2;
    static constexpr int OVL = OVH + 16 * VPS * 2;
    static constexpr int OB = OVL + 16 * VPS * 2;    // Distance key bias (Float32 per slot)
    template <bool DIST>
    static constexpr int bytes() { return OB + (DIST ? G::LPX * 4 : 0); }
};

template <int P, bool CPLX, bool DIST>
__global__ __launch_bounds__(1024, 1) void kernel2h_fwd(Args a) {
    using G = f2d::Geo<P, 1, 2, 8>;
    using H = HGeo<P>;
    constexpr int WH = 2, THREADS = 1024;
    constexpr int CR = G::CR, HH = G::HH, HWD = G::HWD, NKW = G::NKW, NBLK = G::NBLK;
    constexpr int NPX = G::NPX, KS = H::KS, VPS = H::VPS;
    constexpr int NCH = NBLK > 12 ? 2 : 1;
    constexpr int CHB = (NBLK + NCH - 1) / NCH;
    constexpr int PFB = (NCH - 1) * CHB;
    static_assert(NPX <= THREADS, "one staged pixel per thread");
    static_assert(HH % 2 == 0, "row pairs");
    char *const lds = reinterpret_cast<char *>(circatt_lds2);

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int wh = wv % WH, ww = wv / WH;
    const int j = lane & 15, g = lane >> 4;
    const int jh = j & 7, jw = j >> 3;

    auto opaque = [](int v) {
        asm volatile("" : "+v"(v));
        return v;
    };
    // key rows: element j of block (bi, bj) at slot 8 wh + 2 bi + (j & 1) + CR (2 ww + 8 bj + j / 2)
    const int slotA = 8 * wh + (j & 1) + CR * (2 * ww + (j >> 1));
    const char *const pK = lds + opaque(H::OK + (slotA * KS + 4 * g) * 2);
    // value rows: channel j, keys 4g .. 4g+3 of block (bi, bj): plane j,
    // row pair 4 wh + bi, column 2 ww + 8 bj + 2 g, two halves per column
    const int vbase = j * VPS + (4 * wh) * 2 * HWD + 2 * (2 * ww + 2 * g);
    const char *const pVh = lds + opaque(H::OVH + vbase * 2);
    const char *const pVl = lds + opaque(H::OVL + vbase * 2);
    // Distance key bias of elements 4g .. 4g+3
    const int slotE = 8 * wh + CR * (2 * ww + 2 * g);
    const float *const pB = reinterpret_cast<const float *>(lds + opaque(H::OB + slotE * 4));

    const int ubytes = a.unit_stride * 4;

    // ---- prefetch registers ----
    float hk[16], hvv[16];
    int hslot;
    float nq[4];

    auto decode = [&](int item, int &unit, int &h0, int &w0) {
        const int ntiles = a.tiles_h * a.tiles_w;
        unit = item / ntiles;
        const int tile = item - unit * ntiles;
        const int th = tile % a.tiles_h;
        h0 = th * G::TH;
        w0 = (tile - th) / a.tiles_h * G::TW;
    };
    const bool big = a.n1 >= HH && a.n2 >= HWD;
    const int px = threadIdx.x;
    const int kw = px / HH, kh = px - kw * HH;
    auto load_stage = [&](int item) {
        int unit, h0, w0;
        decode(item, unit, h0, w0);
        const int hs0 = pmod(h0 - P, a.n1), ws0 = pmod(w0 - P, a.n2);
        const int64_t uoff = (int64_t)unit * a.unit_stride;
        const auto r0 = f2d::rsrc(a.k + uoff, ubytes);
        const auto r1 = f2d::rsrc(a.v + uoff, ubytes);
        hslot = px < NPX ? kh + CR * kw : -1;
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
            for (int c = 0; c < 8; ++c) {
                const f2d::f2 x0 = f2d::bload2(r0, gp * 8, c * a.P * 8);
                const f2d::f2 x1 = f2d::bload2(r1, gp * 8, c * a.P * 8);
                hk[2 * c] = x0[0];
                hk[2 * c + 1] = x0[1];
                hvv[2 * c] = x1[0];
                hvv[2 * c + 1] = x1[1];
            }
        } else {
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                hk[c] = f2d::bload(r0, gp * 4, c * a.P * 4);
                hvv[c] = f2d::bload(r1, gp * 4, c * a.P * 4);
            }
        }
    };
    auto load_regs = [&](int item) {
        int unit, h0, w0;
        decode(item, unit, h0, w0);
        const int rh = h0 + 8 * wh + jh, rw = w0 + 2 * ww + jw;
        const bool rvalid = rh < a.n1 && rw < a.n2;
        const int rpix = rvalid ? rh + a.n1 * rw : 0;
        const int64_t uoff = (int64_t)unit * a.unit_stride;
        const auto r0 = f2d::rsrc(a.q + uoff, ubytes);
        const int vo = f2d::comp_off<CPLX>(a.P, rpix, 4 * g) * 4;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int so = (CPLX ? 2 * a.P * (s >> 1) + (s & 1) : a.P * s) * 4;
            nq[s] = f2d::bload(r0, vo, so);
        }
    };

    int k = 0;
    int item = f2d::item_of(a, 0);
    if (item >= a.nitems) return;
    load_stage(item);
    load_regs(item);

    while (true) {
        int unit, h0, w0;
        decode(item, unit, h0, w0);
        const int rh = h0 + 8 * wh + jh, rw = w0 + 2 * ww + jw;
        const bool rvalid = rh < a.n1 && rw < a.n2;
        const int rpix = rvalid ? rh + a.n1 * rw : 0;
        const int64_t uoff = (int64_t)unit * a.unit_stride;
        const int64_t soff = (int64_t)unit * a.P;
        const float c2 = a.c2;

        __syncthreads();  // the previous item's LDS reads are done
        if (hslot >= 0) {
            // keys: [16 hi | 16 lo] halves at the slot
            h2 kh2[8], kl2[8];
            float n2 = 0.f;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                split2(hk[2 * c], hk[2 * c + 1], kh2[c], kl2[c]);
                if constexpr (DIST) n2 += hk[2 * c] * hk[2 * c] + hk[2 * c + 1] * hk[2 * c + 1];
            }
            char *kp = lds + H::OK + hslot * KS * 2;
#pragma unroll
            for (int c = 0; c < 8; c += 4) {
                *reinterpret_cast<f4 *>(kp + 4 * c) =
                    f4{__builtin_bit_cast(float, kh2[c]), __builtin_bit_cast(float, kh2[c + 1]),
                       __builtin_bit_cast(float, kh2[c + 2]), __builtin_bit_cast(float, kh2[c + 3])};
                *reinterpret_cast<f4 *>(kp + 32 + 4 * c) =
                    f4{__builtin_bit_cast(float, kl2[c]), __builtin_bit_cast(float, kl2[c + 1]),
                       __builtin_bit_cast(float, kl2[c + 2]), __builtin_bit_cast(float, kl2[c + 3])};
            }
            if constexpr (DIST)
                reinterpret_cast<float *>(lds + H::OB)[hslot] = -0.5f * c2 * n2;
            // values: channel planes, (row pair, column, row & 1) order
            const int vo = (kh >> 1) * 2 * HWD + 2 * kw + (kh & 1);
            _Float16 *vh = reinterpret_cast<_Float16 *>(lds + H::OVH) + vo;
            _Float16 *vl = reinterpret_cast<_Float16 *>(lds + H::OVL) + vo;
#pragma unroll
            for (int c = 0; c < 16; c += 2) {
                h2 hi, lo;
                split2(hvv[c], hvv[c + 1], hi, lo);
                vh[c * VPS] = hi[0];
                vh[(c + 1) * VPS] = hi[1];
                vl[c * VPS] = lo[0];
                vl[(c + 1) * VPS] = lo[1];
            }
        }
        // queries, pre-scaled by c2 and split
        h4 qh, ql;
        float raw2 = 0.f;
        {
            h2 a0, a1, b0, b1;
            split2(nq[0] * c2, nq[1] * c2, a0, b0);
            split2(nq[2] * c2, nq[3] * c2, a1, b1);
            qh = h4{a0[0], a0[1], a1[0], a1[1]};
            ql = h4{b0[0], b0[1], b1[0], b1[1]};
            if constexpr (DIST)
                raw2 = nq[0] * nq[0] + nq[1] * nq[1] + nq[2] * nq[2] + nq[3] * nq[3];
        }
        const float sq = DIST ? gsum(raw2) : 0.f;
        __syncthreads();  // halo staged

        const int nitem = f2d::item_of(a, k + 1);
        const bool has_next = nitem < a.nitems;
        auto prefetch = [&]() {
            if (has_next) {
                load_stage(nitem);
                load_regs(nitem);
            }
        };

        float m = -1e30f, lsum = 0.f;
        f4 acc[2] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
        auto chunk = [&](auto CH) {
            constexpr int ci = decltype(CH)::value;
            constexpr int cb = ci * CHB;
            constexpr int ce = cb + CHB < NBLK ? cb + CHB : NBLK;
            if constexpr (cb == PFB) prefetch();
            f4 S[CHB];
            static_for<cb, ce>([&](auto B) {
                constexpr int b = decltype(B)::value;
                constexpr int bi = b / NKW, bj = b % NKW;
                constexpr int koff = (2 * bi + CR * 8 * bj) * KS * 2;  // bytes
                BLOCK_FENCE();
                const h4 ah = *reinterpret_cast<const h4 *>(pK + koff);
                const h4 al = *reinterpret_cast<const h4 *>(pK + koff + 32);
                f4 s0 = f4{0.f, 0.f, 0.f, 0.f};
                if constexpr (DIST) {
                    constexpr int boff = 2 * bi + CR * 8 * bj;
                    const f2 lo = *reinterpret_cast<const f2 *>(pB + boff);
                    const f2 hi = *reinterpret_cast<const f2 *>(pB + boff + CR);
                    s0 = f4{lo[0], lo[1], hi[0], hi[1]};
                }
                s0 = mfmah(ah, qh, s0);
                s0 = mfmah(al, qh, s0);
                s0 = mfmah(ah, ql, s0);
                S[b - cb] = s0;
            });
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
                acc[0] *= alpha;
                acc[1] *= alpha;
            }
            m = mn;
            static_for<cb, ce>([&](auto B) {
                constexpr int b = decltype(B)::value;
                constexpr int bi = b / NKW, bj = b % NKW;
                // value rows of block (bi, bj): row pair bi, column offset 8 bj
                constexpr int voff = (bi * 2 * HWD + 2 * 8 * bj) * 2;  // bytes
                BLOCK_FENCE();
                float p[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    p[r] = __builtin_amdgcn_exp2f(S[b - cb][r] - m);
                    lsum += p[r];
                }
                h2 p01h, p01l, p23h, p23l;
                split2(p[0], p[1], p01h, p01l);
                split2(p[2], p[3], p23h, p23l);
                const h4 ph = h4{p01h[0], p01h[1], p23h[0], p23h[1]};
                const h4 pl = h4{p01l[0], p01l[1], p23l[0], p23l[1]};
                const h4 vh = *reinterpret_cast<const h4 *>(pVh + voff);
                const h4 vl = *reinterpret_cast<const h4 *>(pVl + voff);
                f4 &ac = acc[b & 1];
                ac = mfmah(vh, ph, ac);
                ac = mfmah(vh, pl, ac);
                ac = mfmah(vl, ph, ac);
            });
        };
        static_for<0, NCH>(chunk);
        const float l = gsum(lsum);
        const float inv = 1.f / l;
        if (rvalid) {
            float *yb = a.yout + uoff;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                yb[f2d::comp_off<CPLX>(a.P, rpix, 4 * g + r)] = (acc[0][r] + acc[1][r]) * inv;
            if (g == 0)
                a.lse_out[soff + rpix] = (m + __log2f(l)) * kLn2 - (DIST ? 0.5f * sq * a.scale : 0.f);
        }

        if (!has_next) break;
        ++k;
        item = nitem;
    }
}

template <int P, bool CPLX, bool DIST>
hipError_t launch_fwd(const Args &a0, int cus, hipStream_t s) {
    using G = f2d::Geo<P, 1, 2, 8>;
    constexpr int bytes = HGeo<P>::template bytes<DIST>();
    static_assert(bytes <= (int)f2d::kLdsCap, "halo does not fit LDS");
    auto kern = kernel2h_fwd<P, CPLX, DIST>;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    Args a = a0;
    a.tiles_h = (a.n1 + G::TH - 1) / G::TH;
    a.tiles_w = (a.n2 + G::TW - 1) / G::TW;
    const int64_t nitems = (int64_t)a.tiles_h * a.tiles_w * a.nunits;
    if (nitems <= 0 || nitems > INT32_MAX / 2) return hipErrorNotSupported;
    a.nitems = (int)nitems;
    a.per_xcd = (int)((nitems + 7) / 8);
    int64_t grid = std::min<int64_t>(cus, 8LL * a.per_xcd);
    grid = std::max<int64_t>(8, grid / 8 * 8);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(1024), bytes, s, a);
    return hipGetLastError();
}

inline hipError_t dispatch_fwd(int p, bool cplx, bool dist, const Args &a, int cus, hipStream_t s) {
#define CIRCATT_F2H_CASE(PP)                                                             \
    if (p == PP) {                                                                       \
        if (cplx) return dist ? launch_fwd<PP, true, true>(a, cus, s)                    \
                              : launch_fwd<PP, true, false>(a, cus, s);                  \
        return dist ? launch_fwd<PP, false, true>(a, cus, s)                             \
                    : launch_fwd<PP, false, false>(a, cus, s);                           \
    }
    CIRCATT_F2H_CASE(1)
    CIRCATT_F2H_CASE(2)
    CIRCATT_F2H_CASE(3)
    CIRCATT_F2H_CASE(5)
    CIRCATT_F2H_CASE(7)
#undef CIRCATT_F2H_CASE
    return hipErrorNotSupported;
}


// ---------------------------------------------------------------------------
// Split-half backward passes.
//   BWDQ  (query-centric): registers hold queries (c2-scaled), dY, Y; LDS
//         holds keys and values as [16 hi | 16 lo] slots.  Products:
//         S = K.Q, dP = V.dY (rows from the slots), dQ = K^T.dS (rows from
//         the key slots read transposed, one half per key).
//   BWDKV (key-centric): registers hold keys (c2-scaled) and values; LDS
//         holds queries and dY as slots plus the per-query terms
//         -lse log2(e) [- c2 |q|^2 / 2] and -D.  Products: S^T = Q.K,
//         dP^T = dY.V, dV = dY^T.P^T, dK = Q^T.dS^T.
// ---------------------------------------------------------------------------
template <int P, int MODE, bool DIST>
struct BGeo {
    using G = f2d::Geo<P, 1, 2, 8>;
    static constexpr int KS = 40;
    static constexpr int OT0 = 0;                         // tensor 0 slots (K or Q)
    static constexpr int OT1 = G::LPX * KS * 2;           // tensor 1 slots (V or dY)
    static constexpr int OS0 = 2 * G::LPX * KS * 2;       // scalars (Float32 per slot)
    static constexpr int OS1 = OS0 + G::LPX * 4;
    static constexpr int NSCAL = MODE == f2d::BWDKV ? 2 : (DIST ? 1 : 0);
    static constexpr int bytes = OS0 + NSCAL * G::LPX * 4;
};

template <int P, bool CPLX, bool DIST, int MODE>
__global__ __launch_bounds__(1024, 1) void kernel2h_bwd(Args a) {
    using G = f2d::Geo<P, 1, 2, 8>;
    using H = BGeo<P, MODE, DIST>;
    constexpr int WH = 2;
    constexpr int CR = G::CR, HH = G::HH, HWD = G::HWD, NKW = G::NKW, NBLK = G::NBLK;
    constexpr int NPX = G::NPX, KS = H::KS;
    constexpr int PFB = NBLK / 2;
    constexpr bool KV = MODE == f2d::BWDKV;
    static_assert(NPX <= 1024, "one staged pixel per thread");
    char *const lds = reinterpret_cast<char *>(circatt_lds2);

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int wh = wv % WH, ww = wv / WH;
    const int j = lane & 15, g = lane >> 4;
    const int jh = j & 7, jw = j >> 3;

    auto opaque = [](int v) {
        asm volatile("" : "+v"(v));
        return v;
    };
    // product-1 rows: element j of a block, channels 4g .. 4g+3
    const int slotA = 8 * wh + (j & 1) + CR * (2 * ww + (j >> 1));
    const char *const pA0 = lds + opaque(H::OT0 + (slotA * KS + 4 * g) * 2);
    const char *const pA1 = lds + opaque(H::OT1 + (slotA * KS + 4 * g) * 2);
    // product-2 rows (transposed): channel j of elements 4g .. 4g+3
    const int slotE = 8 * wh + CR * (2 * ww + 2 * g);
    const _Float16 *const pT0 = reinterpret_cast<const _Float16 *>(lds + opaque(H::OT0 + (slotE * KS + j) * 2));
    const _Float16 *const pT1 = reinterpret_cast<const _Float16 *>(lds + opaque(H::OT1 + (slotE * KS + j) * 2));
    // per-slot scalars of elements 4g .. 4g+3
    const float *const pS0 = reinterpret_cast<const float *>(lds + opaque(H::OS0 + slotE * 4));
    const float *const pS1 = reinterpret_cast<const float *>(lds + opaque(H::OS1 + slotE * 4));

    const int ubytes = a.unit_stride * 4;

    // ---- prefetch registers ----
    float h0v[16], h1v[16], hs0 = 0.f, hs1 = 0.f;
    int hslot;
    float nr0[4], nr1[4], nry[4];
    float nlse = 0.f;

    auto decode = [&](int item, int &unit, int &h0, int &w0) {
        const int ntiles = a.tiles_h * a.tiles_w;
        unit = item / ntiles;
        const int tile = item - unit * ntiles;
        const int th = tile % a.tiles_h;
        h0 = th * G::TH;
        w0 = (tile - th) / a.tiles_h * G::TW;
    };
    const bool big = a.n1 >= HH && a.n2 >= HWD;
    const int px = threadIdx.x;
    const int kw = px / HH, kh = px - kw * HH;
    auto load_stage = [&](int item) {
        int unit, h0, w0;
        decode(item, unit, h0, w0);
        const int hsh = pmod(h0 - P, a.n1), wsh = pmod(w0 - P, a.n2);
        const int64_t uoff = (int64_t)unit * a.unit_stride;
        const auto r0 = f2d::rsrc((KV ? a.q : a.k) + uoff, ubytes);
        const auto r1 = f2d::rsrc((KV ? a.dy : a.v) + uoff, ubytes);
        hslot = px < NPX ? kh + CR * kw : -1;
        int gh = hsh + kh, gw = wsh + kw;
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
            for (int c = 0; c < 8; ++c) {
                const f2d::f2 x0 = f2d::bload2(r0, gp * 8, c * a.P * 8);
                const f2d::f2 x1 = f2d::bload2(r1, gp * 8, c * a.P * 8);
                h0v[2 * c] = x0[0];
                h0v[2 * c + 1] = x0[1];
                h1v[2 * c] = x1[0];
                h1v[2 * c + 1] = x1[1];
            }
        } else {
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                h0v[c] = f2d::bload(r0, gp * 4, c * a.P * 4);
                h1v[c] = f2d::bload(r1, gp * 4, c * a.P * 4);
            }
        }
        if constexpr (KV) {
            const int64_t soff = (int64_t)unit * a.P;
            hs0 = f2d::bload(f2d::rsrc(a.lse + soff, a.P * 4), gp * 4, 0);
            hs1 = f2d::bload(f2d::rsrc(a.dbuf + soff, a.P * 4), gp * 4, 0);
        }
    };
    auto load_regs = [&](int item) {
        int unit, h0, w0;
        decode(item, unit, h0, w0);
        const int rh = h0 + 8 * wh + jh, rw = w0 + 2 * ww + jw;
        const bool rvalid = rh < a.n1 && rw < a.n2;
        const int rpix = rvalid ? rh + a.n1 * rw : 0;
        const int64_t uoff = (int64_t)unit * a.unit_stride;
        const auto r0 = f2d::rsrc((KV ? a.k : a.q) + uoff, ubytes);
        const auto r1 = f2d::rsrc((KV ? a.v : a.dy) + uoff, ubytes);
        const int vo = f2d::comp_off<CPLX>(a.P, rpix, 4 * g) * 4;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int so = (CPLX ? 2 * a.P * (s >> 1) + (s & 1) : a.P * s) * 4;
            nr0[s] = f2d::bload(r0, vo, so);
            nr1[s] = f2d::bload(r1, vo, so);
            if constexpr (!KV) nry[s] = f2d::bload(f2d::rsrc(a.y + uoff, ubytes), vo, so);
        }
        if constexpr (!KV)
            nlse = f2d::bload(f2d::rsrc(a.lse + (int64_t)unit * a.P, a.P * 4), rpix * 4, 0);
    };

    // slot store of 16 Float32 values as [16 hi | 16 lo] halves
    auto store_slot = [&](char *sp, const float (&x)[16]) {
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
    };

    int k = 0;
    int item = f2d::item_of(a, 0);
    if (item >= a.nitems) return;
    load_stage(item);
    load_regs(item);

    while (true) {
        int unit, h0, w0;
        decode(item, unit, h0, w0);
        const int rh = h0 + 8 * wh + jh, rw = w0 + 2 * ww + jw;
        const bool rvalid = rh < a.n1 && rw < a.n2;
        const int rpix = rvalid ? rh + a.n1 * rw : 0;
        const int64_t uoff = (int64_t)unit * a.unit_stride;
        const int64_t soff = (int64_t)unit * a.P;
        const float c2 = a.c2;

        __syncthreads();  // the previous item's LDS reads are done
        if (hslot >= 0) {
            float n2 = 0.f;
            if constexpr (DIST) {
#pragma unroll
                for (int c = 0; c < 16; ++c) n2 += h0v[c] * h0v[c];
            }
            store_slot(lds + H::OT0 + hslot * KS * 2, h0v);
            store_slot(lds + H::OT1 + hslot * KS * 2, h1v);
            if constexpr (KV) {
                reinterpret_cast<float *>(lds + H::OS0)[hslot] =
                    -hs0 * kLog2e - (DIST ? 0.5f * c2 * n2 : 0.f);
                reinterpret_cast<float *>(lds + H::OS1)[hslot] = -hs1;
            } else if constexpr (DIST) {
                reinterpret_cast<float *>(lds + H::OS0)[hslot] = -0.5f * c2 * n2;
            }
        }
        // register operands: the score product's side pre-scaled by c2
        h4 r0h, r0l, r1h, r1l;
        float raw2 = 0.f, rowD = 0.f, rowL = 0.f;
        {
            h2 a0, a1, b0, b1;
            split2(nr0[0] * c2, nr0[1] * c2, a0, b0);
            split2(nr0[2] * c2, nr0[3] * c2, a1, b1);
            r0h = h4{a0[0], a0[1], a1[0], a1[1]};
            r0l = h4{b0[0], b0[1], b1[0], b1[1]};
            split2(nr1[0], nr1[1], a0, b0);
            split2(nr1[2], nr1[3], a1, b1);
            r1h = h4{a0[0], a0[1], a1[0], a1[1]};
            r1l = h4{b0[0], b0[1], b1[0], b1[1]};
            if constexpr (DIST)
                raw2 = nr0[0] * nr0[0] + nr0[1] * nr0[1] + nr0[2] * nr0[2] + nr0[3] * nr0[3];
            if constexpr (!KV) {
                rowD = gsum(nr1[0] * nry[0] + nr1[1] * nry[1] + nr1[2] * nry[2] + nr1[3] * nry[3]);
                rowL = nlse;
            }
        }
        float reg0[4];  // unscaled register pixel (Distance correction)
#pragma unroll
        for (int s = 0; s < 4; ++s) reg0[s] = nr0[s];
        const float sq = DIST ? gsum(raw2) : 0.f;
        __syncthreads();  // halo staged

        const int nitem = f2d::item_of(a, k + 1);
        const bool has_next = nitem < a.nitems;
        auto prefetch = [&]() {
            if (has_next) {
                load_stage(nitem);
                load_regs(nitem);
            }
        };

        // row terms of the BWDQ score and dP products (initial accumulators)
        const float nl = -rowL * kLog2e - (DIST ? 0.5f * c2 * sq : 0.f);
        const float kb = DIST ? -0.5f * c2 * sq : 0.f;  // BWDKV key bias
        f4 acc0[2] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
        f4 acc1[2] = {f4{0.f, 0.f, 0.f, 0.f}, f4{0.f, 0.f, 0.f, 0.f}};
        float corr = 0.f;
        static_for<0, NBLK>([&](auto B) {
            constexpr int b = decltype(B)::value;
            constexpr int bi = b / NKW, bj = b % NKW;
            constexpr int boff = 2 * bi + CR * 8 * bj;  // block slot offset
            constexpr int aoff = boff * KS * 2;         // bytes
            BLOCK_FENCE();
            if constexpr (b == PFB) prefetch();
            const h4 x0h = *reinterpret_cast<const h4 *>(pA0 + aoff);
            const h4 x0l = *reinterpret_cast<const h4 *>(pA0 + aoff + 32);
            const h4 x1h = *reinterpret_cast<const h4 *>(pA1 + aoff);
            const h4 x1l = *reinterpret_cast<const h4 *>(pA1 + aoff + 32);
            f4 s, dp;
            if constexpr (KV) {
                const f2 alo = *reinterpret_cast<const f2 *>(pS0 + boff);
                const f2 ahi = *reinterpret_cast<const f2 *>(pS0 + boff + CR);
                const f2 dlo = *reinterpret_cast<const f2 *>(pS1 + boff);
                const f2 dhi = *reinterpret_cast<const f2 *>(pS1 + boff + CR);
                s = f4{alo[0], alo[1], ahi[0], ahi[1]};
                if constexpr (DIST) s = s + f4{kb, kb, kb, kb};
                dp = f4{dlo[0], dlo[1], dhi[0], dhi[1]};
            } else {
                s = f4{nl, nl, nl, nl};
                if constexpr (DIST) {
                    const f2 lo = *reinterpret_cast<const f2 *>(pS0 + boff);
                    const f2 hi = *reinterpret_cast<const f2 *>(pS0 + boff + CR);
                    s = s + f4{lo[0], lo[1], hi[0], hi[1]};
                }
                dp = f4{-rowD, -rowD, -rowD, -rowD};
            }
            s = mfmah(x0h, r0h, s);
            dp = mfmah(x1h, r1h, dp);
            s = mfmah(x0l, r0h, s);
            dp = mfmah(x1l, r1h, dp);
            s = mfmah(x0h, r0l, s);
            dp = mfmah(x1h, r1l, dp);
            float p[4], ds[4];
            p[0] = mask_sel<lane_mask(P, bi, bj, 0)>(__builtin_amdgcn_exp2f(s[0]), 0.f);
            p[1] = mask_sel<lane_mask(P, bi, bj, 1)>(__builtin_amdgcn_exp2f(s[1]), 0.f);
            p[2] = mask_sel<lane_mask(P, bi, bj, 2)>(__builtin_amdgcn_exp2f(s[2]), 0.f);
            p[3] = mask_sel<lane_mask(P, bi, bj, 3)>(__builtin_amdgcn_exp2f(s[3]), 0.f);
#pragma unroll
            for (int r = 0; r < 4; ++r) ds[r] = p[r] * dp[r];
            if constexpr (DIST) corr += (ds[0] + ds[1]) + (ds[2] + ds[3]);
            h2 d01h, d01l, d23h, d23l;
            split2(ds[0], ds[1], d01h, d01l);
            split2(ds[2], ds[3], d23h, d23l);
            const h4 dsh = h4{d01h[0], d01h[1], d23h[0], d23h[1]};
            const h4 dsl = h4{d01l[0], d01l[1], d23l[0], d23l[1]};
            // transposed rows of tensor 0: channel j of elements 4g + r at
            // slots boff + (r & 1) + CR (r >> 1)
            constexpr int t0 = boff * KS, t1 = (boff + 1) * KS, t2 = (boff + CR) * KS,
                          t3 = (boff + CR + 1) * KS;
            const h4 y0h = h4{pT0[t0], pT0[t1], pT0[t2], pT0[t3]};
            const h4 y0l = h4{pT0[t0 + 16], pT0[t1 + 16], pT0[t2 + 16], pT0[t3 + 16]};
            f4 &a0 = acc0[b & 1];
            a0 = mfmah(y0h, dsh, a0);
            a0 = mfmah(y0l, dsh, a0);
            a0 = mfmah(y0h, dsl, a0);
            if constexpr (KV) {
                h2 p01h, p01l, p23h, p23l;
                split2(p[0], p[1], p01h, p01l);
                split2(p[2], p[3], p23h, p23l);
                const h4 ph = h4{p01h[0], p01h[1], p23h[0], p23h[1]};
                const h4 pl = h4{p01l[0], p01l[1], p23l[0], p23l[1]};
                const h4 y1h = h4{pT1[t0], pT1[t1], pT1[t2], pT1[t3]};
                const h4 y1l = h4{pT1[t0 + 16], pT1[t1 + 16], pT1[t2 + 16], pT1[t3 + 16]};
                f4 &a1 = acc1[b & 1];
                a1 = mfmah(y1h, ph, a1);
                a1 = mfmah(y1l, ph, a1);
                a1 = mfmah(y1h, pl, a1);
            }
        });
        const float cs = DIST ? gsum(corr) : 0.f;
        if (rvalid) {
            if constexpr (!KV) {
                float *ob = a.dq + uoff;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float val = acc0[0][r] + acc0[1][r];
                    if constexpr (DIST) val -= cs * reg0[r];
                    ob[f2d::comp_off<CPLX>(a.P, rpix, 4 * g + r)] = val * a.scale;
                }
                if (g == 0) a.dbuf[soff + rpix] = rowD;
            } else {
                float *vb = a.dv + uoff;
                float *kbp = a.dk + uoff;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int o = f2d::comp_off<CPLX>(a.P, rpix, 4 * g + r);
                    vb[o] = acc1[0][r] + acc1[1][r];
                    float val = acc0[0][r] + acc0[1][r];
                    if constexpr (DIST) val -= cs * reg0[r];
                    kbp[o] = val * a.scale;
                }
            }
        }

        if (!has_next) break;
        ++k;
        item = nitem;
    }
}

template <int P, bool CPLX, bool DIST, int MODE>
hipError_t launch_bwd(const Args &a0, int cus, hipStream_t s) {
    using G = f2d::Geo<P, 1, 2, 8>;
    constexpr int bytes = BGeo<P, MODE, DIST>::bytes;
    static_assert(bytes <= (int)f2d::kLdsCap, "halo does not fit LDS");
    auto kern = kernel2h_bwd<P, CPLX, DIST, MODE>;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    Args a = a0;
    a.tiles_h = (a.n1 + G::TH - 1) / G::TH;
    a.tiles_w = (a.n2 + G::TW - 1) / G::TW;
    const int64_t nitems = (int64_t)a.tiles_h * a.tiles_w * a.nunits;
    if (nitems <= 0 || nitems > INT32_MAX / 2) return hipErrorNotSupported;
    a.nitems = (int)nitems;
    a.per_xcd = (int)((nitems + 7) / 8);
    int64_t grid = std::min<int64_t>(cus, 8LL * a.per_xcd);
    grid = std::max<int64_t>(8, grid / 8 * 8);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(1024), bytes, s, a);
    return hipGetLastError();
}

template <int MODE>
hipError_t dispatch_bwd(int p, bool cplx, bool dist, const Args &a, int cus, hipStream_t s) {
#define CIRCATT_F2H_CASE(PP)                                                             \
    if (p == PP) {                                                                       \
        if (cplx) return dist ? launch_bwd<PP, true, true, MODE>(a, cus, s)              \
                              : launch_bwd<PP, true, false, MODE>(a, cus, s);            \
        return dist ? launch_bwd<PP, false, true, MODE>(a, cus, s)                       \
                    : launch_bwd<PP, false, false, MODE>(a, cus, s);                     \
    }
    CIRCATT_F2H_CASE(1)
    CIRCATT_F2H_CASE(2)
    CIRCATT_F2H_CASE(3)
    CIRCATT_F2H_CASE(5)
    CIRCATT_F2H_CASE(7)
#undef CIRCATT_F2H_CASE
    return hipErrorNotSupported;
}

}  // namespace f2h

hipError_t launch_f2h_fwd(int p, bool cplx, bool dist, const f2d::Args &a, int cus, hipStream_t s);
hipError_t launch_f2h_bwdq(int p, bool cplx, bool dist, const f2d::Args &a, int cus, hipStream_t s);
hipError_t launch_f2h_bwdkv(int p, bool cplx, bool dist, const f2d::Args &a, int cus, hipStream_t s);

}  // namespace circatt
