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
//   * the forward keeps all scores of its 16 queries in registers (22 blocks
//     x 4 values at ws = 15), takes the exact row maximum, and never rescales.
//
// Work decomposition (as in fused_impl.h): persistent workgroups of four
// wavefronts walk XCD-contiguous runs of (8x8 tile, unit) items; the
// circularly wrapped halo of the other side is staged in LDS with the next
// item's global loads issued into registers before the current item is
// computed.  Wavefront w holds the 8 (dim 1) x 2 (dim 2) register pixels at
// tile columns 2w, 2w+1 (lane j -> (j % 8, j / 8)) and walks the 2 x 8 LDS
// blocks covering their windows (element e -> (e % 2, e / 2)).
#pragma once
#include <stdint.h>

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

__device__ __forceinline__ f4 mfma(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// compile-time loop: f(std::integral_constant<int, I>) for I in [0, N)
template <int I, int N>
struct SFor {
    template <typename F>
    __device__ __forceinline__ static void run(F &f) {
        f(std::integral_constant<int, I>{});
        SFor<I + 1, N>::run(f);
    }
};
template <int N>
struct SFor<N, N> {
    template <typename F>
    __device__ __forceinline__ static void run(F &) {}
};
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    SFor<0, N>::run(f);
}

// Geometry of one (P, NT) instantiation.
template <int P_, int NT_>
struct Geo {
    static constexpr int P = P_;
    static constexpr int NT = NT_;          // 16-component tiles per pixel
    static constexpr int NC = 16 * NT;      // real components per pixel
    static constexpr int NS = 4 * NT;       // MFMA k-steps per product
    static constexpr int PS = NC + 4;       // LDS floats per staged pixel
    static constexpr int TH = 8, TW = 8;    // register tile of a workgroup
    static constexpr int NKH = 4 + P;       // 2-row LDS blocks along dim 1
    static constexpr int NKW = (2 + 2 * P + 7) / 8;  // 8-column LDS blocks along dim 2
    static constexpr int NBLK = NKH * NKW;
    static constexpr int HH = 2 * NKH;      // staged rows (= TH + 2P)
    static constexpr int HWD = 6 + 8 * NKW; // staged columns (>= TW + 2P)
    static constexpr int CR = HH + ((2 - HH % 4) + 4) % 4;  // LDS column stride, 2 mod 4
    static constexpr int NPX = HH * HWD;    // staged pixels
    static constexpr int LPX = CR * HWD;    // LDS pixel slots per tensor
    static constexpr int PPT = (NPX + 255) / 256;  // staged pixels per thread
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
    int64_t P;            // pixels per image
    int64_t unit_stride;  // floats per (head, batch) unit = P * NC
    float scale, c2;      // similarity scale, scale * log2(e)
    int tiles_h, tiles_w, nitems, per_xcd;
};

// Real component `comp` of pixel `pix` in a unit of NC components.
template <bool CPLX>
__device__ __forceinline__ int64_t comp_off(int64_t P, int64_t pix, int comp) {
    if constexpr (CPLX) return 2 * (pix + P * (comp >> 1)) + (comp & 1);
    return pix + P * comp;
}

// Work item k of this workgroup: XCD x = blockIdx % 8 owns items
// [x * per_xcd, (x + 1) * per_xcd), walked by its workgroups in turn.
__device__ __forceinline__ int item_of(const Args &a, int k) {
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, nslot = gridDim.x >> 3;
    const int it = xcd * a.per_xcd + slot + k * nslot;
    return it < min(a.nitems, (xcd + 1) * a.per_xcd) ? it : a.nitems;
}

enum { FWD = 0, BWDQ = 1, BWDKV = 2 };

template <int MODE, bool DIST>
struct ModeCfg {
    static constexpr int NTEN = 2;                                       // staged tensors
    static constexpr int NSCAL = MODE == BWDKV ? 2 : (DIST ? 1 : 0);     // staged scalars
};

template <int P, int NT, bool CPLX, bool DIST, int MODE>
struct LdsSize {
    using G = Geo<P, NT>;
    using M = ModeCfg<MODE, DIST>;
    static constexpr int floats = M::NTEN * G::LPX * G::PS + M::NSCAL * G::LPX;
    static constexpr size_t bytes = (size_t)floats * 4;
};

template <int P, int NT, bool CPLX, bool DIST, int MODE>
__global__ __launch_bounds__(256, (LdsSize<P, NT, CPLX, DIST, MODE>::bytes <= 80 * 1024) ? 2 : 1)
void kernel2d(Args a) {
    using G = Geo<P, NT>;
    using M = ModeCfg<MODE, DIST>;
    constexpr int NC = G::NC, NS = G::NS, PS = G::PS, CR = G::CR, HH = G::HH, NKW = G::NKW;
    constexpr int NBLK = G::NBLK, PPT = G::PPT, NPX = G::NPX, LPX = G::LPX;
    constexpr int NTEN = M::NTEN, NSCAL = M::NSCAL;
    // LDS layout (floats): tensor 0, tensor 1 ([slot][PS]), then scalars ([slot])
    constexpr int OT1 = LPX * PS;
    constexpr int OS0 = NTEN * LPX * PS;
    constexpr int OS1 = OS0 + LPX;
    float *const lds = circatt_lds2;

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int jh = j & 7, jw = j >> 3;

    // lane bases (LDS pixel slots): block (bi, bj) of this wave starts at
    // slot 2 bi + CR (2 wv + 8 bj); element e sits (e % 2) + CR (e / 2) further
    const int slotA = (j & 1) + CR * (2 * wv + (j >> 1));  // element j (A rows of products 1)
    const int slotE = CR * (2 * wv + 2 * g);               // element 4g (r = 0)
    const int baseA = slotA * PS + 4 * g;
    const int baseT = slotE * PS + j;

    // ---- prefetch registers ----
    float hv[PPT][NTEN][NC];
    float hs[PPT][NSCAL > 0 ? NSCAL : 1];
    int hslot[PPT];
    float nr0[NS], nr1[NS], nry[NS];
    float nlse = 0.f;

    auto decode = [&](int item, int &unit, int &h0, int &w0) {
        const int ntiles = a.tiles_h * a.tiles_w;
        unit = item / ntiles;
        const int tile = item - unit * ntiles;
        const int th = tile % a.tiles_h;
        h0 = th * G::TH;
        w0 = (tile - th) / a.tiles_h * G::TW;
    };

    auto load_stage = [&](int item) {
        int unit, h0, w0;
        decode(item, unit, h0, w0);
        const int64_t uoff = (int64_t)unit * a.unit_stride;
        const float *src0 = (MODE == BWDKV ? a.q : a.k) + uoff;
        const float *src1 = (MODE == BWDKV ? a.dy : a.v) + uoff;
#pragma unroll
        for (int pp = 0; pp < PPT; ++pp) {
            const int px0 = threadIdx.x + 256 * pp;
            const bool pv = px0 < NPX;
            const int px = pv ? px0 : 0;
            const int kw = px / HH, kh = px - kw * HH;
            hslot[pp] = pv ? kh + CR * kw : -1;
            const int64_t gp = pmod(h0 - P + kh, a.n1) + (int64_t)a.n1 * pmod(w0 - P + kw, a.n2);
            if constexpr (CPLX) {
                const float2 *s0 = reinterpret_cast<const float2 *>(src0) + gp;
                const float2 *s1 = reinterpret_cast<const float2 *>(src1) + gp;
#pragma unroll
                for (int c = 0; c < NC / 2; ++c) {
                    const float2 x0 = s0[(int64_t)c * a.P];
                    const float2 x1 = s1[(int64_t)c * a.P];
                    hv[pp][0][2 * c] = x0.x;
                    hv[pp][0][2 * c + 1] = x0.y;
                    hv[pp][1][2 * c] = x1.x;
                    hv[pp][1][2 * c + 1] = x1.y;
                }
            } else {
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    hv[pp][0][c] = src0[gp + (int64_t)c * a.P];
                    hv[pp][1][c] = src1[gp + (int64_t)c * a.P];
                }
            }
            if constexpr (MODE == BWDKV) {
                const int64_t soff = (int64_t)unit * a.P;
                hs[pp][0] = a.lse[soff + gp];
                hs[pp][1] = a.dbuf[soff + gp];
            }
        }
    };

    auto load_regs = [&](int item) {
        int unit, h0, w0;
        decode(item, unit, h0, w0);
        const int rh = h0 + jh, rw = w0 + 2 * wv + jw;
        const bool rvalid = rh < a.n1 && rw < a.n2;
        const int64_t rpix = rvalid ? (int64_t)rh + (int64_t)a.n1 * rw : 0;
        const int64_t uoff = (int64_t)unit * a.unit_stride;
        const float *b0 = (MODE == BWDKV ? a.k : a.q) + uoff;
        const float *b1 = (MODE == BWDKV ? a.v : a.dy) + uoff;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int comp = 16 * (s >> 2) + 4 * g + (s & 3);
            const int64_t o = comp_off<CPLX>(a.P, rpix, comp);
            nr0[s] = b0[o];
            if constexpr (MODE != FWD) nr1[s] = b1[o];
            if constexpr (MODE == BWDQ) nry[s] = a.y[uoff + o];
        }
        if constexpr (MODE == BWDQ) nlse = a.lse[(int64_t)unit * a.P + rpix];
    };

    int k = 0;
    int item = item_of(a, 0);
    if (item >= a.nitems) return;  // uniform over the workgroup
    load_stage(item);
    load_regs(item);

    while (true) {
        int unit, h0, w0;
        decode(item, unit, h0, w0);
        const int rh = h0 + jh, rw = w0 + 2 * wv + jw;
        const bool rvalid = rh < a.n1 && rw < a.n2;
        const int64_t rpix = rvalid ? (int64_t)rh + (int64_t)a.n1 * rw : 0;
        const int64_t uoff = (int64_t)unit * a.unit_stride;
        const int64_t soff = (int64_t)unit * a.P;
        const float c2 = a.c2;

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
            raw2 += nr0[s] * nr0[s];
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

        // ---- issue the next item's global loads ----
        const int nitem = item_of(a, k + 1);
        const bool has_next = nitem < a.nitems;
        if (has_next) {
            load_stage(nitem);
            load_regs(nitem);
        }

        if constexpr (MODE == FWD) {
            // scores of all blocks: S[b][r] = c2 q.k (+ Distance key bias)
            f4 S[NBLK];
            static_for<NBLK>([&](auto B) {
                constexpr int b = decltype(B)::value;
                constexpr int bi = b / NKW, bj = b % NKW;
                constexpr int boff = 2 * bi + CR * 8 * bj;  // block slot offset
                f4 acc = f4{0.f, 0.f, 0.f, 0.f};
                if constexpr (DIST) {
                    const f2 lo = *reinterpret_cast<const f2 *>(&lds[OS0 + slotE + boff]);
                    const f2 hi = *reinterpret_cast<const f2 *>(&lds[OS0 + slotE + boff + CR]);
                    acc = f4{lo[0], lo[1], hi[0], hi[1]};
                }
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const f4 x = *reinterpret_cast<const f4 *>(&lds[baseA + boff * PS + 16 * t]);
                    acc = mfma(x[0], reg0[4 * t + 0], acc);
                    acc = mfma(x[1], reg0[4 * t + 1], acc);
                    acc = mfma(x[2], reg0[4 * t + 2], acc);
                    acc = mfma(x[3], reg0[4 * t + 3], acc);
                }
                S[b] = acc;
            });
            // window mask and exact row maximum
            float mx = -INFINITY;
            static_for<NBLK>([&](auto B) {
                constexpr int b = decltype(B)::value;
                constexpr int bi = b / NKW, bj = b % NKW;
                S[b][0] = mask_sel<lane_mask(P, bi, bj, 0)>(S[b][0], -INFINITY);
                S[b][1] = mask_sel<lane_mask(P, bi, bj, 1)>(S[b][1], -INFINITY);
                S[b][2] = mask_sel<lane_mask(P, bi, bj, 2)>(S[b][2], -INFINITY);
                S[b][3] = mask_sel<lane_mask(P, bi, bj, 3)>(S[b][3], -INFINITY);
                mx = fmaxf(mx, fmaxf(fmaxf(S[b][0], S[b][1]), fmaxf(S[b][2], S[b][3])));
            });
            const float m = gmax(mx);
            float lsum = 0.f;
            f4 acc[2][NT];
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[u][t] = f4{0.f, 0.f, 0.f, 0.f};
            static_for<NBLK>([&](auto B) {
                constexpr int b = decltype(B)::value;
                constexpr int bi = b / NKW, bj = b % NKW;
                constexpr int boff = 2 * bi + CR * 8 * bj;
                float p[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    p[r] = __builtin_amdgcn_exp2f(S[b][r] - m);
                    lsum += p[r];
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int roff = ((r & 1) + CR * (r >> 1)) * PS;
#pragma unroll
                    for (int t = 0; t < NT; ++t)
                        acc[b & 1][t] = mfma(lds[OT1 + baseT + boff * PS + roff + 16 * t], p[r],
                                             acc[b & 1][t]);
                }
            });
            const float l = gsum(lsum);
            const float inv = 1.f / l;
            if (rvalid) {
                float *yb = a.yout + uoff;
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        yb[comp_off<CPLX>(a.P, rpix, 16 * t + 4 * g + r)] =
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
            static_for<NBLK>([&](auto B) {
                constexpr int b = decltype(B)::value;
                constexpr int bi = b / NKW, bj = b % NKW;
                constexpr int boff = 2 * bi + CR * 8 * bj;
                f4 s = cS, dp = cD;
                if constexpr (DIST) {
                    const f2 lo = *reinterpret_cast<const f2 *>(&lds[OS0 + slotE + boff]);
                    const f2 hi = *reinterpret_cast<const f2 *>(&lds[OS0 + slotE + boff + CR]);
                    s = s + f4{lo[0], lo[1], hi[0], hi[1]};
                }
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const f4 x = *reinterpret_cast<const f4 *>(&lds[baseA + boff * PS + 16 * t]);
                    const f4 w =
                        *reinterpret_cast<const f4 *>(&lds[OT1 + baseA + boff * PS + 16 * t]);
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
                            mfma(lds[baseT + boff * PS + roff + 16 * t], ds[r], acc[b & 1][t]);
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
                        ob[comp_off<CPLX>(a.P, rpix, 16 * t + 4 * g + r)] = val * a.scale;
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
            static_for<NBLK>([&](auto B) {
                constexpr int b = decltype(B)::value;
                constexpr int bi = b / NKW, bj = b % NKW;
                constexpr int boff = 2 * bi + CR * 8 * bj;
                const f2 alo = *reinterpret_cast<const f2 *>(&lds[OS0 + slotE + boff]);
                const f2 ahi = *reinterpret_cast<const f2 *>(&lds[OS0 + slotE + boff + CR]);
                const f2 dlo = *reinterpret_cast<const f2 *>(&lds[OS1 + slotE + boff]);
                const f2 dhi = *reinterpret_cast<const f2 *>(&lds[OS1 + slotE + boff + CR]);
                f4 s = f4{alo[0], alo[1], ahi[0], ahi[1]};
                if constexpr (DIST) s = s + f4{kb, kb, kb, kb};
                f4 dp = f4{dlo[0], dlo[1], dhi[0], dhi[1]};
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const f4 x = *reinterpret_cast<const f4 *>(&lds[baseA + boff * PS + 16 * t]);
                    const f4 w =
                        *reinterpret_cast<const f4 *>(&lds[OT1 + baseA + boff * PS + 16 * t]);
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
                        accv[b & 1][t] = mfma(lds[OT1 + baseT + boff * PS + roff + 16 * t], p[r],
                                              accv[b & 1][t]);
                        acck[b & 1][t] =
                            mfma(lds[baseT + boff * PS + roff + 16 * t], ds[r], acck[b & 1][t]);
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
                        const int64_t o = comp_off<CPLX>(a.P, rpix, 16 * t + 4 * g + r);
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
template <int P, int NT, bool CPLX, bool DIST, int MODE>
hipError_t launch(const Args &a0, int cus, hipStream_t s) {
    using LS = LdsSize<P, NT, CPLX, DIST, MODE>;
    auto kern = kernel2d<P, NT, CPLX, DIST, MODE>;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)LS::bytes);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    Args a = a0;
    const int wg_per_cu = LS::bytes <= 80 * 1024 ? 2 : 1;
    int64_t grid = (int64_t)cus * wg_per_cu;
    grid = std::min<int64_t>(grid, 8LL * a.per_xcd);
    grid = std::max<int64_t>(8, grid / 8 * 8);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(256), LS::bytes, s, a);
    return hipGetLastError();
}

// Launch of one mode for the compiled-in shapes: half widths P in
// {1, 2, 3, 5, 7}, 16 or 32 real components per pixel, Float32 or
// ComplexF32, Dot or Distance.  Other shapes return hipErrorNotSupported
// without launching.
template <int MODE>
hipError_t dispatch(int p, int nt, bool cplx, bool dist, const Args &a, int cus, hipStream_t s) {
#define CIRCATT_F2D_CASE(PP, NTT)                                                      \
    if (p == PP && nt == NTT) {                                                        \
        if (cplx) return dist ? launch<PP, NTT, true, true, MODE>(a, cus, s)           \
                              : launch<PP, NTT, true, false, MODE>(a, cus, s);         \
        return dist ? launch<PP, NTT, false, true, MODE>(a, cus, s)                    \
                    : launch<PP, NTT, false, false, MODE>(a, cus, s);                  \
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
    return hipErrorNotSupported;
}

inline bool supported(int nsp, int p, int ncr) {
    return nsp == 2 && (p == 1 || p == 2 || p == 3 || p == 5 || p == 7) && (ncr == 16 || ncr == 32);
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
