// Host planning and dispatch of the windowed-tile MFMA kernels (kernels in
// fused_impl.h, one translation unit per mode in fused_<mode>.hip).
#include "fused2d_impl.h"
#include "fused2h_impl.h"
#include "fused_impl.h"
#include "fused_wide_impl.h"

namespace circatt {

// ---------------------------------------------------------------------------
// host planning and dispatch
// ---------------------------------------------------------------------------
namespace {

using Plan = FusedPlan;

int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

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
    a.cl = pr.cl;
    a.nheads = pr.nheads;
    a.ncrall = pr.nheads * pr.dh * pr.ncomp;
    a.scale = pr.scale;
    a.c2 = pr.scale * kLog2e;
    pl.nc = a.ncr <= 16 ? 16 : a.ncr <= 32 ? 32 : a.ncr <= 64 ? 64 : 0;
    if (pl.nc == 0) return pl;
    const bool dist = pr.kind == 1;
    const int ntensor = mode == MODE_SIM ? 1 : 2;
    const int nscalar = mode == MODE_BWDKV ? 2 : (dist ? 1 : 0);
    const int ppt = pl.nc * ntensor <= 32 ? 2 : 1;
    // (Distance: nc floats after the halo hold the item's centre)
    a.hg = plan_halo(pr.g.nsp, pr.g.p, pl.nc, ntensor, nscalar, ppt, dist ? pl.nc : 0);
    if (!a.hg.ok) return pl;
    if (pr.g.nsp == 2) {
        a.tiles_h = (pr.g.n1 + 7) / 8;
        a.tiles_w = (pr.g.n2 + 7) / 8;
    } else {
        a.tiles_h = (pr.g.n1 + 63) / 64;
        a.tiles_w = 1;
    }
    pl.lds_bytes = (size_t)a.hg.lds_floats * sizeof(float);
    const int64_t nitems = (int64_t)a.tiles_h * a.tiles_w * pr.nunits;
    if (nitems <= 0 || nitems > INT32_MAX / 2) return pl;
    a.nitems = (int)nitems;
    a.per_xcd = (int)((nitems + 7) / 8);
    // persistent grid: a multiple of 8 workgroups (one run per XCD), at most
    // one workgroup per item of each XCD run
    const int wg_per_cu = (int)std::max<size_t>(1, std::min<size_t>(2, kLdsMax / pl.lds_bytes));
    int64_t grid = (int64_t)device_cus() * wg_per_cu;
    grid = std::min<int64_t>(grid, 8LL * a.per_xcd);
    grid = std::max<int64_t>(8, grid / 8 * 8);
    pl.grid = dim3((unsigned)grid);
    pl.ok = true;
    return pl;
}

// Channel-chunked kernels (fused_wide_impl.h) for heads wider than 64 real
// components.
struct WidePlan {
    FArgs a;
    size_t lds_bytes;
    dim3 grid;
    bool ok;
};

WidePlan make_wide_plan(FusedMode mode, const FusedProblem &pr) {
    WidePlan wp{};
    if (mode == MODE_SIM) return wp;
    const bool dist = pr.kind == 1;
    const int ntensor = mode == MODE_FWD ? 1 : 2;
    const int nscal = mode == MODE_BWDKV ? 2 : (dist ? 1 : 0);
    const wide::Plan w = wide::plan(pr.g.nsp, pr.g.p, ntensor, nscal);
    if (!w.ok) return wp;
    FArgs &a = wp.a;
    a.q = pr.q; a.k = pr.k; a.v = pr.v; a.y = pr.y; a.dy = pr.dy; a.lse = pr.lse;
    a.yout = pr.yout; a.lse_out = pr.lse_out; a.dq = pr.dq; a.dk = pr.dk; a.dv = pr.dv;
    a.dbuf = pr.dbuf;
    a.g = pr.g;
    a.hg = w.hg;
    a.dh = pr.dh;
    a.ncomp = pr.ncomp;
    a.ncr = pr.dh * pr.ncomp;
    a.unit_stride = pr.g.P * pr.dh * pr.ncomp;
    a.cl = pr.cl;
    a.nheads = pr.nheads;
    a.ncrall = pr.nheads * pr.dh * pr.ncomp;
    a.scale = pr.scale;
    a.c2 = pr.scale * kLog2e;
    a.rb = w.rb;
    a.cr = w.cr;
    a.nst = w.nst;
    a.ncc = (a.ncr + wide::CC - 1) / wide::CC;
    a.noc = (a.ncr + wide::OC - 1) / wide::OC;
    if (pr.g.nsp == 2) {
        a.tiles_h = (pr.g.n1 + 7) / 8;
        a.tiles_w = (pr.g.n2 + 7) / 8;
    } else {
        a.tiles_h = (pr.g.n1 + 63) / 64;
        a.tiles_w = 1;
    }
    const int64_t nitems = (int64_t)a.tiles_h * a.tiles_w * pr.nunits;
    if (nitems <= 0 || nitems > INT32_MAX / 2) return wp;
    a.nitems = (int)nitems;
    a.per_xcd = (int)((nitems + 7) / 8);
    int64_t grid = (int64_t)device_cus() * 2;
    grid = std::min<int64_t>(grid, 8LL * a.per_xcd);
    grid = std::max<int64_t>(8, grid / 8 * 8);
    wp.grid = dim3((unsigned)grid);
    wp.lds_bytes = (size_t)w.lds_floats * sizeof(float);
    wp.ok = true;
    return wp;
}

}  // namespace

bool fused_supported(FusedMode mode, const FusedProblem &pr) {
    Plan pl = make_plan(mode, pr);
    return pl.ok || make_wide_plan(mode, pr).ok;
}

// Compile-time-window 2D kernels (fused2d_impl.h) for the shapes they cover;
// hipErrorNotSupported otherwise.
hipError_t launch_f2d(FusedMode mode, const FusedProblem &pr, hipStream_t s) {
    const int ncr = pr.dh * pr.ncomp;
    // one-dimensional signals: the split-half kernels of the windows they
    // instantiate (no Float32 matrix-core counterpart)
    const bool one = pr.g.nsp == 1 && math_mode() == CIRCATT_MATH_SPLIT_F16 &&
                     f2h::supported1(pr.g.p, ncr) && pr.g.P * ncr * 4 < (int64_t)INT32_MAX;
    if (mode == MODE_SIM || !(one || f2d::supported(pr.g.nsp, pr.g.p, ncr, pr.g.P)) ||
        pr.nunits > INT32_MAX)
        return hipErrorNotSupported;
    f2d::Args a{};
    a.q = pr.q; a.k = pr.k; a.v = pr.v; a.y = pr.y; a.dy = pr.dy; a.lse = pr.lse;
    a.yout = pr.yout; a.lse_out = pr.lse_out; a.dq = pr.dq; a.dk = pr.dk; a.dv = pr.dv;
    a.dbuf = pr.dbuf;
    a.n1 = pr.g.n1;
    a.n2 = pr.g.n2;
    a.P = (int)pr.g.P;
    a.unit_stride = (int)(pr.g.P * ncr);
    a.cl = pr.cl;
    a.nheads = pr.nheads;
    a.ncrall = pr.nheads * ncr;
    a.scale = pr.scale;
    a.c2 = pr.scale * kLog2e;
    a.nunits = (int)pr.nunits;
    const int nt = ncr / 16;
    const bool cplx = pr.ncomp == 2, dist = pr.kind == 1;
    const int cus = device_cus();
    if (one) {
        if (nt == 1) {
            if (mode == MODE_FWD) return launch_f1h_fwd(pr.g.p, cplx, dist, a, cus, s);
            if (mode == MODE_BWDQ) return launch_f1h_bwdq(pr.g.p, cplx, dist, a, cus, s);
            return launch_f1h_bwdkv(pr.g.p, cplx, dist, a, cus, s);
        }
        if (mode == MODE_FWD) return launch_f1h2_fwd(pr.g.p, cplx, dist, a, cus, s);
        if (mode == MODE_BWDQ) return launch_f1h2_bwdq(pr.g.p, cplx, dist, a, cus, s);
        return launch_f1h2_bwdkv(pr.g.p, cplx, dist, a, cus, s);
    }
    if (nt == 1 && math_mode() == CIRCATT_MATH_SPLIT_F16) {
        hipError_t e = hipErrorNotSupported;
        if (mode == MODE_FWD) e = launch_f2h_fwd(pr.g.p, cplx, dist, a, cus, s);
        if (mode == MODE_BWDQ) e = launch_f2h_bwdq(pr.g.p, cplx, dist, a, cus, s);
        if (mode == MODE_BWDKV) e = launch_f2h_bwdkv(pr.g.p, cplx, dist, a, cus, s);
        if (e != hipErrorNotSupported) return e;
    }
    if (nt == 2 && math_mode() == CIRCATT_MATH_SPLIT_F16) {
        hipError_t e = hipErrorNotSupported;
        if (mode == MODE_FWD) e = launch_f2h2_fwd(pr.g.p, cplx, dist, a, cus, s);
        if (mode == MODE_BWDQ) e = launch_f2h2_bwdq(pr.g.p, cplx, dist, a, cus, s);
        if (mode == MODE_BWDKV) e = launch_f2h2_bwdkv(pr.g.p, cplx, dist, a, cus, s);
        if (e != hipErrorNotSupported) return e;
    }
    switch (mode) {
    case MODE_FWD: return launch_f2d_fwd(pr.g.p, nt, cplx, dist, a, cus, s);
    case MODE_BWDQ: return launch_f2d_bwdq(pr.g.p, nt, cplx, dist, a, cus, s);
    case MODE_BWDKV: return launch_f2d_bwdkv(pr.g.p, nt, cplx, dist, a, cus, s);
    default: return hipErrorNotSupported;
    }
}

hipError_t launch_fused(FusedMode mode, const FusedProblem &pr, hipStream_t s) {
    if (mode != MODE_SIM) {
        hipError_t e = launch_f2d(mode, pr, s);
        if (e != hipErrorNotSupported) return e;
    }
    Plan pl = make_plan(mode, pr);
    if (!pl.ok) {
        const WidePlan wp = make_wide_plan(mode, pr);
        if (!wp.ok) return hipErrorNotSupported;
        return launch_wide(mode, pr.g.nsp, pr.kind == 1, wp.a, wp.lds_bytes, wp.grid, s);
    }
    const bool dist = pr.kind == 1;
    switch (mode) {
    case MODE_FWD: return launch_fused_fwd(pl, pr.g.nsp, dist, s);
    case MODE_SIM: return launch_fused_sim(pl, pr.g.nsp, dist, s);
    case MODE_BWDQ: return launch_fused_bwdq(pl, pr.g.nsp, dist, s);
    case MODE_BWDKV: return launch_fused_bwdkv(pl, pr.g.nsp, dist, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace circatt
