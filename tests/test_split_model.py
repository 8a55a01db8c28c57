"""CPU checks of the split-half arithmetic (tests/split_model.py, a numpy
restatement of csrc/fused2h_impl.h's products and power-of-two scaling)
against the float64 oracle, at magnitudes from 1e-7 to 1e4.

They pin (1) the split itself: hi + lo carries 22 bits while |x| >= 2^-3 and
an absolute error of at most 2^-25 below, and overflows at 65520; (2) that
the products without scaling lose Float32's range (dq, dk vanish at the
upstream-gradient scale of the reference's own loss, test/grad.jl:58-61);
(3) that with the kernels' scaling rules every output stays within the
tolerances at every magnitude.  The GPU kernels are checked against the
same oracle by tests/test_gpu_magnitudes.py.
"""
import math

import numpy as np
import pytest

from conftest import TOL_FWD, TOL_GRAD, rel_err

import oracle as O  # noqa: E402
import split_model as M  # noqa: E402


def test_split_error_bounds():
    rng = np.random.default_rng(1)
    for e in range(-30, 15):
        x = (rng.uniform(1, 2, 4096) * 2.0 ** e * rng.choice([-1, 1], 4096)).astype(np.float32)
        err = np.abs(M.rep(x) - x.astype(np.float64))
        if e >= -3:
            # both halves normal: 22 significant bits
            assert np.all(err <= np.abs(x) * 2.0 ** -22), e
        else:
            # lo subnormal (spacing 2^-24): absolute error up to half of it
            assert np.all(err <= 2.0 ** -25), e
            if e <= -12:
                assert err.max() > np.abs(x).max() * 2.0 ** -20, e  # relative precision lost
    big = np.array([65519.0, 65520.0, -70000.0], np.float32)
    hi, _ = M.split(big)
    assert np.isfinite(hi[0]) and np.isinf(hi[1]) and np.isinf(hi[2])


def test_shift_rule():
    assert M.shift_of(1.0) == 0 and M.shift_of(0.25) == 0 and M.shift_of(31.9) == 0
    for m in (1e-7, 1e-3, 0.2, 32.0, 1e4, 3e30):
        s = M.shift_of(m)
        assert 4.0 <= m * 2.0 ** s < 8.0, m
    assert M.shift_of(0.0) == 0


def unit_inputs(seed, dims, dh, scales):
    rng = np.random.default_rng(seed)
    P = int(np.prod(dims))
    return [(rng.standard_normal((dh, P)) * s).astype(np.float32) for s in scales]


def model_errors(kind, dims, ws, q, k, v, dy, scaled):
    dh, P = q.shape
    shape = (1, dh, *reversed(dims))
    qo, ko, vo, dyo = (a.astype(np.float64).reshape(shape) for a in (q, k, v, dy))
    yr, _ = O.attention_fwd(kind, qo, ko, vo, ws)
    gr = O.attention_bwd(kind, qo, ko, vo, dyo, ws)
    y, lse = M.fused_fwd(kind, q, k, v, ws, dims, scaled)
    g = M.fused_bwd(kind, q, k, v, y.astype(np.float32), dy, lse, ws, dims, scaled)
    return [rel_err(y, yr.reshape(dh, P))] + [rel_err(a, b.reshape(dh, P)) for a, b in zip(g, gr)]


@pytest.mark.parametrize("kind", [0, 1])
def test_unscaled_split_loses_small_gradients(kind):
    """Without scaling, an upstream gradient of ~1e-7 makes dS round to zero in
    f16: dq and dk vanish (error 1), and v of 1e-3 already costs y 1e-5."""
    dims, ws = (16, 16), 15
    q, k, v, dy = unit_inputs(7, dims, 16, (1, 1, 1, 1.2e-7))
    e = model_errors(kind, dims, ws, q, k, v, dy, scaled=False)
    assert e[1] > 0.5 and e[2] > 0.5, e
    q, k, v, dy = unit_inputs(8, dims, 16, (1, 1, 1e-3, 1e-3))
    e = model_errors(kind, dims, ws, q, k, v, dy, scaled=False)
    assert e[0] > TOL_FWD and e[1] > TOL_GRAD, e


CASES = [((16, 16), 15), ((16, 16), 7), ((12, 10), 5), ((9, 11), 3)]


SCALINGS = [(w, m) for w in ("v_dy", "q_k", "all") for m in (1e-7, 1e-5, 1e-3, 1.0, 1e2, 1e4)
            if w == "v_dy" or m <= 1]


@pytest.mark.parametrize("dims,ws", CASES)
@pytest.mark.parametrize("which,mag", SCALINGS)
@pytest.mark.parametrize("kind", [0, 1])
def test_scaled_split_within_tolerance(dims, ws, which, mag, kind):
    """With the per-item power-of-two scaling every output meets the bar at
    every magnitude of v and dy and at every magnitude of q and k up to 1
    (beyond, the scores themselves pass ~1e3 and a Float32 softmax is
    ill-conditioned whatever the arithmetic; the GPU tests bound that regime
    by the reference's own Float32 error)."""
    sv = mag if which in ("v_dy", "all") else 1.0
    sq = mag if which in ("q_k", "all") else 1.0
    seed = 40 + ws + int(math.log10(mag)) + 3 * kind
    q, k, v, dy = unit_inputs(seed, dims, 16, (sq, sq, sv, sv))
    e = model_errors(kind, dims, ws, q, k, v, dy, scaled=True)
    assert e[0] < TOL_FWD, e
    assert max(e[1:]) < TOL_GRAD, e


def offset_inputs(seed, dims, dh, c):
    rng = np.random.default_rng(seed)
    P = int(np.prod(dims))
    q, k = ((rng.standard_normal((dh, P)) + c).astype(np.float32) for _ in range(2))
    v, dy = (rng.standard_normal((dh, P)).astype(np.float32) for _ in range(2))
    return q, k, v, dy


def model_errors_c(kind, dims, ws, q, k, v, dy, **kw):
    dh, P = q.shape
    shape = (1, dh, *reversed(dims))
    qo, ko, vo, dyo = (a.astype(np.float64).reshape(shape) for a in (q, k, v, dy))
    yr, _ = O.attention_fwd(kind, qo, ko, vo, ws)
    gr = O.attention_bwd(kind, qo, ko, vo, dyo, ws)
    y, lse = M.fused_fwd(kind, q, k, v, ws, dims, True, **kw)
    g = M.fused_bwd(kind, q, k, v, y.astype(np.float32), dy, lse, ws, dims, True, **kw)
    return [rel_err(y, yr.reshape(dh, P))] + [rel_err(a, b.reshape(dh, P)) for a, b in zip(g, gr)]


@pytest.mark.parametrize("dims,ws", [((16, 16), 15), ((12, 10), 5), ((9, 11), 3)])
@pytest.mark.parametrize("c", [3.0, 10.0, 30.0])
def test_distance_centred_on_offset_inputs(dims, ws, c):
    """Distance similarity is translation-invariant (src/similarity.jl:55-78
    forms -|x - y|^2 / 2 directly).  The kernels' expansion q.k - |k|^2/2
    - |q|^2/2 is not: on q, k = N(0,1) + c its Float32 terms grow with c^2.
    Centred on one key pixel per pass (a different one in each pass) the
    expansion meets the usual bar at every offset; uncentred it is at least
    five times worse from c = 10 (near the forward bar there) and misses the
    gradient bar at c = 30."""
    q, k, v, dy = offset_inputs(60 + ws + int(c), dims, 16, c)
    e = model_errors_c(1, dims, ws, q, k, v, dy)
    assert e[0] < TOL_FWD and max(e[1:]) < TOL_GRAD, e
    if c >= 10:
        e0 = model_errors_c(1, dims, ws, q, k, v, dy, centre_px=None)
        assert min(a / b for a, b in zip(e0, e)) > 5, (e0, e)
        if c >= 30:
            assert max(e0[1:]) > TOL_GRAD, e0


@pytest.mark.parametrize("dims,ws", [((16, 16), 15), ((12, 10), 5)])
@pytest.mark.parametrize("kind,mag", [(0, 3e2), (0, 1e3), (0, 1e4), (1, 1e2), (1, 1e3), (1, 1e4)])
def test_slow_walk_within_flash_bound(dims, ws, kind, mag):
    """q, k scaled so far that the split-half walks take their slow form
    (q normalised per pixel, every score unscaled by 2^-eu after its
    product): the modelled kernels stay within the large-score bar of
    tests/large_scores.py for y, dq, dk and dv, and the same model with the
    unscale's sign flipped (a planted mistake) fails it."""
    from large_scores import abs_err, flash_bounds
    rng = np.random.default_rng(70 + ws + kind)
    P = int(np.prod(dims))
    q, k, v, dy = (rng.standard_normal((16, P)).astype(np.float32) for _ in range(4))
    q, k = q * np.float32(mag), k * np.float32(mag)
    shape = (1, 16, *reversed(dims))
    qo, ko, vo, dyo = (a.reshape(shape) for a in (q, k, v, dy))
    yr, _ = O.attention_fwd(kind, *(a.astype(np.float64) for a in (qo, ko, vo)), ws)
    gr = O.attention_bwd(kind, *(a.astype(np.float64) for a in (qo, ko, vo, dyo)), ws)
    refs = [yr.reshape(16, P)] + [g.reshape(16, P) for g in gr]
    bars = flash_bounds(kind, qo, ko, vo, dyo, ws, 1, refs)
    with np.errstate(all="ignore"):
        for sign in (1, -1):
            y, lse = M.fused_fwd(kind, q, k, v, ws, dims, True, slow_sign=sign)
            g = M.fused_bwd(kind, q, k, v, y.astype(np.float32), dy, lse, ws, dims, True,
                            slow_sign=sign)
            ok = [abs_err(a, r) <= b for a, r, b in zip([y, *g], refs, bars)]
            if sign == 1:
                assert all(ok), ([abs_err(a, r) / b for a, r, b in zip([y, *g], refs, bars)])
            else:
                assert not all(ok)
