"""GPU parity of the fused kernels across FP32's range of magnitudes.

The default fused kernels split every Float32 operand into two f16 halves
(csrc/fused2h_impl.h) and rescale operands by powers of two per work item so
that the halves keep Float32's range.  These tests scale the seeded N(0,1)
inputs of the parity cases by factors from 1e-7 to 1e4 and compare y, dq, dk,
dv with the float64 oracle at the usual bar (1e-5 forward, 1e-4 gradients).

Large q and k make the scores large, and a Float32 computation of the softmax
is then ill-conditioned whatever the arithmetic: the reference's own Float32
algorithm (the oracle's float32 build, unfused, A materialised) misses 1e-4
on dq, dk from q, k ~ 1e2 on, and a flash-style backward, which recomputes
P = exp(S - lse) from the stored lse, loses more.  For q, k scaled past 1
every output is held to the large-score bar of tests/large_scores.py: 8x the
error of a Float32 flash-style restatement, or of the unit roundoff on the
magnitude of the terms the output sums, whichever is larger.  From about
q, k x 1e2 the split-half backward passes switch waves to their slow walk
(q normalised per pixel, each score unscaled by 2^-eu after its product;
at x 1e2 only the waves holding the largest values), and from x 1e4 the
forward too; a slow walk with a wrong unscale fails that bar (shown on the
CPU model by tests/test_split_model.py).
"""
import math

import numpy as np
import pytest

from conftest import TOL_FWD, TOL_GRAD, rel_err
from large_scores import abs_err, flash_bounds

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle as O  # noqa: E402


@pytest.fixture(scope="module")
def ca(cuda):
    import circulant_attention
    return circulant_attention


def seeded(seed, shape, cplx=False):
    rng = np.random.default_rng(seed)
    if cplx:
        a = (rng.standard_normal(shape) + 1j * rng.standard_normal(shape)) / np.sqrt(2)
        return a.astype(np.complex64)
    return rng.standard_normal(shape).astype(np.float32)


def dev(a, cuda):
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def host(t):
    t = t.detach().cpu()
    return t.numpy().astype(np.complex128 if t.is_complex() else np.float64)


def f64(a):
    return a.astype(np.complex128 if np.iscomplexobj(a) else np.float64)


def fused(ca, cuda, kind, q, k, v, dy, ws, nh):
    tq, tk, tv = (dev(a, cuda).requires_grad_(True) for a in (q, k, v))
    simfun = ca.DotSimilarity() if kind == 0 else ca.DistanceSimilarity()
    if nh == 1:
        y, _ = ca.circulant_attention(simfun, tq, tk, tv, ws, materialize=False)
    else:
        y, _ = ca.circulant_mh_attention(simfun, tq, tk, tv, ws, nh, materialize=False,
                                         honor_simfun=True)
    td = dev(dy, cuda)
    loss = (y * td.conj()).real.sum() if y.is_complex() else (y * td).sum()
    loss.backward()
    return host(y), host(tq.grad), host(tk.grad), host(tv.grad)


# (dims, ws, C, B, nheads): 16 real components per head, every window of the
# split-half kernels, partial tiles and halos that wrap
CASES = [((40, 24), 15, 64, 1, 4), ((20, 18), 11, 16, 2, 1), ((17, 13), 7, 32, 1, 2),
         ((12, 10), 5, 16, 2, 1), ((9, 11), 3, 16, 1, 1)]
# 32 real components per head (the 8x16-tile kernels), every window they cover
CASES32 = [((20, 18), 11, 32, 2, 1), ((17, 13), 7, 64, 1, 2), ((12, 10), 5, 32, 1, 1),
           ((9, 11), 3, 64, 1, 2)]
# one-dimensional signals (the 1D split-half kernels: windows 15 and 63, 16 and
# 32 real components per head; lengths that are and are not multiples of 4
# select the row DMA or the per-pixel loads for real signals)
CASES1D = [((300,), 63, 32, 1, 2), ((258,), 15, 16, 2, 1), ((260,), 63, 32, 2, 1), ((130,), 15, 64, 1, 2)]
MAGS = [1e-7, 1e-5, 1e-3, 1e2, 1e4]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-ws{c[1]}")
@pytest.mark.parametrize("which", ["v_dy", "q_k", "all"])
@pytest.mark.parametrize("mag", MAGS)
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [0, 1])
def test_fused_across_magnitudes(ca, cuda, case, which, mag, cplx, kind):
    _across_magnitudes(ca, cuda, case, which, mag, cplx, kind, 0)


@pytest.mark.parametrize("case", CASES32, ids=lambda c: f"{c[0]}-ws{c[1]}")
@pytest.mark.parametrize("which", ["v_dy", "q_k", "all"])
@pytest.mark.parametrize("mag", MAGS)
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [0, 1])
def test_fused_across_magnitudes_32(ca, cuda, case, which, mag, cplx, kind):
    _across_magnitudes(ca, cuda, case, which, mag, cplx, kind, 50)


@pytest.mark.parametrize("case", CASES1D, ids=lambda c: f"{c[0]}-ws{c[1]}-C{c[2]}-h{c[4]}")
@pytest.mark.parametrize("which", ["v_dy", "q_k", "all"])
@pytest.mark.parametrize("mag", MAGS)
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [0, 1])
def test_fused_across_magnitudes_1d(ca, cuda, case, which, mag, cplx, kind):
    _across_magnitudes(ca, cuda, case, which, mag, cplx, kind, 80)


def _across_magnitudes(ca, cuda, case, which, mag, cplx, kind, seed0):
    dims, ws, C, B, nh = case
    if cplx:
        C //= 2  # the same real components per head either way
    shape = (B, C, *reversed(dims))
    seed = 3000 + seed0 + 17 * ws + int(math.log10(mag)) + 7 * kind + (100 if cplx else 0)
    q, k, v, dy = (seeded(seed + i, shape, cplx) for i in range(4))
    sv = mag if which in ("v_dy", "all") else 1.0
    sq = mag if which in ("q_k", "all") else 1.0
    q, k = (a * np.float32(sq) for a in (q, k))
    v, dy = (a * np.float32(sv) for a in (v, dy))
    print(f"magnitudes: dims={dims} ws={ws} C={C} nh={nh} which={which} mag={mag} "
          f"cplx={cplx} kind={kind}", flush=True)
    y, dq, dk, dv = fused(ca, cuda, kind, q, k, v, dy, ws, nh)
    yr, _ = O.attention_fwd(kind, *(f64(a) for a in (q, k, v)), ws, nh)
    gr = O.attention_bwd(kind, *(f64(a) for a in (q, k, v, dy)), ws, nh)
    if sq > 1:
        bars = flash_bounds(kind, q, k, v, dy, ws, nh, [yr, *gr])
        for name, o, r, b in zip(("y", "dq", "dk", "dv"), (y, dq, dk, dv), (yr, *gr), bars):
            assert abs_err(o, r) <= b, (name, abs_err(o, r), b)
        return
    assert rel_err(y, yr) < TOL_FWD
    for name, g, r in zip(("dq", "dk", "dv"), (dq, dk, dv), gr):
        assert rel_err(g, r) < TOL_GRAD, (name, rel_err(g, r))


@pytest.mark.parametrize("kind", [0, 1])
def test_fused_at_the_reference_loss_scale(ca, cuda, kind):
    """test/grad.jl:58-61 trains on sum(abs2, y - z) / length(y): at cfg3's
    size (16.8M values) the upstream gradient 2(y - z)/length(y) is ~1e-7.
    The cfg3 geometry at reduced size, with dy of that scale."""
    dims, ws, C, B, nh = (48, 32), 15, 64, 2, 4
    shape = (B, C, *reversed(dims))
    q, k, v, z = (seeded(3500 + i + 10 * kind, shape) for i in range(4))
    yr, _ = O.attention_fwd(kind, *(f64(a) for a in (q, k, v)), ws, nh)
    n_cfg3 = 256 * 256 * 64 * 4
    dy = (2.0 * (yr - z) / n_cfg3).astype(np.float32)
    assert 1e-8 < np.abs(dy).max() < 1e-6
    y, dq, dk, dv = fused(ca, cuda, kind, q, k, v, dy, ws, nh)
    gr = O.attention_bwd(kind, *(f64(a) for a in (q, k, v, dy)), ws, nh)
    assert rel_err(y, yr) < TOL_FWD
    for name, g, r in zip(("dq", "dk", "dv"), (dq, dk, dv), gr):
        assert np.abs(g).max() > 0, name
        assert rel_err(g, r) < TOL_GRAD, (name, rel_err(g, r))


def central_gap(kind, q, k, ws, nh, tile_h=16, tile_w=16, crows=2, ccols=16, crow0=8):
    """Largest (over queries) of max_window(s) - max_central(s) in log2 units,
    where the central keys are the block pair the split-half forward takes its
    reference maximum from: crows halo rows from tile row 8 wh + crow0 - P of
    the query's wavefront and ccols halo columns from 2 ww - P (rows 8, 9 x 16
    columns for 2x8 LDS blocks at ws 15; 8..11 x 8 for the 4x4 blocks at ws 11;
    4..7 x 8 for 2x8 blocks at ws 5 and 7; 0..7 x 4 for 4x4 blocks at ws 3), on
    tiles of tile_h x tile_w pixels (16 x 16, or 8 x 16 for 32 real components)."""
    dims = O.spatial_dims(q)
    n1, n2 = dims
    P = (ws - 1) // 2
    qf, kf = O._flat(q, nh), O._flat(k, nh)
    dh = qf.shape[1]
    S = O.similarity(kind, f64(qf), f64(kf), dims, ws, 1.0 / math.sqrt(dh))
    S = S.reshape(qf.shape[0], n1 * n2, ws * ws) * (1.0 / math.log(2.0))
    _, colval = O.pattern(dims, ws, 1)
    cols = colval.reshape(n1 * n2, -1) - 1
    best = -np.inf
    for r in range(n1 * n2):
        h, w = r % n1, r // n1
        th, tw = h % tile_h, w % tile_w
        wh, ww = th // 8, tw // 2
        rows = {(h - th + 8 * wh + crow0 - P + d) % n1 for d in range(crows)}
        cset = {(w - tw + 2 * ww - P + d) % n2 for d in range(ccols)}
        central = np.array([(c % n1) in rows and (c // n1) in cset for c in cols[r]])
        gap = S[:, r, :].max(axis=1) - np.where(central, S[:, r, :], -np.inf).max(axis=1)
        best = max(best, float(gap.max()))
    return best


# the central pair of each window: (first row, rows, columns) of the key region
CENTRAL = {3: (0, 8, 4), 5: (4, 4, 8), 7: (4, 4, 8), 11: (8, 4, 8), 15: (8, 2, 16)}


@pytest.mark.parametrize("ws", [3, 5, 7, 11, 15])
@pytest.mark.parametrize("kind", [0, 1])
def test_fused_forward_redo_path(ca, cuda, ws, kind):
    """The split-half forward takes its softmax reference maximum from a
    central block pair and redoes an item with the exact row maximum when
    some score passes it by more than 8 (log2 units).  q and k scaled by 2.5
    make such scores common; the test first checks on the CPU that they
    occur, then the GPU result against the oracle."""
    dims, C, B, nh = (40, 24), 32, 1, 2
    shape = (B, C, *reversed(dims))
    q, k, v, dy = (seeded(3600 + i + ws + 5 * kind, shape) for i in range(4))
    q, k = q * np.float32(2.5), k * np.float32(2.5)
    crow0, crows, ccols = CENTRAL[ws]
    assert central_gap(kind, q, k, ws, nh, crows=crows, ccols=ccols, crow0=crow0) > 8.5
    y, dq, dk, dv = fused(ca, cuda, kind, q, k, v, dy, ws, nh)
    yr, _ = O.attention_fwd(kind, *(f64(a) for a in (q, k, v)), ws, nh)
    gr = O.attention_bwd(kind, *(f64(a) for a in (q, k, v, dy)), ws, nh)
    assert rel_err(y, yr) < TOL_FWD
    for name, g, r in zip(("dq", "dk", "dv"), (dq, dk, dv), gr):
        assert rel_err(g, r) < TOL_GRAD, (name, rel_err(g, r))


@pytest.mark.parametrize("ws", [3, 7, 11])
@pytest.mark.parametrize("kind", [0, 1])
def test_fused_forward_redo_path_32(ca, cuda, ws, kind):
    """The redo path of the forward for 32 real components per head (8x16
    tiles), q and k scaled by 2.5 as above."""
    dims, C, B, nh = (40, 24), 64, 1, 2
    shape = (B, C, *reversed(dims))
    q, k, v, dy = (seeded(3700 + i + 5 * kind + ws, shape) for i in range(4))
    q, k = q * np.float32(2.5), k * np.float32(2.5)
    crow0, crows, ccols = CENTRAL[ws]
    assert central_gap(kind, q, k, ws, nh, tile_h=8, crows=crows, ccols=ccols, crow0=crow0) > 8.5
    y, dq, dk, dv = fused(ca, cuda, kind, q, k, v, dy, ws, nh)
    yr, _ = O.attention_fwd(kind, *(f64(a) for a in (q, k, v)), ws, nh)
    gr = O.attention_bwd(kind, *(f64(a) for a in (q, k, v, dy)), ws, nh)
    assert rel_err(y, yr) < TOL_FWD
    for name, g, r in zip(("dq", "dk", "dv"), (dq, dk, dv), gr):
        assert rel_err(g, r) < TOL_GRAD, (name, rel_err(g, r))


def central_gap_1d(kind, q, k, ws, nh, tile):
    """central_gap for one-dimensional signals: the wavefront of query r holds
    the 16 queries from r - r % 16 and its key region starts P pixels before
    them; the central pair is that region's keys 32 pc .. 32 pc + 31,
    pc = (8 + P) // 32, on tiles of `tile` pixels (256 for 16 real components
    per head, 128 for 32)."""
    (n1,) = O.spatial_dims(q)
    P = (ws - 1) // 2
    pc = (8 + P) // 32
    qf, kf = O._flat(q, nh), O._flat(k, nh)
    dh = qf.shape[1]
    S = O.similarity(kind, f64(qf), f64(kf), (n1,), ws, 1.0 / math.sqrt(dh))
    S = S.reshape(qf.shape[0], n1, ws) * (1.0 / math.log(2.0))
    _, colval = O.pattern((n1,), ws, 1)
    cols = colval.reshape(n1, -1) - 1
    best = -np.inf
    for r in range(n1):
        start = r - r % tile + 16 * ((r % tile) // 16) - P + 32 * pc
        cset = {(start + d) % n1 for d in range(32)}
        central = np.array([c in cset for c in cols[r]])
        gap = S[:, r, :].max(axis=1) - np.where(central, S[:, r, :], -np.inf).max(axis=1)
        best = max(best, float(gap.max()))
    return best


@pytest.mark.parametrize("case", [((400,), 32, 2, 256), ((300,), 32, 1, 128)],
                         ids=["16-components", "32-components"])
@pytest.mark.parametrize("kind", [0, 1])
def test_fused_forward_redo_path_1d(ca, cuda, case, kind):
    """The redo path of the one-dimensional forward at window 63 (reference
    maximum from the central pair of a wavefront's 78-key region), q and k
    scaled by 2.5 so that scores more than 8 above it occur; checked on the
    CPU first, then the GPU result against the oracle."""
    dims, C, nh, tile = case
    ws, B = 63, 1
    shape = (B, C, *reversed(dims))
    q, k, v, dy = (seeded(3800 + i + 5 * kind + dims[0], shape) for i in range(4))
    q, k = q * np.float32(2.5), k * np.float32(2.5)
    assert central_gap_1d(kind, q, k, ws, nh, tile) > 8.5
    y, dq, dk, dv = fused(ca, cuda, kind, q, k, v, dy, ws, nh)
    yr, _ = O.attention_fwd(kind, *(f64(a) for a in (q, k, v)), ws, nh)
    gr = O.attention_bwd(kind, *(f64(a) for a in (q, k, v, dy)), ws, nh)
    assert rel_err(y, yr) < TOL_FWD
    for name, g, r in zip(("dq", "dk", "dv"), (dq, dk, dv), gr):
        assert rel_err(g, r) < TOL_GRAD, (name, rel_err(g, r))
