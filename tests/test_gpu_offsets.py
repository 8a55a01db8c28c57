"""GPU parity on inputs that are not centred: q, k = N(0,1) + c.

Distance similarity is translation-invariant: the reference forms
-|x - y|^2 / 2 from the differences (src/similarity.jl:55-78), so adding c to
every component of q and k changes nothing, and its own Float32 result stays
near 6e-7 at any offset.  The fused kernels form the same score by expansion,
q.k - |k|^2 / 2 - |q|^2 / 2, whose Float32 terms grow with c^2 unless both
sides are first centred on a common point (the kernels take k at each tile's
first pixel).  These tests hold Distance to the usual bar (1e-5 forward, 1e-4
gradients) at c = 3, 10, 30 on every fused kernel family, 1D and 2D, real and
complex, 16, 32 and more real components per head, with the split-half and the
Float32 matrix-core arithmetic; and the unfused similarity and attention too.

Dot similarity is not translation-invariant: the offset raises the scores to
dh c^2 / sqrt(dh) (3600 at c = 30, dh = 16), where a Float32 softmax is
ill-conditioned whatever the arithmetic.  Dot is held to the large-score bar
of tests/large_scores.py there (8x a Float32 flash-style restatement, never
below the usual tolerance).
"""
import numpy as np
import pytest

from conftest import TOL_FWD, TOL_GRAD, rel_err
from large_scores import abs_err, flash_bounds

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle as O  # noqa: E402

OFFSETS = [3.0, 10.0, 30.0]


@pytest.fixture(scope="module")
def ca(cuda):
    import circulant_attention
    return circulant_attention


def offset_inputs(seed, shape, cplx, c):
    """q, k = N(0,1) + c (complex: N(0,1/2) + c(1 + i)); v, dy = N(0,1);
    float32-representable, returned as float64/complex128 copies."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(4):
        if cplx:
            a = (rng.standard_normal(shape) + 1j * rng.standard_normal(shape)) / np.sqrt(2)
            if i < 2:
                a = a + c * (1 + 1j)
            out.append(a.astype(np.complex64).astype(np.complex128))
        else:
            a = rng.standard_normal(shape) + (c if i < 2 else 0.0)
            out.append(a.astype(np.float32).astype(np.float64))
    return out


def dev(a, cuda):
    if np.iscomplexobj(a):
        return torch.from_numpy(a.astype(np.complex64)).to(cuda)
    return torch.from_numpy(a.astype(np.float32)).to(cuda)


def host(t):
    t = t.detach().cpu()
    return t.numpy().astype(np.complex128 if t.is_complex() else np.float64)


def run(ca, cuda, kind, q, k, v, dy, ws, nh, materialize):
    tq, tk, tv = (dev(a, cuda).requires_grad_(True) for a in (q, k, v))
    simfun = ca.DotSimilarity() if kind == 0 else ca.DistanceSimilarity()
    if nh == 1:
        y, A = ca.circulant_attention(simfun, tq, tk, tv, ws, materialize=materialize)
    else:
        y, A = ca.circulant_mh_attention(simfun, tq, tk, tv, ws, nh, materialize=materialize,
                                         honor_simfun=True)
    td = dev(dy, cuda)
    loss = (y * td.conj()).real.sum() if y.is_complex() else (y * td).sum()
    loss.backward()
    return host(y), host(tq.grad), host(tk.grad), host(tv.grad)


def check(kind, outs, q, k, v, dy, ws, nh):
    yr, _ = O.attention_fwd(kind, q, k, v, ws, nh)
    gr = O.attention_bwd(kind, q, k, v, dy, ws, nh)
    refs = [yr, *gr]
    names = ("y", "dq", "dk", "dv")
    if kind == 1:
        errs = [rel_err(o, r) for o, r in zip(outs, refs)]
        assert errs[0] < TOL_FWD and max(errs[1:]) < TOL_GRAD, dict(zip(names, errs))
    else:
        q32, k32, v32, dy32 = (a.astype(np.complex64 if np.iscomplexobj(a) else np.float32)
                               for a in (q, k, v, dy))
        bars = flash_bounds(kind, q32, k32, v32, dy32, ws, nh, refs)
        ratios = {n: abs_err(o, r) / b for n, o, r, b in zip(names, outs, refs, bars)}
        assert max(ratios.values()) <= 1.0, ratios


# (dims, ws, C, B, nheads); C is the real component count per pixel (halved
# for complex data so that a head keeps the same real components)
FUSED = [
    # split-half kernels, 16 real components per head, every window they cover
    ((40, 24), 15, 64, 1, 4), ((20, 18), 11, 16, 2, 1), ((17, 13), 7, 32, 1, 2),
    ((12, 10), 5, 16, 2, 1), ((9, 11), 3, 16, 1, 1),
    # split-half 8x16-tile kernels, 32 real components per head
    ((20, 18), 11, 32, 1, 1), ((12, 10), 5, 64, 1, 2),
    # run-time-window kernel: 2D ws 31 and 9, padded components, 1D windows
    ((40, 36), 31, 32, 1, 1), ((24, 20), 9, 24, 1, 1), ((300,), 63, 32, 2, 1),
    ((200,), 15, 16, 1, 1), ((100,), 5, 64, 1, 1),
    # channel-chunked kernel, heads wider than 64 real components
    ((20, 18), 7, 80, 1, 1), ((100,), 9, 96, 1, 1),
]


def _ids(c):
    return f"{'x'.join(map(str, c[0]))}-ws{c[1]}-C{c[2]}-h{c[4]}"


@pytest.mark.parametrize("case", FUSED, ids=_ids)
@pytest.mark.parametrize("c", OFFSETS)
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [0, 1])
def test_fused_offset_inputs(ca, cuda, case, c, cplx, kind):
    _fused(ca, cuda, case, c, cplx, kind, 0)


F32_CASES = [cs for cs in FUSED if len(cs[0]) == 2 and cs[1] <= 15 and cs[2] // cs[4] in (16, 32)]


@pytest.fixture
def f32_math(ca):
    from circulant_attention import _lib as L
    old = L.lib.circatt_get_math()
    L.check(L.lib.circatt_set_math(L.MATH_F32))
    yield
    L.check(L.lib.circatt_set_math(old))


@pytest.mark.parametrize("case", F32_CASES, ids=_ids)
@pytest.mark.parametrize("c", OFFSETS)
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [0, 1])
def test_fused_offset_inputs_f32_math(ca, cuda, f32_math, case, c, cplx, kind):
    _fused(ca, cuda, case, c, cplx, kind, 500)


def _fused(ca, cuda, case, c, cplx, kind, seed0):
    dims, ws, C, B, nh = case
    if cplx:
        C //= 2
    shape = (B, C, *reversed(dims))
    seed = 7000 + seed0 + 13 * ws + int(c) + 3 * kind + (100 if cplx else 0)
    q, k, v, dy = offset_inputs(seed, shape, cplx, c)
    print(f"offsets: fused dims={dims} ws={ws} C={C} nh={nh} c={c} cplx={cplx} kind={kind}",
          flush=True)
    outs = run(ca, cuda, kind, q, k, v, dy, ws, nh, materialize=False)
    check(kind, outs, q, k, v, dy, ws, nh)


UNFUSED = [((20, 13), 15, 16, 2, 1), ((200,), 15, 16, 1, 1), ((100,), 5, 8, 2, 1),
           ((40, 36), 31, 8, 1, 1), ((17, 13), 7, 32, 1, 2)]


@pytest.mark.parametrize("case", UNFUSED, ids=_ids)
@pytest.mark.parametrize("c", OFFSETS)
@pytest.mark.parametrize("cplx", [False, True])
def test_unfused_distance_offset_inputs(ca, cuda, case, c, cplx):
    """The A-materialising path with Distance: the similarity (S itself, the
    returned Circulant) and the attention's y and gradients."""
    dims, ws, C, B, nh = case
    shape = (B, C, *reversed(dims))
    q, k, v, dy = offset_inputs(7500 + ws + int(c) + (50 if cplx else 0), shape, cplx, c)
    print(f"offsets: unfused dims={dims} ws={ws} C={C} nh={nh} c={c} cplx={cplx}", flush=True)
    P = int(np.prod(dims))
    S = ca.circulant_similarity(ca.DistanceSimilarity(), dev(q, cuda), dev(k, cuda), ws)
    ref = O.similarity(1, q.reshape(B, C, P), k.reshape(B, C, P), dims, ws)
    assert rel_err(host(S.nzval).reshape(B, -1), ref) < TOL_FWD
    outs = run(ca, cuda, 1, q, k, v, dy, ws, nh, materialize=True)
    check(1, outs, q, k, v, dy, ws, nh)
