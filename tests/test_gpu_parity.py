"""GPU parity: every libcircatt entry point against the CPU oracle on
identical seeded inputs (float32 inputs, float64 oracle).

Bar: CSR indices bit-exact; forward values within 1e-5 and gradients within
1e-4 (max-norm relative error, conftest.rel_err).  Shapes mirror the
reference's tests (test/rrule.jl:1-6: 8^S x 4 x 2, ws = 5; test/grad.jl:6-7,
46-56: 10^S x 8 x 2, ws = 3, nheads = 2), the benchmark configurations at
sizes the oracle finishes in seconds, and the degenerate ws > N patterns.
"""
import math

import numpy as np
import pytest

from conftest import TOL_FWD, TOL_GRAD, rel_err

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle as O  # noqa: E402


@pytest.fixture(scope="module")
def ca(cuda):
    import circulant_attention
    return circulant_attention


def seeded(seed, shape, cplx=False):
    """float32-representable inputs (complex: re, im ~ N(0, 1/2))."""
    rng = np.random.default_rng(seed)
    if cplx:
        a = (rng.standard_normal(shape) + 1j * rng.standard_normal(shape)) / np.sqrt(2)
        return a.astype(np.complex64).astype(np.complex128)
    return rng.standard_normal(shape).astype(np.float32).astype(np.float64)


def dev(a, cuda):
    if np.iscomplexobj(a):
        return torch.from_numpy(a.astype(np.complex64)).to(cuda)
    return torch.from_numpy(a.astype(np.float32)).to(cuda)


def host(t):
    t = t.detach().cpu()
    return t.numpy().astype(np.complex128 if t.is_complex() else np.float64)


def shape_of(dims, C, B):
    return (B, C, *reversed(dims))


# ---------------------------------------------------------------------------
# pattern (bit-exact)
# ---------------------------------------------------------------------------
PATTERN_CASES = [((8,), 5), ((8, 8), 5), ((12, 10), 3), ((32, 32), 7), ((4,), 5), ((2,), 5),
                 ((4, 4), 5), ((3, 5), 7), ((1, 6), 3), ((128, 96), 15), ((262144,), 63),
                 ((17,), 1),
                 # windows past 15 in 2D (cfg4a's ws = 31), and past the image
                 ((70, 40), 31), ((37, 9), 19), ((20, 24), 31)]


@pytest.mark.parametrize("dims,ws", PATTERN_CASES)
def test_pattern_bitexact(ca, cuda, dims, ws):
    from circulant_attention import _lib as L
    from circulant_attention._functions import ptr, stream_ptr, geometry
    nsp, n1, n2 = geometry(dims)
    P, K, nb = int(np.prod(dims)), ws ** len(dims), 2
    rowptr = torch.empty((nb, P + 1), dtype=torch.int32, device=cuda)
    colval = torch.empty((nb, P * K), dtype=torch.int32, device=cuda)
    L.check(L.lib.circatt_pattern(nsp, n1, n2, ws, nb, ptr(rowptr), ptr(colval), stream_ptr()))
    rp, cv = O.pattern(dims, ws, nb)
    assert np.array_equal(rowptr.cpu().numpy(), rp)
    assert np.array_equal(colval.cpu().numpy(), cv)


def test_pattern_bitexact_cfg4a_full_size(ca, cuda):
    """Benchmark configuration cfg4a's pattern at full size: 512x512, ws = 31 (961 slots per
    row, 251,920,384 entries), rowPtr and colVal bit-exact."""
    from circulant_attention import _lib as L
    from circulant_attention._functions import ptr, stream_ptr
    P, K = 512 * 512, 31 * 31
    rowptr = torch.empty((1, P + 1), dtype=torch.int32, device=cuda)
    colval = torch.empty((1, P * K), dtype=torch.int32, device=cuda)
    L.check(L.lib.circatt_pattern(2, 512, 512, 31, 1, ptr(rowptr), ptr(colval), stream_ptr()))
    rp, cv = O.pattern((512, 512), 31, 1)
    assert np.array_equal(rowptr.cpu().numpy(), rp)
    assert np.array_equal(colval.cpu().numpy(), cv)


def test_readme_quickstart_shape(ca, cuda):
    """README.md:55-71: A has size (12288, 12288, 1, 2) and 5529600 entries."""
    q = dev(seeded(1002, shape_of((128, 96), 64, 2)), cuda)
    S = ca.circulant_similarity(ca.DotSimilarity(), q, q, 15)
    assert S.size() == (12288, 12288, 1, 2)
    assert S.data.nnz == 5_529_600
    rp, cv = O.pattern((128, 96), 15, 1)
    assert np.array_equal(S.data.colVal[0, 0].cpu().numpy(), cv[0])
    assert np.array_equal(S.data.rowPtr[1, 0].cpu().numpy(), rp[0])


# ---------------------------------------------------------------------------
# similarity / softmax / apply / sums
# ---------------------------------------------------------------------------
SIM_CASES = [((8,), 5, 4), ((8, 8), 5, 4), ((12, 10), 3, 8), ((32, 32), 7, 16), ((4, 4), 5, 4),
             ((2,), 5, 3), ((20, 13), 15, 64), ((9, 7), 3, 80), ((70,), 63, 32),
             # windows past 15 (sub-row kernel), with and without interior segments
             ((70, 40), 31, 8), ((160, 6), 17, 4), ((700,), 63, 4), ((37, 9), 19, 3),
             ((10, 40), 17, 3), ((40,), 63, 2),
             # odd channel counts (the row kernel stages real channels in pairs)
             ((12, 10), 5, 7), ((200, 4), 9, 3)]


@pytest.mark.parametrize("dims,ws,C", SIM_CASES)
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [0, 1])
def test_similarity(ca, cuda, dims, ws, C, cplx, kind):
    B = 2
    x = seeded(11, shape_of(dims, C, B), cplx)
    y = seeded(12, shape_of(dims, C, B), cplx)
    simfun = ca.DotSimilarity() if kind == 0 else ca.DistanceSimilarity()
    S = ca.circulant_similarity(simfun, dev(x, cuda), dev(y, cuda), ws)
    P = int(np.prod(dims))
    ref = O.similarity(kind, x.reshape(B, C, P), y.reshape(B, C, P), dims, ws)
    assert S.size() == (P, P, 1, B)
    assert rel_err(host(S.nzval).reshape(B, -1), ref) < TOL_FWD


@pytest.mark.parametrize("dims", [(96, 256), (200, 96)])
@pytest.mark.parametrize("ws", [7, 11])
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [0, 1])
def test_similarity_many_rows(ca, cuda, dims, ws, cplx, kind):
    """The row-blocked similarity kernel on many 64-pixel row segments, 4
    units, against the oracle.  Neither width is a multiple of 64, so partial
    segments and the border body run; rows of 200 pixels also have interior
    segments."""
    C, B = 6, 4
    x = seeded(13, shape_of(dims, C, B), cplx)
    y = seeded(14, shape_of(dims, C, B), cplx)
    simfun = ca.DotSimilarity() if kind == 0 else ca.DistanceSimilarity()
    S = ca.circulant_similarity(simfun, dev(x, cuda), dev(y, cuda), ws)
    P = int(np.prod(dims))
    ref = O.similarity(kind, x.reshape(B, C, P), y.reshape(B, C, P), dims, ws)
    assert rel_err(host(S.nzval).reshape(B, -1), ref) < TOL_FWD


@pytest.mark.parametrize("K,rows", [(1, 10), (9, 1000), (225, 3000), (961, 70), (3969, 5)])
def test_softmax_and_pullback(ca, cuda, K, rows):
    from circulant_attention._functions import SoftmaxFn
    a = seeded(21, (rows, K)) * 4
    t = dev(a, cuda).requires_grad_(True)
    out = SoftmaxFn.apply(t)
    assert rel_err(host(out), O.softmax(a, K)) < TOL_FWD
    g = seeded(22, (rows, K))
    out.backward(dev(g, cuda))
    ref = O.softmax_bwd(O.softmax(a, K), g, K)
    assert rel_err(host(t.grad), ref) < TOL_GRAD


APPLY_CASES = [((8,), 5, 4), ((8, 8), 5, 4), ((12, 10), 3, 8), ((4, 4), 5, 3), ((2,), 5, 2),
               ((33, 17), 11, 16),
               # 2D rows with interior 64-pixel segments (and a partial last one);
               # 203 is odd, so its border segments stage x float by float
               ((200, 12), 11, 16), ((256, 6), 15, 8), ((203, 5), 7, 4),
               # windows past 15 (sub-rows of 16 window columns), 2D and 1D,
               # with and without interior segments
               ((70, 40), 31, 8), ((400, 3), 17, 4), ((300,), 63, 8), ((1000,), 63, 4),
               ((37, 9), 19, 3),
               # window wider than the image along dim 1 (columns wrap more than once)
               ((10, 40), 17, 3), ((40,), 63, 2),
               # 2D windows 17 .. 31 (workgroup kernel over 4 image rows): interior
               # segments, a partial last segment and a partial last row group
               ((300, 22), 31, 8), ((150, 10), 21, 5),
               # 2D windows 13 and 15 on small grids (the same kernel with the deep
               # schedule and 16-component passes): interior and border segments,
               # odd channel counts, rows fewer than the window
               ((300, 14), 15, 8), ((130, 9), 13, 5), ((70, 6), 15, 20)]


@pytest.mark.parametrize("dims,ws,C", APPLY_CASES)
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("trans", [False, True])
def test_apply(ca, cuda, dims, ws, C, cplx, trans):
    B, P, K = 2, int(np.prod(dims)), ws ** len(dims)
    nz = seeded(31, (B, 1, P, K))
    x = seeded(32, shape_of(dims, C, B), cplx)
    A = ca.Circulant(dev(nz, cuda), ws, dims)
    f = ca.circulant_transposed_attention if trans else ca.otimes
    y = f(A, dev(x, cuda))
    ref = O.apply(nz.reshape(B, -1), x.reshape(B, C, P), dims, ws, trans=trans)
    assert rel_err(host(y).reshape(B, C, P), ref) < TOL_FWD
    rs, cs = O.rowsum(nz.reshape(B, -1), P, K), O.colsum(nz.reshape(B, -1), dims, ws)
    assert rel_err(host(A.sum(2)).reshape(B, P), rs) < TOL_FWD
    assert rel_err(host(A.sum(1)).reshape(B, P), cs) < TOL_FWD


SIM_BWD_CASES = [((20, 13), 15, 8), ((70, 40), 31, 8), ((300, 22), 31, 8), ((150, 10), 21, 5),
                 ((400, 3), 17, 4), ((10, 40), 17, 3), ((300,), 63, 4), ((300, 14), 15, 8),
                 ((130, 9), 13, 5), ((40, 30), 11, 8)]


@pytest.mark.parametrize("dims,ws,C", SIM_BWD_CASES)
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [0, 1])
def test_similarity_bwd(ca, cuda, dims, ws, C, cplx, kind):
    """circatt_similarity_bwd (both products in one grid) against the
    oracle's composition of the similarity rrules (src/rrules.jl:1-32):
    dx = s (dS ⊠ y - [Distance] rowsum(dS) .* x), dy = s (dSᵀ ⊠ x -
    [Distance] colsum(dS) .* y)."""
    from circulant_attention import _lib as L
    from circulant_attention._functions import ptr, stream_ptr, geometry
    B, P, K = 2, int(np.prod(dims)), ws ** len(dims)
    nsp, n1, n2 = geometry(dims)
    dS = seeded(41, (B, P, K))
    x = seeded(42, shape_of(dims, C, B), cplx)
    y = seeded(43, shape_of(dims, C, B), cplx)
    scale = 0.37
    tx, ty, tS = dev(x, cuda), dev(y, cuda), dev(dS, cuda)
    dx, dy = torch.empty_like(tx), torch.empty_like(ty)
    L.check(L.lib.circatt_similarity_bwd(kind, L.C32 if cplx else L.F32, nsp, n1, n2, ws, C, B,
                                         scale, ptr(tS), ptr(tx), ptr(ty), ptr(dx), ptr(dy),
                                         stream_ptr()))
    torch.cuda.synchronize()
    nzf, xf, yf = dS.reshape(B, -1), x.reshape(B, C, P), y.reshape(B, C, P)
    rdx = O.apply(nzf, yf, dims, ws, trans=False)
    rdy = O.apply(nzf, xf, dims, ws, trans=True)
    if kind == 1:
        rdx = rdx - O.rowsum(nzf, P, K)[:, None, :] * xf
        rdy = rdy - O.colsum(nzf, dims, ws)[:, None, :] * yf
    assert rel_err(host(dx).reshape(B, C, P), scale * rdx) < TOL_FWD
    assert rel_err(host(dy).reshape(B, C, P), scale * rdy) < TOL_FWD


# ---------------------------------------------------------------------------
# attention: unfused (returns A) and fused (no A), forward and backward
# ---------------------------------------------------------------------------
ATT_CASES = [
    # (dims, ws, C, B, nheads, seed)
    ((8,), 5, 4, 2, 1, 100),      # test/rrule.jl shapes
    ((8, 8), 5, 4, 2, 1, 101),
    ((10,), 3, 8, 2, 2, 102),     # test/grad.jl shapes
    ((10, 10), 3, 8, 2, 2, 103),
    ((32, 32), 7, 16, 1, 1, 1001),  # benchmark configuration cfg1
    ((12, 10), 3, 4, 2, 1, 104),  # non-square
    ((4, 4), 5, 4, 2, 1, 105),    # ws > N
    ((4,), 5, 4, 2, 1, 106),
    ((40, 24), 15, 64, 1, 4, 1003),  # cfg3 geometry, reduced size
    ((36, 30), 11, 32, 2, 2, 1005),  # cfg5 geometry, reduced size
    ((70, 40), 31, 32, 1, 1, 1004),  # cfg4a geometry, reduced size
    ((300,), 63, 32, 2, 1, 1014),    # cfg4b geometry, reduced size
    # compile-time-window 2D kernels (16 or 32 real components per head):
    # partial tiles, halos that wrap more than once, ws > N
    ((9, 7), 5, 16, 2, 1, 107),
    ((5, 13), 3, 32, 1, 2, 108),
    ((20, 11), 15, 16, 1, 1, 109),
    ((8, 8), 15, 32, 1, 2, 110),
    ((17, 26), 11, 64, 1, 4, 111),
    ((24, 16), 7, 32, 2, 1, 112),
    # 32 real components per head (real C / nheads = 32, complex C / nheads = 16) on the
    # split-half 8x16 tiles: partial tiles, halos that wrap more than once, ws > N
    ((9, 7), 5, 32, 2, 1, 113),
    ((5, 13), 11, 64, 1, 2, 114),
    ((13, 21), 11, 16, 1, 1, 115),
    ((30, 17), 3, 32, 1, 1, 116),
    # one-dimensional split-half kernels (ws 15 and 63; 16 or 32 real
    # components per head): partial tiles, signals shorter than a tile,
    # windows that wrap more than once
    ((200,), 15, 16, 2, 1, 117),
    ((50,), 63, 16, 1, 1, 118),
    ((1000,), 15, 32, 1, 2, 119),
    ((37,), 15, 32, 2, 1, 120),
    ((700,), 63, 64, 1, 2, 121),
    # (real signals whose length is a multiple of 4 take the row-DMA loads:
    # ws 63 with 16 components, ws 15 with 32, a signal shorter than the halo)
    ((400,), 63, 16, 1, 1, 122),
    ((104,), 15, 32, 1, 1, 123),
    ((24,), 63, 16, 2, 1, 124),
]


def _attention_case(ca, cuda, dims, ws, C, B, nheads, seed, cplx, kind, materialize):
    shape = shape_of(dims, C, B)
    q, k, v, dy = (seeded(seed + i, shape, cplx) for i in range(4))
    tq, tk, tv = (dev(a, cuda).requires_grad_(True) for a in (q, k, v))
    simfun = ca.DotSimilarity() if kind == 0 else ca.DistanceSimilarity()
    if nheads == 1:
        y, A = ca.circulant_attention(simfun, tq, tk, tv, ws, materialize=materialize)
    else:
        y, A = ca.circulant_mh_attention(simfun, tq, tk, tv, ws, nheads,
                                         materialize=materialize, honor_simfun=True)
    yr, Ar = O.attention_fwd(kind, q, k, v, ws, nheads)
    assert rel_err(host(y), yr) < TOL_FWD
    if materialize:
        P = int(np.prod(dims))
        assert A.size() == ((P, P, 1, B) if nheads == 1 else (P, P, nheads, B))
        assert rel_err(host(A.nzval).reshape(Ar.shape), Ar) < TOL_FWD
    else:
        assert A is None
    td = dev(dy, cuda)
    loss = (y * td.conj()).real.sum() if y.is_complex() else (y * td).sum()
    loss.backward()
    gq, gk, gv = O.attention_bwd(kind, q, k, v, dy, ws, nheads)
    assert rel_err(host(tq.grad), gq) < TOL_GRAD
    assert rel_err(host(tk.grad), gk) < TOL_GRAD
    assert rel_err(host(tv.grad), gv) < TOL_GRAD


@pytest.mark.parametrize("case", ATT_CASES, ids=lambda c: f"{c[0]}-ws{c[1]}-C{c[2]}-h{c[4]}")
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [0, 1])
def test_attention_unfused(ca, cuda, case, cplx, kind):
    _attention_case(ca, cuda, *case, cplx, kind, materialize=True)


@pytest.mark.parametrize("case", ATT_CASES, ids=lambda c: f"{c[0]}-ws{c[1]}-C{c[2]}-h{c[4]}")
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [0, 1])
def test_attention_fused(ca, cuda, case, cplx, kind):
    _attention_case(ca, cuda, *case, cplx, kind, materialize=False)


@pytest.mark.parametrize("case", [ATT_CASES[0], ATT_CASES[3], ATT_CASES[5], ATT_CASES[9]],
                         ids=lambda c: f"{c[0]}-ws{c[1]}-C{c[2]}-h{c[4]}")
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [0, 1])
def test_attention_grad_through_A(ca, cuda, case, cplx, kind):
    """circulant_attention / circulant_mh_attention return (y, A)
    (src/attention.jl:19-25, 38-42); a loss on both, Re<y, dy> + <A_nz, G>,
    differentiates through A's softmax and similarity as well."""
    dims, ws, C, B, nheads, seed = case
    shape = shape_of(dims, C, B)
    q, k, v, dy = (seeded(seed + 50 + i, shape, cplx) for i in range(4))
    tq, tk, tv = (dev(a, cuda).requires_grad_(True) for a in (q, k, v))
    simfun = ca.DotSimilarity() if kind == 0 else ca.DistanceSimilarity()
    if nheads == 1:
        y, A = ca.circulant_attention(simfun, tq, tk, tv, ws)
    else:
        y, A = ca.circulant_mh_attention(simfun, tq, tk, tv, ws, nheads, honor_simfun=True)
    G = seeded(seed + 60, tuple(A.nzval.shape))
    td = dev(dy, cuda)
    ly = (y * td.conj()).real.sum() if y.is_complex() else (y * td).sum()
    (ly + (A.nzval * dev(G, cuda)).sum()).backward()
    gq, gk, gv = O.attention_bwd(kind, q, k, v, dy, ws, nheads, dA_out=G.reshape(B * nheads, -1))
    assert rel_err(host(tq.grad), gq) < TOL_GRAD
    assert rel_err(host(tk.grad), gk) < TOL_GRAD
    assert rel_err(host(tv.grad), gv) < TOL_GRAD


# the 2D compile-time-window cases again, with the Float32 matrix-core kernels
# (the default above is the split-half arithmetic)
F32_CASES = [c for c in ATT_CASES if len(c[0]) == 2 and c[1] in (3, 5, 7, 11, 15)
             and (c[2] // c[4]) in (16, 32)]


@pytest.fixture
def f32_math(ca):
    from circulant_attention import _lib as L
    old = L.lib.circatt_get_math()
    L.check(L.lib.circatt_set_math(L.MATH_F32))
    yield
    L.check(L.lib.circatt_set_math(old))


@pytest.mark.parametrize("case", F32_CASES, ids=lambda c: f"{c[0]}-ws{c[1]}-C{c[2]}-h{c[4]}")
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [0, 1])
def test_attention_fused_f32_math(ca, cuda, f32_math, case, cplx, kind):
    _attention_case(ca, cuda, *case, cplx, kind, materialize=False)


def test_fused_lse(ca, cuda):
    from circulant_attention import _lib as L
    from circulant_attention._functions import ptr, stream_ptr
    dims, ws, C, B, nh = (24, 20), 15, 32, 2, 2
    for kind in (0, 1):
        q, k, v = (seeded(200 + i, shape_of(dims, C, B)) for i in range(3))
        tq, tk, tv = (dev(a, cuda) for a in (q, k, v))
        y = torch.empty_like(tq)
        lse = torch.empty((B * nh, 480), dtype=torch.float32, device=cuda)
        L.check(L.lib.circatt_fused_fwd(kind, 0, 2, 24, 20, ws, C, nh, B, ptr(tq), ptr(tk),
                                        ptr(tv), ptr(y), ptr(lse), stream_ptr()))
        ref = O.attention_lse(kind, q, k, ws, nh)
        assert np.max(np.abs(host(lse) - ref)) < 1e-5 * np.max(np.abs(ref)) + 1e-5


def test_fused_step_graph_replay(ca, cuda):
    """The fused step's three entry points captured as one HIP graph (the way
    bench.py times the step): every replay, with eager work and a
    synchronisation between replays, reproduces the eager outputs bit for bit."""
    import ctypes

    from circulant_attention import _lib as L
    from circulant_attention._functions import ptr
    dims, ws, C, B, nh = (40, 24), 15, 64, 1, 4  # split-half kernels
    n1, n2 = dims
    g = torch.Generator(device=cuda)
    g.manual_seed(7)
    q, k, v, dy = (torch.randn(shape_of(dims, C, B), device=cuda, generator=g) for _ in range(4))
    wbytes = L.lib.circatt_fused_bwd_workspace_bytes(2, n1, n2, nh, B)
    work = torch.empty((wbytes // 4,), device=cuda)

    def buffers():
        return [torch.empty_like(q) for _ in range(4)] + [
            torch.empty((B * nh, n1 * n2), device=cuda)]

    def step(bufs, s):
        y, dq, dk, dv, lse = bufs
        L.check(L.lib.circatt_fused_fwd(0, L.F32, 2, n1, n2, ws, C, nh, B, ptr(q), ptr(k), ptr(v),
                                        ptr(y), ptr(lse), s))
        L.check(L.lib.circatt_fused_bwd_dq(0, L.F32, 2, n1, n2, ws, C, nh, B, ptr(q), ptr(k),
                                           ptr(v), ptr(y), ptr(dy), ptr(lse), ptr(dq), ptr(work),
                                           wbytes, s))
        L.check(L.lib.circatt_fused_bwd_dkdv(0, L.F32, 2, n1, n2, ws, C, nh, B, ptr(q), ptr(k),
                                             ptr(v), ptr(dy), ptr(lse), ptr(dk), ptr(dv),
                                             ptr(work), wbytes, s))

    ref = buffers()
    step(ref, ctypes.c_void_p(torch.cuda.current_stream(cuda).cuda_stream))
    torch.cuda.synchronize()
    out = buffers()
    cs = torch.cuda.Stream(cuda)
    graph = torch.cuda.CUDAGraph()
    cs.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.graph(graph, stream=cs):
        step(out, ctypes.c_void_p(cs.cuda_stream))
    torch.cuda.synchronize()
    for r in range(3):
        for t in out:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("y", "dq", "dk", "dv", "lse"), out, ref):
            assert torch.equal(a, b), (r, name)


def test_mh_attention_ignores_simfun(ca, cuda):
    """src/attention.jl:40 drops simfun: multi-head attention is always Dot."""
    dims, ws, C, B, nh = (10, 10), 3, 8, 2, 2
    q, k, v = (dev(seeded(300 + i, shape_of(dims, C, B)), cuda) for i in range(3))
    y1, _ = ca.circulant_mh_attention(ca.DistanceSimilarity(), q, k, v, ws, nh)
    y2, _ = ca.circulant_mh_attention(ca.DotSimilarity(), q, k, v, ws, nh)
    assert torch.equal(y1, y2)
    yr, _ = O.attention_fwd(0, *(host(t) for t in (q, k, v)), ws, nh)
    assert rel_err(host(y1), yr) < TOL_FWD


def test_composition_cfg5_style(ca, cuda):
    """README.md:128-134 / benchmark configuration cfg5 (reduced): C = A + m*B, w = C ⨷ u."""
    dims, ws, Cc, Bb, nh = (20, 16), 11, 32, 2, 2
    shape = shape_of(dims, Cc, Bb)
    q, k, v = (seeded(400 + i, shape, True) for i in range(3))
    tq, tk, tv = (dev(a, cuda) for a in (q, k, v))
    y, A = ca.circulant_mh_attention(ca.DotSimilarity(), tq, tk, tv, ws, nh)
    u, Bm = ca.circulant_mh_attention(ca.DotSimilarity(), y, y, y, ws, nh)
    m = seeded(403, (Bb, nh, 1, 1))  # Julia size (1, 1, nheads, B)
    Cm = A + ca.scale(dev(m, cuda), Bm)
    w = ca.Otimes(Cm, u)
    yr, Ar = O.attention_fwd(0, q, k, v, ws, nh)
    ur, Br = O.attention_fwd(0, host(y), host(y), host(y), ws, nh)
    Cr = O.axpby(np.ones(Bb * nh), Ar, m.reshape(-1), Br)
    P = int(np.prod(dims))
    wr = O.apply(Cr, host(u).reshape(Bb * nh, Cc // nh, P), dims, ws).reshape(shape)
    assert rel_err(host(Cm.nzval).reshape(Cr.shape), Cr) < TOL_FWD
    assert rel_err(host(w), wr) < TOL_FWD
    # sums over batch dims (src/array.jl:132-154)
    s3 = Cm.sum(3)
    assert s3.size() == (P, P, 1, Bb)
    ref3 = Cr.reshape(Bb, nh, -1).sum(axis=1)
    assert rel_err(host(s3.nzval).reshape(Bb, -1), ref3) < TOL_FWD


def test_cat_heads_then_otimes(ca, cuda):
    """README.md:145-148: D = cat(A, B; dims=3) has 2·nheads heads; D ⨷ w
    splits w into 2·nheads heads and applies head g's matrix to it."""
    dims, ws, Cc, Bb, nh = (12, 10), 5, 16, 2, 2
    shape = shape_of(dims, Cc, Bb)
    q, k, v, w = (seeded(700 + i, shape) for i in range(4))
    tq, tk, tv = (dev(a, cuda) for a in (q, k, v))
    _, A = ca.circulant_mh_attention(ca.DotSimilarity(), tq, tk, tv, ws, nh)
    _, Bm = ca.circulant_mh_attention(ca.DotSimilarity(), tv, tq, tk, ws, nh)
    D = ca.cat(A, Bm, dims=3)
    P = int(np.prod(dims))
    assert D.size() == (P, P, 2 * nh, Bb)
    assert D == ca.cat(A, Bm, dims=3) and not (D == ca.cat(Bm, A, dims=3))
    z = ca.Otimes(D, dev(w, cuda))
    _, Ar = O.attention_fwd(0, q, k, v, ws, nh)
    _, Br = O.attention_fwd(0, v, q, k, ws, nh)
    K = ws ** len(dims)
    Dr = np.concatenate([Ar.reshape(Bb, nh, P * K), Br.reshape(Bb, nh, P * K)], axis=1)
    zr = O.apply(Dr.reshape(Bb * 2 * nh, P * K), w.reshape(Bb * 2 * nh, Cc // (2 * nh), P),
                 dims, ws).reshape(shape)
    assert rel_err(host(z), zr) < TOL_FWD


def test_cat_carries_gradients(ca, cuda):
    """cat(A, B; dims=3) ⨷ w equals A ⨷ (first half of w's channels) next to
    B ⨷ (second half), and gradients reach q, k, v and w through cat as they
    do through the two separate products."""
    dims, ws, Cc, Bb, nh = (12, 10), 5, 16, 2, 2
    shape = shape_of(dims, Cc, Bb)
    q, k, v, w, g = (seeded(720 + i, shape) for i in range(5))
    tq, tk, tv, tw = (dev(a, cuda).requires_grad_(True) for a in (q, k, v, w))
    _, A = ca.circulant_mh_attention(ca.DotSimilarity(), tq, tk, tv, ws, nh)
    _, Bm = ca.circulant_mh_attention(ca.DotSimilarity(), tv, tq, tk, ws, nh)
    z = ca.Otimes(ca.cat(A, Bm, dims=3), tw)
    z2 = torch.cat([ca.Otimes(A, tw[:, :Cc // 2]), ca.Otimes(Bm, tw[:, Cc // 2:])], dim=1)
    assert rel_err(host(z), host(z2)) < 1e-6
    tg = dev(g, cuda)
    grads = []
    for out in (z, z2):
        for t in (tq, tk, tv, tw):
            t.grad = None
        (out * tg).sum().backward(retain_graph=True)
        grads.append([host(t.grad) for t in (tq, tk, tv, tw)])
    for a, b in zip(*grads):
        assert np.abs(a).max() > 0
        assert rel_err(a, b) < 1e-6


def test_scale_rrule(ca, cuda):
    """test/rrule.jl:22 scale(a, A) with a (1,1,2,2) against A (P,P,1,2):
    broadcast over the batch dims; gradients by the rrule of src/rrules.jl:94-114."""
    dims, ws, P, K = (8, 8), 5, 64, 25
    nz = seeded(500, (2, 1, P, K))
    a = seeded(501, (2, 2, 1, 1))
    gout = seeded(502, (2, 2, P, K))
    tA = dev(nz, cuda).requires_grad_(True)
    ta = dev(a, cuda).requires_grad_(True)
    Z = ca.scale(ta, ca.Circulant(tA, ws, dims))
    assert Z.size() == (P, P, 2, 2)
    ref = a.reshape(2, 2, 1, 1) * nz
    assert rel_err(host(Z.nzval), ref) < TOL_FWD
    (Z.nzval * dev(gout, cuda)).sum().backward()
    assert rel_err(host(ta.grad), (gout * nz).sum(axis=(2, 3), keepdims=True)) < TOL_GRAD
    assert rel_err(host(tA.grad), (gout * a).sum(axis=1, keepdims=True)) < TOL_GRAD


def test_adjacency_apply_chain_matches_oracle(ca, cuda):
    """test/grad.jl:88-97: A = circulant_adjacency(simfun, x, y, ws); z = A ⊗ x."""
    dims, ws, C, B = (12, 12), 3, 8, 2
    for kind in (0, 1):
        x, y, g = (seeded(600 + i, shape_of(dims, C, B)) for i in range(3))
        tx, ty = (dev(a, cuda).requires_grad_(True) for a in (x, y))
        simfun = ca.DotSimilarity() if kind == 0 else ca.DistanceSimilarity()
        A = ca.circulant_adjacency(simfun, tx, ty, ws)
        z = ca.otimes(A, tx)
        (z * dev(g, cuda)).sum().backward()
        P = int(np.prod(dims))
        xf, yf, gf = (a.reshape(B, C, P) for a in (x, y, g))
        Sr = O.similarity(kind, xf, yf, dims, ws)
        Ar = O.softmax(Sr, ws * ws)
        zr = O.apply(Ar, xf, dims, ws)
        assert rel_err(host(z).reshape(B, C, P), zr) < TOL_FWD
        # reference composition of rrules (rrules.jl:58-72, 42-56, 1-32)
        dA = O.similarity(0, gf, xf, dims, ws)
        dx_apply = O.apply(Ar, gf, dims, ws, trans=True)
        dS = O.softmax_bwd(Ar, dA, ws * ws)
        dx_sim = O.apply(dS, yf, dims, ws)
        dy_sim = O.apply(dS, xf, dims, ws, trans=True)
        if kind == 1:
            dx_sim = dx_sim - O.rowsum(dS, P, ws * ws)[:, None] * xf
            dy_sim = dy_sim - O.colsum(dS, dims, ws)[:, None] * yf
        assert rel_err(host(tx.grad).reshape(B, C, P), dx_apply + dx_sim) < TOL_GRAD
        assert rel_err(host(ty.grad).reshape(B, C, P), dy_sim) < TOL_GRAD


# ---------------------------------------------------------------------------
# full-size configurations: size-independent properties
# ---------------------------------------------------------------------------

def test_cfg2_unfused_full_size(ca, cuda):
    """Benchmark configuration cfg2 (README quickstart): unfused forward returning A at full
    size, y and A against the oracle; CSR indices bit-exact."""
    dims, ws, C, B = (128, 96), 15, 64, 2
    q, k, v = (seeded(1002 + 10 * i, shape_of(dims, C, B)) for i in range(3))
    y, A = ca.circulant_attention(ca.DotSimilarity(), *(dev(a, cuda) for a in (q, k, v)), ws)
    yr, Ar = O.attention_fwd(0, q, k, v, ws)
    assert rel_err(host(y), yr) < TOL_FWD
    assert rel_err(host(A.nzval).reshape(Ar.shape), Ar) < TOL_FWD
    rp, cv = O.pattern(dims, ws, 1)
    assert np.array_equal(A.data.colVal[1, 0].cpu().numpy(), cv[0])


def test_cfg3_fused_matches_unfused_full_size(ca, cuda):
    """Benchmark configuration cfg3 at full size (256x256x64x4, 4 heads, ws=15): the fused
    kernels agree with the unfused composition (itself checked against the
    oracle above) for y and all gradients; rows of A sum to one."""
    dims, ws, C, B, nh = (256, 256), 15, 64, 4, 4
    g = torch.Generator(device=cuda)
    g.manual_seed(1003)
    q, k, v, dy = (torch.randn(shape_of(dims, C, B), device=cuda, generator=g) for _ in range(4))
    grads = []
    outs = []
    for materialize in (True, False):
        tq, tk, tv = (t.clone().requires_grad_(True) for t in (q, k, v))
        y, A = ca.circulant_mh_attention(ca.DotSimilarity(), tq, tk, tv, ws, nh,
                                         materialize=materialize)
        (y * dy).sum().backward()
        outs.append(y.detach())
        grads.append((tq.grad, tk.grad, tv.grad))
        if materialize:
            rs = A.sum(2)
            assert torch.max(torch.abs(rs - 1)).item() < 1e-5
        del A, y
    assert rel_err(host(outs[1]), host(outs[0])) < TOL_FWD
    for a, b in zip(grads[1], grads[0]):
        assert rel_err(host(a), host(b)) < TOL_GRAD
