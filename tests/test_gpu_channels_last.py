"""Channels-last fused attention (CIRCATT_CHANNELS_LAST OR-ed into dtype).

The kernels read and write (C, spatial..., B) tensors in place; the
arithmetic is the planar path's, element for element, so y, lse, dq, dk, dv
must equal the planar results bit for bit after the layout permutation.  The
planar path itself is pinned against the oracle in test_gpu_parity.py and
test_gpu_magnitudes.py.  Cases cover every fused kernel family: split-half
(2D, 16 real components per head on 16x16 tiles, 32 on 8x16 tiles), Float32
matrix cores (2D, 32 components at ws 15, or CIRCATT_MATH_F32), and the
run-time-window kernels (1D, 2D windows past 15, 64 components).
"""
import ctypes

import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

# (spatial fastest-first, C, nheads, B, ws, kind, complex, math)
CASES = [
    ((24, 20), 32, 2, 2, 7, 0, False, "split"),     # split-half kernels
    ((24, 20), 32, 2, 2, 15, 1, False, "split"),    # split-half, Distance, streamed forward
    ((16, 18), 16, 2, 1, 5, 0, True, "split"),      # split-half, ComplexF32
    ((24, 20), 32, 2, 2, 11, 0, False, "f32"),      # Float32 matrix cores, 16 components
    ((20, 16), 64, 2, 2, 7, 1, False, "split"),     # split-half, 32 components (8x16 tiles)
    ((20, 16), 32, 2, 1, 3, 0, True, "split"),      # split-half, ComplexF32 32 components
    ((28, 20), 32, 2, 2, 11, 1, True, "split"),     # split-half, ComplexF32 32 components, streamed forward
    ((24, 20), 32, 2, 2, 11, 1, False, "split"),    # split-half, 16 components, 4x4 blocks, streamed forward
    ((20, 12), 16, 1, 2, 3, 0, False, "split"),     # split-half, 16 components, 4x4 blocks, ws 3
    ((20, 16), 64, 2, 2, 15, 0, False, "split"),    # Float32 matrix cores, 32 components at ws 15
    ((20, 16), 64, 2, 2, 7, 1, False, "f32"),       # Float32 matrix cores, 32 components
    ((150,), 32, 1, 2, 9, 0, False, "split"),       # run-time window, 1D
    ((260,), 32, 2, 2, 15, 1, False, "split"),      # split-half, 1D, 16 components
    ((300,), 64, 2, 1, 63, 0, True, "split"),       # split-half, 1D, ComplexF32 32 components
    ((40, 36), 16, 1, 1, 19, 1, False, "split"),    # run-time window, 2D ws 19
    ((18, 14), 128, 2, 1, 5, 0, False, "split"),    # run-time window, 64 components
]


def ids(c):
    sp, C, nh, B, ws, kind, cplx, math = c
    return f"{'x'.join(map(str, sp))}-C{C}-nh{nh}-B{B}-ws{ws}-{'dist' if kind else 'dot'}-" \
           f"{'c32' if cplx else 'f32'}-{math}"


def to_cl(t):
    """(B, C, *rev_spatial) planar -> (B, *rev_spatial, C) channels-last."""
    return t.movedim(1, -1).contiguous()


def from_cl(t):
    return t.movedim(-1, 1).contiguous()


def run(L, ptr, kind, dt, spatial, C, nh, B, ws, q, k, v, dy):
    nsp = len(spatial)
    n1, n2 = spatial[0], (spatial[1] if nsp == 2 else 1)
    P = n1 * n2
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    y = torch.empty_like(q)
    lse = torch.empty((B * nh, P), device=q.device)
    L.check(L.lib.circatt_fused_fwd(kind, dt, nsp, n1, n2, ws, C, nh, B, ptr(q), ptr(k), ptr(v),
                                    ptr(y), ptr(lse), s))
    wb = L.lib.circatt_fused_bwd_workspace_bytes(nsp, n1, n2, nh, B)
    work = torch.empty((wb // 4,), device=q.device)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    L.check(L.lib.circatt_fused_bwd(kind, dt, nsp, n1, n2, ws, C, nh, B, ptr(q), ptr(k), ptr(v),
                                    ptr(y), ptr(dy), ptr(lse), ptr(dq), ptr(dk), ptr(dv),
                                    ptr(work), wb, s))
    torch.cuda.synchronize()
    return y, lse, dq, dk, dv


@pytest.mark.parametrize("case", CASES, ids=ids)
def test_channels_last_matches_planar_bitwise(cuda, case):
    from circulant_attention import _lib as L
    from circulant_attention._functions import ptr

    spatial, C, nh, B, ws, kind, cplx, math = case
    L.check(L.lib.circatt_set_math(L.MATH_F32 if math == "f32" else L.MATH_SPLIT_F16))
    try:
        g = torch.Generator(device=cuda)
        g.manual_seed(11 + ws)
        dtype = torch.complex64 if cplx else torch.float32
        shape = (B, C, *reversed(spatial))
        q, k, v, dy = (torch.randn(shape, device=cuda, dtype=dtype, generator=g) for _ in range(4))
        dt = L.C32 if cplx else L.F32
        planar = run(L, ptr, kind, dt, spatial, C, nh, B, ws, q, k, v, dy)
        cl = run(L, ptr, kind, dt | L.CHANNELS_LAST, spatial, C, nh, B, ws,
                 to_cl(q), to_cl(k), to_cl(v), to_cl(dy))
        for name, a, b in zip(("y", "lse", "dq", "dk", "dv"), planar, cl):
            b = b if name == "lse" else from_cl(b)
            assert torch.equal(a, b), (name, (a - b).abs().max().item())
    finally:
        L.check(L.lib.circatt_set_math(L.MATH_SPLIT_F16))


def test_channels_last_autograd_matches_planar(cuda):
    """circulant_mh_attention(..., materialize=False, channels_last=True)
    against the planar call, values and gradients."""
    import circulant_attention as ca

    g = torch.Generator(device=cuda)
    g.manual_seed(5)
    B, C, n2, n1, nh, ws = 2, 32, 20, 24, 2, 7
    q, k, v = (torch.randn((B, C, n2, n1), device=cuda, generator=g) for _ in range(3))
    w = torch.randn((B, C, n2, n1), device=cuda, generator=g)
    qp, kp, vp = (t.clone().requires_grad_(True) for t in (q, k, v))
    y, A = ca.circulant_mh_attention(ca.DotSimilarity(), qp, kp, vp, ws, nh, materialize=False)
    assert A is None
    (y * w).sum().backward()
    qc, kc, vc = (to_cl(t).requires_grad_(True) for t in (q, k, v))
    yc, _ = ca.circulant_mh_attention(ca.DotSimilarity(), qc, kc, vc, ws, nh, materialize=False,
                                      channels_last=True)
    (yc * to_cl(w)).sum().backward()
    assert torch.equal(from_cl(yc.detach()), y.detach())
    for a, b in ((qp, qc), (kp, kc), (vp, vc)):
        assert torch.equal(a.grad, from_cl(b.grad))
