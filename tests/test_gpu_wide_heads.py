"""Fused attention for heads wider than 64 real components (the
channel-chunked kernels of csrc/fused_wide_impl.h), against the float64
oracle: forward within 1e-5, gradients within 1e-4 (max-norm relative).

The reference's similarity loops over any channel count
(src/similarity.jl:97-99); these cases cover 80, 96, 128 and 160 real
components per head (chunks of 32 for the scores, output passes of 64, so
partial chunks and passes occur), 1D and 2D windows, real and complex,
Dot and Distance, several heads, and the channels-last layout.
"""
import numpy as np
import pytest

from conftest import TOL_FWD, TOL_GRAD, rel_err

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle as O  # noqa: E402
from test_gpu_parity import dev, host, seeded, shape_of  # noqa: E402

# (dims fastest-first, ws, C, B, nheads, complex)
CASES = [
    ((18, 14), 7, 128, 1, 1, False),    # one head of 128 components
    ((16, 12), 5, 64, 2, 1, True),      # ComplexF32 head of 64 channels = 128 components
    ((20, 16), 11, 160, 1, 2, False),   # two heads of 80
    ((14, 12), 15, 96, 1, 1, False),    # 96: three score chunks, two output passes
    ((150,), 9, 96, 2, 1, False),       # 1D
    ((70,), 31, 40, 1, 1, True),        # 1D, complex 80 components, wide window
]


def ids(c):
    dims, ws, C, B, nh, cplx = c
    return f"{'x'.join(map(str, dims))}-ws{ws}-C{C}-B{B}-h{nh}-{'c32' if cplx else 'f32'}"


@pytest.mark.parametrize("kind", [0, 1], ids=["dot", "dist"])
@pytest.mark.parametrize("case", CASES, ids=ids)
def test_wide_head_fused_matches_oracle(cuda, case, kind):
    import circulant_attention as ca

    dims, ws, C, B, nheads, cplx = case
    shape = shape_of(dims, C, B)
    q, k, v, dy = (seeded(900 + ws + i, shape, cplx) for i in range(4))
    tq, tk, tv = (dev(a, cuda).requires_grad_(True) for a in (q, k, v))
    simfun = ca.DotSimilarity() if kind == 0 else ca.DistanceSimilarity()
    y, A = ca.circulant_mh_attention(simfun, tq, tk, tv, ws, nheads, materialize=False,
                                     honor_simfun=True)
    assert A is None
    yr, _ = O.attention_fwd(kind, q, k, v, ws, nheads)
    assert rel_err(host(y), yr) < TOL_FWD
    td = dev(dy, cuda)
    loss = (y * td.conj()).real.sum() if y.is_complex() else (y * td).sum()
    loss.backward()
    gq, gk, gv = O.attention_bwd(kind, q, k, v, dy, ws, nheads)
    assert rel_err(host(tq.grad), gq) < TOL_GRAD
    assert rel_err(host(tk.grad), gk) < TOL_GRAD
    assert rel_err(host(tv.grad), gv) < TOL_GRAD


def test_wide_head_lse(cuda):
    import ctypes

    from circulant_attention import _lib as L
    from circulant_attention._functions import ptr
    dims, ws, C, B, nh = (18, 14), 7, 128, 1, 1
    n1, n2 = dims
    for kind in (0, 1):
        q, k, v = (seeded(950 + i, shape_of(dims, C, B)) for i in range(3))
        tq, tk, tv = (dev(a, cuda) for a in (q, k, v))
        y = torch.empty_like(tq)
        lse = torch.empty((B * nh, n1 * n2), dtype=torch.float32, device=cuda)
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        L.check(L.lib.circatt_fused_fwd(kind, L.F32, 2, n1, n2, ws, C, nh, B, ptr(tq), ptr(tk),
                                        ptr(tv), ptr(y), ptr(lse), s))
        ref = O.attention_lse(kind, q, k, ws, nh)
        assert np.max(np.abs(host(lse) - ref)) < 1e-5 * np.max(np.abs(ref)) + 1e-5


def test_wide_head_channels_last_matches_planar(cuda):
    import circulant_attention as ca

    g = torch.Generator(device=cuda)
    g.manual_seed(21)
    B, C, n2, n1, nh, ws = 1, 192, 12, 16, 2, 7  # heads of 96
    q, k, v, w = (torch.randn((B, C, n2, n1), device=cuda, generator=g) for _ in range(4))
    qp, kp, vp = (t.clone().requires_grad_(True) for t in (q, k, v))
    y, _ = ca.circulant_mh_attention(ca.DotSimilarity(), qp, kp, vp, ws, nh, materialize=False)
    (y * w).sum().backward()
    cl = lambda t: t.movedim(1, -1).contiguous()
    qc, kc, vc = (cl(t).requires_grad_(True) for t in (q, k, v))
    yc, _ = ca.circulant_mh_attention(ca.DotSimilarity(), qc, kc, vc, ws, nh, materialize=False,
                                      channels_last=True)
    (yc * cl(w)).sum().backward()
    back = lambda t: t.movedim(-1, 1).contiguous()
    assert torch.equal(back(yc.detach()), y.detach())
    for a, b in ((qp, qc), (kp, kc), (vp, vc)):
        assert torch.equal(a.grad, back(b.grad))
