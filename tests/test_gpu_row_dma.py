"""The one-dimensional split-half kernels load planar Float32 rows by 16-byte
LDS DMA when the signal length is a multiple of 4 and every tensor is 16-byte
aligned, and by dword loads into registers otherwise.  Both take the same
arithmetic, so the same inputs at an aligned and at a 4-byte-offset address
must give the same bits (the selection in csrc/fused2h_impl.h, wide_rows)."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

# (length, C, nheads, B, ws, kind)
CASES = [
    (256, 16, 1, 2, 15, 0),
    (260, 32, 2, 1, 15, 1),
    (400, 32, 1, 2, 63, 1),
    (128, 64, 2, 1, 63, 0),
]


def ids(c):
    n, C, nh, B, ws, kind = c
    return f"{n}-C{C}-nh{nh}-B{B}-ws{ws}-{'dist' if kind else 'dot'}"


def run(L, ptr, kind, n, C, nh, B, ws, q, k, v, dy):
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    y = torch.empty_like(q)
    lse = torch.empty((B * nh, n), device=q.device)
    L.check(L.lib.circatt_fused_fwd(kind, L.F32, 1, n, 1, ws, C, nh, B, ptr(q), ptr(k), ptr(v),
                                    ptr(y), ptr(lse), s))
    wb = L.lib.circatt_fused_bwd_workspace_bytes(1, n, 1, nh, B)
    work = torch.empty((wb // 4,), device=q.device)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    L.check(L.lib.circatt_fused_bwd(kind, L.F32, 1, n, 1, ws, C, nh, B, ptr(q), ptr(k), ptr(v),
                                    ptr(y), ptr(dy), ptr(lse), ptr(dq), ptr(dk), ptr(dv),
                                    ptr(work), wb, s))
    torch.cuda.synchronize()
    return y, lse, dq, dk, dv


def offset_copy(t):
    """t's values in a buffer one float past a 16-byte boundary."""
    buf = torch.empty(t.numel() + 4, device=t.device, dtype=t.dtype)
    view = buf[1:1 + t.numel()].view(t.shape)
    view.copy_(t)
    assert view.data_ptr() % 16 == 4
    return view


@pytest.mark.parametrize("case", CASES, ids=ids)
def test_row_dma_matches_register_loads_bitwise(cuda, case):
    from circulant_attention import _lib as L
    from circulant_attention._functions import ptr

    n, C, nh, B, ws, kind = case
    g = torch.Generator(device=cuda)
    g.manual_seed(700 + n + ws)
    q, k, v, dy = (torch.randn((B, C, n), device=cuda, generator=g) for _ in range(4))
    assert all(t.data_ptr() % 16 == 0 for t in (q, k, v, dy))
    aligned = run(L, ptr, kind, n, C, nh, B, ws, q, k, v, dy)
    shifted = run(L, ptr, kind, n, C, nh, B, ws, *(offset_copy(t) for t in (q, k, v, dy)))
    for name, a, b in zip(("y", "lse", "dq", "dk", "dv"), aligned, shifted):
        assert torch.equal(a, b), (name, (a - b).abs().max().item())
