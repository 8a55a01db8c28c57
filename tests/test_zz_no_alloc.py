"""circatt_fused_bwd_noalloc: the fused backward with its per-row D in the
library's static device scratch instead of a caller workspace.  Its outputs
must equal circatt_fused_bwd's bit for bit (same kernels), on two calls in a
row, the second with a smaller problem, so that a stale or mis-addressed
scratch would show.  Sizes beyond the scratch are rejected on the host."""
import ctypes

import pytest

from conftest import rel_err

FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first


def test_noalloc_rejects_beyond_scratch():
    from circulant_attention import _lib as L
    rows = L.lib.circatt_fused_bwd_noalloc_max_rows()
    assert rows == 4 * 1024 * 1024
    # 2048 x 2048 pixels x 2 heads: 8M rows of D, twice the scratch
    rc = L.lib.circatt_fused_bwd_noalloc(0, 0, 2, 2048, 2048, 3, 32, 2, 1, FAKE, FAKE, FAKE,
                                         FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None)
    assert rc == L.ERR_INVALID
    assert "static scratch" in L.lib.circatt_last_error().decode()
    rc = L.lib.circatt_fused_bwd_noalloc(0, 0, 2, 16, 16, 4, 32, 2, 1, FAKE, FAKE, FAKE,
                                         FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None)
    assert rc == L.ERR_INVALID and "odd" in L.lib.circatt_last_error().decode()


# (spatial fastest-first, C, B, nheads, ws, kind, complex); each pair runs the
# larger problem first, then a smaller one
CASES = [
    [((48, 40), 64, 2, 4, 15, 0, False), ((20, 16), 64, 1, 4, 15, 0, False)],  # split-half
    [((30, 22), 32, 2, 1, 7, 1, True), ((9, 7), 32, 1, 1, 7, 1, True)],        # Float32 MFMA
    [((300,), 32, 2, 1, 63, 1, False), ((70,), 32, 1, 1, 63, 1, False)],        # 1D split-half: row DMA, then per-pixel loads
    [((28, 20), 32, 2, 2, 11, 0, True), ((9, 7), 32, 1, 2, 11, 0, True)],      # split-half, 32 components
]


@pytest.mark.gpu
@pytest.mark.parametrize("pair", CASES, ids=["split-half", "f32-cplx-dist", "1d-ws63", "split-half-32"])
def test_noalloc_matches_workspace_entry_point(cuda, pair):
    import torch

    from circulant_attention import _lib as L
    from circulant_attention._functions import ptr, stream_ptr

    for dims, C, B, nh, ws, kind, cplx in pair:
        print(f"noalloc case dims={dims} C={C} B={B} nh={nh} ws={ws} kind={kind} cplx={cplx}",
              flush=True)
        nsp = len(dims)
        n1, n2 = dims[0], (dims[1] if nsp == 2 else 1)
        P = n1 * n2
        dt = L.C32 if cplx else L.F32
        dtype = torch.complex64 if cplx else torch.float32
        g = torch.Generator(device=cuda)
        g.manual_seed(P + C)
        shape = (B, C, *reversed(dims))
        q, k, v, dy = (torch.randn(shape, device=cuda, dtype=dtype, generator=g)
                       for _ in range(4))
        y = torch.empty_like(q)
        lse = torch.empty((B * nh, P), device=cuda)
        s = stream_ptr()
        L.check(L.lib.circatt_fused_fwd(kind, dt, nsp, n1, n2, ws, C, nh, B, ptr(q), ptr(k),
                                        ptr(v), ptr(y), ptr(lse), s))
        wbytes = L.lib.circatt_fused_bwd_workspace_bytes(nsp, n1, n2, nh, B)
        work = torch.empty((wbytes // 4,), device=cuda)
        ref = [torch.empty_like(q) for _ in range(3)]
        L.check(L.lib.circatt_fused_bwd(kind, dt, nsp, n1, n2, ws, C, nh, B, ptr(q), ptr(k),
                                        ptr(v), ptr(y), ptr(dy), ptr(lse), *map(ptr, ref),
                                        ptr(work), wbytes, s))
        out = [torch.full_like(q, float("nan")) for _ in range(3)]
        L.check(L.lib.circatt_fused_bwd_noalloc(kind, dt, nsp, n1, n2, ws, C, nh, B, ptr(q),
                                                ptr(k), ptr(v), ptr(y), ptr(dy), ptr(lse),
                                                *map(ptr, out), s))
        torch.cuda.synchronize()
        for name, a, b in zip(("dq", "dk", "dv"), out, ref):
            assert torch.equal(a, b), (name, rel_err(a.cpu().numpy(), b.cpu().numpy()))
