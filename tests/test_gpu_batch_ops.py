"""GPU tests of the batch-dimension entry points (csrc/batch_ops.hip) and of
the Circulant operations built on them.

circatt_fill, circatt_copy_blocks, circatt_sum_middle and
circatt_count_unequal replace the array-library kernels the reference runs
on a Circulant's CSR arrays through CUDA.jl (CUDA.ones, repeat, cat, sum over
dims, ==: src/circulant.jl:68,90, src/array.jl:9,49-64,87-154,179-186).  Each
is checked bit-exactly against a numpy restatement through the C ABI; the
Circulant methods (repeat, cat, sum over batch dims, scale, ==, copy, the
pullbacks of the row and column sums) against numpy on the same values,
gradients included.
"""
import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ca(cuda):
    import circulant_attention
    return circulant_attention


def L():
    from circulant_attention import _lib
    return _lib


def sp():
    from circulant_attention._functions import stream_ptr
    return stream_ptr()


def addr(t, off=0):
    return ctypes.c_void_p(t.data_ptr() + off)


@pytest.mark.parametrize("n", [0, 1, 7, 1000, 1 << 20, (1 << 20) + 3])
@pytest.mark.parametrize("value", [1.0, -0.0, 3.25, float("nan")])
def test_fill(ca, cuda, n, value):
    t = torch.full((n + 2,), 7.0, device=cuda)
    lib = L()
    lib.check(lib.lib.circatt_fill(addr(t, 4), n, value, sp()))
    h = t.cpu().numpy()
    ref = np.full(n + 2, 7.0, np.float32)
    ref[1:n + 1] = np.float32(value)
    assert np.array_equal(h.view(np.uint32), ref.view(np.uint32))


def copy_blocks_ref(dst, src, block, ni, dsi, ssi, no, dso, sso, doff, soff):
    out = dst.copy()
    for o in range(no):
        for i in range(ni):
            d = doff + o * dso + i * dsi
            s = soff + o * sso + i * ssi
            out[d:d + block] = src[s:s + block]
    return out


COPY_CASES = [
    # block, ninner, dsi, ssi, nouter, dso, sso, dst_off, src_off
    (64, 3, 64, 0, 2, 192, 64, 0, 0),       # repeat 3x of 2 blocks (16-byte units)
    (4, 100, 4, 0, 5, 400, 4, 0, 0),        # broadcast of 5 scalars over 100 slots
    (48, 1, 0, 0, 7, 112, 48, 16, 0),       # cat: part into a wider row, offset
    (12, 2, 16, 12, 3, 40, 24, 4, 8),       # 4-byte units
    (6, 3, 6, 6, 2, 18, 18, 2, 2),          # 2-byte aligned: byte units
    (5, 4, 7, 5, 3, 30, 20, 1, 3),          # odd everything: byte units
    (1 << 16, 8, 1 << 16, 0, 3, 1 << 19, 1 << 16, 0, 0),  # larger replicate
]


@pytest.mark.parametrize("case", COPY_CASES)
def test_copy_blocks(ca, cuda, case):
    block, ni, dsi, ssi, no, dso, sso, doff, soff = case
    rng = np.random.default_rng(block + ni)
    dn = doff + (no - 1) * dso + (ni - 1) * dsi + block + 16
    sn = soff + (no - 1) * sso + (ni - 1) * ssi + block + 16
    src = rng.integers(0, 256, sn, dtype=np.uint8)
    dst = rng.integers(0, 256, dn, dtype=np.uint8)
    ts, td = torch.from_numpy(src).to(cuda), torch.from_numpy(dst).to(cuda)
    lib = L()
    lib.check(lib.lib.circatt_copy_blocks(addr(td, doff), addr(ts, soff), block, ni, dsi, ssi, no,
                                          dso, sso, sp()))
    ref = copy_blocks_ref(dst, src, block, ni, dsi, ssi, no, dso, sso, doff, soff)
    assert np.array_equal(td.cpu().numpy(), ref)


def test_copy_blocks_rejects_overlap(ca, cuda):
    t = torch.zeros(1024, dtype=torch.uint8, device=cuda)
    lib = L()
    # destination blocks overlapping each other, and source overlapping destination
    assert lib.lib.circatt_copy_blocks(addr(t, 512), addr(t), 64, 3, 32, 64, 1, 0, 0, sp()) == lib.ERR_INVALID
    assert lib.lib.circatt_copy_blocks(addr(t, 32), addr(t), 64, 1, 0, 0, 1, 0, 0, sp()) == lib.ERR_INVALID
    assert "overlap" in lib.lib.circatt_last_error().decode()


@pytest.mark.parametrize("inner,nsum,outer", [(1, 4, 1), (1, 3, 5), (37, 1, 2), (1000, 4, 3),
                                              (9, 16, 11), (4096, 2, 16), (5, 0, 2)])
def test_sum_middle(ca, cuda, inner, nsum, outer):
    rng = np.random.default_rng(inner + nsum)
    x = rng.standard_normal((outer, nsum, inner)).astype(np.float32)
    tx = torch.from_numpy(x).to(cuda)
    out = torch.full((outer, inner), 5.0, device=cuda)
    lib = L()
    lib.check(lib.lib.circatt_sum_middle(addr(tx), addr(out), inner, nsum, outer, sp()))
    acc = np.zeros((outer, inner))
    for s in range(nsum):  # double accumulation in order of s
        acc = acc + x[:, s, :].astype(np.float64)
    assert np.array_equal(out.cpu().numpy(), acc.astype(np.float32))


def test_count_unequal(ca, cuda):
    lib = L()
    cnt = torch.full((1,), 99, dtype=torch.int64, device=cuda)
    a = np.arange(100000, dtype=np.float32)
    b = a.copy()
    b[[3, 500, 99999]] = -1.0
    ta, tb = torch.from_numpy(a).to(cuda), torch.from_numpy(b).to(cuda)
    lib.check(lib.lib.circatt_count_unequal(1, a.size, addr(ta), addr(tb), addr(cnt), sp()))
    assert int(cnt.item()) == 3
    # floats: -0 == 0 and NaN != NaN; words: the bit patterns
    x = torch.tensor([0.0, float("nan"), 1.0, 2.0], device=cuda)
    y = torch.tensor([-0.0, float("nan"), 1.0, 3.0], device=cuda)
    lib.check(lib.lib.circatt_count_unequal(1, 4, addr(x), addr(y), addr(cnt), sp()))
    assert int(cnt.item()) == 2
    lib.check(lib.lib.circatt_count_unequal(0, 4, addr(x), addr(y), addr(cnt), sp()))
    assert int(cnt.item()) == 2  # -0 vs 0 differ as words; the NaNs have equal bits
    ia = torch.arange(1000, dtype=torch.int32, device=cuda)
    lib.check(lib.lib.circatt_count_unequal(0, 1000, addr(ia), addr(ia), addr(cnt), sp()))
    assert int(cnt.item()) == 0
    lib.check(lib.lib.circatt_count_unequal(0, 0, None, None, addr(cnt), sp()))
    assert int(cnt.item()) == 0


# ---------------------------------------------------------------------------
# Circulant operations on these entry points
# ---------------------------------------------------------------------------
def seeded(seed, shape):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def test_new_repeat_copy_eq(ca, cuda):
    """Circulant{T}(M, dims) has nzVal = 1 (src/circulant.jl:68,90);
    repeat(A, 1, 1, r3, r4) tiles the batch dims as Julia's repeat
    (src/array.jl:49-52), with gradients summed back; copy and ==."""
    dims, ws = (8, 6), 3
    A0 = ca.Circulant.new(ws, (*dims, 2, 3), device=cuda)
    assert torch.equal(A0.nzval, torch.ones_like(A0.nzval))
    a = seeded(1, (3, 2, 48, 9))  # Julia batch (2, 3)
    ta = torch.from_numpy(a).to(cuda).requires_grad_(True)
    A = ca.Circulant(ta, ws, dims)
    R = A.repeat(1, 1, 2, 3)
    assert R.size() == (48, 48, 4, 9)
    ref = np.tile(a, (3, 2, 1, 1))  # Julia repeat tiles each dim whole
    assert np.array_equal(R.nzval.detach().cpu().numpy(), ref)
    w = seeded(2, ref.shape)
    (R.nzval * torch.from_numpy(w).to(cuda)).sum().backward()
    gref = w.reshape(3, 3, 2, 2, 48, 9).astype(np.float64).sum(axis=(0, 2))
    np.testing.assert_allclose(ta.grad.cpu().numpy(), gref, rtol=1e-6, atol=1e-6)
    C = A.copy()
    assert C == A and C.nzval.data_ptr() != A.nzval.data_ptr()
    C.nzval.data[0, 1, 5, 2] += 1.0
    assert not (C == A)


@pytest.mark.parametrize("dims_cat", [3, 4])
def test_cat_values_and_gradients(ca, cuda, dims_cat):
    """cat(A, B; dims) along heads (3) or batches (4) (src/array.jl:62-64,
    README.md:145-148), with gradients split back to the parts."""
    dims, ws = (8, 6), 3
    a, b = seeded(3, (2, 2, 48, 9)), seeded(4, (2, 3, 48, 9) if dims_cat == 3 else (1, 2, 48, 9))
    ta = torch.from_numpy(a).to(cuda).requires_grad_(True)
    tb = torch.from_numpy(b).to(cuda).requires_grad_(True)
    D = ca.cat(ca.Circulant(ta, ws, dims), ca.Circulant(tb, ws, dims), dims=dims_cat)
    ax = 1 if dims_cat == 3 else 0
    ref = np.concatenate([a, b], axis=ax)
    assert np.array_equal(D.nzval.detach().cpu().numpy(), ref)
    w = seeded(5, ref.shape)
    (D.nzval * torch.from_numpy(w).to(cuda)).sum().backward()
    wa, wb = np.split(w, [a.shape[ax]], axis=ax)
    assert np.array_equal(ta.grad.cpu().numpy(), wa) and np.array_equal(tb.grad.cpu().numpy(), wb)


@pytest.mark.parametrize("d", [3, 4])
def test_sum_batch_dim_gradients(ca, cuda, d):
    dims, ws = (8, 6), 3
    a = seeded(6, (3, 2, 48, 9))
    ta = torch.from_numpy(a).to(cuda).requires_grad_(True)
    S = ca.Circulant(ta, ws, dims).sum(d)
    ax = 1 if d == 3 else 0
    acc = np.zeros_like(np.sum(a, axis=ax, keepdims=True), dtype=np.float64)
    for i in range(a.shape[ax]):
        acc = acc + np.take(a, [i], axis=ax).astype(np.float64)
    assert np.array_equal(S.nzval.detach().cpu().numpy(), acc.astype(np.float32))
    w = seeded(7, acc.shape)
    (S.nzval * torch.from_numpy(w).to(cuda)).sum().backward()
    assert np.array_equal(ta.grad.cpu().numpy(), np.broadcast_to(w, a.shape))


@pytest.mark.parametrize("cshape", [(2, 1, 1, 1), (1, 3, 1, 1), (2, 3, 1, 1)])
@pytest.mark.parametrize("abatch", [(2, 3), (1, 3), (2, 1)])
def test_scale_broadcasts(ca, cuda, cshape, abatch):
    """scale(c, A) with c of Julia size (1, 1, nh', B') broadcast against A's
    batch (src/array.jl:179-186), values and gradients to c and A.  Shapes
    are torch order: c (B', nh', 1, 1), A's batch (B, nh)."""
    dims, ws = (8, 6), 3
    rb = tuple(max(x, y) for x, y in zip(cshape[:2], abatch))
    a = seeded(8, (*abatch, 48, 9))
    c = seeded(9, cshape)
    ta = torch.from_numpy(a).to(cuda).requires_grad_(True)
    tc = torch.from_numpy(c).to(cuda).requires_grad_(True)
    Z = ca.scale(tc, ca.Circulant(ta, ws, dims))
    ref = c * a  # numpy broadcasting of (B, nh, 1, 1) against (B', nh', P, K)
    assert Z.nzval.shape == (*rb, 48, 9)
    np.testing.assert_allclose(Z.nzval.detach().cpu().numpy(), ref, rtol=1e-6, atol=0)
    w = seeded(10, ref.shape)
    (Z.nzval * torch.from_numpy(w).to(cuda)).sum().backward()
    ga = (w * c).astype(np.float64)
    ga = ga.sum(axis=tuple(i for i in range(2) if a.shape[i] == 1), keepdims=True)
    gc = (w.astype(np.float64) * a).sum(axis=(2, 3), keepdims=True)
    gc = gc.sum(axis=tuple(i for i in range(2) if c.shape[i] == 1), keepdims=True)
    np.testing.assert_allclose(ta.grad.cpu().numpy(), ga, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(tc.grad.cpu().numpy(), gc, rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("dims", [(8, 6), (11,)])
def test_row_and_column_sum_pullbacks(ca, cuda, dims):
    """d/dA of sum(A; dims=2) (row sums) broadcasts the cotangent over each
    row's slots; of sum(A; dims=1) (column sums) gives slot (r, t) the
    cotangent of its column colVal(r, t)."""
    import oracle as O
    ws = 3
    P = int(np.prod(dims))
    K = ws ** len(dims)
    a = seeded(11, (2, 1, P, K))
    ta = torch.from_numpy(a).to(cuda).requires_grad_(True)
    A = ca.Circulant(ta, ws, dims)
    g = seeded(12, (2, 1, P))
    for d in (1, 2):
        ta.grad = None
        s = A.sum(d)
        (s.reshape(2, 1, P) * torch.from_numpy(g).to(cuda)).sum().backward()
        if d == 2:
            ref = np.broadcast_to(g[..., None], a.shape)
        else:
            _, colval = O.pattern(dims, ws, 1)
            ref = g[:, :, colval.reshape(P, K) - 1]
        assert np.array_equal(ta.grad.cpu().numpy(), ref)
