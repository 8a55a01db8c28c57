"""The reference's own training compositions (test/grad.jl) through
libcircatt, against the same compositions built on the CPU in float64 from
the oracle's pieces, plus full-size checks of configurations the other files
run only reduced.

test/grad.jl:9-41 (`dnn`, `dnn_mh`): convolutions produce x, k, q, v; then
A = circulant_(mh_)adjacency(simfun, k, q, W), B = the same of (x, x),
C = alpha*A + (1 - alpha)*B, z = C ⊗ v (C ⨷ v for heads), a last
convolution, and the loss sum(abs2, y - z) / length(y) differentiated with
respect to every convolution weight and alpha.  test/grad.jl:84-113: the
adjacency chains A ⊗ x and (theta*A) ⨷ x with gradients to the weight and
theta.  The convolutions are torch's (cross-correlation, real arithmetic for
complex signals) on both sides; the reference uses NNlib's, which is outside
the path under test.  Weights are N(0, 1/36) instead of N(0, 1) so that the
3x3x4 convolutions give O(1) activations: with N(0, 1) weights the unscaled
adjacency scores reach ~1e2 and the Float32 reference itself is
ill-conditioned (the softmax rounds to one-hot rows).
"""
import math

import numpy as np
import pytest

from conftest import TOL_FWD, TOL_GRAD, rel_err

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle as O  # noqa: E402

WS, NHEADS = 3, 2


@pytest.fixture(scope="module")
def ca(cuda):
    import circulant_attention
    return circulant_attention


def conv(x, w):
    """Valid cross-correlation over the spatial dims, complex by real parts."""
    f = torch.nn.functional.conv2d if x.dim() == 4 else torch.nn.functional.conv1d
    if not x.is_complex():
        return f(x, w)
    xr, xi, wr, wi = x.real, x.imag, w.real, w.imag
    return torch.complex(f(xr, wr) - f(xi, wi), f(xr, wi) + f(xi, wr))


# ---------------------------------------------------------------------------
# float64 CPU compositions of the oracle's pieces, with the rrules of
# src/rrules.jl as their pullbacks
# ---------------------------------------------------------------------------
def _np(t):
    return t.detach().numpy()


class RefAdjacency(torch.autograd.Function):
    """A_nz (nb, P*K) = softmax(similarity(kind, x, y)); x, y (nb, C, P)."""

    @staticmethod
    def forward(ctx, x, y, kind, dims, ws):
        K = ws ** len(dims)
        A = O.softmax(O.similarity(kind, _np(x), _np(y), dims, ws), K)
        ctx.save_for_backward(x, y)
        ctx.meta = (kind, dims, ws, A)
        return torch.from_numpy(A)

    @staticmethod
    def backward(ctx, dA):
        x, y = ctx.saved_tensors
        kind, dims, ws, A = ctx.meta
        P, K = int(np.prod(dims)), ws ** len(dims)
        xn, yn = _np(x), _np(y)
        dS = O.softmax_bwd(A, _np(dA), K)                       # rrules.jl:42-56
        dx = O.apply(dS, yn, dims, ws)                           # rrules.jl:18-32
        dy = O.apply(dS, xn, dims, ws, trans=True)
        if kind == O.DISTANCE:                                   # rrules.jl:1-16
            dx = dx - O.rowsum(dS, P, K)[:, None, :] * xn
            dy = dy - O.colsum(dS, dims, ws)[:, None, :] * yn
        return torch.from_numpy(dx), torch.from_numpy(dy), None, None, None


class RefApply(torch.autograd.Function):
    """y = A ⊗ x; x (nb, C, P)."""

    @staticmethod
    def forward(ctx, A, x, dims, ws):
        ctx.save_for_backward(A, x)
        ctx.meta = (dims, ws)
        return torch.from_numpy(O.apply(_np(A), _np(x), dims, ws))

    @staticmethod
    def backward(ctx, dy):
        A, x = ctx.saved_tensors
        dims, ws = ctx.meta
        dA = O.similarity(O.DOT, _np(dy), _np(x), dims, ws)     # rrules.jl:58-72
        dx = O.apply(_np(A), _np(dy), dims, ws, trans=True)
        return torch.from_numpy(dA), torch.from_numpy(dx), None, None


def ref_adjacency(kind, x, y, nheads):
    """(B, nheads, P*K) adjacency of x against y, heads split as
    src/attention.jl:44 (nheads = 1: circulant_adjacency)."""
    B, C = x.shape[0], x.shape[1]
    dims = tuple(reversed(x.shape[2:]))
    P = int(np.prod(dims))
    A = RefAdjacency.apply(x.reshape(B * nheads, C // nheads, P),
                           y.reshape(B * nheads, C // nheads, P), kind, dims, WS)
    return A.reshape(B, nheads, -1)


def ref_apply(A, v, nheads):
    B, C = v.shape[0], v.shape[1]
    dims = tuple(reversed(v.shape[2:]))
    P = int(np.prod(dims))
    y = RefApply.apply(A.reshape(B * nheads, -1), v.reshape(B * nheads, C // nheads, P), dims, WS)
    return y.reshape(v.shape)


def dnn_ref(x, params, kind, mh):
    wx, wk, wq, wv, wz, alpha = params
    nh = NHEADS if mh else 1
    xx, k, q, v = (conv(x, w) for w in (wx, wk, wq, wv))
    A = ref_adjacency(kind, k, q, nh)
    Bm = ref_adjacency(kind, xx, xx, nh)
    a = alpha.reshape(1, -1, 1)  # Julia (1, 1, heads, 1)
    Cm = a * A + (1 - a) * Bm
    return conv(ref_apply(Cm, v, nh), wz)


def dnn_gpu(ca, x, params, simfun, mh):
    """test/grad.jl:9-41 written with the drop-in API."""
    wx, wk, wq, wv, wz, alpha = params
    xx, k, q, v = (conv(x, w) for w in (wx, wk, wq, wv))
    if mh:
        A = ca.circulant_mh_adjacency(simfun, k, q, WS, NHEADS)
        Bm = ca.circulant_mh_adjacency(simfun, xx, xx, WS, NHEADS)
    else:
        A = ca.circulant_adjacency(simfun, k, q, WS)
        Bm = ca.circulant_adjacency(simfun, xx, xx, WS)
    Cm = alpha * A + (1 - alpha) * Bm
    z = ca.Otimes(Cm, v) if mh else ca.otimes(Cm, v)
    return conv(z, wz)


def randn(rng, shape, cplx, scale=1.0):
    if cplx:
        a = (rng.standard_normal(shape) + 1j * rng.standard_normal(shape)) / math.sqrt(2)
        return (a * scale).astype(np.complex64)
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def grad_jl_inputs(seed, nsp, cplx):
    """Shapes of test/grad.jl:46-56: x 12^N x 4 x 2, y 8^N x 4 x 2, kernels 3^N."""
    rng = np.random.default_rng(seed)
    sp = (12,) * nsp
    x = randn(rng, (2, 4, *sp), cplx)
    y = randn(rng, (2, 4, *((8,) * nsp)), cplx)
    ks = (3,) * nsp
    ws = [randn(rng, (8, 4, *ks), cplx, 1 / 6) for _ in range(4)]
    wz = randn(rng, (4, 8, *ks), cplx, 1 / 6)
    return x, y, ws + [wz]


def loss_fn(y, z):
    return (y - z).abs().pow(2).sum() / y.numel()  # sum(abs2, y - z) / length(y)


@pytest.mark.parametrize("mh", [False, True], ids=["dnn", "dnn_mh"])
@pytest.mark.parametrize("nsp", [1, 2])
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [0, 1])
def test_grad_jl_dnn(ca, cuda, mh, nsp, cplx, kind):
    """test/grad.jl:9-41, 58-78: z and the gradients of all six parameters."""
    x, y, ws = grad_jl_inputs(900 + 10 * nsp + 2 * kind + (5 if cplx else 0), nsp, cplx)
    nh = NHEADS if mh else 1
    alpha = np.full((1, nh, 1, 1), 0.8, np.float32)  # 0.8f0 * ones(1, 1, nh, 1)
    simfun = ca.DotSimilarity() if kind == 0 else ca.DistanceSimilarity()

    gp = [torch.from_numpy(a).to(cuda).requires_grad_(True) for a in ws + [alpha]]
    z = dnn_gpu(ca, torch.from_numpy(x).to(cuda), gp, simfun, mh)
    assert z.shape == (2, 4, *((8,) * nsp))
    loss_fn(torch.from_numpy(y).to(cuda), z).backward()

    to64 = (lambda a: a.astype(np.complex128)) if cplx else (lambda a: a.astype(np.float64))
    rp = [torch.from_numpy(to64(a)).requires_grad_(True) for a in ws]
    rp.append(torch.from_numpy(alpha.astype(np.float64)).requires_grad_(True))
    zr = dnn_ref(torch.from_numpy(to64(x)), rp, kind, mh)
    loss_fn(torch.from_numpy(to64(y)), zr).backward()

    assert rel_err(z.detach().cpu().numpy(), zr.detach().numpy()) < TOL_FWD
    for name, g, r in zip(("Wx", "Wk", "Wq", "Wv", "Wz", "alpha"), gp, rp):
        assert g.grad is not None, name
        assert rel_err(g.grad.cpu().numpy(), r.grad.numpy()) < TOL_GRAD, name


@pytest.mark.parametrize("mh", [False, True], ids=["adjacency", "mh_adjacency"])
@pytest.mark.parametrize("nsp", [1, 2])
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [0, 1])
def test_grad_jl_adjacency_chain(ca, cuda, mh, nsp, cplx, kind):
    """test/grad.jl:84-113: x = conv(z1, wx), y = conv(z2, wx);
    A = circulant_(mh_)adjacency(simfun, x, y, W); z = A ⊗ x or (theta*A) ⨷ x;
    loss sum(abs2, z); gradients to wx (and theta)."""
    rng = np.random.default_rng(950 + 10 * nsp + 2 * kind + (5 if cplx else 0))
    sp = (12,) * nsp
    z1, z2 = randn(rng, (2, 4, *sp), cplx), randn(rng, (2, 4, *sp), cplx)
    wx = randn(rng, (8, 4, *((3,) * nsp)), cplx, 1 / 6)
    theta = np.full((1, NHEADS, 1, 1), 0.8, np.float32)
    simfun = ca.DotSimilarity() if kind == 0 else ca.DistanceSimilarity()

    tw = torch.from_numpy(wx).to(cuda).requires_grad_(True)
    tt = torch.from_numpy(theta).to(cuda).requires_grad_(True)
    xg, yg = conv(torch.from_numpy(z1).to(cuda), tw), conv(torch.from_numpy(z2).to(cuda), tw)
    if mh:
        A = ca.circulant_mh_adjacency(simfun, xg, yg, WS, NHEADS)
        zg = ca.Otimes(tt * A, xg)
    else:
        zg = ca.otimes(ca.circulant_adjacency(simfun, xg, yg, WS), xg)
    zg.abs().pow(2).sum().backward()

    to64 = (lambda a: a.astype(np.complex128)) if cplx else (lambda a: a.astype(np.float64))
    rw = torch.from_numpy(to64(wx)).requires_grad_(True)
    rt = torch.from_numpy(theta.astype(np.float64)).requires_grad_(True)
    xr, yr = conv(torch.from_numpy(to64(z1)), rw), conv(torch.from_numpy(to64(z2)), rw)
    nh = NHEADS if mh else 1
    A = ref_adjacency(kind, xr, yr, nh)
    if mh:
        A = rt.reshape(1, -1, 1) * A
    zr = ref_apply(A, xr, nh)
    zr.abs().pow(2).sum().backward()

    assert rel_err(zg.detach().cpu().numpy(), zr.detach().numpy()) < TOL_FWD
    assert rel_err(tw.grad.cpu().numpy(), rw.grad.numpy()) < TOL_GRAD
    if mh:
        assert rel_err(tt.grad.cpu().numpy(), rt.grad.numpy()) < TOL_GRAD


# ---------------------------------------------------------------------------
# in-place variants and the remaining Circulant algebra (src/array.jl)
# ---------------------------------------------------------------------------
def seeded(seed, shape, cplx=False):
    rng = np.random.default_rng(seed)
    return randn(rng, shape, cplx)


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("cplx", [False, True])
def test_inplace_variants(ca, cuda, kind, cplx):
    """circulant_similarity! / circulant_adjacency! / softmax!
    (src/similarity.jl:31-53, 105-116, 144-148) write into the given
    Circulant's nzVal and equal their allocating counterparts."""
    dims, ws, C, B = (12, 10), 5, 6, 2
    x, y = (torch.from_numpy(seeded(960 + i + kind, (B, C, *reversed(dims)), cplx)).to(cuda)
            for i in range(2))
    simfun = ca.DotSimilarity() if kind == 0 else ca.DistanceSimilarity()
    A = ca.Circulant.new(ws, (*dims, 1, B), device=cuda)
    buf = A.nzval.data_ptr()
    out = ca.circulant_similarity_(A, simfun, x, y)
    assert out is A and A.nzval.data_ptr() == buf
    S = ca.circulant_similarity(simfun, x, y, ws)
    assert torch.equal(A.nzval, S.nzval)
    P = int(np.prod(dims))
    Sr = O.similarity(kind, x.cpu().numpy().reshape(B, C, P), y.cpu().numpy().reshape(B, C, P),
                      dims, ws)
    assert rel_err(A.nzval.cpu().numpy().reshape(B, -1), Sr) < TOL_FWD

    Bc = ca.Circulant.new(ws, (*dims, 1, B), device=cuda)
    out = ca.softmax_(Bc, A)  # softmax!(B, A): B = softmax(A)
    assert out is Bc and torch.equal(A.nzval, S.nzval)
    Ar = O.softmax(Sr, ws * ws)
    assert rel_err(Bc.nzval.cpu().numpy().reshape(B, -1), Ar) < TOL_FWD
    ca.softmax_(A)  # in place
    assert torch.equal(A.nzval, Bc.nzval)

    D = ca.Circulant.new(ws, (*dims, 1, B), device=cuda)
    buf = D.nzval.data_ptr()
    assert ca.circulant_adjacency_(D, simfun, x, y) is D and D.nzval.data_ptr() == buf
    assert torch.equal(D.nzval, ca.circulant_adjacency(simfun, x, y, ws).nzval)


def test_circulant_algebra_leftovers(ca, cuda):
    """dot (src/array.jl:83-85), unary - (:79), sum over dims 4, (1, 2), 3
    and : (:132-177), and show (:44-47) on a (P, P, nh, B) Circulant."""
    dims, ws, nh, B = (8, 6), 3, 3, 2
    P, K = 48, 9
    a = seeded(970, (B, nh, P, K))
    b = seeded(971, (B, nh, P, K))
    A = ca.Circulant(torch.from_numpy(a).to(cuda), ws, dims)
    Bm = ca.Circulant(torch.from_numpy(b).to(cuda), ws, dims)
    assert A.size() == (P, P, nh, B)
    d = A.dot(Bm)
    assert abs(float(d) - float((a.astype(np.float64) * b).sum())) < 1e-5 * np.abs(a * b).sum()
    N = -A
    assert torch.equal(N.nzval, -A.nzval)
    s4 = A.sum(4)
    assert s4.size() == (P, P, nh, 1)
    assert rel_err(s4.nzval.cpu().numpy(), a.astype(np.float64).sum(axis=0, keepdims=True)) < 1e-6
    s3 = A.sum(3)
    assert s3.size() == (P, P, 1, B)
    assert rel_err(s3.nzval.cpu().numpy(), a.astype(np.float64).sum(axis=1, keepdims=True)) < 1e-6
    s12 = A.sum((1, 2))
    assert tuple(s12.shape) == (B, nh, 1, 1)
    assert rel_err(s12.cpu().numpy(), a.astype(np.float64).sum(axis=(2, 3))[..., None, None]) < 1e-6
    tot = A.sum()
    assert abs(float(tot) - float(a.astype(np.float64).sum())) < 1e-5 * np.abs(a).sum()
    text = repr(A)
    assert "kernel-length 3" in text and "spatial-size (8, 6)" in text


# ---------------------------------------------------------------------------
# full-size configurations
# ---------------------------------------------------------------------------
def test_cfg2_backward_full_size(ca, cuda):
    """Benchmark configuration cfg2 (README.md:55-71, 128x96x64x2, ws = 15) at full size, the
    unfused path: y, A and the gradients of q, k, v for an N(0,1) dy against
    the oracle (the forward alone is test_gpu_parity's)."""
    dims, ws, C, B = (128, 96), 15, 64, 2
    shape = (B, C, *reversed(dims))
    q, k, v, dy = (seeded(1002 + 10 * i, shape).astype(np.float64) for i in range(4))
    tq, tk, tv = (torch.from_numpy(a.astype(np.float32)).to(cuda).requires_grad_(True)
                  for a in (q, k, v))
    y, A = ca.circulant_attention(ca.DotSimilarity(), tq, tk, tv, ws)
    (y * torch.from_numpy(dy.astype(np.float32)).to(cuda)).sum().backward()
    yr, Ar = O.attention_fwd(0, q, k, v, ws)
    gr = O.attention_bwd(0, q, k, v, dy, ws, A=Ar)
    assert rel_err(y.detach().cpu().numpy(), yr) < TOL_FWD
    for name, t, r in zip(("dq", "dk", "dv"), (tq, tk, tv), gr):
        assert rel_err(t.grad.cpu().numpy(), r) < TOL_GRAD, name


FULL = {
    # name: (dims, C, B, nheads, ws, kind, complex) of the benchmark configurations
    "cfg4a": ((512, 512), 32, 1, 1, 31, 1, False),
    "cfg4b": ((262144,), 32, 2, 1, 63, 1, False),
    "cfg5": ((320, 320), 32, 2, 2, 11, 0, True),
}


@pytest.mark.parametrize("name", list(FULL))
def test_fused_matches_unfused_full_size(ca, cuda, name):
    """Benchmark configurations cfg4a, cfg4b and cfg5 at full size: the fused kernels agree
    with the unfused composition (itself checked against the oracle by the
    reduced-size tests) for y and all gradients; rows of A sum to one."""
    dims, C, B, nh, ws, kind, cplx = FULL[name]
    g = torch.Generator(device=cuda)
    g.manual_seed(1000 + len(name))
    dtype = torch.complex64 if cplx else torch.float32
    shape = (B, C, *reversed(dims))
    q, k, v, dy = (torch.randn(shape, device=cuda, dtype=dtype, generator=g) for _ in range(4))
    simfun = ca.DotSimilarity() if kind == 0 else ca.DistanceSimilarity()
    outs, grads = [], []
    for materialize in (True, False):
        tq, tk, tv = (t.clone().requires_grad_(True) for t in (q, k, v))
        if nh == 1:
            y, A = ca.circulant_attention(simfun, tq, tk, tv, ws, materialize=materialize)
        else:
            y, A = ca.circulant_mh_attention(simfun, tq, tk, tv, ws, nh, materialize=materialize)
        loss = (y * dy.conj()).real.sum() if cplx else (y * dy).sum()
        loss.backward()
        outs.append(y.detach().cpu().numpy())
        grads.append([t.grad.cpu().numpy() for t in (tq, tk, tv)])
        if materialize:
            assert torch.max(torch.abs(A.sum(2) - 1)).item() < 1e-5
        del A, y, loss
        torch.cuda.empty_cache()
    assert rel_err(outs[1], outs[0]) < TOL_FWD
    for nm, a, b in zip(("dq", "dk", "dv"), grads[1], grads[0]):
        assert rel_err(a, b) < TOL_GRAD, nm


@pytest.mark.parametrize("nnz,nb", [(1, 1), (7, 3), (4096, 2), (65537, 2), (1000003, 1),
                                    (12_390_400, 1), (300, 70000)])
@pytest.mark.parametrize("with_y", [False, True])
def test_batch_dot(cuda, nnz, nb, with_y):
    """circatt_batch_dot against float64 sums: odd and aligned lengths, more
    chunks than one workgroup, more batches than one grid row (70000), and
    operands offset by one float (no 16-byte alignment)."""
    from circulant_attention import _lib as L
    from circulant_attention._functions import ptr, stream_ptr
    if nnz * nb > 30_000_000:
        pytest.skip("size")
    g = torch.Generator(device=cuda)
    g.manual_seed(nnz + nb)
    X = torch.randn(nnz * nb + 1, device=cuda, generator=g)[1:]  # misaligned by 4 bytes
    Y = torch.randn(nnz * nb, device=cuda, generator=g) if with_y else None
    out = torch.empty(nb, device=cuda)
    wb = L.lib.circatt_batch_dot_workspace_bytes(nnz, nb)
    work = torch.empty((wb + 7) // 8, dtype=torch.float64, device=cuda)
    L.check(L.lib.circatt_batch_dot(nnz, nb, ptr(X), ptr(Y), ptr(out), ptr(work), wb,
                                    stream_ptr()))
    x = X.cpu().numpy().astype(np.float64).reshape(nb, nnz)
    ref = (x * Y.cpu().numpy().astype(np.float64).reshape(nb, nnz)).sum(1) if with_y else x.sum(1)
    scale = (np.abs(x) * (np.abs(Y.cpu().numpy().reshape(nb, nnz)) if with_y else 1)).sum(1)
    assert np.all(np.abs(out.cpu().numpy() - ref) <= 1e-6 * scale + 1e-30)
    out2 = torch.empty_like(out)
    L.check(L.lib.circatt_batch_dot(nnz, nb, ptr(X), ptr(Y), ptr(out2), ptr(work), wb,
                                    stream_ptr()))
    assert torch.equal(out, out2)  # fixed summation order


def test_dot_and_sums_carry_gradients(ca, cuda):
    """dot(X, Y), sum(A) and sum(A; dims=(1,2)) are differentiable: d/dX of
    dot is Y, of the sums a broadcast of the cotangent."""
    dims, ws, nh, B = (8, 6), 3, 2, 2
    a, b = seeded(980, (B, nh, 48, 9)), seeded(981, (B, nh, 48, 9))
    ta = torch.from_numpy(a).to(cuda).requires_grad_(True)
    tb = torch.from_numpy(b).to(cuda).requires_grad_(True)
    A, Bm = ca.Circulant(ta, ws, dims), ca.Circulant(tb, ws, dims)
    A.dot(Bm).backward()
    assert torch.equal(ta.grad, tb.detach()) and torch.equal(tb.grad, ta.detach())
    ta.grad = None
    (A.sum() * 3).backward()
    assert torch.all(ta.grad == 3)
    ta.grad = None
    w = torch.arange(B * nh, dtype=torch.float32, device=cuda).reshape(B, nh, 1, 1)
    (A.sum((1, 2)) * w).sum().backward()
    assert torch.equal(ta.grad, w.expand(B, nh, 48, 9))


# ---------------------------------------------------------------------------
# the transposed apply and its rrule
# ---------------------------------------------------------------------------
def _f64(a):
    return a.astype(np.complex128 if np.iscomplexobj(a) else np.float64)


@pytest.mark.parametrize("mh", [False, True], ids=["transposed", "mh_transposed"])
@pytest.mark.parametrize("nsp", [1, 2])
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [0, 1])
def test_transposed_attention_gradients(ca, cuda, mh, nsp, cplx, kind):
    """y = Aᵀ ⊗ v for A = circulant_(mh_)adjacency(simfun, q/sqrt(tau),
    k/sqrt(tau)): circulant_transposed_attention (src/attention.jl:72-80) and
    circulant_mh_transposed_attention (:98-103), differentiated through the
    transposed apply's rrule (src/rrules.jl:74-88: dA = sim_Dot(v, dy),
    dv = A ⊠ dy), the softmax and the similarity, against the oracle's
    composition (pinned by finite differences in tests/test_oracle.py)."""
    dims = (14,) if nsp == 1 else (12, 10)
    ws, C, B = 5, 8, 2
    nh = 2 if mh else 1
    shape = (B, C, *reversed(dims))
    seed = 990 + 10 * kind + 20 * nsp + (5 if cplx else 0) + (40 if mh else 0)
    q, k, v, dy = (seeded(seed + i, shape, cplx) for i in range(4))
    tq, tk, tv = (torch.from_numpy(a).to(cuda).requires_grad_(True) for a in (q, k, v))
    s4 = (C // nh) ** -0.25  # q, k / sqrt(tau), tau = sqrt(channels per head)
    simfun = ca.DotSimilarity() if kind == 0 else ca.DistanceSimilarity()
    if mh:
        A = ca.circulant_mh_adjacency(simfun, tq * s4, tk * s4, ws, nh)
        y = ca.circulant_mh_transposed_attention(A, tv)
    else:
        A = ca.circulant_adjacency(simfun, tq * s4, tk * s4, ws)
        y = ca.circulant_transposed_attention(A, tv)
    td = torch.from_numpy(dy).to(cuda)
    loss = (y * td.conj()).real.sum() if cplx else (y * td).sum()
    loss.backward()
    yr, _ = O.attention_fwd(kind, *(_f64(a) for a in (q, k, v)), ws, nh, trans=True)
    gr = O.attention_bwd(kind, *(_f64(a) for a in (q, k, v, dy)), ws, nh, trans=True)
    assert rel_err(y.detach().cpu().numpy(), yr) < TOL_FWD
    for name, t, r in zip(("dq", "dk", "dv"), (tq, tk, tv), gr):
        assert rel_err(t.grad.cpu().numpy(), r) < TOL_GRAD, name


def test_cfg5_composition_full_size(ca, cuda):
    """Benchmark configuration cfg5 / README.md:128-134 at full size (320x320, 32 complex
    channels, B = 2, 2 heads, ws = 11): y, A = mh attention; u, B = mh
    attention of (y, y, y); C = A + m*B with m of Julia size (1, 1, 2, 2);
    w = C ⨷ u.  A, B, C and w against the oracle (the float64 C restatement,
    at full size), rows of A and B summing to one, and linearity of ⨷:
    C ⨷ u = A ⨷ u + m (B ⨷ u)."""
    dims, ws, Cc, Bb, nh = (320, 320), 11, 32, 2, 2
    P, K = 320 * 320, 121
    shape = (Bb, Cc, *reversed(dims))
    q, k, v = (seeded(1005 + i, shape, True) for i in range(3))
    m = seeded(1008, (Bb, nh, 1, 1))
    tq, tk, tv = (torch.from_numpy(a).to(cuda) for a in (q, k, v))
    y, A = ca.circulant_mh_attention(ca.DotSimilarity(), tq, tk, tv, ws, nh)
    u, Bm = ca.circulant_mh_attention(ca.DotSimilarity(), y, y, y, ws, nh)
    tm = torch.from_numpy(m).to(cuda)
    Cm = A + ca.scale(tm, Bm)
    w = ca.Otimes(Cm, u)
    # rows of the two adjacencies sum to one; linearity of the apply
    for X in (A, Bm):
        assert torch.max(torch.abs(X.sum(2) - 1)).item() < 1e-5
    lin = ca.Otimes(A, u) + ca.Otimes(ca.scale(tm, Bm), u)
    assert rel_err(w.cpu().numpy(), lin.cpu().numpy()) < TOL_FWD
    # against the oracle, step by step
    yr, Ar = O.attention_fwd(0, *(_f64(a) for a in (q, k, v)), ws, nh)
    assert rel_err(A.nzval.cpu().numpy().reshape(Ar.shape), Ar) < TOL_FWD
    assert rel_err(y.cpu().numpy(), yr) < TOL_FWD
    yh = _f64(y.cpu().numpy())
    ur, Br = O.attention_fwd(0, yh, yh, yh, ws, nh)
    assert rel_err(Bm.nzval.cpu().numpy().reshape(Br.shape), Br) < TOL_FWD
    assert rel_err(u.cpu().numpy(), ur) < TOL_FWD
    Cr = O.axpby(np.ones(Bb * nh), Ar, m.reshape(-1), Br)
    del Ar, Br
    assert rel_err(Cm.nzval.cpu().numpy().reshape(Cr.shape), Cr) < TOL_FWD
    uh = _f64(u.cpu().numpy()).reshape(Bb * nh, Cc // nh, P)
    wr = O.apply(Cr, uh, dims, ws).reshape(shape)
    assert rel_err(w.cpu().numpy(), wr) < TOL_FWD
    assert Cm.nzval.numel() == Bb * nh * P * K
