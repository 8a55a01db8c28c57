"""Pins the CPU oracle (oracle/) before it is trusted as the parity reference.

The reference (Julia + CUDA.jl + cuSPARSE) cannot run here and ships no
golden vectors, so each oracle function is checked against what the
mathematics fixes, chosen so that a dropped term, a wrong sign or index or a
transposed operand fails:
  * pattern: the known-answer rows derived by hand from src/circulant.jl:6-44,
    README.md:71's nnz count, the sorted-window closed form, the Kronecker
    identity of src/misc.jl:13-17, rowPtr = 1 + K r and symmetry;
  * similarity / softmax / apply: dense P x P brute force with a circular
    window mask (numpy matmul, independent of the CSR slot order);
  * attention: dense masked attention (README.md:7-12) and the README
    identity softmax(similarity) ⊗ v == y (README.md:114-118);
  * backward: central finite differences in float64 of the forward, as the
    reference's own tests do (test/rrule.jl:18-22), plus planted mistakes in
    the oracle's composition that these checks must catch.
"""
import itertools

import numpy as np
import pytest

import oracle as O

rng = np.random.default_rng(0)


def window_counts(dims, ws):
    """Dense (P, P) multiplicity matrix of the circular window: entry (r, c) =
    number of offsets d in [-p, p]^nsp with r + d = c (mod N)."""
    p = (ws - 1) // 2
    if len(dims) == 1:
        (N,) = dims
        M = np.zeros((N, N), np.int64)
        for r in range(N):
            for d in range(-p, p + 1):
                M[r, (r + d) % N] += 1
        return M
    N1, N2 = dims
    P = N1 * N2
    M = np.zeros((P, P), np.int64)
    for i2, i1 in itertools.product(range(N2), range(N1)):
        for d2, d1 in itertools.product(range(-p, p + 1), repeat=2):
            M[i1 + N1 * i2, (i1 + d1) % N1 + N1 * ((i2 + d2) % N2)] += 1
    return M


def csr_dense(nz_b, colval, P, K):
    """Dense (P, P) matrix of one batch of nzVal (duplicates accumulate)."""
    A = np.zeros((P, P), nz_b.dtype)
    rows = np.repeat(np.arange(P), K)
    np.add.at(A, (rows, colval - 1), nz_b)
    return A


# ---------------------------------------------------------------------------
# pattern
# ---------------------------------------------------------------------------

def test_pattern_known_rows():
    # Derived by hand from cartesian_circulant (src/circulant.jl:6-19):
    # 1D N=8, ws=5, row 1: shift s = 1-2-1 = -2, slots 1..5 -> offsets 0,1,2,-2,-1.
    _, cv = O.pattern((8,), 5)
    rows = cv[0].reshape(8, 5)
    assert rows[0].tolist() == [1, 2, 3, 7, 8]
    assert rows[1].tolist() == [1, 2, 3, 4, 8]
    assert rows[4].tolist() == [3, 4, 5, 6, 7]  # interior row: no shift
    assert rows[7].tolist() == [1, 2, 6, 7, 8]
    _, cv = O.pattern((8, 8), 3)
    assert cv[0].reshape(64, 9)[0].tolist() == [1, 2, 8, 9, 10, 16, 57, 58, 64]
    # ws > N: unsorted rows with duplicates, reproduced literally
    _, cv = O.pattern((2,), 5)
    assert cv[0].reshape(2, 5)[0].tolist() == [1, 2, 1, 1, 2]
    _, cv = O.pattern((4,), 5)
    assert cv[0].reshape(4, 5)[0].tolist() == [1, 2, 3, 3, 4]


def test_pattern_readme_count():
    # README.md:59,71: 128x96, ws=15, B=2 -> (12288, 12288, 1, 2), 5529600 entries
    rowptr, colval = O.pattern((128, 96), 15, nb=2)
    assert colval.size == 5_529_600
    assert rowptr.shape == (2, 12289)
    assert np.array_equal(rowptr[0], 1 + 225 * np.arange(12289))
    assert np.array_equal(rowptr[0], rowptr[1]) and np.array_equal(colval[0], colval[1])


@pytest.mark.parametrize("dims", [(n,) for n in range(1, 26)] +
                         [(a, b) for a in (1, 2, 3, 5, 8, 10) for b in (1, 3, 4, 7, 10)])
def test_pattern_closed_form(dims):
    """For ws <= N the rows are the ascending sorted window (no duplicates);
    for every ws each row is the window as a multiset."""
    for ws in (1, 3, 5, 7, 9, 11):
        _, cv = O.pattern(dims, ws)
        P = int(np.prod(dims))
        K = ws ** len(dims)
        rows = cv[0].reshape(P, K) - 1
        M = window_counts(dims, ws)
        for r in range(P):
            multiset = np.repeat(np.arange(P), M[r])
            assert np.array_equal(np.sort(rows[r]), multiset)
            if ws <= min(dims):
                assert np.array_equal(rows[r], multiset)  # sorted ascending


@pytest.mark.parametrize("dims,ws", [((6, 5), 3), ((4, 7), 5), ((3, 3), 5), ((10, 8), 7)])
def test_pattern_kron_identity(dims, ws):
    """2D pattern = kron(circ(N2), circ(N1)) (src/misc.jl:13-17), with counts."""
    N1, N2 = dims
    _, c1 = O.pattern((N1,), ws)
    _, c2 = O.pattern((N2,), ws)
    _, cc = O.pattern(dims, ws)
    D1 = csr_dense(np.ones(N1 * ws), c1[0], N1, ws)
    D2 = csr_dense(np.ones(N2 * ws), c2[0], N2, ws)
    D = csr_dense(np.ones(N1 * N2 * ws * ws), cc[0], N1 * N2, ws * ws)
    assert np.array_equal(D, np.kron(D2, D1))
    assert np.array_equal(D, D.T)  # c in win(r) <=> r in win(c), with multiplicity


def test_pattern_rejects_even_window():
    with pytest.raises(ValueError):
        O.pattern((8,), 4)


# ---------------------------------------------------------------------------
# similarity, softmax, apply vs dense brute force
# ---------------------------------------------------------------------------

def rand_signal(shape, cplx):
    if cplx:
        return (rng.standard_normal(shape) + 1j * rng.standard_normal(shape)) / np.sqrt(2)
    return rng.standard_normal(shape)


CASES = [((8,), 5), ((8, 8), 5), ((12, 10), 3), ((4,), 5), ((4, 4), 5), ((2,), 5), ((5, 3), 7)]


@pytest.mark.parametrize("dims,ws", CASES)
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [O.DOT, O.DISTANCE])
def test_similarity_dense(dims, ws, cplx, kind):
    P, K, nb, C = int(np.prod(dims)), ws ** len(dims), 2, 3
    x = rand_signal((nb, C, P), cplx)
    y = rand_signal((nb, C, P), cplx)
    nz = O.similarity(kind, x, y, dims, ws, scale=0.7).reshape(nb, P, K)
    _, cv = O.pattern(dims, ws)
    rows = np.repeat(np.arange(P), K)
    cols = cv[0] - 1
    for b in range(nb):
        if kind == O.DOT:
            dense = np.real(x[b].T @ np.conj(y[b]))  # (P, P): Re(x_r . conj(y_c))
        else:
            diff = x[b].T[:, None, :] - y[b].T[None, :, :]
            dense = -0.5 * np.sum(np.abs(diff) ** 2, axis=2)
        np.testing.assert_allclose(nz[b].ravel(), 0.7 * dense[rows, cols], rtol=1e-12,
                                   atol=1e-12)


@pytest.mark.parametrize("K", [1, 5, 49])
def test_softmax_rows(K):
    a = rng.standard_normal((3, 7, K)) * 5
    out = O.softmax(a, K)
    e = np.exp(a - a.max(axis=-1, keepdims=True))
    np.testing.assert_allclose(out, e / e.sum(-1, keepdims=True), rtol=1e-13)
    da = rng.standard_normal(a.shape)
    ds = O.softmax_bwd(out, da, K)
    # Jacobian of softmax applied row by row: (diag(s) - s s^T) da
    for idx in np.ndindex(a.shape[:-1]):
        s = out[idx]
        J = np.diag(s) - np.outer(s, s)
        np.testing.assert_allclose(ds[idx], J @ da[idx], rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("dims,ws", CASES)
@pytest.mark.parametrize("cplx", [False, True])
def test_apply_dense(dims, ws, cplx):
    P, K, nb, C = int(np.prod(dims)), ws ** len(dims), 2, 3
    nz = rng.standard_normal((nb, P * K))
    x = rand_signal((nb, C, P), cplx)
    _, cv = O.pattern(dims, ws)
    y = O.apply(nz, x, dims, ws, trans=False)
    yt = O.apply(nz, x, dims, ws, trans=True)
    for b in range(nb):
        A = csr_dense(nz[b], cv[0], P, K)
        np.testing.assert_allclose(y[b], (A @ x[b].T).T, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(yt[b], (A.T @ x[b].T).T, rtol=1e-12, atol=1e-12)
    rs = O.rowsum(nz, P, K)
    cs = O.colsum(nz, dims, ws)
    for b in range(nb):
        A = csr_dense(nz[b], cv[0], P, K)
        np.testing.assert_allclose(rs[b], A.sum(axis=1), rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(cs[b], A.sum(axis=0), rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# attention forward vs dense masked attention; README identity
# ---------------------------------------------------------------------------

def dense_attention(kind, q, k, v, ws, nheads):
    """Dense circular-window attention with multiplicities, per head."""
    dims = O.spatial_dims(q)
    M = window_counts(dims, ws)
    qf, kf, vf = (O._flat(a, nheads) for a in (q, k, v))
    y = np.zeros_like(vf)
    for b in range(qf.shape[0]):
        Q, Kk, V = qf[b].T, kf[b].T, vf[b].T  # (P, dh)
        if kind == O.DOT:
            S = np.real(Q @ np.conj(Kk).T)
        else:
            S = -0.5 * np.sum(np.abs(Q[:, None, :] - Kk[None, :, :]) ** 2, axis=2)
        S = S / np.sqrt(qf.shape[1])
        W = M * np.exp(S - S.max(axis=1, keepdims=True))
        W = W / W.sum(axis=1, keepdims=True)
        y[b] = (W @ V).T
    return y.reshape(q.shape)


ATT_CASES = [((8,), 5, 1), ((8, 8), 5, 1), ((6, 5), 3, 2), ((4, 4), 5, 1), ((3,), 5, 2),
             ((10, 10), 3, 2)]


@pytest.mark.parametrize("dims,ws,nheads", ATT_CASES)
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [O.DOT, O.DISTANCE])
def test_attention_fwd_dense(dims, ws, nheads, cplx, kind):
    B, C = 2, 4
    shape = (B, C, *reversed(dims))
    q, k, v = (rand_signal(shape, cplx) for _ in range(3))
    y, A = O.attention_fwd(kind, q, k, v, ws, nheads)
    np.testing.assert_allclose(y, dense_attention(kind, q, k, v, ws, nheads), rtol=1e-11,
                               atol=1e-12)
    # README.md:114-118: softmax(similarity(q/sqrt(t), k/sqrt(t))) ⊗ v == y
    qf, kf, vf = (O._flat(a, nheads) for a in (q, k, v))
    t = np.sqrt(qf.shape[1])
    S = O.similarity(kind, qf / np.sqrt(t), kf / np.sqrt(t), dims, ws)
    u = O.apply(O.softmax(S, ws ** len(dims)), vf, dims, ws)
    np.testing.assert_allclose(u.reshape(y.shape), y, rtol=1e-12, atol=1e-13)
    # lse of the scaled similarity
    lse = O.attention_lse(kind, q, k, ws, nheads)
    K = ws ** len(dims)
    Sd = O.similarity(kind, qf, kf, dims, ws, 1 / np.sqrt(qf.shape[1])).reshape(-1, K)
    np.testing.assert_allclose(np.exp(Sd - lse.reshape(-1, 1)), A.reshape(-1, K), rtol=1e-12)


# ---------------------------------------------------------------------------
# backward vs central finite differences
# ---------------------------------------------------------------------------

def fd_grads(kind, q, k, v, dy, ws, nheads, h=1e-6, trans=False):
    def loss(qq, kk, vv):
        y, _ = O.attention_fwd(kind, qq, kk, vv, ws, nheads, trans=trans)
        return np.sum(np.real(y * np.conj(dy)))

    grads = []
    for which in range(3):
        args = [q.copy(), k.copy(), v.copy()]
        g = np.zeros_like(args[which])
        flat = args[which].reshape(-1)
        gflat = g.reshape(-1)
        comps = [1.0, 1j] if np.iscomplexobj(flat) else [1.0]
        for i in range(flat.size):
            for unit in comps:
                old = flat[i]
                flat[i] = old + h * unit
                lp = loss(*args)
                flat[i] = old - h * unit
                lm = loss(*args)
                flat[i] = old
                gflat[i] += (lp - lm) / (2 * h) * unit
        grads.append(g)
    return grads


FD_CASES = [((5,), 3, 1), ((4, 3), 3, 1), ((3, 3), 5, 2), ((6,), 5, 2)]


@pytest.mark.parametrize("dims,ws,nheads", FD_CASES)
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [O.DOT, O.DISTANCE])
def test_attention_bwd_fd(dims, ws, nheads, cplx, kind):
    B, C = 2, 2 * nheads
    shape = (B, C, *reversed(dims))
    q, k, v, dy = (rand_signal(shape, cplx) for _ in range(4))
    dq, dk, dv = O.attention_bwd(kind, q, k, v, dy, ws, nheads)
    fq, fk, fv = fd_grads(kind, q, k, v, dy, ws, nheads)
    for got, ref in ((dq, fq), (dk, fk), (dv, fv)):
        np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-7)


# (the plain attention's finite-difference test above also covers the 3x3
# image at ws 5 with two heads, which takes 20 s per case)
@pytest.mark.parametrize("dims,ws,nheads", [((4, 3), 3, 1), ((5,), 3, 2)])
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [O.DOT, O.DISTANCE])
def test_transposed_attention_bwd_fd(dims, ws, nheads, cplx, kind):
    """y = Aᵀ ⊗ v of the adjacency (circulant_transposed_attention and its
    multi-head form, src/attention.jl:72-80, 98-103): the rrule of
    src/rrules.jl:74-88 (dA = sim_Dot(v, dy), dv = A ⊠ dy) composed with the
    softmax and similarity pullbacks, against central finite differences; the
    plain apply's pullback (dA = sim_Dot(dy, v)) in its place fails."""
    B, C = 2, 2 * nheads
    shape = (B, C, *reversed(dims))
    q, k, v, dy = (rand_signal(shape, cplx) for _ in range(4))
    got = O.attention_bwd(kind, q, k, v, dy, ws, nheads, trans=True)
    ref = fd_grads(kind, q, k, v, dy, ws, nheads, trans=True)
    for a, b in zip(got, ref):
        np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-7)
    wrong = O.attention_bwd(kind, q, k, v, dy, ws, nheads, trans=False)
    assert max(np.max(np.abs(a - b)) for a, b in zip(wrong, ref)) > 1e-3


@pytest.mark.parametrize("dims,ws,nheads", [((4, 3), 3, 1), ((6,), 5, 2)])
@pytest.mark.parametrize("cplx", [False, True])
@pytest.mark.parametrize("kind", [O.DOT, O.DISTANCE])
def test_attention_bwd_with_A_cotangent_fd(dims, ws, nheads, cplx, kind):
    """A loss on both outputs (y, A) of circulant_attention (src/attention.jl:19-25):
    L = Re<y, dy> + <A_nz, G>, against central finite differences."""
    B, C = 2, 2 * nheads
    shape = (B, C, *reversed(dims))
    q, k, v, dy = (rand_signal(shape, cplx) for _ in range(4))
    _, A0 = O.attention_fwd(kind, q, k, v, ws, nheads)
    G = np.random.default_rng(77).standard_normal(A0.shape)

    def loss(qq, kk, vv):
        y, A = O.attention_fwd(kind, qq, kk, vv, ws, nheads)
        return np.sum(np.real(y * np.conj(dy))) + np.sum(A * G)

    got = O.attention_bwd(kind, q, k, v, dy, ws, nheads, dA_out=G)
    h = 1e-6
    for which, g_got in enumerate(got):
        args = [q.copy(), k.copy(), v.copy()]
        flat = args[which].reshape(-1)
        ref = np.zeros_like(flat)
        for i in range(flat.size):
            for unit in ([1.0, 1j] if np.iscomplexobj(flat) else [1.0]):
                old = flat[i]
                flat[i] = old + h * unit
                lp = loss(*args)
                flat[i] = old - h * unit
                lm = loss(*args)
                flat[i] = old
                ref[i] += (lp - lm) / (2 * h) * unit
        np.testing.assert_allclose(g_got.reshape(-1), ref, rtol=1e-6, atol=1e-7)
    # the A term matters: without it the gradients differ
    plain = O.attention_bwd(kind, q, k, v, dy, ws, nheads)
    assert max(np.max(np.abs(a - b)) for a, b in zip(plain[:2], got[:2])) > 1e-3


def _dk_without_distance_correction(q, k, v, dy, ws):
    """A planted mistake: the Distance rrule's colsum(dS) .* k term dropped
    (the Dot pullback applied to a Distance forward).  The rowsum term of dq
    is no test: softmax's pullback makes every row of dS sum to zero."""
    dims = O.spatial_dims(q)
    K = ws ** len(dims)
    _, A = O.attention_fwd(O.DISTANCE, q, k, v, ws)
    qf, kf, vf, dyf = (O._flat(a) for a in (q, k, v, dy))
    s4 = qf.shape[1] ** -0.25
    dA = O.similarity(O.DOT, dyf, vf, dims, ws)
    dS = O.softmax_bwd(A, dA, K)
    assert np.max(np.abs(O.rowsum(dS, int(np.prod(dims)), K))) < 1e-12
    return (O.apply(dS, qf * s4, dims, ws, trans=True) * s4).reshape(k.shape)


def test_fd_catches_planted_mistakes():
    dims, ws = (4, 3), 3
    shape = (1, 2, *reversed(dims))
    q, k, v, dy = (rand_signal(shape, False) for _ in range(4))
    fq, fk, fv = fd_grads(O.DISTANCE, q, k, v, dy, ws, 1)
    bad = _dk_without_distance_correction(q, k, v, dy, ws)
    assert np.max(np.abs(bad - fk)) > 1e-3
    # transposed operand: dv computed with A instead of Aᵀ
    _, A = O.attention_fwd(O.DISTANCE, q, k, v, ws)
    bad_dv = O.apply(A, O._flat(dy), dims, ws, trans=False).reshape(v.shape)
    assert np.max(np.abs(bad_dv - fv)) > 1e-3
    # a wrong sign on the similarity scale fails the dense forward check
    y_bad, _ = O.attention_fwd(O.DOT, -q, k, v, ws)
    assert np.max(np.abs(y_bad - dense_attention(O.DOT, q, k, v, ws, 1))) > 1e-3


def test_mh_attention_heads_are_independent():
    """Head g of batch b is flattened batch g + nheads*b (src/attention.jl:44):
    running each head's channels alone gives the same per-head output."""
    dims, ws, nheads = (6, 4), 3, 2
    q, k, v = (rand_signal((2, 4, 4, 6), False) for _ in range(3))
    y, _ = O.attention_fwd(O.DOT, q, k, v, ws, nheads)
    for g in range(nheads):
        sl = slice(2 * g, 2 * g + 2)
        yg, _ = O.attention_fwd(O.DOT, q[:, sl], k[:, sl], v[:, sl], ws, 1)
        np.testing.assert_allclose(y[:, sl], yg, rtol=1e-13, atol=1e-14)
