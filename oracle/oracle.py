"""CPU oracle for the circulant attention path (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this module, and only as the checker or the baseline.  The
product (``circulantattention.jl_amd``) never imports it.

Primitives are the C restatement in ``circatt_oracle.c`` (float64 build for
parity, float32 build for the CPU baseline); the compositions below restate
``src/attention.jl`` and ``src/rrules.jl`` of the reference step by step.

Array convention (memory order identical to the reference's Julia arrays):
a Julia array of size ``(N1, N2, C, B)`` is a numpy array of shape
``(B, C, N2, N1)``; the pixel index is ``r = i1 + N1*i2``.  Internally
signals are handled as ``(nb, C, P)``.  Complex signals are numpy complex
arrays; the C code sees them as interleaved (re, im) pairs.
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_BUILD = os.path.join(_HERE, "_build")

DOT = 0
DISTANCE = 1


def build() -> None:
    """Compile the C restatement (both precisions) with the committed Makefile."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)


_LIBS: dict = {}


def _lib(precision: str = "f64"):
    if precision in _LIBS:
        return _LIBS[precision]
    path = os.path.join(_BUILD, f"liboracle_{precision}.so")
    if not os.path.exists(path):
        build()
    lib = ctypes.CDLL(path)
    real = ctypes.c_double if precision == "f64" else ctypes.c_float
    P = ctypes.c_void_p
    i64 = ctypes.c_int64
    lib.oc_pattern.argtypes = [ctypes.c_int, i64, i64, i64, i64, P, P]
    lib.oc_pattern.restype = ctypes.c_int
    lib.oc_cartesian_circulant_1d.argtypes = [i64, i64, i64, P, P]
    lib.oc_cartesian_circulant_2d.argtypes = [i64, i64, i64, i64, P, P]
    lib.oc_similarity.argtypes = [ctypes.c_int, ctypes.c_int, i64, i64, i64, i64, P, real, P, P, P]
    lib.oc_softmax.argtypes = [i64, i64, P, P]
    lib.oc_softmax_bwd.argtypes = [i64, i64, P, P, P]
    lib.oc_apply.argtypes = [ctypes.c_int, ctypes.c_int, i64, i64, i64, i64, P, P, P, P]
    lib.oc_rowsum.argtypes = [i64, i64, i64, P, P]
    lib.oc_colsum.argtypes = [i64, i64, i64, P, P, P]
    _LIBS[precision] = lib
    return lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _real_dtype(precision):
    return np.float64 if precision == "f64" else np.float32


def _as_real_view(x: np.ndarray, precision: str):
    """Return (contiguous real array, ncomp) for a real or complex signal."""
    rd = _real_dtype(precision)
    if np.iscomplexobj(x):
        cd = np.complex128 if precision == "f64" else np.complex64
        xc = np.ascontiguousarray(x, dtype=cd)
        return xc.view(rd), 2, xc
    xr = np.ascontiguousarray(x, dtype=rd)
    return xr, 1, xr


def geometry(dims, ws):
    """(nsp, n1, n2, P, K) for spatial dims given fastest-first (N1[, N2])."""
    dims = tuple(int(d) for d in dims)
    if len(dims) == 1:
        return 1, dims[0], 1, dims[0], ws
    if len(dims) == 2:
        return 2, dims[0], dims[1], dims[0] * dims[1], ws * ws
    raise ValueError("only 1 or 2 spatial dims")


def cartesian_circulant(n, dims, ws):
    """1-based (i, j) of CSR slot n, literal src/circulant.jl:6-44."""
    lib = _lib()
    i = ctypes.c_int64()
    j = ctypes.c_int64()
    if len(dims) == 1:
        lib.oc_cartesian_circulant_1d(n, dims[0], ws, ctypes.byref(i), ctypes.byref(j))
    else:
        lib.oc_cartesian_circulant_2d(n, dims[0], dims[1], ws, ctypes.byref(i), ctypes.byref(j))
    return i.value, j.value


def pattern(dims, ws, nb=1):
    """rowptr (nb, P+1), colval (nb, P*K), Int32 1-based (src/circulant.jl:64-106,
    src/array.jl:6-11)."""
    nsp, n1, n2, P, K = geometry(dims, ws)
    rowptr = np.empty((nb, P + 1), np.int32)
    colval = np.empty((nb, P * K), np.int32)
    rc = _lib().oc_pattern(nsp, n1, n2, ws, nb, _ptr(rowptr), _ptr(colval))
    if rc != 0:
        raise ValueError(f"filter size M={ws} must be odd.")
    return rowptr, colval


def similarity(kind, x, y, dims, ws, scale=1.0, precision="f64"):
    """nzVal (nb, P*K) of circulant_similarity(kind, x, y, ws) * scale.

    x, y: (nb, C, P) real or complex.  src/similarity.jl:55-103, 138-142.
    """
    nsp, n1, n2, P, K = geometry(dims, ws)
    nb, C = x.shape[0], x.shape[1]
    _, colval = pattern(dims, ws, 1)
    xr, ncomp, _kx = _as_real_view(x, precision)
    yr, _, _ky = _as_real_view(y, precision)
    nz = np.empty((nb, P * K), _real_dtype(precision))
    _lib(precision).oc_similarity(kind, ncomp, P, C, nb, K, _ptr(colval), scale, _ptr(xr),
                                  _ptr(yr), _ptr(nz))
    return nz


def softmax(nz, K, precision="f64"):
    """Row softmax of nzVal over each row's K slots (src/similarity.jl:105-126)."""
    a = np.ascontiguousarray(nz, _real_dtype(precision))
    out = np.empty_like(a)
    _lib(precision).oc_softmax(K, a.size // K, _ptr(a), _ptr(out))
    return out


def softmax_bwd(A, dA, K, precision="f64"):
    """NNlib.∇softmax_data on nzVal (src/rrules.jl:42-56)."""
    a = np.ascontiguousarray(A, _real_dtype(precision))
    da = np.ascontiguousarray(dA, _real_dtype(precision))
    ds = np.empty_like(a)
    _lib(precision).oc_softmax_bwd(K, a.size // K, _ptr(a), _ptr(da), _ptr(ds))
    return ds


def apply(nz, x, dims, ws, trans=False, precision="f64"):
    """A ⊗ x (trans=False) or Aᵀ ⊗ x (trans=True); x (nb, C, P) real or complex.

    CSR SpMM of src/batchedmul.jl:82-110 called from src/attention.jl:53-80.
    """
    nsp, n1, n2, P, K = geometry(dims, ws)
    nb, C = x.shape[0], x.shape[1]
    _, colval = pattern(dims, ws, 1)
    xr, ncomp, xkeep = _as_real_view(x, precision)
    a = np.ascontiguousarray(nz, _real_dtype(precision))
    y = np.empty_like(xkeep)
    yr = y.view(_real_dtype(precision)) if ncomp == 2 else y
    _lib(precision).oc_apply(1 if trans else 0, ncomp, P, C, nb, K, _ptr(colval), _ptr(a),
                             _ptr(xr), _ptr(yr))
    return y


def rowsum(nz, P, K, precision="f64"):
    """sum(A; dims=2) as (nb, P) (src/array.jl:126-130)."""
    a = np.ascontiguousarray(nz, _real_dtype(precision))
    nb = a.size // (P * K)
    out = np.empty((nb, P), _real_dtype(precision))
    _lib(precision).oc_rowsum(P, K, nb, _ptr(a), _ptr(out))
    return out


def colsum(nz, dims, ws, precision="f64"):
    """sum(A; dims=1) as (nb, P) (src/array.jl:119-124)."""
    nsp, n1, n2, P, K = geometry(dims, ws)
    a = np.ascontiguousarray(nz, _real_dtype(precision))
    nb = a.size // (P * K)
    _, colval = pattern(dims, ws, 1)
    out = np.empty((nb, P), _real_dtype(precision))
    _lib(precision).oc_colsum(P, K, nb, _ptr(colval), _ptr(a), _ptr(out))
    return out


# ---------------------------------------------------------------------------
# Compositions: src/attention.jl and src/rrules.jl
# ---------------------------------------------------------------------------

def _flat(x, nheads=1):
    """(B, C, *spatial) -> (nb=nheads*B, C/nheads, P): splitheads
    (src/attention.jl:44): head g uses channels g*dh .. (g+1)*dh-1 and the
    flattened batch index is g + nheads*b."""
    B, C = x.shape[0], x.shape[1]
    P = int(np.prod(x.shape[2:]))
    return x.reshape(B * nheads, C // nheads, P)


def spatial_dims(x):
    """Fastest-first spatial dims (N1[, N2]) of a (B, C, [N2,] N1) array."""
    return tuple(reversed(x.shape[2:]))


def attention_fwd(kind, q, k, v, ws, nheads=1, precision="f64", trans=False):
    """y, A_nz of circulant_attention (src/attention.jl:19-26) or, for
    nheads > 1, of circulant_mh_attention's per-head computation
    (src/attention.jl:38-42).  tau = sqrt(channels per head); q and k are each
    divided by sqrt(tau), so S(q,k) is scaled by 1/sqrt(dh).  trans: y is the
    transposed apply Aᵀ ⊗ v of the same adjacency
    (circulant_transposed_attention / circulant_mh_transposed_attention,
    src/attention.jl:72-80, 98-103)."""
    dims = spatial_dims(q)
    nsp, n1, n2, P, K = geometry(dims, ws)
    qf, kf, vf = (_flat(a, nheads) for a in (q, k, v))
    dh = qf.shape[1]
    scale = 1.0 / math.sqrt(dh)
    S = similarity(kind, qf, kf, dims, ws, scale, precision)
    A = softmax(S, K, precision)
    y = apply(A, vf, dims, ws, trans, precision)
    return y.reshape(q.shape), A


def attention_bwd(kind, q, k, v, dy, ws, nheads=1, precision="f64", A=None, dA_out=None,
                  trans=False):
    """(dq, dk, dv) for the composition adjacency -> ⊗ (the path
    test/grad.jl:17-21 differentiates) with the rrules of src/rrules.jl:
      ⊗ (:58-72):        dA = sim_Dot(dy, v), dv = Aᵀ ⊠ dy
                         (+ dA_out, a cotangent on the returned A, shaped
                         like A_nz: circulant_attention returns (y, A),
                         src/attention.jl:19-25, and both can enter a loss)
      softmax (:42-56):  dS = A ∘ (dA - rowsum(A ∘ dA))
      Dot (:18-32):      dq̃ = dS ⊠ k̃, dk̃ = dSᵀ ⊠ q̃
      Distance (:1-16):  dq̃ = dS ⊠ k̃ - rowsum(dS)∘q̃, dk̃ = dSᵀ ⊠ q̃ - colsum(dS)∘k̃
      q̃ = q/sqrt(tau) (src/attention.jl:21):  dq = dq̃/sqrt(tau), same for k.
    trans (y = Aᵀ ⊗ v, the rrule of src/rrules.jl:74-88):
                         dA = sim_Dot(v, dy), dv = A ⊠ dy.
    """
    dims = spatial_dims(q)
    nsp, n1, n2, P, K = geometry(dims, ws)
    qf, kf, vf, dyf = (_flat(a, nheads) for a in (q, k, v, dy))
    dh = qf.shape[1]
    s4 = dh ** -0.25  # 1/sqrt(tau), tau = sqrt(dh)
    if A is None:
        _, A = attention_fwd(kind, q, k, v, ws, nheads, precision)
    if trans:
        dA = similarity(DOT, vf, dyf, dims, ws, 1.0, precision)
    else:
        dA = similarity(DOT, dyf, vf, dims, ws, 1.0, precision)
    if dA_out is not None:
        dA = dA + np.asarray(dA_out, dA.dtype).reshape(dA.shape)
    dv = apply(A, dyf, dims, ws, not trans, precision)
    dS = softmax_bwd(A, dA, K, precision)
    qt, kt = qf * s4, kf * s4
    dqt = apply(dS, kt, dims, ws, False, precision)
    dkt = apply(dS, qt, dims, ws, True, precision)
    if kind == DISTANCE:
        rs = rowsum(dS, P, K, precision)
        cs = colsum(dS, dims, ws, precision)
        dqt = dqt - rs[:, None, :] * qt
        dkt = dkt - cs[:, None, :] * kt
    dq = (dqt * s4).reshape(q.shape)
    dk = (dkt * s4).reshape(k.shape)
    return dq, dk, dv.reshape(v.shape)


def attention_flash_f32(kind, q, k, v, dy, ws, nheads=1):
    """(y, dq, dk, dv) of a Float32 flash-style restatement of the same
    composition: the forward keeps only lse = m + log(sum exp(S - m)) per row
    (Float32) and the backward recomputes S (rounded on its own) and
    P = exp(S - lse) from it instead of reading the stored A, with D = <dy, y> for the softmax pullback
    (dS = P o (dP - D), the identity of src/rrules.jl:42-56 for a real A).
    S, the products and every reduction are Float32 (the oracle's float32
    build), so its error against the float64 oracle is what a Float32
    algorithm of this form incurs; the fused kernels are held to a multiple
    of it where the scores are large."""
    f = np.float32
    dims = spatial_dims(q)
    nsp, n1, n2, P, K = geometry(dims, ws)
    qf, kf, vf, dyf = (_flat(a, nheads) for a in (q, k, v, dy))
    nb, dh = qf.shape[0], qf.shape[1]
    S = similarity(kind, qf, kf, dims, ws, 1.0 / math.sqrt(dh), "f32").reshape(nb, P, K)
    m = S.max(axis=2, keepdims=True)
    l = np.exp(S - m, dtype=f).sum(axis=2, keepdims=True, dtype=f)
    lse = (m + np.log(l, dtype=f)).astype(f)
    A = (np.exp(S - m, dtype=f) / l).astype(f).reshape(nb, P * K)
    y = apply(A, vf, dims, ws, False, "f32")
    # the backward's own evaluation of S: the channel sums in reverse order,
    # so that it rounds independently of the forward's (as a backward pass
    # that recomputes the scores in its own products does)
    Sb = similarity(kind, qf[:, ::-1], kf[:, ::-1], dims, ws, 1.0 / math.sqrt(dh), "f32")
    # (p <= 1: lse bounds every score, but the two roundings need not agree)
    Pr = np.exp(np.minimum(Sb.reshape(nb, P, K) - lse, 0).astype(f), dtype=f).reshape(nb, P * K)
    dA = similarity(DOT, dyf, vf, dims, ws, 1.0, "f32")
    yd = (np.conj(y) if np.iscomplexobj(y) else y)
    D = np.real(np.sum(dyf.astype(y.dtype) * yd, axis=1, dtype=y.dtype)).astype(f)  # (nb, P)
    dS = (Pr.reshape(nb, P, K) * (dA.reshape(nb, P, K) - D[:, :, None])).astype(f)
    dS = dS.reshape(nb, P * K)
    dv = apply(Pr, dyf, dims, ws, True, "f32")
    s4 = f(dh ** -0.25)
    qt, kt = (qf * s4).astype(qf.dtype), (kf * s4).astype(kf.dtype)
    dqt = apply(dS, kt, dims, ws, False, "f32")
    dkt = apply(dS, qt, dims, ws, True, "f32")
    if kind == DISTANCE:
        dqt = dqt - rowsum(dS, P, K, "f32")[:, None, :] * qt
        dkt = dkt - colsum(dS, dims, ws, "f32")[:, None, :] * kt
    return (y.reshape(q.shape), (dqt * s4).reshape(q.shape), (dkt * s4).reshape(k.shape),
            dv.reshape(v.shape))


def attention_term_scales(kind, q, k, v, dy, ws, nheads=1):
    """Float64 magnitudes of the terms each output sums, one scalar per
    output (y, dq, dk, dv): max of A (x) |v|; of G (x) |k| (+ rowsum(G) |q|
    for Distance) scaled like dq, with G = A o (|dA| + |D|) bounding |dS|; the
    transposed forms for dk; A^T (x) |dy|.  A Float32 computation of an
    output commits rounding errors of the order of the unit roundoff times
    this scale, whatever the output's own size (a row whose softmax is one-hot
    has dS = 0 exactly, but its terms are not small)."""
    dims = spatial_dims(q)
    nsp, n1, n2, P, K = geometry(dims, ws)
    qf, kf, vf, dyf = (np.abs(_flat(a, nheads)).astype(np.float64) for a in (q, k, v, dy))
    dh = qf.shape[1]
    nb = qf.shape[0]
    _, A = attention_fwd(kind, q, k, v, ws, nheads)
    dA = similarity(DOT, _flat(dy, nheads), _flat(v, nheads), dims, ws, 1.0)
    D = np.sum((A * dA).reshape(nb, P, K), axis=2)
    G = (A.reshape(nb, P, K) * (np.abs(dA).reshape(nb, P, K) + np.abs(D)[:, :, None]))
    G = G.reshape(nb, P * K)
    s2 = 1.0 / math.sqrt(dh)
    ty = apply(A, vf, dims, ws, False)
    tq = apply(G, kf, dims, ws, False)
    tk = apply(G, qf, dims, ws, True)
    if kind == DISTANCE:
        tq = tq + rowsum(G, P, K)[:, None, :] * qf
        tk = tk + colsum(G, dims, ws)[:, None, :] * kf
    tv = apply(A, dyf, dims, ws, True)
    return float(ty.max()), float(tq.max() * s2), float(tk.max() * s2), float(tv.max())


def attention_lse(kind, q, k, ws, nheads=1):
    """Per-row log-sum-exp of the scaled similarity, (nb, P), float64."""
    dims = spatial_dims(q)
    nsp, n1, n2, P, K = geometry(dims, ws)
    qf, kf = _flat(q, nheads), _flat(k, nheads)
    S = similarity(kind, qf, kf, dims, ws, 1.0 / math.sqrt(qf.shape[1])).reshape(-1, P, K)
    m = S.max(axis=2, keepdims=True)
    return (m[..., 0] + np.log(np.exp(S - m).sum(axis=2))).reshape(qf.shape[0], P)


def axpby(alpha, X, beta, Y):
    """Z = alpha_b * X + beta_b * Y on nzVal (nb, nnz): src/array.jl:66-81,
    179-189 (+, -, c*X, scale by a (1,1,nh,B) array)."""
    a = np.asarray(alpha, np.float64).reshape(-1, 1)
    out = a * np.asarray(X, np.float64)
    if Y is not None:
        out = out + np.asarray(beta, np.float64).reshape(-1, 1) * np.asarray(Y, np.float64)
    return out
