"""Numerical model of the split-half fused kernels (csrc/fused2h_impl.h),
test infrastructure only.

The kernels carry every Float32 operand x of a matrix product as two f16
halves, hi = f16(x) and lo = f16(x - hi), and take a product on the f16
matrix cores with Float32 accumulation:
  * score-type products (contraction over channels: q.k, dy.v) take all four
    terms hi.hi + hi.lo + lo.hi + lo.lo, i.e. the product of the two
    represented values hi + lo;
  * apply-type products (contraction over keys: P.v, dS.k, dS.q, P.dy) take
    hi.hi + hi.lo + lo.hi, without lo.lo.
f16 has a 5-bit exponent: lo turns subnormal (fixed spacing 2^-24) once
|x| < 2^-3, and every half overflows at 65520.  To keep FP32's range the
kernels scale operands by powers of two before the split (exact) and undo the
scale on the Float32 results.  This module restates that arithmetic in numpy
(float16 rounding is numpy's round-to-nearest-even with subnormals, as the
hardware's conversions; products of halves are exact in float64, and the
float64 sums stand in for the kernels' Float32 accumulation) so that the
scaling rules can be checked against the float64 oracle at any magnitude on
the CPU.

``scaled=False`` models the kernels without scaling (every shift 0).

Scaling rules (one tile of query pixels and its halo of key pixels; here the
whole image, which the halo covers for the windows used in the tests):
  * an operand staged for the whole tile (the halo tensors and, in the
    key-centric pass, v) gets one shift s from the maximum magnitude over what
    is staged: s = 0 when that maximum lies in [2^-2, 2^5), else the shift
    that brings it into [4, 8);
  * the register operand of a score product absorbs its partner's shift:
    q' = q * c2 * 2^-s_k (c2 = log2(e)/sqrt(dh)), so scores keep their
    scale; if some |q'| reaches 2^15 (both operands large) the score product
    is taken with q normalised per pixel and the score unscaled after the
    product (the kernels' slow path);
  * dy in the query-centric pass is normalised per pixel (same window rule).

Distance similarity is formed by expansion, -|q-k|^2/2 = q.k - |k|^2/2 -
|q|^2/2, with -|k|^2/2 a per-key bias in the score product's initial
accumulator and -|q|^2/2 folded into the row's lse.  Each pass first centres
both operands on one pixel of the item's keys (q - mu, k - mu; the kernels
take mu = k at the tile's first pixel): |q-k|^2 is unchanged, but the
expansion's terms then scale with the spread of the data instead of its
offset.  Uncentred, the Float32 roundings of the bias, of the accumulated
score and of the stored lse (``f32acc``, modelled as one rounding each) and
the halves' 2^-22 per operand grow with |q||k|, which at q, k = N(0,1) + 10
already exceeds the tolerances.  ``centre_px`` gives the centre pixel of the
forward, query-centric and key-centric passes (different per pass, as in the
kernels, whose tiles differ: the stored lse is the centre-independent
log-sum-exp of the true scores); None models the kernels before centring.
"""
from __future__ import annotations

import math

import numpy as np

LOG2E = 1.0 / math.log(2.0)
LN2 = math.log(2.0)
F16_LIMIT = 2.0 ** 15


def split(x):
    """(hi, lo) of float32 values as float64 copies of their f16 halves."""
    x = np.asarray(x, np.float32)
    hi = x.astype(np.float16)
    lo = (x - hi.astype(np.float32)).astype(np.float16)
    return hi.astype(np.float64), lo.astype(np.float64)


def rep(x):
    """The value a split operand represents, hi + lo."""
    hi, lo = split(x)
    return hi + lo


def shift_of(maxabs, keep=True):
    """Power-of-two shift for an operand whose largest magnitude is maxabs:
    0 inside [2^-2, 2^5) (with keep), else the shift to [4, 8)."""
    m = float(maxabs)
    if m == 0.0 or not math.isfinite(m):
        return 0
    e = math.frexp(m)[1]  # m in [2^(e-1), 2^e)
    if keep and -1 <= e <= 5:
        return 0
    return 3 - e


def ldexp(x, s):
    return np.ldexp(np.asarray(x, np.float64), s)


def f32(x):
    return np.asarray(x, np.float32)


def window_cols(dims, ws):
    """(P, K) 0-based key pixels of every query pixel's window."""
    import oracle as O
    _, colval = O.pattern(dims, ws, 1)
    P = int(np.prod(dims))
    return colval.reshape(P, -1).astype(np.int64) - 1


def score(a, b, cols):
    """Score-type product: sum_m rep(a[m, r]) * rep(b[m, cols[r, t]]) -> (P, K)."""
    ra, rb = rep(a), rep(b)
    return np.einsum("mr,mrt->rt", ra, rb[:, cols])


def apply_rows(x, w, cols, trans=False):
    """Apply-type product without lo.lo: out[m, r] = sum_t x[m, c] w[r, t]
    (c = cols[r, t]); trans scatters to c instead (out[m, c] += x[m, r] w)."""
    xh, xl = split(x)
    wh, wl = split(w)
    wrep = wh + wl
    if not trans:
        return (np.einsum("mrt,rt->mr", (xh + xl)[:, cols], wrep)
                - np.einsum("mrt,rt->mr", xl[:, cols], wl))
    P = w.shape[0]
    out = np.zeros((x.shape[0], P))
    full = np.einsum("mr,rt->mrt", xh + xl, wrep) - np.einsum("mr,rt->mrt", xl, wl)
    for t in range(cols.shape[1]):
        np.add.at(out.T, cols[:, t], full[:, :, t].T)
    return out


def _pixel_shifts(x, keep=True):
    return np.array([shift_of(np.max(np.abs(x[:, r])), keep) for r in range(x.shape[1])])


def _scores(qs, kx, c2, sk, cols, init, slow_ok=True, lim=F16_LIMIT, slow_sign=1):
    """Scores in log2 units of register operand qs (raw) against staged kx
    (already shifted by sk).  Fast path q' = q c2 2^-sk; a pixel whose |q'|
    reaches lim takes the slow path: q c2 normalised per pixel to [4, 8) and
    the product unscaled by 2^-(shift + sk) (``slow_sign`` = -1 flips that
    unscale, a planted mistake).  Returns (scores, per-pixel slow flags)."""
    qp = f32(qs * c2 * 2.0 ** -sk)
    fast = score(qp, kx, cols) + init
    big = np.max(np.abs(qp), axis=0) >= lim if slow_ok else np.zeros(qs.shape[1], bool)
    if not big.any():
        return fast, big
    sq = _pixel_shifts(qs * c2, keep=False)
    qn = f32(ldexp(qs * c2, sq[None, :]))
    slow = ldexp(score(qn, kx, cols), -slow_sign * (sq[:, None] + sk)) + init
    return np.where(big[:, None], slow, fast), big


def bwd_lim(kx):
    """The backward passes' slow-walk threshold on |q'|: 2^15, or lower so
    that scores stay below 2^20 (|kx| < 2^e gives 2^(16 - e))."""
    m = float(np.max(np.abs(kx)))
    e = math.frexp(m)[1] if m > 0 else -126
    return min(F16_LIMIT, 2.0 ** (16 - e))


def _centred(x, mu):
    """x - mu per component, rounded to float32 as the kernels subtract."""
    return f32(x.astype(np.float32) - mu.astype(np.float32)[:, None])


def _r32(x, on):
    return np.asarray(x, np.float32).astype(np.float64) if on else np.asarray(x, np.float64)


def fused_fwd(kind, q, k, v, ws, dims, scaled=True, centre_px=(0, 1, 2), f32acc=True,
              slow_sign=1):
    """y (dh, P) and lse (P,) of one unit; q, k, v: (dh, P) float32 values."""
    dh, P = q.shape
    cols = window_cols(dims, ws)
    scale = 1.0 / math.sqrt(dh)
    c2 = scale * LOG2E
    if kind == 1 and centre_px is not None:
        mu = k[:, centre_px[0]].copy()
        q, k = _centred(q, mu), _centred(k, mu)
    sk = shift_of(np.max(np.abs(k))) if scaled else 0
    sv = shift_of(np.max(np.abs(v))) if scaled else 0
    kx, vx = f32(ldexp(k, sk)), f32(ldexp(v, sv))
    if kind == 1:
        n2 = _r32(np.sum(k.astype(np.float64) ** 2, axis=0), f32acc)
        kb = _r32(-0.5 * c2 * n2, f32acc)
    else:
        kb = np.zeros(P)
    s, _ = _scores(q, kx, c2, sk, cols, kb[cols], slow_ok=scaled, slow_sign=slow_sign)
    s = _r32(s, f32acc)
    m = s.max(axis=1, keepdims=True)
    p = np.exp2(s - m)
    l = p.sum(axis=1)
    y = ldexp(apply_rows(vx, p, cols) / l[None, :], -sv)
    lse = _r32((m[:, 0] + np.log2(l)) * LN2, f32acc)
    if kind == 1:
        sq = _r32(np.sum(q.astype(np.float64) ** 2, axis=0), f32acc)
        lse = lse - _r32(0.5 * scale * sq, f32acc)
    return y, _r32(lse, f32acc)


def fused_bwd(kind, q, k, v, y, dy, lse, ws, dims, scaled=True, centre_px=(0, 1, 2),
              f32acc=True, slow_sign=1):
    """(dq, dk, dv) of one unit as the two backward passes compute them."""
    dh, P = q.shape
    cols = window_cols(dims, ws)
    scale = 1.0 / math.sqrt(dh)
    c2 = scale * LOG2E
    D = np.sum(dy.astype(np.float64) * y.astype(np.float64), axis=0)
    dist = kind == 1
    lse = np.asarray(lse, np.float64)

    def centred(px):
        if not dist or centre_px is None:
            return q, k
        mu = k[:, px].copy()
        return _centred(q, mu), _centred(k, mu)

    def norms(qc, kc):
        return (_r32(np.sum(qc.astype(np.float64) ** 2, axis=0), f32acc),
                _r32(np.sum(kc.astype(np.float64) ** 2, axis=0), f32acc))

    # query-centric pass: staged k, v; registers q, dy
    qc, kc = centred(centre_px[1] if centre_px is not None else 0)
    q2, k2 = norms(qc, kc)
    sk = shift_of(np.max(np.abs(kc))) if scaled else 0
    sv = shift_of(np.max(np.abs(v))) if scaled else 0
    sd = _pixel_shifts(dy) if scaled else np.zeros(P, int)
    kx, vx = f32(ldexp(kc, sk)), f32(ldexp(v, sv))
    dyx = f32(ldexp(dy, sd[None, :]))
    rowt = _r32(-lse * LOG2E - (0.5 * c2 * q2 if dist else 0.0), f32acc)
    init = rowt[:, None] + (_r32(-0.5 * c2 * k2, f32acc)[cols] if dist else 0.0)
    s, slow = _scores(qc, kx, c2, sk, cols, init, slow_ok=scaled, lim=bwd_lim(kx),
                      slow_sign=slow_sign)
    s = _r32(s, f32acc)
    p = np.exp2(np.where(slow[:, None], np.minimum(s, 0.0), s))
    dp = score(dyx, vx, cols) - ldexp(D, sd + sv)[:, None]
    ds = f32(p * dp)
    acc = apply_rows(kx, ds, cols)
    dq = ldexp(acc, -(sd + sv + sk)[None, :])
    if dist:
        dq = dq - ldexp(ds.astype(np.float64).sum(axis=1), -(sd + sv))[None, :] * qc
    dq = dq * scale

    # key-centric pass: staged q, dy; registers k, v (v shifted as a whole)
    qc, kc = centred(centre_px[2] if centre_px is not None else 0)
    q2, k2 = norms(qc, kc)
    sq = shift_of(np.max(np.abs(qc))) if scaled else 0
    sd2 = shift_of(np.max(np.abs(dy))) if scaled else 0
    sv2 = shift_of(np.max(np.abs(v))) if scaled else 0
    qx, dyx2 = f32(ldexp(qc, sq)), f32(ldexp(dy, sd2))
    vr = f32(ldexp(v, sv2))
    # the window is symmetric: the queries whose windows hold key c are the
    # keys of c's own window, cols[c]
    colt = _r32(-lse * LOG2E - (0.5 * c2 * q2 if dist else 0.0), f32acc)
    init = colt[cols] + (_r32(-0.5 * c2 * k2, f32acc)[:, None] if dist else 0.0)
    s, slow = _scores(kc, qx, c2, sq, cols, init, slow_ok=scaled, lim=bwd_lim(qx),
                      slow_sign=slow_sign)
    s = _r32(s, f32acc)
    p = np.exp2(np.where(slow[:, None], np.minimum(s, 0.0), s))
    dp = score(vr, dyx2, cols) - ldexp(D, sv2 + sd2)[cols]
    ds = f32(p * dp)
    acc0 = apply_rows(qx, ds, cols)
    acc1 = apply_rows(dyx2, f32(p), cols)
    dk = ldexp(acc0, -(sv2 + sd2 + sq))
    if dist:
        dk = dk - ldexp(ds.astype(np.float64).sum(axis=1), -(sv2 + sd2))[None, :] * kc
    dk = dk * scale
    dv = ldexp(acc1, -sd2)
    return dq, dk, dv
