"""Error bars for inputs whose scores are large (test infrastructure).

With q and k scaled or offset far from N(0,1) the scores reach 1e3 and more,
and a Float32 softmax is ill-conditioned whatever the arithmetic: the float64
gradients can be exactly zero (one-hot rows) while any Float32 computation of
them commits rounding errors of the order of its summed terms.  The bar used
there is, per output (y, dq, dk, dv), 8x the larger of

  * the error of a Float32 flash-style restatement of the same composition
    (``oracle.attention_flash_f32``: lse kept per row, S recomputed with its
    own rounding in the backward, P = exp(S - lse) clamped to 1), and
  * the unit roundoff 2^-24 times the magnitude of the terms the output sums
    (``oracle.attention_term_scales``),

and never below the usual tolerance.  Errors are compared as max-norm absolute
errors, so that a reference which is exactly zero stays meaningful.

For Distance the factor is 16: the restatement forms -|q - k|^2 / 2 from the
differences, as the reference does, while the fused kernels expand it into
three Float32 terms, q.k - |k|^2 / 2 - |q|^2 / 2, each as large as the score
itself when q and k are scaled (not offset) far from N(0,1): measured on
MI355X at q, k x 1e2 the kernels' error is 10-12x the restatement's there.
A wrong slow-walk unscale is off by orders of magnitude more under either
factor (tests/test_split_model.py).
"""
from __future__ import annotations

import numpy as np

from conftest import TOL_FWD, TOL_GRAD

import oracle as O  # noqa: E402

U32 = 2.0 ** -24


def abs_err(out, ref):
    out = np.asarray(out)
    ref = np.asarray(ref)
    dt = np.complex128 if (np.iscomplexobj(out) or np.iscomplexobj(ref)) else np.float64
    return float(np.max(np.abs(out.astype(dt) - ref.astype(dt)))) if ref.size else 0.0


def flash_bounds(kind, q, k, v, dy, ws, nheads, refs):
    """Absolute error bars for (y, dq, dk, dv) against the float64 refs."""
    fl = O.attention_flash_f32(kind, q, k, v, dy, ws, nheads)
    ts = O.attention_term_scales(kind, q, k, v, dy, ws, nheads)
    factor = 16.0 if kind == O.DISTANCE else 8.0
    out = []
    for i, (f, r, t) in enumerate(zip(fl, refs, ts)):
        tol = (TOL_FWD if i == 0 else TOL_GRAD) * float(np.max(np.abs(r)))
        out.append(max(tol, factor * max(abs_err(np.asarray(f).reshape(np.shape(r)), r), U32 * t)))
    return out
