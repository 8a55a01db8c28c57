"""torch.autograd.Functions over the libcircatt C ABI.

Each Function's forward calls one entry point and its backward restates the
matching ChainRules rrule of the reference (src/rrules.jl) with libcircatt
calls.  Tensors are device tensors in the reference's memory order: a Julia
signal of size (N1[, N2], C, nb) is a torch tensor (nb, C[, N2], N1); a
Circulant's nzVal (P*K, nb) is a tensor (nb, P, K).  torch provides device
memory and the current HIP stream only.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib as L


def stream_ptr(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def require(t: torch.Tensor, name: str):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must live on a HIP device (libcircatt has no CPU path)")
    if t.dtype not in (torch.float32, torch.complex64):
        raise TypeError(f"{name} must be float32 or complex64, got {t.dtype}")


def dtype_code(t: torch.Tensor) -> int:
    return L.C32 if t.is_complex() else L.F32


def geometry(spatial):
    """(nsp, n1, n2) for fastest-first spatial dims."""
    if len(spatial) == 1:
        return 1, spatial[0], 1
    if len(spatial) == 2:
        return 2, spatial[0], spatial[1]
    raise AssertionError(f"{len(spatial)} spatial dims; only 1 and 2 are supported")


def _c(t):
    return t.contiguous()


def similarity_raw(kind, x, y, spatial, ws, scale):
    """nzval (nb, P, K) = scale * sim(x, y); x, y: (nb, C, *spatial-reversed)."""
    nsp, n1, n2 = geometry(spatial)
    nb, C = x.shape[0], x.shape[1]
    P = int(math.prod(spatial))
    K = ws ** nsp
    nz = torch.empty((nb, P, K), dtype=torch.float32, device=x.device)
    L.check(L.lib.circatt_similarity(kind, dtype_code(x), nsp, n1, n2, ws, C, nb, scale,
                                     ptr(x), ptr(y), ptr(nz), stream_ptr(x.device)),
            "circatt_similarity")
    return nz


def apply_raw(nz, x, spatial, ws, trans):
    nsp, n1, n2 = geometry(spatial)
    nb, C = x.shape[0], x.shape[1]
    y = torch.empty_like(x)
    L.check(L.lib.circatt_apply(1 if trans else 0, dtype_code(x), nsp, n1, n2, ws, C, nb,
                                ptr(nz), ptr(x), ptr(y), stream_ptr(x.device)), "circatt_apply")
    return y


def axpby_raw(alpha, X, beta=None, Y=None, nb=1):
    """Z = alpha_b X + beta_b Y; alpha/beta are floats or (nb,) device tensors."""
    Z = torch.empty_like(X)
    nnz = X.numel() // nb
    a_t = alpha if isinstance(alpha, torch.Tensor) else None
    b_t = beta if isinstance(beta, torch.Tensor) else None
    a0 = 0.0 if a_t is not None else float(alpha)
    b0 = 0.0 if (b_t is not None or beta is None) else float(beta)
    L.check(L.lib.circatt_axpby(nnz, nb, ptr(a_t), a0, ptr(X), ptr(b_t), b0, ptr(Y), ptr(Z),
                                stream_ptr(X.device)), "circatt_axpby")
    return Z


def fill_raw(t, value):
    """t[...] = value (circatt_fill); t contiguous float32."""
    L.check(L.lib.circatt_fill(ptr(t), t.numel(), float(value), stream_ptr(t.device)),
            "circatt_fill")
    return t


def copy_blocks_raw(dst, src, block, ninner, dsi, ssi, nouter, dso, sso, dst_off=0, src_off=0):
    """Strided device block copy (circatt_copy_blocks); sizes, strides and
    offsets in bytes."""
    L.check(L.lib.circatt_copy_blocks(ctypes.c_void_p(dst.data_ptr() + dst_off),
                                      ctypes.c_void_p(src.data_ptr() + src_off), block, ninner,
                                      dsi, ssi, nouter, dso, sso, stream_ptr(dst.device)),
            "circatt_copy_blocks")
    return dst


def replicate_raw(x, inner, r, outer):
    """x viewed as (outer, inner) -> (outer, r, inner): every inner block
    repeated r times (repeat or broadcast over one batch dim)."""
    x = _c(x)
    out = torch.empty((outer, r, inner), dtype=x.dtype, device=x.device)
    es = x.element_size()
    return copy_blocks_raw(out, x, inner * es, r, inner * es, 0, outer, r * inner * es, inner * es)


def sum_middle_raw(x, inner, nsum, outer):
    """x viewed as (outer, nsum, inner) -> (outer, inner), summed over nsum
    (circatt_sum_middle, double accumulation in order)."""
    x = _c(x)
    out = torch.empty((outer, inner), dtype=torch.float32, device=x.device)
    L.check(L.lib.circatt_sum_middle(ptr(x), ptr(out), inner, nsum, outer, stream_ptr(x.device)),
            "circatt_sum_middle")
    return out


def count_unequal(a, b, floats=True):
    """Number of positions where a and b differ (circatt_count_unequal),
    read back to the host."""
    a, b = _c(a), _c(b)
    cnt = torch.empty((1,), dtype=torch.int64, device=a.device)
    L.check(L.lib.circatt_count_unequal(1 if floats else 0, a.numel(), ptr(a), ptr(b), ptr(cnt),
                                        stream_ptr(a.device)), "circatt_count_unequal")
    return int(cnt.item())


class ReplicateFn(torch.autograd.Function):
    """(outer, inner) -> (outer, r, inner): repeat(A, 1, 1, ...) over one batch
    dim (src/array.jl:9,49-52) and the broadcasts of scale (src/array.jl:179-186);
    pullback: the sum over the r copies."""

    @staticmethod
    def forward(ctx, x, inner, r, outer):
        ctx.meta = (inner, r, outer, x.shape)
        return replicate_raw(x, inner, r, outer)

    @staticmethod
    def backward(ctx, g):
        inner, r, outer, shape = ctx.meta
        return sum_middle_raw(g, inner, r, outer).reshape(shape), None, None, None


class SumMiddleFn(torch.autograd.Function):
    """(outer, nsum, inner) -> (outer, 1, inner): sum(A; dims=d) over one batch
    dim (src/array.jl:132-154); pullback: the cotangent replicated nsum times."""

    @staticmethod
    def forward(ctx, x, inner, nsum, outer):
        ctx.meta = (inner, nsum, outer, x.shape)
        return sum_middle_raw(x, inner, nsum, outer).reshape(outer, 1, inner)

    @staticmethod
    def backward(ctx, g):
        inner, nsum, outer, shape = ctx.meta
        return replicate_raw(g, inner, nsum, outer).reshape(shape), None, None, None


class CatFn(torch.autograd.Function):
    """Parts viewed as (outer, inner_i) joined into (outer, sum_i inner_i)
    (cat along a batch dim, src/array.jl:62-64); pullback: each part's
    columns copied back out."""

    @staticmethod
    def forward(ctx, outer, *parts):
        parts = [_c(p) for p in parts]
        inners = [p.numel() // outer for p in parts]
        tot = sum(inners)
        out = torch.empty((outer, tot), dtype=parts[0].dtype, device=parts[0].device)
        es = out.element_size()
        off = 0
        for p, n in zip(parts, inners):
            copy_blocks_raw(out, p, n * es, 1, 0, 0, outer, tot * es, n * es, dst_off=off * es)
            off += n
        ctx.meta = (outer, inners, [p.shape for p in parts])
        return out

    @staticmethod
    def backward(ctx, g):
        outer, inners, shapes = ctx.meta
        g = _c(g)
        tot = sum(inners)
        es = g.element_size()
        grads, off = [], 0
        for n, shp in zip(inners, shapes):
            d = torch.empty((outer, n), dtype=g.dtype, device=g.device)
            copy_blocks_raw(d, g, n * es, 1, 0, 0, outer, n * es, tot * es, src_off=off * es)
            grads.append(d.reshape(shp))
            off += n
        return (None, *grads)


class SimilarityFn(torch.autograd.Function):
    """nzval = scale * circulant_similarity(kind, x, y, ws): forward
    src/similarity.jl:31-103, pullback src/rrules.jl:1-32."""

    @staticmethod
    def forward(ctx, kind, x, y, spatial, ws, scale):
        x, y = _c(x), _c(y)
        ctx.save_for_backward(x, y)
        ctx.meta = (kind, spatial, ws, scale)
        return similarity_raw(kind, x, y, spatial, ws, scale)

    @staticmethod
    def backward(ctx, dS):
        x, y = ctx.saved_tensors
        kind, spatial, ws, scale = ctx.meta
        nsp, n1, n2 = geometry(spatial)
        dS = _c(dS)
        nb, C = x.shape[0], x.shape[1]
        dx = torch.empty_like(x) if ctx.needs_input_grad[1] else None
        dy = torch.empty_like(y) if ctx.needs_input_grad[2] else None
        L.check(L.lib.circatt_similarity_bwd(kind, dtype_code(x), nsp, n1, n2, ws, C, nb, scale,
                                             ptr(dS), ptr(x), ptr(y), ptr(dx), ptr(dy),
                                             stream_ptr(x.device)), "circatt_similarity_bwd")
        return None, dx, dy, None, None, None


class SoftmaxFn(torch.autograd.Function):
    """Row softmax of nzval: src/similarity.jl:105-126, pullback src/rrules.jl:42-56."""

    @staticmethod
    def forward(ctx, nz):
        nz = _c(nz)
        K = nz.shape[-1]
        out = torch.empty_like(nz)
        L.check(L.lib.circatt_softmax(K, nz.numel() // K, ptr(nz), ptr(out),
                                      stream_ptr(nz.device)), "circatt_softmax")
        ctx.save_for_backward(out)
        return out

    @staticmethod
    def backward(ctx, dA):
        (A,) = ctx.saved_tensors
        dA = _c(dA)
        K = A.shape[-1]
        dS = torch.empty_like(A)
        L.check(L.lib.circatt_softmax_bwd(K, A.numel() // K, ptr(A), ptr(dA), ptr(dS),
                                          stream_ptr(A.device)), "circatt_softmax_bwd")
        return dS


class ApplyFn(torch.autograd.Function):
    """y = A ⊗ x (trans False) or Aᵀ ⊗ x (trans True): src/attention.jl:53-80;
    pullbacks src/rrules.jl:58-88:
      ⊗:  ∂A = sim_Dot(Δy, x),  ∂x = Aᵀ ⊗ Δy
      ⊗ᵀ: ∂A = sim_Dot(x, Δy),  ∂x = A ⊗ Δy"""

    @staticmethod
    def forward(ctx, nz, x, spatial, ws, trans):
        nz, x = _c(nz), _c(x)
        ctx.save_for_backward(nz, x)
        ctx.meta = (spatial, ws, trans)
        return apply_raw(nz, x, spatial, ws, trans)

    @staticmethod
    def backward(ctx, dy):
        nz, x = ctx.saved_tensors
        spatial, ws, trans = ctx.meta
        dy = _c(dy)
        dA = dx = None
        if ctx.needs_input_grad[0]:
            a, b = (x, dy) if trans else (dy, x)
            dA = similarity_raw(L.DOT, a, b, spatial, ws, 1.0).view_as(nz)
        if ctx.needs_input_grad[1]:
            dx = apply_raw(nz, dy, spatial, ws, not trans)
        return dA, dx, None, None, None


class AxpbyFn(torch.autograd.Function):
    """Z = alpha_b X + beta_b Y over nzval batches (src/array.jl:66-81, 179-189),
    pullback of scale as src/rrules.jl:94-114."""

    @staticmethod
    def forward(ctx, alpha, X, beta, Y, nb):
        X = _c(X)
        Y = _c(Y) if Y is not None else None
        ctx.save_for_backward(X, Y, alpha if isinstance(alpha, torch.Tensor) else None,
                              beta if isinstance(beta, torch.Tensor) else None)
        ctx.scalars = (alpha if not isinstance(alpha, torch.Tensor) else None,
                       beta if not isinstance(beta, torch.Tensor) else None)
        ctx.nb = nb
        return axpby_raw(alpha, X, beta, Y, nb)

    @staticmethod
    def backward(ctx, dZ):
        X, Y, a_t, b_t = ctx.saved_tensors
        a_s, b_s = ctx.scalars
        nb = ctx.nb
        dZ = _c(dZ)
        alpha = a_t if a_t is not None else a_s
        beta = b_t if b_t is not None else b_s
        dX = axpby_raw(alpha, dZ, None, None, nb) if ctx.needs_input_grad[1] else None
        dY = None
        if Y is not None and ctx.needs_input_grad[3]:
            dY = axpby_raw(beta, dZ, None, None, nb)
        da = batch_dot(dZ, X, nb) if (a_t is not None and ctx.needs_input_grad[0]) else None
        db = None
        if b_t is not None and Y is not None and ctx.needs_input_grad[2]:
            db = batch_dot(dZ, Y, nb)
        return da, dX, db, dY, None


def batch_dot_raw(A, B, nb):
    """(nb,) per-batch sums of A .* B (B None: of A) over nzval slices, with
    circatt_batch_dot (double accumulation in a fixed order)."""
    A = _c(A)
    B = _c(B) if B is not None else None
    nnz = A.numel() // nb
    out = torch.empty((nb,), dtype=torch.float32, device=A.device)
    wbytes = L.lib.circatt_batch_dot_workspace_bytes(nnz, nb)
    work = torch.empty(((wbytes + 7) // 8,), dtype=torch.float64, device=A.device)
    L.check(L.lib.circatt_batch_dot(nnz, nb, ptr(A), ptr(B), ptr(out), ptr(work), wbytes,
                                    stream_ptr(A.device)), "circatt_batch_dot")
    return out


class BatchDotFn(torch.autograd.Function):
    """out[b] = sum_i A[b, i] B[b, i] (B None: sum_i A[b, i]) over nb batches
    of nzval: dot (src/array.jl:83-85), sum(A) and sum(A; dims=(1,2))
    (src/array.jl:132-177).  Pullback: g_b B and g_b A (circatt_axpby)."""

    @staticmethod
    def forward(ctx, A, B, nb):
        A = _c(A)
        B = _c(B) if B is not None else None
        ctx.save_for_backward(A, B)
        ctx.nb = nb
        return batch_dot_raw(A, B, nb)

    @staticmethod
    def backward(ctx, g):
        A, B = ctx.saved_tensors
        nb = ctx.nb
        g = _c(g.to(torch.float32))
        dA = dB = None
        if B is None:
            if ctx.needs_input_grad[0]:
                dA = replicate_raw(g, 1, A.numel() // nb, nb).reshape(A.shape)
        else:
            if ctx.needs_input_grad[0]:
                dA = axpby_raw(g, B, None, None, nb).reshape(A.shape)
            if ctx.needs_input_grad[1]:
                dB = axpby_raw(g, A, None, None, nb).reshape(B.shape)
        return dA, dB, None


def batch_dot(A, B, nb):
    """(nb,) per-batch sums of A .* B over nzval slices (the ∂c of the scale
    rrule, src/rrules.jl:101-104)."""
    return batch_dot_raw(A, B, nb)


class FusedAttentionFn(torch.autograd.Function):
    """y = softmax(scale*sim(q,k)) ⊗ v without materialising A
    (circatt_fused_fwd / circatt_fused_bwd).  Same value and gradients as the
    composition circulant_adjacency -> ⊗ of src/attention.jl:19-42.

    Planar tensors are (B, C, *reversed(spatial)) (the reference's Julia
    (spatial..., C, B)); with channels_last they are (B, *reversed(spatial), C)
    (Julia (C, spatial..., B)) and the kernels read and write that layout."""

    @staticmethod
    def forward(ctx, kind, q, k, v, spatial, ws, nheads, channels_last=False):
        q, k, v = _c(q), _c(k), _c(v)
        nsp, n1, n2 = geometry(spatial)
        B = q.shape[0]
        C = q.shape[-1] if channels_last else q.shape[1]
        P = int(math.prod(spatial))
        code = dtype_code(q) | (L.CHANNELS_LAST if channels_last else 0)
        y = torch.empty_like(q)
        lse = torch.empty((B * nheads, P), dtype=torch.float32, device=q.device)
        L.check(L.lib.circatt_fused_fwd(kind, code, nsp, n1, n2, ws, C, nheads, B,
                                        ptr(q), ptr(k), ptr(v), ptr(y), ptr(lse),
                                        stream_ptr(q.device)), "circatt_fused_fwd")
        ctx.save_for_backward(q, k, v, y, lse)
        ctx.meta = (kind, spatial, ws, nheads, C, code)
        return y

    @staticmethod
    def backward(ctx, dy):
        q, k, v, y, lse = ctx.saved_tensors
        kind, spatial, ws, nheads, C, code = ctx.meta
        nsp, n1, n2 = geometry(spatial)
        B = q.shape[0]
        dy = _c(dy)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        wbytes = L.lib.circatt_fused_bwd_workspace_bytes(nsp, n1, n2, nheads, B)
        ws_buf = torch.empty((wbytes // 4,), dtype=torch.float32, device=q.device)
        L.check(L.lib.circatt_fused_bwd(kind, code, nsp, n1, n2, ws, C, nheads, B,
                                        ptr(q), ptr(k), ptr(v), ptr(y), ptr(dy), ptr(lse),
                                        ptr(dq), ptr(dk), ptr(dv), ptr(ws_buf), wbytes,
                                        stream_ptr(q.device)), "circatt_fused_bwd")
        return None, dq, dk, dv, None, None, None, None
