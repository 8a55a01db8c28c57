"""Circulant type and the circulant attention API, mirroring
CirculantAttention.jl (names, argument meaning, assertion messages).

Memory order follows the reference's Julia arrays (column-major): a Julia
signal of size (N1, N2, C, B) is a torch tensor of shape (B, C, N2, N1) and a
1D signal (L, C, B) is (B, C, L).  ``spatial_size`` is reported fastest-first
like Julia, i.e. (N1, N2).  A Circulant of Julia size (P, P, nh, B) stores
nzVal as a tensor (B, nh, P, K); rowPtr / colVal are the reference's Int32
1-based CSR indices, built on the device on first access.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib as L
from ._functions import (AxpbyFn, ApplyFn, BatchDotFn, CatFn, FusedAttentionFn, ReplicateFn,
                         SimilarityFn, SoftmaxFn, SumMiddleFn, count_unequal, fill_raw, geometry,
                         ptr, replicate_raw, require, similarity_raw, stream_ptr)


class AbstractSimilarity:
    kind = None

    def __repr__(self):
        return f"{type(self).__name__}()"

    def __eq__(self, other):
        return type(self) is type(other)

    def __hash__(self):
        return hash(type(self))


class DotSimilarity(AbstractSimilarity):
    """S_ij = Real(q[i]^H k[j])  (src/similarity.jl:3-15)."""
    kind = L.DOT


class DistanceSimilarity(AbstractSimilarity):
    """S_ij = -sum(abs2, q[i] - k[j]) / 2  (src/similarity.jl:17-29, :71-75;
    the reference docstring omits the minus sign, its kernel has it)."""
    kind = L.DISTANCE


def _kind(simfun) -> int:
    if isinstance(simfun, type) and issubclass(simfun, AbstractSimilarity):
        simfun = simfun()
    if not isinstance(simfun, AbstractSimilarity):
        raise TypeError(f"simfun must be DotSimilarity() or DistanceSimilarity(), got {simfun!r}")
    return simfun.kind


def _spatial(x: torch.Tensor):
    """Fastest-first spatial size of a (nb, C, *reversed spatial) tensor."""
    return tuple(reversed(x.shape[2:]))


_PATTERNS: dict = {}


def _pattern(spatial, ws, device):
    """(rowptr (P+1,), colval (P*K,)) Int32 1-based, one batch, cached per device."""
    key = (str(device), tuple(spatial), ws)
    if key not in _PATTERNS:
        nsp, n1, n2 = geometry(spatial)
        P = int(math.prod(spatial))
        K = ws ** nsp
        rowptr = torch.empty((P + 1,), dtype=torch.int32, device=device)
        colval = torch.empty((P * K,), dtype=torch.int32, device=device)
        L.check(L.lib.circatt_pattern(nsp, n1, n2, ws, 1, ptr(rowptr), ptr(colval),
                                      stream_ptr(device)), "circatt_pattern")
        _PATTERNS[key] = (rowptr, colval)
    return _PATTERNS[key]


@dataclass
class CSRData:
    """The fields of CUDA.jl's CuSparseArrayCSR that the reference and its tests
    touch (test/utils.jl:1-5, test/rrule.jl:10): rowPtr (B.., P+1), colVal
    (B.., P*K), nzVal (B.., P*K), dims (Julia size), nnz (total stored)."""
    rowPtr: torch.Tensor
    colVal: torch.Tensor
    nzVal: torch.Tensor
    dims: tuple
    nnz: int


class Circulant:
    """Circulant{T,N,M,S} (src/array.jl:1-18): a batched circulant-sparse CSR
    matrix of Julia size (P, P, batch...) with window `kernel_length` over
    `spatial_size`.  `nzval` (torch, (*reversed(batch), P, K)) is the only
    differentiable field, as in test/utils.jl:13-30."""

    def __init__(self, nzval: torch.Tensor, kernel_length: int, spatial_size):
        self.nzval = nzval
        self.kernel_length = int(kernel_length)
        self.spatial_size = tuple(int(s) for s in spatial_size)
        nsp = len(self.spatial_size)
        if nsp not in (1, 2):
            raise AssertionError("only 1 or 2 spatial dims are supported")
        if tuple(nzval.shape[-2:]) != (self.P, self.K):
            raise AssertionError(f"nzval trailing shape {tuple(nzval.shape[-2:])} != (P, K) = "
                                 f"{(self.P, self.K)}")

    # ---- constructors (src/array.jl:6-17, :29) ----
    @classmethod
    def new(cls, ws: int, dims, device="cuda", dtype=torch.float32):
        """Circulant{T}(M, dims): dims = (spatial..., batch...) in Julia order;
        nzVal initialised to ones (src/circulant.jl:69,91)."""
        if ws % 2 != 1:
            raise AssertionError(f"filter size M={ws} must be odd.")
        dims = tuple(int(d) for d in dims)
        spatial, batch = dims[:-2], dims[-2:]
        P = int(math.prod(spatial))
        K = ws ** len(spatial)
        nz = torch.empty((*reversed(batch), P, K), dtype=torch.float32, device=device)
        return cls(fill_raw(nz, 1.0), ws, spatial)

    # ---- metadata ----
    @property
    def nsp(self):
        return len(self.spatial_size)

    @property
    def P(self):
        return int(math.prod(self.spatial_size))

    @property
    def K(self):
        return self.kernel_length ** self.nsp

    @property
    def batch(self):
        """Julia-order batch dims, e.g. (nheads, B)."""
        return tuple(reversed(self.nzval.shape[:-2]))

    @property
    def nb(self):
        return int(math.prod(self.batch)) if self.batch else 1

    @property
    def device(self):
        return self.nzval.device

    def size(self, i=None):
        """Julia size (P, P, batch...); i is 1-based like Julia."""
        s = (self.P, self.P, *self.batch)
        return s if i is None else s[i - 1]

    @property
    def shape(self):
        return self.size()

    def ndims(self):
        return len(self.size())

    @property
    def data(self) -> CSRData:
        rowptr, colval = _pattern(self.spatial_size, self.kernel_length, self.device)
        rb = tuple(reversed(self.batch))
        return CSRData(rowPtr=rowptr.expand(*rb, rowptr.numel()),
                       colVal=colval.expand(*rb, colval.numel()),
                       nzVal=self.nzval.reshape(*rb, self.P * self.K),
                       dims=self.size(), nnz=self.nzval.numel())

    def __repr__(self):
        """show (src/array.jl:44-47): the type, kernel length, spatial size,
        then a summary of the CSR data."""
        size = "×".join(str(d) for d in self.size())
        return (f"Circulant{{Float32, {self.ndims()}, {self.kernel_length}, {self.nsp}}} with "
                f"kernel-length {self.kernel_length}, spatial-size {self.spatial_size}, and data,\n"
                f"{size} batched CSR with {self.P * self.K * self.nb} stored entries "
                f"(Float32 nzVal, Int32 rowPtr and colVal) on {self.device}")

    # ---- shape utilities (src/array.jl:49-60) ----
    def reshape(self, *dims):
        """reshape(A, :, :, dims...): the first two dims stay (P, P); the
        batch dims are re-split (Julia order; one -1 or ':' allowed)."""
        dims = [(-1 if d in (":", Ellipsis, None) else int(d)) for d in dims]
        if len(dims) < 3:
            raise AssertionError("reshape needs at least 3 dims")
        for d in dims[:2]:
            if d not in (-1, self.P):
                raise AssertionError(f"the first two dims of a Circulant are {self.P}")
        batch = dims[2:]
        if batch.count(-1) > 1:
            raise AssertionError("only one batch dim can be inferred")
        if -1 in batch:
            known = int(math.prod(d for d in batch if d != -1))
            batch[batch.index(-1)] = self.nb // known
        if int(math.prod(batch)) != self.nb:
            raise AssertionError(f"cannot reshape batch {self.batch} to {tuple(batch)}")
        nz = self.nzval.reshape(*reversed(batch), self.P, self.K)
        return Circulant(nz, self.kernel_length, self.spatial_size)

    def repeat(self, *counts):
        """repeat(A, 1, 1, n3, n4, ...) (src/array.jl:49-52, the same call
        that replicates the pattern over the batch at src/array.jl:9): tiles
        the batch dims; the two (P, P) dims cannot be repeated."""
        counts = [int(c) for c in counts]
        if len(counts) < 2 or counts[0] != 1 or counts[1] != 1:
            raise AssertionError("repeat(A, 1, 1, counts...): the (P, P) dims of a Circulant "
                                 "cannot be repeated")
        batch = list(self.batch) + [1] * max(0, len(counts) - 2 - len(self.batch))
        reps = counts[2:] + [1] * (len(batch) - len(counts[2:]))
        nz = self.nzval.reshape(*reversed(batch), self.P, self.K)
        for j, c in enumerate(reps):
            if c > 1:
                nz = _replicate_axis(nz, len(batch) - 1 - j, c)
        return Circulant(nz, self.kernel_length, self.spatial_size)

    def __eq__(self, other):
        """A == B (src/array.jl:101-115): sizes, spatial size, kernel length
        and the CSR data.  rowPtr and colVal are a function of (spatial size,
        kernel length), so equal metadata means equal indices and only nzVal
        is compared."""
        if not isinstance(other, Circulant):
            return NotImplemented
        return (self.size() == other.size() and self.spatial_size == other.spatial_size
                and self.kernel_length == other.kernel_length
                and count_unequal(self.nzval, other.nzval) == 0)

    __hash__ = None

    def copy(self):
        n = self.nzval.numel()
        nz = ReplicateFn.apply(self.nzval, n, 1, 1).reshape(self.nzval.shape)
        return Circulant(nz, self.kernel_length, self.spatial_size)

    def similar(self):
        return Circulant(torch.empty_like(self.nzval), self.kernel_length, self.spatial_size)

    def _same(self, other):
        if not isinstance(other, Circulant):
            return False
        return (other.kernel_length == self.kernel_length
                and other.spatial_size == self.spatial_size and other.batch == self.batch)

    # ---- algebra on nzVal (src/array.jl:66-81, 179-189) ----
    def __add__(self, other):
        if not self._same(other):
            raise AssertionError("Circulant + Circulant needs equal kernel length, spatial "
                                 "size and batch dims")
        nz = AxpbyFn.apply(1.0, self.nzval, 1.0, other.nzval, self.nb)
        return Circulant(nz, self.kernel_length, self.spatial_size)

    def __sub__(self, other):
        if not self._same(other):
            raise AssertionError("Circulant - Circulant needs equal kernel length, spatial "
                                 "size and batch dims")
        nz = AxpbyFn.apply(1.0, self.nzval, -1.0, other.nzval, self.nb)
        return Circulant(nz, self.kernel_length, self.spatial_size)

    def __neg__(self):
        return (-1.0) * self

    def __mul__(self, c):
        if isinstance(c, (int, float)):
            return self.__rmul__(c)
        return NotImplemented

    def __rmul__(self, c):
        if isinstance(c, (int, float)):
            nz = AxpbyFn.apply(float(c), self.nzval, None, None, self.nb)
            return Circulant(nz, self.kernel_length, self.spatial_size)
        if isinstance(c, torch.Tensor):
            return scale(c, self)
        return NotImplemented

    def dot(self, other):
        """dot(X, Y) = dot(X.nzVal, Y.nzVal) (src/array.jl:83-85)."""
        if not self._same(other):
            raise AssertionError("dot needs matching Circulants")
        return BatchDotFn.apply(self.nzval, other.nzval, 1).reshape(())

    def sum(self, dims=None):
        """sum(A; dims) (src/array.jl:156-177): dims=None (:) -> scalar,
        1 -> (1, P, batch..), 2 -> (P, 1, batch..), (1, 2) -> (1, 1, batch..),
        batch dims (>2) -> Circulant summed over them."""
        nsp, n1, n2 = geometry(self.spatial_size)
        rb = tuple(reversed(self.batch))
        if dims is None:
            return BatchDotFn.apply(self.nzval, None, 1).reshape(())
        if isinstance(dims, int):
            dims = (dims,)
        dims = tuple(dims)
        if dims in ((1,), (2,)):
            return CirculantSum.apply(self.nzval, self.spatial_size, self.kernel_length,
                                      dims[0] == 1).reshape(
                *rb, *((self.P, 1) if dims[0] == 1 else (1, self.P)))
        if dims == (1, 2):
            return BatchDotFn.apply(self.nzval, None, self.nb).reshape(*rb, 1, 1)
        if all(d > 2 for d in dims):
            nz = self.nzval
            axes = tuple(len(rb) - (d - 2) for d in dims)  # Julia dim d -> torch axis
            for ax in sorted(axes, reverse=True):
                nz = _sum_batch_axis(nz, ax)
            return Circulant(nz, self.kernel_length, self.spatial_size)
        raise NotImplementedError(f"dims={dims} not implemented.")


def _sum_batch_axis(nz, ax):
    """Sum nzval over one batch axis (keepdim) with circatt_sum_middle."""
    shape = list(nz.shape)
    outer, inner = int(math.prod(shape[:ax])), int(math.prod(shape[ax + 1:]))
    out = SumMiddleFn.apply(nz, inner, shape[ax], outer)
    shape[ax] = 1
    return out.reshape(shape)


def _replicate_axis(nz, ax, count):
    """repeat along torch axis ax (Julia's repeat: the whole axis tiled count
    times) with circatt_copy_blocks."""
    shape = list(nz.shape)
    outer, inner = int(math.prod(shape[:ax])), int(math.prod(shape[ax:]))
    out = ReplicateFn.apply(nz, inner, count, outer)
    shape[ax] *= count
    return out.reshape(shape)


class CirculantSum(torch.autograd.Function):
    """sum(A; dims=1) (colsum) / sum(A; dims=2) (rowsum), src/array.jl:119-130."""

    @staticmethod
    def forward(ctx, nz, spatial, ws, col):
        nsp, n1, n2 = geometry(spatial)
        nz = nz.contiguous()
        P = int(math.prod(spatial))
        nb = nz.numel() // (P * ws ** nsp)
        out = torch.empty((nb, P), dtype=torch.float32, device=nz.device)
        fn = L.lib.circatt_colsum if col else L.lib.circatt_rowsum
        L.check(fn(nsp, n1, n2, ws, nb, ptr(nz), ptr(out), stream_ptr(nz.device)), "sum")
        ctx.meta = (spatial, ws, col, nz.shape)
        return out

    @staticmethod
    def backward(ctx, g):
        # d/dnz of a row (column) sum is the row's (column's) cotangent
        # broadcast to its entries: the dS of the Distance rrule pattern.
        spatial, ws, col, shape = ctx.meta
        nsp = len(spatial)
        P = int(math.prod(spatial))
        K = ws ** nsp
        g = g.contiguous().reshape(-1, P)
        nb = g.shape[0]
        if not col:
            return replicate_raw(g, 1, K, nb * P).reshape(shape), None, None, None
        # column sums: entry (r, t) takes the cotangent of its column c(r, t),
        # which is the Dot similarity of a one-channel signal of ones
        # (rows r) with g (columns c): 1 * g[c(r, t)], exact
        ones = fill_raw(torch.empty((nb, 1, *reversed(spatial)), dtype=torch.float32,
                                    device=g.device), 1.0)
        dA = similarity_raw(L.DOT, ones, g.reshape(nb, 1, *reversed(spatial)), spatial, ws, 1.0)
        return dA.reshape(shape), None, None, None


# ---------------------------------------------------------------------------
# API (src/similarity.jl, src/attention.jl)
# ---------------------------------------------------------------------------

def kernel_length(A: Circulant) -> int:
    """kernel_length(A) (src/array.jl:31): the window size ws."""
    return A.kernel_length


def spatial_dims(A: Circulant) -> int:
    """spatial_dims(A) (src/array.jl:32): 1 or 2."""
    return A.nsp


def spatial_size(A: Circulant) -> tuple:
    """spatial_size(A) (src/array.jl:33): (N1,) or (N1, N2), fastest first."""
    return A.spatial_size


def cat(*As: Circulant, dims: int = 3) -> Circulant:
    """cat(As...; dims=3) (src/array.jl:62-64): concatenate along a batch
    dim (Julia dim >= 3), e.g. cat(A, B; dims=3) gives (P, P, 2nheads, B)
    (README.md:145-148).  The reference body names the array type instead of
    a Circulant for the spatial size (`spatial_size(A)` with A the type
    parameter) and so throws; here the first argument's spatial size and
    kernel length are used, and all arguments must share them."""
    if not As:
        raise AssertionError("cat needs at least one Circulant")
    A0 = As[0]
    dims = int(dims)
    if dims < 3:
        raise AssertionError("Circulants concatenate along batch dims (dims >= 3) only")
    for A in As:
        if not isinstance(A, Circulant):
            raise AssertionError("cat concatenates Circulants")
        if A.kernel_length != A0.kernel_length or A.spatial_size != A0.spatial_size:
            raise AssertionError("cat needs equal kernel length and spatial size")
    nd = max(dims - 2, max(len(A.batch) for A in As))

    def padded(A):
        b = list(A.batch) + [1] * (nd - len(A.batch))
        return A.nzval.reshape(*reversed(b), A.P, A.K), b

    parts = [padded(A) for A in As]
    ax = dims - 3                      # Julia batch dim -> index into Julia-order batch
    for _, b in parts[1:]:
        if [d for i, d in enumerate(b) if i != ax] != \
                [d for i, d in enumerate(parts[0][1]) if i != ax]:
            raise AssertionError("cat: batch dims other than `dims` must match")
    td = nd - 1 - ax                   # torch axis of the joined batch dim
    shp = list(parts[0][0].shape)
    outer = int(math.prod(shp[:td]))
    shp[td] = sum(p.shape[td] for p, _ in parts)
    nz = CatFn.apply(outer, *[p for p, _ in parts]).reshape(shp)
    return Circulant(nz, A0.kernel_length, A0.spatial_size)


def circulant(M: int, x: torch.Tensor) -> Circulant:
    """circulant(M, x): Float32 Circulant of x's spatial size with batch
    (1, B) (src/array.jl:29)."""
    require(x, "x")
    return Circulant.new(M, (*_spatial(x), 1, x.shape[0]), device=x.device)


def _check_pair(x, y):
    require(x, "x")
    require(y, "y")
    if x.shape != y.shape:
        raise AssertionError(f"x and y must have equal sizes, got {tuple(x.shape)} and "
                             f"{tuple(y.shape)}")
    if x.dtype != y.dtype:
        raise AssertionError("x and y must have equal element types")
    if x.dim() not in (3, 4):
        raise AssertionError("signals must be (B, C, L) or (B, C, N2, N1)")


def circulant_similarity(simfun, x, y, W: int) -> Circulant:
    """circulant_similarity(simfun, x, y, W) (src/similarity.jl:128-142).
    Row i of the result is pixel i of x, columns are pixels of y; the result
    is a Float32 Circulant of Julia size (P, P, 1, B)."""
    _check_pair(x, y)
    if W % 2 != 1:
        raise AssertionError(f"filter size M={W} must be odd.")
    spatial = _spatial(x)
    nz = SimilarityFn.apply(_kind(simfun), x, y, spatial, W, 1.0)
    return Circulant(nz.reshape(x.shape[0], 1, *nz.shape[1:]), W, spatial)


def circulant_similarity_(A: Circulant, simfun, x, y) -> Circulant:
    """circulant_similarity!(A, simfun, x, y) (src/similarity.jl:31-53): writes
    into A.nzval (not differentiable)."""
    _check_pair(x, y)
    spatial = _spatial(x)
    if A.nsp != len(spatial):
        raise AssertionError(f"spatial_dims ({A.nsp}) of circulant matrix must match those of "
                             f"data signal ({len(spatial)}).")
    if A.nb != x.shape[0]:
        raise AssertionError(f"batchdim of circulant matrix ({A.nb}) must match that of x, y "
                             f"({x.shape[0]}).")
    if tuple(spatial) != A.spatial_size:
        raise AssertionError(f"spatial size {tuple(spatial)} of x does not match A's "
                             f"{A.spatial_size}")
    if not A.nzval.is_contiguous():
        raise AssertionError("circulant_similarity! needs A's nzVal contiguous")
    nsp, n1, n2 = geometry(spatial)
    x, y = x.contiguous(), y.contiguous()
    # written in place by the kernel (no temporary)
    L.check(L.lib.circatt_similarity(_kind(simfun), L.C32 if x.is_complex() else L.F32, nsp, n1,
                                     n2, A.kernel_length, x.shape[1], A.nb, 1.0, ptr(x), ptr(y),
                                     ptr(A.nzval), stream_ptr(x.device)), "circatt_similarity")
    return A


def softmax(A: Circulant) -> Circulant:
    """NNlib.softmax(A::Circulant): row softmax (src/similarity.jl:118-126)."""
    return Circulant(SoftmaxFn.apply(A.nzval), A.kernel_length, A.spatial_size)


def softmax_(A: Circulant, B: Circulant = None) -> Circulant:
    """NNlib.softmax!(A, B=A) (src/similarity.jl:113-116), not differentiable."""
    B = A if B is None else B
    if not (A.nzval.is_contiguous() and B.nzval.is_contiguous()):
        raise AssertionError("softmax! needs contiguous nzVal")
    if A.size() != B.size() or A.kernel_length != B.kernel_length:
        raise AssertionError("softmax!(A, B): A and B must have the same size and pattern")
    # in place when B is A (circatt_softmax allows in == out)
    L.check(L.lib.circatt_softmax(A.K, A.P * A.nb, ptr(B.nzval), ptr(A.nzval),
                                  stream_ptr(A.nzval.device)), "circatt_softmax")
    return A


def circulant_adjacency(simfun, x, y, W: int) -> Circulant:
    """softmax ∘ circulant_similarity (src/similarity.jl:151-161)."""
    return softmax(circulant_similarity(simfun, x, y, W))


def circulant_adjacency_(A: Circulant, simfun, x, y) -> Circulant:
    """circulant_adjacency!(A, simfun, x, y) (src/similarity.jl:144-148)."""
    circulant_similarity_(A, simfun, x, y)
    return softmax_(A)


def _splitheads(x, nheads):
    """splitheads (src/attention.jl:44): (B, C, ...) -> (B*nheads, C/nheads, ...);
    head g of batch b becomes flattened batch g + nheads*b."""
    B, C = x.shape[0], x.shape[1]
    if C % nheads != 0:
        raise AssertionError(f"channels ({C}) must be divisible by nheads ({nheads})")
    return x.reshape(B * nheads, C // nheads, *x.shape[2:])


def circulant_attention(*args, materialize: bool = True, channels_last: bool = False):
    """Two forms, as in the reference:

    * ``y, A = circulant_attention(simfun, q, k, v, W)`` / ``(q, k, v, W)``
      (src/attention.jl:19-26): q and k are scaled by 1/sqrt(sqrt(C)), A is the
      row-softmax adjacency (Julia size (P, P, 1, B)) and y = A ⊗ v.  With
      ``materialize=False`` the fused kernels compute y without forming A and
      ``None`` is returned in A's place.  ``channels_last=True`` (fused only)
      takes and returns (B, *reversed(spatial), C) tensors, Julia
      (C, spatial..., B), read and written in place by the kernels.
    * ``y = circulant_attention(A, x)`` = ``A ⊗ x`` (src/attention.jl:53-70).
    """
    if len(args) == 2 and isinstance(args[0], Circulant):
        return _apply(args[0], args[1], trans=False)
    if len(args) == 4:
        args = (DotSimilarity(),) + tuple(args)
    if len(args) != 5:
        raise TypeError("circulant_attention(simfun, q, k, v, W), (q, k, v, W) or (A, x)")
    simfun, q, k, v, W = args
    return _attention(_kind(simfun), q, k, v, W, 1, materialize, channels_last)


def _attention(kind, q, k, v, W, nheads, materialize, channels_last=False):
    _check_pair(q, k)
    _check_pair(q, v)
    if W % 2 != 1:
        raise AssertionError(f"filter size M={W} must be odd.")
    if channels_last:
        if materialize:
            raise AssertionError("channels_last needs materialize=False (the fused kernels)")
        if q.dim() < 3:
            raise AssertionError("channels_last tensors are (B, *spatial, C)")
        spatial = tuple(reversed(q.shape[1:-1]))
        C = q.shape[-1]
        if C % nheads != 0:
            raise AssertionError(f"channels ({C}) must be divisible by nheads ({nheads})")
        return FusedAttentionFn.apply(kind, q, k, v, spatial, W, nheads, True), None
    spatial = _spatial(q)
    if not materialize:
        return FusedAttentionFn.apply(kind, q, k, v, spatial, W, nheads), None
    qr, kr, vr = (_splitheads(t, nheads) for t in (q, k, v))
    dh = qr.shape[1]
    tau = math.sqrt(dh)
    # q ./ sqrt(tau), k ./ sqrt(tau) fold into a similarity scale of 1/tau
    S = SimilarityFn.apply(kind, qr, kr, spatial, W, 1.0 / tau)
    A = SoftmaxFn.apply(S)
    y = ApplyFn.apply(A, vr, spatial, W, False)
    B = q.shape[0]
    A = Circulant(A.reshape(B, nheads, *A.shape[1:]), W, spatial)
    return y.reshape(q.shape), A


def circulant_mh_attention(*args, materialize: bool = True, honor_simfun: bool = False,
                           channels_last: bool = False):
    """Two forms, as in the reference:

    * ``y, A = circulant_mh_attention(simfun, q, k, v, W, nheads)``
      (src/attention.jl:38-42): attention per head of C/nheads channels; A has
      Julia size (P, P, nheads, B).  The reference ignores ``simfun`` and
      always uses DotSimilarity (src/attention.jl:40); that is reproduced
      unless ``honor_simfun=True``.  ``materialize=False`` selects the fused
      kernels (A is not formed, ``None`` is returned in its place);
      ``channels_last=True`` with it takes (B, *reversed(spatial), C) tensors.
    * ``y = circulant_mh_attention(A, x)`` = ``A ⨷ x`` (src/attention.jl:89-96).
    """
    if len(args) == 2 and isinstance(args[0], Circulant):
        return _mh_apply(args[0], args[1], trans=False)
    if len(args) == 5:
        # src/attention.jl:43 forwards to a method that does not exist in the
        # reference (MethodError); here it means DotSimilarity.
        args = (DotSimilarity(),) + tuple(args)
    if len(args) != 6:
        raise TypeError("circulant_mh_attention(simfun, q, k, v, W, nheads) or (A, x)")
    simfun, q, k, v, W, nheads = args
    kind = _kind(simfun) if honor_simfun else L.DOT
    return _attention(kind, q, k, v, W, int(nheads), materialize, channels_last)


def circulant_mh_adjacency(simfun, x, y, W: int, nheads: int) -> Circulant:
    """circulant_mh_adjacency (src/attention.jl:46-51): adjacency per head,
    Julia size (P, P, nheads, B)."""
    xr, yr = _splitheads(x, nheads), _splitheads(y, nheads)
    A = circulant_adjacency(simfun, xr, yr, W)
    return A.reshape(":", ":", nheads, x.shape[0])


def _apply(A: Circulant, x: torch.Tensor, trans: bool):
    require(x, "x")
    spatial = _spatial(x)
    if A.nsp != len(spatial):
        raise AssertionError(f"spatial-dims ({A.nsp}) of A must match spatial dims of x "
                             f"({len(spatial)})")
    if tuple(spatial) != A.spatial_size:
        raise AssertionError(f"spatial size {tuple(spatial)} of x does not match A's "
                             f"{A.spatial_size}")
    if A.nb != x.shape[0]:
        raise AssertionError(f"batch of A ({A.nb}) must match that of x ({x.shape[0]})")
    nz = A.nzval.reshape(A.nb, A.P, A.K)
    return ApplyFn.apply(nz, x, spatial, A.kernel_length, trans)


def otimes(A: Circulant, x: torch.Tensor) -> torch.Tensor:
    """A ⊗ x = circulant_attention(A, x) (src/attention.jl:53-70)."""
    return _apply(A, x, trans=False)


def circulant_transposed_attention(A: Circulant, x: torch.Tensor) -> torch.Tensor:
    """Aᵀ ⊗ x (src/attention.jl:72-80)."""
    return _apply(A, x, trans=True)


def _mh_apply(A: Circulant, x, trans):
    if len(A.batch) != 2:
        raise AssertionError("⨷ needs a Circulant of Julia size (P, P, nheads, B)")
    nheads = A.batch[0]
    y = _apply(A.reshape(":", ":", ":"), _splitheads(x, nheads), trans)
    return y.reshape(x.shape)


def Otimes(A: Circulant, x: torch.Tensor) -> torch.Tensor:
    """A ⨷ x = circulant_mh_attention(A, x) (src/attention.jl:89-96)."""
    return _mh_apply(A, x, trans=False)


def circulant_mh_transposed_attention(A: Circulant, x: torch.Tensor) -> torch.Tensor:
    """(src/attention.jl:98-103)."""
    return _mh_apply(A, x, trans=True)


def scale(c: torch.Tensor, A: Circulant) -> Circulant:
    """scale(c, A) = c .* A with c of Julia size (1, 1, batch...) broadcast over
    A's batch dims (src/array.jl:179-189).  c is a torch tensor of shape
    (*reversed(batch), 1, 1)."""
    require(c, "c")
    if c.is_complex():
        raise NotImplementedError("complex scale factors are not supported")
    if c.dim() < 2 or c.shape[-1] != 1 or c.shape[-2] != 1:
        raise AssertionError("Scaling of non-batchdims of CuSparseArrayCSR not implemented")
    cb = tuple(reversed(c.shape[:-2]))  # Julia batch dims of c
    ab = A.batch
    nd = max(len(cb), len(ab))
    cb = cb + (1,) * (nd - len(cb))
    ab = ab + (1,) * (nd - len(ab))
    out = []
    for ci, ai in zip(cb, ab):
        if ci != ai and 1 not in (ci, ai):
            raise AssertionError(f"cannot broadcast scale factor {cb} against batch {ab}")
        out.append(max(ci, ai))
    rb = tuple(reversed(out))
    nz = A.nzval.reshape(*tuple(reversed(ab)), A.P, A.K)
    alpha = c.reshape(*tuple(reversed(cb)))
    # broadcast A's values and the factors to the joint batch (Julia batch
    # dim j is torch axis nd - 1 - j)
    for j in range(nd):
        ax = nd - 1 - j
        if ab[j] == 1 and out[j] > 1:
            nz = _broadcast_axis(nz, ax, out[j])
        if cb[j] == 1 and out[j] > 1:
            alpha = _broadcast_axis(alpha, ax, out[j])
    nb = int(math.prod(rb))
    z = AxpbyFn.apply(alpha.reshape(nb), nz, None, None, nb)
    return Circulant(z.reshape(*rb, A.P, A.K), A.kernel_length, A.spatial_size)


def _broadcast_axis(x, ax, count):
    """x with a size-1 torch axis ax broadcast to count (materialised with
    circatt_copy_blocks)."""
    shape = list(x.shape)
    outer, inner = int(math.prod(shape[:ax])), int(math.prod(shape[ax + 1:]))
    out = ReplicateFn.apply(x, inner, count, outer)
    shape[ax] = count
    return out.reshape(shape)
