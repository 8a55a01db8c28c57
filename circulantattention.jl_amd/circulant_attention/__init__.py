"""MI355X circulant attention: host binding of libcircatt mirroring the
exports of CirculantAttention.jl (src/CirculantAttention.jl:18-25).

Julia name              -> here
  Circulant, circulant  -> Circulant, circulant
  circulant_similarity(!), DotSimilarity, DistanceSimilarity
                        -> circulant_similarity(_), DotSimilarity, DistanceSimilarity
  circulant_adjacency(!)-> circulant_adjacency(_)
  circulant_attention, circulant_mh_attention, circulant_mh_adjacency
                        -> same names
  ⊗, ⨷                  -> otimes (also ``A @ x``), Otimes
  NNlib.softmax(!)      -> softmax(_)
  CirculantAttention.scale, sum(A; dims), +, -, *, ==, dot
                        -> scale, Circulant.sum, operators, Circulant.dot
  cat(As...; dims), repeat(A, counts...)
                        -> cat, Circulant.repeat
  kernel_length, spatial_dims, spatial_size (unexported accessors)
                        -> same names
Gradients flow through torch.autograd with the reference's rrules
(src/rrules.jl); Zygote.accum's role is played by autograd accumulation.

`layers` holds downstream modules in the manner of GroupCDL (README.md:33-38):
CircAttBlock and GroupThresholding, on channels-last feature maps.
"""
from . import _lib
from .circulant import (AbstractSimilarity, Circulant, DistanceSimilarity, DotSimilarity, Otimes,
                        cat, circulant, circulant_adjacency, circulant_adjacency_, circulant_attention,
                        circulant_mh_adjacency, circulant_mh_attention,
                        circulant_mh_transposed_attention, circulant_similarity,
                        circulant_similarity_, circulant_transposed_attention, otimes, scale,
                        kernel_length, softmax, softmax_, spatial_dims, spatial_size)

from .layers import CircAttBlock, GroupThresholding  # noqa: E402

Circulant.__matmul__ = lambda A, x: otimes(A, x)

__all__ = [
    "AbstractSimilarity", "Circulant", "DistanceSimilarity", "DotSimilarity", "Otimes",
    "cat", "circulant", "circulant_adjacency", "circulant_adjacency_", "circulant_attention",
    "circulant_mh_adjacency", "circulant_mh_attention", "circulant_mh_transposed_attention",
    "circulant_similarity", "circulant_similarity_", "circulant_transposed_attention", "otimes",
    "kernel_length", "scale", "softmax", "softmax_", "spatial_dims", "spatial_size",
    "CircAttBlock", "GroupThresholding",
]
