"""Downstream layers over the circulant attention entry points, in the manner
of GroupCDL (the reference's README.md:33-38 points to it as the example
consumer): an attention block for channels-last feature maps, and the
group-sparse thresholding whose group norms are circulant-attention sums.

Both take channels-last tensors (B, *spatial_slow_first, C), the layout of
`torch.nn.Linear` over the channel axis, so 1x1 projections need no
transposes and the fused kernels read the tensors in place
(`CIRCATT_CHANNELS_LAST`).  A spatial size (H, W) here is the reference's
Julia (W, H): the last spatial axis before C is the fastest.
"""
from __future__ import annotations

import torch

from .circulant import (AbstractSimilarity, Circulant, DistanceSimilarity, DotSimilarity,
                        Otimes, circulant_mh_adjacency, circulant_mh_attention)


class CircAttBlock(torch.nn.Module):
    """x + W_o · MHA(W_q x, W_k x, W_v x) with circulant (windowed, circularly
    wrapped) multi-head attention of window `window` over the spatial axes.

    x: (B, *spatial, channels), channels-last.  The attention is the fused
    path of circulant_mh_attention (src/attention.jl:38-42, A never formed)
    with the similarity `simfun` honoured; its scale is the reference's
    1/sqrt(channels per head)."""

    def __init__(self, channels: int, window: int, nheads: int = 1,
                 simfun: AbstractSimilarity = DotSimilarity(), bias: bool = True):
        super().__init__()
        if channels % nheads != 0:
            raise AssertionError(f"channels ({channels}) must be divisible by nheads ({nheads})")
        if window % 2 != 1:
            raise AssertionError(f"filter size M={window} must be odd.")
        self.window, self.nheads, self.simfun = window, nheads, simfun
        # separate projections: each output is a contiguous channels-last tensor
        self.q = torch.nn.Linear(channels, channels, bias=bias)
        self.k = torch.nn.Linear(channels, channels, bias=bias)
        self.v = torch.nn.Linear(channels, channels, bias=bias)
        self.o = torch.nn.Linear(channels, channels, bias=bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y, _ = circulant_mh_attention(self.simfun, self.q(x), self.k(x), self.v(x), self.window,
                                      self.nheads, materialize=False, honor_simfun=True,
                                      channels_last=True)
        return x + self.o(y)


class GroupThresholding(torch.nn.Module):
    """GroupCDL-style group-sparse thresholding of codes z (B, *spatial, M):

        Γ = rowsoftmax(simfun(θ_i, θ_j)) over the circulant window, per head
            of M / nheads channels, with θ = W_θ f a projection of features f;
        ξ = Γ ⨷ z²                      (non-local group energies)
        z ← z · relu(1 − τ / sqrt(ξ + ε))  (τ > 0 per channel)

    Γ is the reference's circulant_mh_adjacency (unscaled similarity,
    src/similarity.jl:144-161, src/attention.jl:46-51) and ξ its ⨷.  With
    `fused=True` (default) ξ comes from the fused attention kernels on the
    channels-last tensors, Γ never formed: attention scales q and k by
    dh^(-1/4) each (src/attention.jl:20-21), so θ enters as θ dh^(1/4).
    `adjacency(f)` returns Γ as a Circulant (planar, materialised) for callers
    that reuse it over several iterations, as GroupCDL does; `forward(z, f,
    A=Γ)` then applies it."""

    def __init__(self, channels: int, feat_channels: int, window: int, nheads: int = 1,
                 simfun: AbstractSimilarity = DistanceSimilarity(), tau: float = 0.1,
                 eps: float = 1e-6, fused: bool = True):
        super().__init__()
        if channels % nheads != 0:
            raise AssertionError(f"channels ({channels}) must be divisible by nheads ({nheads})")
        if window % 2 != 1:
            raise AssertionError(f"filter size M={window} must be odd.")
        self.window, self.nheads, self.simfun = window, nheads, simfun
        self.eps, self.fused = eps, fused
        self.theta = torch.nn.Linear(feat_channels, channels, bias=False)
        self.tau = torch.nn.Parameter(torch.full((channels,), float(tau)))

    def _theta(self, f: torch.Tensor) -> torch.Tensor:
        return self.theta(f)

    def adjacency(self, f: torch.Tensor) -> Circulant:
        """Γ (Julia size (P, P, nheads, B)) from features f (B, *spatial, F)."""
        th = self._theta(f).movedim(-1, 1).contiguous()  # planar (B, M, *spatial)
        return circulant_mh_adjacency(self.simfun, th, th, self.window, self.nheads)

    def energy(self, z: torch.Tensor, f: torch.Tensor = None, A: Circulant = None) -> torch.Tensor:
        """ξ = Γ ⨷ z² (channels-last, like z)."""
        z2 = z * z
        if A is not None:
            return Otimes(A, z2.movedim(-1, 1).contiguous()).movedim(1, -1).contiguous()
        if self.fused:
            dh = z.shape[-1] // self.nheads
            th = self._theta(f) * dh ** 0.25
            xi, _ = circulant_mh_attention(self.simfun, th, th, z2, self.window, self.nheads,
                                           materialize=False, honor_simfun=True,
                                           channels_last=True)
            return xi
        return self.energy(z, A=self.adjacency(f))

    def forward(self, z: torch.Tensor, f: torch.Tensor = None, A: Circulant = None) -> torch.Tensor:
        if f is None and A is None:
            raise AssertionError("GroupThresholding needs features f or an adjacency A")
        xi = self.energy(z, f, A)
        return z * torch.relu(1.0 - self.tau / torch.sqrt(xi + self.eps))


__all__ = ["CircAttBlock", "GroupThresholding"]
