# Drop-in replacement of CirculantAttention.jl v1.0.1 (same module name, same
# exports: src/CirculantAttention.jl:1-30 of the reference) whose compute runs
# in libcircatt.so, the MI355X (gfx950) HIP library of this repository,
# through ccall.  Device arrays are AMDGPU.jl's ROCArrays (memory and streams
# only); every operation of the reference's hot path -- pattern, similarity,
# softmax, ⊗ and its transpose, their pullbacks, the Circulant algebra and the
# fused attention -- is a libcircatt entry point declared in
# include/circatt.h.  The library path is ENV["CIRCATT_LIB"] or the
# libcircatt.so built next to this package (circulantattention.jl_amd/).
module CirculantAttention

const CircAtt = CirculantAttention
export CircAtt

using AMDGPU
import Adapt

using LinearAlgebra

using NNlib
import ChainRulesCore as CRC
import Zygote

include("libcircatt.jl")
include("devops.jl")

include("array.jl")
export Circulant, circulant

include("similarity.jl")
export circulant_similarity, circulant_similarity!, DotSimilarity, DistanceSimilarity
export circulant_adjacency, circulant_adjacency!

include("attention.jl")
export circulant_attention, circulant_mh_attention, circulant_mh_adjacency, ⊗, ⨷ # \otimes and \Otimes

include("batchedmul.jl")

include("rrules.jl")
include("zygote.jl")

end
