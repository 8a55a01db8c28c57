# Similarity, softmax and adjacency (reference: src/similarity.jl:1-161) on
# libcircatt: circatt_similarity writes nzVal in place in the reference's CSR
# order, circatt_softmax normalises each row's K slots.

abstract type AbstractSimilarity end

@doc raw"""
    DotSimilarity()

Selects the inner-product score between the channel vectors of query pixel
`i` and key pixel `j`: ``S_{ij} = \mathrm{Re}\,\langle k_j, q_i\rangle``
(the real part of the Hermitian product for complex signals).  Pass it to
`circulant_similarity`, `circulant_adjacency` or `circulant_attention`.

See also [`DistanceSimilarity`](@ref).
"""
struct DotSimilarity <: AbstractSimilarity end

@doc raw"""
    DistanceSimilarity()

Selects minus half the squared Euclidean distance between the channel
vectors of query pixel `i` and key pixel `j`:
``S_{ij} = -\tfrac{1}{2}\lVert q_i - k_j\rVert^2`` (the sign and the half are
those of the reference's kernel, src/similarity.jl:55-78).

See also [`DotSimilarity`](@ref).
"""
struct DistanceSimilarity <: AbstractSimilarity end

simkind(::DotSimilarity) = CIRCATT_DOT
simkind(::DistanceSimilarity) = CIRCATT_DISTANCE

"""nzVal of A = scale * simfun(x, y) on A's pattern; x is the row (query)
argument, y the column (key) argument."""
function similarity_into!(A::Circulant{Tv, NA, W, S}, simfun::AbstractSimilarity,
                          x::AbstractArray{Tx,N}, y::AbstractArray{Tx,N}, scale::Real) where {Tv, NA, W, S, Tx, N}
    @assert S == N - 2 "spatial_dims ($(S)) of circulant matrix must match those of data signal ($(N-2))."
    @assert nbatch(A) == size(x, N) "batchdim of circulant matrix ($(nbatch(A))) must match that of x, y ($(size(x,N)))."
    @assert size(x) == size(y) "x and y must have the same size"
    nsp, n1, n2 = geom(spatial_size(A))
    check(circatt_similarity(simkind(simfun), dtype_code(Tx), nsp, n1, n2, Int32(W),
                             Int64(size(x, N-1)), Int64(size(x, N)), Cfloat(scale), cvoid_ptr(x),
                             cvoid_ptr(y), cfloat_ptr(A.data.nzVal), stream_ptr()),
          "circatt_similarity")
    return A
end

function circulant_similarity!(A::Circulant, simfun::AbstractSimilarity, x, y)
    similarity_into!(A, simfun, x, y, 1f0)
end

"""
    circulant_similarity(simfun::AbstractSimilarity, x, y, W::Int)

A new `Circulant` of size (P, P, 1, B) holding, for every pixel `i` of `x`
and every pixel `j` in the circularly wrapped W-wide window around it, the
score of `simfun` between the channels of `x` at `i` and of `y` at `j`
(batch by batch).  Pixels are linear (column-major) indices; W is odd.

See also [`DotSimilarity`](@ref), [`DistanceSimilarity`](@ref).
"""
function circulant_similarity(simfun::AbstractSimilarity, x::AbstractArray{T,N}, y::AbstractArray{T,N}, W::Integer)::Circulant where {T,N}
    S = Circulant(Int(W), (size(x)[1:N-2]..., 1, size(x, N)))
    circulant_similarity!(S, simfun, x, y)
    return S
end

"""scale * circulant_similarity(simfun, x, y, W): the q ./ sqrt(τ), k ./ sqrt(τ)
of src/attention.jl:20-21 folded into the similarity (its own rrule)."""
function scaled_similarity(simfun::AbstractSimilarity, x::AbstractArray{T,N}, y::AbstractArray{T,N}, W::Integer, scale::Real) where {T,N}
    S = Circulant(Int(W), (size(x)[1:N-2]..., 1, size(x, N)))
    return similarity_into!(S, simfun, x, y, scale)
end

function circulant_softmax!(Y::CircCSR, X::CircCSR=Y)
    @assert size(Y) == size(X) "softmax!(A, B): A and B must have the same size"
    K = slots(X)
    check(circatt_softmax(Int64(K), Int64(length(X.nzVal) ÷ K), cfloat_ptr(X.nzVal),
                          cfloat_ptr(Y.nzVal), stream_ptr()), "circatt_softmax")
    return Y
end
circulant_softmax(X::CircCSR) = circulant_softmax!(similar(X), X)

function NNlib.softmax!(A::Circulant{T,N,M}, B::Circulant{T,N,M}=A) where {T,N,M}
    circulant_softmax!(A.data, B.data)
    return A
end

"""
    NNlib.softmax(A::Circulant)

A new `Circulant` whose rows (the W^S window slots of each pixel) are
normalised by a softmax.
"""
function NNlib.softmax(A::Circulant)
    data = circulant_softmax(A.data)
    return Circulant(data, kernel_length(A), spatial_size(A))
end

function circulant_adjacency!(A::Circulant, simfun, x, y)
    circulant_similarity!(A, simfun, x, y)
    NNlib.softmax!(A)
    return A
end

"""
    circulant_adjacency(simfun::AbstractSimilarity, x, y, W::Int)

The row-softmax of `circulant_similarity(simfun, x, y, W)`: each row holds
the attention weights of one pixel over its window.

See also [`circulant_similarity`](@ref), [`NNlib.softmax`](@ref).
"""
function circulant_adjacency(simfun::AbstractSimilarity, x, y, W::Integer)
    A = circulant_similarity(simfun, x, y, W)
    B = NNlib.softmax(A)
    return B
end
