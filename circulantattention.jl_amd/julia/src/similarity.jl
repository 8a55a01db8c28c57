# Similarity, softmax and adjacency (reference: src/similarity.jl:1-161) on
# libcircatt: circatt_similarity writes nzVal in place in the reference's CSR
# order, circatt_softmax normalises each row's K slots.

abstract type AbstractSimilarity end

@doc raw"""
    DotSimilarity()

Used in `circulant_attention`, `circulant_similarity`, and `circulant_adjacency` to indicate use of
dot-product similarity:

``
    S_{ij} = \mathrm{Real}(q[i]^H k[j]).
``

See also [`DistanceSimilarity`](@ref).
"""
struct DotSimilarity <: AbstractSimilarity end

@doc raw"""
    DistanceSimilarity()

Used in `circulant_attention`, `circulant_similarity`, and `circulant_adjacency` to indicate use of
distance similarity (the reference's kernel computes the negated half, src/similarity.jl:55-78):

``
    S_{ij} = -\frac{1}{2}\mathrm{sum}(\mathrm{abs2}, q[i] - k[j]).
``

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

Returns Circulant matrix with circulant-sparse data. Each non-zero `S[i,j,b]` is
populated by `simfun` evaluated at the linearized pixel locations of `x` and `y`,
i.e. `S[i,j,b] = simfun(x[...,i,b], y[...,j,b], W)` for max(i⃗, j⃗) ≤ W.

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

Row-wise softmax of Circulant matrix `A`.
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

Equivalent to `(softmax ∘ circulant_similarity)(simfun, x, y, W)`.

See also [`circulant_similarity`](@ref), [`NNlib.softmax`](@ref).
"""
function circulant_adjacency(simfun::AbstractSimilarity, x, y, W::Integer)
    A = circulant_similarity(simfun, x, y, W)
    B = NNlib.softmax(A)
    return B
end
