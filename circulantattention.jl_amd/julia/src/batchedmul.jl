# NNlib.batched_mul(!) with a Circulant on the left (reference:
# src/batchedmul.jl:13-41): a (P, P, nb) Circulant, possibly wrapped in
# batched_transpose / batched_adjoint, times a dense (P, C, nb) array.  The
# product is circatt_apply; real nzVal times a complex right-hand side needs
# no promotion copy of A (the reference's src/batchedmul.jl:43-80 converts A).
# nzVal is real, so the adjoint is the transpose.

const CircT = NNlib.BatchedTranspose{T, <:Circulant} where {T}
const CircA = NNlib.BatchedAdjoint{T, <:Circulant} where {T}

circ_and_trans(A::Circulant) = (A, false)
circ_and_trans(A::CircT) = (parent(A), true)
circ_and_trans(A::CircA) = (parent(A), true)

function circ_mul!(C::AbstractArray{T,3}, A, B::AbstractArray{T,3}) where {T}
    Ac, trans = circ_and_trans(A)
    @assert size(B, 1) == size(Ac, 1) && size(B, 3) == nbatch(Ac) "batched_mul: size mismatch"
    return apply!(C, Ac, B, trans)
end

NNlib.batched_mul(A::Circulant, B::AbstractArray{T,3}) where {T} = circ_mul!(similar(B), A, B)
NNlib.batched_mul(A::CircT, B::AbstractArray{T,3}) where {T} = circ_mul!(similar(B), A, B)
NNlib.batched_mul(A::CircA, B::AbstractArray{T,3}) where {T} = circ_mul!(similar(B), A, B)

NNlib.batched_mul!(C::AbstractArray{T,3}, A::Circulant, B::AbstractArray{T,3}) where {T} = circ_mul!(C, A, B)
NNlib.batched_mul!(C::AbstractArray{T,3}, A::CircT, B::AbstractArray{T,3}) where {T} = circ_mul!(C, A, B)
NNlib.batched_mul!(C::AbstractArray{T,3}, A::CircA, B::AbstractArray{T,3}) where {T} = circ_mul!(C, A, B)
