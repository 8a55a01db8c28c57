# Attention and the ⊗ / ⨷ applies (reference: src/attention.jl:1-103).
# Unfused forms return the adjacency A like the reference; with
# materialize=false the fused libcircatt kernels compute y without forming A
# (circatt_fused_fwd / circatt_fused_bwd) and `nothing` is returned for A.

@doc raw"""
    y, A = circulant_attention(simfun::AbstractSimilarity, q, k, v, W::Int; materialize=true)

Sliding-window attention with circular boundaries: `A` is the adjacency of
`q` against `k` (`simfun` scores over each pixel's W-wide window, row
softmax) and `y = A ⊗ v`.  Both `q` and `k` are divided by the fourth root of
the channel count first, so the scores carry a factor ``1/\sqrt{C}``.  With
`materialize=false` the fused kernels produce `y` without forming `A`, which
is then returned as `nothing`.
"""
function circulant_attention(simfun::AbstractSimilarity, q::T, k::T, v::T, W::Int; materialize::Bool=true,
                             channels_last::Bool=false) where {Tv, N, T<: AbstractArray{Tv,N}}
    if !materialize || channels_last
        @assert !materialize "channels_last needs materialize=false (the fused kernels)"
        return (fused_attention(simfun, q, k, v, W, 1, channels_last), nothing)
    end
    τ = sqrt(real(Tv)(size(k, N-1)))
    # q ./ sqrt(τ), k ./ sqrt(τ) (src/attention.jl:20-21) scale the similarity by 1/τ
    S = scaled_similarity(simfun, q, k, W, 1 / τ)
    A = NNlib.softmax(S)
    y = A ⊗ v
    return y, A
end
circulant_attention(q::T, k::T, v::T, W::Int; kws...) where T = circulant_attention(DotSimilarity(), q, k, v, W; kws...)

@doc raw"""
    y, A = circulant_mh_attention(simfun::AbstractSimilarity, q, k, v, W::Int, nheads::Int;
                                  materialize=true, honor_simfun=false)

Circulant attention per head: the channels of `q`, `k` and `v` split into
`nheads` consecutive groups (the channel count must be a multiple of
`nheads`), each group attended on its own and the outputs placed back in
channel order.  `A` has one (P, P) matrix per head and batch:
`size(A) == (P, P, nheads, B)`.  Like the reference (src/attention.jl:40)
the dot similarity is used whatever `simfun` is, unless `honor_simfun=true`.
"""
function circulant_mh_attention(simfun::AbstractSimilarity, q::T, k::T, v::T, W::Int, nheads::Int;
                                materialize::Bool=true, honor_simfun::Bool=false,
                                channels_last::Bool=false) where {Tv, N, T<: AbstractArray{Tv,N}}
    sim = honor_simfun ? simfun : DotSimilarity()
    Cax = channels_last ? 1 : N-1
    @assert size(q, Cax) % nheads == 0 "channels ($(size(q, Cax))) must be divisible by nheads ($nheads)"
    if !materialize || channels_last
        @assert !materialize "channels_last needs materialize=false (the fused kernels)"
        return (fused_attention(sim, q, k, v, W, nheads, channels_last), nothing)
    end
    qr, kr, vr = splitheads.((q, k, v), nheads)
    yr, A = circulant_attention(sim, qr, kr, vr, W)
    return reshape(yr, size(q)...), _circulant_reshape(A, :, :, nheads, size(q, N))
end
# the reference forwards this form to a method that does not exist
# (src/attention.jl:43); here it means the dot similarity
circulant_mh_attention(q::T, k::T, v::T, W::Int, nheads::Int; kws...) where T =
    circulant_mh_attention(DotSimilarity(), q, k, v, W, nheads; kws...)
splitheads(x::AbstractArray{T,N}, nheads) where {T,N} = reshape(x, ntuple(i->size(x,i), N-2)..., size(x, N-1) ÷ nheads, :)

function circulant_mh_adjacency(simfun, x::AbstractArray{T,N}, y, W::Integer, nheads::Int) where {T, N}
    xr, yr = splitheads.((x, y), nheads)
    A = circulant_adjacency(simfun, xr, yr, W)
    return _circulant_reshape(A, :, :, nheads, size(x, N))
end

"""y = op(A) ⊗ x with op = identity or transpose (circatt_apply); x, y are
(spatial..., C, nb) or (P, C, nb) with nb = A's batch."""
function apply!(y::AbstractArray{T}, A::Circulant, x::AbstractArray{T}, trans::Bool) where {T}
    nsp, n1, n2 = geom(spatial_size(A))
    P, nb = size(A, 1), nbatch(A)
    C = length(x) ÷ (P * nb)
    @assert length(x) == P * C * nb && length(y) == length(x) "x must hold (P, C, $nb) values for A"
    check(circatt_apply(Cint(trans), dtype_code(T), nsp, n1, n2, Int32(kernel_length(A)),
                        Int64(C), Int64(nb), cfloat_ptr(A.data.nzVal), cvoid_ptr(x), cvoid_ptr(y),
                        stream_ptr()), "circatt_apply")
    return y
end

function circulant_attention!(y::AbstractArray{T, N}, A::Circulant{Ta, Na}, x::AbstractArray{T, N}) where {Ta, Na, T, N}
    @assert spatial_dims(A) == N - 2 "spatial-dims ($(spatial_dims(A)) of A must match spatial dims of x ($(N-2))"
    return apply!(y, A, x, false)
end

@doc raw"""
    y = circulant_attention(A::Circulant, x::AbstractArray)
    y = A ⊗ x # \otimes

The product of the sparse circulant matrix `A` (one per batch) with the
pixels-by-channels matrix of `x`; `y` has the size of `x`.
See also [`circulant_adjacency`](@ref).
"""
circulant_attention(A::Circulant, x) = circulant_attention!(similar(x), A, x)

const ⊗ = circulant_attention

function circulant_transposed_attention!(y::AbstractArray{T, N}, A::Circulant{Ta, Na}, x::AbstractArray{T, N}) where {Ta, Na, T, N}
    @assert spatial_dims(A) == N - 2 "spatial-dims ($(spatial_dims(A)) of A must match spatial dims of x ($(N-2))"
    return apply!(y, A, x, true)
end
circulant_transposed_attention(A::Circulant, x) = circulant_transposed_attention!(similar(x), A, x)

@doc raw"""
    y = circulant_mh_attention(A::Circulant, x::AbstractArray)
    y = A ⨷ x # \Otimes

⊗ per head: `A` of size (P, P, nheads, B) applied to the `nheads` channel
groups of `x`.
"""
function circulant_mh_attention(A::Circulant{Ta, 4}, x::AbstractArray{T, N}) where {Ta, T, N}
    nheads = size(A, 3)
    xr = splitheads(x, nheads)
    yr = A ⊗ xr
    return reshape(yr, size(x)...)
end

const ⨷ = circulant_mh_attention

function circulant_mh_transposed_attention(A::Circulant{Ta, 4}, x::AbstractArray{T, N}) where {Ta, T, N}
    nheads = size(A, 3)
    xr = splitheads(x, nheads)
    yr = circulant_transposed_attention(A, xr)
    return reshape(yr, size(x)...)
end

# ---- fused path (no A) -----------------------------------------------------

"""y of circulant (multi-head) attention from the fused kernels, without
forming A; the per-row log-sum-exp is kept for the pullback.  Planar arrays
are (spatial..., C, B); with `cl = true` they are channels-last
(C, spatial..., B), read and written in place (CIRCATT_CHANNELS_LAST)."""
function fused_forward(simfun::AbstractSimilarity, q::AbstractArray{T,N}, k, v, W::Int, nheads::Int, cl::Bool=false) where {T,N}
    spat = cl ? size(q)[2:N-1] : size(q)[1:N-2]
    nsp, n1, n2 = geom(spat)
    C, B = (cl ? size(q, 1) : size(q, N-1)), size(q, N)
    y = similar(q)
    lse = ROCArray{Float32}(undef, prod(spat), nheads * B)
    code = dtype_code(T) | (cl ? CIRCATT_CHANNELS_LAST : Cint(0))
    check(circatt_fused_fwd(simkind(simfun), code, nsp, n1, n2, Int32(W), Int64(C),
                            Int64(nheads), Int64(B), cvoid_ptr(q), cvoid_ptr(k), cvoid_ptr(v),
                            cvoid_ptr(y), cfloat_ptr(lse), stream_ptr()), "circatt_fused_fwd")
    return y, lse
end

fused_attention(simfun, q, k, v, W::Int, nheads::Int, cl::Bool=false) = first(fused_forward(simfun, q, k, v, W, nheads, cl))

function fused_backward(simfun, q::AbstractArray{T,N}, k, v, y, dy, lse, W::Int, nheads::Int, cl::Bool=false) where {T,N}
    spat = cl ? size(q)[2:N-1] : size(q)[1:N-2]
    nsp, n1, n2 = geom(spat)
    C, B = (cl ? size(q, 1) : size(q, N-1)), size(q, N)
    dq, dk, dv = similar(q), similar(k), similar(v)
    wb = circatt_fused_bwd_workspace_bytes(nsp, n1, n2, Int64(nheads), Int64(B))
    work = ROCArray{Float32}(undef, cld(wb, 4))
    code = dtype_code(T) | (cl ? CIRCATT_CHANNELS_LAST : Cint(0))
    check(circatt_fused_bwd(simkind(simfun), code, nsp, n1, n2, Int32(W), Int64(C),
                            Int64(nheads), Int64(B), cvoid_ptr(q), cvoid_ptr(k), cvoid_ptr(v),
                            cvoid_ptr(y), cvoid_ptr(dy), cfloat_ptr(lse), cvoid_ptr(dq),
                            cvoid_ptr(dk), cvoid_ptr(dv), cvoid_ptr(work), Int64(wb),
                            stream_ptr()), "circatt_fused_bwd")
    return dq, dk, dv
end
