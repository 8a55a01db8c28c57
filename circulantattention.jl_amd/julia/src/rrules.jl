# ChainRules of the path (reference: src/rrules.jl:1-114), with every pullback
# a libcircatt call: circatt_similarity_bwd (both products and, for Distance,
# the row and column sums of dS in one call), circatt_softmax_bwd,
# circatt_similarity (∂A of ⊗) and circatt_apply (its ∂x), circatt_axpby and
# circatt_batch_dot (scale), circatt_fused_bwd (fused attention).

"""Cotangent on device memory shaped like `like` (dense ROCArray): a
ROCArray as is, a constant (Fill) filled on the device, a host array
uploaded; anything else is rejected rather than staged through the host."""
as_device(Δ::ROCArray, like) = Δ
as_device(Δ::Zygote.FillArrays.Fill, like) = dfill!(similar(like), Δ.value)
function as_device(Δ::Array, like)
    @assert size(Δ) == size(like) "cotangent of size $(size(Δ)) for an output of size $(size(like))"
    return reshape(upload(convert(Array{eltype(like)}, Δ)), size(like))
end
as_device(Δ::AbstractArray, like) = throw(ArgumentError(
    "libcircatt takes device cotangents (ROCArray), a Fill or a host Array; got $(typeof(Δ))"))

cotangent_nzval(Δ::Circulant) = Δ.data.nzVal
cotangent_nzval(Δ::CircCSR) = Δ.nzVal

"""dx, dy of nzVal = scale * simfun(x, y) for the cotangent ΔS (a Circulant
on the same pattern)."""
function similarity_pullback(simfun, x::AbstractArray{T,N}, y, W, scale, ΔS) where {T,N}
    spat = size(x)[1:N-2]
    nsp, n1, n2 = geom(spat)
    dx, dy = similar(x), similar(y)
    dS = cotangent_nzval(ΔS)
    check(circatt_similarity_bwd(simkind(simfun), dtype_code(T), nsp, n1, n2, Int32(W),
                                 Int64(size(x, N-1)), Int64(size(x, N)), Cfloat(scale),
                                 cfloat_ptr(dS), cvoid_ptr(x), cvoid_ptr(y), cvoid_ptr(dx),
                                 cvoid_ptr(dy), stream_ptr()), "circatt_similarity_bwd")
    return dx, dy
end

# Distance (src/rrules.jl:1-16): ∂x = ΔS ⊠ Y - rowsum(ΔS) .* X, ∂y = ΔSᵀ ⊠ X - colsum(ΔS) .* Y
# Dot (src/rrules.jl:18-32):      ∂x = ΔS ⊠ Y,                ∂y = ΔSᵀ ⊠ X
function CRC.rrule(::typeof(circulant_similarity), simfun::AbstractSimilarity, x::AbstractArray{T,N}, y::AbstractArray{T,N}, W) where {T,N}
    project_x = CRC.ProjectTo(x)
    project_y = CRC.ProjectTo(y)
    function sim_pullback(dS)
        dx, dy = similarity_pullback(simfun, x, y, W, 1f0, CRC.unthunk(dS))
        return (CRC.NoTangent(), CRC.NoTangent(), project_x(dx), project_y(dy), CRC.NoTangent())
    end
    S = circulant_similarity(simfun, x, y, W)
    return S, sim_pullback
end

# the q ./ sqrt(τ), k ./ sqrt(τ) of src/attention.jl:20-21 and their
# broadcast pullbacks, folded into the similarity's scale
function CRC.rrule(::typeof(scaled_similarity), simfun::AbstractSimilarity, x::AbstractArray{T,N}, y::AbstractArray{T,N}, W, scale) where {T,N}
    project_x = CRC.ProjectTo(x)
    project_y = CRC.ProjectTo(y)
    function scaled_sim_pullback(dS)
        dx, dy = similarity_pullback(simfun, x, y, W, scale, CRC.unthunk(dS))
        return (CRC.NoTangent(), CRC.NoTangent(), project_x(dx), project_y(dy), CRC.NoTangent(), CRC.NoTangent())
    end
    S = scaled_similarity(simfun, x, y, W, scale)
    return S, scaled_sim_pullback
end

function CRC.rrule(::typeof(_circulant_reshape), X::Circulant{T,N,M}, dims...) where {T,N,M}
    project_X = CRC.ProjectTo(X)
    function reshape_pullback(dX)
        return (CRC.NoTangent(), project_X(reshape(CRC.unthunk(dX), size(X)...)), map(_->CRC.NoTangent(), dims)...)
    end
    return reshape(X, dims...), reshape_pullback
end

# src/rrules.jl:42-56: dS = A .* (dA .- sum(A .* dA; dims=slots))
function CRC.rrule(::typeof(NNlib.softmax), X::Circulant{T, N, M}) where {T, N, M}
    Y = NNlib.softmax(X)
    project_X = CRC.ProjectTo(X)
    function softmax_pullback(∂Y)
        ΔY = CRC.unthunk(∂Y)
        K = slots(X.data)
        dV = similar(Y.data.nzVal)
        check(circatt_softmax_bwd(Int64(K), Int64(length(dV) ÷ K), cfloat_ptr(Y.data.nzVal),
                                  cfloat_ptr(cotangent_nzval(ΔY)), cfloat_ptr(dV), stream_ptr()),
              "circatt_softmax_bwd")
        data = CircCSR(X.data.rowPtr, X.data.colVal, dV, size(X))
        ΔZ = Circulant(data, kernel_length(X), spatial_size(X))
        return (CRC.NoTangent(), project_X(ΔZ))
    end
    return Y, softmax_pullback
end

# src/rrules.jl:58-72: ∂A = Dot similarity of (Δc, b) on A's pattern, ∂b = Aᵀ ⊗ Δc
function CRC.rrule(::typeof(circulant_attention), A::Circulant{T, N, M}, b::AbstractArray{Tb,Nb}) where {T, N, M, Tb, Nb}
    project_A = CRC.ProjectTo(A)
    project_b = CRC.ProjectTo(b)
    function circulant_attention_pullback(dc)
        Δc = as_device(CRC.unthunk(dc), b)
        ∂A = CRC.@thunk project_A(reshape(circulant_similarity(DotSimilarity(), Δc, b, M), size(A)...))
        ∂b = CRC.@thunk project_b(circulant_transposed_attention(A, Δc))
        return (CRC.NoTangent(), ∂A, ∂b)
    end
    return A ⊗ b, circulant_attention_pullback
end

function CRC.rrule(::typeof(circulant_transposed_attention), A::Circulant{T, N, M}, b::AbstractArray{Tb,Nb}) where {T, N, M, Tb, Nb}
    project_A = CRC.ProjectTo(A)
    project_b = CRC.ProjectTo(b)
    function circulant_transposed_attention_pullback(dc)
        Δc = as_device(CRC.unthunk(dc), b)
        ∂A = CRC.@thunk project_A(reshape(circulant_similarity(DotSimilarity(), b, Δc, M), size(A)...))
        ∂b = CRC.@thunk project_b(A ⊗ Δc)
        return (CRC.NoTangent(), ∂A, ∂b)
    end
    return circulant_transposed_attention(A, b), circulant_transposed_attention_pullback
end

function LinearAlgebra.dot(f::Zygote.FillArrays.Fill{T,N}, A::Circulant{T,N}) where {T,N}
    return f.value * sum(A)
end

"""A Circulant on A's pattern with batch size sz[3:end] and every value v
(a constant cotangent made a Circulant on the device)."""
function filled_like(A::Circulant, sz::Tuple, v)
    C = Circulant{Float32}(kernel_length(A), (spatial_size(A)..., sz[3:end]...))
    dfill!(C.data.nzVal, v)
    return C
end

_scale_collectnz(X::Circulant) = X.data.nzVal
_scale_collectnz(X::Zygote.FillArrays.Fill) = X.value

# src/rrules.jl:94-114
function CRC.rrule(::typeof(scale), c::AbstractArray{T,N}, A::Circulant{T,N}) where {T,N}
    project_c = CRC.ProjectTo(c)
    project_A = CRC.ProjectTo(A)
    function scale_pullback(dB)
        ΔB = CRC.unthunk(dB)
        ∂c = CRC.@thunk begin
            # per-slice dots of ΔB with A (A broadcast to ΔB's batch), then
            # summed over the batch dims where c has size 1, all on the device
            bs = size(ΔB)[3:end]
            ab = ntuple(i -> size(A, i + 2), length(bs))
            Anz = reshape(A.data.nzVal, :, ab...)
            Ab = ab == bs ? Anz : dbroadcast(Anz, (size(Anz, 1), bs...))
            nb = prod(bs; init=1)
            g = _scale_collectnz(ΔB)
            per = if g isa Number
                d = batch_dot(Ab, nothing, nb)
                axpby!(d, Float32(g), d, nothing, nothing, 1)
            else
                batch_dot(g, Ab, nb)
            end
            s = reshape(per, bs...)
            for d in 1:length(bs)
                size(c, d + 2) == 1 && bs[d] > 1 && (s = dsum(s, d))
            end
            project_c(reshape(s, size(c)...))
        end
        ∂A = CRC.@thunk begin
            ΔBc = ΔB isa Zygote.FillArrays.Fill ? filled_like(A, size(ΔB), ΔB.value) : ΔB
            sumdims = filter(d -> size(A,d)==1, 1:ndims(A))
            project_A(sum(scale(c, ΔBc); dims=sumdims))
        end
        return (CRC.NoTangent(), ∂c, ∂A)
    end
    return scale(c, A), scale_pullback
end

# fused attention (no A): circatt_fused_bwd recomputes the probabilities from
# the forward's log-sum-exp; the result equals the composition of the rules
# above for y
function CRC.rrule(::typeof(fused_attention), simfun::AbstractSimilarity, q::AbstractArray{T,N}, k, v, W::Int, nheads::Int, cl::Bool=false) where {T,N}
    y, lse = fused_forward(simfun, q, k, v, W, nheads, cl)
    function fused_attention_pullback(Δy)
        dy = as_device(CRC.unthunk(Δy), y)
        dq, dk, dv = fused_backward(simfun, q, k, v, y, dy, lse, W, nheads, cl)
        return (CRC.NoTangent(), CRC.NoTangent(), dq, dk, dv, CRC.NoTangent(), CRC.NoTangent(), CRC.NoTangent())
    end
    return y, fused_attention_pullback
end
