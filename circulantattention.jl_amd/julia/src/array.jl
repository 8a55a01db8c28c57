# The Circulant type (reference: src/array.jl:1-189) over a batched CSR held
# in ROCArrays.  The CSR keeps the field names the reference's code and tests
# read from CUDA.jl's CuSparseArrayCSR -- rowPtr (P+1, batch...), colVal
# (P*K, batch...), nzVal (P*K, batch...), dims, nnz -- and nzVal stays
# assignable (test/rrule.jl:10-12 replaces it).  Indices are Int32 and
# 1-based, bit-identical to the reference's (circatt_pattern); values are
# Float32.

"""Batched CSR of a Circulant: (P, P, batch...) with K slots per row."""
mutable struct CircCSR{T, N, V<:AbstractArray{T}, I<:AbstractArray{Int32}} <: AbstractArray{T, N}
    rowPtr::I
    colVal::I
    nzVal::V
    dims::NTuple{N, Int}
end
CircCSR(rowPtr::I, colVal::I, nzVal::V, dims::NTuple{N,Int}) where {T, N, V<:AbstractArray{T}, I} =
    CircCSR{T, N, V, I}(rowPtr, colVal, nzVal, dims)

Base.size(A::CircCSR) = A.dims
Base.size(A::CircCSR, i::Integer) = i <= length(A.dims) ? A.dims[i] : 1
Base.eltype(::CircCSR{T}) where {T} = T
function Base.getproperty(A::CircCSR, s::Symbol)
    s === :nnz && return length(getfield(A, :nzVal))
    return getfield(A, s)
end
Base.copy(A::CircCSR) = CircCSR(dcopy(A.rowPtr), dcopy(A.colVal), dcopy(A.nzVal), A.dims)
Base.similar(A::CircCSR) = CircCSR(dcopy(A.rowPtr), dcopy(A.colVal), similar(A.nzVal), A.dims)

nbatch(A::CircCSR) = prod(A.dims[3:end]; init=1)
slots(A::CircCSR) = length(A.nzVal) ÷ (A.dims[1] * nbatch(A))   # K

# scalar reads copy row i's slots to the host one by one (debugging and
# printing only)
function Base.getindex(A::CircCSR{T,N}, I::Vararg{Int,N}) where {T,N}
    i, j = I[1], I[2]
    b = LinearIndices(A.dims[3:end])[I[3:end]...]
    K = slots(A)
    base = (b - 1) * A.dims[1] * K + (i - 1) * K
    s = zero(T)
    for t in 1:K
        read_scalar(A.colVal, base + t) == j && (s += read_scalar(A.nzVal, base + t))
    end
    return s
end

# the reference's == of two CSR arrays (src/array.jl:87-101): sizes, then
# nzVal, rowPtr and colVal element by element, compared on the device
function Base.:(==)(A::CircCSR, B::CircCSR)
    size(A) == size(B) || return false
    return count_unequal(A.nzVal, B.nzVal) == 0 && count_unequal(A.rowPtr, B.rowPtr) == 0 &&
           count_unequal(A.colVal, B.colVal) == 0
end

function Base.show(io::IO, ::MIME"text/plain", A::CircCSR)
    print(io, join(size(A), "×"), " batched CSR with $(A.nnz) stored entries (",
          eltype(A.nzVal), " nzVal, Int32 rowPtr and colVal) on ", AMDGPU.device())
end
Base.show(io::IO, A::CircCSR) = print(io, join(size(A), "×"), " batched CSR")

"""Pattern of a Circulant with kernel length M over spatial size spatsize,
replicated over batchsize: rowPtr, colVal from circatt_pattern
(cucirculant + repeat, src/circulant.jl:46-106, src/array.jl:6-11), nzVal = 1."""
function circulant_csr(::Type{T}, M::Int, spatsize::NTuple{S,Int}, batchsize::Tuple) where {T, S}
    @assert isodd(M) "filter size M=$M must be odd."
    T === Float32 || throw(ArgumentError("libcircatt stores Circulant values as Float32, got $T"))
    nsp, n1, n2 = geom(spatsize)
    P = prod(spatsize)
    K = M^S
    nb = prod(batchsize; init=1)
    rowPtr = ROCArray{Int32}(undef, P + 1, batchsize...)
    colVal = ROCArray{Int32}(undef, P * K, batchsize...)
    check(circatt_pattern(nsp, n1, n2, Int32(M), Int64(nb), dptr(rowPtr), dptr(colVal),
                          stream_ptr()), "circatt_pattern")
    nzVal = dfill!(ROCArray{Float32}(undef, P * K, batchsize...), 1f0)
    return CircCSR(rowPtr, colVal, nzVal, (P, P, batchsize...))
end

struct Circulant{T, N, M, S, A<:AbstractArray{T, N}} <: AbstractArray{T, N}
    data::A
    kernel_length::Int
    spatial_size::NTuple{S, Int}

    function Circulant{T}(M::Int, dims::NTuple{N,Int}) where {T,N}
        spatsize, batchsize = dims[1:N-2], dims[N-1:end]
        data = circulant_csr(T, M, spatsize, batchsize)
        Circulant(data, M, spatsize)
    end
    function Circulant(M::Int, dims::NTuple{N,Int}) where N
        Circulant{Float32}(M, dims)
    end
    function Circulant(D::A, M::Int, spatsize::NTuple{S,Int}) where {T, N, S, A<:AbstractArray{T,N}}
        new{T, N, M, S, A}(D, M, spatsize)
    end
end
Circulant(A::Circulant) = A
Circulant(a::T, M, spatdims) where T <: Number = a

function Adapt.adapt_structure(to, A::CircCSR)
    CircCSR(Adapt.adapt(to, A.rowPtr), Adapt.adapt(to, A.colVal), Adapt.adapt(to, A.nzVal), A.dims)
end
function Adapt.adapt_structure(to, A::Circulant{T, N, M}) where {T, N, M}
    Circulant(Adapt.adapt_structure(to, A.data), M, A.spatial_size)
end

# eager release of a Circulant's device arrays (the reference's
# CUDA.unsafe_free!, src/array.jl:27)
function AMDGPU.unsafe_free!(A::CircCSR)
    AMDGPU.unsafe_free!(A.rowPtr)
    AMDGPU.unsafe_free!(A.colVal)
    AMDGPU.unsafe_free!(A.nzVal)
    return nothing
end
AMDGPU.unsafe_free!(A::Circulant) = AMDGPU.unsafe_free!(A.data)

"""circulant(M, x): a Circulant shaped for signal x (src/array.jl:29)."""
circulant(M::Int, x::AbstractArray{T, N}) where {T,N} =
    Circulant{real(T)}(M, (size(x)[1:N-2]..., 1, size(x,N)))

kernel_length(A::Circulant{T, N, M}) where {T, N, M} = M
spatial_dims(A::Circulant{T, N, M, S}) where {T, N, M, S} = S
spatial_size(A::Circulant) = A.spatial_size

Base.eltype(A::Circulant{T}) where T = T
Base.size(A::Circulant) = size(A.data)
Base.size(A::Circulant, i::Int) = size(A.data, i)
Base.ndims(A::Circulant) = ndims(A.data)
Base.getindex(A::Circulant, idxs...) = Base.getindex(A.data, idxs...)

Base.similar(A::Circulant{T, N, M}) where {T, N, M} = Circulant(similar(A.data), M, spatial_size(A))
Base.copy(A::Circulant{T, N, M}) where {T, N, M} = Circulant(copy(A.data), M, spatial_size(A))

function Base.show(io::IO, m::MIME"text/plain", A::Circulant{T, N, M}) where {T, N, M}
    print(io, typeof(A), " with kernel-length $M, spatial-size $(spatial_size(A)), and data,\n")
    show(io, m, A.data)
end
Base.show(io::IO, A::Circulant{T, N, M}) where {T, N, M} =
    print(io, "Circulant(", join(size(A), "×"), ", kernel-length $M)")

nbatch(A::Circulant) = nbatch(A.data)

# ---- shape utilities (src/array.jl:49-64) ----------------------------------

"""Batch dims after reshape(A, dims...): the first two dims stay (P, P)
(Colon or P), the rest redistribute the batch; one Colon may absorb it."""
function batch_reshape(A::CircCSR, dims)
    P = A.dims[1]
    length(dims) >= 2 || throw(DimensionMismatch("a Circulant keeps its two (P, P) dims"))
    for d in dims[1:2]
        (d isa Colon || d == P) || throw(DimensionMismatch("a Circulant keeps its two (P, P) dims"))
    end
    rest = collect(Any, dims[3:end])
    nb = nbatch(A)
    known = prod(Int[d for d in rest if !(d isa Colon)]; init=1)
    ncolon = count(d -> d isa Colon, rest)
    ncolon <= 1 || throw(DimensionMismatch("at most one Colon among the batch dims"))
    out = Int[d isa Colon ? nb ÷ known : d for d in rest]
    prod(out; init=1) == nb || throw(DimensionMismatch("cannot reshape batch $(A.dims[3:end]) to $(Tuple(out))"))
    return Tuple(out)
end

function Base.reshape(A::CircCSR, dims::Union{Colon,Int}...)
    bs = batch_reshape(A, dims)
    rp = reshape(A.rowPtr, size(A.rowPtr, 1), bs...)
    cv = reshape(A.colVal, size(A.colVal, 1), bs...)
    nz = reshape(A.nzVal, size(A.nzVal, 1), bs...)
    return CircCSR(rp, cv, nz, (A.dims[1], A.dims[2], bs...))
end

function Base.reshape(A::Circulant{T, N, M}, dims::Union{Colon,Int}...) where {T, N, M}
    Circulant(reshape(A.data, dims...), M, spatial_size(A))
end

function _circulant_reshape(A::Circulant{T, N, M}, dims...) where {T, N, M}
    reshape(A, dims...)
end

# Julia's repeat over the batch dims (src/array.jl:9,49-52), on the device
function Base.repeat(A::CircCSR, counts::Int...)
    (length(counts) >= 2 && counts[1] == 1 && counts[2] == 1) ||
        throw(ArgumentError("repeat(A, 1, 1, counts...): the (P, P) dims of a Circulant cannot be repeated"))
    bc = counts[3:end]
    rp = drepeat(A.rowPtr, bc...)
    cv = drepeat(A.colVal, bc...)
    nz = drepeat(A.nzVal, bc...)
    return CircCSR(rp, cv, nz, (A.dims[1], A.dims[2], size(nz)[2:end]...))
end

function Base.repeat(A::Circulant{T, N, M}, dims::Int...) where {T, N, M}
    data = Base.repeat(A.data, dims...)
    Circulant(data, M, spatial_size(A))
end

# The reference's cat refers to an undefined A (src/array.jl:63) and throws;
# here the first argument's spatial size is taken.
function Base.cat(As::Circulant{T, N, M}...; dims=3) where {T, N, M}
    dims isa Integer && dims >= 3 || throw(ArgumentError("cat of Circulants joins batch dims (dims >= 3)"))
    d = dims - 1
    rp = dcat((A.data.rowPtr for A in As)...; dims=d)
    cv = dcat((A.data.colVal for A in As)...; dims=d)
    nz = dcat((A.data.nzVal for A in As)...; dims=d)
    P = size(As[1], 1)
    Circulant(CircCSR(rp, cv, nz, (P, P, size(nz)[2:end]...)), M, spatial_size(As[1]))
end

# ---- algebra on nzVal (src/array.jl:66-81, 179-189) ------------------------

"""Z = alpha X + beta Y over nb slices of nzVal (circatt_axpby); alpha, beta
are numbers or per-slice Float32 ROCArrays; Y may be nothing."""
function axpby!(Z::ROCArray{Float32}, alpha, X::ROCArray{Float32}, beta, Y, nb::Integer)
    nnz = length(X) ÷ nb
    a_ptr = alpha isa Number ? Ptr{Cfloat}(C_NULL) : cfloat_ptr(alpha)
    b_ptr = beta isa Number || beta === nothing ? Ptr{Cfloat}(C_NULL) : cfloat_ptr(beta)
    a0 = alpha isa Number ? Cfloat(alpha) : 0f0
    b0 = beta isa Number ? Cfloat(beta) : 0f0
    check(circatt_axpby(Int64(nnz), Int64(nb), a_ptr, a0, cfloat_ptr(X), b_ptr, b0,
                        Y === nothing ? Ptr{Cfloat}(C_NULL) : cfloat_ptr(Y), cfloat_ptr(Z),
                        stream_ptr()), "circatt_axpby")
    return Z
end

with_nzval(X::Circulant{T, N, M}, nz) where {T, N, M} =
    Circulant(CircCSR(dcopy(X.data.rowPtr), dcopy(X.data.colVal), nz, size(X)), M, spatial_size(X))

function Base.:(+)(X::Circulant{T, N, M}, Y::Circulant{T, N, M}) where {T, N, M}
    @assert size(X) == size(Y) "Circulant + Circulant needs equal sizes"
    with_nzval(X, axpby!(similar(X.data.nzVal), 1f0, X.data.nzVal, 1f0, Y.data.nzVal, 1))
end

function Base.:(-)(X::Circulant{T, N, M}, Y::Circulant{T, N, M}) where {T, N, M}
    @assert size(X) == size(Y) "Circulant - Circulant needs equal sizes"
    with_nzval(X, axpby!(similar(X.data.nzVal), 1f0, X.data.nzVal, -1f0, Y.data.nzVal, 1))
end

function Base.:(*)(c::Number, X::Circulant)
    with_nzval(X, axpby!(similar(X.data.nzVal), Float32(c), X.data.nzVal, nothing, nothing, 1))
end
Base.:(-)(A::Circulant) = -1*A
Base.:(*)(A::Circulant, c::Number) = c*A

"""(nb,) sums over nb slices of X .* Y (of X without Y), circatt_batch_dot."""
function batch_dot(X::ROCArray{Float32}, Y, nb::Integer)
    nnz = length(X) ÷ nb
    out = ROCArray{Float32}(undef, nb)
    wb = circatt_batch_dot_workspace_bytes(Int64(nnz), Int64(nb))
    work = ROCArray{Float64}(undef, cld(wb, 8))
    check(circatt_batch_dot(Int64(nnz), Int64(nb), cfloat_ptr(X),
                            Y === nothing ? Ptr{Cfloat}(C_NULL) : cfloat_ptr(Y), cfloat_ptr(out),
                            cvoid_ptr(work), Int64(wb), stream_ptr()), "circatt_batch_dot")
    return out
end

function LinearAlgebra.dot(X::Circulant, Y::Circulant)
    @assert size(X) == size(Y) "dot needs equal sizes"
    return read_scalar(batch_dot(X.data.nzVal, Y.data.nzVal, 1))
end

function Base.:(==)(A::Circulant, B::Circulant)
    if axes(A) != axes(B)
        return false
    end
    if spatial_size(A) != spatial_size(B)
        return false
    end
    if kernel_length(A) != kernel_length(B)
        return false
    end
    if A.data != B.data
        return false
    end
    return true
end

# ---- sums (src/array.jl:119-177) -------------------------------------------

"""sum over the K slots of each row (dims=2) or over each column (dims=1):
(P, nb) Float32 from circatt_rowsum / circatt_colsum."""
function rowcol_sum(A::Circulant, col::Bool)
    nsp, n1, n2 = geom(spatial_size(A))
    nb = nbatch(A)
    out = ROCArray{Float32}(undef, size(A, 1), nb)
    f = col ? circatt_colsum : circatt_rowsum
    check(f(nsp, n1, n2, Int32(kernel_length(A)), Int64(nb), cfloat_ptr(A.data.nzVal),
            cfloat_ptr(out), stream_ptr()), col ? "circatt_colsum" : "circatt_rowsum")
    return out
end

"""nzVal summed over batch dims `sdims` (Julia dims >= 3; circatt_sum_middle),
the indices of the first slice kept (src/array.jl:132-154)."""
function sum_batchdims(A::CircCSR, sdims)
    nz, rp, cv = A.nzVal, A.rowPtr, A.colVal
    for d in sort(collect(sdims); rev=true)
        ax = d - 1  # dim of nzVal
        nz = dsum(nz, ax)
        rp = dfirst(rp, ax)
        cv = dfirst(cv, ax)
    end
    return CircCSR(rp, cv, nz, (A.dims[1], A.dims[2], size(nz)[2:end]...))
end

function Base.sum(A::Circulant; dims=:)
    nb = nbatch(A)
    bs = size(A)[3:end]
    if dims isa Colon
        return read_scalar(batch_dot(A.data.nzVal, nothing, 1))
    end
    d = dims isa Integer ? (Int(dims),) : Tuple(Int(x) for x in dims)
    if all(>(2), d)
        return Circulant(sum_batchdims(A.data, d), kernel_length(A), spatial_size(A))
    elseif d == (1,)
        return reshape(rowcol_sum(A, true), 1, size(A, 1), bs...)
    elseif d == (2,)
        return reshape(rowcol_sum(A, false), size(A, 1), 1, bs...)
    elseif d == (1, 2)
        return reshape(batch_dot(A.data.nzVal, nothing, nb), 1, 1, bs...)
    else
        throw(ErrorException("dims=$dims not implemented."))
    end
end

# ---- scale (src/array.jl:179-189) ------------------------------------------

"""scale(c, A) = c .* A with c of size (1, 1, batch...) broadcast against A's
batch dims (src/array.jl:179-189): the factors and A's arrays broadcast on
the device, then circatt_axpby with one factor per slice."""
function scale(c::ROCArray{Tc}, A::Circulant{Ta, N, M}) where {Tc<:Real, Ta, N, M}
    @assert size(c, 1) == 1 && size(c, 2) == 1 "Scaling of non-batchdims of CuSparseArrayCSR not implemented"
    nd = max(ndims(c), ndims(A)) - 2
    cb = ntuple(i -> size(c, i + 2), nd)
    ab = ntuple(i -> size(A, i + 2), nd)
    rb = ntuple(i -> max(cb[i], ab[i]), nd)
    for i in 1:nd
        (cb[i] == rb[i] || cb[i] == 1) && (ab[i] == rb[i] || ab[i] == 1) ||
            throw(DimensionMismatch("cannot broadcast scale factor $cb against batch $ab"))
    end
    Tc === Float32 || throw(ArgumentError("libcircatt scale factors are Float32, got $Tc"))
    X = dbroadcast(reshape(A.data.nzVal, :, ab...), (size(A.data.nzVal, 1), rb...))
    if ab == rb  # the new Circulant gets its own index arrays, as the reference's copies
        rp, cv = dcopy(A.data.rowPtr), dcopy(A.data.colVal)
    else
        rp = dbroadcast(reshape(A.data.rowPtr, :, ab...), (size(A.data.rowPtr, 1), rb...))
        cv = dbroadcast(reshape(A.data.colVal, :, ab...), (size(A.data.colVal, 1), rb...))
    end
    alpha = dbroadcast(reshape(c, cb...), rb)
    Z = axpby!(similar(X), vec(alpha), X, nothing, nothing, prod(rb; init=1))
    P = size(A, 1)
    return Circulant(CircCSR(rp, cv, Z, (P, P, rb...)), M, spatial_size(A))
end
scale(c::Number, A::Circulant) = c * A
scale(c::Array, A::Circulant) = scale(upload(Float32.(c)), A)

Base.:(*)(c::ROCArray, A::Circulant) = scale(c, A)
