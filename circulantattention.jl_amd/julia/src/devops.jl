# Device-array helpers of the Circulant type, every one a libcircatt call
# (circatt_fill, circatt_copy_blocks, circatt_sum_middle,
# circatt_count_unequal, circatt_memcpy): the package launches no array
# kernels of its own.  Arrays are contiguous ROCArrays; sizes below are in
# elements unless named bytes.

"""x .= v on the device (Float32: circatt_fill; other element types: v
uploaded once, then replicated by circatt_copy_blocks)."""
function dfill!(x::ROCArray{Float32}, v)
    check(circatt_fill(cfloat_ptr(x), Int64(length(x)), Cfloat(v), stream_ptr()), "circatt_fill")
    return x
end
function dfill!(x::ROCArray{T}, v) where {T}
    length(x) == 0 && return x
    one = upload(T[convert(T, v)])
    return copy_blocks!(x, one, 1, length(x), 1, 0, 1, 0, 0)
end

"""Strided block copy (circatt_copy_blocks): for o < nouter, i < ninner the
`block` elements at src[src_off + o*sso + i*ssi] go to dst[dst_off + o*dso +
i*dsi] (strides and offsets in elements of T, 0-based)."""
function copy_blocks!(dst::ROCArray{T}, src::ROCArray{T}, block, ninner, dsi, ssi, nouter, dso, sso;
                      dst_off=0, src_off=0) where {T}
    s = sizeof(T)
    check(circatt_copy_blocks(cvoid_ptr(dst) + dst_off * s, cvoid_ptr(src) + src_off * s,
                              Int64(block * s), Int64(ninner), Int64(dsi * s), Int64(ssi * s),
                              Int64(nouter), Int64(dso * s), Int64(sso * s), stream_ptr()),
          "circatt_copy_blocks")
    return dst
end

"""A device copy of x."""
function dcopy(x::ROCArray{T}) where {T}
    y = similar(x)
    length(x) == 0 && return y
    return copy_blocks!(y, x, length(x), 1, 0, 0, 1, 0, 0)
end

"""Julia's repeat(x, 1, counts...) for the batch dims of an (n, batch...)
array: dim j + 1 tiled counts[j] times, one copy per repeated dim."""
function drepeat(x::ROCArray{T}, counts::Int...) where {T}
    sz = collect(size(x))
    nb = max(length(sz) - 1, length(counts))
    append!(sz, ones(Int, nb + 1 - length(sz)))
    cur = x
    for (j, c) in enumerate(counts)
        c == 1 && continue
        inner = prod(sz[1:j+1])
        outer = prod(sz[j+2:end]; init=1)
        sz[j+1] *= c
        out = similar(x, sz...)
        copy_blocks!(out, cur, inner, c, inner, 0, outer, inner * c, inner)
        cur = out
    end
    return cur === x ? reshape(dcopy(x), sz...) : reshape(cur, sz...)
end

"""x with its size-1 dims broadcast to `to` (a size of the same length)."""
function dbroadcast(x::ROCArray{T}, to::Tuple) where {T}
    sz = collect(size(x))
    append!(sz, ones(Int, length(to) - length(sz)))
    cur = reshape(x, sz...)
    for d in eachindex(sz)
        (sz[d] == to[d]) && continue
        sz[d] == 1 || throw(DimensionMismatch("cannot broadcast $(size(x)) to $to"))
        inner = prod(sz[1:d-1]; init=1)
        outer = prod(sz[d+1:end]; init=1)
        sz[d] = to[d]
        out = similar(x, sz...)
        copy_blocks!(out, cur, inner, to[d], inner, 0, outer, inner * to[d], inner)
        cur = out
    end
    return cur
end

"""cat of arrays that agree in every dim but d (circatt_copy_blocks)."""
function dcat(xs::ROCArray{T}...; dims::Int) where {T}
    sz = collect(size(xs[1]))
    append!(sz, ones(Int, dims - length(sz)))
    outer = prod(sz[dims+1:end]; init=1)
    inners = [length(x) ÷ outer for x in xs]
    tot = sum(inners)
    sz[dims] = sum(size(x, dims) for x in xs)
    out = similar(xs[1], sz...)
    off = 0
    for (x, n) in zip(xs, inners)
        copy_blocks!(out, x, n, 1, 0, 0, outer, tot, n; dst_off=off)
        off += n
    end
    return out
end

"""sum over dim d, keeping it as size 1 (circatt_sum_middle: summed in
double in order)."""
function dsum(x::ROCArray{Float32}, d::Int)
    sz = collect(size(x))
    inner = prod(sz[1:d-1]; init=1)
    outer = prod(sz[d+1:end]; init=1)
    n = sz[d]
    sz[d] = 1
    out = similar(x, sz...)
    check(circatt_sum_middle(cfloat_ptr(x), cfloat_ptr(out), Int64(inner), Int64(n),
                             Int64(outer), stream_ptr()), "circatt_sum_middle")
    return out
end

"""The first slice along dim d (selectdim(x, d, 1:1)), as a new array."""
function dfirst(x::ROCArray{T}, d::Int) where {T}
    sz = collect(size(x))
    inner = prod(sz[1:d-1]; init=1)
    outer = prod(sz[d+1:end]; init=1)
    n = sz[d]
    sz[d] = 1
    out = similar(x, sz...)
    return copy_blocks!(out, x, inner, 1, 0, 0, outer, inner, inner * n)
end

"""Number of differing elements (circatt_count_unequal; Float32 compared as
floats, other types as 32-bit words), read back to the host."""
function count_unequal(a::ROCArray{T}, b::ROCArray{T}) where {T}
    @assert length(a) == length(b)
    kind = T === Float32 ? Cint(1) : Cint(0)
    n = length(a) * sizeof(T) ÷ 4
    cnt = ROCArray{Int64}(undef, 1)
    check(circatt_count_unequal(kind, Int64(n), cvoid_ptr(a), cvoid_ptr(b),
                                reinterpret(Ptr{Int64}, dptr(cnt)), stream_ptr()),
          "circatt_count_unequal")
    return read_scalar(cnt)
end

"""The element at 1-based index i of a device array, copied to the host
(circatt_memcpy after the calling task's stream)."""
function read_scalar(x::ROCArray{T}, i::Integer=1) where {T}
    check(circatt_stream_synchronize(stream_ptr()), "circatt_stream_synchronize")
    h = Ref{T}()
    GC.@preserve h check(circatt_memcpy(Base.unsafe_convert(Ptr{Cvoid}, h),
                                        cvoid_ptr(x) + (i - 1) * sizeof(T), Int64(sizeof(T)),
                                        Cint(1)), "circatt_memcpy")
    return h[]
end

"""A host array copied to the device (circatt_memcpy)."""
function upload(h::Array{T}) where {T}
    x = ROCArray{T}(undef, size(h))
    check(circatt_stream_synchronize(stream_ptr()), "circatt_stream_synchronize")
    GC.@preserve h check(circatt_memcpy(cvoid_ptr(x), pointer(h), Int64(sizeof(h)), Cint(0)),
                         "circatt_memcpy")
    return x
end
