# Raw bindings of include/circatt.h: one Julia function per C entry point,
# same name, same argument order, each a single ccall whose argument types
# are the header's (int -> Cint, int64_t -> Int64, int32_t -> Int32,
# float -> Cfloat, pointers -> Ptr).  tests/test_julia_binding.py checks
# every ccall here against the header.  Higher layers pass device pointers
# from dptr and the current HIP stream from stream_ptr.

const libcircatt = get(ENV, "CIRCATT_LIB", normpath(joinpath(@__DIR__, "..", "..", "libcircatt.so")))

const CIRCATT_OK = Cint(0)
const CIRCATT_ERR_INVALID = Cint(-1)
const CIRCATT_ERR_UNSUPPORTED = Cint(-2)
const CIRCATT_ERR_HIP = Cint(-3)

const CIRCATT_DOT = Cint(0)
const CIRCATT_DISTANCE = Cint(1)
const CIRCATT_F32 = Cint(0)
const CIRCATT_C32 = Cint(1)
# OR-ed into dtype of the fused entry points: (C, spatial..., B) tensors
const CIRCATT_CHANNELS_LAST = Cint(16)
const CIRCATT_MATH_SPLIT_F16 = Cint(0)
const CIRCATT_MATH_F32 = Cint(1)

circatt_version() = ccall((:circatt_version, libcircatt), Cint, ())

circatt_set_math(mode) = ccall((:circatt_set_math, libcircatt), Cint, (Cint,), mode)

circatt_get_math() = ccall((:circatt_get_math, libcircatt), Cint, ())

circatt_last_error() = ccall((:circatt_last_error, libcircatt), Cstring, ())

circatt_pattern(nsp, n1, n2, ws, nb, rowptr, colval, stream) =
    ccall((:circatt_pattern, libcircatt), Cint,
          (Cint, Int64, Int64, Int32, Int64, Ptr{Int32}, Ptr{Int32}, Ptr{Cvoid}),
          nsp, n1, n2, ws, nb, rowptr, colval, stream)

circatt_similarity(kind, dtype, nsp, n1, n2, ws, C, nb, scale, x, y, nzval, stream) =
    ccall((:circatt_similarity, libcircatt), Cint,
          (Cint, Cint, Cint, Int64, Int64, Int32, Int64, Int64, Cfloat, Ptr{Cvoid}, Ptr{Cvoid},
           Ptr{Cfloat}, Ptr{Cvoid}),
          kind, dtype, nsp, n1, n2, ws, C, nb, scale, x, y, nzval, stream)

circatt_softmax(K, rows, in, out, stream) =
    ccall((:circatt_softmax, libcircatt), Cint,
          (Int64, Int64, Ptr{Cfloat}, Ptr{Cfloat}, Ptr{Cvoid}),
          K, rows, in, out, stream)

circatt_softmax_bwd(K, rows, A, dA, dS, stream) =
    ccall((:circatt_softmax_bwd, libcircatt), Cint,
          (Int64, Int64, Ptr{Cfloat}, Ptr{Cfloat}, Ptr{Cfloat}, Ptr{Cvoid}),
          K, rows, A, dA, dS, stream)

circatt_apply(trans, dtype, nsp, n1, n2, ws, C, nb, nzval, x, y, stream) =
    ccall((:circatt_apply, libcircatt), Cint,
          (Cint, Cint, Cint, Int64, Int64, Int32, Int64, Int64, Ptr{Cfloat}, Ptr{Cvoid},
           Ptr{Cvoid}, Ptr{Cvoid}),
          trans, dtype, nsp, n1, n2, ws, C, nb, nzval, x, y, stream)

circatt_similarity_bwd(kind, dtype, nsp, n1, n2, ws, C, nb, scale, dS, x, y, dx, dy, stream) =
    ccall((:circatt_similarity_bwd, libcircatt), Cint,
          (Cint, Cint, Cint, Int64, Int64, Int32, Int64, Int64, Cfloat, Ptr{Cfloat}, Ptr{Cvoid},
           Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}),
          kind, dtype, nsp, n1, n2, ws, C, nb, scale, dS, x, y, dx, dy, stream)

circatt_rowsum(nsp, n1, n2, ws, nb, nzval, out, stream) =
    ccall((:circatt_rowsum, libcircatt), Cint,
          (Cint, Int64, Int64, Int32, Int64, Ptr{Cfloat}, Ptr{Cfloat}, Ptr{Cvoid}),
          nsp, n1, n2, ws, nb, nzval, out, stream)

circatt_colsum(nsp, n1, n2, ws, nb, nzval, out, stream) =
    ccall((:circatt_colsum, libcircatt), Cint,
          (Cint, Int64, Int64, Int32, Int64, Ptr{Cfloat}, Ptr{Cfloat}, Ptr{Cvoid}),
          nsp, n1, n2, ws, nb, nzval, out, stream)

circatt_axpby(nnz, nb, alpha, alpha0, X, beta, beta0, Y, Z, stream) =
    ccall((:circatt_axpby, libcircatt), Cint,
          (Int64, Int64, Ptr{Cfloat}, Cfloat, Ptr{Cfloat}, Ptr{Cfloat}, Cfloat, Ptr{Cfloat},
           Ptr{Cfloat}, Ptr{Cvoid}),
          nnz, nb, alpha, alpha0, X, beta, beta0, Y, Z, stream)

circatt_batch_dot_workspace_bytes(nnz, nb) =
    ccall((:circatt_batch_dot_workspace_bytes, libcircatt), Int64, (Int64, Int64), nnz, nb)

circatt_batch_dot(nnz, nb, X, Y, out, workspace, workspace_bytes, stream) =
    ccall((:circatt_batch_dot, libcircatt), Cint,
          (Int64, Int64, Ptr{Cfloat}, Ptr{Cfloat}, Ptr{Cfloat}, Ptr{Cvoid}, Int64, Ptr{Cvoid}),
          nnz, nb, X, Y, out, workspace, workspace_bytes, stream)

circatt_fused_fwd(kind, dtype, nsp, n1, n2, ws, C, nheads, B, q, k, v, y, lse, stream) =
    ccall((:circatt_fused_fwd, libcircatt), Cint,
          (Cint, Cint, Cint, Int64, Int64, Int32, Int64, Int64, Int64, Ptr{Cvoid}, Ptr{Cvoid},
           Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cfloat}, Ptr{Cvoid}),
          kind, dtype, nsp, n1, n2, ws, C, nheads, B, q, k, v, y, lse, stream)

circatt_fused_bwd_workspace_bytes(nsp, n1, n2, nheads, B) =
    ccall((:circatt_fused_bwd_workspace_bytes, libcircatt), Int64,
          (Cint, Int64, Int64, Int64, Int64), nsp, n1, n2, nheads, B)

circatt_fused_bwd(kind, dtype, nsp, n1, n2, ws, C, nheads, B, q, k, v, y, dy, lse, dq, dk, dv,
                  workspace, workspace_bytes, stream) =
    ccall((:circatt_fused_bwd, libcircatt), Cint,
          (Cint, Cint, Cint, Int64, Int64, Int32, Int64, Int64, Int64, Ptr{Cvoid}, Ptr{Cvoid},
           Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cfloat}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
           Ptr{Cvoid}, Int64, Ptr{Cvoid}),
          kind, dtype, nsp, n1, n2, ws, C, nheads, B, q, k, v, y, dy, lse, dq, dk, dv,
          workspace, workspace_bytes, stream)

circatt_fused_bwd_dq(kind, dtype, nsp, n1, n2, ws, C, nheads, B, q, k, v, y, dy, lse, dq,
                     workspace, workspace_bytes, stream) =
    ccall((:circatt_fused_bwd_dq, libcircatt), Cint,
          (Cint, Cint, Cint, Int64, Int64, Int32, Int64, Int64, Int64, Ptr{Cvoid}, Ptr{Cvoid},
           Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cfloat}, Ptr{Cvoid}, Ptr{Cvoid}, Int64,
           Ptr{Cvoid}),
          kind, dtype, nsp, n1, n2, ws, C, nheads, B, q, k, v, y, dy, lse, dq, workspace,
          workspace_bytes, stream)

circatt_fused_bwd_dkdv(kind, dtype, nsp, n1, n2, ws, C, nheads, B, q, k, v, dy, lse, dk, dv,
                       workspace, workspace_bytes, stream) =
    ccall((:circatt_fused_bwd_dkdv, libcircatt), Cint,
          (Cint, Cint, Cint, Int64, Int64, Int32, Int64, Int64, Int64, Ptr{Cvoid}, Ptr{Cvoid},
           Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cfloat}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Int64,
           Ptr{Cvoid}),
          kind, dtype, nsp, n1, n2, ws, C, nheads, B, q, k, v, dy, lse, dk, dv, workspace,
          workspace_bytes, stream)

circatt_fused_bwd_noalloc_max_rows() =
    ccall((:circatt_fused_bwd_noalloc_max_rows, libcircatt), Int64, ())

circatt_fused_bwd_noalloc(kind, dtype, nsp, n1, n2, ws, C, nheads, B, q, k, v, y, dy, lse, dq,
                          dk, dv, stream) =
    ccall((:circatt_fused_bwd_noalloc, libcircatt), Cint,
          (Cint, Cint, Cint, Int64, Int64, Int32, Int64, Int64, Int64, Ptr{Cvoid}, Ptr{Cvoid},
           Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cfloat}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid},
           Ptr{Cvoid}),
          kind, dtype, nsp, n1, n2, ws, C, nheads, B, q, k, v, y, dy, lse, dq, dk, dv, stream)

circatt_fill(dst, n, value, stream) =
    ccall((:circatt_fill, libcircatt), Cint, (Ptr{Cfloat}, Int64, Cfloat, Ptr{Cvoid}),
          dst, n, value, stream)

circatt_copy_blocks(dst, src, block_bytes, ninner, dst_stride_inner, src_stride_inner, nouter,
                    dst_stride_outer, src_stride_outer, stream) =
    ccall((:circatt_copy_blocks, libcircatt), Cint,
          (Ptr{Cvoid}, Ptr{Cvoid}, Int64, Int64, Int64, Int64, Int64, Int64, Int64, Ptr{Cvoid}),
          dst, src, block_bytes, ninner, dst_stride_inner, src_stride_inner, nouter,
          dst_stride_outer, src_stride_outer, stream)

circatt_sum_middle(src, dst, inner, nsum, outer, stream) =
    ccall((:circatt_sum_middle, libcircatt), Cint,
          (Ptr{Cfloat}, Ptr{Cfloat}, Int64, Int64, Int64, Ptr{Cvoid}),
          src, dst, inner, nsum, outer, stream)

circatt_count_unequal(kind, n, a, b, count, stream) =
    ccall((:circatt_count_unequal, libcircatt), Cint,
          (Cint, Int64, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Int64}, Ptr{Cvoid}),
          kind, n, a, b, count, stream)

circatt_malloc(ptr, bytes) =
    ccall((:circatt_malloc, libcircatt), Cint, (Ptr{Ptr{Cvoid}}, Int64), ptr, bytes)

circatt_free(ptr) = ccall((:circatt_free, libcircatt), Cint, (Ptr{Cvoid},), ptr)

circatt_memcpy(dst, src, bytes, kind) =
    ccall((:circatt_memcpy, libcircatt), Cint, (Ptr{Cvoid}, Ptr{Cvoid}, Int64, Cint),
          dst, src, bytes, kind)

circatt_stream_synchronize(stream) =
    ccall((:circatt_stream_synchronize, libcircatt), Cint, (Ptr{Cvoid},), stream)

# ---- helpers ---------------------------------------------------------------

"""Throw the reference's exception for a libcircatt status: its @assert
messages come back as AssertionError, everything else as ErrorException."""
function check(rc::Integer, what::AbstractString="libcircatt")
    rc == CIRCATT_OK && return nothing
    msg = unsafe_string(circatt_last_error())
    isempty(msg) && (msg = what)
    rc == CIRCATT_ERR_INVALID && throw(AssertionError(msg))
    rc == CIRCATT_ERR_UNSUPPORTED && throw(ErrorException("not supported by libcircatt: " * msg))
    throw(ErrorException(msg))
end

"""Device address of a contiguous ROCArray (C_NULL for nothing)."""
dptr(x::ROCArray{T}) where {T} = pointer(x)
dptr(::Nothing) = C_NULL
dptr(x::AbstractArray) = throw(ArgumentError(
    "libcircatt takes contiguous ROCArrays (device memory); got $(typeof(x))"))

"""The calling task's HIP stream (AMDGPU.jl's), as a hipStream_t."""
stream_ptr() = reinterpret(Ptr{Cvoid}, AMDGPU.stream().stream)

cfloat_ptr(x) = reinterpret(Ptr{Cfloat}, dptr(x))
cvoid_ptr(x) = reinterpret(Ptr{Cvoid}, dptr(x))

dtype_code(::Type{Float32}) = CIRCATT_F32
dtype_code(::Type{ComplexF32}) = CIRCATT_C32
dtype_code(::Type{T}) where {T} =
    throw(ArgumentError("libcircatt signals are Float32 or ComplexF32, got $T"))

"""(nsp, n1, n2) of a spatial size (N1,) or (N1, N2)."""
geom(s::NTuple{1,Int}) = (Cint(1), Int64(s[1]), Int64(1))
geom(s::NTuple{2,Int}) = (Cint(2), Int64(s[1]), Int64(s[2]))
geom(s::Tuple) = throw(ArgumentError("libcircatt supports 1 or 2 spatial dims, got $(length(s))"))

"""Select the arithmetic of the fused kernels (CIRCATT_MATH_SPLIT_F16 or
CIRCATT_MATH_F32); process-wide."""
set_math!(mode::Integer) = check(circatt_set_math(Cint(mode)), "circatt_set_math")
