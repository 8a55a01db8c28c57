# Gradient accumulation of Circulant cotangents (reference: src/zygote.jl:1-7):
# the sum of two cotangents on one pattern is circatt_axpby.

function Zygote.accum(x::T, y::T) where T <: Circulant
    x === nothing ? y :
    y === nothing ? x :
    x + y
end

Zygote.accum(x::T, y::T, z::T...) where T <: Circulant = Zygote.accum(Zygote.accum(x, y), z...)
