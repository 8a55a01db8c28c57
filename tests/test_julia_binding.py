"""CPU checks of the Julia drop-in (circulantattention.jl_amd/julia): Julia is
not installed here or on the GPU box, so the module is not executed; these
tests pin what can be checked without it.

* every ccall in julia/src/libcircatt.jl names a function of
  include/circatt.h with the header's return type and argument types, in
  order (int -> Cint, int64_t -> Int64, int32_t -> Int32, float -> Cfloat,
  T* -> Ptr{T}, void** -> Ptr{Ptr{Cvoid}}, const char* -> Cstring), and every
  header function is bound exactly once;
* no other Julia file calls ccall (everything goes through those bindings),
  and none launches array kernels of its own or stages device data through
  the host: AMDGPU.ones/zeros, fill!, repeat, cat, copy(selectdim ...),
  copyto!, Array(...) and dotted broadcast operators do not appear outside
  comments and docstrings (the Circulant's fill, repeat, cat, batch sums,
  broadcasts and == are libcircatt entry points, devops.jl);
* the module exports every name the reference exports
  (src/CirculantAttention.jl:4,19,22-23,26) and defines the reference's
  method extensions and rules: NNlib.softmax(!), NNlib.batched_mul(!),
  CRC.rrule for circulant_similarity, _circulant_reshape, NNlib.softmax,
  circulant_attention, circulant_transposed_attention and scale
  (src/rrules.jl), Zygote.accum (src/zygote.jl), Adapt.adapt_structure
  (src/array.jl:22-25).
"""
import os
import re

from conftest import ROOT

JL = os.path.join(ROOT, "circulantattention.jl_amd", "julia")
HEADER = os.path.join(ROOT, "include", "circatt.h")

C_TO_JL = {"int": "Cint", "int64_t": "Int64", "int32_t": "Int32", "float": "Cfloat",
           "void": "Cvoid", "char": "UInt8"}


def c_type_to_julia(decl):
    """Julia spelling of a C parameter or return type ('const float *nzval')."""
    decl = re.sub(r"\bconst\b", "", decl).strip()
    stars = decl.count("*")
    base = decl.replace("*", " ").split()
    typ = base[0]
    if typ == "char" and stars == 1:
        return "Cstring"
    jl = C_TO_JL[typ]
    for _ in range(stars):
        jl = f"Ptr{{{jl}}}"
    return jl


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("#"))
    text = text.replace('extern "C" {', "").replace("}", "")
    out = {}
    for stmt in text.split(";"):
        m = re.match(r"\s*([A-Za-z_][\w\s\*]*?)\b(circatt_\w+)\s*\(([^)]*)\)\s*$", stmt, flags=re.S)
        if not m:
            continue
        ret, name, params = m.group(1).strip(), m.group(2), " ".join(m.group(3).split())
        args = [] if params in ("", "void") else [p.strip() for p in params.split(",")]
        # drop the parameter name (last identifier) unless only a type is given
        types = []
        for a in args:
            a = a.strip()
            mm = re.match(r"^(.*?[\s\*])(\w+)$", a)
            types.append(c_type_to_julia(mm.group(1) if mm else a))
        out[name] = (c_type_to_julia(ret), types)
    return out


def _balanced(s, i):
    """Index just past the parenthesised group starting at s[i] == '('."""
    depth = 0
    for j in range(i, len(s)):
        if s[j] == "(":
            depth += 1
        elif s[j] == ")":
            depth -= 1
            if depth == 0:
                return j + 1
    raise ValueError("unbalanced")


def julia_ccalls(path):
    """[(name, return type, [arg types])] of every ccall in a Julia file."""
    s = open(path).read()
    calls = []
    for m in re.finditer(r"ccall\(\(:(\w+),\s*libcircatt\),\s*", s):
        name = m.group(1)
        i = m.end()
        # return type up to the next top-level comma
        j = s.index(",", i)
        ret = s[i:j].strip()
        k = s.index("(", j)
        end = _balanced(s, k)
        inner = s[k + 1:end - 1]
        parts, depth, cur = [], 0, ""
        for ch in inner:
            if ch in "({":
                depth += 1
            elif ch in ")}":
                depth -= 1
            if ch == "," and depth == 0:
                parts.append(cur.strip())
                cur = ""
            else:
                cur += ch
        if cur.strip():
            parts.append(cur.strip())
        calls.append((name, ret, parts))
    return calls


def test_every_ccall_matches_the_header():
    hdr = header_functions()
    assert len(hdr) >= 25
    calls = julia_ccalls(os.path.join(JL, "src", "libcircatt.jl"))
    names = [c[0] for c in calls]
    assert sorted(names) == sorted(hdr), set(names) ^ set(hdr)
    for name, ret, args in calls:
        hret, hargs = hdr[name]
        assert ret == hret, (name, ret, hret)
        assert args == hargs, (name, args, hargs)


def test_header_parser_reads_known_signatures():
    hdr = header_functions()
    assert hdr["circatt_last_error"] == ("Cstring", [])
    assert hdr["circatt_malloc"] == ("Cint", ["Ptr{Ptr{Cvoid}}", "Int64"])
    assert hdr["circatt_pattern"][1][:5] == ["Cint", "Int64", "Int64", "Int32", "Int64"]
    assert hdr["circatt_similarity"][1][8] == "Cfloat"
    assert hdr["circatt_similarity"][1][11] == "Ptr{Cfloat}"


def test_only_the_bindings_call_ccall():
    src = os.path.join(JL, "src")
    for f in os.listdir(src):
        if f.endswith(".jl") and f != "libcircatt.jl":
            assert not re.search(r"\bccall\(", open(os.path.join(src, f)).read()), f


def jl_sources():
    src = os.path.join(JL, "src")
    return "\n".join(open(os.path.join(src, f)).read() for f in sorted(os.listdir(src))
                     if f.endswith(".jl"))


# src/CirculantAttention.jl:4, 19, 22-23, 26 of the reference
REFERENCE_EXPORTS = ["CircAtt", "Circulant", "circulant", "circulant_similarity",
                     "circulant_similarity!", "DotSimilarity", "DistanceSimilarity",
                     "circulant_adjacency", "circulant_adjacency!", "circulant_attention",
                     "circulant_mh_attention", "circulant_mh_adjacency", "⊗", "⨷"]


def test_module_exports_the_reference_names():
    text = open(os.path.join(JL, "src", "CirculantAttention.jl")).read()
    assert re.search(r"^module CirculantAttention$", text, flags=re.M)
    exported = set()
    for line in re.findall(r"^export (.*)$", text, flags=re.M):
        line = line.split("#")[0]
        exported.update(x.strip() for x in line.split(","))
    assert set(REFERENCE_EXPORTS) <= exported, set(REFERENCE_EXPORTS) - exported


def test_method_extensions_and_rules_are_defined():
    text = jl_sources()
    for pattern in [r"function NNlib\.softmax!\(", r"function NNlib\.softmax\(",
                    r"NNlib\.batched_mul\(A::Circulant", r"NNlib\.batched_mul!\(",
                    r"CRC\.rrule\(::typeof\(circulant_similarity\)",
                    r"CRC\.rrule\(::typeof\(_circulant_reshape\)",
                    r"CRC\.rrule\(::typeof\(NNlib\.softmax\)",
                    r"CRC\.rrule\(::typeof\(circulant_attention\), A::Circulant",
                    r"CRC\.rrule\(::typeof\(circulant_transposed_attention\)",
                    r"CRC\.rrule\(::typeof\(scale\)", r"function Zygote\.accum\(",
                    r"Adapt\.adapt_structure\(to, A::Circulant",
                    r"function LinearAlgebra\.dot\(f::Zygote\.FillArrays\.Fill",
                    r"Base\.:\(\+\)\(X::Circulant", r"Base\.:\(-\)\(X::Circulant",
                    r"Base\.:\(\*\)\(c::Number, X::Circulant", r"function Base\.sum\(A::Circulant",
                    r"function Base\.cat\(As::Circulant", r"function Base\.:\(==\)\(A::Circulant",
                    r"function Base\.show\(io::IO, m::MIME\"text/plain\", A::Circulant",
                    r"mutable struct CircCSR", r"struct Circulant\{T, N, M, S, A<:AbstractArray"]:
        assert re.search(pattern, text), pattern


def test_project_toml_names_the_package():
    text = open(os.path.join(JL, "Project.toml")).read()
    assert 'name = "CirculantAttention"' in text
    for dep in ("AMDGPU", "ChainRulesCore", "NNlib", "Zygote", "Adapt"):
        assert re.search(rf"^{dep} = \"[0-9a-f-]{{36}}\"$", text, flags=re.M), dep


def _code_only(text):
    """Julia source without docstrings, string literals and comments."""
    text = re.sub(r'(@doc\s+raw)?"""(.*?)"""', "", text, flags=re.S)
    text = re.sub(r'"(?:[^"\\\n]|\\.)*"', '""', text)
    return "\n".join(l.split("#")[0] for l in text.splitlines())


FORBIDDEN = [r"AMDGPU\.(ones|zeros|fill|rand|randn)\b", r"(?<![\w.])fill!\(",
             r"(?<![\w.])repeat\(", r"(?<![\w.])cat\(", r"copy\(\s*selectdim", r"copyto!\(",
             r"(?<![\w.])Array\(", r"\s\.(\*|\+|-|/|\^|=|÷)\s", r"\)\.(\*|\+|-|/)"]


def test_no_array_kernels_or_host_staging_outside_libcircatt():
    src = os.path.join(JL, "src")
    for f in sorted(os.listdir(src)):
        if not f.endswith(".jl"):
            continue
        code = _code_only(open(os.path.join(src, f)).read())
        for pat in FORBIDDEN:
            m = re.search(pat, code)
            assert m is None, (f, pat, code[max(0, m.start() - 60):m.end() + 20])


def test_forbidden_patterns_are_caught():
    """The guard's patterns match the calls it exists to keep out."""
    bad = ["nz = AMDGPU.ones(Float32, 4)", "fill!(similar(x), 1)", "r = repeat(x, 1, 2)",
           "c = cat(a, b; dims=2)", "copy(selectdim(x, 2, 1:1))", "copyto!(y, x)",
           "h = Array(x)", "y = c .* x", "z = (a).+ b"]
    for line in bad:
        assert any(re.search(p, _code_only(line)) for p in FORBIDDEN), line
    ok = ["function Base.repeat(A::CircCSR, counts::Int...)", "data = Base.repeat(A.data, 2)",
          "dfill!(x, 1f0)", "# c .* A in a comment", '"""Array(x) in a docstring"""',
          "splitheads.((q, k, v), nheads)", "function Base.cat(As::Circulant...; dims=3)",
          'throw(ArgumentError("repeat(A, 1, 1, counts...)"))']
    for line in ok:
        assert not any(re.search(p, _code_only(line)) for p in FORBIDDEN), line
