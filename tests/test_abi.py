"""CPU tests of the C ABI: the library loads, exports every symbol that
include/circatt.h declares, and validates arguments on the host (the
reference's @assert checks) before any HIP call.  No kernel runs here."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "circatt.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(circatt_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    from circulant_attention import _lib
    return _lib


def test_exports_every_declared_symbol(L):
    syms = declared_symbols()
    assert len(syms) >= 18
    for s in syms:
        assert hasattr(L.lib, s), f"{s} declared in circatt.h but not exported"
    assert set(syms) == set(L.SIGNATURES), "ctypes signatures must cover the header exactly"


def test_version(L):
    assert L.lib.circatt_version() >= 10000


NULL = None
FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first


def expect(L, rc, code, fragment):
    assert rc == code, (rc, L.lib.circatt_last_error())
    assert fragment in L.lib.circatt_last_error().decode()


def test_even_window_rejected(L):
    rc = L.lib.circatt_pattern(2, 8, 8, 4, 1, FAKE, FAKE, NULL)
    expect(L, rc, L.ERR_INVALID, "must be odd")


def test_bad_spatial_dims(L):
    rc = L.lib.circatt_pattern(3, 8, 8, 3, 1, FAKE, FAKE, NULL)
    expect(L, rc, L.ERR_INVALID, "nsp")
    rc = L.lib.circatt_pattern(2, 0, 8, 3, 1, FAKE, FAKE, NULL)
    expect(L, rc, L.ERR_INVALID, "spatial size")


def test_null_pointers(L):
    rc = L.lib.circatt_pattern(1, 8, 1, 3, 1, NULL, FAKE, NULL)
    expect(L, rc, L.ERR_INVALID, "rowptr is NULL")
    rc = L.lib.circatt_similarity(0, 0, 2, 8, 8, 3, 4, 1, 1.0, FAKE, NULL, FAKE, NULL)
    expect(L, rc, L.ERR_INVALID, "y is NULL")


def test_int32_index_overflow(L):
    # P*K must fit Int32 colVal (src/circulant.jl:64,86)
    rc = L.lib.circatt_pattern(2, 20000, 20000, 15, 1, FAKE, FAKE, NULL)
    expect(L, rc, L.ERR_INVALID, "Int32")


def test_unsupported_dtype_and_kind(L):
    rc = L.lib.circatt_similarity(0, 7, 2, 8, 8, 3, 4, 1, 1.0, FAKE, FAKE, FAKE, NULL)
    expect(L, rc, L.ERR_UNSUPPORTED, "dtype")
    rc = L.lib.circatt_similarity(5, 0, 2, 8, 8, 3, 4, 1, 1.0, FAKE, FAKE, FAKE, NULL)
    expect(L, rc, L.ERR_INVALID, "kind")


def test_channels_last_flag_only_on_fused_entry_points(L):
    # the unfused entry points take planar signals only
    rc = L.lib.circatt_similarity(0, L.F32 | L.CHANNELS_LAST, 2, 8, 8, 3, 4, 1, 1.0, FAKE, FAKE,
                                  FAKE, NULL)
    expect(L, rc, L.ERR_UNSUPPORTED, "dtype")
    rc = L.lib.circatt_apply(0, L.C32 | L.CHANNELS_LAST, 2, 8, 8, 3, 2, 1, FAKE, FAKE,
                             ctypes.c_void_p(0x2000), NULL)
    expect(L, rc, L.ERR_UNSUPPORTED, "dtype")
    # the fused ones validate the rest as before
    rc = L.lib.circatt_fused_fwd(0, L.F32 | L.CHANNELS_LAST, 2, 8, 8, 3, 6, 4, 1, FAKE, FAKE,
                                 FAKE, FAKE, FAKE, NULL)
    expect(L, rc, L.ERR_INVALID, "divisible by nheads")
    rc = L.lib.circatt_fused_fwd(0, 7 | L.CHANNELS_LAST, 2, 8, 8, 3, 4, 1, 1, FAKE, FAKE, FAKE,
                                 FAKE, FAKE, NULL)
    expect(L, rc, L.ERR_UNSUPPORTED, "dtype")


def test_heads_must_divide_channels(L):
    rc = L.lib.circatt_fused_fwd(0, 0, 2, 8, 8, 3, 6, 4, 1, FAKE, FAKE, FAKE, FAKE, FAKE, NULL)
    expect(L, rc, L.ERR_INVALID, "divisible by nheads")


def test_fused_bwd_workspace(L):
    assert L.lib.circatt_fused_bwd_workspace_bytes(2, 256, 256, 4, 4) == 256 * 256 * 16 * 4
    assert L.lib.circatt_fused_bwd_workspace_bytes(1, 100, 1, 1, 2) == 800
    assert L.lib.circatt_fused_bwd_workspace_bytes(3, 1, 1, 1, 1) == -1
    rc = L.lib.circatt_fused_bwd(0, 0, 2, 8, 8, 3, 4, 1, 1, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                                 ctypes.c_void_p(0x2000), ctypes.c_void_p(0x3000),
                                 ctypes.c_void_p(0x4000), FAKE, 16, NULL)
    expect(L, rc, L.ERR_INVALID, "workspace")


def test_aliasing_rejected(L):
    rc = L.lib.circatt_apply(0, 0, 1, 8, 1, 3, 2, 1, FAKE, FAKE, FAKE, NULL)
    expect(L, rc, L.ERR_INVALID, "alias")


def test_python_layer_refuses_cpu_tensors():
    torch = pytest.importorskip("torch")
    import circulant_attention as ca
    x = torch.randn(1, 4, 8, 8)
    with pytest.raises(ValueError, match="HIP device"):
        ca.circulant_similarity(ca.DotSimilarity(), x, x, 3)
    with pytest.raises(AssertionError, match="must be odd"):
        ca.Circulant.new(4, (8, 8, 1, 1), device="cpu")


def test_math_mode_switch(L):
    """circatt_set_math accepts the two documented modes, keeps the last one,
    and rejects anything else without changing the mode."""
    old = L.lib.circatt_get_math()
    try:
        assert L.lib.circatt_set_math(L.MATH_F32) == L.OK
        assert L.lib.circatt_get_math() == L.MATH_F32
        expect(L, L.lib.circatt_set_math(7), L.ERR_INVALID, "math")
        assert L.lib.circatt_get_math() == L.MATH_F32
        assert L.lib.circatt_set_math(L.MATH_SPLIT_F16) == L.OK
        assert L.lib.circatt_get_math() == L.MATH_SPLIT_F16
        expect(L, L.lib.circatt_set_math(-1), L.ERR_INVALID, "math")
    finally:
        L.lib.circatt_set_math(old)


def test_batch_dot_validation(L):
    assert L.lib.circatt_batch_dot_workspace_bytes(1000, 3) == 3 * 8
    assert L.lib.circatt_batch_dot_workspace_bytes(65536 * 1024 * 4, 2) == 2 * 1024 * 8
    assert L.lib.circatt_batch_dot_workspace_bytes(-1, 1) == -1
    rc = L.lib.circatt_batch_dot(100, 2, FAKE, NULL, ctypes.c_void_p(0x2000),
                                 ctypes.c_void_p(0x3000), 8, NULL)
    expect(L, rc, L.ERR_INVALID, "workspace")
    rc = L.lib.circatt_batch_dot(100, 2, NULL, NULL, FAKE, FAKE, 64, NULL)
    expect(L, rc, L.ERR_INVALID, "X is NULL")
