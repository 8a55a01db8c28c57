"""The Circulant batch utilities: cat (src/array.jl:62-64, README.md:145-148),
repeat (src/array.jl:49-52) and == (src/array.jl:101-115).  They move nzVal
between batch slots only, so the expected values are written out slot by
slot.  The argument checks run on the host before any launch (CPU tests);
the data movement is libcircatt's (circatt_copy_blocks,
circatt_count_unequal), so those tests are marked gpu."""
import pytest

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ca():
    import circulant_attention
    return circulant_attention


def circ(ca, nh, B, base, dims=(4, 3), ws=3, device="cpu"):
    P, K = dims[0] * dims[1], ws ** len(dims)
    nz = torch.arange(B * nh * P * K, dtype=torch.float32).reshape(B, nh, P, K) + base
    return ca.Circulant(nz.to(device), ws, dims)


@pytest.fixture
def gcirc(ca, cuda):
    return lambda *a, **k: circ(ca, *a, device=cuda, **k)


@pytest.mark.gpu
def test_cat_dims3_stacks_heads(ca, gcirc):
    A, Bm = gcirc(2, 3, 0.0), gcirc(1, 3, 1000.0)
    D = ca.cat(A, Bm, dims=3)
    assert D.size() == (12, 12, 3, 3)
    for b in range(3):
        assert torch.equal(D.nzval[b, 0], A.nzval[b, 0])
        assert torch.equal(D.nzval[b, 1], A.nzval[b, 1])
        assert torch.equal(D.nzval[b, 2], Bm.nzval[b, 0])


@pytest.mark.gpu
def test_cat_dims4_stacks_batches(ca, gcirc):
    A, Bm = gcirc(2, 1, 0.0), gcirc(2, 2, 500.0)
    D = ca.cat(A, Bm, dims=4)
    assert D.size() == (12, 12, 2, 3)
    assert torch.equal(D.nzval[0], A.nzval[0])
    assert torch.equal(D.nzval[1], Bm.nzval[0])
    assert torch.equal(D.nzval[2], Bm.nzval[1])


@pytest.mark.gpu
def test_cat_dims5_adds_a_batch_dim(ca, gcirc):
    A, Bm = gcirc(2, 2, 0.0), gcirc(2, 2, 7.0)
    D = ca.cat(A, Bm, dims=5)
    assert D.size() == (12, 12, 2, 2, 2)
    assert torch.equal(D.nzval[0], A.nzval) and torch.equal(D.nzval[1], Bm.nzval)


def test_cat_rejects_mismatches(ca):
    A = circ(ca, 2, 2, 0.0)
    with pytest.raises(AssertionError, match="batch dims"):
        ca.cat(A, circ(ca, 2, 3, 0.0), dims=3)
    with pytest.raises(AssertionError, match="kernel length"):
        ca.cat(A, circ(ca, 2, 2, 0.0, dims=(4, 3), ws=1), dims=3)
    with pytest.raises(AssertionError, match="batch dims"):
        ca.cat(A, A, dims=2)


@pytest.mark.gpu
def test_repeat_tiles_batch_dims(ca, gcirc):
    A = gcirc(2, 1, 0.0)
    R = A.repeat(1, 1, 2, 3)
    assert R.size() == (12, 12, 4, 3)
    for b in range(3):
        for h in range(4):
            assert torch.equal(R.nzval[b, h], A.nzval[0, h % 2])


def test_repeat_rejects_pixel_dims(ca):
    with pytest.raises(AssertionError, match="cannot be repeated"):
        circ(ca, 2, 1, 0.0).repeat(2, 1, 1, 1)


@pytest.mark.gpu
def test_equality(ca, gcirc):
    A = gcirc(2, 2, 0.0)
    assert A == A.copy()
    assert not (A == gcirc(2, 2, 1.0))
    assert not (A == A.reshape(12, 12, 4, 1))
    assert not (A == gcirc(2, 2, 0.0, dims=(3, 4)))
    assert ca.cat(A, A, dims=3) == A.repeat(1, 1, 2, 1)


def test_accessors(ca):
    """kernel_length / spatial_dims / spatial_size (src/array.jl:31-33) and
    size (P, P, batch...) of a 2D and a 1D Circulant."""
    A = circ(ca, 2, 3, 0.0, dims=(4, 3), ws=3)
    assert (ca.kernel_length(A), ca.spatial_dims(A), ca.spatial_size(A)) == (3, 2, (4, 3))
    assert A.size() == (12, 12, 2, 3)
    L = ca.Circulant(torch.zeros(2, 1, 10, 5), 5, (10,))
    assert (ca.kernel_length(L), ca.spatial_dims(L), ca.spatial_size(L)) == (5, 1, (10,))
    assert L.size() == (10, 10, 1, 2)


def test_bench_refuses_several_gpus():
    """bench.py runs on one GPU: --gpus N > 1 exits with status 2 and a JSON
    error line before touching a device."""
    import json
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in json.loads(r.stdout.strip().splitlines()[-1])["error"]


def test_product_path_uses_no_torch_kernels_on_circulant_data():
    """The Circulant's values are filled, copied, repeated, concatenated,
    summed over batch dims, broadcast and compared by libcircatt entry points
    (circatt_fill, circatt_copy_blocks, circatt_sum_middle,
    circatt_count_unequal), not by torch kernels: none of these torch calls
    appears in the package's Circulant and Function modules."""
    import os
    import re
    pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                       "circulantattention.jl_amd", "circulant_attention")
    forbidden = [r"torch\.(gather|cat|ones|zeros|full|equal|stack|where)\(", r"\.clone\(",
                 r"\.repeat\(", r"\.expand\([^)]*\)\.(contiguous|reshape|clone)", r"\.index_select\(",
                 r"\.scatter", r"\.copy_\(", r"\.fill_\("]
    for name in ("circulant.py", "_functions.py"):
        code = "\n".join(l.split("#")[0] for l in open(os.path.join(pkg, name)).read().splitlines())
        code = re.sub(r'"""(.*?)"""', "", code, flags=re.S)
        for pat in forbidden:
            m = re.search(pat, code)
            assert m is None, (name, pat, code[max(0, m.start() - 80):m.end() + 20])
