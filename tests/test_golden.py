"""Golden vector from the reference itself: the README's picture of the
128x96, ws = 15 Circulant (README.md:72-112), i.e. the sparsity pattern of
the README-quickstart configuration (cfg2) as the reference printed it.

The oracle's pattern (and, in the GPU test, libcircatt's pattern) rendered by
Julia's braille spy algorithm (tests/golden/spy.py) must reproduce the
picture character for character.  Planted mistakes (transposed spatial dims,
another window, an off-by-one column shift, a pattern without the circular
wrap) must not.
"""
import os

import numpy as np
import pytest

import oracle as O
from golden import spy

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "readme_spy_128x96_ws15.txt")
DIMS, WS = (128, 96), 15
P = 128 * 96


@pytest.fixture(scope="module")
def picture():
    pic = spy.load(FIXTURE)
    assert len(pic) == 19 and all(len(line) == 40 for line in pic)
    return pic


def test_oracle_pattern_reproduces_readme_picture(picture):
    rp, cv = O.pattern(DIMS, WS, 2)
    for b in range(2):  # both batches print the same picture (README.md:72-112)
        assert spy.render_csr(rp[b], cv[b], P) == picture


def test_canvas_75_does_not_match(picture):
    """The only free parameter of the rendering is pinned by the picture."""
    rp, cv = O.pattern(DIMS, WS, 1)
    assert spy.render_csr(rp[0], cv[0], P, scale=75) != picture


@pytest.mark.parametrize("mistake", ["transposed", "ws13", "shift", "nowrap"])
def test_planted_pattern_mistakes_fail(picture, mistake):
    if mistake == "transposed":
        rp, cv = O.pattern((96, 128), WS, 1)
        rp, cv = rp[0], cv[0]
    elif mistake == "ws13":
        rp, cv = O.pattern(DIMS, 13, 1)
        rp, cv = rp[0], cv[0]
    else:
        rp, cv = O.pattern(DIMS, WS, 1)
        rp, cv = rp[0], cv[0].astype(np.int64)
        if mistake == "shift":
            cv = (cv % P) + 1  # every column one pixel further (wrapping)
        else:
            # keep only the entries whose window does not wrap around the
            # image border (what a non-circular band would store)
            r = np.repeat(np.arange(P), WS * WS)
            c = cv - 1
            dh = np.abs(c % 128 - r % 128)
            dw = np.abs(c // 128 - r // 128)
            keep = (dh <= 7) & (dw <= 7)
            cv = cv[keep]
            rp = np.concatenate([[1], 1 + np.cumsum(np.bincount(r[keep], minlength=P))])
    assert spy.render_csr(rp, cv, P) != picture


@pytest.mark.gpu
def test_hip_pattern_reproduces_readme_picture(picture):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from circulant_attention import _lib as L
    from circulant_attention._functions import ptr, stream_ptr
    dev = torch.device("cuda:0")
    nb, K = 2, WS * WS
    rowptr = torch.empty((nb, P + 1), dtype=torch.int32, device=dev)
    colval = torch.empty((nb, P * K), dtype=torch.int32, device=dev)
    L.check(L.lib.circatt_pattern(2, 128, 96, WS, nb, ptr(rowptr), ptr(colval), stream_ptr()))
    rp, cv = rowptr.cpu().numpy(), colval.cpu().numpy()
    for b in range(nb):
        assert spy.render_csr(rp[b], cv[b], P) == picture
