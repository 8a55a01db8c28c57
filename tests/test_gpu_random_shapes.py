"""Fused attention on seeded random shapes against the float64 oracle.

Image sizes 2..37 along each dimension (partial tiles, halos that wrap more
than once, windows wider than the image), every window of the split-half
kernels, 16 and 32 real components per head, real and complex, Dot and
Distance, one or two heads and batches; the same bar as the fixed cases of
test_gpu_parity.py (1e-5 forward, 1e-4 gradients)."""
import random

import pytest

from test_gpu_parity import _attention_case  # noqa: F401  (fixtures ca, cuda come from there)
from test_gpu_parity import ca  # noqa: F401

pytestmark = pytest.mark.gpu


def cases(n=48, seed=20261202):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        ws = rng.choice([3, 5, 7, 11, 15])
        cplx = rng.random() < 0.4
        per = rng.choice([16, 32]) if not cplx else rng.choice([8, 16])
        nh = rng.choice([1, 2])
        out.append(((rng.randint(2, 37), rng.randint(2, 37)), ws, per * nh, rng.choice([1, 2]), nh,
                    rng.choice([0, 1]), cplx, 9000 + i))
    return out


@pytest.mark.parametrize("case", cases(), ids=lambda c: f"{c[0][0]}x{c[0][1]}-ws{c[1]}-C{c[2]}-B{c[3]}-h{c[4]}-"
                                                       f"{'dist' if c[5] else 'dot'}-{'c32' if c[6] else 'f32'}")
def test_fused_random_shape(ca, cuda, case):  # noqa: F811
    dims, ws, C, B, nh, kind, cplx, seed = case
    print(f"random shape: dims={dims} ws={ws} C={C} B={B} nh={nh} kind={kind} cplx={cplx}", flush=True)
    _attention_case(ca, cuda, dims, ws, C, B, nh, seed, cplx, kind, materialize=False)


def cases_1d(n=32, seed=20261203):
    """One-dimensional signals: lengths 2..700 (single partial tiles, several
    tiles, lengths that are and are not multiples of 4, which select the
    row-DMA or the per-pixel loads), the split-half windows 15 and 63 and, for
    the routing, 7 and 31."""
    rng = random.Random(seed)
    out = []
    for i in range(n):
        ws = rng.choice([15, 15, 63, 63, 7, 31])
        cplx = rng.random() < 0.3
        per = rng.choice([16, 32]) if not cplx else rng.choice([8, 16])
        nh = rng.choice([1, 2])
        n1 = rng.choice([rng.randint(2, 40), rng.randint(41, 300), rng.randint(301, 700)])
        out.append(((n1,), ws, per * nh, rng.choice([1, 2]), nh, rng.choice([0, 1]), cplx, 9500 + i))
    return out


@pytest.mark.parametrize("case", cases_1d(), ids=lambda c: f"{c[0][0]}-ws{c[1]}-C{c[2]}-B{c[3]}-h{c[4]}-"
                                                          f"{'dist' if c[5] else 'dot'}-{'c32' if c[6] else 'f32'}")
def test_fused_random_shape_1d(ca, cuda, case):  # noqa: F811
    dims, ws, C, B, nh, kind, cplx, seed = case
    print(f"random 1D shape: dims={dims} ws={ws} C={C} B={B} nh={nh} kind={kind} cplx={cplx}", flush=True)
    _attention_case(ca, cuda, dims, ws, C, B, nh, seed, cplx, kind, materialize=False)
