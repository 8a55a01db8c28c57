"""Braille sparsity picture of a CSR pattern, as Julia prints a large sparse
matrix (test infrastructure).

This restates the published algorithm of `_show_with_braille_chars` in Julia's
SparseArrays standard library (the reference's README output at
README.md:72-112 comes from it via CUDA.jl's display of a CuSparseArrayCSR;
SparseArrays ships with Julia and is not pinned by the reference, which has no
Manifest).  The matrix (m x n) is scaled onto a canvas of scale_h x scale_w
dots; entry (i, j) (1-based) lands on dot
    si = round((i - 1) * (scale_h - 1) / (m - 1) + 1)
    sj = round((j - 1) * (scale_w - 1) / (n - 1) + 1)
(round half to even), dots are grouped 2 wide x 4 high into braille cells,
and the grid is framed by the bracket characters.  The canvas size is the one
free parameter (it follows the terminal size); the README picture has 19
lines of 38 cells, which allows 73..76 dots high and 75..76 wide, and the
square matrix needs equal sides, so 75 or 76.
"""
import numpy as np

_BLANK = 0x2800
# dot bits for (column in cell, row in cell): left column rows 0..3, then right
_DOTS = [0x01, 0x02, 0x04, 0x40, 0x08, 0x10, 0x20, 0x80]


def render(rows, cols, m, n, scale_h, scale_w):
    """rows, cols: 1-based coordinates of the stored entries."""
    rows = np.asarray(rows, np.int64)
    cols = np.asarray(cols, np.int64)
    ncell_w = (scale_w - 1) // 2 + 1
    ncell_h = (scale_h - 1) // 4 + 1
    grid = np.zeros((ncell_h, ncell_w), np.int64)
    rowscale = max(1, scale_h - 1) / max(1, m - 1)
    colscale = max(1, scale_w - 1) / max(1, n - 1)
    si = np.rint((rows - 1) * rowscale + 1).astype(np.int64)
    sj = np.rint((cols - 1) * colscale + 1).astype(np.int64)
    bits = np.asarray(_DOTS)[((sj - 1) % 2) * 4 + (si - 1) % 4]
    np.bitwise_or.at(grid, ((si - 1) // 4, (sj - 1) // 2), bits)
    out = []
    for li in range(ncell_h):
        left = "⎡" if li == 0 else ("⎣" if li == ncell_h - 1 else "⎢")
        right = "⎤" if li == 0 else ("⎦" if li == ncell_h - 1 else "⎥")
        out.append(left + "".join(chr(_BLANK + int(b)) for b in grid[li]) + right)
    return out


def render_csr(rowptr, colval, P, scale=76):
    """Picture of one batch of a Circulant: row = CSR row, column = colVal."""
    rowptr = np.asarray(rowptr, np.int64)
    counts = np.diff(rowptr)
    rows = np.repeat(np.arange(1, P + 1), counts)
    return render(rows, np.asarray(colval, np.int64), P, P, scale, scale)


def load(path):
    with open(path, encoding="utf-8") as f:
        return f.read().rstrip("\n").split("\n")
