"""CPU checks of the split-half kernels' tile geometry (csrc/fused2h_impl.h,
HGeo and hmask), restated here: for every window the kernels instantiate and
both head widths, the LDS blocks of a wavefront cover each query's window
exactly once under the lane masks, the 16-byte row reads of a block fall in
distinct banks, the reads stay within a slot column, and the staged halo and
its scalars fit the 160 KiB of LDS.  A wrong block shape, element layout,
column stride or mask fails one of these.  The GPU parity tests
(test_gpu_parity.py, test_gpu_magnitudes.py) check the kernels themselves."""
import pytest

LDS_CAP = 160 * 1024


def geo(P, NT):
    WH = 2 if NT == 1 else 1
    TH, TW = 8 * WH, 16
    BR = 4 if P in (1, 5) else 2
    BC = 16 // BR
    NKH = (8 + 2 * P + BR - 1) // BR
    NKW = (2 + 2 * P + BC - 1) // BC
    HH = TH + 2 * P
    HWD = 2 * 7 + BC * NKW
    CR = HH + ((2 - HH % 4) + 4) % 4 if BR == 2 else HH + ((4 - HH % 16) + 16) % 16
    SB = (32 * NT + 8) * 2
    SWC = HWD if NT == 1 else TW + 2 * P
    return dict(WH=WH, TH=TH, TW=TW, BR=BR, BC=BC, NKH=NKH, NKW=NKW, HH=HH, HWD=HWD, CR=CR,
                SB=SB, SWC=SWC, LPX=CR * HWD, THREADS=64 * 8 * WH)


def element(BR, bi, bj, g, r):
    """Wave-relative key position of element 4 g + r of block (bi, bj)."""
    if BR == 2:  # row-major: element e at block row e // 8, column e % 8
        return 2 * bi + (g >> 1), 8 * bj + 4 * (g & 1) + r
    return 4 * bi + r, 4 * bj + g


CASES = [(P, NT) for NT in (1, 2) for P in (1, 2, 3, 5, 7) if not (NT == 2 and P == 7)]


@pytest.mark.parametrize("P,NT", CASES)
def test_blocks_cover_each_window_once(P, NT):
    G = geo(P, NT)
    seen = {}
    for bi in range(G["NKH"]):
        for bj in range(G["NKW"]):
            for g in range(4):
                for r in range(4):
                    kr, kc = element(G["BR"], bi, bj, g, r)
                    for j in range(16):
                        u1, u2 = kr - (j & 7), kc - (j >> 3)
                        if 0 <= u1 <= 2 * P and 0 <= u2 <= 2 * P:  # the lane's mask bit
                            key = (j, u1, u2)
                            assert key not in seen, (key, seen.get(key), (bi, bj, g, r))
                            seen[key] = (bi, bj, g, r)
    assert len(seen) == 16 * (2 * P + 1) ** 2


@pytest.mark.parametrize("P,NT", CASES)
def test_block_rows_read_conflict_free(P, NT):
    """Score-type rows: lanes j = 0..15 of a lane group read 16 bytes at
    slot(element j) * SB; distinct 16-byte units modulo 256 bytes (64 banks of
    4 bytes) mean no bank conflict within the group."""
    G = geo(P, NT)
    units = set()
    for j in range(16):
        row, col = element(G["BR"], 0, 0, j >> 2, j & 3)
        units.add(((row + G["CR"] * col) * G["SB"] // 16) % 16)
    assert len(units) == 16


@pytest.mark.parametrize("P,NT", [c for c in CASES if c[0] not in (1, 5)])
def test_transposing_reads_conflict_free(P, NT):
    """Apply-type rows of 2x8 blocks: lane j of lane group g reads 8 bytes,
    channels 4 (j & 3) .. + 3 of element 4 g + (j >> 2), at
    slot * SB + 8 (j & 3) (+ 32 for the low halves, + 64 per sub-pixel).  The
    32 lanes of groups (0, 1) and of groups (2, 3) read 256 bytes each: every
    4-byte bank of the 64 must be hit once.  2x2 element groups hit half of
    them twice."""
    G = geo(P, NT)
    for h in range(NT):
        for lo in (0, 32):
            for half in (0, 1):
                banks = []
                for lane in range(32 * half, 32 * half + 32):
                    j, g = lane & 15, lane >> 4
                    row, col = element(2, 0, 0, g, j >> 2)
                    a = (row + G["CR"] * col) * G["SB"] + 64 * h + lo + 8 * (j & 3)
                    banks += [(a // 4) % 64, (a // 4 + 1) % 64]
                assert sorted(banks) == list(range(64)), (h, lo, half)


@pytest.mark.parametrize("P,NT", CASES)
def test_reads_stay_in_slots_and_halo_fits(P, NT):
    G = geo(P, NT)
    # a wavefront's block rows stay within its slot column; its columns within the slots
    assert 8 * (G["WH"] - 1) + G["BR"] * G["NKH"] <= G["CR"]
    assert 2 * 7 + G["BC"] * G["NKW"] <= G["HWD"]
    # every key of a window lies in a staged row and column
    assert 8 * (G["WH"] - 1) + 7 + 2 * P < G["HH"] and 2 * 7 + 1 + 2 * P < G["SWC"]
    assert G["HH"] * G["SWC"] <= G["THREADS"]  # one staged pixel per thread
    for nscal in (0, 1, 2):  # scalars: none, Distance key bias, the key-centric pass's two
        assert 2 * G["LPX"] * G["SB"] + nscal * G["LPX"] * 4 + 16 <= LDS_CAP


def test_4x4_blocks_do_less_work_at_ws_11():
    two_by_eight = (4 + 5) * ((2 + 10 + 7) // 8) * 16
    g = geo(5, 2)
    assert g["BR"] == 4 and g["NKH"] * g["NKW"] * 16 == 240 and two_by_eight == 288


def banded_tile(t, tiles_h, tiles_w):
    """circatt_common.h banded_tile: bands of 8 tile rows, column by column."""
    full = (tiles_h >> 3) * 8 * tiles_w
    if t < full:
        band, r = divmod(t, 8 * tiles_w)
        return 8 * band + (r & 7), r >> 3
    bh, r = tiles_h & 7, t - full
    return (tiles_h & ~7) + r % bh, r // bh


def test_banded_tile_order_is_a_bijection_with_compact_runs():
    for th_n in range(1, 41):
        for tw_n in range(1, 23):
            tiles = [banded_tile(t, th_n, tw_n) for t in range(th_n * tw_n)]
            assert sorted(tiles) == [(h, w) for h in range(th_n) for w in range(tw_n)], (th_n, tw_n)
    # 64 consecutive tiles of a full band form an 8 x 8 block
    tiles = [banded_tile(t, 64, 64) for t in range(64 * 5, 64 * 6)]
    assert {h for h, _ in tiles} == set(range(8)) and len({w for _, w in tiles}) == 8


# ---- one-dimensional signals (HGeo<P, NT, true>) ----

def geo1(P, NT):
    """The 1D geometry: 16 (16 real components) or 8 (32) wavefronts of 16
    register pixels stacked along the line, 16x1 LDS blocks, one slot column."""
    WH = 16 if NT == 1 else 8
    TH = 16 * WH
    NKH = (16 + 2 * P + 15) // 16
    HH = TH + 2 * P
    CR = 16 * (WH - 1) + 16 * NKH
    SB = (32 * NT + 8) * 2
    return dict(WH=WH, TH=TH, NKH=NKH, HH=HH, CR=CR, SB=SB, THREADS=64 * WH, LPX=CR)


CASES1 = [(P, NT) for P in (7, 31) for NT in (1, 2)]


def hmask1(P, bi, g, r, j):
    """Lane mask bit of element 4 g + r of block bi for query j (fused2h_impl.h hmask, BR = 16)."""
    kr = 16 * bi + 4 * g + r
    return 0 <= kr - j <= 2 * P


@pytest.mark.parametrize("P,NT", CASES1)
def test_1d_blocks_cover_each_window_once(P, NT):
    """Query j of a wavefront (pixel h0 + 16 wh + j) meets block bi's element e
    at slot 16 wh + 16 bi + e, i.e. pixel h0 - P + 16 wh + 16 bi + e: window
    offset 16 bi + e - P - j.  Under the lane masks every offset -P .. P occurs
    exactly once per query."""
    G = geo1(P, NT)
    for j in range(16):
        offs = [16 * bi + 4 * g + r - P - j
                for bi in range(G["NKH"]) for g in range(4) for r in range(4) if hmask1(P, bi, g, r, j)]
        assert sorted(offs) == list(range(-P, P + 1)), j


@pytest.mark.parametrize("P,NT", CASES1)
def test_1d_reads_stay_in_slots_and_halo_fits(P, NT):
    G = geo1(P, NT)
    # the last wavefront's last block ends inside the column; staged rows fit
    assert 16 * (G["WH"] - 1) + 16 * G["NKH"] <= G["CR"]
    assert G["HH"] <= G["CR"]
    # every key of every window lies in a staged row: wavefront wh's query j
    # reads rows 16 wh + j .. 16 wh + j + 2P
    assert 16 * (G["WH"] - 1) + 15 + 2 * P < G["HH"]
    assert G["HH"] <= G["THREADS"]  # one staged pixel per thread
    for nscal in (0, 1, 2):
        assert 2 * G["LPX"] * G["SB"] + nscal * G["LPX"] * 4 + 16 <= LDS_CAP


@pytest.mark.parametrize("P,NT", CASES1)
def test_1d_block_rows_read_conflict_free(P, NT):
    """Score-type rows of a 16x1 block: 16 consecutive slots, an odd number of
    16-byte units apart, fall on 16 distinct units of 256 bytes."""
    G = geo1(P, NT)
    units = {(j * G["SB"] // 16) % 16 for j in range(16)}
    assert len(units) == 16


# ---- one-dimensional planar rows by 16-byte DMA (LGeo WIDE) ----

def wide1(P, NT, mode, dist):
    """LDS layout of the row-DMA kernels (fused2h_impl.h LGeo, WIDE)."""
    G = geo1(P, NT)
    NCH = 16 * NT
    XA = (4 - P % 4) % 4
    NXS = (G["HH"] + XA + 3) // 4 * 4
    NRT = {"fwd": 1, "bwdq": 3, "bwdkv": 2}[mode]
    nscal = 2 if mode == "bwdkv" else (1 if dist else 0)
    OX = 2 * G["LPX"] * G["SB"] + nscal * G["LPX"] * 4
    OXS = OX + 16
    OXR = OXS + 2 * NCH * NXS * 4
    return dict(G, NCH=NCH, XA=XA, NXS=NXS, NRT=NRT, OXS=OXS, OXR=OXR,
                bytes=OXR + NRT * NCH * G["TH"] * 4)


@pytest.mark.parametrize("P,NT", CASES1)
def test_1d_wide_rows_fit_and_align(P, NT):
    for mode in ("fwd", "bwdq", "bwdkv"):
        for dist in (False, True):
            W = wide1(P, NT, mode, dist)
            assert W["bytes"] <= LDS_CAP, (mode, dist)
            # 16-byte DMA destinations: row starts and 256-pixel parts
            assert W["OXS"] % 16 == 0 and W["OXR"] % 16 == 0 and W["NXS"] % 4 == 0
            assert W["TH"] <= 256  # one instruction (64 lanes x 4 pixels) per register row
            # the halo origin h0 - P moved back by XA is a multiple of 4
            assert (P + W["XA"]) % 4 == 0 and W["NXS"] >= W["HH"] + W["XA"]


@pytest.mark.parametrize("P,NT", CASES1)
@pytest.mark.parametrize("n1", [4, 24, 100, 260, 1000, 4096])
def test_1d_wide_staged_rows_hold_the_halo(P, NT, n1):
    """Lane l of part m loads pixels o4 + 4 (64 m + l) .. + 3 (mod n1) into XS
    positions 4 (64 m + l) ..; the staged pixel px then reads position
    px + XA, which must hold pixel (h0 - P + px) mod n1, and no 4-pixel chunk
    may straddle the wrap."""
    W = wide1(P, NT, "fwd", False)
    XA, NXS, TH, HH = W["XA"], W["NXS"], W["TH"], W["HH"]
    for h0 in range(0, n1, TH):
        hsh = (h0 - P) % n1            # the kernel's halo origin
        o4 = hsh - XA if hsh >= XA else hsh - XA + n1
        assert o4 % 4 == 0 and 0 <= o4 < n1
        row = {}
        for l4 in range(NXS // 4):
            p4 = o4 + 4 * l4
            p4 = (p4 - n1 if p4 >= n1 else p4) if n1 >= NXS else p4 % n1
            assert p4 % 4 == 0 and p4 + 3 < n1
            for e in range(4):
                row[4 * l4 + e] = p4 + e
        for px in range(HH):
            assert row[px + XA] == (h0 - P + px) % n1, (h0, px)
