"""CPU check of the apply kernels' chunk staging on border tiles
(csrc/apply_rb.hip: the 2D row kernel, A2 and apply2_body, and the
wide-window kernel, AW and apply_wide_body), restated here.

The border form stages every slot of every chunk with a single-slot load
whose source element undoes the reference's rotation of the slot order near
the image border (src/circulant.jl:10-14, 30-39).  The mixed form stages
the chunks that are not rotated in 16-byte pieces, masks the piece lanes of
rotated chunks (gap lanes stay active), and covers the run of rotated chunks
with a window of single-slot loads.  For every window, both directions and
the border tiles of several image widths, every slot that the products read
must hold the same source element in both forms, no load may write past the
chunk buffer, and every piece instruction must keep an active lane (so that
it is issued and the load counts of the waits hold).  A wrong run start, a
window too short or a mask on the wrong chunk fails one of these.  The GPU
parity tests check the kernels themselves."""
import pytest


def geo(WS, trans):
    P = (WS - 1) // 2
    NSRC = 64 + 2 * P if trans else 64
    WSP = (WS + 3) & ~3
    Q = WSP // 4
    BLK = 4 * Q + 1
    NSLOT = (NSRC + 3) // 4 * BLK
    NZ4 = (NSLOT + 63) // 64
    NZ1 = (4 * NSLOT + 63) // 64
    NZB = max(NZ4 * 256, NZ1 * 64)
    ND = (2 * P * WSP + 4 * ((2 * P + 3) // 4) + 63) // 64
    return dict(P=P, NSRC=NSRC, WSP=WSP, Q=Q, BLK=BLK, NZ4=NZ4, NZ1=NZ1, NZB=NZB, ND=ND)


def shift0(c, n, p):
    return c - p if c + 1 <= p else (p - n + c + 1 if c + 1 > n - p else 0)


def fold(v, ws):
    return v + ws if v < 0 else (v - ws if v >= ws else v)


def piece_slot(G, f):
    kb, r = divmod(f, G["BLK"])
    rq = r if r < 4 * G["Q"] else 0
    w = min(4 * kb + rq // G["Q"], G["NSRC"] - 1)
    return kb, r, w, rq % G["Q"]


def border_form(G, WS, trans, n1, f1):
    off = G["P"] if trans else 0
    lds = {}
    for m in range(G["NZ1"]):
        for lane in range(64):
            _, _, w, q = piece_slot(G, (lane + 64 * m) >> 2)
            j = 4 * q + ((lane + 64 * m) & 3)
            col = (f1 - off + w) % n1
            lds[64 * m + lane] = {(col, fold((j if j < WS else 0) + shift0(col, n1, G["P"]), WS))}
    return lds


def mixed_form(G, WS, trans, n1, f1):
    P, off = G["P"], (G["P"] if trans else 0)
    lds = {}
    for m in range(G["NZ4"]):
        active = 0
        for lane in range(64):
            _, r, w, q = piece_slot(G, lane + 64 * m)
            col = (f1 - off + w) % n1
            if r >= 4 * G["Q"] or shift0(col, n1, P) == 0:
                active += 1
                for t in range(4):
                    lds.setdefault(256 * m + 4 * lane + t, set()).add((col, 4 * q + t))
        assert active > 0, ("piece instruction without an active lane", m)
    c0 = (f1 - off) % n1
    d = (n1 - P - c0) % n1
    a0 = d if d < G["NSRC"] else 0
    zbase = min(a0 * G["WSP"] + 4 * (a0 >> 2), G["NZB"] - 64 * G["ND"])
    for i in range(G["ND"]):
        for lane in range(64):
            ps = zbase + 64 * i + lane
            sl = ps >> 2
            kb, r = divmod(sl, G["BLK"])
            w = 4 * kb + r // G["Q"]
            j = 4 * (r % G["Q"]) + (ps & 3)
            col, e = 0, 0
            if r < 4 * G["Q"] and w < G["NSRC"]:
                col = (f1 - off + w) % n1
                e = fold(j + shift0(col, n1, P), WS) if j < WS else 0
            lds.setdefault(ps, set()).add((col, e))
    return lds


def border_tiles(G, n1):
    """Tile columns apply2_tile sends to a border form (launch_rb's fa, fb)."""
    edge = max(8, 2 * G["P"])  # kHalo = 8
    tiles1 = (n1 + 63) // 64
    fa = (edge + 63) // 64
    fb = (n1 - 64 - edge) // 64 + 1 if n1 - 64 - edge >= 0 else 0
    fb = max(min(fb, tiles1), fa)
    return [t for t in range(tiles1) if not fa <= t < fb]


@pytest.mark.parametrize("WS", [3, 5, 7, 9, 11, 13, 15])
@pytest.mark.parametrize("trans", [False, True])
def test_mixed_border_staging_matches_single_slot_staging(WS, trans):
    G = geo(WS, trans)
    assert 64 * G["ND"] <= G["NZB"]
    lo = G["NSRC"] + 2 * G["P"]  # apply2_tile's condition for the mixed form
    for n1 in sorted({lo, lo + 1, lo + 3, 96, 128, 130, 200, 256, 320, 511, 512}):
        if n1 < lo:
            continue
        for t1 in border_tiles(G, n1):
            f1 = 64 * t1
            ref = border_form(G, WS, trans, n1, f1)
            mix = mixed_form(G, WS, trans, n1, f1)
            assert max(mix) < G["NZB"] and max(ref) < G["NZB"]
            for w in range(G["NSRC"]):
                for j in range(WS):
                    pos = w * G["WSP"] + 4 * (w // 4) + j
                    assert mix.get(pos) == ref[pos], (n1, t1, w, j, mix.get(pos), ref[pos])


def test_a_planted_short_window_is_caught():
    """The check above fails when the window is one load short at ws = 15."""
    G = geo(15, True)
    G["ND"] -= 1
    n1, f1 = 128, 0
    ref, mix = border_form(G, 15, True, n1, f1), mixed_form(G, 15, True, n1, f1)
    bad = [(w, j) for w in range(G["NSRC"]) for j in range(15)
           if mix.get(w * G["WSP"] + 4 * (w // 4) + j) != ref[w * G["WSP"] + 4 * (w // 4) + j]]
    assert bad


# Wide windows (apply_wide_body, AW): sub-chunks of kJC = 16 slots of window
# row dd's slots 16 jc .. 16 jc + 15; the mixed form applies for p <= 15 with
# a window of kNDW single-slot loads per lane.
KJC, WIDE_MIX_P = 16, 15
KNDW = (2 * WIDE_MIX_P * KJC + 4 * ((2 * WIDE_MIX_P + 3) // 4) + 63) // 64


def wide_geo(trans):
    NSRC = 64 + KJC - 1 if trans else 64
    Q, BLK = KJC // 4, KJC + 1
    NSLOT = (NSRC + 3) // 4 * BLK
    NZ4, NZ1 = (NSLOT + 63) // 64, (4 * NSLOT + 63) // 64
    return dict(NSRC=NSRC, Q=Q, BLK=BLK, NZ4=NZ4, NZ1=NZ1, NZB=max(NZ4 * 256, NZ1 * 64))


def wide_slot(G, f):
    kb, r = divmod(f, G["BLK"])
    rq = r if r < 4 * G["Q"] else 0
    return r, min(4 * kb + rq // G["Q"], G["NSRC"] - 1), rq % G["Q"]


def wide_forms(G, WS, n1, c0, jc):
    P = (WS - 1) // 2
    ref, mix = {}, {}
    for m in range(G["NZ1"]):  # border form: single slots (zo_border)
        for lane in range(64):
            _, w, q = wide_slot(G, (lane + 64 * m) >> 2)
            j = KJC * jc + 4 * q + ((lane + 64 * m) & 3)
            col = (c0 + w) % n1
            ref[64 * m + lane] = {(col, fold(j + shift0(col, n1, P), WS) if j < WS else 0)}
    for m in range(G["NZ4"]):  # mixed form: pieces of columns not rotated
        active = 0
        for lane in range(64):
            r, w, q = wide_slot(G, lane + 64 * m)
            col = (c0 + w) % n1
            if r >= 4 * G["Q"] or shift0(col, n1, P) == 0:
                active += 1
                for t in range(4):
                    mix.setdefault(256 * m + 4 * lane + t, set()).add((col, KJC * jc + 4 * q + t))
        assert active > 0
    d = (n1 - P - c0 % n1) % n1
    a0 = d if d < G["NSRC"] else 0
    zb = min(a0 * KJC + 4 * (a0 >> 2), G["NZB"] - 64 * KNDW)
    for i in range(KNDW):
        for lane in range(64):
            ps = zb + 64 * i + lane
            kb, r = divmod(ps >> 2, G["BLK"])
            w = 4 * kb + r // G["Q"]
            j = KJC * jc + 4 * (r % G["Q"]) + (ps & 3)
            col, e = 0, 0
            if r < 4 * G["Q"] and w < G["NSRC"]:
                col = (c0 + w) % n1
                e = fold(j + shift0(col, n1, P), WS) if j < WS else 0
            mix.setdefault(ps, set()).add((col, e))
    return ref, mix


@pytest.mark.parametrize("WS", [17, 19, 23, 27, 31])
@pytest.mark.parametrize("trans", [False, True])
def test_wide_mixed_border_staging_matches_single_slot_staging(WS, trans):
    G = wide_geo(trans)
    P = (WS - 1) // 2
    assert P <= WIDE_MIX_P and 64 * KNDW <= G["NZB"]
    njc = (WS + KJC - 1) // KJC
    lo = G["NSRC"] + 2 * P
    for n1 in sorted({lo, lo + 1, lo + 5, 128, 200, 512, 1000}):
        edge = 2 * P + KJC  # set_wide's interior margin
        tiles1 = (n1 + 63) // 64
        fa = (edge + 63) // 64
        fb = max(min((n1 - 64 - edge) // 64 + 1 if n1 - 64 - edge >= 0 else 0, tiles1), fa)
        for t1 in [t for t in range(tiles1) if not fa <= t < fb]:
            f1 = 64 * t1
            for jc in range(njc):
                c0 = f1 - (KJC * jc - P) - (KJC - 1) if trans else f1
                ref, mix = wide_forms(G, WS, n1, c0, jc)
                assert max(mix) < G["NZB"] and max(ref) < G["NZB"]
                for w in range(G["NSRC"]):
                    for jj in range(min(KJC, WS - KJC * jc)):  # slots read (the rest read as zero)
                        pos = w * KJC + 4 * (w // 4) + jj
                        assert mix.get(pos) == ref[pos], (n1, t1, jc, w, jj)
