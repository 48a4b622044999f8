"""Host replay of the scans' LDS traffic, phase by phase (no GPU).

The forward and reverse scans pass tiles between the waves of a workgroup
through LDS: the state (or its gradient) transposed, Vn (or dVn), and in the
level-0 reverse scan mix_0 dO and every wave's private copy of its operand
slices. A workgroup barrier separates the phases of a step; where a step
ends without one, its last phase runs together with the next step's first.
For every kernel configuration the op launches, this test enumerates, per
phase, the LDS elements each wave writes and reads (both planes of a split
tile), from the same index formulas as the kernels (csrc/scan.hip,
csrc/scan_bwd.hip), and checks:

  * no element is written by one wave and read or written by another within
    one phase (including the merged end-of-step / start-of-step phase);
  * every element a phase reads was written earlier in the same step (no
    read of a slot the step has not filled);
  * a wave's private operand region is touched by that wave only, stays
    inside its bounds, and is filled before it is read in each step.

A missing barrier, a wrong row stride, or two waves' tiles overlapping would
fail one of these.
"""

import itertools

import pytest

WAVE = 64
BV = 32          # columns of V per scan workgroup
CT = BV // 16


def lanes():
    return range(WAVE)


class SplitLDS:
    """A split bf16 tile: hi plane, then lo plane, ``plane`` elements apart."""

    def __init__(self, name, plane):
        self.name, self.plane = name, plane

    def span(self, off, n):
        return [(self.name, p * self.plane + off + e) for p in (0, 1) for e in range(n)]


class Phase:
    def __init__(self):
        self.w, self.r = {}, {}

    def write(self, wave, cells):
        self.w.setdefault(wave, set()).update(cells)

    def read(self, wave, cells):
        self.r.setdefault(wave, set()).update(cells)


def check_phases(phases, bounds):
    """phases: list of Phase for one step, in order; the last one merges with
    the first of the next step when the step ends without a barrier (the
    caller passes merged=True)."""
    written = set()
    for i, ph in enumerate(phases):
        waves = set(ph.w) | set(ph.r)
        for a, b in itertools.permutations(waves, 2):
            wa = ph.w.get(a, set())
            assert not (wa & ph.w.get(b, set())), f"phase {i}: waves {a}, {b} write one slot"
            assert not (wa & ph.r.get(b, set())), f"phase {i}: wave {b} reads what wave {a} writes"
        for cells in list(ph.w.values()) + list(ph.r.values()):
            for name, e in cells:
                assert 0 <= e < bounds[name], f"{name}[{e}] outside {bounds[name]}"
        for wv, cells in ph.r.items():
            missing = cells - written - ph.w.get(wv, set())
            assert not missing, f"phase {i}: wave {wv} reads unwritten {sorted(missing)[:4]}"
        for cells in ph.w.values():
            written |= cells


def merged(last, first):
    ph = Phase()
    for src in (last, first):
        for wv, c in src.w.items():
            ph.write(wv, c)
        for wv, c in src.r.items():
            ph.read(wv, c)
    return ph


def acc_row(l, r=0):
    return 4 * (l >> 4) + r


# --------------------------------------------------------------- forward scan

def scan_fwd_step(K, M, OUT, NWV=4):
    """csrc/scan.hip scan_fwd_kernel, bf16 (KS = 32, KPL = 8, PAD = 8)."""
    KS, PAD = 32, 8
    LDS_ST, LDS_VN = K + PAD, M + PAD
    sST, sVn = SplitLDS("st", BV * LDS_ST), SplitLDS("vn", BV * LDS_VN)
    RTS, RTV = K // 16, M // 16
    TPW = RTS * CT // NWV
    NVT = RTV * CT
    NVP = -(-NVT // NWV)
    ONE_RT = NWV % RTV == 0
    NSK, NSM = K // KS, -(-M // KS)

    def vn_tile(wv, p):
        if ONE_RT:
            g = wv + NWV * p
            return g < NVT, g % RTV, g // RTV
        return True, wv + NWV * (p // CT), p % CT

    A, B, C = Phase(), Phase(), Phase()
    for wv in range(NWV):
        for l in lanes():
            for i in range(TPW):
                g = wv * TPW + i
                rt, ct = g // CT, g % CT
                A.write(wv, sST.span((ct * 16 + (l & 15)) * LDS_ST + rt * 16 + acc_row(l), 4))
            for p in range(NVP):
                ok, rt, ct = vn_tile(wv, p)
                if not ok:
                    continue
                brow = (ct * 16 + (l & 15)) * LDS_ST + 8 * (l >> 4)
                for s in range(NSK):
                    B.read(wv, sST.span(brow + s * KS, 8))
                B.write(wv, sVn.span((ct * 16 + (l & 15)) * LDS_VN + rt * 16 + acc_row(l), 4))
                if OUT:
                    vrow = (ct * 16 + (l & 15)) * LDS_VN + 8 * (l >> 4)
                    for s in range(NSM):
                        C.read(wv, sVn.span(vrow + s * KS, 8))
            for i in range(TPW):
                ct = (wv * TPW + i) % CT
                vrow = (ct * 16 + (l & 15)) * LDS_VN + 8 * (l >> 4)
                for s in range(NSM):
                    if s * KS + 8 * (l >> 4) < M:
                        C.read(wv, sVn.span(vrow + s * KS, 8))
    bounds = {"st": 2 * BV * LDS_ST, "vn": 2 * BV * LDS_VN}
    # no barrier at the end of a step: C runs together with the next step's A
    return [A, B, merged(C, A)], bounds


@pytest.mark.parametrize("K,M,OUT", [(128, 64, True), (64, 64, True), (128, 64, False),
                                     (128, 32, False), (128, 16, False), (128, 128, False),
                                     (64, 128, False)])
def test_forward_scan_phases(K, M, OUT):
    phases, bounds = scan_fwd_step(K, M, OUT)
    check_phases(phases, bounds)


# ------------------------------------------------------- reverse scan, levels >= 1

def scan_bwd_upper_step(K, M):
    """csrc/scan_bwd.hip scan_bwd_kernel, bf16: dS'^T then dVn^T; no barrier
    at the end of a step."""
    KS, PAD = 32, 8
    LDS_ST, LDS_VN = K + PAD, M + PAD
    sdS, sdV = SplitLDS("dst", BV * LDS_ST), SplitLDS("dvn", BV * LDS_VN)
    RTS, RTV = K // 16, M // 16
    TPW, RPW = RTS * CT // 4, -(-RTV // 4)
    NSK, NSM = K // KS, -(-M // KS)
    A, B, C = Phase(), Phase(), Phase()
    for wv in range(4):
        for l in lanes():
            for i in range(TPW):
                g = wv * TPW + i
                rt, ct = g // CT, g % CT
                A.write(wv, sdS.span((ct * 16 + (l & 15)) * LDS_ST + rt * 16 + acc_row(l), 4))
            for p in range(RPW):
                rt = wv + 4 * p
                if rt >= RTV:
                    continue
                for ct in range(CT):
                    srow = (ct * 16 + (l & 15)) * LDS_ST + 8 * (l >> 4)
                    for s in range(NSK):
                        B.read(wv, sdS.span(srow + s * KS, 8))
                    B.write(wv, sdV.span((ct * 16 + (l & 15)) * LDS_VN + rt * 16 + acc_row(l), 4))
            for i in range(TPW):
                ct = i % CT
                vrow = (ct * 16 + (l & 15)) * LDS_VN + 8 * (l >> 4)
                for s in range(NSM):
                    if s * KS + 8 * (l >> 4) < M:
                        C.read(wv, sdV.span(vrow + s * KS, 8))
    bounds = {"dst": 2 * BV * LDS_ST, "dvn": 2 * BV * LDS_VN}
    return [A, B, merged(C, A)], bounds


@pytest.mark.parametrize("K,M", [(128, 64), (128, 128), (128, 32), (128, 16), (64, 64),
                                 (64, 16)])
def test_reverse_scan_upper_phases(K, M):
    phases, bounds = scan_bwd_upper_step(K, M)
    check_phases(phases, bounds)


# ------------------------------------------------------------ reverse scan, level 0

def frag_ofs(r, c, C):
    return ((r >> 4) * (C >> 5) + (c >> 5)) * 512 + ((((c & 31) >> 3) << 4) + (r & 15)) * 8 + (c & 7)


def slice_pos(ncw, r, cq):
    if ncw == 16:
        return (2 * r + cq) ^ (((r >> 3) & 1) << 3)
    return 4 * r + (cq ^ (((r >> 3) & 1) << 1))


def seg_of(ncw, i, l):
    if ncw == 16:
        return 2 * i + (l >> 5), (l & 31) >> 1, l & 1
    return i, l >> 2, l & 3


def tr_addr(ncw, l, ctl, s, hh):
    """Element offset (in one plane of a slice copy) that lane l hands
    ds_read_b64_tr_b16 for the A fragment of X^T, column tile ctl, k-step s,
    half hh (scan_bwd.hip tr_frag)."""
    run = 16 * ncw // 8
    xr = 32 * s + 8 * (l >> 4) + 4 * hh + ((l & 15) >> 2)
    cq = 2 * ctl + ((l & 3) >> 1)
    return ((xr >> 4) * run + slice_pos(ncw, xr & 15, cq)) * 8 + 4 * (l & 1)


def tr16(addrs, lds):
    """ds_read_b64_tr_b16 on 64 lanes: in each group of 16, lane q reads 4
    values D[q] at its address; lane p receives D[4 j + p // 4][p % 4], j =
    0..3 (the layout the GPU probe of the instruction showed)."""
    out = []
    for l in range(64):
        g, p = l >> 4, l & 15
        out.append([lds[addrs[16 * g + 4 * j + (p >> 2)] + (p & 3)] for j in range(4)])
    return out


@pytest.mark.parametrize("R,C,ncw", [(128, 64, 16), (64, 64, 16), (64, 128, 32), (64, 64, 16)])
def test_slice_copy_gives_transposed_fragments(R, C, ncw):
    """Every wave's slice copy, read with the transposing LDS read, yields the
    A fragments of X^T (row l % 16 of a tile, reduction indices
    32 s + 8 (l / 16) .. + 7), for every wave's column range."""
    import random
    rnd = random.Random(R * C + ncw)
    X = [[rnd.randrange(1 << 16) for _ in range(C)] for _ in range(R)]
    glob = [0] * (R * C)
    for r in range(R):
        for c in range(C):
            glob[frag_ofs(r, c, C)] = X[r][c]
    run = 16 * ncw // 8
    plane = (R // 16) * run * 8
    nl = R * ncw // 512
    for wv in range(C // ncw):
        c0 = ncw * wv
        lds = [None] * plane
        for i in range(nl):
            for l in lanes():
                rb, r, cq = seg_of(ncw, i, l)
                src = (rb * (C // 32) + c0 // 32) * 512 + (c0 % 32) * 16 + (16 * cq + r) * 8
                dst = (rb * run + slice_pos(ncw, r, cq)) * 8
                assert all(lds[dst + e] is None for e in range(8)), "slot written twice"
                lds[dst:dst + 8] = glob[src:src + 8]
        assert sum(x is not None for x in lds) == R * ncw
        for ctl in range(ncw // 16):
            for s in range(R // 32):
                frag = [[] for _ in lanes()]
                for hh in range(2):
                    got = tr16([tr_addr(ncw, l, ctl, s, hh) for l in lanes()], lds)
                    for l in lanes():
                        frag[l] += got[l]
                for l in lanes():
                    want = [X[32 * s + 8 * (l >> 4) + e][c0 + 16 * ctl + (l & 15)] for e in range(8)]
                    assert frag[l] == want, (wv, ctl, s, l)


def test_transposed_reads_are_bank_conflict_free():
    """The 32 lanes of a half-wave read 256 bytes of the slice copy spread
    over all 64 four-byte banks."""
    for ncw, R in ((16, 128), (16, 64), (32, 64)):
        for ctl in range(ncw // 16):
            for s in range(R // 32):
                for hh in range(2):
                    for half in (0, 1):
                        banks = set()
                        for l in range(32 * half, 32 * half + 32):
                            a = tr_addr(ncw, l, ctl, s, hh) * 2
                            banks |= {(a // 4) % 64, (a // 4 + 1) % 64}
                        assert len(banks) == 64, (ncw, R, ctl, s, hh, half)


def scan_bwd_l0_step(K):
    """csrc/scan_bwd.hip scan_bwd_l0_kernel, bf16 (M = 64): slice copies,
    dS'^T and (mix_0 dO)^T, then dVn^T; a barrier ends the step."""
    M, KS, PAD = 64, 32, 8
    LDS_ST, LDS_VN = K + PAD, M + PAD
    sdS, sdV, sdO = (SplitLDS("dst", BV * LDS_ST), SplitLDS("dvn", BV * LDS_VN),
                     SplitLDS("dot", BV * LDS_VN))
    TPW = (K // 16) * CT // 4
    TRT = TPW // CT
    ncw = 16 * TRT
    DOE = M * BV // 256

    def plane(R, n):
        return (R // 16) * (16 * n // 8) * 8

    pk, pq, pw = plane(K, 16), plane(M, 16), plane(M, ncw)
    opw = 2 * (pk + pq + 2 * pw)
    regions = {"K": (0, pk, K, 16), "Q": (2 * pk, pq, M, 16), "W": (2 * (pk + pq), pw, M, ncw),
               "G": (2 * (pk + pq) + 2 * pw, pw, M, ncw)}

    def op_cells(wv, reg, offs):
        base, pl, _, _ = regions[reg]
        return [("op", wv * opw + base + p * pl + o) for p in (0, 1) for o in offs]

    A, B, C = Phase(), Phase(), Phase()
    for wv in range(4):
        for reg, (base, pl, R, n) in regions.items():
            for i in range(R * n // 512):
                for l in lanes():
                    rb, r, cq = seg_of(n, i, l)
                    d = (rb * (16 * n // 8) + slice_pos(n, r, cq)) * 8
                    A.write(wv, op_cells(wv, reg, range(d, d + 8)))
        for l in lanes():
            tid = wv * WAVE + l
            for i in range(TPW):
                g = wv * TPW + i
                rt, ct = g // CT, g % CT
                A.write(wv, sdS.span((ct * 16 + (l & 15)) * LDS_ST + rt * 16 + acc_row(l), 4))
            c, vl = tid // (BV // DOE), (tid % (BV // DOE)) * DOE
            for q in range(DOE):
                A.write(wv, sdO.span((vl + q) * LDS_VN + c, 1))
            for s in range(K // KS):
                for hh in range(2):
                    a = tr_addr(16, l, 0, s, hh)
                    B.read(wv, op_cells(wv, "K", range(a, a + 4)))
            for s in range(M // KS):
                for hh in range(2):
                    a = tr_addr(16, l, 0, s, hh)
                    B.read(wv, op_cells(wv, "Q", range(a, a + 4)))
            for ct in range(CT):
                srow = (ct * 16 + (l & 15)) * LDS_ST + 8 * (l >> 4)
                orow = (ct * 16 + (l & 15)) * LDS_VN + 8 * (l >> 4)
                for s in range(K // KS):
                    B.read(wv, sdS.span(srow + s * KS, 8))
                for s in range(M // KS):
                    B.read(wv, sdO.span(orow + s * KS, 8))
                B.write(wv, sdV.span((ct * 16 + (l & 15)) * LDS_VN + wv * 16 + acc_row(l), 4))
            for t in range(TRT):
                for s in range(M // KS):
                    for hh in range(2):
                        a = tr_addr(ncw, l, t, s, hh)
                        C.read(wv, op_cells(wv, "W", range(a, a + 4)))
                        C.read(wv, op_cells(wv, "G", range(a, a + 4)))
                for ct in range(CT):
                    vrow = (ct * 16 + (l & 15)) * LDS_VN + 8 * (l >> 4)
                    for s in range(M // KS):
                        C.read(wv, sdV.span(vrow + s * KS, 8))
                        C.read(wv, sdO.span(vrow + s * KS, 8))
    bounds = {"dst": 2 * BV * LDS_ST, "dvn": 2 * BV * LDS_VN, "dot": 2 * BV * LDS_VN,
              "op": 4 * opw}
    # each wave touches only its own region of the slice copies
    for ph in (A, B, C):
        for wv, cells in list(ph.w.items()) + list(ph.r.items()):
            for name, e in cells:
                if name == "op":
                    assert wv * opw <= e < (wv + 1) * opw, (wv, e)
    # the step ends with a barrier
    return [A, B, C], bounds, opw


@pytest.mark.parametrize("K", [128, 64])
def test_reverse_scan_level0_phases(K):
    phases, bounds, opw = scan_bwd_l0_step(K)
    check_phases(phases, bounds)
    # the whole LDS of the kernel fits one CU (160 KB)
    assert (bounds["dst"] + bounds["dvn"] + bounds["dot"] + bounds["op"]) * 2 <= 160 * 1024
