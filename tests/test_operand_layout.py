"""The tiled operand layout of the S8 GEMMs (csrc/s8.h tiled_index,
csrc/s8.hip tile_offsets, tile_offsets_km, bkm_lane, bkm_lane_f16,
load_b_km and the epilogue's put_row), checked on the CPU.

The address arithmetic of those functions is restated here and run over
element ids: a tiled operand in memory, the direct-to-LDS loads of one K
stage (lane l of a load writes LDS bytes 16 l .. 16 l + 15 of its 1 KB), the
fragment reads (ds_read_b64_tr_b16: within a 16-lane group, lane 4a + b
receives element b of the 8-byte reads of lanes a, a + 4, a + 8, a + 12),
and the LDS bank of every 4-byte word a read touches.  The GPU parity tests
check the kernels themselves; this file pins the scheme: every element lands
once, each lane receives exactly its fragment, the transposed reads are
conflict-free for 32 banks serving 16 lanes and 64 banks serving 32, and the
epilogue's stores address the same bytes as tiled_index.
"""
import pytest


def tiled_index(r, c, ld):
    return ((((r >> 4) * (ld >> 4)) + (c >> 4)) << 8) + ((r & 15) << 4) + (c & 15)


def swz4(r):
    return ((r >> 1) ^ (r >> 2)) & 3


def swzt(row, piece):
    return 2 * (((row >> 1) ^ piece) & 1)


def swzt_h(row):
    return 2 * ((row >> 1) & 1)


def sw23(p):
    """s8.hip sw23: bits 2 and 3 of a fragment row index swapped."""
    return (p & ~12) | ((p & 4) << 1) | ((p & 8) >> 1)


def plane_hi(idx):
    return 2 * (idx & ~15) + (idx & 15)


def memory(form, rows, ld):
    """byte offset -> element id of a tiled operand (ld in elements)."""
    m = {}
    for r in range(rows):
        for c in range(ld):
            if form == "planes":
                h = plane_hi(tiled_index(r, c, ld))
                m[2 * h] = ("hi", r, c)
                m[2 * (h + 16)] = ("lo", r, c)
            elif form == "f32":
                m[4 * tiled_index(r, c, ld)] = ("f", r, c)
            else:  # f16: pieces of 16 rows x 32 columns
                m[(((r >> 4) * (ld >> 5) + (c >> 5)) << 10) + ((r & 15) << 6) + 2 * (c & 31)] = ("x", r, c)
    return m


UNIT = {"planes": 2, "f32": 4, "f16": 2}


def load(mem, form, offsets, lds, base):
    for lane, g in enumerate(offsets):
        for b in range(0, 16, UNIT[form]):
            assert base + 16 * lane + b not in lds, "two loads wrote one LDS byte"
            lds[base + 16 * lane + b] = mem.get(g + b)


def test_tiled_index_is_a_bijection_keeping_row_blocks_in_place():
    rows, ld = 48, 64
    seen = set()
    for r in range(rows):
        for c in range(ld):
            t = tiled_index(r, c, ld)
            assert t not in seen
            seen.add(t)
            # a 16-row block occupies the elements of its 16 rows
            assert (r // 16) * 16 * ld <= t < (r // 16 + 1) * 16 * ld
            # the 64-byte run of a row's K group is contiguous
            assert t % 16 == c % 16
    assert seen == set(range(rows * ld))


@pytest.mark.parametrize("form", ["planes", "f32", "f16"])
@pytest.mark.parametrize("tm,waves", [(128, 4), (256, 4), (256, 8)])
def test_row_major_tile_loads(form, tm, waves):
    """tile_offsets: the loads of one 16-deep stage (32-deep for FP16) of
    rows row0 .. row0 + tm - 1 leave logical chunk kc of tile row r at LDS
    slot kc ^ swz4(r) of row r, as the fragment reads expect."""
    ld, row0, kt = 256, tm, 3
    mem = memory(form, row0 + tm, ld)
    ldu = ld // 2 if form == "f16" else ld  # 4-byte units
    base = 64 * (16 * kt)  # stage base: 64 k0 bytes, k0 = 16 kt units
    n = tm * 16 * 4 // 1024 // waves
    lds = {}
    for w in range(waves):
        for i in range(n):
            blk = (row0 >> 4) + w * n + i
            offs = [base + blk * (ldu >> 4) * 1024 + (l >> 2) * 64 + (((l & 3) ^ swz4(l >> 2)) << 4) for l in range(64)]
            load(mem, form, offs, lds, (w * n + i) * 1024)
    for r in range(tm):
        for kc in range(4):
            addr = (r * 4 + (kc ^ swz4(r))) << 4
            for b in range(0, 16, UNIT[form]):
                if form == "planes":
                    want = ("hi" if kc < 2 else "lo", row0 + r, 16 * kt + 8 * (kc & 1) + b // 2)
                elif form == "f32":
                    want = ("f", row0 + r, 16 * kt + 4 * kc + b // 4)
                else:
                    want = ("x", row0 + r, 32 * kt + 8 * kc + b // 2)
                assert lds[addr + b] == want


def tr16(lds, addr_of):
    out = {}
    for lane in range(64):
        grp, a, b = lane >> 4, (lane & 15) >> 2, lane & 3
        out[lane] = [lds.get(addr_of(16 * grp + a + 4 * t) + 2 * b) for t in range(4)]
    return out


def conflicts(addr_of, lanes_per_cycle, banks):
    worst = 0
    for start in range(0, 64, lanes_per_cycle):
        words = {}
        for lane in range(start, start + lanes_per_cycle):
            a = addr_of(lane) // 4
            for w in (a, a + 1):
                words.setdefault(w % banks, set()).add(w)
        worst = max(worst, max(len(v) for v in words.values()) - 1)
    return worst


def km_stage(form, tn, waves, ld, k0, n0):
    """tile_offsets_km: the LDS tile of one K-major stage of a tiled operand
    with ld columns (rows k0.., columns n0 .. n0 + tn - 1)."""
    rows = k0 + 32
    mem = memory(form, rows, ld)
    f16 = form == "f16"
    ldu, n0u = (ld // 2, n0 // 2) if f16 else (ld, n0)
    kmrow = 2 * tn if f16 else 4 * tn
    block_pieces = kmrow // 64
    # issue_stage: 4 k0 ld KMSTEP bytes for a stage at k0 (4-byte units; FP16
    # stages of 32 rows advance k0 by 16, KMSTEP 2): k0 rows of 4 ld_u bytes
    base = k0 * 4 * ldu
    n = tn // 16 // waves
    lds = {}
    for w in range(waves):
        for i in range(n):
            q = w * n + i
            hb, jj = (q // block_pieces, q % block_pieces) if f16 else (0, q)
            offs = []
            for l in range(64):
                m = l >> 2
                sw = swzt_h(m) if f16 else (swzt(m, q) if form == "planes" else 0)
                offs.append(base + (hb * (ldu >> 4) + (n0u >> 4) + jj) * 1024 + m * 64 + (((l & 3) ^ sw) << 4))
            load(mem, form, offs, lds, q * 1024)
    return lds


@pytest.mark.parametrize("tn,waves", [(128, 4), (256, 8)])
def test_k_major_planes_reads(tn, waves):
    """bkm_lane + load_b_km (BF16 planes): lane (n, h) of the wave's column
    block j gets B[k0 + 8h .. + 7][n] of each plane, conflict-free."""
    ld, k0, n0 = 512, 32, tn
    lds = km_stage("planes", tn, waves, ld, k0, n0)
    for wn in range(tn // 64):
        def lane_off(lane, pl):
            g, s = lane >> 4, lane & 15
            k = 8 * (g >> 1) + (s >> 2)
            return (4 * wn + (g & 1)) * 1024 + k * 64 + 8 * ((s >> 1) & 1) + (((2 * pl + (s & 1)) ^ swzt(k, g & 1)) << 4)
        for j in range(2):
            for pl in range(2):
                for second in range(2):
                    addr_of = lambda sl: lane_off(sl, pl) + 2048 * j + 256 * second
                    got = tr16(lds, addr_of)
                    for lane in range(64):
                        n, h = 64 * wn + 32 * j + sw23(lane & 31), lane >> 5
                        want = [("hi" if pl == 0 else "lo", k0 + 8 * h + 4 * second + t, n0 + n) for t in range(4)]
                        assert got[lane] == want
                    assert conflicts(addr_of, 16, 32) == 0 and conflicts(addr_of, 32, 64) == 0


@pytest.mark.parametrize("tn,waves", [(128, 4), (256, 8)])
def test_k_major_f16_reads(tn, waves):
    """bkm_lane_f16 + load_b_km (FP16, 32-deep stages): lane (n, h) of
    block j gets B[k0 + 16 half + 8h .. + 7][n], conflict-free."""
    ld, k0, n0 = 512, 64, tn
    lds = km_stage("f16", tn, waves, ld, k0, n0)
    block_bytes = (2 * tn) // 64 * 1024
    for wn in range(tn // 64):
        def lane_off(lane, j):
            g, s = lane >> 4, lane & 15
            k = 8 * (g >> 1) + (s >> 2)
            return (2 * wn + j) * 1024 + k * 64 + 8 * ((s >> 1) & 1) + (((2 * (g & 1) + (s & 1)) ^ swzt_h(k)) << 4)
        for j in range(2):
            for half in range(2):
                for second in range(2):
                    addr_of = lambda sl: lane_off(sl, j) + half * block_bytes + 256 * second
                    got = tr16(lds, addr_of)
                    for lane in range(64):
                        n, h = 64 * wn + 32 * j + sw23(lane & 31), lane >> 5
                        want = [("x", k0 + 16 * half + 8 * h + 4 * second + t, n0 + n) for t in range(4)]
                        assert got[lane] == want
                    assert conflicts(addr_of, 16, 32) == 0 and conflicts(addr_of, 32, 64) == 0


@pytest.mark.parametrize("tn,waves", [(128, 4), (256, 8)])
def test_k_major_f32_reads(tn, waves):
    """load_b_km (FP32 mode, natural column order): lane (n, h) reads
    B[k0 + 8h + q][n] at (4 wn + pp) KB + 512 h + 4 (lane & 15) + 2 KB j +
    64 q."""
    ld, k0, n0 = 512, 32, tn
    lds = km_stage("f32", tn, waves, ld, k0, n0)
    for wn in range(tn // 64):
        for lane in range(64):
            base = (4 * wn + ((lane >> 4) & 1)) * 1024 + 512 * (lane >> 5) + 4 * (lane & 15)
            for j in range(2):
                for q in range(8):
                    n, k = 64 * wn + 32 * j + (lane & 31), 8 * (lane >> 5) + q
                    assert lds[base + 2048 * j + 64 * q] == ("f", k0 + k, n0 + n)


@pytest.mark.parametrize("form", ["planes", "f32", "f16"])
def test_epilogue_staged_stores_address_tiled_elements(form):
    """put_row (transposed outputs, staged in LDS): lane ech of the 8 lanes of output row gr writes chunk ech of
    columns gc0 .. gc0 + 31 at (gr & ~15) 4 ld + (gr & 15) 64 + 64 gc0 +
    1024 (ech >> 2) + 16 (ech & 3) (FP16: (gr & ~15) 2 ld + (gr & 15) 64 +
    32 gc0 + 8 ech); those are the bytes tiled_index gives its elements, and
    the 8 rows of a store instruction cover two 512-byte ranges."""
    ld = 256
    mem = memory(form, 64, ld)
    for gr0 in (0, 8, 40):
        for gc0 in (0, 32, 224):
            spans = set()
            for er in range(8):
                gr = gr0 + er
                for ech in range(8):
                    if form == "f16":
                        off = (gr & ~15) * 2 * ld + (gr & 15) * 64 + 32 * gc0 + 8 * ech
                        cols = [gc0 + 4 * ech + e for e in range(4)]
                        assert [mem[off + 2 * e] for e in range(4)] == [("x", gr, c) for c in cols]
                        spans.add(off // 512)
                        continue
                    off = (gr & ~15) * 4 * ld + (gr & 15) * 64 + 64 * gc0 + ((ech >> 2) << 10) + ((ech & 3) << 4)
                    if form == "f32":
                        cols = [gc0 + 4 * ech + e for e in range(4)]
                        assert [mem[off + 4 * e] for e in range(4)] == [("f", gr, c) for c in cols]
                    else:  # chunk ech: plane (ech >> 1) & 1 of columns 16 (ech >> 2) + 8 (ech & 1) .. + 7
                        plane = "lo" if (ech >> 1) & 1 else "hi"
                        cols = [gc0 + 16 * (ech >> 2) + 8 * (ech & 1) + e for e in range(8)]
                        assert [mem[off + 2 * e] for e in range(8)] == [(plane, gr, c) for c in cols]
                    spans.add(off // 512)
            assert len(spans) == (1 if form == "f16" else 2)


def col16(e, lh, natural=False):
    """s8.hip col16: the column of register e of a lane of half lh (FP32
    mode reads its B fragments unpermuted: the natural MFMA order)."""
    return 8 * (e >> 2) + 4 * lh + (e & 3) if natural else 16 * (e >> 3) + 8 * lh + (e & 7)


def test_swapped_mfma_layout_puts_consecutive_columns_in_a_lane():
    """The MFMAs take the B fragment first, so the accumulator is
    D = Bfrag A^T: register e of lane l holds D[8 (e >> 2) + 4 (l >> 5) +
    (e & 3)][l & 31] (the 32x32 MFMA output layout), and D[p][m] =
    C[m][sw23(p)] because lane p of the B fragment holds B row sw23(p).
    So register e of lane (r, h) holds C[r][col16(e)]: 8 consecutive columns
    of each 16-column K group per lane, every column of the block once
    per row.  (FP32 mode reads B unpermuted: C[r][8 (e >> 2) + 4 h + (e & 3)].)"""
    for lane in range(64):
        r, lh = lane & 31, lane >> 5
        cols = []
        for e in range(16):
            p = 8 * (e >> 2) + 4 * lh + (e & 3)
            assert sw23(p) == col16(e, lh)
            cols.append(sw23(p))
        assert cols[:8] == list(range(8 * lh, 8 * lh + 8))
        assert cols[8:] == list(range(16 + 8 * lh, 16 + 8 * lh + 8))
    assert sorted(col16(e, h) for h in range(2) for e in range(16)) == list(range(32))
    for lane in range(64):
        r, lh = lane & 31, lane >> 5
        assert [8 * (e >> 2) + 4 * lh + (e & 3) for e in range(16)] == [col16(e, lh, True) for e in range(16)]


@pytest.mark.parametrize("form,natural", [("planes", False), ("f32", False), ("f32", True),
                                          ("f32_rowmajor", False), ("f32_rowmajor", True), ("f16", False)])
def test_epilogue_direct_stores_address_tiled_elements(form, natural):
    """put_direct: lane (r, h) stores its 16 values of row gr = R + r,
    columns cb + col16(e); every store writes 16 bytes that are exactly the
    bytes of those elements (tiled_index, planes hi/lo, FP16 32-column
    pieces, or row-major FP32), and the block's 32 x 32 elements are each
    written once."""
    ld = 256
    mem = memory(form if form != "f32_rowmajor" else "f32", 64, ld)
    if form == "f32_rowmajor":
        mem = {}
        for row in range(64):
            for c in range(ld):
                for b in range(4):
                    mem[4 * (row * ld + c) + b] = ("f", row, c)
    for R in (0, 32):
        for cb in (0, 32, 224):
            seen = {}
            for lane in range(64):
                r, lh = lane & 31, lane >> 5
                gr = R + r
                val = {e: (gr, cb + col16(e, lh, natural)) for e in range(16)}
                stores = []  # (byte offset, [elements], bytes per element, plane)
                if form == "f16":
                    base = (gr & ~15) * 2 * ld + ((gr & 15) << 6) + 32 * cb + 16 * lh
                    for g in range(2):
                        stores.append((base + 32 * g, [val[8 * g + e] for e in range(8)], 2, "x"))
                elif form == "planes":
                    base = (gr & ~15) * 4 * ld + ((gr & 15) << 6) + 64 * cb + 16 * lh
                    for g in range(2):
                        stores.append((base + 1024 * g, [val[8 * g + e] for e in range(8)], 2, "hi"))
                        stores.append((base + 1024 * g + 32, [val[8 * g + e] for e in range(8)], 2, "lo"))
                else:
                    tl = form == "f32"
                    base = ((gr & ~15) * 4 * ld + ((gr & 15) << 6) + 64 * cb) if tl else gr * 4 * ld + 4 * cb
                    for e4 in range(4):
                        c = col16(4 * e4, lh, natural)
                        off = base + (1024 * (c >> 4) + 4 * (c & 15) if tl else 4 * c)
                        stores.append((off, [val[4 * e4 + t] for t in range(4)], 4, "f"))
                for off, elems, size, plane in stores:
                    assert len(elems) * size == 16
                    for t, (row, col) in enumerate(elems):
                        assert mem[off + size * t] == (plane, row, col)
                        key = (plane, row, col)
                        assert key not in seen
                        seen[key] = True
            planes = ("hi", "lo") if form == "planes" else ("x",) if form == "f16" else ("f",)
            assert sorted(seen) == sorted((p, R + r, cb + c) for p in planes for r in range(32) for c in range(32))
