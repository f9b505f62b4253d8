"""The fast kernel's work split, checked on the CPU.

The runtime's planner (dfq_debug_make_plan, the same code dfq_qmm uses) is run for many
shapes; the kernel's split and fix-up rules (qmm_kernels.hip: unit ranges per workgroup and
wave, per-unit LDS partial slots, per-tile arrival counters, workspace publish with a
last-arriver sum)
are replayed here unit by unit.  Every (k-block, tile, chunk) unit must be computed
exactly once, every tile must be written exactly once with all of its units, and every
workspace / LDS slot index must stay inside what the planner sized.  The order in which a
workgroup's waves take its units does not change which arrival completes a tile's count, so
replaying the workgroup's take order covers every interleaving of its waves.
"""
import ctypes

import numpy as np
import pytest

import dflash_qmm



def make_plan(M, N, K, bits, gs, cus=256, lds=163840):
    lib = dflash_qmm.load_library()
    out = (ctypes.c_int * 15)()
    rc = lib.dfq_debug_make_plan(M, N, K, bits, gs, cus, lds, out)
    if rc:
        return None
    keys = ["T", "SS", "nkb", "Gkb", "nslot_kb", "kr", "lds_bytes", "need_ws", "ch", "umax",
            "chunks", "reduce", "ring", "aligned", "burst"]
    return dict(zip(keys, list(out)))


def wg_start(c, base, rem):
    return c * base + min(c, rem)


def owner_wg(u, base, rem):
    big = rem * (base + 1)
    return u // (base + 1) if u < big else rem + (u - big) // base


def kblock(p, kb):
    """Chunks [c0, c0 + SS) of k-block kb and its workgroup split (the kernel's kblock): base
    and rem count units, or tiles in an aligned split."""
    c0 = kb * p["chunks"] // p["nkb"]
    SS = (kb + 1) * p["chunks"] // p["nkb"] - c0
    base, rem = divmod(p["T"] * (1 if p["aligned"] else SS), p["Gkb"])
    return c0, SS, base, rem


def wg_range(p, kb, cl):
    """Units [a, b) of workgroup cl of k-block kb (the kernel's range_start)."""
    _, SS, base, rem = kblock(p, kb)
    scale = SS if p["aligned"] else 1
    return wg_start(cl, base, rem) * scale, wg_start(cl + 1, base, rem) * scale


def tile_first_owner(p, kb, t):
    _, SS, base, rem = kblock(p, kb)
    return owner_wg(t, base, rem) if p["aligned"] else owner_wg(t * SS, base, rem)


def tile_owners(p, kb, t):
    _, SS, base, rem = kblock(p, kb)
    if p["aligned"]:
        return 1
    return owner_wg(t * SS + SS - 1, base, rem) - owner_wg(t * SS, base, rem) + 1


def take_order(a, b, SS):
    """Units of a workgroup range in the order its waves take them (the kernel's unit_of):
    the tile shared with the next workgroup first, then the rest from a."""
    s1 = max(a, ((b - 1) // SS) * SS)
    return list(range(s1, b)) + list(range(a, s1))


def replay(p):
    T, nkb, G, nslot = p["T"], p["nkb"], p["Gkb"], p["nslot_kb"]
    chunks, umax, R = p["chunks"], p["umax"], p["ring"]
    # the ring of partial slots holds at least every unit one tile can have in a range
    assert R <= umax and R >= min(-(-chunks // nkb), umax), (R, umax)
    seen = set()
    y_writes = {}
    ws_slots = {}
    arrivals = {}
    parts_of = {}        # tile -> number of parts anywhere in the split

    for kb in range(nkb):
        c0, SS, base, rem = kblock(p, kb)
        assert SS in (chunks // nkb, -(-chunks // nkb)) and SS <= p["SS"]
        assert p["kr"] == p["SS"] * (p["kr"] // p["SS"])
        assert (base + (1 if rem else 0)) * (SS if p["aligned"] else 1) <= umax
        for t in range(T):
            parts_of[t] = parts_of.get(t, 0) + tile_owners(p, kb, t)
    max_parts = max(parts_of.values())
    # aligned splits (two to eight k-blocks, the kernels' exchange tree has three levels)
    # finish every tile in the kernel, by the pair exchange or a tree of them; other splits
    # with three or more parts take the second pass
    if p["aligned"]:
        assert 2 <= nkb <= 8 and max_parts == nkb and not p["reduce"], (max_parts, p)
    else:
        assert p["reduce"] == int(max_parts > 2), (max_parts, p["reduce"])

    def finalize(t, units):
        assert t not in y_writes, f"tile {t} written twice"
        assert units == {(kb, t, c) for kb in range(nkb) for c in range(kblock(p, kb)[1])}, t
        y_writes[t] = True

    def publish(t, kb, j, units):
        """pair exchange (two parts) or a reduce slot; the tile is final once all parts are in"""
        assert 0 <= j < nslot, (t, j, nslot)
        assert (t, kb, j) not in ws_slots, f"slot {(t, kb, j)} written twice"
        ws_slots[(t, kb, j)] = units
        arrivals[t] = arrivals.get(t, 0) + 1
        if arrivals[t] == parts_of[t]:
            allu = set()
            for (t2, kb2, j2), uu in ws_slots.items():
                if t2 == t:
                    allu |= uu
            finalize(t, allu)

    for kb in range(nkb):
        c0, SS, base, rem = kblock(p, kb)
        for cl in range(G):
            a, b = wg_range(p, kb, cl)
            order = take_order(a, b, SS) if b > a else []
            assert sorted(order) == list(range(a, b))
            if b <= a:
                continue
            ta, tlast = a // SS, (b - 1) // SS
            ntl = tlast - ta + 1
            assert ntl <= (umax + (chunks // nkb) - 1) // (chunks // nkb) + 1  # LDS counters
            part = {}
            tcnt = [0] * ntl
            gen = list(range(R))                              # slot generations
            g_of = {u: g for g, u in enumerate(order)}
            for g, u in enumerate(order):                     # any wave, one unit at a time
                key = (kb, u // SS, u % SS)
                assert key not in seen, f"unit {key} computed twice"
                seen.add(key)
                assert 0 <= u - a < umax
                assert gen[g % R] == g, (kb, cl, g)           # its ring slot is released
                part[g % R] = key
                t = u // SS
                u0, u1 = max(a, t * SS), min(b, (t + 1) * SS)
                tcnt[t - ta] += 1
                if tcnt[t - ta] == u1 - u0:                   # the arrival that completes t
                    g0 = g_of[u0]
                    assert [g_of[uu] for uu in range(u0, u1)] == list(range(g0, g0 + u1 - u0))
                    units = {part[(g0 + i) % R] for i in range(u1 - u0)}
                    for i in range(u1 - u0):                  # the summing wave releases every
                        gen[(g0 + i) % R] = g0 + i + R        # slot (the sum is in the output area)
                    if u0 == t * SS and u1 == (t + 1) * SS and nkb == 1:
                        finalize(t, units)
                    else:
                        publish(t, kb, cl - tile_first_owner(p, kb, t), units)
            assert all(c == min(b, (t + 1) * SS) - max(a, t * SS)
                       for c, t in zip(tcnt, range(ta, tlast + 1)))
    assert len(seen) == sum(T * kblock(p, kb)[1] for kb in range(nkb))
    assert sorted(y_writes) == list(range(T))
    need_ws = nkb > 1 or nslot > 1
    assert p["need_ws"] == int(need_ws)
    if not need_ws:
        assert not ws_slots


SHAPES = [
    (8, 17408, 5120, 4, 64), (1, 17408, 5120, 4, 64), (8, 5120, 17408, 4, 64),
    (8, 7168, 5120, 8, 64), (8, 5120, 5120, 8, 64), (8, 7168, 5120, 4, 32),
    (1, 4096, 4096, 4, 64), (8, 1024, 5120, 4, 64), (8, 16, 128, 4, 64), (3, 40, 256, 4, 64),
    (8, 257, 640, 4, 64), (8, 48, 16384, 4, 64), (4, 5000, 12288, 4, 64), (8, 17, 8192, 8, 64),
    (8, 333, 768, 4, 128), (8, 130, 1024, 8, 128), (8, 200, 512, 8, 32), (2, 3, 2560, 4, 64),
    (8, 100000, 256, 4, 64), (5, 999, 3072, 8, 64),
    (8, 512, 5120, 4, 64), (8, 2048, 5120, 4, 64), (8, 1024, 16384, 4, 64), (8, 64, 1536, 4, 64),
    # two row tiles (9..16 rows)
    (16, 17408, 5120, 4, 64), (9, 17408, 5120, 4, 64), (16, 5120, 17408, 4, 64),
    (16, 7168, 5120, 8, 64), (12, 1024, 5120, 4, 32), (16, 48, 16384, 4, 128),
    (16, 257, 1024, 8, 128), (10, 16, 512, 4, 64),
]


def _unpack_test_shapes():
    """The one-hot unpack test's shapes (every format, c8 / mt16 / c1, narrow and reduce)."""
    out = []
    for bits in (4, 8):
        for gs in (32, 64, 128):
            kss = (512 // bits) * ((2 if gs == 128 else 1) if bits == 4 else gs // 32)
            ck = (16 if (bits, gs) == (4, 32) else 8) * gs   # the c8 kernels' chunk
            k1 = 3 * kss + (kss if (3 * kss) % ck == 0 else 0)
            out += [(8, 40, 2 * ck, bits, gs), (16, 48, ck, bits, gs), (7, 24, k1, bits, gs)]
    out += [(M, 64, 64 * gs, bits, gs) for (bits, gs, M) in
            ((4, 64, 8), (8, 32, 8), (4, 64, 12), (8, 128, 5))]
    out += [(8, 48, 256 * 64, 4, 64), (16, 48, 256 * 64, 8, 64)]
    out += [(16, 256, 5120, 4, 64), (12, 256, 5120, 8, 64)]
    return out


# two k-blocks of whole tiles per workgroup (the aligned split)
ALIGNED_SHAPES = [(16, 1024, 5120, 4, 32), (10, 3000, 5120, 4, 128), (14, 3333, 4608, 4, 64),
                  (16, 4000, 5120, 8, 32), (16, 2000, 4096, 4, 64), (16, 40, 5120, 4, 64),
                  (16, 1024, 5120, 4, 64)]


# the C5 projections and LM head at 8 and 16 rows, the one-hot unpack shapes, and the
# no-allocation entry point's sequence
EXTRA_SHAPES = ([(m, n, k, 4, 64) for m in (8, 16) for (n, k) in
                 ((5120, 5120), (7168, 5120), (1024, 5120), (5120, 17408), (151936, 5120),
                  (34816, 5120))]
                + _unpack_test_shapes()
                + [(16, 4096, 5120, 8, 64), (6, 1024, 5120, 4, 128), (3, 40, 256, 4, 32)]
                + [(8, 1024, 17408, 4, 64), (8, 1000, 16384, 4, 64), (6, 5120, 17408, 8, 64),
                   (16, 3000, 7680, 4, 64), (13, 777, 9216, 4, 128)]
                + ALIGNED_SHAPES)


@pytest.mark.parametrize("shape", ALIGNED_SHAPES)
def test_aligned_shapes_take_the_aligned_split(shape):
    p = make_plan(*shape)
    assert p["aligned"] == 1 and p["nkb"] == 2 and p["reduce"] == 0 and p["nslot_kb"] == 1, p
    assert -(-p["T"] // p["Gkb"]) <= 12, p


def test_the_aligned_split_stops_at_twelve_tiles_per_workgroup():
    """Up to twelve tiles per workgroup the aligned split measured faster than the second
    pass (the 16-row headline shape has nine), and at 9..16 rows over two k-blocks up to
    twenty-four (twenty at N = 40000); from thirty on, the second pass.  A split whose
    output blocks would not fit in LDS keeps the second pass too."""
    p = make_plan(16, 17408, 5120, 4, 64)
    assert p["aligned"] == 1 and p["reduce"] == 0 and p["nkb"] == 2, p
    assert -(-p["T"] // p["Gkb"]) == 9, p
    for shape in [(16, 40000, 4096, 4, 64), (16, 40000, 4096, 4, 32), (16, 40000, 4096, 8, 64)]:
        p = make_plan(*shape)
        assert p["aligned"] == 1 and p["reduce"] == 0 and p["nkb"] == 2, (shape, p)
        assert -(-p["T"] // p["Gkb"]) == 20, (shape, p)
    for shape in [(16, 60000, 4096, 4, 64), (13, 80000, 4096, 4, 32), (16, 151936, 5120, 4, 64)]:
        p = make_plan(*shape)
        assert p["aligned"] == 0 and p["reduce"] == 1 and p["nkb"] == 2, (shape, p)


def test_up_to_twelve_rows_take_one_k_block_where_it_pays():
    """9..12 rows at K = 5120 stage one k-block of x (up to 16 items a staging thread) with a
    ring shrunk to fit, where each range holds at least three tiles and one round of
    workgroups covers the split; elsewhere two k-blocks stay."""
    for M in (9, 10, 11, 12):
        for N in (17408, 34816):
            p = make_plan(M, N, 5120, 4, 64)
            assert (p["nkb"], p["Gkb"], p["reduce"]) == (1, 256, 0), (M, N, p)
            assert p["ring"] >= p["SS"] and p["lds_bytes"] <= 163840, (M, N, p)
    for shape in [(12, 7168, 5120, 4, 64),     # under two tiles a range
                  (16, 40000, 4096, 4, 64),    # would need two rounds of workgroups
                  (13, 17408, 5120, 4, 64)]:   # over 16 items a staging thread
        assert make_plan(*shape)["nkb"] == 2, shape


def test_more_workgroups_than_cus_come_in_whole_rounds():
    """A split that does not fit one workgroup per CU takes 2, 3, ... times as many, so that
    no round of workgroups runs with a few of them alone."""
    for shape in [(9, 151936, 5120, 4, 64), (16, 151936, 5120, 4, 64),
                  (16, 151936, 5120, 4, 128), (10, 151936, 5120, 4, 128)]:
        p = make_plan(*shape)
        g0 = 256 // p["nkb"]
        assert p["Gkb"] % g0 == 0, (shape, p)
    for cus in (80, 304):
        p = make_plan(16, 151936, 5120, 4, 64, cus=cus)
        assert p["Gkb"] % (cus // p["nkb"]) == 0, (cus, p)
        replay(p)


@pytest.mark.parametrize("shape", SHAPES + EXTRA_SHAPES)
def test_split_covers_every_unit_once(shape):
    p = make_plan(*shape)
    assert p is not None, shape
    replay(p)


@pytest.mark.parametrize("cus", [1, 7, 80, 256, 304])
def test_split_for_other_cu_counts(cus):
    for shape in [(8, 17408, 5120, 4, 64), (8, 48, 16384, 4, 64), (1, 300, 1024, 8, 32)]:
        replay(make_plan(*shape, cus=cus))


def test_planner_respects_lds_and_staging_limits():
    for (M, N, K, bits, gs) in [(8, 5120, 17408, 4, 64), (1, 5120, 17408, 4, 64),
                                (8, 64, 65536, 4, 128), (16, 5120, 17408, 4, 64),
                                (16, 17408, 5120, 8, 32), (12, 17408, 5120, 4, 64),
                                (10, 151936, 5120, 4, 64)]:
        p = make_plan(M, N, K, bits, gs)
        items = 16 if (M > 8 and p["nkb"] == 1) else 12  # x items a staging thread holds
        assert M * p["kr"] // 8 <= 8 * items * 64
        assert p["lds_bytes"] <= 163840
        assert p["SS"] == -(-p["chunks"] // p["nkb"]) and p["kr"] * p["chunks"] == K * p["SS"]


def test_long_k_uses_few_uneven_k_blocks():
    # K = 17408 at M = 8: 34 chunks of 512 k; three k-blocks of 11-12 chunks fit LDS
    p = make_plan(8, 5120, 17408, 4, 64)
    assert p["nkb"] == 3 and p["chunks"] == 34 and p["SS"] == 12


def test_three_k_blocks_take_whole_tiles_up_to_twelve_a_workgroup():
    """Three k-blocks of whole tiles per workgroup finish every tile with a chain of two pair
    exchanges, no second pass: the down projection (four tiles a workgroup), narrow N, and
    9..16 rows from K = 7680.
    From thirteen tiles a workgroup on the stream-K split with the second pass stays."""
    for shape, tiles in [((8, 5120, 17408, 4, 64), 4), ((8, 1024, 17408, 4, 64), 1),
                         ((8, 1000, 16384, 4, 64), 1), ((6, 5120, 17408, 8, 64), 4),
                         ((16, 3000, 7680, 4, 64), 3), ((12, 1024, 9216, 4, 64), 1)]:
        p = make_plan(*shape)
        assert (p["nkb"], p["aligned"], p["reduce"], p["nslot_kb"]) == (3, 1, 0, 1), (shape, p)
        assert -(-p["T"] // p["Gkb"]) == tiles and 3 * p["Gkb"] <= 256, (shape, p)
        assert p["lds_bytes"] <= 163840
    p = make_plan(8, 17408, 17408, 4, 64)
    assert (p["nkb"], p["aligned"], p["reduce"]) == (3, 0, 1), p


def test_narrow_n_splits_k_in_two_with_one_tile_per_workgroup():
    # N = 1024 at K = 5120: 64 tiles over 256 workgroups would spread each tile over four
    # (a reduce split); two k-blocks of one tile per workgroup pair every tile instead
    p = make_plan(8, 1024, 5120, 4, 64)
    assert (p["nkb"], p["Gkb"], p["nslot_kb"], p["reduce"]) == (2, 64, 1, 0)
    # wide enough N keeps one k-block over every CU
    assert make_plan(8, 2048, 5120, 4, 64)["nkb"] == 1
    # long K: a workgroup's share of two k-blocks would be too long; six k-blocks of whole
    # tiles (at most two a workgroup, 40 workgroups each) sum each tile over a tree of exchanges
    p = make_plan(8, 1024, 32768, 4, 64)
    assert (p["nkb"], p["Gkb"], p["aligned"], p["reduce"]) == (6, 40, 1, 0), p


def test_tree_splits_only_where_they_measured_faster():
    # 16 rows at N = 5120, K = 17408: with its ring shrunk the second pass's split fits one
    # round of 6 x 42 workgroups, which measured faster than eight k-blocks of ten tiles
    p = make_plan(16, 5120, 17408, 4, 64)
    assert (p["nkb"], p["Gkb"], p["aligned"], p["reduce"]) == (6, 42, 0, 1), p
    # many tiles a workgroup (56 and 68 here) keep the second pass's split
    for shape in [(16, 28672, 16384, 4, 128), (11, 34816, 16384, 4, 128)]:
        p = make_plan(*shape)
        assert p["reduce"] == 1 and p["aligned"] == 0, (shape, p)
    # 9..15 rows there: the tree of as many k-blocks as the second pass's split, at most 8
    # tiles a workgroup (12 rows: five k-blocks of 48 workgroups, seven tiles each)
    for m, nkb in [(9, 4), (10, 4), (12, 5), (13, 6), (15, 6)]:
        p = make_plan(m, 5120, 17408, 4, 64)
        assert (p["nkb"], p["aligned"], p["reduce"]) == (nkb, 1, 0), (m, p)
        assert -(-320 // p["Gkb"]) <= 8 and p["Gkb"] % 8 == 0, (m, p)
    # ... but not where the tree needs more k-blocks than the second pass's split (4-bit g32
    # at 10 rows: six against four), nor at 8 rows (eight tiles a workgroup at K = 32768)
    assert make_plan(10, 5120, 17408, 4, 32)["reduce"] == 1
    assert make_plan(8, 5120, 32768, 4, 64)["reduce"] == 1
    # other CU counts (another partition of the chip) never take a tree of four or more
    for cus in (32, 64, 128, 304):
        p = make_plan(16, 5120, 17408, 4, 64, cus=cus)
        assert not (p["aligned"] and p["nkb"] >= 4), (cus, p)


def test_outputs_leave_at_the_end_where_workgroups_hold_many_tiles():
    # the LM head (38 tiles a workgroup) and the C5 gate|up (10): outputs written at the end
    # of each workgroup; the headline shape (6) and C3 (4 per k-block): as each tile finishes
    assert make_plan(8, 151936, 5120, 4, 64)["burst"] == 1
    assert make_plan(8, 34816, 5120, 4, 64)["burst"] == 1
    assert make_plan(1, 32768, 512, 4, 64)["burst"] == 1
    assert make_plan(8, 17408, 5120, 4, 64)["burst"] == 0
    assert make_plan(8, 7168, 5120, 4, 64)["burst"] == 0
    p = make_plan(8, 5120, 17408, 4, 64)
    assert p["aligned"] == 1 and p["burst"] == 0
    # reduce splits holding many tiles per workgroup leave their parts at the end too
    for shape in [(16, 60000, 4096, 4, 64), (12, 60000, 6144, 4, 64), (16, 151936, 5120, 4, 64)]:
        p = make_plan(*shape)
        assert p["reduce"] == 1 and p["burst"] == 1, shape
    # aligned and narrow splits pair every tile: nothing left for the end
    assert make_plan(8, 1024, 5120, 4, 64)["burst"] == 0


def test_sixteen_rows_fit_lds_with_two_row_tiles():
    # x sums (8*mt floats per group) and partial tiles (512*mt bytes) double with mt = 2;
    # K = 5120 at 16 rows stages 16 x 2560 per k-block
    p = make_plan(16, 17408, 5120, 4, 64)
    assert p["nkb"] == 2 and p["kr"] == 2560 and p["lds_bytes"] <= 163840
    rs = 2 * p["kr"] + 16
    xsum_off = (17 * rs + 15) & ~15
    need = xsum_off + (p["kr"] // 64) * 64 + p["ring"] * 1028
    assert need <= p["lds_bytes"]


def test_planner_rejects_unsupported_shapes():
    assert make_plan(17, 64, 512, 4, 64) is None    # more than 16 rows per launch
    assert make_plan(9, 64, 384, 4, 64) is None     # 9..16 rows need 8-group chunks
    assert make_plan(8, 64, 500, 4, 64) is None     # K not a multiple of the super-step
    assert make_plan(8, 64, 192, 4, 128) is None


WAVES = 12          # streaming waves per workgroup (DFQ_WAVES)
PF_LOADS = 4        # 16-byte weight loads in flight per lane (DFQ_PF_LOADS)


def fmt_consts(bits, gs, ch):
    """Per-format constants of the kernel (Cfg): steps per super-step, k per super-step,
    groups per super-step, and the prefetch depth for chunks of ch super-steps."""
    kstep = 512 // bits
    ns = (2 if gs == 128 else 1) if bits == 4 else gs // 32
    kss = kstep * ns
    gps = kss // gs
    pf = max(1, min(8, PF_LOADS // (ch * ns)))
    return ns, kss, gps, pf


def fetched_units(a, b, SS, U, wave, pf):
    """Every unit a wave may load (the kernel's issue): its initial take indices (the unused
    fetch of a wave with none goes to the range's first unit, clamped to the k-block's last),
    and any unit of the range a later take can return."""
    L = b - a
    s1 = max(a, ((b - 1) // SS) * SS) if L > 0 else a
    nrot = b - s1

    def unit_of(g):
        return s1 + g if g < nrot else a + (g - nrot)

    lu = min(a, U - 1)
    out = []
    for i in range(pf):
        g = wave * pf + i
        u = unit_of(g) if g < L else lu
        lu = u
        out.append(u)
    return out + [unit_of(g) for g in range(L)]


@pytest.mark.parametrize("shape", SHAPES + EXTRA_SHAPES)
def test_prefetch_addresses_stay_in_bounds(shape):
    M, N, K, bits, gs = shape
    p = make_plan(*shape)
    ns, kss, gps, pf = fmt_consts(bits, gs, p["ch"])
    ch = p["ch"]
    kch = kss * ch
    RB = K * bits // 8                      # bytes per weight row
    GPR = K // gs                           # groups per row
    T, G = p["T"], p["Gkb"]
    sv = 16 if ch > 1 else 4                # bytes of one scale/bias load per lane
    for kb in range(p["nkb"]):
        c0, SS, base, rem = kblock(p, kb)
        U = T * SS
        kr = SS * kch
        k0 = c0 * kch
        assert k0 + kr <= K and M * (kr // 8) <= WAVES * 64 * (96 // WAVES)
        for cl in range(G):
            a, b = wg_range(p, kb, cl)
            units = set()
            for wave in range(WAVES):
                units.update(fetched_units(a, b, SS, U, wave, pf))
            for u in units:
                assert 0 <= u < U, (kb, cl, u, U)
                t, c = divmod(u, SS)
                row0 = t * 16
                rmax = 15 if row0 + 16 <= N else N - 1 - row0     # the kernel's row clamp
                assert 0 <= rmax <= 15
                kc = k0 + c * kch
                last_w = (row0 + rmax) * RB + kc * bits // 8 + 3 * 16 + (ch * ns - 1) * 64 + 16
                assert last_w <= N * RB, (kb, cl, u)
                lane_s = 0 if ch > 1 else (4 if gps == 4 else 0)
                last_s = ((row0 + rmax) * GPR + kc // gs) * 2 + lane_s + sv
                assert last_s <= N * GPR * 2, (kb, cl, u)




QMV_WAVES, QMV_ROWS = 8, 4   # the stock-path GEMV's waves per workgroup and rows per group


@pytest.mark.parametrize("shape", [(17408, 5120, 4), (4096, 4096, 4), (151936, 5120, 4),
                                   (5120, 17408, 4), (1, 256, 4), (3, 2048, 4), (37, 2560, 4),
                                   (1000, 5120, 8), (257, 768, 8), (5120, 5120, 8),
                                   (130, 2560, 4), (40, 640, 8), (100000, 256, 4)])
def test_stock_gemv_split_writes_every_row_once(shape):
    """The stock-path GEMV's split (qmv_layout and the kernel): workgroup b owns rows
    [b*base + min(b, rem), ...); groups of 4 of its rows go to its waves (the first
    QMV_WAVES by index, the rest from a counter starting there), so every group is taken
    once whatever the order; loads stay in bounds (rows clamped to the workgroup's last, the
    chunk to the row's last)."""
    N, K, bits = shape
    kpl = 128 // bits
    nchunk = K // kpl
    nsteps = -(-nchunk // 64)
    G = max(1, min(256, -(-N // (QMV_ROWS * QMV_WAVES))))
    base, rem = divmod(N, G)
    written = []
    for b in range(G):
        lo, nrows = b * base + min(b, rem), base + (1 if b < rem else 0)
        ngroups = -(-nrows // QMV_ROWS)
        takes = list(range(min(QMV_WAVES, ngroups))) + list(range(QMV_WAVES, ngroups))
        assert sorted(takes) == list(range(ngroups))
        for g in takes:
            for r in range(QMV_ROWS):
                row = lo + min(g * QMV_ROWS + r, nrows - 1)
                assert lo <= row < lo + nrows <= N
                if g * QMV_ROWS + r < nrows:
                    written.append(lo + g * QMV_ROWS + r)
            for j in range(nsteps + 1):          # the clamped reload past the last step
                for lane in (0, 63):
                    c = min(lane + 64 * min(j, nsteps - 1), nchunk - 1)
                    assert 0 <= c < nchunk and (c * kpl) // 32 < K // 32
    assert sorted(written) == list(range(N))


def _tree_sets(kb, nparts):
    """The word sets part kb exchanges at, level by level, as the kernel's publish walks its
    tree: at level L the node holding kb meets its sibling at set r - 1, r = the right
    child's first k-block, when that child exists."""
    out, L = [], 1
    while (1 << (L - 1)) < nparts:
        r = ((kb >> L) * 2 + 1) << (L - 1)
        if r < nparts:
            out.append(r)
        L += 1
    return out


@pytest.mark.parametrize("nparts", range(2, 9))
def test_exchange_tree_has_one_writer_and_a_fixed_order(nparts):
    """Every arrival order of the parts at the tree's exchanges (first arrival deposits, the
    second adds and carries on) ends with exactly one writer holding the same fp32 sum, the
    tree's own order: (P0 + P1) + P2 for three parts."""
    import random

    def tree_sum(v, lo, hi):
        if hi - lo == 1:
            return np.float32(v[lo])
        h = 1
        while 2 * h < hi - lo:
            h *= 2
        return np.float32(tree_sum(v, lo, lo + h) + tree_sum(v, lo + h, hi))

    sets_used = sorted({r for kb in range(nparts) for r in _tree_sets(kb, nparts)})
    assert sets_used == list(range(1, nparts))          # nparts - 1 sets, all distinct
    rng = random.Random(nparts)
    for trial in range(200):
        v = np.random.default_rng(trial).normal(size=nparts).astype(np.float32) * 1000
        words, writers = {}, []

        def party(kb):
            w, go = np.float32(v[kb]), True
            for r in _tree_sets(kb, nparts):
                if not go:
                    break
                yield
                old = words.get(r)
                if old is None:
                    words[r], go = w, False
                else:
                    w, words[r] = np.float32(w + old), None
            if go:
                writers.append(w)

        live = {kb: party(kb) for kb in range(nparts)}
        while live:
            kb = rng.choice(sorted(live))
            try:
                next(live[kb])
            except StopIteration:
                del live[kb]
        assert len(writers) == 1
        assert writers[0] == tree_sum(v, 0, nparts)
