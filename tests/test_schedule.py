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

import pytest

import dflash_qmm



def make_plan(M, N, K, bits, gs, cus=256, lds=163840):
    lib = dflash_qmm.load_library()
    out = (ctypes.c_int * 10)()
    rc = lib.dfq_debug_make_plan(M, N, K, bits, gs, cus, lds, out)
    if rc:
        return None
    keys = ["T", "SS", "nkb", "Gkb", "nslot_kb", "kr", "lds_bytes", "need_ws", "ch", "umax"]
    return dict(zip(keys, list(out)))


def wg_start(c, base, rem):
    return c * base + min(c, rem)


def owner_wg(u, base, rem):
    big = rem * (base + 1)
    return u // (base + 1) if u < big else rem + (u - big) // base


def take_order(a, b, SS):
    """Units of a workgroup range in the order its waves take them (the kernel's unit_of):
    the tile shared with the next workgroup first, then the rest from a."""
    s1 = max(a, ((b - 1) // SS) * SS)
    return list(range(s1, b)) + list(range(a, s1))


def replay(p):
    T, SS, nkb, G, nslot = p["T"], p["SS"], p["nkb"], p["Gkb"], p["nslot_kb"]
    U = T * SS
    base, rem = divmod(U, G)
    umax = base + (1 if rem else 0)
    assert p["umax"] == umax
    seen = set()
    y_writes = {}
    ws_slots = {}
    arrivals = {}

    def finalize(t, units):
        assert t not in y_writes, f"tile {t} written twice"
        assert units == {(kb, t, s) for kb in range(nkb) for s in range(SS)}, f"tile {t} units"
        y_writes[t] = True

    def publish(t, kb, j, units):
        assert 0 <= j < nkb * nslot, (t, j, nslot)
        assert (t, j) not in ws_slots, f"slot {(t, j)} written twice"
        ws_slots[(t, j)] = units
        nwg = owner_wg(t * SS + SS - 1, base, rem) - owner_wg(t * SS, base, rem) + 1
        arrivals[t] = arrivals.get(t, 0) + 1
        if arrivals[t] == nkb * nwg:
            allu = set()
            for kb2 in range(nkb):
                for j2 in range(nwg):
                    allu |= ws_slots[(t, kb2 * nslot + j2)]
            finalize(t, allu)

    for kb in range(nkb):
        for cl in range(G):
            a, b = wg_start(cl, base, rem), wg_start(cl + 1, base, rem)
            order = take_order(a, b, SS)
            assert sorted(order) == list(range(a, b))
            ta, tlast = a // SS, (b - 1) // SS
            ntl = tlast - ta + 1
            assert ntl <= (umax + SS - 1) // SS + 1          # LDS counters sized for this
            part = {}
            tcnt = [0] * ntl
            for u in order:                                   # any wave, one unit at a time
                key = (kb, u // SS, u % SS)
                assert key not in seen, f"unit {key} computed twice"
                seen.add(key)
                assert 0 <= u - a < umax                      # its LDS partial slot
                part[u - a] = key
                t = u // SS
                u0, u1 = max(a, t * SS), min(b, (t + 1) * SS)
                tcnt[t - ta] += 1
                if tcnt[t - ta] == u1 - u0:                   # the arrival that completes t
                    units = {part[uu - a] for uu in range(u0, u1)}
                    if u0 == t * SS and u1 == (t + 1) * SS and nkb == 1:
                        finalize(t, units)
                    else:
                        first = owner_wg(t * SS, base, rem)
                        publish(t, kb, kb * nslot + (cl - first), units)
            assert all(c == min(b, (t + 1) * SS) - max(a, t * SS)
                       for c, t in zip(tcnt, range(ta, tlast + 1)))
    assert len(seen) == nkb * U
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
]


@pytest.mark.parametrize("shape", SHAPES)
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
                                (8, 64, 65536, 4, 128)]:
        p = make_plan(M, N, K, bits, gs)
        assert M * p["kr"] // 8 <= 12 * 512
        assert p["lds_bytes"] <= 163840
        assert K % p["kr"] == 0 and K // p["kr"] == p["nkb"]


def test_planner_rejects_unsupported_shapes():
    assert make_plan(9, 64, 512, 4, 64) is None     # more than 8 rows per launch
    assert make_plan(8, 64, 500, 4, 64) is None     # K not a multiple of the super-step
    assert make_plan(8, 64, 192, 4, 128) is None
