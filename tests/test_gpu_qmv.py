"""The stock path's few-row GEMV (dfq_qmm_fallback for one dtype, 4/8-bit, group 32/64/128).

MLX's stock op, which the drop-in layer falls through to (SmallMQuantizedMatmul.swift:265),
runs a GEMV for few rows.  The library's stand-in does the same: one launch per 4 rows, each
weight row read once a launch.  Pinned three ways:

* bit-exact one-hot rows: with x[m] = e_k, power-of-two scales and small integer biases, y is a
  column of the dequantised matrix and the GEMV's factored form is exact, so y must equal the
  oracle's dequant bit for bit, at every k position of several lane chunks, in every format;
* against the fp64 oracle at 1..8 rows (5..8 rows take two launches), ragged N, K whose last
  step covers part of the lanes, a linear bias, and the benchmark shapes at full size;
* the path taken: the GEMV, not the per-element kernel, for these shapes.
"""
import numpy as np
import pytest

from gpu_util import announce, download, to_dev16, upload
from onehot import exact_case
from oracle.qmm_oracle import BF16, F16, config_case, from_bits, make_case, to_bits, \
    tolerance_check

pytestmark = pytest.mark.gpu

TOL = 1e-2
FORMATS = [(bits, gs, dt) for bits in (4, 8) for gs in (32, 64, 128) for dt in (BF16, F16)]


@pytest.mark.parametrize("bits,gs,dt", FORMATS)
def test_one_hot_rows_are_exact(ctx, bits, gs, dt):
    import torch
    kpl = 128 // bits                # k of one lane chunk
    K = 80 * kpl                     # 80 chunks: one full step of 64 lanes, one of 16
    N = 37
    w, sb, bb, deq = exact_case(N, K, bits, gs, dt, seed=bits * 1000 + gs + dt)
    rng = np.random.default_rng(5)
    pos = np.concatenate([np.arange(0, 3 * kpl), rng.integers(0, K, size=21), [K - 1]])
    tdt = torch.bfloat16 if dt == BF16 else torch.float16
    wd = torch.from_numpy(w.view(np.int32)).cuda()
    sd, bd = to_dev16(sb, dt), to_dev16(bb, dt)
    for M in (1, 4, 7):
        assert ctx.stock_gemv_launches(M, N, K, bits, gs, dt) == (M + 3) // 4
        P = pos[: len(pos) - len(pos) % M]
        x = torch.zeros(len(P), K, dtype=tdt, device="cuda")
        x[torch.arange(len(P), device="cuda"), torch.from_numpy(P).cuda()] = 1.0
        y = torch.empty(len(P), N, dtype=tdt, device="cuda")
        announce(f"stock gemv one-hot bits={bits} gs={gs} dt={dt} M={M} calls={len(P) // M}")
        for c in range(len(P) // M):
            ctx.fallback(x[c * M:(c + 1) * M], wd, sd, bd, bits, gs, out=y[c * M:(c + 1) * M])
        torch.cuda.synchronize()
        got = y.view(torch.int16).cpu().numpy().view(np.uint16)
        want = to_bits(deq[:, P].T, dt)
        bad = np.argwhere(got != want)
        assert bad.size == 0, (M, len(bad), from_bits(got[tuple(bad[0])], dt),
                               deq[bad[0][1], P[bad[0][0]]])


CASES = [  # (M, N, K, bits, gs, dtype)
    (1, 1, 256, 4, 64, BF16), (1, 3, 2048, 4, 32, BF16), (2, 17, 2560, 4, 128, F16),
    (3, 1000, 5120, 4, 64, BF16), (4, 257, 768, 8, 32, BF16), (4, 96, 1536, 8, 64, F16),
    (5, 333, 1024, 8, 128, BF16), (6, 200, 4096, 4, 64, F16), (7, 40, 640, 8, 64, BF16),
    (8, 4096, 1024, 4, 64, BF16), (8, 130, 2560, 4, 32, F16),
]


@pytest.mark.parametrize("case", CASES)
def test_stock_gemv_matches_oracle(ctx, oracle, case):
    M, N, K, bits, gs, dt = case
    c = make_case(M, N, K, bits=bits, gs=gs, xdt=dt, seed=M * 7 + N + K, lbias=True)
    x, w, s, b, lb = upload(c)
    assert ctx.stock_gemv_launches(M, N, K, bits, gs, dt) == (M + 3) // 4
    announce(f"stock gemv M={M} N={N} K={K} bits={bits} gs={gs} dt={dt}")
    y = download(ctx.fallback(x, w, s, b, bits, gs, lbias=lb))
    rel, ok = tolerance_check(y, oracle.qmm_f64(c))
    assert rel <= TOL and ok, (case, rel)


@pytest.mark.parametrize("name,M", [("c1_m1_k4096_n4096_f16", 1),
                                    ("c2_gateup_k5120_n17408", 1),
                                    ("c2_gateup_k5120_n17408", 4)])
def test_stock_gemv_at_benchmark_shapes(ctx, oracle, name, M):
    c = config_case(name, M)
    x, w, s, b, _ = upload(c)
    assert ctx.stock_gemv_launches(M, c.N, c.K, c.bits, c.gs, c.xdt) == 1
    announce(f"stock gemv {name} M={M}")
    y = download(ctx.fallback(x, w, s, b, c.bits, c.gs))
    rel, ok = tolerance_check(y, oracle.qmm_f64(c))
    assert rel <= TOL and ok, (name, M, rel)


def test_stock_gemv_is_deterministic_and_row_independent(ctx):
    """Each output of the GEMV depends on its own row of x only, with a fixed summation
    order (the split of a launch's work depends on N and K, not on M, and the two waves that
    share a row add their sums on a zero slot): rows 0-2 of a 4-row call equal a 3-row call
    on those rows bit for bit, rows 4-6 of a 7-row call (its second launch) equal them too, and
    repeats are identical at one and at four rows."""
    import torch
    c = make_case(4, 1500, 3072, bits=4, gs=64, seed=77)
    x, w, s, b, _ = upload(c)
    announce("stock gemv row independence")
    y4 = ctx.fallback(x, w, s, b, 4, 64)
    again = ctx.fallback(x, w, s, b, 4, 64)
    y3 = ctx.fallback(x[:3].contiguous(), w, s, b, 4, 64)
    x7 = torch.cat([x, x[:3]]).contiguous()
    y7 = ctx.fallback(x7, w, s, b, 4, 64)
    one = [ctx.fallback(x[:1].contiguous(), w, s, b, 4, 64) for _ in range(2)]
    torch.cuda.synchronize()
    eq = lambda a, b: torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert eq(y4, again) and eq(one[0], one[1])
    assert eq(y4[:3], y3) and eq(y7[:4], y4) and eq(y7[4:], y3)


def test_mixed_dtypes_and_two_bit_codes_take_the_per_element_path(ctx):
    assert ctx.stock_gemv_launches(4, 64, 256, 2, 64, BF16) == 0
    assert ctx.stock_gemv_launches(4, 64, 256, 4, 16, BF16) == 0
    assert ctx.stock_gemv_launches(4, 64, 200, 4, 40, BF16) == 0
