"""Parity of the gfx950 fast kernel (through the C ABI) with the CPU oracle.

Bar: max|y - y_ref| / max|y_ref| <= 1e-2 against the oracle's fp64 result on identical
seeded inputs (bf16/fp16 output, fp32 accumulation), plus the reference test's own rule
max|d| <= 0.02 * max(max|ref|, 1) (SmallMQuantizedMatmulTests.swift:74-79).  Integer and
index behaviour (row independence, determinism, workspace re-arming) is checked bit-exact.
"""
import numpy as np
import pytest

from gpu_util import announce, download, upload
from oracle.qmm_oracle import BF16, F16, config_case, make_case, tolerance_check

pytestmark = pytest.mark.gpu

TOL = 1e-2

# (M, N, K, bits, gs, dtype): every format, ragged N, single-super-step K, k-block splits.
SMALL_CASES = [
    (1, 16, 128, 4, 64, BF16),
    (8, 16, 128, 4, 64, BF16),
    (3, 40, 256, 4, 64, BF16),
    (8, 257, 640, 4, 64, BF16),
    (5, 1000, 1024, 4, 64, BF16),
    (8, 4096, 1024, 4, 64, BF16),
    (7, 300, 512, 4, 32, BF16),
    (8, 333, 768, 4, 128, BF16),
    (8, 200, 512, 8, 32, BF16),
    (6, 200, 512, 8, 64, BF16),
    (8, 130, 1024, 8, 128, BF16),
    (2, 64, 256, 4, 64, F16),
    (8, 96, 512, 4, 32, F16),
    (4, 96, 512, 4, 128, F16),
    (8, 96, 512, 8, 32, F16),
    (8, 96, 512, 8, 64, F16),
    (8, 96, 512, 8, 128, F16),
    (8, 48, 16384, 4, 64, BF16),     # several k-blocks and workgroups per tile
    (1, 5000, 12288, 4, 64, BF16),   # k-blocks with many tiles
    (8, 17, 8192, 8, 64, BF16),
]

# 9..16 rows: two row tiles per weight tile in one launch (every format), and the two-launch
# path for K that is not a multiple of 8 groups (the last case).
SIXTEEN_ROW_CASES = [
    (9, 16, 512, 4, 64, BF16),
    (16, 257, 1024, 4, 64, BF16),
    (12, 300, 512, 4, 32, BF16),
    (16, 333, 1024, 4, 128, BF16),
    (16, 200, 512, 8, 32, F16),
    (13, 130, 1024, 8, 64, BF16),
    (16, 130, 1024, 8, 128, F16),
    (11, 96, 1024, 4, 64, F16),
    (16, 48, 16384, 4, 64, BF16),    # several k-blocks and workgroups per tile
    (15, 5000, 12288, 4, 64, BF16),
    (10, 100, 384, 4, 64, BF16),     # one-super-step chunks: two launches of up to 8 rows
]


# Narrow N: two k-blocks of one tile per workgroup, every tile finished by the pair exchange
# (the planner's split for few tiles); every format, 1..16 rows, ragged N.
NARROW_CASES = [
    (8, 1024, 5120, 4, 64, BF16),
    (1, 1024, 5120, 4, 64, BF16),
    (8, 512, 5120, 4, 64, F16),
    (6, 64, 1536, 4, 64, BF16),
    (8, 1024, 5120, 8, 64, BF16),
    (8, 1024, 5120, 4, 32, BF16),
    (8, 1024, 5120, 4, 128, F16),
    (9, 1024, 5120, 4, 64, BF16),
    (16, 512, 2048, 8, 64, BF16),
    (3, 200, 3072, 4, 64, BF16),
    (8, 1000, 6144, 8, 128, BF16),
]


# Two k-blocks whose workgroups take whole tiles (the aligned split: every tile has exactly one
# part per k-block, finished by the pair exchange, no second pass), which the planner takes for
# 9..16 rows at long K where each workgroup holds at most two tiles: ragged N, one and two
# tiles per workgroup, a k-block pair of unequal length (K = 9 chunks), fewer tiles than
# workgroups.
ALIGNED_CASES = [
    (16, 1024, 5120, 4, 32, F16),
    (10, 3000, 5120, 4, 128, BF16),
    (14, 3333, 4608, 4, 64, BF16),
    (16, 4000, 5120, 8, 32, BF16),
    (16, 2000, 4096, 4, 64, BF16),
    (16, 40, 5120, 4, 64, F16),
    # twenty tiles a workgroup (two k-blocks at 9..16 rows take up to 24)
    (16, 40000, 4096, 4, 64, BF16),
    (16, 40000, 4096, 4, 32, F16),
    (12, 40000, 6144, 8, 64, BF16),
]


def run_fast(ctx, c):
    x, w, s, b, lb = upload(c)
    return ctx.qmm(x, w, s, b, c.bits, c.gs, lbias=lb)


@pytest.mark.parametrize("M,N,K,bits,gs,dt", SMALL_CASES)
def test_small_shapes_match_oracle(ctx, oracle, M, N, K, bits, gs, dt):
    c = make_case(M, N, K, bits=bits, gs=gs, xdt=dt, seed=M * 1000 + N + K + bits + gs,
                  lbias=(N % 2 == 1))
    announce(f"small M={M} N={N} K={K} bits={bits} gs={gs} dt={dt}")
    y = download(run_fast(ctx, c))
    ref = oracle.qmm_f64(c)
    rel, ok = tolerance_check(y, ref)
    assert rel <= TOL and ok, f"max rel err {rel:.3e}"


@pytest.mark.parametrize("M,N,K,bits,gs,dt", NARROW_CASES)
def test_narrow_n_split_matches_oracle_and_repeats(ctx, oracle, M, N, K, bits, gs, dt):
    import torch
    p = ctx.plan(M, N, K, bits, gs)
    assert p["nkb"] == 2 and p["reduce"] == 0 and p["nslot_kb"] == 1, p
    c = make_case(M, N, K, bits=bits, gs=gs, xdt=dt, seed=7 * M + N + K + bits + gs,
                  lbias=(N % 2 == 0))
    announce(f"narrow M={M} N={N} K={K} bits={bits} gs={gs} dt={dt}")
    x, w, s, b, lb = upload(c)
    y = ctx.qmm(x, w, s, b, c.bits, c.gs, lbias=lb)
    torch.cuda.synchronize()
    rel, ok = tolerance_check(download(y), oracle.qmm_f64(c))
    assert rel <= TOL and ok, f"max rel err {rel:.3e}"
    for _ in range(3):                       # the pair exchange leaves the workspace re-armed
        y2 = ctx.qmm(x, w, s, b, c.bits, c.gs, lbias=lb)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), y2.view(torch.int16))


# Three k-blocks of whole tiles (1..8 rows at K of 15360..17408, 9..16 rows from K = 7680): every tile has three parts,
# summed by a chain of two pair exchanges, no second pass.  Ragged N, one and four tiles per
# workgroup, 8-bit fp16, group 32, and group 128 with five chunks a k-block.
THREE_BLOCK_CASES = [
    (8, 1000, 16384, 4, 64, BF16),
    (6, 5000, 17408, 8, 64, F16),
    (7, 777, 16896, 4, 32, BF16),
    (8, 3000, 15360, 4, 128, F16),
    (12, 1024, 9216, 4, 64, BF16),           # two row tiles: 9..16 rows
    (16, 3000, 7680, 4, 64, F16),
    (13, 777, 9216, 4, 128, BF16),
]


# Four to eight k-blocks of whole tiles, each tile's parts summed over a tree of exchanges in
# one XCD's L2 (at most two tiles a workgroup, or where the second pass's split would need a
# second round of workgroups): 9..16 rows at long K, a narrow N at very long K, 8-bit and
# group 32.
TREE_CASES = [
    (16, 640, 17408, 4, 64, BF16),           # six k-blocks, one tile a workgroup
    (16, 1024, 24576, 4, 64, F16),           # eight k-blocks, two tiles a workgroup
    (9, 1000, 17408, 4, 64, BF16),           # four k-blocks
    (8, 1024, 32768, 4, 64, BF16),           # six k-blocks at 8 rows
    (12, 1280, 17408, 8, 128, BF16),
    (16, 1024, 17408, 4, 32, F16),
]


@pytest.mark.parametrize("M,N,K,bits,gs,dt", TREE_CASES)
def test_tree_of_exchanges_matches_oracle_and_repeats(ctx, oracle, M, N, K, bits, gs, dt):
    p = ctx.plan(M, N, K, bits, gs)
    assert 4 <= p["nkb"] <= 8, p
    check_aligned(ctx, oracle, M, N, K, bits, gs, dt, p["nkb"])


# 9..16 rows at long K whose second pass's split fits one round: the tree of as many k-blocks,
# up to 8 tiles a workgroup
ROWS_TREE_CASES = [
    (9, 5120, 17408, 4, 64, BF16),           # four k-blocks, five tiles a workgroup
    (13, 5120, 17408, 4, 64, F16),           # six k-blocks, eight tiles
    (16, 4096, 16384, 4, 64, BF16),          # six k-blocks
    (11, 5120, 17408, 4, 128, BF16),
    (12, 5120, 17408, 8, 64, F16),           # five k-blocks, 8-bit
]


@pytest.mark.parametrize("M,N,K,bits,gs,dt", ROWS_TREE_CASES)
def test_tree_at_nine_to_sixteen_rows(ctx, oracle, M, N, K, bits, gs, dt):
    p = ctx.plan(M, N, K, bits, gs)
    assert 4 <= p["nkb"] <= 8 and -(-((N + 15) // 16) // p["Gkb"]) <= 8, p
    check_aligned(ctx, oracle, M, N, K, bits, gs, dt, p["nkb"])


@pytest.mark.parametrize("M,N,K,bits,gs,dt", ALIGNED_CASES)
def test_aligned_split_matches_oracle_and_repeats(ctx, oracle, M, N, K, bits, gs, dt):
    check_aligned(ctx, oracle, M, N, K, bits, gs, dt, 2)


@pytest.mark.parametrize("M,N,K,bits,gs,dt", THREE_BLOCK_CASES)
def test_three_block_aligned_split_matches_oracle_and_repeats(ctx, oracle, M, N, K, bits, gs,
                                                              dt):
    check_aligned(ctx, oracle, M, N, K, bits, gs, dt, 3)


def check_aligned(ctx, oracle, M, N, K, bits, gs, dt, nkb):
    import torch
    p = ctx.plan(M, N, K, bits, gs)
    assert p["aligned"] == 1 and p["nkb"] == nkb and p["reduce"] == 0, p
    c = make_case(M, N, K, bits=bits, gs=gs, xdt=dt, seed=11 * M + N + K + bits + gs,
                  lbias=(N % 2 == 1))
    announce(f"aligned M={M} N={N} K={K} bits={bits} gs={gs} dt={dt}")
    x, w, s, b, lb = upload(c)
    y = ctx.qmm(x, w, s, b, c.bits, c.gs, lbias=lb)
    torch.cuda.synchronize()
    rel, ok = tolerance_check(download(y), oracle.qmm_f64(c))
    assert rel <= TOL and ok, f"max rel err {rel:.3e}"
    for _ in range(3):                       # pair exchange: deterministic, workspace re-armed
        y2 = ctx.qmm(x, w, s, b, c.bits, c.gs, lbias=lb)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), y2.view(torch.int16))


# 9..12 rows whose x fits one k-block (up to 16 staged items a thread, a ring shrunk to fit):
# a stream-K split of one round with the pair exchange at range boundaries
ONE_K_BLOCK_CASES = [
    (10, 17408, 5120, 4, 64, BF16),
    (11, 34816, 5120, 4, 64, F16),           # burst: tiles written at the end
    (12, 17408, 5120, 8, 64, BF16),
    (9, 20000, 5120, 4, 64, F16),
]

# splits that take whole rounds of workgroups (2, 3, ... per CU)
ROUND_CASES = [
    (4, 11008, 11008, 4, 64, BF16),          # one-super-step chunks, two rounds
    (1, 2000, 32768, 4, 64, F16),            # two rounds, the second pass
]


def check_repeat(ctx, oracle, M, N, K, bits, gs, dt, what):
    import torch
    c = make_case(M, N, K, bits=bits, gs=gs, xdt=dt, seed=13 * M + N + K + bits + gs,
                  lbias=(N % 2 == 0))
    announce(f"{what} M={M} N={N} K={K} bits={bits} gs={gs} dt={dt}")
    x, w, s, b, lb = upload(c)
    y = ctx.qmm(x, w, s, b, c.bits, c.gs, lbias=lb)
    torch.cuda.synchronize()
    rel, ok = tolerance_check(download(y), oracle.qmm_f64(c))
    assert rel <= TOL and ok, f"max rel err {rel:.3e}"
    for _ in range(2):
        y2 = ctx.qmm(x, w, s, b, c.bits, c.gs, lbias=lb)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), y2.view(torch.int16))


@pytest.mark.parametrize("M,N,K,bits,gs,dt", ONE_K_BLOCK_CASES)
def test_one_k_block_at_nine_to_twelve_rows(ctx, oracle, M, N, K, bits, gs, dt):
    p = ctx.plan(M, N, K, bits, gs)
    assert p["nkb"] == 1 and p["Gkb"] <= ctx.num_cus and p["reduce"] == 0, p
    check_repeat(ctx, oracle, M, N, K, bits, gs, dt, "one k-block")


@pytest.mark.parametrize("M,N,K,bits,gs,dt", ROUND_CASES)
def test_whole_rounds_of_workgroups(ctx, oracle, M, N, K, bits, gs, dt):
    p = ctx.plan(M, N, K, bits, gs)
    g0 = ctx.num_cus // p["nkb"]
    assert p["Gkb"] > g0 and p["Gkb"] % g0 == 0, p
    check_repeat(ctx, oracle, M, N, K, bits, gs, dt, "rounds")


@pytest.mark.parametrize("M,N,K,bits,gs,dt", SIXTEEN_ROW_CASES)
def test_sixteen_row_shapes_match_oracle(ctx, oracle, M, N, K, bits, gs, dt):
    c = make_case(M, N, K, bits=bits, gs=gs, xdt=dt, seed=M * 1000 + N + K + bits + gs,
                  lbias=(N % 2 == 0))
    announce(f"sixteen-row M={M} N={N} K={K} bits={bits} gs={gs} dt={dt}")
    y = download(run_fast(ctx, c))
    ref = oracle.qmm_f64(c)
    rel, ok = tolerance_check(y, ref)
    assert rel <= TOL and ok, f"max rel err {rel:.3e}"


@pytest.mark.parametrize("name,M", [
    ("c1_m1_k4096_n4096_f16", 1),
    ("c2_gateup_k5120_n17408", 1), ("c2_gateup_k5120_n17408", 2),
    ("c2_gateup_k5120_n17408", 4), ("c2_gateup_k5120_n17408", 6),
    ("c2_gateup_k5120_n17408", 8),
    ("c3_down_k17408_n5120", 8),
    ("c4_qkv_8bit_g64", 8), ("c4_o_8bit_g64", 8),
    ("c4_qkv_4bit_g32", 8), ("c4_o_4bit_g32", 8),
    ("c2_gateup_k5120_n17408", 9), ("c2_gateup_k5120_n17408", 10),
    ("c2_gateup_k5120_n17408", 11), ("c2_gateup_k5120_n17408", 12),
    ("c3_down_k17408_n5120", 12),
    ("c2_gateup_k5120_n17408", 16), ("c3_down_k17408_n5120", 16),
    ("c4_qkv_8bit_g64", 16), ("c4_o_4bit_g32", 16),
])
def test_benchmark_configs_match_oracle(ctx, oracle, name, M):
    c = config_case(name, M)
    announce(f"config {name} M={M}")
    y = download(run_fast(ctx, c))
    ref = oracle.qmm_f64(c)
    rel, ok = tolerance_check(y, ref)
    assert rel <= TOL and ok, f"{name} M={M}: max rel err {rel:.3e}"


def test_rows_are_independent_of_m(ctx):
    """Row r of an 8-row call is bit-identical to the 1-row call on x[r]."""
    import torch
    c = config_case("c2_gateup_k5120_n17408", 8)
    x, w, s, b, _ = upload(c)
    announce("row independence c2 M=8 vs M=1")
    y8 = ctx.qmm(x, w, s, b, 4, 64)
    for r in (0, 3, 7):
        y1 = ctx.qmm(x[r:r + 1].contiguous(), w, s, b, 4, 64)
        assert torch.equal(y8[r:r + 1].view(torch.int16), y1.view(torch.int16)), f"row {r}"


@pytest.mark.parametrize("M", [8, 16])
def test_repeat_calls_are_bit_identical(ctx, M):
    """Deterministic fix-up order and a re-armed workspace: same bits on every call."""
    import torch
    c = config_case("c3_down_k17408_n5120", M)
    x, w, s, b, _ = upload(c)
    announce(f"determinism c3 M={M} x3")
    ys = [ctx.qmm(x, w, s, b, 4, 64).clone() for _ in range(3)]
    for y in ys[1:]:
        assert torch.equal(ys[0].view(torch.int16), y.view(torch.int16))


def test_sixteen_rows_take_one_launch(ctx):
    """16 rows of the gate/up shape are planned as one launch over the weights."""
    p = ctx.plan(16, 17408, 5120, 4, 64)
    assert p["ch"] > 1 and p["T"] == 1088


def test_kernel_output_is_not_the_generic_path(ctx):
    """Negative control (SmallMQuantizedMatmulTests.swift:94-102): the fast kernel's
    accumulation order differs from the generic path's, so at least one output moves."""
    import torch
    c = config_case("c2_gateup_k5120_n17408", 8)
    x, w, s, b, _ = upload(c)
    announce("negative control c2 M=8 fast vs generic")
    fast = ctx.qmm(x, w, s, b, 4, 64)
    slow = ctx.fallback(x, w, s, b, 4, 64)
    assert slow.dtype == fast.dtype
    assert not torch.equal(fast.view(torch.int16), slow.view(torch.int16))
    rel, ok = tolerance_check(download(fast), download(slow))
    assert rel <= TOL and ok


def test_generic_path_matches_oracle(ctx, oracle):
    for (M, N, K, bits, gs, dt) in [(3, 50, 256, 4, 64, BF16), (2, 40, 256, 8, 32, F16),
                                    (4, 33, 512, 2, 64, BF16), (5, 64, 384, 4, 128, BF16)]:
        c = make_case(M, N, K, bits=bits, gs=gs, xdt=dt, seed=K + N, lbias=True)
        x, w, s, b, lb = upload(c)
        announce(f"generic M={M} N={N} K={K} bits={bits} gs={gs}")
        y = download(ctx.fallback(x, w, s, b, bits, gs, lbias=lb))
        rel, ok = tolerance_check(y, oracle.qmm_f64(c))
        assert rel <= TOL and ok, (M, N, K, bits, gs, rel)


def test_generic_path_promotes_mixed_dtypes(ctx, oracle):
    """fp16 x against bf16 scales: MLX promotes to fp32, and so does the generic path."""
    import torch
    c = make_case(4, 64, 256, bits=4, gs=64, xdt=F16, sdt=BF16, seed=9)
    x, w, s, b, _ = upload(c)
    announce("generic mixed dtype")
    y = ctx.fallback(x, w, s, b, 4, 64)
    assert y.dtype == torch.float32
    rel, ok = tolerance_check(download(y), oracle.qmm_f64(c))
    assert rel <= 1e-5 and ok
