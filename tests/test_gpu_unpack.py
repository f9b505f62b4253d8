"""Bit-exact GPU pin of the kernel's integer unpack and dequantisation.

With one-hot activation rows (x[m] = e_k) the product is a column of the dequantised
matrix: y[m, n] = s[n, k/gs] * q[n, k] + b[n, k/gs].  Scales are powers of two and biases
small integers, chosen per group so that every such value is exact in fp32 and in the output
dtype; the kernel's factored form (s * sum x (MAGIC + q) + (b - MAGIC s) * sum x) is then
exact too, and y must equal the oracle's bit-exact dequant (Sources/DFlashKit/
SmallMQuantizedMatmul.swift:55-71: code t of a word is (p >> bits*t) & mask, element 0 in the
low bits; dequant s*q + b) bit for bit.  The one-hot rows walk every k position of a chunk
(8 quantisation groups, several super-steps), so a mistake confined to a few codes, lanes,
words or groups cannot hide under a tolerance.

Covered: every bits x group size x dtype in the 1..8-row form with 8-group chunks (c8), the
9..16-row form (mt16) and one-super-step chunks (c1), plus the narrow split (two k-blocks,
one tile per workgroup, pair exchange), the aligned split (two k-blocks of whole tiles per
workgroup), three k-blocks of whole tiles (chained pair exchange) and a reduce split
(several k-blocks, second pass); and the same over the packed layout (dfq_pack_weights,
dfq_qmm_packed) for every format at 1..8 and 9..16 rows and in each split.
"""
import numpy as np
import pytest

from gpu_util import announce, to_dev16
from onehot import exact_case
from oracle.qmm_oracle import BF16, F16, from_bits, to_bits

pytestmark = pytest.mark.gpu

FORMATS = [(bits, gs, dt) for bits in (4, 8) for gs in (32, 64, 128) for dt in (BF16, F16)]


def kss(bits, gs):
    return (512 // bits) * ((2 if gs == 128 else 1) if bits == 4 else gs // 32)


def chunk_groups(bits, gs, M=8):
    """Groups of the chunks the planner picks where K allows: 8; 16 for 4-bit group 32 at up
    to 8 rows (the c16 kernels)."""
    return 16 if (bits, gs) == (4, 32) and M <= 8 else 8


def chunk_k(bits, gs, M=8):
    return chunk_groups(bits, gs, M) * gs


def run_one_hot(ctx, N, K, bits, gs, dt, M, positions, seed, expect_plan=None, packed=False):
    """y for one-hot rows at `positions` (M per call) against the exact dequant columns;
    with `packed`, through the packed layout."""
    import torch
    if expect_plan is not None:
        p = ctx.plan(M, N, K, bits, gs)
        for key, val in expect_plan.items():
            assert p[key] == val, (key, p)
    w, sb, bb, deq = exact_case(N, K, bits, gs, dt, seed)
    pos = np.asarray(positions, dtype=np.int64)
    pad = (-len(pos)) % M
    pos = np.concatenate([pos, pos[:pad]])
    calls = len(pos) // M
    tdt = torch.bfloat16 if dt == BF16 else torch.float16
    wd = torch.from_numpy(w.view(np.int32)).cuda()
    sd, bd = to_dev16(sb, dt), to_dev16(bb, dt)
    x = torch.zeros(len(pos), K, dtype=tdt, device="cuda")
    x[torch.arange(len(pos), device="cuda"), torch.from_numpy(pos).cuda()] = 1.0
    y = torch.empty(len(pos), N, dtype=tdt, device="cuda")
    announce(f"one-hot bits={bits} gs={gs} dt={dt} M={M} N={N} K={K} calls={calls} "
             f"packed={packed}")
    pw = ctx.pack(wd, sd, bd, bits, gs) if packed else None
    for c in range(calls):
        if packed:
            ctx.qmm_packed(x[c * M:(c + 1) * M], pw, out=y[c * M:(c + 1) * M])
        else:
            ctx.qmm(x[c * M:(c + 1) * M], wd, sd, bd, bits, gs, out=y[c * M:(c + 1) * M])
    torch.cuda.synchronize()
    got = y.view(torch.int16).cpu().numpy().view(np.uint16)
    want = to_bits(deq[:, pos].T, dt)
    bad = np.argwhere(got != want)
    assert bad.size == 0, (
        f"{len(bad)} of {got.size} outputs differ; first (row k={pos[bad[0][0]]}, n={bad[0][1]}):"
        f" got {from_bits(got[tuple(bad[0])], dt)} want {deq[bad[0][1], pos[bad[0][0]]]}")


@pytest.mark.parametrize("bits,gs,dt", FORMATS)
def test_unpack_is_exact_up_to_8_rows(ctx, bits, gs, dt):
    """1..8 rows, 8-group chunks: every k of two chunks, ragged N (a partial last tile)."""
    K = 2 * chunk_k(bits, gs)
    run_one_hot(ctx, 40, K, bits, gs, dt, 8, range(K), seed=bits * 1000 + gs + dt,
                expect_plan={"ch": chunk_k(bits, gs) // kss(bits, gs), "nkb": 1})


@pytest.mark.parametrize("bits,gs,dt", FORMATS)
def test_unpack_is_exact_for_16_rows(ctx, bits, gs, dt):
    """9..16 rows in one launch (two row tiles per weight tile): every k of one chunk."""
    K = chunk_k(bits, gs, 16)
    run_one_hot(ctx, 48, K, bits, gs, dt, 16, range(K), seed=bits * 2000 + gs + dt,
                expect_plan={"ch": chunk_k(bits, gs, 16) // kss(bits, gs)})


@pytest.mark.parametrize("dt", [BF16, F16])
def test_unpack_is_exact_with_8_group_chunks_at_4bit_group_32(ctx, dt):
    """4-bit group 32 with K a multiple of 8 groups but not of 16 (K = 768): the 1..8-row
    kernels take 8-group chunks there; every k."""
    run_one_hot(ctx, 40, 768, 4, 32, dt, 8, range(768), seed=9100 + dt,
                expect_plan={"ch": 2})


@pytest.mark.parametrize("bits,gs,dt", FORMATS)
def test_unpack_is_exact_with_one_super_step_chunks(ctx, bits, gs, dt):
    """K not a multiple of a chunk: one-super-step chunks (c1), every k."""
    K = 3 * kss(bits, gs)
    if K % chunk_k(bits, gs) == 0:
        K += kss(bits, gs)
    run_one_hot(ctx, 24, K, bits, gs, dt, 7, range(K), seed=bits * 3000 + gs + dt,
                expect_plan={"ch": 1})


@pytest.mark.parametrize("bits,gs,dt,M", [(4, 64, BF16, 8), (8, 32, F16, 8), (4, 64, BF16, 12),
                                           (8, 128, F16, 5)])
def test_unpack_is_exact_in_the_narrow_split(ctx, bits, gs, dt, M):
    """Few tiles, long K: two k-blocks of one tile per workgroup (pair exchange).  Every k of
    the first and the last chunk, and of one chunk in the second k-block's start."""
    ck = chunk_k(bits, gs)
    K = 8 * ck
    pos = list(range(ck)) + list(range(4 * ck, 5 * ck)) + list(range(7 * ck, 8 * ck))
    run_one_hot(ctx, 64, K, bits, gs, dt, M, pos, seed=bits * 4000 + gs + dt,
                expect_plan={"nkb": 2, "reduce": 0, "nslot_kb": 1})


@pytest.mark.parametrize("bits,gs,dt,M", [(4, 64, BF16, 16), (8, 64, F16, 12)])
def test_unpack_is_exact_in_the_aligned_split(ctx, bits, gs, dt, M):
    """Two k-blocks of whole tiles per workgroup (16 tiles, K = 10 chunks): every k of the
    first chunk of each k-block and of the last chunk."""
    ck = chunk_k(bits, gs)
    K = 10 * ck
    pos = list(range(ck)) + list(range(5 * ck, 6 * ck)) + list(range(9 * ck, 10 * ck))
    run_one_hot(ctx, 256, K, bits, gs, dt, M, pos, seed=bits * 6000 + gs + dt,
                expect_plan={"nkb": 2, "aligned": 1, "reduce": 0})


@pytest.mark.parametrize("bits,gs,dt,M", [(4, 64, BF16, 8), (8, 64, F16, 16)])
def test_unpack_is_exact_in_a_reduce_split(ctx, bits, gs, dt, M):
    """Several k-blocks and workgroups per tile, summed by the second pass: every k of the
    first, a middle and the last chunk."""
    ck = chunk_k(bits, gs)
    K = 48 * ck
    pos = list(range(ck)) + list(range(23 * ck, 24 * ck)) + list(range(47 * ck, 48 * ck))
    run_one_hot(ctx, 48, K, bits, gs, dt, M, pos, seed=bits * 5000 + gs + dt,
                expect_plan={"reduce": 1})


@pytest.mark.parametrize("bits,gs,dt,M", [(4, 64, BF16, 8), (8, 64, F16, 7)])
def test_unpack_is_exact_in_the_three_block_aligned_split(ctx, bits, gs, dt, M):
    """Three k-blocks of whole tiles per workgroup, summed by a chain of two pair exchanges:
    every k of the first chunk of each k-block and of the last chunk (K = 32 chunks)."""
    ck = chunk_k(bits, gs)
    K = 32 * ck
    pos = (list(range(ck)) + list(range(10 * ck, 11 * ck)) + list(range(21 * ck, 22 * ck))
           + list(range(31 * ck, 32 * ck)))
    run_one_hot(ctx, 48, K, bits, gs, dt, M, pos, seed=bits * 7000 + gs + dt,
                expect_plan={"nkb": 3, "aligned": 1, "reduce": 0})


@pytest.mark.parametrize("bits,gs,dt", FORMATS)
@pytest.mark.parametrize("M", [8, 16])
def test_unpack_is_exact_over_the_packed_layout(ctx, bits, gs, dt, M):
    """The packed layout, 1..8 and 9..16 rows: every k of two chunks, ragged N."""
    K = 2 * chunk_k(bits, gs)
    run_one_hot(ctx, 40, K, bits, gs, dt, M, range(K), seed=bits * 7000 + gs + dt + M,
                packed=True)


@pytest.mark.parametrize("bits,gs,dt,M,N,chunks,plan", [
    (4, 64, BF16, 8, 64, 8, {"nkb": 2, "reduce": 0, "nslot_kb": 1}),    # narrow
    (8, 64, F16, 12, 256, 10, {"nkb": 2, "aligned": 1, "reduce": 0}),   # aligned
    (4, 64, BF16, 8, 48, 64, {"reduce": 1}),                           # reduce
    # 4-bit group 32 at 16 rows: 8-group chunks over 16-group packed units, six k-blocks,
    # two of which start half way into a unit
    (4, 32, F16, 16, 48, 34, {"reduce": 1, "nkb": 6, "ch": 2}),
])
def test_unpack_is_exact_over_the_packed_layout_in_each_split(ctx, bits, gs, dt, M, N, chunks,
                                                              plan):
    """The packed layout in the narrow, aligned and reduce splits: every k of the first, a
    middle and the last chunk."""
    ck = chunk_k(bits, gs)
    K = chunks * ck
    mid = chunks // 2
    pos = list(range(ck)) + list(range(mid * ck, (mid + 1) * ck)) + \
        list(range((chunks - 1) * ck, chunks * ck))
    run_one_hot(ctx, N, K, bits, gs, dt, M, pos, seed=bits * 8000 + gs + dt, expect_plan=plan,
                packed=True)


@pytest.mark.parametrize("bits,gs,dt,M,N,K", [(4, 64, BF16, 16, 640, 17408),
                                              (8, 64, F16, 16, 640, 17408),
                                              (4, 64, BF16, 8, 1024, 32768)])
def test_unpack_is_exact_in_a_tree_of_exchanges(ctx, bits, gs, dt, M, N, K):
    """Six k-blocks of whole tiles, each tile's parts summed over a tree of exchanges: every k
    of the first chunk of each k-block and of the last chunk."""
    p = ctx.plan(M, N, K, bits, gs)
    assert p["nkb"] == 6 and p["aligned"] == 1 and p["reduce"] == 0, p
    ck = chunk_k(bits, gs, M)
    starts = [kb * p["chunks"] // p["nkb"] for kb in range(p["nkb"])] + [p["chunks"] - 1]
    pos = [c * ck + k for c in sorted(set(starts)) for k in range(ck)]
    run_one_hot(ctx, N, K, bits, gs, dt, M, pos, seed=bits * 9000 + gs + dt + M)
