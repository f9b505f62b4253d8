"""The fused gate|up projection with its SiLU-mul epilogue (dfq_qmm_silu_gate_up).

The weight, scales, biases and linear bias of the gate and up projections are interleaved by
8 rows on the device (dfq_interleave_gate_up).  The epilogue must be bit-identical to the same
qmm on the interleaved weight followed by dfq_silu_mul on its de-interleaved output (same
split, same sums, g and u rounded before silu), and within the parity tolerance of the fp64
oracle: silu(round(g)) * round(u) with g and u from the oracle's gate and up matmuls.
"""
import numpy as np
import pytest

from gpu_util import announce, download, to_dev16, upload
from oracle.qmm_oracle import BF16, F16, from_bits, make_case, to_bits, tolerance_check

pytestmark = pytest.mark.gpu

TOL = 1e-2

CASES = [
    # (M, H, K, bits, gs, dtype, linear bias)
    (8, 17408, 5120, 4, 64, BF16, False),   # the C5 gate|up: tiles shared by two workgroups
    (8, 1024, 512, 4, 64, BF16, True),      # linear bias
    (16, 2048, 1024, 4, 64, BF16, False),   # two row tiles
    (8, 2048, 16384, 4, 64, BF16, False),   # a reduce split
    (5, 1536, 1024, 8, 64, F16, True),      # 8-bit, fp16
    (12, 1024, 384, 4, 64, BF16, False),    # one-super-step chunks: two launches of <= 8 rows
    (8, 256, 5120, 4, 64, BF16, True),      # narrow: two k-blocks, one tile per workgroup
    (6, 2048, 2048, 8, 128, F16, True),     # 8-bit g128
    (16, 1024, 1024, 4, 32, BF16, True),    # 4-bit g32, two row tiles
    (1, 4096, 4096, 4, 64, F16, False),     # one row
    (8, 2560, 17408, 4, 64, BF16, True),    # three k-blocks of whole tiles: chained exchange
    (7, 512, 16384, 8, 64, F16, False),     # the same, one tile per workgroup
    (16, 1504, 7680, 4, 64, BF16, True),    # the same with two row tiles
    (16, 17408, 5120, 4, 64, BF16, False),  # two k-blocks: every tile's (g, u) words exchanged
    (16, 512, 24576, 4, 64, F16, True),     # eight k-blocks: a tree of (g, u) exchanges
]


def deinterleave(torch, y, H):
    """[M, 2H] interleaved by 8 columns -> [M, 2H] as gate | up."""
    M = y.shape[0]
    v = y.view(M, H // 8, 2, 8)
    return torch.cat([v[:, :, 0, :].reshape(M, H), v[:, :, 1, :].reshape(M, H)], dim=1).contiguous()


@pytest.mark.parametrize("M,H,K,bits,gs,dt,lb", CASES)
def test_epilogue_matches_qmm_then_silu_and_oracle(ctx, oracle, M, H, K, bits, gs, dt, lb):
    import torch
    cg = make_case(M, H, K, bits=bits, gs=gs, xdt=dt, seed=M + H + K, lbias=lb)
    cu = make_case(M, H, K, bits=bits, gs=gs, xdt=dt, seed=M + H + K + 1, lbias=lb)
    cu.x = cg.x
    x, wg, sg, bg, lbg = upload(cg)
    _, wu, su, bu, lbu = upload(cu)
    announce(f"gate|up interleave H={H} K={K}")
    w = ctx.interleave_gate_up(wg, wu)
    s = ctx.interleave_gate_up(sg, su)
    b = ctx.interleave_gate_up(bg, bu)
    l = ctx.interleave_gate_up(lbg, lbu) if lb else None
    torch.cuda.synchronize()
    announce(f"gate|up epilogue M={M} H={H} K={K} bits={bits} dt={dt}")
    h = ctx.qmm_silu_gate_up(x, w, s, b, bits, gs, lbias=l)
    y = ctx.qmm(x, w, s, b, bits, gs, lbias=l)
    ref = ctx.silu_mul(deinterleave(torch, y, H))
    torch.cuda.synchronize()
    assert torch.equal(h.view(torch.int16), ref.view(torch.int16))
    g64 = oracle.qmm_f64(cg)
    u64 = oracle.qmm_f64(cu)
    gr = from_bits(to_bits(g64, dt), dt).astype(np.float64)
    ur = from_bits(to_bits(u64, dt), dt).astype(np.float64)
    h64 = gr / (1.0 + np.exp(-gr)) * ur
    rel, ok = tolerance_check(download(h), h64)
    assert rel <= TOL and ok, f"max rel err {rel:.3e}"


def test_epilogue_needs_h_a_multiple_of_8(ctx):
    import torch
    import dflash_qmm
    x = torch.zeros(8, 512, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(2 * 12, 64, dtype=torch.int32, device="cuda")
    s = torch.zeros(2 * 12, 8, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(dflash_qmm.DfqError):
        ctx.qmm_silu_gate_up(x, w, s, s, 4, 64)
