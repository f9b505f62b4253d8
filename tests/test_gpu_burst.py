"""Splits whose workgroups hold many tiles write their outputs at the end of the workgroup
("burst"): every tile without a pair exchange goes from the LDS output area to y, with
16-byte row stores where a row's 8 columns are aligned and in range and element stores
elsewhere, after the streaming; in a reduce split (two k-blocks of 9..16 rows) each tile's
part goes to its workspace slot at that point instead, for the second pass.  These shapes
take that path (asserted from the plan) at sizes the oracle checks in seconds: every row
count 1..16, bf16 and fp16, 4- and 8-bit, group 32, 64 and 128, a linear bias, N that is not
a multiple of 16 or of 8 (element stores), and the gate|up epilogue; each against the fp64
oracle within the parity bar and bit-identical on a repeat call (which also shows the
workspace left zero).  The fused greedy accept at burst shapes is in
test_gpu_lm_head_accept.py.
"""
import numpy as np
import pytest

from gpu_util import announce, download, upload
from oracle.qmm_oracle import BF16, F16, from_bits, make_case, to_bits, tolerance_check

pytestmark = pytest.mark.gpu

TOL = 1e-2

CASES = [
    # (M, N, K, bits, gs, dtype, linear bias, reduce split)
    (1, 32768, 512, 4, 64, BF16, False, 0),
    (8, 32768, 512, 4, 64, BF16, True, 0),
    (16, 32768, 512, 4, 64, F16, False, 0),     # two row tiles
    (12, 33000, 512, 4, 64, BF16, True, 0),     # last tile 8 columns wide
    (8, 33003, 512, 4, 64, BF16, False, 0),     # rows not 16-byte aligned: element stores
    (5, 40000, 1024, 8, 64, F16, True, 0),      # 8-bit, two chunks per tile
    (8, 36000, 1024, 4, 32, BF16, False, 0),    # group 32
    (3, 40000, 2048, 8, 128, BF16, True, 0),    # 8-bit g128
    # two k-blocks of stream-K ranges (over 24 tiles a workgroup): parts to the workspace at
    # the end, second pass
    (16, 60000, 4096, 4, 64, BF16, True, 1),
    (16, 60000, 4096, 8, 64, F16, False, 1),
    (16, 52000, 4096, 4, 32, BF16, False, 1),   # group 32, one super-step per chunk half
    (12, 60000, 6144, 4, 64, BF16, False, 1),
    # 9..16 rows whose x fits one k-block with a shrunk ring: no second pass
    (13, 40000, 4096, 4, 32, BF16, False, 0),
    (16, 40000, 4096, 4, 128, F16, True, 0),    # g128, a ring of ten slots
]


@pytest.mark.parametrize("M,N,K,bits,gs,dt,lb,red", CASES)
def test_burst_split_matches_oracle_and_repeats(ctx, oracle, M, N, K, bits, gs, dt, lb, red):
    import torch
    plan = ctx.plan(M, N, K, bits, gs)
    assert plan["burst"] == 1 and plan["reduce"] == red, plan
    c = make_case(M, N, K, bits=bits, gs=gs, xdt=dt, seed=3 * M + N + K, lbias=lb)
    x, w, s, b, lbias = upload(c)
    announce(f"burst qmm M={M} N={N} K={K} bits={bits} gs={gs} dt={dt} plan={plan}")
    y1 = ctx.qmm(x, w, s, b, bits, gs, lbias=lbias)
    y2 = ctx.qmm(x, w, s, b, bits, gs, lbias=lbias)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    rel, ok = tolerance_check(download(y1), oracle.qmm_f64(c))
    assert rel <= TOL and ok, f"max rel err {rel:.3e}"


def deinterleave(torch, y, H):
    """[M, 2H] interleaved by 8 columns -> [M, 2H] as gate | up."""
    M = y.shape[0]
    v = y.view(M, H // 8, 2, 8)
    return torch.cat([v[:, :, 0, :].reshape(M, H), v[:, :, 1, :].reshape(M, H)], dim=1).contiguous()


@pytest.mark.parametrize("M,H,K,dt,lb", [(8, 16384, 512, BF16, True), (16, 16384, 512, F16, False),
                                         (1, 20000, 512, BF16, False),
                                         (16, 30000, 4096, BF16, True)])  # reduce split
def test_burst_gate_up_epilogue(ctx, oracle, M, H, K, dt, lb):
    import torch
    assert ctx.plan(M, 2 * H, K, 4, 64)["burst"] == 1
    cg = make_case(M, H, K, bits=4, gs=64, xdt=dt, seed=M + H, lbias=lb)
    cu = make_case(M, H, K, bits=4, gs=64, xdt=dt, seed=M + H + 1, lbias=lb)
    cu.x = cg.x
    x, wg, sg, bg, lbg = upload(cg)
    _, wu, su, bu, lbu = upload(cu)
    w = ctx.interleave_gate_up(wg, wu)
    s = ctx.interleave_gate_up(sg, su)
    b = ctx.interleave_gate_up(bg, bu)
    l = ctx.interleave_gate_up(lbg, lbu) if lb else None
    torch.cuda.synchronize()
    announce(f"burst gate|up M={M} H={H} K={K} dt={dt}")
    h = ctx.qmm_silu_gate_up(x, w, s, b, 4, 64, lbias=l)
    y = ctx.qmm(x, w, s, b, 4, 64, lbias=l)
    ref = ctx.silu_mul(deinterleave(torch, y, H))
    torch.cuda.synchronize()
    assert torch.equal(h.view(torch.int16), ref.view(torch.int16))
    g64 = oracle.qmm_f64(cg)
    u64 = oracle.qmm_f64(cu)
    gr = from_bits(to_bits(g64, dt), dt).astype(np.float64)
    ur = from_bits(to_bits(u64, dt), dt).astype(np.float64)
    rel, ok = tolerance_check(download(h), gr / (1.0 + np.exp(-gr)) * ur)
    assert rel <= TOL and ok, f"max rel err {rel:.3e}"
