"""dfq_qmm_noalloc: dfq_qmm with the library's fixed per-GPU scratch as its workspace.

Through the C ABI, its outputs must be bit-identical to dfq_qmm's (same split, same kernels,
only the workspace differs) on calls in a row of decreasing size, which also shows the
scratch is left zero for the next call; a shape whose workspace exceeds the scratch is
refused before any launch.
"""
import numpy as np
import pytest

import dflash_qmm
from gpu_util import announce, upload
from oracle.qmm_oracle import BF16, F16, make_case

pytestmark = pytest.mark.gpu

SCRATCH_MAX = 64 << 20   # DFQ_SCRATCH_MAX_BYTES


def noalloc(ctx, c, x, w, s, b, lb, y, stream=None):
    rc = ctx.lib.dfq_qmm_noalloc(ctx.handle, x.data_ptr(), w.data_ptr(), s.data_ptr(),
                                 b.data_ptr(), lb.data_ptr() if lb is not None else None,
                                 y.data_ptr(), c.M, c.N, c.K, c.bits, c.gs, c.xdt, c.sdt,
                                 c.xdt, dflash_qmm._stream(stream))
    return rc


# decreasing in size (M, N, K, bits, gs, dtype, linear bias, split the planner must give):
#   12 rows of the headline shape: one k-block with 16 staged x items a thread;
#   the headline shape: one k-block, the pair exchange of tiles shared by two workgroups;
#   a 16-row reduce split: parts in workspace slots, summed and re-zeroed by the second pass;
#   a one-row split over two whole rounds of workgroups;
#   the down projection: three k-blocks of whole tiles, a chain of two pair exchanges;
#   16 rows of 8-bit: two k-blocks, each tile in one workgroup of each, paired;
#   a narrow N at six rows: two k-blocks of one tile per workgroup;
#   a tiny shape that needs no workspace
CASES = [
    (12, 17408, 5120, 4, 64, BF16, False, dict(nkb=1, Gkb=256, reduce=0)),
    (8, 17408, 5120, 4, 64, BF16, False, dict(nkb=1, reduce=0)),
    (16, 60000, 4096, 4, 64, BF16, False, dict(reduce=1)),
    (4, 11008, 11008, 4, 64, F16, True, dict(nkb=1, Gkb=512, reduce=0)),
    (8, 5120, 17408, 4, 64, BF16, True, dict(nkb=3, aligned=1, reduce=0)),
    (16, 4096, 5120, 8, 64, F16, False, dict(nkb=2, reduce=0, nslot_kb=1)),
    (6, 1024, 5120, 4, 128, BF16, True, dict(nkb=2, reduce=0)),
    (3, 40, 256, 4, 32, F16, False, dict(need_ws=0)),
]


@pytest.fixture
def fresh():
    """A context of its own, whose split cache no other test has filled."""
    import torch
    c = dflash_qmm.Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()


def test_noalloc_matches_qmm_on_calls_in_a_row(fresh):
    """Each shape goes through dfq_qmm_noalloc before dfq_qmm has planned it on this context
    (the split comes from the no-allocation table), then through dfq_qmm on a fresh workspace:
    bit-identical."""
    import torch
    ctx = fresh
    for i, (M, N, K, bits, gs, dt, lbias, want_plan) in enumerate(CASES):
        c = make_case(M, N, K, bits=bits, gs=gs, xdt=dt, seed=900 + i, lbias=lbias)
        x, w, s, b, lb = upload(c)
        tdt = torch.bfloat16 if dt == BF16 else torch.float16
        got = torch.empty(M, N, dtype=tdt, device="cuda")
        announce(f"noalloc call {i}: M={M} N={N} K={K} bits={bits} gs={gs}, before dfq_qmm")
        rc = noalloc(ctx, c, x, w, s, b, lb, got)
        assert rc == 0, ctx.lib.dfq_last_error()
        plan = ctx.plan(M, N, K, bits, gs)
        assert all(plan[k] == v for k, v in want_plan.items()), (i, plan)
        need = ctx.workspace_bytes(M, N, K, bits, gs)
        assert need <= SCRATCH_MAX
        announce(f"noalloc call {i}: dfq_qmm, workspace {need}")
        want = ctx.qmm(x, w, s, b, bits, gs, lbias=lb)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"call {i}"
    # the first shape once more, after the others: the scratch was left re-armed
    M, N, K, bits, gs, dt, lbias, _ = CASES[0]
    c = make_case(M, N, K, bits=bits, gs=gs, xdt=dt, seed=900)
    x, w, s, b, _ = upload(c)
    announce("noalloc repeat of call 0")
    want = ctx.qmm(x, w, s, b, bits, gs)
    got = torch.empty_like(want)
    assert noalloc(ctx, c, x, w, s, b, None, got) == 0
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_noalloc_refuses_a_shape_past_the_scratch(ctx):
    """600000 x 5120 at 16 rows needs more workspace than the scratch holds: refused with
    DFQ_ERR_WORKSPACE before any launch (the pointers are never dereferenced)."""
    M, N, K = 16, 600000, 5120
    fake = 1 << 40
    rc = ctx.lib.dfq_qmm_noalloc(ctx.handle, fake, fake, fake, fake, None, fake, M, N, K, 4,
                                 64, BF16, BF16, BF16, None)
    assert rc == 3, ctx.lib.dfq_last_error()
    assert b"scratch" in ctx.lib.dfq_last_error()
    assert ctx.workspace_bytes(M, N, K, 4, 64) > SCRATCH_MAX
