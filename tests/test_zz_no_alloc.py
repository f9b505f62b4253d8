"""dfq_qmm_noalloc: dfq_qmm with the library's fixed per-GPU scratch as its workspace.

Through the C ABI, its outputs must be bit-identical to dfq_qmm's (same split, same kernels,
only the workspace differs) on calls in a row of decreasing size, which also shows the
scratch is left zero for the next call; a shape whose workspace exceeds the scratch is
refused before any launch.
"""
import ctypes

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


# decreasing in size; the first three need a workspace (pair exchange, reduce split, narrow
# split), the fourth a reduce split of 16 rows, the last one none
CASES = [
    (8, 17408, 5120, 4, 64, BF16, False),
    (8, 5120, 17408, 4, 64, BF16, True),
    (16, 4096, 5120, 8, 64, F16, False),
    (6, 1024, 5120, 4, 128, BF16, True),
    (3, 40, 256, 4, 32, F16, False),
]


def test_noalloc_matches_qmm_on_calls_in_a_row(ctx):
    import torch
    for i, (M, N, K, bits, gs, dt, lbias) in enumerate(CASES):
        c = make_case(M, N, K, bits=bits, gs=gs, xdt=dt, seed=900 + i, lbias=lbias)
        need = ctx.workspace_bytes(M, N, K, bits, gs)
        assert need <= SCRATCH_MAX
        x, w, s, b, lb = upload(c)
        announce(f"noalloc call {i}: M={M} N={N} K={K} bits={bits} gs={gs} ws={need}")
        want = ctx.qmm(x, w, s, b, bits, gs, lbias=lb)
        got = torch.empty_like(want)
        rc = noalloc(ctx, c, x, w, s, b, lb, got)
        assert rc == 0, ctx.lib.dfq_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"call {i}"
    # the same first shape once more, after the others: the scratch was left re-armed
    M, N, K, bits, gs, dt, lbias = CASES[0]
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
    assert ctx.workspace_bytes(M, N, K, 4, 64) > SCRATCH_MAX
    fake = 1 << 40
    rc = ctx.lib.dfq_qmm_noalloc(ctx.handle, fake, fake, fake, fake, None, fake, M, N, K, 4,
                                 64, BF16, BF16, BF16, None)
    assert rc == 3, ctx.lib.dfq_last_error()
    assert b"scratch" in ctx.lib.dfq_last_error()
