"""The C call sequence of the Swift package's greedyAccept (dflash-swift_amd/swift/Sources/
DFlashKitHIP/SmallMQuantizedMatmulHIP.swift), replayed through ctypes, since no Swift toolchain is here to
run the package itself: the workspace sized in 4-byte words, (need + 3) / 4 of them, cleared
once with dfq_workspace_clear and then reused by every later call without a clear; one buffer
of rows + 1 int32 holding the tokens with the accepted count behind them (accepted =
tokens + rows); the proposals copied in with dfq_memcpy_h2d; no logits buffer; the results
copied out with dfq_memcpy_d2h.  Two verify rounds in a row on the same buffers must give
the oracle's tokens and accepted run (DFlashSpeculativeGenerator.swift:555-571).
"""
import ctypes

import numpy as np
import pytest

import dflash_qmm
from gpu_util import announce, upload
from oracle.qmm_oracle import BF16, argmax_accept, make_case

pytestmark = pytest.mark.gpu


def test_greedy_accept_call_sequence_of_the_swift_package(ctx):
    import torch
    lib, h = ctx.lib, ctx.handle
    rows, vocab, K, bits, gs = 8, 32000, 2048, 4, 64
    c = make_case(rows, vocab, K, bits=bits, gs=gs, xdt=BF16, seed=4242)
    x, w, s, b, _ = upload(c)
    # the expected tokens: the oracle's argmax over the fast kernel's own logits (whose
    # parity with the oracle's matmul other tests pin), so that near-ties cannot differ
    logits = ctx.qmm(x, w, s, b, bits, gs)
    torch.cuda.synchronize()
    want_tok, _ = argmax_accept(logits.view(torch.int16).cpu().numpy().view(np.uint16), BF16)

    stream = torch.cuda.Stream()
    sp = dflash_qmm._stream(stream)
    need = ctypes.c_size_t(0)
    assert lib.dfq_qmm_argmax_accept_workspace_bytes(h, rows, vocab, K, bits, gs,
                                                     ctypes.byref(need)) == 0
    ws_bytes = max(1, (need.value + 3) // 4) * 4
    ptrs = []
    for nbytes in (ws_bytes, (rows + 1) * 4, max(1, rows - 1) * 4):
        p = ctypes.c_void_p()
        assert lib.dfq_malloc(h, nbytes, ctypes.byref(p)) == 0
        ptrs.append(p.value)
    ws, out, props = ptrs
    assert lib.dfq_workspace_clear(h, ws, ws_bytes, sp) == 0
    try:
        for rnd, n_match in enumerate((3, rows - 1)):
            # proposals: the first n_match equal the true tokens, the next one differs
            prop = want_tok[:rows - 1].astype(np.int32).copy()
            if n_match < rows - 1:
                prop[n_match] = (prop[n_match] + 1) % vocab
            assert lib.dfq_memcpy_h2d(h, props, prop.ctypes.data, prop.nbytes, sp) == 0
            announce(f"swift greedyAccept sequence round {rnd}")
            rc = lib.dfq_qmm_argmax_accept(h, x.data_ptr(), w.data_ptr(), s.data_ptr(),
                                           b.data_ptr(), None, None, rows, vocab, K, bits, gs,
                                           BF16, props, out, out + 4 * rows, ws, ws_bytes, sp)
            assert rc == 0, lib.dfq_last_error()
            host = np.zeros(rows + 1, dtype=np.int32)
            assert lib.dfq_memcpy_d2h(h, host.ctypes.data, out, host.nbytes, sp) == 0
            assert host[:rows].tolist() == want_tok.tolist(), rnd
            assert int(host[rows]) == n_match, (rnd, host[rows])
        # the workspace is zero again after the calls (the next round needs no clear)
        back = np.ones(ws_bytes // 4, dtype=np.uint32)
        assert lib.dfq_memcpy_d2h(h, back.ctypes.data, ws, ws_bytes, sp) == 0
        qmm_ws = ctx.workspace_bytes(rows, vocab, K, bits, gs)
        assert not back[:qmm_ws // 4].any()
    finally:
        for p in ptrs:
            lib.dfq_free(h, p)
