"""The LM head fused with the greedy accept (dfq_qmm_argmax_accept).

Its tokens and accepted count must be identical to dfq_qmm followed by dfq_argmax_accept on
that output (itself pinned against the oracle's argmax_accept, and here once more directly),
its logits (when asked for) identical to dfq_qmm's, and its workspace zero again after every
call.  Cases: the C5 LM head (151936 x 5120, tiles shared by two workgroups) at 8 rows and at
16 rows (a split with a second pass, which runs as the pair of calls); whole tiles; the
narrow split; fp16 with a linear bias; one-super-step chunks (also the pair of calls); a tie
across workgroups (two identical weight rows dominating every row: the first index wins) and
a row of NaN (token -1).
Reference: acceptedPrefix, DFlashSpeculativeGenerator.swift:555-571 (argMax, ==, cumprod and
sum at :562-564).
"""
import numpy as np
import pytest

from gpu_util import announce, upload
from oracle.qmm_oracle import BF16, F16, argmax_accept, make_case

pytestmark = pytest.mark.gpu

CASES = [
    # (M, V, K, bits, gs, dtype, linear bias, words)
    (8, 151936, 5120, 4, 64, BF16, False, True),    # the C5 LM head: pair exchange
    (16, 151936, 5120, 4, 64, BF16, False, True),   # 16 rows: a second pass -> two calls
    (8, 4096, 1024, 4, 64, BF16, False, False),     # whole tiles per workgroup
    (8, 1000, 5120, 4, 64, BF16, False, False),     # narrow: two k-blocks, one tile each
    (5, 3000, 2048, 8, 64, F16, True, False),       # fp16, 8-bit, linear bias
    (1, 32000, 4096, 4, 64, BF16, False, False),    # one row: nothing to accept
    (12, 20000, 1024, 4, 32, BF16, False, False),   # 12 rows, group 32
    (8, 3000, 640, 4, 64, BF16, True, False),       # K not 8 groups' worth: two calls
    (8, 32768, 512, 4, 64, BF16, False, False),     # outputs written at the workgroup's end
    (16, 32768, 512, 4, 64, F16, True, False),      # the same, 16 rows, fp16, linear bias
    (3, 40000, 1024, 8, 64, BF16, False, False),    # the same, 8-bit, tiles cut by ranges
    (8, 5000, 17408, 4, 64, BF16, True, False),     # three k-blocks: chained pair exchange
    (16, 3000, 7680, 4, 64, F16, False, False),     # the same with two row tiles
]


def reference(ctx, torch, x, w, s, b, lb, bits, gs, props):
    logits = ctx.qmm(x, w, s, b, bits, gs, lbias=lb)
    ws = torch.zeros(256, dtype=torch.uint8, device="cuda")
    tokens, acc = ctx.argmax_accept(logits, props, ws=ws)
    torch.cuda.synchronize()
    return logits, tokens.cpu().numpy(), int(acc.item())


@pytest.mark.parametrize("M,V,K,bits,gs,dt,lb,words", CASES)
def test_fused_accept_matches_the_two_calls(ctx, M, V, K, bits, gs, dt, lb, words):
    import torch
    c = make_case(M, V, K, bits=bits, gs=gs, xdt=dt, seed=M * 31 + V + K, lbias=lb,
                  words=words)
    x, w, s, b, lbias = upload(c)
    announce(f"fused accept M={M} V={V} K={K} bits={bits} gs={gs} dt={dt} "
             f"plan={ctx.plan(M, V, K, bits, gs)}")
    logits, want_tok, _ = reference(ctx, torch, x, w, s, b, lbias, bits, gs, None)
    lbits = logits.view(torch.int16).cpu().numpy().view(np.uint16)
    oracle_tok, _ = argmax_accept(lbits, dt)
    assert want_tok.tolist() == oracle_tok.tolist()
    need = ctx.qmm_argmax_accept_workspace_bytes(M, V, K, bits, gs)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    # the two-call form (a second pass, or one-super-step chunks) keeps its logits in the
    # workspace's tail, which is not re-zeroed
    pl = ctx.plan(M, V, K, bits, gs)
    tail = (M * V * 2 + 255) // 256 * 256 if pl["reduce"] or pl["ch"] == 1 else 0
    for agree in sorted({0, M // 2, M - 1}):          # proposals matching the first `agree`
        props = want_tok[: M - 1].astype(np.int32).copy()
        if agree < M - 1:
            props[agree] = (props[agree] + 1) % V
        p_dev = torch.from_numpy(props).cuda() if M > 1 else None
        _, _, want_acc = reference(ctx, torch, x, w, s, b, lbias, bits, gs, p_dev)
        assert want_acc == min(agree, M - 1)
        for with_logits in (False, True):
            announce(f"fused accept M={M} V={V} agree={agree} logits={with_logits}")
            out = torch.full_like(logits, 7.0) if with_logits else None
            tokens, acc = ctx.qmm_argmax_accept(x, w, s, b, bits, gs, proposals=p_dev,
                                                lbias=lbias, logits=out, ws=ws)
            torch.cuda.synchronize()
            assert tokens.cpu().numpy().tolist() == want_tok.tolist()
            assert int(acc.item()) == want_acc
            if with_logits:
                assert torch.equal(out.view(torch.int16), logits.view(torch.int16))
            assert int(ws[:need - tail].count_nonzero().item()) == 0   # zero again


@pytest.mark.parametrize("V,K,far", [(8192, 1024, 5000), (32768, 512, 30000)])
def test_fused_accept_ties_and_nan_rows(ctx, V, K, far):
    """x is made non-negative, so every logit is positive, and columns 100 and `far` get the
    same codes and biases with every scale 0.5 (the others are ~0.02): in every row they are
    equal and the largest, and the first
    index, 100, wins although the two lie in tiles finished by different workgroups.  Row 3
    of x is NaN: every logit of the row is NaN and its token is -1.  The second shape writes
    its outputs (and folds their keys) at the end of each workgroup."""
    import torch
    M = 8
    c = make_case(M, V, K, bits=4, gs=64, seed=77)
    c.x = c.x & np.uint16(0x7FFF)
    c.w[far] = c.w[100]
    c.scales[100] = 0x3F00                                       # bf16 0.5
    c.scales[far] = 0x3F00
    c.biases[far] = c.biases[100]
    x, w, s, b, _ = upload(c)
    x[3] = float("nan")
    announce("fused accept ties / NaN")
    logits, want_tok, _ = reference(ctx, torch, x, w, s, b, None, 4, 64, None)
    assert want_tok[3] == -1
    assert (want_tok[[0, 1, 2, 4, 5, 6, 7]] == 100).all()
    assert ctx.plan(M, V, K, 4, 64)["burst"] == int(V == 32768)
    tokens, acc = ctx.qmm_argmax_accept(x, w, s, b, 4, 64)
    torch.cuda.synchronize()
    assert tokens.cpu().numpy().tolist() == want_tok.tolist()
    assert int(acc.item()) == 0                                  # no proposals
