"""The chain kernel (dfq_chain): a layer's ops in one persistent launch.

Every op's output must be bit-identical to the same ops run one by one (dfq_qmm,
dfq_silu_mul): the chain runs the same split and the same arithmetic, only the launch and the
waits between ops differ.  The first op is also checked against the oracle.  The chain holds
two layers of q|k|v, o, gate|up, silu*up and down, where the long-K down projection is a
reduce split (two k-blocks), and buffers are reused across layers.  The timeout path is driven
from the host with a zero wait limit: every wait then fails at once, the error flag is set,
and the kernel still runs to its end.
"""
import numpy as np
import pytest

import dflash_qmm
from gpu_util import announce, download, to_dev16
from oracle.qmm_oracle import BF16, make_case, tolerance_check

pytestmark = pytest.mark.gpu

M = 8
D, QKV, H = 1024, 1536, 8192   # model width, q|k|v width, MLP hidden width


def weights(torch, N, K, seed):
    c = make_case(1, N, K, bits=4, gs=64, seed=seed)
    w = torch.from_numpy(c.w.view(np.int32)).cuda()
    return c, w, to_dev16(c.scales, BF16), to_dev16(c.biases, BF16)


def build(torch, layers=2, seed=0):
    """(ops, buffers, input case, weights of op 0): two layers on ping-pong buffers."""
    bf = torch.bfloat16
    xc = make_case(M, D, D, seed=seed + 999)
    x = to_dev16(xc.x, BF16)
    A = torch.empty(M, QKV, dtype=bf, device="cuda")
    B = torch.empty(M, D, dtype=bf, device="cuda")
    GU = torch.empty(M, 2 * H, dtype=bf, device="cuda")
    Hb = torch.empty(M, H, dtype=bf, device="cuda")
    C = [torch.empty(M, D, dtype=bf, device="cuda") for _ in range(2)]
    ops, first = [], None
    inp = x
    for li in range(layers):
        shapes = [(QKV, D, inp, A), (D, QKV, A, B), (2 * H, D, B, GU)]
        for k, (N, K, src, dst) in enumerate(shapes):
            c, w, s, b = weights(torch, N, K, seed + 10 * li + k)
            if first is None:
                first = (c, w, s, b)
            ops.append({"kind": "qmm", "x": src, "y": dst, "w": w, "scales": s, "biases": b,
                        "N": N, "K": K})
        ops.append({"kind": "silu_mul", "x": GU, "y": Hb, "N": H})
        c, w, s, b = weights(torch, D, H, seed + 10 * li + 5)
        out = C[li % 2]
        ops.append({"kind": "qmm", "x": Hb, "y": out, "w": w, "scales": s, "biases": b,
                    "N": D, "K": H})
        inp = out
    return ops, x, xc, first


def run_one_by_one(torch, ctx, ops):
    """The same ops as separate calls; returns a copy of every op's output."""
    outs = []
    for o in ops:
        if o["kind"] == "qmm":
            ctx.qmm(o["x"], o["w"], o["scales"], o["biases"], 4, 64, out=o["y"])
        elif o["kind"] == "qmm_silu_gate_up":
            ctx.qmm_silu_gate_up(o["x"], o["w"], o["scales"], o["biases"], 4, 64, out=o["y"])
        else:
            ctx.silu_mul(o["x"], o["y"])
        torch.cuda.synchronize()
        outs.append(o["y"].clone())
    return outs


def test_chain_plan_uses_a_reduce_split(ctx):
    p = ctx.plan(M, D, H, 4, 64)
    assert p["nkb"] == 2 and p["reduce"] == 1


def test_chain_matches_calls_one_by_one(ctx, oracle):
    import torch
    ops, x, xc, (c0, *_r) = build(torch)
    announce("chain: one-by-one reference")
    ref = run_one_by_one(torch, ctx, ops)
    # op 0 against the oracle
    case0 = type(c0)(x=xc.x, w=c0.w, scales=c0.scales, biases=c0.biases, M=M, N=c0.N, K=c0.K,
                     bits=4, gs=64, xdt=BF16, sdt=BF16)
    rel, ok = tolerance_check(download(ref[0]), oracle.qmm_f64(case0))
    assert rel <= 1e-2 and ok
    chain = ctx.chain(M, 4, 64, ops)
    for rep in range(3):
        for o in ops:
            o["y"].fill_(0)
        announce(f"chain launch {rep}")
        chain.launch()
        torch.cuda.synchronize()
        assert not chain.failed()
        # the last writer of each buffer is the last op that names it
        last = {}
        for j, o in enumerate(ops):
            last[id(o["y"])] = j
        for j, o in enumerate(ops):
            if last[id(o["y"])] == j:
                assert torch.equal(o["y"].view(torch.int16), ref[j].view(torch.int16)), (rep, j)
    chain.close()


def test_chain_replays_in_a_graph(ctx):
    import torch
    ops, x, xc, _ = build(torch, layers=1, seed=3)
    chain = ctx.chain(M, 4, 64, ops)
    stream = torch.cuda.Stream()
    announce("chain graph capture")
    ctx.graph_begin(stream)
    chain.launch(stream)
    graph = ctx.graph_end(stream)
    for rep in range(3):
        x.copy_(torch.randn(M, D, device="cuda").to(torch.bfloat16))
        torch.cuda.synchronize()
        ref = run_one_by_one(torch, ctx, ops)
        for o in ops:
            o["y"].fill_(0)
        torch.cuda.synchronize()
        announce(f"chain graph replay {rep}")
        graph.launch(stream)
        stream.synchronize()
        assert not chain.failed()
        assert torch.equal(ops[-1]["y"].view(torch.int16), ref[-1].view(torch.int16)), rep
    graph.close()
    chain.close()


def test_chain_wait_timeout_sets_the_error_flag_and_ends(ctx):
    import torch
    ops, x, xc, _ = build(torch, layers=1, seed=5)
    ref = run_one_by_one(torch, ctx, ops)
    chain = ctx.chain(M, 4, 64, ops)
    chain.set_timeout(0)
    announce("chain with a zero wait limit")
    chain.launch()
    torch.cuda.synchronize()
    assert chain.failed()
    chain.reset()
    chain.set_timeout(100_000_000)
    announce("chain after reset")
    chain.launch()
    torch.cuda.synchronize()
    assert not chain.failed()
    assert torch.equal(ops[-1]["y"].view(torch.int16), ref[-1].view(torch.int16))
    chain.close()


def test_independent_ops_match_calls_one_by_one(ctx):
    """q, k, v and o-like ops that all read the layer input, marked independent, plus a
    dependent op and a reduce split followed by an op marked independent (which must then
    wait anyway): every output bit-identical to the ops run one by one, over repeated
    launches."""
    import torch
    bf = torch.bfloat16
    xc = make_case(M, D, D, seed=77)
    x = to_dev16(xc.x, BF16)
    outs = [torch.empty(M, n, dtype=bf, device="cuda") for n in (QKV, D, D, D, D, D)]
    shapes = [(QKV, D, x, 0, False), (D, D, x, 1, True), (D, D, x, 2, True),
              (D, QKV, outs[0], 3, False), (D, D, x, 4, True)]
    ops = []
    for k, (N, K, src, oi, ind) in enumerate(shapes):
        c, w, s, b = weights(torch, N, K, 50 + k)
        ops.append({"kind": "qmm", "x": src, "y": outs[oi], "w": w, "scales": s, "biases": b,
                    "N": N, "K": K, "independent": ind})
    # a reduce split, then an op marked independent that reads its output
    hb = torch.randn(M, H, device="cuda").to(bf)
    c, w, s, b = weights(torch, D, H, 60)
    ops.append({"kind": "qmm", "x": hb, "y": outs[5], "w": w, "scales": s, "biases": b,
                "N": D, "K": H, "independent": True})
    tail = torch.empty(M, D, dtype=bf, device="cuda")
    c, w, s, b = weights(torch, D, D, 61)
    ops.append({"kind": "qmm", "x": outs[5], "y": tail, "w": w, "scales": s, "biases": b,
                "N": D, "K": D, "independent": True})
    ref = run_one_by_one(torch, ctx, ops)
    chain = ctx.chain(M, 4, 64, ops)
    for rep in range(3):
        for o in ops:
            o["y"].fill_(0)
        announce(f"independent chain launch {rep}")
        chain.launch()
        torch.cuda.synchronize()
        assert not chain.failed()
        for j, o in enumerate(ops):
            assert torch.equal(o["y"].view(torch.int16), ref[j].view(torch.int16)), (rep, j)
    chain.close()


def test_chain_with_the_gate_up_epilogue(ctx):
    """A layer whose MLP is the fused gate|up epilogue then down: bit-identical to the calls."""
    import torch
    bf = torch.bfloat16
    x = to_dev16(make_case(M, D, D, seed=91).x, BF16)
    A = torch.empty(M, QKV, dtype=bf, device="cuda")
    Hb = torch.empty(M, H, dtype=bf, device="cuda")
    out = torch.empty(M, D, dtype=bf, device="cuda")
    ops = []
    c, w, s, b = weights(torch, QKV, D, 92)
    ops.append({"kind": "qmm", "x": x, "y": A, "w": w, "scales": s, "biases": b, "N": QKV, "K": D})
    c, w, s, b = weights(torch, 2 * H, QKV, 93)      # read as an interleaved gate|up weight
    ops.append({"kind": "qmm_silu_gate_up", "x": A, "y": Hb, "w": w, "scales": s, "biases": b,
                "N": 2 * H, "K": QKV})
    c, w, s, b = weights(torch, D, H, 94)
    ops.append({"kind": "qmm", "x": Hb, "y": out, "w": w, "scales": s, "biases": b, "N": D, "K": H})
    ref = run_one_by_one(torch, ctx, ops)
    chain = ctx.chain(M, 4, 64, ops)
    for rep in range(2):
        for o in ops:
            o["y"].fill_(0)
        announce(f"gate|up chain launch {rep}")
        chain.launch()
        torch.cuda.synchronize()
        assert not chain.failed()
        for j, o in enumerate(ops):
            assert torch.equal(o["y"].view(torch.int16), ref[j].view(torch.int16)), (rep, j)
    chain.close()


def test_chain_rejects_what_it_cannot_run(ctx):
    import torch
    ops, x, xc, _ = build(torch, layers=1)
    with pytest.raises(dflash_qmm.DfqError):
        ctx.chain(9, 4, 64, ops)                       # more than 8 rows
    with pytest.raises(dflash_qmm.DfqError):
        ctx.chain(M, 4, 64, [ops[3]] + ops[:3])        # op 0 must be a qmm
    bad = dict(ops[0], K=D - 128)                       # K not a multiple of 8 groups
    with pytest.raises(dflash_qmm.DfqError):
        ctx.chain(M, 4, 64, [bad])
