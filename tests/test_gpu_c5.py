"""Full-size parity of the 64-layer verify forward's operators (the C5 configuration): every
projection shape of one layer and the LM head at 4-bit group 64, bf16, against the fp64
oracle; one full-size fused layer captured as one HIP graph and replayed against its eager
run; and the LM head's logits through the greedy accept against the oracle's argmax.

The shapes are those of the target layers that enableSmallMQuantizedMatmul(in:) swaps
(Sources/DFlashKit/SmallMQuantizedMatmul.swift:303-317), run by the verify forward of
Sources/DFlashKit/DFlashSpeculativeGenerator.swift:389-398, whose logits go through
acceptedPrefix (:555-571).  Bar: max|y - y_ref| / max|y_ref| <= 1e-2 (bf16 out, fp32
accumulate) plus the reference test's rule max|d| <= 0.02 * max(max|ref|, 1)
(SmallMQuantizedMatmulTests.swift:74-79); graph replays and the argmax over the device's own
logits are checked bit-exact.
"""
import numpy as np
import pytest

from gpu_util import announce, download, to_dev16, upload
from oracle.qmm_oracle import (BF16, argmax_accept, from_bits, make_case, to_bits,
                               tolerance_check)

pytestmark = pytest.mark.gpu

TOL = 1e-2

# (name, N, K) of one verify-pass layer and the LM head
C5_SHAPES = [
    ("q", 5120, 5120),
    ("o", 5120, 5120),
    ("qkv", 7168, 5120),
    ("k", 1024, 5120),
    ("v", 1024, 5120),
    ("down", 5120, 17408),
    ("lm_head", 151936, 5120),
]


@pytest.mark.parametrize("M", [8, 16])
@pytest.mark.parametrize("name,N,K", C5_SHAPES)
def test_c5_projection_matches_oracle(ctx, oracle, name, N, K, M):
    seed = 500 + N + K + M
    c = make_case(M, N, K, bits=4, gs=64, seed=seed, words=True)
    announce(f"c5 {name} M={M} N={N} K={K} plan={ctx.plan(M, N, K, 4, 64)}")
    x, w, s, b, _ = upload(c)
    y = download(ctx.qmm(x, w, s, b, 4, 64))
    rel, ok = tolerance_check(y, oracle.qmm_f64(c))
    assert rel <= TOL and ok, f"{name} M={M}: max rel err {rel:.3e}"


def bf16_ulp(v):
    """bf16 spacing at |v| (8 significant bits)."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def test_c5_lm_head_feeds_the_greedy_accept(ctx, oracle):
    """LM head logits (151936 x 5120) on the device, then dfq_argmax_accept on them:
    tokens equal the first-index argmax of the device's own logits bit for bit, and the
    oracle's argmax wherever the oracle's top two logits are more than one bf16 spacing
    apart (closer rows may round either way and are skipped; most rows are clear)."""
    import torch
    M, V, K = 8, 151936, 5120
    c = make_case(M, V, K, bits=4, gs=64, seed=4242, words=True)
    x, w, s, b, _ = upload(c)
    announce("c5 lm_head -> argmax_accept")
    logits = ctx.qmm(x, w, s, b, 4, 64)
    torch.cuda.synchronize()
    ref = oracle.qmm_f64(c)
    rel, ok = tolerance_check(download(logits), ref)
    assert rel <= TOL and ok, f"lm_head: max rel err {rel:.3e}"
    lbits = logits.view(torch.int16).cpu().numpy().view(np.uint16)
    dev_tokens, _ = argmax_accept(lbits, BF16)
    top2 = np.sort(ref, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 1.01 * bf16_ulp(top2[:, 1])
    ref_tokens = np.argmax(ref, axis=1)
    assert clear.sum() >= M // 2, "too few rows with a clear maximum to check"
    # proposals agree with the oracle for the first 4 verify rows, then differ
    props = ref_tokens[: M - 1].astype(np.int32).copy()
    props[4] = (props[4] + 1) % V
    p_dev = torch.from_numpy(props).cuda()
    ws = torch.zeros(256, dtype=torch.uint8, device="cuda")
    tokens, acc = ctx.argmax_accept(logits, p_dev, ws=ws)
    torch.cuda.synchronize()
    got = tokens.cpu().numpy()
    assert got.tolist() == dev_tokens.tolist()
    for m in range(M):
        if clear[m]:
            assert got[m] == ref_tokens[m], f"row {m}: {got[m]} vs oracle {ref_tokens[m]}"
    _, want_acc = argmax_accept(lbits, BF16, props)
    assert int(acc.item()) == want_acc
    if clear[:5].all():
        assert want_acc == 4


def test_c5_fused_layer_graph_matches_eager_and_oracle(ctx, oracle):
    """One full-size fused layer (q|k|v 7168x5120, o 5120x5120, gate|up 2x17408x5120 with
    the SiLU-mul epilogue, down 5120x17408 reading its output), each op against the oracle on
    the device's own input, then captured as one HIP graph and replayed three times, with
    eager work between replays, bit-identical to the eager run."""
    import torch
    M, D, QKV, H = 8, 5120, 7168, 17408
    cq = make_case(M, QKV, D, seed=71, words=True)
    co = make_case(M, D, D, seed=72, words=True)
    cg = make_case(M, H, D, seed=73, words=True)
    cu = make_case(M, H, D, seed=74, words=True)
    cd = make_case(M, D, H, seed=75, words=True)
    for c in (co, cg, cu):
        c.x = cq.x
    x, wq, sq, bq, _ = upload(cq)
    _, wo, so, bo, _ = upload(co)
    _, wg, sg, bg, _ = upload(cg)
    _, wu, su, bu, _ = upload(cu)
    _, wd, sd, bd, _ = upload(cd)
    announce("c5 fused layer: interleave gate|up")
    w_gu = ctx.interleave_gate_up(wg, wu)
    s_gu = ctx.interleave_gate_up(sg, su)
    b_gu = ctx.interleave_gate_up(bg, bu)
    shapes = [(QKV, D), (D, D), (2 * H, D), (D, H)]
    need = max(ctx.workspace_bytes(M, N, K, 4, 64) for (N, K) in shapes)
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device="cuda")
    bf = torch.bfloat16
    yq = torch.empty(M, QKV, dtype=bf, device="cuda")
    yo = torch.empty(M, D, dtype=bf, device="cuda")
    h = torch.empty(M, H, dtype=bf, device="cuda")
    yd = torch.empty(M, D, dtype=bf, device="cuda")
    stream = torch.cuda.Stream()

    def layer():
        ctx.qmm(x, wq, sq, bq, 4, 64, out=yq, ws=ws, stream=stream)
        ctx.qmm(x, wo, so, bo, 4, 64, out=yo, ws=ws, stream=stream)
        ctx.qmm_silu_gate_up(x, w_gu, s_gu, b_gu, 4, 64, out=h, ws=ws, stream=stream)
        ctx.qmm(h, wd, sd, bd, 4, 64, out=yd, ws=ws, stream=stream)

    announce("c5 fused layer eager")
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        layer()
    torch.cuda.synchronize()
    eager = [t.clone() for t in (yq, yo, h, yd)]
    for c, y in ((cq, yq), (co, yo)):
        rel, ok = tolerance_check(download(y), oracle.qmm_f64(c))
        assert rel <= TOL and ok, f"max rel err {rel:.3e}"
    g64 = oracle.qmm_f64(cg)
    u64 = oracle.qmm_f64(cu)
    gr = from_bits(to_bits(g64, BF16), BF16).astype(np.float64)
    ur = from_bits(to_bits(u64, BF16), BF16).astype(np.float64)
    rel, ok = tolerance_check(download(h), gr / (1.0 + np.exp(-gr)) * ur)
    assert rel <= TOL and ok, f"gate|up epilogue: max rel err {rel:.3e}"
    cd.x = h.view(torch.int16).cpu().numpy().view(np.uint16)
    rel, ok = tolerance_check(download(yd), oracle.qmm_f64(cd))
    assert rel <= TOL and ok, f"down: max rel err {rel:.3e}"

    torch.cuda.synchronize()
    ctx.graph_begin(stream)
    layer()
    gr_ = ctx.graph_end(stream)
    for rep in range(3):
        announce(f"c5 fused layer replay {rep}")
        for t in (yq, yo, h, yd):
            t.fill_(5.0)                                  # eager work between replays
        torch.cuda.synchronize()
        gr_.launch(stream)
        torch.cuda.synchronize()
        for e, t in zip(eager, (yq, yo, h, yd)):
            assert torch.equal(e.view(torch.int16), t.view(torch.int16)), f"replay {rep}"
        assert int(ws.count_nonzero().item()) == 0
    gr_.close()
