"""Graph capture of a layer's matmul chain, and one workspace shared across shapes."""
import pytest
import torch

from gpu_util import announce, upload
from oracle.qmm_oracle import make_case

pytestmark = pytest.mark.gpu

# One verify-pass layer at reduced width: q, k, v, o, gate, up, down (K, N).
LAYER = [(1024, 1024), (1024, 256), (1024, 256), (1024, 1024), (1024, 2816), (1024, 2816),
         (2816, 1024)]


def test_graph_replays_match_eager(ctx):
    dev = "cuda"
    layers = []
    for i, (K, N) in enumerate(LAYER):
        c = make_case(8, N, K, bits=4, gs=64, seed=40 + i)
        x, w, s, b, _ = upload(c)
        layers.append((x, w, s, b, torch.empty(8, N, dtype=torch.bfloat16, device=dev), K, N))
    need = max(ctx.workspace_bytes(8, N, K, 4, 64) for (K, N) in LAYER)
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=dev)
    stream = torch.cuda.Stream()

    def enqueue():
        for (x, w, s, b, y, K, N) in layers:
            ctx.qmm(x, w, s, b, 4, 64, out=y, ws=ws, stream=stream)

    announce("graph eager reference")
    with torch.cuda.stream(stream):
        enqueue()
    torch.cuda.synchronize()
    eager = [l[4].clone() for l in layers]
    for l in layers:
        l[4].zero_()
    torch.cuda.synchronize()
    ctx.graph_begin(stream)
    enqueue()
    g = ctx.graph_end(stream)
    for rep in range(3):
        announce(f"graph replay {rep}")
        for l in layers:
            l[4].fill_(7.0)      # eager work between replays
        torch.cuda.synchronize()
        g.launch(stream)
        torch.cuda.synchronize()
        for e, l in zip(eager, layers):
            assert torch.equal(e.view(torch.int16), l[4].view(torch.int16)), f"replay {rep}"
    g.close()


def test_composed_layer_graphs_match_eager(ctx):
    """Three layers captured one graph each, chained through their inputs (each layer reads
    the previous layer's output), composed into one graph (dfq_graph_compose): every replay
    equals the eager chain, with eager work and synchronisations between replays, and the
    parts still replay on their own afterwards."""
    dev = "cuda"
    K = 1024
    chain = []
    x0 = upload(make_case(8, K, K, bits=4, gs=64, seed=70))[0]
    for i, N in enumerate((K, 2048, K)):
        kin = K if i != 2 else 2048
        c = make_case(8, N, kin, bits=4, gs=64, seed=71 + i)
        _, w, s, b, _ = upload(c)
        chain.append((w, s, b, torch.empty(8, N, dtype=torch.bfloat16, device=dev), kin, N))
    need = max(ctx.workspace_bytes(8, N, kin, 4, 64) for (_, _, _, _, kin, N) in chain)
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=dev)
    stream = torch.cuda.Stream()

    def layer(i):
        w, s, b, y, kin, N = chain[i]
        inp = x0 if i == 0 else chain[i - 1][3]
        ctx.qmm(inp, w, s, b, 4, 64, out=y, ws=ws, stream=stream)

    announce("composed graphs: eager reference")
    with torch.cuda.stream(stream):
        for i in range(3):
            layer(i)
    torch.cuda.synchronize()
    eager = [c[3].clone() for c in chain]
    parts = []
    for i in range(3):
        ctx.graph_begin(stream)
        layer(i)
        parts.append(ctx.graph_end(stream))
    fwd = ctx.graph_compose(parts)
    for rep in range(3):
        announce(f"composed graphs: replay {rep}")
        for c in chain:
            c[3].fill_(5.0)
        torch.cuda.synchronize()
        fwd.launch(stream)
        torch.cuda.synchronize()
        for i, (e, c) in enumerate(zip(eager, chain)):
            assert torch.equal(e.view(torch.int16), c[3].view(torch.int16)), (rep, i)
    announce("composed graphs: parts on their own")
    for c in chain:
        c[3].fill_(5.0)
    torch.cuda.synchronize()
    for gr in parts:
        gr.launch(stream)
    torch.cuda.synchronize()
    for e, c in zip(eager, chain):
        assert torch.equal(e.view(torch.int16), c[3].view(torch.int16))
    fwd.close()
    for gr in parts:
        gr.close()


def test_one_workspace_serves_every_shape(ctx):
    """Each call leaves the workspace zero, so shapes can alternate on one workspace."""
    shapes = [(8, 48, 16384), (1, 5000, 12288), (8, 17408, 5120), (8, 48, 16384)]
    cases = [make_case(M, N, K, bits=4, gs=64, seed=N + K) for (M, N, K) in shapes]
    need = max(ctx.workspace_bytes(c.M, c.N, c.K, 4, 64) for c in cases)
    shared = torch.zeros(need, dtype=torch.uint8, device="cuda")
    for c in cases:
        x, w, s, b, _ = upload(c)
        announce(f"shared workspace M={c.M} N={c.N} K={c.K}")
        fresh = torch.zeros(need, dtype=torch.uint8, device="cuda")
        y1 = ctx.qmm(x, w, s, b, 4, 64, ws=shared)
        y2 = ctx.qmm(x, w, s, b, 4, 64, ws=fresh)
        torch.cuda.synchronize()
        assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
        assert int(shared.count_nonzero().item()) == 0


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_silu_mul_matches_oracle(ctx, dt):
    import numpy as np
    from gpu_util import download, to_dev16
    from oracle.qmm_oracle import BF16, F16, silu_mul_f64, to_bits
    code = BF16 if dt == "bf16" else F16
    rng = np.random.default_rng(11)
    M, N = 8, 1003
    g = rng.normal(0.0, 2.0, size=(M, N))
    u = rng.normal(0.0, 1.0, size=(M, N))
    gu_bits = to_bits(np.concatenate([g, u], axis=1), code)
    gu = to_dev16(gu_bits, code)
    announce(f"silu_mul {dt} M={M} N={N}")
    h = download(ctx.silu_mul(gu))
    torch.cuda.synchronize()
    ref = silu_mul_f64(gu_bits, code)
    ulp = 2.0 ** -8 if code == BF16 else 2.0 ** -11
    assert np.all(np.abs(h - ref) <= 2 * ulp * np.abs(ref) + 1e-6)


def test_fused_mlp_chain_matches_oracle(ctx):
    """gate||up as one matmul (N = 2*hidden), the SiLU-mul, then down: each stage checked
    against the oracle on the previous stage's device output, and a graph replay of the
    chain against the eager run."""
    import numpy as np
    from gpu_util import download
    from oracle.qmm_oracle import BF16, make_case, qmm_f64, silu_mul_f64
    D, H = 512, 768
    cg = make_case(8, 2 * H, D, bits=4, gs=64, seed=71)     # rows 0..H-1 gate, H.. up
    cd = make_case(8, D, H, bits=4, gs=64, seed=72)
    x, wg, sg, bg, _ = upload(cg)
    _, wd, sd, bd, _ = upload(cd)
    ws = torch.zeros(max(ctx.workspace_bytes(8, 2 * H, D, 4, 64),
                         ctx.workspace_bytes(8, D, H, 4, 64), 256), dtype=torch.uint8,
                     device="cuda")
    gu = torch.empty(8, 2 * H, dtype=torch.bfloat16, device="cuda")
    h = torch.empty(8, H, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(8, D, dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.Stream()

    def chain():
        ctx.qmm(x, wg, sg, bg, 4, 64, out=gu, ws=ws, stream=stream)
        ctx.silu_mul(gu, h, stream=stream)
        ctx.qmm(h, wd, sd, bd, 4, 64, out=y, ws=ws, stream=stream)

    announce("fused mlp chain eager")
    with torch.cuda.stream(stream):
        chain()
    torch.cuda.synchronize()
    gu_bits = gu.view(torch.int16).cpu().numpy().view(np.uint16)
    h_bits = h.view(torch.int16).cpu().numpy().view(np.uint16)
    ref_gu = qmm_f64(cg.x, BF16, cg.w, cg.scales, cg.biases, BF16, 4, 64)
    ref_h = silu_mul_f64(gu_bits, BF16)
    ref_y = qmm_f64(h_bits, BF16, cd.w, cd.scales, cd.biases, BF16, 4, 64)
    for got, ref in ((download(gu), ref_gu), (download(h), ref_h), (download(y), ref_y)):
        assert np.max(np.abs(got - ref)) <= 1e-2 * max(np.max(np.abs(ref)), 1.0)
    eager = y.clone()
    ctx.graph_begin(stream)
    chain()
    gr = ctx.graph_end(stream)
    for rep in range(2):
        announce(f"fused mlp chain replay {rep}")
        y.fill_(3.0)
        torch.cuda.synchronize()
        gr.launch(stream)
        torch.cuda.synchronize()
        assert torch.equal(eager.view(torch.int16), y.view(torch.int16))
    gr.close()


@pytest.mark.parametrize("dt,M,V", [("bf16", 8, 151936), ("f16", 3, 1000), ("bf16", 1, 4097),
                                    ("bf16", 5, 3001), ("f16", 16, 20000)])
def test_argmax_accept_matches_oracle(ctx, dt, M, V):
    import numpy as np
    from gpu_util import to_dev16
    from oracle.qmm_oracle import BF16, F16, argmax_accept, to_bits
    code = BF16 if dt == "bf16" else F16
    rng = np.random.default_rng(M * 7 + V)
    a = rng.normal(0.0, 3.0, size=(M, V)).astype(np.float32)
    a[0, V // 3] = a[0, (2 * V) // 3] = 50.0            # a tie: the first index wins
    if M > 2:
        a[2, :] = np.nan
        a[2, V - 1] = -7.0                               # one number among NaNs
    if M > 4:
        a[3, :] = -np.inf
        a[3, V // 2] = -1e30 if dt == "bf16" else -60000.0   # the one finite value wins
        a[4, 5] = np.inf                                 # +inf beats every finite logit
    bits = to_bits(a, code)
    logits = to_dev16(bits, code)
    want_tokens, _ = argmax_accept(bits, code)
    ws = torch.zeros(256, dtype=torch.uint8, device="cuda")
    for agree in range(M):                               # proposals matching the first `agree`
        props = want_tokens[: M - 1].copy()
        if agree < M - 1:
            props[agree] = (props[agree] + 1) % V
        _, want_acc = argmax_accept(bits, code, props)
        announce(f"argmax_accept {dt} M={M} V={V} agree={agree}")
        p_dev = torch.from_numpy(props.astype(np.int32)).cuda() if M > 1 else None
        tokens, acc = ctx.argmax_accept(logits, p_dev, ws=ws)
        torch.cuda.synchronize()
        assert tokens.cpu().numpy().tolist() == want_tokens.tolist()
        assert int(acc.item()) == want_acc == min(agree, M - 1)
        assert int(ws.count_nonzero().item()) == 0       # the workspace is zero again
