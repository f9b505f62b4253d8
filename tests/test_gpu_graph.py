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
