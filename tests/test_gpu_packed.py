"""The packed weight layout (dfq_pack_weights) and the fast kernel over it.

The pack is a byte permutation of the MLX arrays; it is checked byte for byte against a numpy
restatement of the layout (pack_reference below).  The kernels over it load the same values
into the same registers as over the MLX layout, so dfq_qmm_packed, dfq_qmm_silu_gate_up_packed
and dfq_qmm_argmax_accept_packed must equal dfq_qmm, dfq_qmm_silu_gate_up and
dfq_qmm_argmax_accept bit for bit -- the MLX-layout kernels are pinned against the oracle by
the parity, one-hot and accept tests -- across formats, dtypes, 1..16 rows, ragged N (the
pack's zero rows past N) and every split (one k-block, narrow, aligned, three k-blocks,
reduce, outputs written at the end of the workgroup).
"""
import numpy as np
import pytest

from gpu_util import announce, upload
from oracle.qmm_oracle import BF16, F16, make_case

pytestmark = pytest.mark.gpu


def pack_reference(w_words, s_bits, b_bits, N, K, bits, gs):
    """The packed layout on the CPU: unit (t, c) of 16 rows x cg groups (8; 16 at 4-bit group
    32) at (t*chunks + c) * ub; piece i of its codes holds, at 16 * (16 q + n), bytes
    64 i + 16 q of the chunk's codes of row 16 t + n; then scales (qq = 0) and biases (qq = 1)
    of row n, 2 cg bytes, at (16 qq + n) * 2 cg; rows past N zero."""
    cg = 16 if (bits, gs) == (4, 32) else 8
    ck = cg * gs
    cb = 16 * ck * bits // 8
    chunks, T = K // ck, -(-N // 16)
    wb = np.zeros((T * 16, K * bits // 8), dtype=np.uint8)
    wb[:N] = np.ascontiguousarray(w_words).view(np.uint8).reshape(N, -1)
    sb = np.zeros((T * 16, K // gs * 2), dtype=np.uint8)
    bb = np.zeros_like(sb)
    sb[:N] = np.ascontiguousarray(s_bits).view(np.uint8).reshape(N, -1)
    bb[:N] = np.ascontiguousarray(b_bits).view(np.uint8).reshape(N, -1)
    out = np.zeros((T, chunks, cb + 64 * cg), dtype=np.uint8)
    for t in range(T):
        rows = slice(16 * t, 16 * t + 16)
        for c in range(chunks):
            codes = wb[rows, c * cb // 16:(c + 1) * cb // 16]          # [16 n][cb/16]
            pieces = codes.reshape(16, cb // 1024, 4, 16)               # [n][i][q][16]
            out[t, c, :cb] = pieces.transpose(1, 2, 0, 3).reshape(-1)   # [i][q][n][16]
            sbytes = 2 * cg                                             # a row's scales
            out[t, c, cb:cb + 16 * sbytes] = sb[rows, c * sbytes:(c + 1) * sbytes].reshape(-1)
            out[t, c, cb + 16 * sbytes:] = bb[rows, c * sbytes:(c + 1) * sbytes].reshape(-1)
    return out.reshape(-1)


@pytest.mark.parametrize("N,K,bits,gs,dt", [(40, 512, 4, 64, BF16), (33, 1024, 8, 64, F16),
                                            (16, 512, 4, 32, BF16), (50, 2048, 4, 128, F16),
                                            (17, 1024, 8, 128, BF16), (100, 768, 8, 32, BF16)])
def test_pack_matches_the_layout(ctx, N, K, bits, gs, dt):
    import torch
    c = make_case(1, N, K, bits=bits, gs=gs, xdt=dt, seed=N + K)
    _, w, s, b, _ = upload(c)
    announce(f"pack N={N} K={K} bits={bits} gs={gs}")
    pw = ctx.pack(w, s, b, bits, gs)
    torch.cuda.synchronize()
    got = pw.data.cpu().numpy()
    want = pack_reference(c.w, c.scales, c.biases, N, K, bits, gs)
    assert got.size == want.size
    assert np.array_equal(got, want)


def _eq(a, b):
    import torch
    return torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16))


CASES = [  # (M, N, K, bits, gs, dtype, linear bias)
    (8, 17408, 5120, 4, 64, BF16, False),   # the headline: one k-block, pair exchange
    (1, 17408, 5120, 4, 64, BF16, False),
    (16, 17408, 5120, 4, 64, BF16, False),  # two row tiles, aligned two-k-block split
    (8, 5120, 17408, 4, 64, BF16, True),    # three k-blocks of whole tiles
    (8, 1024, 5120, 4, 64, BF16, False),    # narrow: two k-blocks, one tile each
    (12, 40000, 4096, 4, 64, F16, False),   # 12 rows, pair exchange
    (12, 17408, 5120, 4, 64, BF16, True),   # 12 rows in one k-block: 16 x items a thread
    (8, 1024, 32768, 4, 64, BF16, True),    # the reduce split's second pass
    (8, 7168, 5120, 8, 64, BF16, False),
    (5, 5120, 5120, 4, 32, BF16, True),
    (16, 333, 1024, 4, 128, F16, False),    # ragged N: zero rows past N in the last tile
    (7, 130, 1024, 8, 128, BF16, True),
    (3, 200, 512, 8, 32, F16, False),
    (8, 32768, 512, 4, 64, BF16, False),    # outputs written at the end of the workgroup
]


@pytest.mark.parametrize("case", CASES)
def test_packed_kernel_equals_the_mlx_layout(ctx, case):
    import torch
    M, N, K, bits, gs, dt, lb = case
    c = make_case(M, N, K, bits=bits, gs=gs, xdt=dt, seed=M + N + K, lbias=lb,
                  words=N * K > 4_000_000)
    x, w, s, b, lbias = upload(c)
    announce(f"packed qmm M={M} N={N} K={K} bits={bits} gs={gs} plan={ctx.plan(M, N, K, bits, gs)}")
    pw = ctx.pack(w, s, b, bits, gs)
    want = ctx.qmm(x, w, s, b, bits, gs, lbias=lbias)
    got = ctx.qmm_packed(x, pw, lbias=lbias)
    again = ctx.qmm_packed(x, pw, lbias=lbias)
    torch.cuda.synchronize()
    assert _eq(got, want) and _eq(again, want)


def test_packed_gate_up_epilogue_equals_the_mlx_layout(ctx):
    import torch
    H, K = 2048, 5120
    cg = make_case(8, H, K, bits=4, gs=64, seed=5, words=True)
    cu = make_case(8, H, K, bits=4, gs=64, seed=6, words=True)
    x, wg, sg, bg, _ = upload(cg)
    _, wu, su, bu, _ = upload(cu)
    w_gu, s_gu, b_gu = (ctx.interleave_gate_up(a, b) for a, b in ((wg, wu), (sg, su), (bg, bu)))
    announce("packed gate|up epilogue")
    want = ctx.qmm_silu_gate_up(x, w_gu, s_gu, b_gu, 4, 64)
    got = ctx.qmm_silu_gate_up_packed(x, ctx.pack(w_gu, s_gu, b_gu, 4, 64))
    torch.cuda.synchronize()
    assert _eq(got, want)


@pytest.mark.parametrize("M,V,K", [(8, 151936, 5120), (16, 32768, 512), (5, 3000, 2048)])
def test_packed_lm_head_accept_equals_the_mlx_layout(ctx, M, V, K):
    import torch
    c = make_case(M, V, K, bits=4, gs=64, seed=M + V, words=V * K > 4_000_000)
    x, w, s, b, _ = upload(c)
    props = torch.zeros(max(1, M - 1), dtype=torch.int32, device="cuda")
    announce(f"packed accept M={M} V={V} K={K}")
    pw = ctx.pack(w, s, b, 4, 64)
    lg_a = torch.empty(M, V, dtype=torch.bfloat16, device="cuda")
    lg_b = torch.empty_like(lg_a)
    ta, aa = ctx.qmm_argmax_accept(x, w, s, b, 4, 64, proposals=props, logits=lg_a)
    tb, ab = ctx.qmm_argmax_accept_packed(x, pw, proposals=props, logits=lg_b)
    tc, ac = ctx.qmm_argmax_accept_packed(x, pw, proposals=props)   # no logits written
    torch.cuda.synchronize()
    assert _eq(lg_a, lg_b)
    assert torch.equal(ta, tb) and torch.equal(ta, tc)
    assert int(aa.item()) == int(ab.item()) == int(ac.item())


def test_packed_refuses_k_without_whole_chunks(ctx):
    import ctypes
    nb = ctypes.c_size_t(7)
    assert ctx.lib.dfq_packed_bytes(64, 640, 4, 64, ctypes.byref(nb)) != 0 and nb.value == 0
    assert ctx.lib.dfq_packed_bytes(64, 1024, 4, 64, ctypes.byref(nb)) == 0
    assert nb.value == 4 * 2 * (4096 + 512)
    assert ctx.lib.dfq_packed_bytes(64, 256, 4, 32, ctypes.byref(nb)) != 0   # 16 groups a chunk
    assert ctx.lib.dfq_packed_bytes(64, 1024, 4, 32, ctypes.byref(nb)) == 0
    assert nb.value == 4 * 2 * (4096 + 1024)


# ---- the drop-in layer over the packed layout ------------------------------------------------

CK_LAYERS = [
    # (prefix, N, K, bits, gs, linear bias, scale dtype)
    ("model.layers.0.self_attn.q_proj", 4096, 1024, 4, 64, False, BF16),
    ("model.layers.0.self_attn.o_proj", 4100, 2048, 4, 64, True, BF16),   # ragged last tile
    ("model.layers.0.mlp.down_proj", 4096, 1024, 8, 64, False, BF16),
    ("model.layers.1.mlp.gate_proj", 4096, 512, 4, 32, False, BF16),      # g32: never swapped
    ("model.layers.1.mlp.up_proj", 4096, 1024, 4, 64, True, F16),         # fp16 scales
    ("model.layers.1.mlp.down_proj", 4096, 320, 4, 64, False, BF16),      # 5 groups: as stored
]


def _build_checkpoint(tmp_path):
    from ckpt_util import write_model_dir
    layers, q = [], {"group_size": 64, "bits": 4}
    for i, (prefix, N, K, bits, gs, lb, sdt) in enumerate(CK_LAYERS):
        c = make_case(8, N, K, bits=bits, gs=gs, xdt=BF16, sdt=sdt, seed=200 + i, lbias=lb)
        layers.append((prefix, c, lb))
        if bits != 4 or gs != 64:
            q[prefix] = {"bits": bits, "group_size": gs}
    write_model_dir(tmp_path, layers, q, shards=2)
    return {p: c for p, c, _ in layers}


def _d2h(ctx, addr, nbytes):
    out = np.empty(nbytes, dtype=np.uint8)
    import dflash_qmm
    dflash_qmm._check(ctx.lib.dfq_memcpy_d2h(ctx.handle, out.ctypes.data, addr, nbytes, None),
                      "d2h")
    return out


def _slices(ctx, c, x):
    """The fast kernel over the MLX arrays, 16 rows a launch (what a packed layer's stock
    path computes)."""
    import torch
    _, w, s, b, lb = upload(c)
    return torch.cat([ctx.qmm(x[r:r + 16], w, s, b, c.bits, c.gs, lbias=lb)
                      for r in range(0, x.shape[0], 16)])


def test_checkpoint_loads_packed_and_matches_the_mlx_layout(ctx, tmp_path):
    import torch
    import dflash_qmm
    from gpu_util import to_dev16
    cases = _build_checkpoint(tmp_path)
    ck = dflash_qmm.Checkpoint(str(tmp_path))
    announce("checkpoint load, MLX layout and packed")
    plain = ck.load_model(ctx)
    packed = ck.load_model(ctx, packed=True)
    assert len(plain) == len(packed) == len(CK_LAYERS)
    packs = {p for (p, N, K, bits, gs, lb, sdt) in CK_LAYERS
             if K % ((16 if (bits, gs) == (4, 32) else 8) * gs) == 0}
    for (prefix, N, K, bits, gs, lb, sdt) in CK_LAYERS:
        leaf = packed.leaf(prefix)
        assert (leaf.packed is not None) == (prefix in packs), prefix
        if prefix not in packs:
            continue
        assert leaf.weight is None and leaf.scales is None and leaf.biases is None
        assert (leaf.bias is not None) == lb
        c = cases[prefix]
        nb = ctypes_size(ctx, N, K, bits, gs)
        want = pack_reference(c.w, c.scales, c.biases, N, K, bits, gs)
        assert nb == want.size and np.array_equal(_d2h(ctx, leaf.packed, nb), want), prefix
    assert dflash_qmm.enable_small_m_quantized_matmul(plain) == \
        dflash_qmm.enable_small_m_quantized_matmul(packed) == 4
    for (prefix, N, K, bits, gs, lb, sdt) in CK_LAYERS:
        c = cases[prefix]
        a, p = plain.leaf(prefix), packed.leaf(prefix)
        assert a.is_small_m == p.is_small_m
        for rows in (1, 2, 8, 16, 17, 33):
            x = to_dev16(make_case(rows, N, K, bits=bits, gs=gs, xdt=sdt, seed=rows).x, sdt)
            announce(f"packed leaf {prefix} rows={rows}")
            ya, yp = a(x), p(x)
            took_a, took_p = a.last_took_kernel, p.last_took_kernel
            torch.cuda.synchronize()
            assert took_a == took_p
            if prefix not in packs or took_p:
                assert _eq(ya, yp), (prefix, rows)       # the same path, the same kernel
            else:
                assert _eq(yp, _slices(ctx, c, x)), (prefix, rows)
                rel = float(((yp.float() - ya.float()).abs().max() /
                             ya.float().abs().max().clamp_min(1.0)).item())
                assert rel <= 1e-2, (prefix, rows, rel)  # the stock path, another kernel
    up = packed.leaf("model.layers.1.mlp.up_proj")
    with pytest.raises(dflash_qmm.DfqError):            # fp16 scales take fp16 x
        up(torch.zeros(2, 1024, dtype=torch.bfloat16, device="cuda"))
    del a, p, up, leaf, plain, packed
    import gc
    gc.collect()
    ck.close()


def ctypes_size(ctx, N, K, bits, gs):
    import ctypes
    nb = ctypes.c_size_t()
    assert ctx.lib.dfq_packed_bytes(N, K, bits, gs, ctypes.byref(nb)) == 0
    return nb.value


def test_small_m_layer_takes_a_packed_copy(ctx):
    import torch
    import dflash_qmm
    c = make_case(8, 4096, 2048, bits=4, gs=64, seed=31, lbias=True)
    x8, w, s, b, lb = upload(c)
    stock = dflash_qmm.QuantizedLinear(ctx, w, s, b, lb, group_size=64, bits=4)
    with pytest.raises(dflash_qmm.DfqError):
        stock_h = dflash_qmm.SmallMQuantizedLinear.pack(stock)  # a stock layer has no copy
        del stock_h
    lay = dflash_qmm.SmallMQuantizedLinear(stock)
    x1 = x8[:1].contiguous()
    announce("small-M layer before the packed copy")
    before8, before1 = lay(x8), lay(x1)
    assert lay.packed is None
    lay.pack()
    lay.pack()                                           # a second call does nothing
    addr = lay.packed
    assert addr is not None and lay.packed == addr
    announce("small-M layer over its packed copy")
    after8, after1 = lay(x8), lay(x1)
    torch.cuda.synchronize()
    assert _eq(before8, after8) and lay.last_took_kernel is False   # rows=1: the stock path
    assert _eq(before1, after1)
    model = dflash_qmm.Model(layer=lay)                  # the model's handle shares the copy
    assert model.leaf("layer").packed == addr
    g32 = make_case(8, 4096, 512, bits=4, gs=32, seed=32)
    _, w2, s2, b2, _ = upload(g32)
    not_eligible = dflash_qmm.SmallMQuantizedLinear(
        dflash_qmm.QuantizedLinear(ctx, w2, s2, b2, group_size=32, bits=4))
    with pytest.raises(dflash_qmm.DfqError):
        not_eligible.pack()
    assert not_eligible.packed is None
