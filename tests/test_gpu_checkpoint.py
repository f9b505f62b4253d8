"""MLX checkpoint -> device buffers -> the drop-in layers, on the GPU.

A sharded checkpoint directory (config.json with per-layer quantisation) is loaded through
dfq_checkpoint_load_model; the device copies must equal the file bytes, and the loaded
layers, after dfq_enable_small_m_quantized_matmul, must match the oracle on the same
inputs (max rel err 1e-2, as the parity tests).
"""
import time

import numpy as np
import pytest

import dflash_qmm
from ckpt_util import case, write_model_dir
from gpu_util import announce, download, to_dev16
from oracle.qmm_oracle import BF16, make_case, tolerance_check

pytestmark = pytest.mark.gpu

TOL = 1e-2

LAYERS = [
    # (prefix, N, K, bits, gs, linear bias)
    ("model.layers.0.self_attn.q_proj", 4096, 1024, 4, 64, False),
    ("model.layers.0.self_attn.k_proj", 512, 1024, 4, 64, False),     # below the N gate
    ("model.layers.0.self_attn.o_proj", 4096, 2048, 4, 64, True),
    ("model.layers.0.mlp.down_proj", 4096, 1024, 8, 64, False),
    ("model.layers.1.mlp.gate_proj", 4096, 512, 4, 32, False),        # g32: stock path
    ("model.embed_tokens", 4096, 512, 4, 64, False),                  # filtered out
]


def build(tmp_path):
    layers = []
    for i, (prefix, N, K, bits, gs, lb) in enumerate(LAYERS):
        layers.append((prefix, case(N, K, bits=bits, gs=gs, seed=100 + i, lbias=lb), lb))
    q = {"group_size": 64, "bits": 4,
         "model.layers.0.mlp.down_proj": {"bits": 8},
         "model.layers.1.mlp.gate_proj": {"group_size": 32}}
    write_model_dir(tmp_path, layers, q, shards=2)
    return {p: c for p, c, _ in layers}


def test_checkpoint_layers_load_and_match_oracle(ctx, oracle, tmp_path):
    import torch
    cases = build(tmp_path)
    ck = dflash_qmm.Checkpoint(str(tmp_path))
    announce("checkpoint load_model")
    model = ck.load_model(ctx, want=lambda p: "embed_tokens" not in p)
    assert ck.last_loaded == len(LAYERS) - 1 and len(model) == len(LAYERS) - 1
    # device bytes are the file bytes
    for prefix in model.paths():
        leaf = model.leaf(prefix)
        for suffix, addr in ((".weight", leaf.weight), (".scales", leaf.scales),
                             (".biases", leaf.biases), (".bias", leaf.bias)):
            if addr is None:
                assert suffix == ".bias"
                continue
            want = ck.read(prefix + suffix)
            got = np.empty_like(want)
            dflash_qmm.load_library()
            dflash_qmm._check(ctx.lib.dfq_memcpy_d2h(ctx.handle, got.ctypes.data, addr,
                                                     got.size, None), "d2h")
            assert np.array_equal(got, want), prefix + suffix
    swapped = dflash_qmm.enable_small_m_quantized_matmul(model)
    # eligible: N >= 4096, K % 512 == 0, group 64, bits 4 or 8 -> q, o, down
    assert swapped == 3
    for prefix in model.paths():
        c = cases[prefix]
        leaf = model.leaf(prefix)
        assert leaf.is_small_m == (prefix.endswith(("q_proj", "o_proj", "down_proj")))
        for rows in (8, 13):
            x = make_case(rows, c.N, c.K, bits=c.bits, gs=c.gs, seed=rows).x
            announce(f"checkpoint forward {prefix} rows={rows}")
            y = leaf(to_dev16(x, BF16))
            torch.cuda.synchronize()
            assert leaf.last_took_kernel == leaf.is_small_m
            ref_case = type(c)(x=x, w=c.w, scales=c.scales, biases=c.biases, M=rows, N=c.N,
                               K=c.K, bits=c.bits, gs=c.gs, xdt=BF16, sdt=c.sdt, lbias=c.lbias)
            rel, ok = tolerance_check(download(y), oracle.qmm_f64(ref_case))
            assert rel <= TOL and ok, (prefix, rows, rel)
    # closing frees the device copies: refused while a model (or a leaf view) is alive
    with pytest.raises(RuntimeError):
        ck.close()
    del leaf, model
    import gc
    gc.collect()
    ck.close()


def test_upload_of_one_tensor(ctx, tmp_path):
    import torch
    build(tmp_path)
    ck = dflash_qmm.Checkpoint(str(tmp_path))
    name = "model.layers.0.self_attn.o_proj.bias"
    want = ck.read(name)
    dst = torch.empty(want.size // 2, dtype=torch.bfloat16, device="cuda")
    announce("checkpoint upload")
    ck.upload(ctx, name, dst)
    got = dst.view(torch.int16).cpu().numpy().view(np.uint8)
    assert np.array_equal(got, want)
    with pytest.raises(dflash_qmm.DfqError):
        ck.upload(ctx, name, dst[:10])   # too small


def test_load_rejects_invalid_layers_before_allocating(ctx, tmp_path):
    build(tmp_path)
    ck = dflash_qmm.Checkpoint(str(tmp_path))
    ck.set_quantization(8, 64, prefix="model.layers.0.self_attn.q_proj")  # wrong for the file
    with pytest.raises(dflash_qmm.DfqError) as e:
        ck.load_model(ctx)
    assert "q_proj" in str(e.value)
    model = ck.load_model(ctx, want=lambda p: "q_proj" not in p)
    assert len(model) == len(LAYERS) - 1


def test_load_rate_of_a_larger_checkpoint(ctx, tmp_path):
    """A 40-layer, ~0.5 GB checkpoint (a quarter of the gate/up rows per layer), read through
    the staging buffers; prints the rate."""
    c = case(4352, 5120, seed=5)   # a quarter of the gate/up rows: 12.5 MB per layer
    layers = [(f"model.layers.{i}.mlp.up_proj", c, False) for i in range(40)]
    write_model_dir(tmp_path, layers, {"group_size": 64, "bits": 4}, shards=4)
    ck = dflash_qmm.Checkpoint(str(tmp_path))
    total = sum(d["nbytes"] for d in ck.tensors())
    # read the files once so that the timed load measures the staging path, not the disk
    for d in ck.tensors():
        ck.read(d["name"])
    announce("checkpoint load rate")
    t0 = time.perf_counter()
    model = ck.load_model(ctx)
    dt = time.perf_counter() - t0
    print(f"[checkpoint] {total / 1e6:.1f} MB in {dt * 1e3:.1f} ms: {total / dt / 1e9:.2f} GB/s",
          flush=True)
    assert len(model) == 40
