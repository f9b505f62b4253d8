"""MLX quantised-checkpoint reading, through the C ABI (no GPU needed).

Files come from two writers: this suite's own (tests/ckpt_util.py, laid out by the
safetensors definition, also used for malformed files) and the safetensors package, so the
reader is checked against the format as the library that defines it writes it.  Layer
discovery follows MLX's loaders: a layer P is quantised when P.scales and P.weight exist,
with bits / group size from config.json's "quantization" object (per-layer entries keyed by
P override the top level); SmallMQuantizedMatmul.swift:245-248 names the fields shared.
"""
import json
import os
import struct

import numpy as np
import pytest

import dflash_qmm
from ckpt_util import case, layer_entries, write_model_dir, write_safetensors
from oracle.qmm_oracle import BF16, F16


def open_ck(path):
    return dflash_qmm.Checkpoint(str(path))


def expect_open_error(path, needle):
    with pytest.raises(dflash_qmm.DfqError) as e:
        open_ck(path)
    assert e.value.status == 2 or e.value.status == 1
    assert needle in str(e.value), str(e.value)


# ---- headers ------------------------------------------------------------------------------

def test_reads_files_written_by_the_safetensors_package(tmp_path):
    import torch
    from safetensors.torch import save_file
    c = case(48, 256, seed=3)
    t = {
        "a.weight": torch.from_numpy(c.w.view(np.int32)).view(torch.uint32)
        if hasattr(torch, "uint32") else torch.from_numpy(c.w.view(np.int32)),
        "a.scales": torch.from_numpy(c.scales.view(np.int16)).view(torch.bfloat16),
        "a.biases": torch.from_numpy(c.biases.view(np.int16)).view(torch.bfloat16),
        "norm.weight": torch.ones(7, dtype=torch.float16),
        "scalar": torch.tensor(2.5, dtype=torch.float32),
    }
    p = tmp_path / "m.safetensors"
    save_file(t, str(p), metadata={"format": "mlx"})
    ck = open_ck(p)
    assert ck.format == "mlx"
    info = {d["name"]: d for d in ck.tensors()}
    assert set(info) == set(t)
    assert info["a.scales"]["dtype"] == "BF16" and info["a.scales"]["shape"] == (48, 4)
    assert info["norm.weight"]["dtype"] == "F16" and info["scalar"]["shape"] == ()
    assert info["a.weight"]["dtype"] in ("U32", "I32")
    assert info["a.weight"]["shape"] == (48, 32)
    # bytes as stored, at the recorded offsets
    assert np.array_equal(ck.read("a.scales").view(np.uint16).reshape(48, 4), c.scales)
    assert np.array_equal(ck.read("a.weight").view(np.uint32).reshape(48, 32), c.w)
    raw = open(p, "rb").read()
    for d in info.values():
        assert raw[d["offset"]:d["offset"] + d["nbytes"]] == ck.read(d["name"]).tobytes()


def test_own_writer_matches_the_package_byte_for_byte_in_data(tmp_path):
    from safetensors.numpy import load_file
    c = case(32, 128, seed=4)
    p = tmp_path / "x.safetensors"
    write_safetensors(p, [("l.weight", "U32", c.w.shape, c.w.tobytes())])
    got = load_file(str(p))["l.weight"]
    assert got.dtype == np.uint32 and np.array_equal(got, c.w)


def test_unicode_and_escapes_in_names(tmp_path):
    p = tmp_path / "u.safetensors"
    name = 'layér/中.\U0001f600"q\\'
    write_safetensors(p, [(name, "U8", (3,), b"abc")])
    ck = open_ck(p)
    assert [d["name"] for d in ck.tensors()] == [name]
    assert ck.read(name).tobytes() == b"abc"


def test_empty_tensors_and_zero_dims(tmp_path):
    p = tmp_path / "e.safetensors"
    write_safetensors(p, [("z", "F32", (0, 5), b""), ("one", "F32", (1,), b"\0\0\x80\x3f")])
    ck = open_ck(p)
    assert ck.tensor("z")["nbytes"] == 0 and ck.tensor("z")["shape"] == (0, 5)
    assert ck.read("one").view(np.float32)[0] == 1.0


@pytest.mark.parametrize("kind,needle", [
    ("short", "too short"),
    ("hlen", "does not fit"),
    ("json", "not JSON"),
    ("notobj", "not a JSON object"),
    ("dtype", "unsupported dtype"),
    ("size", "its shape needs"),
    ("past", "past the end"),
    ("offsets", "bad data_offsets"),
    ("fields", "lacks dtype"),
    ("trailing", "not JSON"),
])
def test_malformed_headers_are_rejected(tmp_path, kind, needle):
    p = tmp_path / f"{kind}.safetensors"
    good = [("t", "F32", (2,), b"\0" * 8)]
    if kind == "short":
        p.write_bytes(b"\x01\x02")
    elif kind == "hlen":
        p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    elif kind == "json":
        write_safetensors(p, good, header_override='{"t": {"dtype": "F32", ')
    elif kind == "notobj":
        write_safetensors(p, good, header_override="[1, 2]")
    elif kind == "dtype":
        write_safetensors(p, [("t", "Q7", (2,), b"\0" * 8)])
    elif kind == "size":
        write_safetensors(p, good, header_override=json.dumps(
            {"t": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}))
    elif kind == "past":
        write_safetensors(p, good, header_override=json.dumps(
            {"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}))
    elif kind == "offsets":
        write_safetensors(p, good, header_override=json.dumps(
            {"t": {"dtype": "F32", "shape": [2], "data_offsets": [8, 0]}}))
    elif kind == "fields":
        write_safetensors(p, good, header_override=json.dumps({"t": {"dtype": "F32"}}))
    elif kind == "trailing":
        write_safetensors(p, good, header_override=json.dumps(
            {"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}) + " }")
    expect_open_error(p, needle)


def test_missing_path_and_empty_directory(tmp_path):
    with pytest.raises(dflash_qmm.DfqError):
        open_ck(tmp_path / "nope.safetensors")
    expect_open_error(tmp_path, "no .safetensors files")


# ---- layers and quantisation parameters ---------------------------------------------------

def sample_dir(root, shards=1):
    layers = [
        ("model.layers.0.self_attn.q_proj", case(64, 512, seed=1), False),
        ("model.layers.0.mlp.down_proj", case(32, 256, bits=8, seed=2), False),
        ("model.layers.0.self_attn.o_proj", case(48, 256, seed=3, lbias=True), True),
        ("model.layers.1.mlp.gate_proj", case(40, 128, gs=32, seed=5), False),
        ("model.embed_tokens", case(16, 128, seed=6), False),
    ]
    norm = np.ones(64, np.uint16) * 0x3F80  # bf16 1.0
    extra = [("model.norm.weight", "BF16", (64,), norm.tobytes())]
    q = {"group_size": 64, "bits": 4,
         "model.layers.0.mlp.down_proj": {"group_size": 64, "bits": 8},
         "model.layers.1.mlp.gate_proj": {"group_size": 32}}
    names = write_model_dir(root, layers, q, extra=extra, shards=shards)
    return layers, names


@pytest.mark.parametrize("shards", [1, 3])
def test_layers_take_bits_and_group_size_from_config(tmp_path, shards):
    layers, names = sample_dir(tmp_path, shards=shards)
    ck = open_ck(tmp_path)
    L = {d["prefix"]: d for d in ck.layers()}
    assert list(L) == sorted(p for p, _, _ in layers)   # sorted; norm.weight is no layer
    for prefix, c, bias in layers:
        d = L[prefix]
        assert d["valid"], d["problem"]
        assert (d["out_features"], d["in_features"], d["bits"], d["group_size"]) == \
            (c.N, c.K, c.bits, c.gs)
        assert d["has_biases"] and d["has_bias"] == bias
    assert len(ck.tensors()) == sum(3 + b for _, _, b in layers) + 1
    shard_of = {d["name"]: d["shard"] for d in ck.tensors()}
    assert max(shard_of.values()) == shards - 1
    # the data of every layer reads back as written, whichever shard holds it
    for prefix, c, bias in layers:
        assert np.array_equal(ck.read(prefix + ".weight").view(np.uint32).reshape(c.w.shape), c.w)
        assert np.array_equal(ck.read(prefix + ".biases").view(np.uint16).reshape(c.biases.shape),
                              c.biases)


def test_shapes_are_checked_against_bits_and_group_size(tmp_path):
    c = case(32, 256, seed=7)
    bad_groups = c.scales[:, :2].copy()
    entries = [("a.weight", "U32", c.w.shape, c.w.tobytes()),
               ("a.scales", "BF16", bad_groups.shape, bad_groups.tobytes()),
               ("a.biases", "BF16", bad_groups.shape, bad_groups.tobytes()),
               ("b.weight", "U32", c.w.shape, c.w.tobytes()),
               ("b.scales", "BF16", c.scales.shape, c.scales.tobytes()),
               ("b.biases", "F16", c.biases.shape, c.biases.tobytes()),
               ("c.weight", "F32", c.w.shape, c.w.tobytes()),
               ("c.scales", "BF16", c.scales.shape, c.scales.tobytes()),
               ("c.biases", "BF16", c.biases.shape, c.biases.tobytes()),
               ("d.weight", "U32", c.w.shape, c.w.tobytes()),
               ("d.scales", "BF16", c.scales.shape, c.scales.tobytes())]
    p = tmp_path / "m.safetensors"
    write_safetensors(p, entries)
    ck = open_ck(p)
    assert all("no bits" in d["problem"] for d in ck.layers())   # no config.json
    ck.set_quantization(4, 64)
    P = {d["prefix"]: d for d in ck.layers()}
    assert P["a"]["problem"].startswith("in_features 256 with group size 64 needs 4 groups")
    assert "biases differ" in P["b"]["problem"]
    assert "not a 2-D U32" in P["c"]["problem"]
    assert "without biases" in P["d"]["problem"]
    # the same words read as 8-bit g64: in_features 128 in 2 groups -> a fits
    ck.set_quantization(8, 64, prefix="a")
    a = [d for d in ck.layers() if d["prefix"] == "a"][0]
    assert a["valid"] and (a["in_features"], a["bits"], a["group_size"]) == (128, 8, 64)


def test_unsupported_modes_and_bits_are_reported(tmp_path):
    layers = [("p", case(16, 128, seed=1), False), ("q", case(16, 128, seed=2), False),
              ("r", case(16, 128, seed=3), False)]
    q = {"group_size": 64, "bits": 4, "q": {"bits": 3}, "r": False}
    write_model_dir(tmp_path / "a", layers, q)
    P = {d["prefix"]: d for d in open_ck(tmp_path / "a").layers()}
    assert P["p"]["valid"]
    assert "bits 3" in P["q"]["problem"]
    assert "off for this layer" in P["r"]["problem"]
    write_model_dir(tmp_path / "b", layers[:1], {"group_size": 32, "bits": 4, "mode": "mxfp4"})
    (d,) = open_ck(tmp_path / "b").layers()
    assert "not affine" in d["problem"]


def test_quantization_config_key_is_read_when_quantization_is_absent(tmp_path):
    c = case(16, 256, bits=8, gs=128, seed=9)
    write_model_dir(tmp_path, [("lin", c, False)], {"group_size": 1, "bits": 1},
                    config_extra=None)
    cfg = json.load(open(tmp_path / "config.json"))
    cfg.pop("quantization")
    cfg["quantization_config"] = {"group_size": 128, "bits": 8}
    json.dump(cfg, open(tmp_path / "config.json", "w"))
    (d,) = open_ck(tmp_path).layers()
    assert d["valid"] and (d["bits"], d["group_size"], d["in_features"]) == (8, 128, 256)


def test_a_name_in_two_shards_is_rejected(tmp_path):
    c = case(16, 128, seed=1)
    for i in (1, 2):
        write_safetensors(tmp_path / f"model-0000{i}-of-00002.safetensors",
                          layer_entries("dup", c))
    expect_open_error(tmp_path, "appears twice")


def test_directory_prefers_model_shards(tmp_path):
    c = case(16, 128, seed=1)
    write_safetensors(tmp_path / "model.safetensors", layer_entries("a", c))
    write_safetensors(tmp_path / "adapters.safetensors", layer_entries("b", c))
    names = [d["name"] for d in open_ck(tmp_path).tensors()]
    assert all(n.startswith("a.") for n in names)
    os.remove(tmp_path / "model.safetensors")
    names = [d["name"] for d in open_ck(tmp_path).tensors()]
    assert all(n.startswith("b.") for n in names)


def test_f16_layers(tmp_path):
    c = case(24, 256, seed=11, sdt=F16)
    write_model_dir(tmp_path, [("h", c, False)], {"group_size": 64, "bits": 4})
    (d,) = open_ck(tmp_path).layers()
    assert d["valid"] and d["dtype"] == F16 and BF16 != F16
