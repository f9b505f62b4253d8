"""Writing small MLX-layout safetensors checkpoints for the checkpoint tests.

write_safetensors lays a file out by the format's definition (8-byte little-endian header
length, a JSON header, the data), so the tests can also produce malformed files; the tests
cross-check it against files written by the safetensors package itself.
"""
import json
import os
import struct

import numpy as np

from oracle.qmm_oracle import BF16, F16, make_case

ST_NAME = {BF16: "BF16", F16: "F16"}


def write_safetensors(path, entries, metadata=None, header_override=None, pad_to=8):
    """entries: list of (name, dtype string, shape, raw bytes).  Returns the header dict."""
    header = {}
    if metadata is not None:
        header["__metadata__"] = metadata
    off = 0
    for name, dt, shape, raw in entries:
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        off += len(raw)
    text = header_override if header_override is not None else json.dumps(header)
    hb = text.encode()
    hb += b" " * ((-len(hb)) % pad_to)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for _, _, _, raw in entries:
            f.write(raw)
    return header


def layer_entries(prefix, case, bias=False):
    """The tensors of one quantised layer in MLX's layout, from an oracle case."""
    dt = ST_NAME[case.sdt]
    out = [
        (prefix + ".weight", "U32", case.w.shape, np.ascontiguousarray(case.w).tobytes()),
        (prefix + ".scales", dt, case.scales.shape, np.ascontiguousarray(case.scales).tobytes()),
        (prefix + ".biases", dt, case.biases.shape, np.ascontiguousarray(case.biases).tobytes()),
    ]
    if bias:
        out.append((prefix + ".bias", dt, case.lbias.shape, case.lbias.tobytes()))
    return out


def write_model_dir(root, layers, quantization, extra=(), shards=1, config_extra=None):
    """A checkpoint directory: config.json plus model-0000i-of-0000n.safetensors shards.
    layers: list of (prefix, case, with_bias).  Tensors are dealt round-robin by layer."""
    os.makedirs(root, exist_ok=True)
    cfg = {"model_type": "test", "quantization": quantization}
    if config_extra:
        cfg.update(config_extra)
    with open(os.path.join(root, "config.json"), "w") as f:
        json.dump(cfg, f)
    per = [[] for _ in range(shards)]
    for i, (prefix, case, bias) in enumerate(layers):
        per[i % shards].extend(layer_entries(prefix, case, bias))
    per[0].extend(extra)
    names = []
    for i in range(shards):
        nm = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
        write_safetensors(os.path.join(root, nm), per[i], metadata={"format": "mlx"})
        names.append(nm)
    return names


def case(N, K, bits=4, gs=64, seed=0, M=8, lbias=False, sdt=BF16):
    return make_case(M, N, K, bits=bits, gs=gs, xdt=BF16, sdt=sdt, seed=seed, lbias=lbias)
