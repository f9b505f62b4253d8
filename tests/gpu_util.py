"""Helpers shared by the GPU tests: moving oracle cases to the device and back."""
import sys

import numpy as np

from oracle.qmm_oracle import BF16, F16, F32, QmmCase, from_bits


def torch_dtype(code):
    import torch
    return {BF16: torch.bfloat16, F16: torch.float16, F32: torch.float32}[code]


def to_dev16(a: np.ndarray, code: int, device="cuda"):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(device)
    return t.view(torch_dtype(code))


def upload(c: QmmCase, device="cuda"):
    """(x, w, scales, biases, lbias) device tensors for a case."""
    import torch
    x = to_dev16(c.x, c.xdt, device)
    w = torch.from_numpy(np.ascontiguousarray(c.w).view(np.int32)).to(device)
    s = to_dev16(c.scales, c.sdt, device)
    b = to_dev16(c.biases, c.sdt, device)
    lb = None if c.lbias is None else to_dev16(c.lbias, c.sdt, device)
    return x, w, s, b, lb


def download(y) -> np.ndarray:
    """Device result -> float64 numpy (exact widening of bf16/fp16/fp32)."""
    import torch
    if y.dtype == torch.float32:
        return y.detach().cpu().numpy().astype(np.float64)
    code = BF16 if y.dtype == torch.bfloat16 else F16
    bits = y.detach().view(torch.int16).cpu().numpy().view(np.uint16)
    return from_bits(bits, code).astype(np.float64)


def announce(msg: str):
    """Name the case before a GPU step, so a fault can be tied to it."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()
