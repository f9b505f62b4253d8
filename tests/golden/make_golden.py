"""Writes tests/golden/qmm_golden.npz: small fixtures from the oracle (test data only).

Each case stores its inputs in the on-device layout (x, w, scales, biases bit patterns), the
exact fp32 dequantised matrix and the fp64 result.  The known-answer words are the
hand-derived unpack vectors of SmallMQuantizedMatmul.swift:57-61 (4-bit) and :65-69 (8-bit).
Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle.qmm_oracle import BF16, F16, COracle, make_case  # noqa: E402

CASES = [  # name, M, N, K, bits, gs, dtype, seed, lbias
    ("b4g64_bf16_m3", 3, 16, 128, 4, 64, BF16, 101, False),
    ("b4g64_bf16_m8_onegroup", 8, 24, 64, 4, 64, BF16, 102, False),
    ("b8g32_f16_m8", 8, 24, 256, 8, 32, F16, 103, True),
    ("b4g128_bf16_m5", 5, 40, 512, 4, 128, BF16, 104, False),
    ("b8g64_bf16_m1", 1, 17, 256, 8, 64, BF16, 105, True),
    ("b4g32_f16_m7", 7, 33, 256, 4, 32, F16, 106, False),
    ("b4g64_bf16_m8_k1024", 8, 48, 1024, 4, 64, BF16, 107, True),
]


def main():
    orc = COracle()
    out = {
        "known_w4": np.array([[0x76543210, 0xFEDCBA98]], dtype=np.uint32),
        "known_codes4": np.arange(16, dtype=np.uint8)[None, :],
        "known_w8": np.array([[0x03020100, 0xFFFE0180]], dtype=np.uint32),
        "known_codes8": np.array([[0, 1, 2, 3, 0x80, 0x01, 0xFE, 0xFF]], dtype=np.uint8),
    }
    names = []
    for (name, M, N, K, bits, gs, dt, seed, lb) in CASES:
        c = make_case(M, N, K, bits=bits, gs=gs, xdt=dt, seed=seed, lbias=lb)
        names.append(name)
        out[f"{name}/meta"] = np.array([M, N, K, bits, gs, dt, int(lb)], dtype=np.int64)
        out[f"{name}/x"] = c.x
        out[f"{name}/w"] = c.w
        out[f"{name}/scales"] = c.scales
        out[f"{name}/biases"] = c.biases
        if lb:
            out[f"{name}/lbias"] = c.lbias
        out[f"{name}/dequant"] = orc.dequant(c.w, c.scales, c.biases, c.sdt, bits, gs, N, K)
        out[f"{name}/y_f64"] = orc.qmm_f64(c)
    out["cases"] = np.array(names)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "qmm_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(names)} cases")


if __name__ == "__main__":
    main()
