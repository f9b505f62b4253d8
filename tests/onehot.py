"""Inputs whose one-hot products are exact: shared by the GPU unpack test and its CPU pin."""
import numpy as np

from oracle.qmm_oracle import dequant, from_bits, pack, to_bits


def exact_case(N, K, bits, gs, dt, seed):
    """Codes uniform; per group s in {1, 1/2, 1/4, 1/8} and b in {0, -1, -2, 2, 1/2}, with b
    set to 0 in a group where s*q + b would not be exact in the dtype for some code (b = 0
    always is: s*q has at most 8 significant bits)."""
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 1 << bits, size=(N, K), dtype=np.uint8)
    G = K // gs
    s = 2.0 ** -rng.integers(0, 4, size=(N, G))
    b = rng.choice([0.0, -1.0, -2.0, 2.0, 0.5], size=(N, G))
    w = pack(codes, bits)
    sb = to_bits(s, dt)

    def deq_of(b):
        bb = to_bits(b, dt)
        return bb, dequant(w, sb, bb, dt, bits, gs, K).astype(np.float64)

    bb, deq = deq_of(b)
    exact = from_bits(to_bits(deq, dt), dt) == deq
    b[~exact.reshape(N, G, gs).all(axis=2)] = 0.0
    bb, deq = deq_of(b)
    assert np.array_equal(from_bits(to_bits(deq, dt), dt), deq), "values must be exact"
    assert np.count_nonzero(b) > b.size // 4, "most groups keep a nonzero bias"
    return w, sb, bb, deq
