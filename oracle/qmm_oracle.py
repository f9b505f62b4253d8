"""CPU oracle for the small-M affine-quantised matmul (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import this module, and only to compare the HIP kernels against: nothing in the
product path calls it.

It holds two independent restatements of the same arithmetic -- numpy code here and the
C code in ``qmm_oracle.c`` (loaded through ctypes) -- so that each pins the other, plus the
seeded input generators for the benchmark configurations.  Reference behaviour followed
(paths relative to the reference repository root):

* ``Sources/DFlashKit/SmallMQuantizedMatmul.swift:56-61`` -- 4-bit code ``t`` of word ``p``
  is ``(p >> 4t) & 15``; element 0 sits in the low bits; row ``n`` starts at word ``n*K/8``.
* ``Sources/DFlashKit/SmallMQuantizedMatmul.swift:64-69`` -- 8-bit: ``(p >> 8t) & 255``,
  row base ``n*K/4``.
* ``Sources/DFlashKit/SmallMQuantizedMatmul.swift:127-129`` -- group ``k // gs``; scale and
  bias at ``[n, g]``.
* ``Sources/DFlashKit/SmallMQuantizedMatmul.swift:59, 69`` -- ``w = float(code) * s + b``.
* ``Sources/DFlashKit/SmallMQuantizedMatmul.swift:209, 288-290`` --
  ``y = x @ dequant(W).T`` (+ optional linear bias).
* ``Sources/DFlashKit/DFlashDecoderLayer.swift:26`` -- the MLP between the swapped
  projections: ``down(silu(gate(x)) * up(x))`` with ``silu(g) = g * sigmoid(g)``.
* ``Sources/DFlashKit/DFlashSpeculativeGenerator.swift:555-571`` -- greedy accept: per-row
  ``argMax`` of the verify logits, ``proposals == targetTokens[..<drafts]``, and the sum of
  the cumulative product of the matches.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

BF16, F16, F32 = 0, 1, 2
DTYPE_NAMES = {BF16: "bf16", F16: "f16", F32: "f32"}

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libqmm_oracle.so")


# ----------------------------------------------------------------------------
# 16-bit float helpers (bit patterns held in uint16 arrays)
# ----------------------------------------------------------------------------

def f32_to_bf16_bits(a) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (NaN quieted)."""
    u = np.ascontiguousarray(np.asarray(a, dtype=np.float32)).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(h) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_f16_bits(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_bits_to_f32(h) -> np.ndarray:
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def to_bits(a, dt: int) -> np.ndarray:
    if dt == BF16:
        return f32_to_bf16_bits(a)
    if dt == F16:
        return f32_to_f16_bits(a)
    return np.asarray(a, dtype=np.float32).copy()


def from_bits(h, dt: int) -> np.ndarray:
    if dt == BF16:
        return bf16_bits_to_f32(h)
    if dt == F16:
        return f16_bits_to_f32(h)
    return np.asarray(h, dtype=np.float32)


# ----------------------------------------------------------------------------
# Packing and dequantisation (numpy restatement)
# ----------------------------------------------------------------------------

def pack(codes: np.ndarray, bits: int) -> np.ndarray:
    """codes[N, K] (uint8) -> w[N, K*bits/32] uint32, element 0 in the low bits."""
    if bits not in (2, 4, 8):
        raise ValueError("bits must be 2, 4 or 8")
    codes = np.asarray(codes, dtype=np.uint32)
    n, k = codes.shape
    per = 32 // bits
    if k % per:
        raise ValueError("K must be a multiple of 32/bits")
    c = codes.reshape(n, k // per, per) & ((1 << bits) - 1)
    shifts = (np.arange(per, dtype=np.uint32) * bits)[None, None, :]
    return np.bitwise_or.reduce(c << shifts, axis=2).astype(np.uint32)


def unpack(w: np.ndarray, bits: int, k: int) -> np.ndarray:
    """w[N, K*bits/32] -> codes[N, K] uint8 (SmallMQuantizedMatmul.swift:57-61, 65-69)."""
    per = 32 // bits
    w = np.asarray(w, dtype=np.uint32)
    shifts = (np.arange(per, dtype=np.uint32) * bits)[None, None, :]
    c = (w[:, :, None] >> shifts) & np.uint32((1 << bits) - 1)
    return c.reshape(w.shape[0], k).astype(np.uint8)


def dequant(w, scales, biases, sdt: int, bits: int, gs: int, k: int) -> np.ndarray:
    """fp32 dequant ``float(q) * s + b``; s*q is exact in fp32, so this is bit-exact."""
    q = unpack(w, bits, k).astype(np.float32)
    s = np.repeat(from_bits(scales, sdt), gs, axis=1)
    b = np.repeat(from_bits(biases, sdt), gs, axis=1)
    return (q * s + b).astype(np.float32)


def qmm_f64(x, xdt, w, scales, biases, sdt, bits, gs, lbias=None, lbdt=BF16) -> np.ndarray:
    """fp64 textbook reference: y = x @ dequant(W).T (+ lbias)."""
    k = np.asarray(x).shape[1]
    q = unpack(w, bits, k).astype(np.float64)
    s = np.repeat(from_bits(scales, sdt).astype(np.float64), gs, axis=1)
    b = np.repeat(from_bits(biases, sdt).astype(np.float64), gs, axis=1)
    wd = q * s + b
    y = from_bits(x, xdt).astype(np.float64) @ wd.T
    if lbias is not None:
        y = y + from_bits(lbias, lbdt).astype(np.float64)[None, :]
    return y


def silu_mul_f64(gu, dt: int) -> np.ndarray:
    """fp64 ``silu(g) * u`` for a fused gate||up output ``gu`` [M, 2N] (bits of dtype dt):
    g = gu[:, :N], u = gu[:, N:], silu(g) = g / (1 + exp(-g))
    (Sources/DFlashKit/DFlashDecoderLayer.swift:26)."""
    a = from_bits(np.asarray(gu), dt).astype(np.float64)
    n = a.shape[1] // 2
    g, u = a[:, :n], a[:, n:]
    return g / (1.0 + np.exp(-g)) * u


def argmax_accept(logits, dt: int, proposals=None):
    """(tokens, accepted) for verify logits [M, V] (bits of dtype dt): tokens[m] is the first
    index of the largest non-NaN logit of row m (-1 if none), accepted the leading run of
    proposals[i] == tokens[i] over i < M-1 (acceptedPrefix,
    Sources/DFlashKit/DFlashSpeculativeGenerator.swift:555-571)."""
    a = from_bits(np.asarray(logits), dt).astype(np.float64)
    tokens = []
    for row in a:
        idx = np.flatnonzero(~np.isnan(row))
        tokens.append(int(idx[np.argmax(row[idx])]) if idx.size else -1)
    tokens = np.array(tokens, dtype=np.int32)
    if proposals is None:
        return tokens, 0
    match = (np.asarray(proposals, dtype=np.int32) == tokens[: len(proposals)]).astype(np.int32)
    return tokens, int(np.cumprod(match).sum())


def out_dtype(xdt: int, sdt: int) -> int:
    """Output dtype of the stock op: MLX type promotion of (x, scales)."""
    if xdt == sdt:
        return xdt
    return F32


# ----------------------------------------------------------------------------
# Seeded inputs for the benchmark configurations
# ----------------------------------------------------------------------------

@dataclass
class QmmCase:
    """One quantised-matmul problem: every array is host memory in its on-device layout."""

    x: np.ndarray        # [M, K] uint16 bits (bf16/fp16)
    w: np.ndarray        # [N, K*bits/32] uint32
    scales: np.ndarray   # [N, K/gs] uint16 bits
    biases: np.ndarray   # [N, K/gs] uint16 bits
    M: int
    N: int
    K: int
    bits: int
    gs: int
    xdt: int
    sdt: int
    lbias: np.ndarray | None = None  # [N] linear bias, same dtype as scales

    @property
    def ydt(self) -> int:
        return out_dtype(self.xdt, self.sdt)


def make_case(M, N, K, bits=4, gs=64, xdt=BF16, sdt=None, seed=0, x_sigma=1.0,
              s_sigma=None, b_sigma=0.01, lbias=False, words=False) -> QmmCase:
    """Generate codes -> scales -> biases -> x (in that order) from one PCG64 stream.

    codes ~ U{0..2^bits-1}; scales ~ |N(0, s_sigma)|; biases ~ N(0, b_sigma);
    x ~ N(0, x_sigma).  s_sigma defaults to 0.02 (4-bit) / 0.004 (8-bit).  words=True draws
    the packed uint32 words directly (uniform words are uniform codes in every slot), which
    is what full-size cases such as a 151936-row LM head use: packing codes one by one there
    takes gigabytes of temporaries.
    """
    sdt = xdt if sdt is None else sdt
    if s_sigma is None:
        s_sigma = 0.02 if bits <= 4 else 0.004
    rng = np.random.Generator(np.random.PCG64(seed))
    if words:
        w = rng.integers(0, 1 << 32, size=(N, K * bits // 32), dtype=np.uint32)
    else:
        codes = rng.integers(0, 1 << bits, size=(N, K), dtype=np.uint8)
        w = pack(codes, bits)
    scales = to_bits(np.abs(rng.normal(0.0, s_sigma, size=(N, K // gs))), sdt)
    biases = to_bits(rng.normal(0.0, b_sigma, size=(N, K // gs)), sdt)
    x = to_bits(rng.normal(0.0, x_sigma, size=(M, K)), xdt)
    lb = to_bits(rng.normal(0.0, 0.05, size=(N,)), sdt) if lbias else None
    return QmmCase(x=x, w=w, scales=scales, biases=biases, M=M, N=N, K=K, bits=bits, gs=gs,
                   xdt=xdt, sdt=sdt, lbias=lb)


# The five benchmark configurations, by name: (kwargs for make_case minus M, list of M).
CONFIGS = {
    # Single matmul, runnable on a CPU: fp16 in/out, seed 0.
    "c1_m1_k4096_n4096_f16": dict(N=4096, K=4096, bits=4, gs=64, xdt=F16, seed=0, Ms=[1]),
    # M sweep of the MLP gate/up shape.
    "c2_gateup_k5120_n17408": dict(N=17408, K=5120, bits=4, gs=64, xdt=BF16, seed=1,
                                   Ms=[1, 2, 4, 6, 8]),
    # MLP down-projection, narrow N / long K.
    "c3_down_k17408_n5120": dict(N=5120, K=17408, bits=4, gs=64, xdt=BF16, seed=2,
                                 x_sigma=0.5, Ms=[8]),
    # Attention projections at 8-bit g64, and the 4-bit g32 variant.
    "c4_qkv_8bit_g64": dict(N=7168, K=5120, bits=8, gs=64, xdt=BF16, seed=3, Ms=[8]),
    "c4_o_8bit_g64": dict(N=5120, K=5120, bits=8, gs=64, xdt=BF16, seed=3, Ms=[8]),
    "c4_qkv_4bit_g32": dict(N=7168, K=5120, bits=4, gs=32, xdt=BF16, seed=3, Ms=[8]),
    "c4_o_4bit_g32": dict(N=5120, K=5120, bits=4, gs=32, xdt=BF16, seed=3, Ms=[8]),
}

# One verify-pass layer of the 64-layer sweep: (name, K, N); plus the LM head.
C5_LAYER = [("q", 5120, 5120), ("k", 5120, 1024), ("v", 5120, 1024), ("o", 5120, 5120),
            ("gate", 5120, 17408), ("up", 5120, 17408), ("down", 17408, 5120)]
C5_LM_HEAD = ("lm_head", 5120, 151936)
C5_LAYERS = 64


def config_case(name: str, M: int) -> QmmCase:
    kw = dict(CONFIGS[name])
    kw.pop("Ms")
    return make_case(M=M, **kw)


def algorithmic_bytes(M, N, K, bits, gs, xbytes=2, sbytes=2, ybytes=2, lbias=False) -> int:
    """Bytes a perfect kernel moves: weights + scales + biases + x + y (+ linear bias)."""
    return (N * K * bits // 8 + 2 * N * (K // gs) * sbytes + M * K * xbytes + M * N * ybytes
            + (N * sbytes if lbias else 0))


# ----------------------------------------------------------------------------
# The C restatement, through ctypes
# ----------------------------------------------------------------------------

class COracle:
    """ctypes handle on oracle/_build/libqmm_oracle.so (built by ``make -C oracle``)."""

    def __init__(self, path: str = _LIB_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        lib = ctypes.CDLL(path)
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        lib.orc_unpack.argtypes = [I, P, I64, I64, P]
        lib.orc_pack.argtypes = [I, P, I64, I64, P]
        lib.orc_dequant.argtypes = [I, I, P, P, P, I, I64, I64, P]
        lib.orc_qmm_f64.argtypes = [I64, I64, I64, I, I, P, I, P, P, P, I, P, I, P]
        lib.orc_qmm_f32.argtypes = [I64, I64, I64, I, I, P, I, P, P, P, I, I, P]
        lib.orc_qmm_ref_kernel.argtypes = [I64, I64, I64, I, P, I, P, P, P, I, P]
        lib.orc_round_output.argtypes = [P, I64, I, P]
        lib.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        lib.orc_f32_to_bf16.restype = ctypes.c_uint16
        lib.orc_f32_to_f16.argtypes = [ctypes.c_float]
        lib.orc_f32_to_f16.restype = ctypes.c_uint16
        lib.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        lib.orc_bf16_to_f32.restype = ctypes.c_float
        lib.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.orc_f16_to_f32.restype = ctypes.c_float
        lib.orc_num_threads.restype = I
        self.lib = lib

    @staticmethod
    def _p(a):
        return None if a is None else a.ctypes.data_as(ctypes.c_void_p)

    def unpack(self, w, bits, n, k):
        out = np.empty((n, k), dtype=np.uint8)
        w = np.ascontiguousarray(w, dtype=np.uint32)
        if self.lib.orc_unpack(bits, self._p(w), n, k, self._p(out)):
            raise ValueError("orc_unpack rejected the shape")
        return out

    def pack(self, codes, bits):
        codes = np.ascontiguousarray(codes, dtype=np.uint8)
        n, k = codes.shape
        out = np.empty((n, k * bits // 32), dtype=np.uint32)
        if self.lib.orc_pack(bits, self._p(codes), n, k, self._p(out)):
            raise ValueError("orc_pack rejected the shape")
        return out

    def dequant(self, w, scales, biases, sdt, bits, gs, n, k):
        out = np.empty((n, k), dtype=np.float32)
        args = [np.ascontiguousarray(a) for a in (w, scales, biases)]
        rc = self.lib.orc_dequant(bits, gs, *[self._p(a) for a in args], sdt, n, k,
                                  self._p(out))
        if rc:
            raise ValueError("orc_dequant rejected the shape")
        return out

    def qmm_f64(self, c: QmmCase) -> np.ndarray:
        y = np.empty((c.M, c.N), dtype=np.float64)
        arrs = [np.ascontiguousarray(a) for a in (c.x, c.w, c.scales, c.biases)]
        lb = None if c.lbias is None else np.ascontiguousarray(c.lbias)
        rc = self.lib.orc_qmm_f64(c.M, c.N, c.K, c.bits, c.gs, self._p(arrs[0]), c.xdt,
                                  self._p(arrs[1]), self._p(arrs[2]), self._p(arrs[3]), c.sdt,
                                  self._p(lb), c.sdt, self._p(y))
        if rc:
            raise ValueError("orc_qmm_f64 rejected the shape")
        return y

    def qmm_f32(self, c: QmmCase, nthreads: int = 0) -> np.ndarray:
        y = np.empty((c.M, c.N), dtype=np.float32)
        arrs = [np.ascontiguousarray(a) for a in (c.x, c.w, c.scales, c.biases)]
        rc = self.lib.orc_qmm_f32(c.M, c.N, c.K, c.bits, c.gs, self._p(arrs[0]), c.xdt,
                                  self._p(arrs[1]), self._p(arrs[2]), self._p(arrs[3]), c.sdt,
                                  nthreads, self._p(y))
        if rc:
            raise ValueError("orc_qmm_f32 rejected the shape")
        return y

    def qmm_ref_kernel(self, c: QmmCase) -> np.ndarray:
        y = np.empty((c.M, c.N), dtype=np.uint16)
        arrs = [np.ascontiguousarray(a) for a in (c.x, c.w, c.scales, c.biases)]
        rc = self.lib.orc_qmm_ref_kernel(c.M, c.N, c.K, c.bits, self._p(arrs[0]), c.xdt,
                                         self._p(arrs[1]), self._p(arrs[2]), self._p(arrs[3]),
                                         c.sdt, self._p(y))
        if rc:
            raise ValueError("orc_qmm_ref_kernel rejected the shape")
        return y

    def round_output(self, y: np.ndarray, ydt: int) -> np.ndarray:
        y = np.ascontiguousarray(y, dtype=np.float64)
        out = np.empty(y.shape, dtype=np.float32 if ydt == F32 else np.uint16)
        self.lib.orc_round_output(self._p(y), y.size, ydt, self._p(out))
        return out

    def num_threads(self) -> int:
        return self.lib.orc_num_threads()


def tolerance_check(y_test: np.ndarray, y_ref: np.ndarray):
    """Return (max_rel_err, ref_style_ok).

    max_rel_err = max|y_test - y_ref| / max|y_ref| (the 1e-2 bar);
    ref_style_ok is the reference test's own rule,
    max|d| <= 0.02 * max(max|ref|, 1)  (SmallMQuantizedMatmulTests.swift:74-79).
    """
    d = np.abs(np.asarray(y_test, np.float64) - np.asarray(y_ref, np.float64))
    mag = float(np.max(np.abs(y_ref))) if y_ref.size else 0.0
    md = float(np.max(d)) if d.size else 0.0
    rel = md / mag if mag > 0 else md
    return rel, md <= 0.02 * max(mag, 1.0)
