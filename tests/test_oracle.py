"""Pins of the CPU oracle (both restatements: numpy and C).

The reference holds no golden vectors for this path (its kernel tests compare against MLX at
run time, Tests/DFlashKitTests/SmallMQuantizedMatmulTests.swift:65-102, and MLX is not
available here).  Each oracle function is therefore pinned by checks that a plausible
mistake cannot pass:

* unpack / pack: hand-derived known answers from the reference's formula
  ``(p >> bits*t) & mask`` (SmallMQuantizedMatmul.swift:57-61, 65-69), brute-force round
  trips over every code value at every position, and agreement of the two restatements;
* dequant: bit-exact agreement of three independent computations (C fp32, numpy fp32, fp64
  rounded once) -- exact because s*q is exact in fp32 -- plus closed forms (s = 0, b = 0);
* qmm: a library fp64 matmul on the dequantised matrix, closed-form special cases (all codes
  zero, one nonzero code, a single group), and invariants (linearity, row independence, row
  permutation of W permutes the columns of y);
* planted mistakes: wrong nibble order, off-by-one group, swapped scale/bias and a transposed
  operand are each shown to fail at least one of the pins above.
"""
import numpy as np
import pytest

from oracle import qmm_oracle as Q
from oracle.qmm_oracle import BF16, F16, F32


# ----------------------------------------------------------------------------------------
# 16-bit float conversions
# ----------------------------------------------------------------------------------------

def test_bf16_and_f16_widening_is_exact_for_every_pattern(oracle):
    h = np.arange(1 << 16, dtype=np.uint16)
    want_bf = (h.astype(np.uint32) << 16).view(np.float32)
    want_f16 = h.view(np.float16).astype(np.float32)
    lib = oracle.lib
    got_bf = np.array([lib.orc_bf16_to_f32(int(v)) for v in h[::97]], dtype=np.float32)
    got_f16 = np.array([lib.orc_f16_to_f32(int(v)) for v in h[::97]], dtype=np.float32)
    # NaN payloads do not survive the round trip through a Python float; compare NaN-ness
    finb = ~np.isnan(want_bf[::97])
    assert np.array_equal(got_bf[finb].view(np.uint32), want_bf[::97][finb].view(np.uint32))
    assert np.all(np.isnan(got_bf[~finb]))
    fin = np.isfinite(want_f16[::97])
    assert np.array_equal(got_f16[fin].view(np.uint32), want_f16[::97][fin].view(np.uint32))
    assert np.all(np.isnan(got_f16[~fin]) == np.isnan(want_f16[::97][~fin]))


def test_f32_rounding_matches_numpy(oracle):
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.normal(0, 1, 2000), rng.normal(0, 1e4, 500), rng.normal(0, 1e-6, 500),
        [0.0, -0.0, 65504.0, 65519.9, 65520.0, 6.1e-5, 5.96e-8, 2.98e-8, 1.0 + 2 ** -8,
         1.0 + 3 * 2 ** -9, -(1.0 + 2 ** -9)],
    ]).astype(np.float32)
    lib = oracle.lib
    f16 = np.array([lib.orc_f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(f16, vals.astype(np.float16).view(np.uint16))
    bf = np.array([lib.orc_f32_to_bf16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(bf, Q.f32_to_bf16_bits(vals))
    # ties round to even: 1 + 2^-8 is halfway between two bf16 values
    assert Q.f32_to_bf16_bits(np.float32(1.0 + 2 ** -8)) == 0x3F80
    assert Q.f32_to_bf16_bits(np.float32(1.0 + 3 * 2 ** -8)) == 0x3F82


# ----------------------------------------------------------------------------------------
# Packing
# ----------------------------------------------------------------------------------------

def test_unpack_known_answers(oracle):
    # (p >> 4t) & 15, element 0 in the low bits
    w4 = np.array([[0x76543210, 0xFEDCBA98]], dtype=np.uint32)
    assert list(Q.unpack(w4, 4, 16)[0]) == list(range(16))
    assert list(oracle.unpack(w4, 4, 1, 16)[0]) == list(range(16))
    # (p >> 8t) & 255
    w8 = np.array([[0x03020100, 0xFFFE0180]], dtype=np.uint32)
    assert list(Q.unpack(w8, 8, 8)[0]) == [0, 1, 2, 3, 0x80, 0x01, 0xFE, 0xFF]
    assert list(oracle.unpack(w8, 8, 1, 8)[0]) == [0, 1, 2, 3, 0x80, 0x01, 0xFE, 0xFF]
    # 2-bit: 16 codes per word
    w2 = np.array([[0xE4E4E4E4]], dtype=np.uint32)  # 0b11100100 repeated -> 0,1,2,3,...
    assert list(Q.unpack(w2, 2, 16)[0]) == [0, 1, 2, 3] * 4


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_pack_unpack_round_trip_every_value_every_slot(oracle, bits):
    per = 32 // bits
    vals = np.arange(1 << bits, dtype=np.uint8)
    # every value at every slot position: (2^bits) rows x per columns, rolled per row
    codes = np.stack([np.roll(np.resize(vals, per * 8), r) for r in range(len(vals))])
    w_np, w_c = Q.pack(codes, bits), oracle.pack(codes, bits)
    assert np.array_equal(w_np, w_c)
    assert np.array_equal(Q.unpack(w_np, bits, codes.shape[1]), codes)
    assert np.array_equal(oracle.unpack(w_c, bits, *codes.shape), codes)


# ----------------------------------------------------------------------------------------
# Dequant
# ----------------------------------------------------------------------------------------

@pytest.mark.parametrize("bits,gs,sdt", [(4, 64, BF16), (8, 32, F16), (4, 128, F16),
                                         (8, 64, BF16), (2, 32, BF16)])
def test_dequant_is_bit_exact_three_ways(oracle, bits, gs, sdt):
    c = Q.make_case(1, 37, 4 * gs, bits=bits, gs=gs, xdt=sdt, seed=bits + gs)
    d_c = oracle.dequant(c.w, c.scales, c.biases, sdt, bits, gs, c.N, c.K)
    d_np = Q.dequant(c.w, c.scales, c.biases, sdt, bits, gs, c.K)
    q = Q.unpack(c.w, bits, c.K).astype(np.float64)
    s = np.repeat(Q.from_bits(c.scales, sdt).astype(np.float64), gs, axis=1)
    b = np.repeat(Q.from_bits(c.biases, sdt).astype(np.float64), gs, axis=1)
    d_64 = (s * q + b).astype(np.float32)  # one rounding of the exact value
    assert np.array_equal(d_c.view(np.uint32), d_np.view(np.uint32))
    assert np.array_equal(d_c.view(np.uint32), d_64.view(np.uint32))


def test_dequant_closed_forms(oracle):
    n, k, gs = 4, 128, 64
    codes = np.full((n, k), 15, dtype=np.uint8)
    w = Q.pack(codes, 4)
    s = Q.to_bits(np.full((n, k // gs), 0.25), BF16)
    zero = Q.to_bits(np.zeros((n, k // gs)), BF16)
    b = Q.to_bits(np.full((n, k // gs), -1.5), BF16)
    assert np.all(oracle.dequant(w, s, zero, BF16, 4, gs, n, k) == 15 * 0.25)
    assert np.all(oracle.dequant(w, zero, b, BF16, 4, gs, n, k) == -1.5)


# ----------------------------------------------------------------------------------------
# The matmul
# ----------------------------------------------------------------------------------------

@pytest.mark.parametrize("M,N,K,bits,gs,xdt", [(1, 16, 64, 4, 64, BF16), (3, 40, 256, 8, 32, F16),
                                               (8, 33, 384, 4, 128, BF16), (5, 7, 96, 2, 32, F16)])
def test_qmm_matches_library_matmul(oracle, M, N, K, bits, gs, xdt):
    c = Q.make_case(M, N, K, bits=bits, gs=gs, xdt=xdt, seed=M + N + K, lbias=True)
    wd = Q.dequant(c.w, c.scales, c.biases, c.sdt, bits, gs, K).astype(np.float64)
    ref = Q.from_bits(c.x, xdt).astype(np.float64) @ wd.T + Q.from_bits(c.lbias, c.sdt)[None, :]
    assert np.allclose(oracle.qmm_f64(c), ref, rtol=1e-12, atol=1e-12)
    assert np.allclose(Q.qmm_f64(c.x, xdt, c.w, c.scales, c.biases, c.sdt, bits, gs,
                                 lbias=c.lbias, lbdt=c.sdt), ref, rtol=1e-12, atol=1e-12)


def test_qmm_all_codes_zero_is_bias_times_group_sums(oracle):
    M, N, K, gs = 3, 5, 256, 64
    c = Q.make_case(M, N, K, bits=4, gs=gs, seed=3)
    c.w = np.zeros_like(c.w)
    x = Q.from_bits(c.x, c.xdt).astype(np.float64)
    xs = x.reshape(M, K // gs, gs).sum(axis=2)                   # [M, G]
    b = Q.from_bits(c.biases, c.sdt).astype(np.float64)          # [N, G]
    assert np.allclose(oracle.qmm_f64(c), xs @ b.T, rtol=1e-12, atol=1e-12)


def test_qmm_single_code_copies_one_x_column(oracle):
    M, N, K, gs = 4, 6, 128, 64
    c = Q.make_case(M, N, K, bits=8, gs=gs, seed=4)
    codes = np.zeros((N, K), dtype=np.uint8)
    codes[2, 77] = 9
    c.w = Q.pack(codes, 8)
    c.scales = Q.to_bits(np.ones((N, K // gs)), c.sdt)
    c.biases = Q.to_bits(np.zeros((N, K // gs)), c.sdt)
    y = oracle.qmm_f64(c)
    x = Q.from_bits(c.x, c.xdt).astype(np.float64)
    want = np.zeros((M, N))
    want[:, 2] = 9 * x[:, 77]
    assert np.array_equal(y, want)


def test_qmm_single_group_and_invariants(oracle):
    c = Q.make_case(6, 24, 64, bits=4, gs=64, seed=5)   # K == gs: one group
    y = oracle.qmm_f64(c)
    # row independence: each row equals the 1-row problem on that row
    for r in range(6):
        c1 = Q.make_case(1, 24, 64, bits=4, gs=64, seed=5)
        c1.w, c1.scales, c1.biases, c1.x = c.w, c.scales, c.biases, c.x[r:r + 1]
        assert np.array_equal(oracle.qmm_f64(c1)[0], y[r])
    # permuting W's rows (with their scales and biases) permutes y's columns
    perm = np.random.default_rng(1).permutation(24)
    cp = Q.make_case(6, 24, 64, bits=4, gs=64, seed=5)
    cp.w, cp.scales, cp.biases = c.w[perm], c.scales[perm], c.biases[perm]
    assert np.array_equal(oracle.qmm_f64(cp), y[:, perm])
    # linearity in x (fp64): y(x1) + y(x2) == y(x1 + x2) up to fp64 rounding
    xa = Q.from_bits(c.x, c.xdt)
    cb = Q.make_case(6, 24, 64, bits=4, gs=64, seed=6)
    xb = Q.from_bits(cb.x, cb.xdt)
    c2 = Q.make_case(6, 24, 64, bits=4, gs=64, seed=5)
    c2.x, c2.xdt = (xa + xb).astype(np.float32), F32
    ca, cbb = Q.make_case(6, 24, 64, bits=4, gs=64, seed=5), Q.make_case(6, 24, 64, bits=4,
                                                                         gs=64, seed=5)
    ca.x, ca.xdt = xa.astype(np.float32), F32
    cbb.x, cbb.xdt = xb.astype(np.float32), F32
    assert np.allclose(oracle.qmm_f64(ca) + oracle.qmm_f64(cbb), oracle.qmm_f64(c2),
                       rtol=1e-12, atol=1e-9)


def test_fp32_restatement_and_reference_kernel_are_close(oracle):
    c = Q.make_case(8, 64, 1024, bits=4, gs=64, seed=8)
    ref = oracle.qmm_f64(c)
    rel32, ok32 = Q.tolerance_check(oracle.qmm_f32(c), ref)
    assert rel32 < 1e-5 and ok32
    rk = Q.from_bits(oracle.qmm_ref_kernel(c), BF16)
    relk, okk = Q.tolerance_check(rk, ref)
    assert relk < 1e-2 and okk
    assert relk > rel32  # bf16-rounded weights: the reference kernel is the coarser one


# ----------------------------------------------------------------------------------------
# Planted mistakes: each must fail at least one pin
# ----------------------------------------------------------------------------------------

def _unpack_big_endian(w, bits, k):
    per = 32 // bits
    shifts = ((per - 1 - np.arange(per, dtype=np.uint32)) * bits)[None, None, :]
    c = (np.asarray(w, np.uint32)[:, :, None] >> shifts) & np.uint32((1 << bits) - 1)
    return c.reshape(w.shape[0], k).astype(np.uint8)


def test_planted_wrong_nibble_order_is_caught():
    w4 = np.array([[0x76543210, 0xFEDCBA98]], dtype=np.uint32)
    assert list(_unpack_big_endian(w4, 4, 16)[0]) != list(range(16))


def test_planted_off_by_one_group_is_caught(oracle):
    c = Q.make_case(2, 8, 256, bits=4, gs=64, seed=11)
    q = Q.unpack(c.w, 4, 256).astype(np.float64)
    s = Q.from_bits(c.scales, c.sdt).astype(np.float64)
    b = Q.from_bits(c.biases, c.sdt).astype(np.float64)
    g = np.minimum((np.arange(256) + 1) // 64, 3)      # group index shifted by one element
    wrong = s[:, g] * q + b[:, g]
    y_wrong = Q.from_bits(c.x, c.xdt).astype(np.float64) @ wrong.T
    rel, ok = Q.tolerance_check(y_wrong, oracle.qmm_f64(c))
    assert rel > 1e-6


def test_planted_swapped_scale_and_bias_is_caught(oracle):
    c = Q.make_case(2, 8, 256, bits=4, gs=64, seed=12)
    cs = Q.make_case(2, 8, 256, bits=4, gs=64, seed=12)
    cs.scales, cs.biases = c.biases, c.scales
    rel, _ = Q.tolerance_check(oracle.qmm_f64(cs), oracle.qmm_f64(c))
    assert rel > 1e-2


def test_planted_transposed_operand_is_caught(oracle):
    c = Q.make_case(16, 16, 64, bits=4, gs=64, seed=13)
    wd = Q.dequant(c.w, c.scales, c.biases, c.sdt, 4, 64, 64).astype(np.float64)
    x = Q.from_bits(c.x, c.xdt).astype(np.float64)
    y_t = wd[:, :16] @ x[:, :16].T       # a transposed-operand slip on a square corner
    rel, _ = Q.tolerance_check(y_t, oracle.qmm_f64(c))
    assert rel > 1e-2


def test_silu_mul_closed_forms():
    """silu(0) = 0; silu(g) - silu(-g) = g (g*sigmoid(g) + g*sigmoid(-g) = g); silu(g) -> g
    for large g and -> 0 for very negative g; u = 0 or u = 1 isolate each factor."""
    from oracle.qmm_oracle import silu_mul_f64, to_bits, from_bits
    g = np.array([[0.0, 1.0, -1.0, 2.5, -2.5, 40.0, -40.0, 0.5]], dtype=np.float32)
    g = from_bits(to_bits(g, BF16), BF16)
    ones = np.ones_like(g)
    h = silu_mul_f64(to_bits(np.concatenate([g, ones], axis=1), BF16), BF16)[0]
    hn = silu_mul_f64(to_bits(np.concatenate([-g, ones], axis=1), BF16), BF16)[0]
    assert h[0] == 0.0
    np.testing.assert_allclose(h - hn, g[0], rtol=1e-12, atol=1e-12)
    assert abs(h[5] - 40.0) < 1e-12 and abs(h[6]) < 1e-15
    np.testing.assert_allclose(h[1], 1.0 / (1.0 + np.exp(-1.0)), rtol=1e-15)
    zero = silu_mul_f64(to_bits(np.concatenate([g, 0 * ones], axis=1), BF16), BF16)
    assert not zero.any()
    u = np.array([[3.0, -2.0, 0.25, 1.0, 1.0, 1.0, 1.0, 1.0]], dtype=np.float32)
    hu = silu_mul_f64(to_bits(np.concatenate([g, u], axis=1), BF16), BF16)[0]
    np.testing.assert_allclose(hu, h * from_bits(to_bits(u, BF16), BF16)[0], rtol=1e-15)


def test_argmax_accept_closed_forms():
    """First index among equal maxima, NaN skipped (an all-NaN row gives -1), -inf rows give
    index 0, and the accepted count is the run of leading matches, checked against a plain
    loop over the same tokens."""
    from oracle.qmm_oracle import argmax_accept, to_bits
    nan, inf = float("nan"), float("inf")
    rows = np.array([[1.0, 3.0, 3.0, 2.0],          # tie -> 1
                     [nan, 0.5, nan, 0.25],         # NaN skipped -> 1
                     [-inf, -inf, -inf, -inf],      # all -inf -> 0
                     [nan, nan, nan, nan],          # no number -> -1
                     [-1.0, -2.0, -0.5, -0.5]],     # negative tie -> 2
                    dtype=np.float32)
    bits = to_bits(rows, BF16)
    tokens, acc = argmax_accept(bits, BF16, proposals=[1, 1, 0, 5])
    assert tokens.tolist() == [1, 1, 0, -1, 2]
    assert acc == 3                                   # 1==1, 1==1, 0==0, 5!=-1
    for props in ([0, 1, 0, -1], [1, 2, 0, -1], [1, 1, 0, -1], []):
        _, acc = argmax_accept(bits, BF16, proposals=props)
        run = 0
        for p_, t in zip(props, tokens):
            if p_ != t:
                break
            run += 1
        assert acc == run
    assert argmax_accept(bits[:1], BF16, proposals=[])[1] == 0


def test_one_hot_columns_catch_a_slip_a_tolerance_misses():
    """The one-hot unpack test compares exact dequant columns bit for bit.  A slip confined to
    one code value in one slot of the first 64 words of a row (code 15 in the top nibble
    read as 14) moves a random-x product of the headline's distributions by well under the
    1e-2 parity bar, yet changes the exact columns it touches."""
    import os
    import sys
    sys.path.insert(0, os.path.dirname(__file__))
    from onehot import exact_case

    def slipped(w, K):
        q = Q.unpack(w, 4, K).astype(np.float32)
        top = q[:, 7:512:8]
        top[top == 15] = 14
        q[:, 7:512:8] = top
        return q

    def deq_from(q, sb, bb, gs=64):
        s = np.repeat(Q.from_bits(sb, Q.BF16), gs, axis=1)
        b = np.repeat(Q.from_bits(bb, Q.BF16), gs, axis=1)
        return (q * s + b).astype(np.float64)

    N, K = 64, 5120
    c = Q.make_case(8, N, K, bits=4, gs=64, seed=21)
    x = Q.from_bits(c.x, c.xdt).astype(np.float64)
    good = Q.dequant(c.w, c.scales, c.biases, c.sdt, 4, 64, K).astype(np.float64)
    rel, ok = Q.tolerance_check(x @ deq_from(slipped(c.w, K), c.scales, c.biases).T, x @ good.T)
    assert 0 < rel < 1e-2 and ok                             # hides under the tolerance
    w, sb, bb, deq = exact_case(16, 512, 4, 64, Q.BF16, 21)
    cols = list(range(7, 512, 8))
    assert not np.array_equal(Q.to_bits(deq_from(slipped(w, 512), sb, bb)[:, cols], Q.BF16),
                              Q.to_bits(deq[:, cols], Q.BF16))  # the exact columns differ
