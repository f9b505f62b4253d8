"""The drop-in layer on the GPU, mirroring the reference's kernel tests.

Reference: Tests/DFlashKitTests/SmallMQuantizedMatmulTests.swift.  `stock` is a plain
QuantizedLinear (the generic path), `fast` is SmallMQuantizedLinear(stock) sharing its
arrays.  The reference builds its layer with MLX's quantiser from normal(scale 0.05) weights
(:47-55); MLX is not available here, so codes, scales and biases are drawn directly with the
same layer shape (out 4096, in 1024, group 64).
"""
import numpy as np
import pytest
import torch

from dflash_qmm import QuantizedLinear, SmallMQuantizedLinear
from gpu_util import announce, upload
from oracle.qmm_oracle import BF16, make_case

pytestmark = pytest.mark.gpu

OUT, IN, TOL = 4096, 1024, 0.02


def make_layer(ctx, bits, out_features=OUT, in_features=IN, group_size=64, seed=7):
    c = make_case(1, out_features, in_features, bits=bits, gs=group_size, seed=seed)
    _, w, s, b, _ = upload(c)
    return QuantizedLinear(ctx, w, s, b, None, group_size=group_size, bits=bits)


def make_input(rows, in_features=IN, seed=11):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return (torch.randn(rows, in_features, device="cuda", generator=g) * 0.1).to(torch.bfloat16)


def assert_agrees(ctx, bits, rows):
    stock = make_layer(ctx, bits)
    fast = SmallMQuantizedLinear(stock)
    x = make_input(rows)
    announce(f"dropin agrees bits={bits} rows={rows}")
    ref = stock(x).float()
    assert not stock.last_took_kernel
    got = fast(x)
    assert fast.last_took_kernel
    assert got.shape == (rows, OUT)
    diff = (ref - got.float()).abs().max().item()
    mag = ref.abs().max().item()
    assert diff <= TOL * max(mag, 1.0), f"{bits}-bit M={rows}: {diff} at {mag}"


@pytest.mark.parametrize("rows", range(2, 17))
def test_4bit_matches_stock(ctx, rows):
    assert_agrees(ctx, 4, rows)


@pytest.mark.parametrize("rows", range(2, 17))
def test_8bit_matches_stock(ctx, rows):
    assert_agrees(ctx, 8, rows)


def test_kernel_output_is_not_bit_identical(ctx):
    stock = make_layer(ctx, 4)
    fast = SmallMQuantizedLinear(stock)
    x = make_input(8)
    announce("dropin not bit identical")
    assert (stock(x) != fast(x)).any().item()


def test_ineligible_shape_returns_the_stock_result(ctx):
    stock = make_layer(ctx, 4, out_features=2048)
    fast = SmallMQuantizedLinear(stock)
    x = make_input(8)
    announce("dropin ineligible shape")
    assert torch.equal(stock(x), fast(x))
    assert not fast.last_took_kernel


def test_row_counts_outside_the_window_return_the_stock_result(ctx):
    """One row (below this chip's crossover, where the stock GEMV is as fast) and more than
    16 rows (more than two row tiles) fall through unchanged, bit for bit."""
    stock = make_layer(ctx, 4)
    fast = SmallMQuantizedLinear(stock)
    for rows in [1, 17, 24, 32]:
        x = make_input(rows)
        announce(f"dropin rows outside window {rows}")
        assert torch.equal(stock(x), fast(x)), f"M={rows}"
        assert not fast.last_took_kernel


def test_float16_input_falls_through_to_stock(ctx):
    stock = make_layer(ctx, 4)
    fast = SmallMQuantizedLinear(stock)
    x = make_input(8).to(torch.float16)
    announce("dropin fp16 falls through")
    ref = stock(x)
    y = fast(x)
    assert y.dtype == ref.dtype == torch.float32
    assert torch.equal(ref, y)


def test_leading_dimensions_are_flattened(ctx):
    """callAsFunction multiplies out the leading dimensions (:255-256, :287)."""
    stock = make_layer(ctx, 4)
    fast = SmallMQuantizedLinear(stock)
    x = make_input(8).reshape(1, 8, IN)
    announce("dropin leading dims")
    y = fast(x)
    assert y.shape == (1, 8, OUT) and fast.last_took_kernel
    assert torch.equal(y.reshape(8, OUT), fast(x.reshape(8, IN)))


def test_linear_bias_is_added(ctx):
    c = make_case(1, OUT, IN, bits=4, gs=64, seed=3, lbias=True)
    _, w, s, b, lb = upload(c)
    stock = QuantizedLinear(ctx, w, s, b, lb, group_size=64, bits=4)
    nob = QuantizedLinear(ctx, w, s, b, None, group_size=64, bits=4)
    fast = SmallMQuantizedLinear(stock)
    x = make_input(8)
    announce("dropin linear bias")
    d = (fast(x).float() - (nob(x).float() + lb.float()[None, :])).abs().max().item()
    assert d <= TOL * max(nob(x).float().abs().max().item(), 1.0)


def test_layer_past_the_kernels_size_limit_falls_through(ctx):
    """An eligible layer whose weights reach 2 GiB (262144 x 16384 at 4 bits) is past the
    fast kernel's own limit: the swapped layer must fall through to the stock path like any
    ineligible call (SmallMQuantizedMatmul.swift:254-266), not fail.  No device memory is
    needed: the descriptor's pointers are never dereferenced, the workspace query answers 0
    and a forward with a null input is refused by the stock path's argument check
    (status 1, took_kernel 0) before any launch."""
    import ctypes
    import dflash_qmm
    lib = dflash_qmm.load_library()
    fake = 1 << 40
    d = dflash_qmm._LinearDesc(fake, fake, fake, None, 262144, 16384, 4, 64, 1, BF16)
    h = ctypes.c_void_p()
    assert lib.dfq_linear_create(ctx.handle, ctypes.byref(d), ctypes.byref(h)) == 0
    fast = ctypes.c_void_p()
    assert lib.dfq_small_m_linear_create(h, ctypes.byref(fast)) == 0
    assert lib.dfq_is_eligible(262144, 16384, 4, 64, 1, 1) == 1
    assert not ctx.supported(8, 262144, 16384, 4, 64)
    nb = ctypes.c_size_t(123)
    assert lib.dfq_linear_workspace_bytes(fast, 8, ctypes.byref(nb)) == 0 and nb.value == 0
    took = ctypes.c_int(-1)
    rc = lib.dfq_linear_forward(fast, None, BF16, 8, None, None, 0, None, ctypes.byref(took))
    assert rc == 1 and took.value == 0, (rc, took.value, lib.dfq_last_error())
    lib.dfq_linear_destroy(fast)
    lib.dfq_linear_destroy(h)
