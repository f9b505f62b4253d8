"""The drop-in layer's gate and module swap, on the CPU.

Mirrors the eligibility tests of the reference (Tests/DFlashKitTests/
SmallMQuantizedMatmulTests.swift:104-133): the eligible shape is swapped, the swap is
idempotent, and each ineligible case -- which violates exactly one bound -- is left alone.
Layers here carry host tensors as stand-in arrays: the gate and the swap only read shapes
and formats, and a layer built without a context cannot be called.
"""
import pytest
import torch

import dflash_qmm
from dflash_qmm import (Model, QuantizedLinear, SmallMQuantizedLinear, SmallMQuantizedMatmul,
                        enable_small_m_quantized_matmul)


def layer(bits=4, out_features=4096, in_features=1024, group_size=64, biases=True,
          mode="affine"):
    words = in_features * bits // 32
    w = torch.zeros(out_features, words, dtype=torch.int32)
    s = torch.zeros(out_features, in_features // group_size, dtype=torch.bfloat16)
    b = torch.zeros_like(s) if biases else None
    return QuantizedLinear(None, w, s, b, None, group_size=group_size, bits=bits, mode=mode)


def test_window_constants_match_the_reference():
    # SmallMQuantizedMatmul.swift:32, 36, 39, 41, 45, 47; minimumRows is the crossover against
    # the stock path measured on this chip (the reference's comment at :29-31 makes it a
    # per-chip constant: 6 on its Apple GPU, 2 on MI355X)
    c = SmallMQuantizedMatmul
    assert (c.minimum_rows, c.maximum_rows, c.rows_per_tile) == (2, 16, 8)
    assert (c.minimum_output_features, c.input_feature_multiple, c.required_group_size) == (
        4096, 512, 64)
    hdr = open(__file__.replace("tests/test_dropin_gate.py", "include/dflash_qmm.h")).read()
    for name, v in [("DFQ_MINIMUM_ROWS", 2), ("DFQ_MAXIMUM_ROWS", 16), ("DFQ_ROWS_PER_TILE", 8),
                    ("DFQ_MINIMUM_OUTPUT_FEATURES", 4096), ("DFQ_INPUT_FEATURE_MULTIPLE", 512),
                    ("DFQ_REQUIRED_GROUP_SIZE", 64)]:
        assert f"#define {name} {v}" in hdr


def test_tiles_for_rows():
    # SmallMQuantizedMatmul.swift:205-207
    assert [SmallMQuantizedMatmul.tiles(r) for r in (1, 6, 8, 9, 16)] == [1, 1, 1, 2, 2]


def test_eligible_shape_is_swapped():
    model = Model(projection=layer(bits=4))
    assert enable_small_m_quantized_matmul(model) == 1
    assert isinstance(model.projection, SmallMQuantizedLinear)
    assert model.projection.is_small_m


def test_swap_is_idempotent():
    model = Model(projection=layer(bits=4))
    assert enable_small_m_quantized_matmul(model) == 1
    assert enable_small_m_quantized_matmul(model) == 0


def test_eight_bit_is_eligible():
    assert SmallMQuantizedMatmul.is_eligible(layer(bits=8))


@pytest.mark.parametrize("reason,kw", [
    ("N below 4096", dict(out_features=2048)),
    ("K not a multiple of 512", dict(in_features=1024 + 64)),
    ("group size 32", dict(group_size=32)),
    ("unsupported bit width", dict(bits=2)),
    ("no biases", dict(biases=False)),
    ("not affine", dict(mode="mxfp4")),
])
def test_ineligible_shapes_are_left_alone(reason, kw):
    lay = layer(**kw)
    assert not SmallMQuantizedMatmul.is_eligible(lay), reason
    model = Model(projection=lay)
    assert enable_small_m_quantized_matmul(model) == 0, reason
    assert not isinstance(model.projection, SmallMQuantizedLinear), reason


def test_three_bit_gate_is_closed():
    # The reference's "unsupported bit width" case uses 3 bits; the gate reads bits only.
    assert dflash_qmm.load_library().dfq_is_eligible(4096, 1024, 3, 64, 1, 1) == 0


def test_swap_counts_only_eligible_leaves():
    model = Model(q=layer(), k=layer(out_features=1024), gate=layer(out_features=17408),
                  down=layer(in_features=17408, out_features=5120), o=layer(group_size=32))
    assert enable_small_m_quantized_matmul(model) == 3
    assert [model.leaf(n).is_small_m for n in ("q", "k", "gate", "down", "o")] == [
        True, False, True, True, False]
    assert len(model) == 5


def test_wrapping_an_ineligible_layer_keeps_the_stock_path():
    """SmallMQuantizedLinear's initialiser is public; wrapping an ineligible layer must not
    route it to the kernel (SmallMQuantizedMatmul.swift:236-240)."""
    wrapped = SmallMQuantizedLinear(layer(out_features=2048))
    assert wrapped.is_small_m
    assert not SmallMQuantizedMatmul.is_eligible(wrapped)


def test_context_free_layer_cannot_be_called():
    lay = layer()
    with pytest.raises(dflash_qmm.DfqError) as e:
        lay.lib.dfq_linear_forward  # noqa: B018 -- symbol present
        import ctypes
        rc = lay.lib.dfq_linear_forward(lay._h, None, 0, 8, None, None, 0, None, None)
        dflash_qmm._check(rc, "dfq_linear_forward")
    assert e.value.status == 6


def test_leaf_views_do_not_own_the_model_leaves():
    """A leaf fetched from the model is a view: dropping it must not destroy the leaf."""
    import gc
    model = Model(projection=layer(bits=4), other=layer(bits=8))
    for _ in range(50):
        v = model.projection
        assert v.shape == (4096, 1024) and not v.is_small_m
        del v
        gc.collect()
    assert len(model) == 2
    assert enable_small_m_quantized_matmul(model) == 2
    for _ in range(50):
        assert model.projection.is_small_m and model.other.is_small_m
        gc.collect()
    assert enable_small_m_quantized_matmul(model) == 0


def test_a_leaf_set_at_two_paths_is_owned_once():
    """A tied layer: one handle set at two paths, and a handle that dfq_model_leaf returned set
    again.  The model must free each handle once (run in a child process with glibc's heap
    checks on, where a double free aborts)."""
    import subprocess
    import sys
    code = r'''
import ctypes, dflash_qmm
lib = dflash_qmm.load_library()
fake = 1 << 40
d = dflash_qmm._LinearDesc(fake, fake, fake, None, 4096, 1024, 4, 64, 1, dflash_qmm.BF16)
h = ctypes.c_void_p()
assert lib.dfq_linear_create(None, ctypes.byref(d), ctypes.byref(h)) == 0
m = ctypes.c_void_p()
assert lib.dfq_model_create(ctypes.byref(m)) == 0
assert lib.dfq_model_set_leaf(m, b"model.embed.proj", h) == 0
assert lib.dfq_model_set_leaf(m, b"lm_head.proj", h) == 0
lib.dfq_model_leaf.restype = ctypes.c_void_p
again = lib.dfq_model_leaf(m, b"lm_head.proj")
assert again == h.value
assert lib.dfq_model_set_leaf(m, b"tied.again", ctypes.c_void_p(again)) == 0
assert lib.dfq_model_leaf_count(m) == 3
assert lib.dfq_enable_small_m_quantized_matmul(m) == 3
assert lib.dfq_model_destroy(m) == 0
print("ok")
'''
    import os
    env = dict(os.environ, MALLOC_CHECK_="3")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env["PYTHONPATH"] = os.pathsep.join([os.path.join(root, "dflash-swift_amd"),
                                         env.get("PYTHONPATH", "")])
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0 and "ok" in r.stdout, (r.returncode, r.stderr[-600:])
