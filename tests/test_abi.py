"""The C-ABI library on the CPU: it loads, exports every function include/dflash_qmm.h
declares, and its host-side checks and error paths behave without a GPU (no kernel is
launched here)."""
import ctypes
import os
import re

import pytest

import dflash_qmm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dflash_qmm.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(dfq_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_function():
    lib = dflash_qmm.load_library()
    names = declared_functions()
    assert len(names) >= 35
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_abi_version_and_status_strings():
    lib = dflash_qmm.load_library()
    assert lib.dfq_abi_version() == 1
    assert lib.dfq_status_string(0) == b"ok"
    assert lib.dfq_status_string(2) == b"unsupported"


def test_init_without_a_device_fails_cleanly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    lib = dflash_qmm.load_library()
    h = ctypes.c_void_p()
    assert lib.dfq_init(0, ctypes.byref(h)) == 5          # DFQ_ERR_NO_DEVICE
    assert not h.value
    assert b"device" in lib.dfq_last_error()
    with pytest.raises(dflash_qmm.DfqError):
        dflash_qmm.Context(0)


def test_null_arguments_are_rejected():
    lib = dflash_qmm.load_library()
    assert lib.dfq_init(0, None) == 1
    assert lib.dfq_qmm(None, None, None, None, None, None, None, 8, 64, 128, 4, 64, 0, 0, 0,
                       None, 0, None) == 1
    assert lib.dfq_qmm_fallback(None, None, None, None, None, None, None, 1, 1, 64, 4, 64, 0,
                                0, 0, None) == 1
    assert lib.dfq_graph_launch(None, None) == 1
    assert lib.dfq_enable_small_m_quantized_matmul(None) == -1


def test_eligibility_gate_matches_the_reference():
    """SmallMQuantizedMatmul.isEligible (SmallMQuantizedMatmul.swift:193-201)."""
    e = dflash_qmm.load_library().dfq_is_eligible
    assert e(4096, 1024, 4, 64, 1, 1) == 1
    assert e(17408, 5120, 8, 64, 1, 1) == 1
    assert e(4095, 1024, 4, 64, 1, 1) == 0       # N below 4096
    assert e(4096, 1024 + 64, 4, 64, 1, 1) == 0  # K not a multiple of 512
    assert e(4096, 1024, 4, 32, 1, 1) == 0       # group size 32
    assert e(4096, 1024, 3, 64, 1, 1) == 0       # 3-bit
    assert e(4096, 1024, 4, 64, 0, 1) == 0       # not affine
    assert e(4096, 1024, 4, 64, 1, 0) == 0       # no biases


def test_fast_path_shape_checks_need_no_device():
    """dfq_qmm_supported's argument checks run on the host; without a context it says no."""
    lib = dflash_qmm.load_library()
    assert lib.dfq_qmm_supported(None, 8, 17408, 5120, 4, 64, 0, 0, 0) == 0


SWIFT = os.path.join(ROOT, "dflash-swift_amd", "swift", "Sources", "DFlashKitHIP",
                     "SmallMQuantizedMatmulHIP.swift")


def _split_top(text):
    """Comma-separated items of `text` at bracket depth 0."""
    items, depth, cur = [], 0, ""
    for ch in text:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            items.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        items.append(cur)
    return items


def _calls(src, name_re):
    """(name, argument count) of every call matching name_re, parentheses balanced."""
    out = []
    for m in re.finditer(name_re + r"\s*\(", src):
        i, depth = m.end(), 1
        while depth:
            depth += {"(": 1, ")": -1}.get(src[i], 0)
            i += 1
        args = src[m.end():i - 1]
        n = 0 if args.strip() in ("", "void") else len(_split_top(args))
        out.append((m.group(1), n))
    return out


def test_swift_shim_calls_match_the_header():
    """The Swift surface (no Swift toolchain here to build it) calls only functions the header
    declares, each with the header's number of arguments, and reads only its constants."""
    hdr = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    arity = dict(_calls(hdr, r"\b(dfq_[a-z0-9_]+)"))
    src = re.sub(r"//[^\n]*", "", open(SWIFT).read())
    calls = _calls(src, r"\b(dfq_[a-z0-9_]+)")
    assert len(calls) >= 15
    for name, n in calls:
        assert name in arity, name
        assert n == arity[name], (name, n, arity[name])
    consts = set(re.findall(r"\b(DFQ_[A-Z_]+)\b", src))
    for c in consts:
        assert re.search(r"\b%s\b" % c, hdr), c


INTEGRATION = os.path.join(ROOT, "INTEGRATION.md")


def _swift_blocks():
    text = open(INTEGRATION).read()
    return re.findall(r"```swift\n(.*?)```", text, flags=re.S)


def test_integration_swift_snippets_match_the_header_and_the_package():
    """The Swift snippets of INTEGRATION.md compile against what exists: every dfq_* call
    names a function the header declares, with its number of arguments; every DFQ_ constant
    is the header's; every call of the package's own API (greedyAccept, the fused-MLP
    helpers, DFQError, QuantizedLinear ...) uses labels the package declares; and members
    read off a context are ones HIPContext has."""
    blocks = _swift_blocks()
    assert len(blocks) >= 4
    code = "\n".join(re.sub(r"//[^\n]*", "", b) for b in blocks)
    hdr = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    arity = dict(_calls(hdr, r"\b(dfq_[a-z0-9_]+)"))
    calls = _calls(code, r"\b(dfq_[a-z0-9_]+)")
    assert calls
    for name, n in calls:
        assert name in arity, name
        assert n == arity[name], (name, n, arity[name])
    for c in set(re.findall(r"\b(DFQ_[A-Z_]+)\b", code)):
        assert re.search(r"\b%s\b" % c, hdr), c
    pkg = re.sub(r"//[^\n]*", "", open(SWIFT).read())
    # labelled calls: name(label: ...) must match a declaration's first label
    for name, label in re.findall(r"\b([a-zA-Z][A-Za-z0-9]*)\(\s*([a-z][A-Za-z0-9]*):", code):
        if name.startswith("dfq_"):
            continue
        decl = re.search(r"(?:func|init|class|struct)\s+%s\b" % name, pkg) or \
            (name in ("DFQError", "QuantizedLinear", "SmallMQuantizedLinear", "HIPContext",
                      "DeviceBuffer") and re.search(r"\b%s\b" % name, pkg))
        assert decl, name
        if name in ("DFQError", "QuantizedLinear", "HIPContext", "DeviceBuffer"):
            inits = re.findall(r"init\(([a-z][A-Za-z0-9]*)\s*:", pkg)
            assert label in inits, (name, label)
        else:
            m = re.search(r"func\s+%s\(\s*([a-z][A-Za-z0-9]*)" % name, pkg)
            assert m and m.group(1) == label, (name, label)
    # members read off a HIPContext value named ctx or context
    members = set(re.findall(r"\b(?:ctx|context)\.([a-zA-Z][A-Za-z0-9]*)", code))
    ctx_src = pkg[pkg.index("public final class HIPContext"):]
    for m in members:
        assert re.search(r"(?:let|var|func)\s+%s\b" % m, ctx_src), m
