"""Python binding of the MI355X small-M affine-quantised matmul (ctypes over the C ABI).

The compute lives in ``libdflash_qmm.so`` (built by ``make -C dflash-swift_amd``): hand-
written gfx950 kernels behind the C ABI of ``include/dflash_qmm.h``.  This module only
marshals pointers; there is no Python or CPU compute path, and importing it raises if the
library is missing.

The classes mirror DFlashKit's Swift surface (paths relative to the reference repository
root):

* :class:`SmallMQuantizedMatmul` -- the window constants, ``is_eligible`` and ``tiles``
  (``Sources/DFlashKit/SmallMQuantizedMatmul.swift:27-225``);
* :class:`QuantizedLinear` / :class:`SmallMQuantizedLinear` -- the stock layer and the
  drop-in subclass that shares its arrays (``:227-293``);
* :func:`enable_small_m_quantized_matmul` -- the module-tree swap (``:295-317``).

Device buffers may be torch tensors (``torch`` is used only as a device allocator here) or
raw integer device pointers.
"""
from __future__ import annotations

import ctypes
import os

__all__ = [
    "BF16", "F16", "F32", "DfqError", "Context", "PackedWeight", "SmallMQuantizedMatmul",
    "QuantizedLinear",
    "SmallMQuantizedLinear", "Model", "enable_small_m_quantized_matmul", "library_path",
    "load_library",
]

BF16, F16, F32 = 0, 1, 2

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_NAME = "libdflash_qmm.so"


def library_path() -> str:
    return os.path.join(_HERE, _LIB_NAME)


class DfqError(RuntimeError):
    """A dfq_* call returned a non-zero status."""

    def __init__(self, status: int, where: str, message: str):
        super().__init__(f"{where}: status {status}: {message}")
        self.status = status


class _LinearDesc(ctypes.Structure):
    _fields_ = [
        ("weight", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("biases", ctypes.c_void_p),
        ("bias", ctypes.c_void_p), ("out_features", ctypes.c_int),
        ("in_features", ctypes.c_int), ("bits", ctypes.c_int), ("group_size", ctypes.c_int),
        ("mode_affine", ctypes.c_int), ("dtype", ctypes.c_int),
    ]


class _TensorInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char_p), ("dtype", ctypes.c_int), ("ndim", ctypes.c_int),
        ("shape", ctypes.c_int64 * 8), ("nbytes", ctypes.c_uint64), ("shard", ctypes.c_int),
        ("offset", ctypes.c_uint64),
    ]


class _LayerInfo(ctypes.Structure):
    _fields_ = [
        ("prefix", ctypes.c_char_p), ("out_features", ctypes.c_int),
        ("in_features", ctypes.c_int), ("bits", ctypes.c_int), ("group_size", ctypes.c_int),
        ("has_biases", ctypes.c_int), ("has_bias", ctypes.c_int), ("dtype", ctypes.c_int),
        ("valid", ctypes.c_int), ("problem", ctypes.c_char_p),
    ]


_WANT_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_char_p, ctypes.c_void_p)


# safetensors dtype names in dfq_st_dtype order
ST_DTYPES = ["BOOL", "U8", "I8", "I16", "U16", "F16", "BF16", "I32", "U32", "F32", "I64", "U64",
             "F64", "F8_E5M2", "F8_E4M3"]

_lib = None


def load_library(path: str | None = None) -> ctypes.CDLL:
    """Load libdflash_qmm.so once; raise loudly if it is not built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or library_path()
    if not os.path.exists(p):
        raise ImportError(f"{p} is not built: run `make -C dflash-swift_amd` (no CPU fallback)")
    lib = ctypes.CDLL(p)
    P, I, S, Z = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)
    PP = ctypes.POINTER(ctypes.c_void_p)
    sig = {
        "dfq_init": ([I, PP], I), "dfq_destroy": ([P], I), "dfq_last_error": ([], ctypes.c_char_p),
        "dfq_status_string": ([I], ctypes.c_char_p), "dfq_abi_version": ([], I),
        "dfq_num_cus": ([P], I), "dfq_malloc": ([P, S, PP], I), "dfq_free": ([P, P], I),
        "dfq_memcpy_h2d": ([P, P, P, S, P], I), "dfq_memcpy_d2h": ([P, P, P, S, P], I),
        "dfq_stream_create": ([P, PP], I), "dfq_stream_destroy": ([P, P], I),
        "dfq_stream_sync": ([P, P], I),
        "dfq_is_eligible": ([I, I, I, I, I, I], I), "dfq_tiles_for": ([I], I),
        "dfq_qmm_supported": ([P, I, I, I, I, I, I, I, I], I),
        "dfq_qmm_workspace_bytes": ([P, I, I, I, I, I, Z], I),
        "dfq_workspace_clear": ([P, P, S, P], I),
        "dfq_qmm": ([P, P, P, P, P, P, P, I, I, I, I, I, I, I, I, P, S, P], I),
        "dfq_qmm_fallback": ([P, P, P, P, P, P, P, I, I, I, I, I, I, I, I, P], I),
        "dfq_qmm_noalloc": ([P, P, P, P, P, P, P, I, I, I, I, I, I, I, I, P], I),
        "dfq_graph_begin": ([P, P], I), "dfq_graph_end": ([P, P, PP], I),
        "dfq_silu_mul": ([P, P, P, I, I, I, P], I),
        "dfq_argmax_accept_workspace_bytes": ([I, ctypes.POINTER(S)], I),
        "dfq_argmax_accept": ([P, P, I, I, I, P, P, P, P, S, P], I),
        "dfq_qmm_argmax_accept_workspace_bytes": ([P, I, I, I, I, I, Z], I),
        "dfq_qmm_argmax_accept": ([P, P, P, P, P, P, P, I, I, I, I, I, I, P, P, P, P, S, P],
                                  I),
        "dfq_graph_launch": ([P, P], I), "dfq_graph_destroy": ([P], I),
        "dfq_graph_compose": ([P, PP, I, PP], I),
        "dfq_packed_bytes": ([I, I, I, I, Z], I),
        "dfq_pack_weights": ([P, P, P, P, I, I, I, I, P, P], I),
        "dfq_qmm_packed": ([P, P, P, P, P, I, I, I, I, I, I, P, S, P], I),
        "dfq_qmm_silu_gate_up_packed": ([P, P, P, P, P, I, I, I, I, I, I, P, S, P], I),
        "dfq_qmm_argmax_accept_packed": ([P, P, P, P, P, I, I, I, I, I, I, P, P, P, P, S, P],
                                         I),
        "dfq_linear_create": ([P, ctypes.POINTER(_LinearDesc), PP], I),
        "dfq_small_m_linear_create": ([P, PP], I), "dfq_linear_destroy": ([P], I),
        "dfq_linear_is_small_m": ([P], I), "dfq_linear_output_dtype": ([P, I], I),
        "dfq_linear_forward": ([P, P, I, I, P, P, S, P, ctypes.POINTER(I)], I),
        "dfq_linear_workspace_bytes": ([P, I, Z], I),
        "dfq_model_create": ([PP], I), "dfq_model_destroy": ([P], I),
        "dfq_model_set_leaf": ([P, ctypes.c_char_p, P], I),
        "dfq_model_leaf": ([P, ctypes.c_char_p], P), "dfq_model_leaf_count": ([P], I),
        "dfq_enable_small_m_quantized_matmul": ([P], I),
        "dfq_debug_plan": ([P, I, I, I, I, I, ctypes.POINTER(I)], I),
        "dfq_debug_make_plan": ([I, I, I, I, I, I, S, ctypes.POINTER(I)], I),
        "dfq_debug_stock_gemv_launches": ([P, I, I, I, I, I, I, ctypes.POINTER(I)], I),
        "dfq_debug_read_units_packed": ([P, P, I, I, I, P, P], I),
        "dfq_debug_read_stream": ([P, P, S, P, P], I),
        "dfq_debug_read_units": ([P, P, P, P, I, I, I, P, P], I),
        "dfq_linear_describe": ([P, ctypes.POINTER(_LinearDesc)], I),
        "dfq_checkpoint_open": ([ctypes.c_char_p, PP], I), "dfq_checkpoint_close": ([P], I),
        "dfq_checkpoint_format": ([P], ctypes.c_char_p),
        "dfq_checkpoint_tensor_count": ([P], I),
        "dfq_checkpoint_tensor": ([P, I, ctypes.POINTER(_TensorInfo)], I),
        "dfq_checkpoint_find": ([P, ctypes.c_char_p, ctypes.POINTER(_TensorInfo)], I),
        "dfq_checkpoint_read": ([P, ctypes.c_char_p, P, S], I),
        "dfq_checkpoint_upload": ([P, P, ctypes.c_char_p, P, S, P], I),
        "dfq_checkpoint_set_quantization": ([P, ctypes.c_char_p, I, I], I),
        "dfq_checkpoint_layer_count": ([P], I),
        "dfq_checkpoint_layer": ([P, I, ctypes.POINTER(_LayerInfo)], I),
        "dfq_checkpoint_load_model": ([P, P, P, _WANT_FN, P, P, ctypes.POINTER(I)], I),
        "dfq_checkpoint_load_model_packed": ([P, P, P, _WANT_FN, P, P, ctypes.POINTER(I)], I),
        "dfq_small_m_linear_pack": ([P, P], I), "dfq_linear_packed": ([P], P),
        "dfq_qmm_silu_gate_up": ([P, P, P, P, P, P, P, I, I, I, I, I, I, P, S, P], I),
        "dfq_interleave_gate_up": ([P, P, P, P, I, S, P], I),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    if lib.dfq_abi_version() != 1:
        raise ImportError("libdflash_qmm.so ABI version mismatch")
    if path is None:
        _lib = lib
    return lib


def _check(status: int, where: str):
    if status:
        lib = load_library()
        raise DfqError(status, where, lib.dfq_last_error().decode(errors="replace"))


def _ptr(a) -> int | None:
    """Device address of a torch tensor, an int, or None."""
    if a is None:
        return None
    if isinstance(a, int):
        return a
    return a.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        try:
            import torch
            if torch.cuda.is_available():
                return torch.cuda.current_stream().cuda_stream or None
        except ImportError:
            pass
        return None
    if isinstance(stream, int):
        return stream or None
    return stream.cuda_stream or None


def dtype_code(t) -> int:
    """dfq dtype code of a torch dtype (or tensor)."""
    import torch
    dt = t.dtype if hasattr(t, "dtype") else t
    return {torch.bfloat16: BF16, torch.float16: F16, torch.float32: F32}[dt]


class Context:
    """A dfq_ctx: the gfx950 code object loaded on one device."""

    def __init__(self, device: int = 0, lib_path: str | None = None):
        self.lib = load_library(lib_path)
        h = ctypes.c_void_p()
        _check(self.lib.dfq_init(device, ctypes.byref(h)), "dfq_init")
        self.handle = h
        self.device = device
        # lazily grown workspaces of the convenience calls, one per stream; a grown one
        # replaces the old, which is kept (a graph or another stream may still hold it)
        self._ws = {}
        self._retired = []

    def close(self):
        if self.handle:
            self.lib.dfq_destroy(self.handle)
            self.handle = None
        self._ws, self._retired = {}, []

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def num_cus(self) -> int:
        return self.lib.dfq_num_cus(self.handle)

    # ---- raw pointer API -------------------------------------------------------------
    def supported(self, M, N, K, bits, gs, xdt=BF16, sdt=None, ydt=None) -> bool:
        sdt = xdt if sdt is None else sdt
        ydt = xdt if ydt is None else ydt
        return bool(self.lib.dfq_qmm_supported(self.handle, M, N, K, bits, gs, xdt, sdt, ydt))

    def workspace_bytes(self, M, N, K, bits, gs) -> int:
        b = ctypes.c_size_t()
        _check(self.lib.dfq_qmm_workspace_bytes(self.handle, M, N, K, bits, gs, ctypes.byref(b)),
               "dfq_qmm_workspace_bytes")
        return b.value

    def workspace_clear(self, ws, nbytes, stream=None):
        _check(self.lib.dfq_workspace_clear(self.handle, _ptr(ws), nbytes, _stream(stream)),
               "dfq_workspace_clear")

    def plan(self, M, N, K, bits, gs) -> dict:
        out = (ctypes.c_int * 15)()
        _check(self.lib.dfq_debug_plan(self.handle, M, N, K, bits, gs, out), "dfq_debug_plan")
        keys = ["T", "SS", "nkb", "Gkb", "nslot_kb", "kr", "lds_bytes", "need_ws", "ch", "umax",
                "chunks", "reduce", "ring", "aligned", "burst"]
        return dict(zip(keys, list(out)))

    def stock_gemv_launches(self, M, N, K, bits, gs, dt=BF16) -> int:
        """GEMV launches the stock path makes for a shape (0: the per-element path)."""
        n = ctypes.c_int(-1)
        _check(self.lib.dfq_debug_stock_gemv_launches(self.handle, M, N, K, bits, gs, dt,
                                                      ctypes.byref(n)),
               "dfq_debug_stock_gemv_launches")
        return n.value

    def read_units(self, w, scales, biases, M, N, K, sink, stream=None):
        """One launch of the fast kernel's own loads for a 4-bit g64 shape (one-k-block
        splits), with no compute; sink holds 12 * num_cus uint32."""
        _check(self.lib.dfq_debug_read_units(self.handle, _ptr(w), _ptr(scales), _ptr(biases),
                                             M, N, K, _ptr(sink), _stream(stream)),
               "dfq_debug_read_units")

    def read_units_packed(self, packed, M, N, K, sink, stream=None):
        """The unit read over a packed array of 4608-byte units (4-bit g64, one k-block)."""
        _check(self.lib.dfq_debug_read_units_packed(self.handle, _ptr(packed), M, N, K,
                                                    _ptr(sink), _stream(stream)),
               "dfq_debug_read_units_packed")

    def read_stream(self, src, nbytes, sink, stream=None):
        """One launch of the plain streaming read of nbytes of src (the bandwidth reference);
        sink holds 8 * num_cus uint32."""
        _check(self.lib.dfq_debug_read_stream(self.handle, _ptr(src), nbytes, _ptr(sink),
                                              _stream(stream)), "dfq_debug_read_stream")

    def qmm_raw(self, x, w, scales, biases, y, M, N, K, bits, gs, xdt, sdt, ydt, lbias=None,
                ws=None, ws_bytes=0, stream=None):
        _check(self.lib.dfq_qmm(self.handle, _ptr(x), _ptr(w), _ptr(scales), _ptr(biases),
                                _ptr(lbias), _ptr(y), M, N, K, bits, gs, xdt, sdt, ydt, _ptr(ws),
                                ws_bytes, _stream(stream)), "dfq_qmm")

    def fallback_raw(self, x, w, scales, biases, y, M, N, K, bits, gs, xdt, sdt, ydt,
                     lbias=None, stream=None):
        _check(self.lib.dfq_qmm_fallback(self.handle, _ptr(x), _ptr(w), _ptr(scales),
                                         _ptr(biases), _ptr(lbias), _ptr(y), M, N, K, bits, gs,
                                         xdt, sdt, ydt, _stream(stream)), "dfq_qmm_fallback")

    # ---- torch conveniences -------------------------------------------------------------
    def workspace(self, nbytes: int, stream=None):
        """A device workspace of at least nbytes for calls on `stream`, owned by this context.

        Each stream gets its own (calls on different streams would race on a shared one).
        A new workspace is zero-filled on `stream` itself, so it is zero before any call
        enqueued after it on that stream; every call leaves it zero again.  A workspace that
        grows is replaced, and the old one is kept until the context closes, since earlier
        work or a captured graph may still use its address.  The convenience calls are
        therefore not capture-safe when they grow a workspace: pass `ws` explicitly to the
        calls a graph captures."""
        import torch
        if nbytes == 0:
            return None
        key = _stream(stream)
        ws = self._ws.get(key)
        if ws is None or ws.numel() < nbytes:
            if ws is not None:
                self._retired.append(ws)
            ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8,
                             device=f"cuda:{self.device}")
            self.workspace_clear(ws, ws.numel(), stream=key)
            self._ws[key] = ws
        return ws

    def qmm(self, x, w, scales, biases, bits, gs, lbias=None, out=None, ws=None, stream=None):
        """y = x @ dequant(w).T on the fast kernel; x [M,K], w [N,K*bits/32] int32/uint32."""
        import torch
        M, K = x.shape
        N = w.shape[0]
        dt = dtype_code(x)
        if out is None:
            out = torch.empty((M, N), dtype=x.dtype, device=x.device)
        need = self.workspace_bytes(M, N, K, bits, gs)
        if ws is None:
            ws = self.workspace(need, stream)
        self.qmm_raw(x, w, scales, biases, out, M, N, K, bits, gs, dt, dtype_code(scales), dt,
                     lbias=lbias, ws=ws, ws_bytes=(ws.numel() if ws is not None else 0),
                     stream=stream)
        return out

    def qmm_silu_gate_up(self, x, w_gu, scales_gu, biases_gu, bits, gs, lbias=None, out=None,
                         ws=None, stream=None):
        """h = silu(x @ Wg.T) * (x @ Wu.T) over a gate|up weight interleaved by 8 rows
        (interleave_gate_up): h is [M, H] with 2H = rows of w_gu."""
        import torch
        M, K = x.shape
        if w_gu.shape[0] % 2:
            raise ValueError("an interleaved gate|up weight has an even number of rows")
        H = w_gu.shape[0] // 2
        if out is None:
            out = torch.empty((M, H), dtype=x.dtype, device=x.device)
        need = self.workspace_bytes(M, 2 * H, K, bits, gs)
        if ws is None:
            ws = self.workspace(need, stream)
        _check(self.lib.dfq_qmm_silu_gate_up(
            self.handle, _ptr(x), _ptr(w_gu), _ptr(scales_gu), _ptr(biases_gu), _ptr(lbias),
            _ptr(out), M, H, K, bits, gs, dtype_code(x), _ptr(ws),
            ws.numel() if ws is not None else 0, _stream(stream)), "dfq_qmm_silu_gate_up")
        return out

    def interleave_gate_up(self, gate, up, stream=None):
        """The gate and up arrays (same shape, rows = H) interleaved in blocks of 8 rows."""
        import torch
        if not (gate.is_contiguous() and up.is_contiguous()) or gate.shape != up.shape:
            raise ValueError("gate and up must be contiguous arrays of one shape")
        H = gate.shape[0]
        out = torch.empty((2 * H,) + tuple(gate.shape[1:]), dtype=gate.dtype, device=gate.device)
        row = gate[0].numel() * gate.element_size()
        _check(self.lib.dfq_interleave_gate_up(self.handle, _ptr(gate), _ptr(up), _ptr(out), H,
                                               row, _stream(stream)), "dfq_interleave_gate_up")
        return out

    def fallback(self, x, w, scales, biases, bits, gs, lbias=None, out=None, out_dtype=None,
                 stream=None):
        import torch
        M, K = x.shape
        N = w.shape[0]
        xdt, sdt = dtype_code(x), dtype_code(scales)
        if out is None:
            ydt = xdt if xdt == sdt else F32
            if out_dtype is not None:
                ydt = dtype_code(out_dtype)
            tdt = {BF16: torch.bfloat16, F16: torch.float16, F32: torch.float32}[ydt]
            out = torch.empty((M, N), dtype=tdt, device=x.device)
        self.fallback_raw(x, w, scales, biases, out, M, N, K, bits, gs, xdt, sdt,
                          dtype_code(out), lbias=lbias, stream=stream)
        return out

    def silu_mul(self, gu, h=None, stream=None):
        """h[m, n] = silu(gu[m, n]) * gu[m, N + n] for a fused gate||up output gu [M, 2N]."""
        import torch
        M, N2 = gu.shape
        N = N2 // 2
        if h is None:
            h = torch.empty((M, N), dtype=gu.dtype, device=gu.device)
        _check(self.lib.dfq_silu_mul(self.handle, _ptr(gu), _ptr(h), M, N, dtype_code(gu),
                                     _stream(stream)), "dfq_silu_mul")
        return h

    def argmax_accept(self, logits, proposals=None, tokens=None, accepted=None, ws=None,
                      stream=None):
        """Greedy accept on the device: (tokens [M] int32, accepted [1] int32) for logits
        [M, V] (M = 1 + drafts) and proposals [M-1] int32 (acceptedPrefix)."""
        import torch
        M, V = logits.shape
        dev = logits.device
        if tokens is None:
            tokens = torch.empty(M, dtype=torch.int32, device=dev)
        if accepted is None:
            accepted = torch.empty(1, dtype=torch.int32, device=dev)
        if ws is None:
            b = ctypes.c_size_t()
            _check(self.lib.dfq_argmax_accept_workspace_bytes(M, ctypes.byref(b)),
                   "dfq_argmax_accept_workspace_bytes")
            ws = torch.zeros(b.value, dtype=torch.uint8, device=dev)
        _check(self.lib.dfq_argmax_accept(self.handle, _ptr(logits), M, V, dtype_code(logits),
                                          _ptr(proposals), _ptr(tokens), _ptr(accepted),
                                          _ptr(ws), ws.numel(), _stream(stream)),
               "dfq_argmax_accept")
        return tokens, accepted

    # ---- the packed layout ---------------------------------------------------------------
    def pack(self, w, scales, biases, bits, gs, stream=None) -> "PackedWeight":
        """The weight, scales and biases of an MLX layer in the packed layout
        (dfq_pack_weights): a new device buffer; the MLX arrays are left as they are."""
        import torch
        N = w.shape[0]
        K = w.shape[1] * 32 // bits
        nb = ctypes.c_size_t()
        _check(self.lib.dfq_packed_bytes(N, K, bits, gs, ctypes.byref(nb)), "dfq_packed_bytes")
        buf = torch.empty(nb.value, dtype=torch.uint8, device=w.device)
        _check(self.lib.dfq_pack_weights(self.handle, _ptr(w), _ptr(scales), _ptr(biases), N, K,
                                         bits, gs, _ptr(buf), _stream(stream)),
               "dfq_pack_weights")
        return PackedWeight(buf, N, K, bits, gs, dtype_code(scales))

    def qmm_packed_raw(self, x, pw, y, M, lbias=None, ws=None, ws_bytes=0, stream=None):
        _check(self.lib.dfq_qmm_packed(self.handle, _ptr(x), _ptr(pw.data), _ptr(lbias), _ptr(y),
                                       M, pw.N, pw.K, pw.bits, pw.gs, pw.dtype, _ptr(ws),
                                       ws_bytes, _stream(stream)), "dfq_qmm_packed")

    def qmm_packed(self, x, pw, lbias=None, out=None, ws=None, stream=None):
        """y = x @ dequant(W).T from a packed weight (pack)."""
        import torch
        M = x.shape[0]
        if out is None:
            out = torch.empty((M, pw.N), dtype=x.dtype, device=x.device)
        if ws is None:
            ws = self.workspace(self.workspace_bytes(M, pw.N, pw.K, pw.bits, pw.gs), stream)
        self.qmm_packed_raw(x, pw, out, M, lbias=lbias, ws=ws,
                            ws_bytes=ws.numel() if ws is not None else 0, stream=stream)
        return out

    def qmm_silu_gate_up_packed(self, x, pw, lbias=None, out=None, ws=None, stream=None):
        """qmm_silu_gate_up over a packed interleaved gate|up weight (N = 2H rows)."""
        import torch
        M, K = x.shape
        H = pw.N // 2
        if out is None:
            out = torch.empty((M, H), dtype=x.dtype, device=x.device)
        if ws is None:
            ws = self.workspace(self.workspace_bytes(M, pw.N, K, pw.bits, pw.gs), stream)
        _check(self.lib.dfq_qmm_silu_gate_up_packed(
            self.handle, _ptr(x), _ptr(pw.data), _ptr(lbias), _ptr(out), M, H, K, pw.bits,
            pw.gs, pw.dtype, _ptr(ws), ws.numel() if ws is not None else 0, _stream(stream)),
            "dfq_qmm_silu_gate_up_packed")
        return out

    def qmm_argmax_accept_packed(self, x, pw, proposals=None, lbias=None, logits=None,
                                 tokens=None, accepted=None, ws=None, stream=None):
        """qmm_argmax_accept over a packed LM-head weight."""
        import torch
        M, K = x.shape
        dev = x.device
        if tokens is None:
            tokens = torch.empty(M, dtype=torch.int32, device=dev)
        if accepted is None:
            accepted = torch.empty(1, dtype=torch.int32, device=dev)
        if ws is None:
            need = self.qmm_argmax_accept_workspace_bytes(M, pw.N, K, pw.bits, pw.gs)
            ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
            self.workspace_clear(ws, ws.numel(), stream=stream)
        _check(self.lib.dfq_qmm_argmax_accept_packed(
            self.handle, _ptr(x), _ptr(pw.data), _ptr(lbias), _ptr(logits), M, pw.N, K,
            pw.bits, pw.gs, pw.dtype, _ptr(proposals), _ptr(tokens), _ptr(accepted), _ptr(ws),
            ws.numel(), _stream(stream)), "dfq_qmm_argmax_accept_packed")
        return tokens, accepted

    def qmm_argmax_accept_workspace_bytes(self, M, V, K, bits, gs) -> int:
        b = ctypes.c_size_t()
        _check(self.lib.dfq_qmm_argmax_accept_workspace_bytes(self.handle, M, V, K, bits, gs,
                                                              ctypes.byref(b)),
               "dfq_qmm_argmax_accept_workspace_bytes")
        return b.value

    def qmm_argmax_accept(self, x, w, scales, biases, bits, gs, proposals=None, lbias=None,
                          logits=None, tokens=None, accepted=None, ws=None, stream=None):
        """The LM head fused with the greedy accept: (tokens [M] int32, accepted [1] int32)
        for x [M, K] against w [V, K*bits/32]; logits [M, V] are written only when given."""
        import torch
        M, K = x.shape
        V = w.shape[0]
        dev = x.device
        if tokens is None:
            tokens = torch.empty(M, dtype=torch.int32, device=dev)
        if accepted is None:
            accepted = torch.empty(1, dtype=torch.int32, device=dev)
        if ws is None:
            need = self.qmm_argmax_accept_workspace_bytes(M, V, K, bits, gs)
            ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
            self.workspace_clear(ws, ws.numel(), stream=stream)
        _check(self.lib.dfq_qmm_argmax_accept(
            self.handle, _ptr(x), _ptr(w), _ptr(scales), _ptr(biases), _ptr(lbias),
            _ptr(logits), M, V, K, bits, gs, dtype_code(x), _ptr(proposals), _ptr(tokens),
            _ptr(accepted), _ptr(ws), ws.numel(), _stream(stream)), "dfq_qmm_argmax_accept")
        return tokens, accepted

    # ---- graphs ---------------------------------------------------------------------------
    def graph_begin(self, stream):
        _check(self.lib.dfq_graph_begin(self.handle, _stream(stream)), "dfq_graph_begin")

    def graph_end(self, stream) -> "Graph":
        g = ctypes.c_void_p()
        _check(self.lib.dfq_graph_end(self.handle, _stream(stream), ctypes.byref(g)),
               "dfq_graph_end")
        return Graph(self.lib, g)

    def graph_compose(self, graphs) -> "Graph":
        """One graph running `graphs` in order (dfq_graph_compose); they stay usable."""
        arr = (ctypes.c_void_p * len(graphs))(*[gr.handle.value for gr in graphs])
        g = ctypes.c_void_p()
        _check(self.lib.dfq_graph_compose(self.handle, arr, len(graphs), ctypes.byref(g)),
               "dfq_graph_compose")
        return Graph(self.lib, g)


class PackedWeight:
    """A weight in the packed layout (Context.pack): its device bytes and format."""

    def __init__(self, data, N, K, bits, gs, dtype):
        self.data, self.N, self.K, self.bits, self.gs, self.dtype = data, N, K, bits, gs, dtype


class Graph:
    def __init__(self, lib, handle):
        self.lib, self.handle = lib, handle

    def launch(self, stream=None):
        _check(self.lib.dfq_graph_launch(self.handle, _stream(stream)), "dfq_graph_launch")

    def close(self):
        if self.handle:
            self.lib.dfq_graph_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class SmallMQuantizedMatmul:
    """The reference enum's statics (SmallMQuantizedMatmul.swift:29-49, 193-207)."""

    minimum_rows = 2   # DFQ_MINIMUM_ROWS: this chip's crossover (the reference's is 6)
    maximum_rows = 16
    rows_per_tile = 8
    minimum_output_features = 4096
    input_feature_multiple = 512
    required_group_size = 64

    @staticmethod
    def is_eligible(layer: "QuantizedLinear") -> bool:
        return bool(load_library().dfq_is_eligible(
            layer.out_features, layer.in_features, layer.bits, layer.group_size,
            int(layer.mode == "affine"), int(layer.biases is not None)))

    @staticmethod
    def tiles(rows: int) -> int:
        return load_library().dfq_tiles_for(rows)


class QuantizedLinear:
    """MLX's QuantizedLinear over device arrays (weight, scales, biases, bias)."""

    def __init__(self, ctx: Context | None, weight, scales, biases, bias=None, group_size=64,
                 bits=4, mode="affine", _handle=None):
        """ctx None gives a layer that can be inspected and swapped but not called."""
        self.ctx = ctx
        self.lib = load_library()
        self.weight, self.scales, self.biases, self.bias = weight, scales, biases, bias
        self.group_size, self.bits, self.mode = group_size, bits, mode
        self.out_features = weight.shape[0]
        self.in_features = weight.shape[1] * 32 // bits
        self._owned = True
        if _handle is not None:
            self._h = _handle
            return
        d = _desc(self)
        h = ctypes.c_void_p()
        _check(self.lib.dfq_linear_create(ctx.handle if ctx else None, ctypes.byref(d),
                                          ctypes.byref(h)), "dfq_linear_create")
        self._h = h

    def __del__(self):
        try:
            if self._h and self._owned:
                self.lib.dfq_linear_destroy(self._h)
            self._h = None
        except Exception:
            pass

    @property
    def is_small_m(self) -> bool:
        return bool(self.lib.dfq_linear_is_small_m(self._h))

    @property
    def packed(self):
        """Device address of the layer's weight in the packed layout, or None."""
        return self.lib.dfq_linear_packed(self._h) or None

    @property
    def shape(self):
        return (self.out_features, self.in_features)

    def output_dtype(self, x):
        import torch
        code = self.lib.dfq_linear_output_dtype(self._h, dtype_code(x))
        return {BF16: torch.bfloat16, F16: torch.float16, F32: torch.float32}[code]

    def __call__(self, x, stream=None):
        """callAsFunction: x[..., in] -> y[..., out]."""
        import torch
        lead = x.shape[:-1]
        rows = 1
        for d in lead:
            rows *= d
        flat = x.reshape(rows, x.shape[-1]).contiguous()
        y = torch.empty((rows, self.out_features), dtype=self.output_dtype(x), device=x.device)
        nb = ctypes.c_size_t()
        _check(self.lib.dfq_linear_workspace_bytes(self._h, rows, ctypes.byref(nb)),
               "dfq_linear_workspace_bytes")
        ws = self.ctx.workspace(nb.value, stream)
        took = ctypes.c_int(0)
        _check(self.lib.dfq_linear_forward(
            self._h, _ptr(flat), dtype_code(x), rows, _ptr(y), _ptr(ws),
            ws.numel() if ws is not None else 0, _stream(stream), ctypes.byref(took)),
            "dfq_linear_forward")
        self.last_took_kernel = bool(took.value)
        return y.reshape(*lead, self.out_features)


def _desc(layer) -> _LinearDesc:
    dt = getattr(layer, "dtype_code", None)
    return _LinearDesc(_ptr(layer.weight), _ptr(layer.scales), _ptr(layer.biases),
                       _ptr(layer.bias), layer.out_features, layer.in_features, layer.bits,
                       layer.group_size, int(layer.mode == "affine"),
                       dt if dt is not None else dtype_code(layer.scales))


class SmallMQuantizedLinear(QuantizedLinear):
    """SmallMQuantizedLinear(other): shares other's arrays (SmallMQuantizedMatmul.swift:243-252)."""

    def __init__(self, other: QuantizedLinear):
        h = ctypes.c_void_p()
        _check(other.lib.dfq_small_m_linear_create(other._h, ctypes.byref(h)),
               "dfq_small_m_linear_create")
        super().__init__(other.ctx, other.weight, other.scales, other.biases, other.bias,
                         other.group_size, other.bits, other.mode, _handle=h)

    def pack(self, stream=None):
        """A packed copy of the weight for the fast kernel's calls (dfq_small_m_linear_pack)."""
        _check(self.lib.dfq_small_m_linear_pack(self._h, _stream(stream)),
               "dfq_small_m_linear_pack")
        return self


class Model:
    """A module tree reduced to named leaf layers (the model owns its own layer handles)."""

    def __init__(self, **leaves: QuantizedLinear):
        self.lib = load_library()
        h = ctypes.c_void_p()
        _check(self.lib.dfq_model_create(ctypes.byref(h)), "dfq_model_create")
        self._h = h
        self._src = {}
        self._paths = []
        self._ctx = None
        self._keep = []  # what the library's leaves point into (a checkpoint)
        for name, leaf in leaves.items():
            self.set_leaf(name, leaf)

    def set_leaf(self, path: str, leaf: QuantizedLinear):
        h = ctypes.c_void_p()
        if leaf.is_small_m:
            _check(self.lib.dfq_small_m_linear_create(leaf._h, ctypes.byref(h)),
                   "dfq_small_m_linear_create")
        else:
            d = _desc(leaf)
            _check(self.lib.dfq_linear_create(leaf.ctx.handle if leaf.ctx else None,
                                              ctypes.byref(d), ctypes.byref(h)),
                   "dfq_linear_create")
        _check(self.lib.dfq_model_set_leaf(self._h, path.encode(), h), "dfq_model_set_leaf")
        self._src[path] = leaf
        if path not in self._paths:
            self._paths.append(path)

    def __getattr__(self, path: str) -> QuantizedLinear:
        if path.startswith("_") or path in ("lib",):
            raise AttributeError(path)
        return self.leaf(path)

    def leaf(self, path: str) -> QuantizedLinear:
        """The current leaf at `path`: a SmallMQuantizedLinear once it has been swapped."""
        h = self.lib.dfq_model_leaf(self._h, path.encode())
        if not h:
            raise KeyError(path)
        h = ctypes.c_void_p(h)
        cls = SmallMQuantizedLinear if self.lib.dfq_linear_is_small_m(h) else QuantizedLinear
        obj = cls.__new__(cls)
        src = self._src.get(path)
        if src is not None:
            QuantizedLinear.__init__(obj, src.ctx, src.weight, src.scales, src.biases, src.bias,
                                     src.group_size, src.bits, src.mode, _handle=h)
        else:
            # a leaf created in the library (a checkpoint load): device addresses as ints
            d = _LinearDesc()
            _check(self.lib.dfq_linear_describe(h, ctypes.byref(d)), "dfq_linear_describe")
            obj.ctx, obj.lib, obj._h = self._ctx, self.lib, h
            obj.weight, obj.scales, obj.biases, obj.bias = d.weight, d.scales, d.biases, d.bias
            obj.group_size, obj.bits = d.group_size, d.bits
            obj.mode = "affine" if d.mode_affine else "other"
            obj.out_features, obj.in_features = d.out_features, d.in_features
            obj.dtype_code = d.dtype
        obj._owned = False  # the model owns the leaf; the view must not destroy it
        obj._model = self   # and keeps the model alive while the view exists
        return obj

    def paths(self) -> list:
        return list(self._paths)

    def __len__(self):
        return self.lib.dfq_model_leaf_count(self._h)

    def __del__(self):
        try:
            if self._h:
                self.lib.dfq_model_destroy(self._h)
                self._h = None
        except Exception:
            pass


def enable_small_m_quantized_matmul(model: Model) -> int:
    """Swap every eligible leaf for a SmallMQuantizedLinear; return how many were swapped."""
    n = model.lib.dfq_enable_small_m_quantized_matmul(model._h)
    if n < 0:
        _check(2, "dfq_enable_small_m_quantized_matmul")
    return n


class Checkpoint:
    """An MLX quantised checkpoint: one .safetensors file or a directory of shards with an
    optional config.json (its "quantization" object gives bits / group size per layer)."""

    def __init__(self, path):
        import weakref
        self.lib = load_library()
        h = ctypes.c_void_p()
        _check(self.lib.dfq_checkpoint_open(os.fsencode(path), ctypes.byref(h)),
               "dfq_checkpoint_open")
        self._h = h
        self._models = weakref.WeakSet()

    @property
    def format(self) -> str:
        return self.lib.dfq_checkpoint_format(self._h).decode()

    @staticmethod
    def _tinfo(t: _TensorInfo) -> dict:
        return {"name": t.name.decode(), "dtype": ST_DTYPES[t.dtype],
                "shape": tuple(t.shape[:t.ndim]), "nbytes": t.nbytes, "shard": t.shard,
                "offset": t.offset}

    def tensors(self) -> list:
        out = []
        for i in range(self.lib.dfq_checkpoint_tensor_count(self._h)):
            t = _TensorInfo()
            _check(self.lib.dfq_checkpoint_tensor(self._h, i, ctypes.byref(t)),
                   "dfq_checkpoint_tensor")
            out.append(self._tinfo(t))
        return out

    def tensor(self, name: str) -> dict:
        t = _TensorInfo()
        _check(self.lib.dfq_checkpoint_find(self._h, name.encode(), ctypes.byref(t)),
               "dfq_checkpoint_find")
        return self._tinfo(t)

    def read(self, name: str):
        """The tensor's bytes as stored (numpy uint8)."""
        import numpy as np
        buf = np.empty(self.tensor(name)["nbytes"], dtype=np.uint8)
        _check(self.lib.dfq_checkpoint_read(self._h, name.encode(), buf.ctypes.data, buf.size),
               "dfq_checkpoint_read")
        return buf

    def upload(self, ctx: Context, name: str, dst, stream=None):
        _check(self.lib.dfq_checkpoint_upload(ctx.handle, self._h, name.encode(), _ptr(dst),
                                              dst.numel() * dst.element_size(), _stream(stream)),
               "dfq_checkpoint_upload")

    def set_quantization(self, bits: int, group_size: int, prefix: str | None = None):
        _check(self.lib.dfq_checkpoint_set_quantization(
            self._h, prefix.encode() if prefix else None, bits, group_size),
            "dfq_checkpoint_set_quantization")

    def layers(self) -> list:
        out = []
        for i in range(self.lib.dfq_checkpoint_layer_count(self._h)):
            L = _LayerInfo()
            _check(self.lib.dfq_checkpoint_layer(self._h, i, ctypes.byref(L)),
                   "dfq_checkpoint_layer")
            out.append({"prefix": L.prefix.decode(), "out_features": L.out_features,
                        "in_features": L.in_features, "bits": L.bits,
                        "group_size": L.group_size, "has_biases": bool(L.has_biases),
                        "has_bias": bool(L.has_bias), "dtype": L.dtype, "valid": bool(L.valid),
                        "problem": L.problem.decode()})
        return out

    def load_model(self, ctx: Context, want=None, model: "Model | None" = None,
                   stream=None, packed=False) -> "Model":
        """Load the quantised layers (those want(prefix) accepts) into device memory as
        stock QuantizedLinear leaves of `model` (a new Model if None); with packed, the
        layers the packed layout serves load in it (dfq_checkpoint_load_model_packed)."""
        model = model if model is not None else Model()
        cb = _WANT_FN(lambda p, _u: int(bool(want(p.decode())))) if want else _WANT_FN()
        n = ctypes.c_int(0)
        fn = "dfq_checkpoint_load_model_packed" if packed else "dfq_checkpoint_load_model"
        _check(getattr(self.lib, fn)(ctx.handle, self._h, model._h, cb, None, _stream(stream),
                                     ctypes.byref(n)), fn)
        model._ctx = ctx
        model._keep.append(self)
        for L in self.layers():
            if L["valid"] and (want is None or want(L["prefix"])) and \
                    L["prefix"] not in model._paths:
                model._paths.append(L["prefix"])
                model._src.pop(L["prefix"], None)
        self._models.add(model)
        self.last_loaded = n.value
        return model

    def close(self):
        if len(self._models):
            raise RuntimeError("models loaded from this checkpoint are still alive")
        if self._h:
            self.lib.dfq_checkpoint_close(self._h)
            self._h = None

    def __del__(self):
        try:
            if self._h:
                self.lib.dfq_checkpoint_close(self._h)
                self._h = None
        except Exception:
            pass
