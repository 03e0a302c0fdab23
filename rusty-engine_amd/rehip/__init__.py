"""Python mirror of rusty-engine's quantized-matrix interface over librehip's C ABI.

`QMat` follows src/qmat.rs: `QMat.from_bytes(ggml_type, bytes, m, n)` (qmat.rs:52-59),
`.matvec(x)` (qmat.rs:80), `.matmul(x, rows)` (qmat.rs:169), `.rows()` / `.cols()`
(qmat.rs:62-73). Errors the reference reports by panicking (unknown type, kernel.rs:2006, 2027) or
through `EngineError` (sizes, quant.rs:402-447) raise `RehipError` with the library's message.
`MoeExperts.forward` mirrors the expert half of moe_layer_forward (moe.rs:360-388) on
router-chosen experts.

The compute runs only on the GPU through librehip.so; there is no CPU fallback. Importing this
module without the built library raises, and every call on a machine without a gfx950 GPU
returns RE_ERR_NODEV.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG, "librehip.so")

Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = 2, 6, 8, 12, 13, 14
QUANT_TYPES = (Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K)
GEOM = {Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176),
        Q6_K: (256, 210)}
TYPE_NAMES = {Q4_0: "Q4_0", Q5_0: "Q5_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K"}
# Unquantized weights (QMat::F32 and the Quant arms without a fused kernel, src/qmat.rs:31-41):
# element size in bytes.
F32, F16, BF16 = 0, 1, 30
DENSE_TYPES = {F32: 4, F16: 2, BF16: 2}
TYPE_NAMES.update({F32: "F32", F16: "F16", BF16: "BF16"})

RE_OK, RE_ERR_TYPE, RE_ERR_SIZE, RE_ERR_ARG, RE_ERR_HIP, RE_ERR_NODEV = 0, 1, 2, 3, 4, 5
MODE_BF16, MODE_F32 = 0, 1

# every symbol include/rehip.h declares
EXPORTS = ("re_init", "re_last_error", "re_version", "re_row_bytes", "re_tiled_bytes", "re_repack",
           "re_qmat_create", "re_qmat_destroy", "re_qmat_rows", "re_qmat_cols", "re_qmat_type",
           "re_qmat_matvec", "re_qmat_matmul", "re_qmat_matvec_dev", "re_qmat_matmul_dev",
           "re_qmat_dequant_dev", "re_dequant", "re_moe_create", "re_moe_destroy", "re_moe_forward",
           "re_moe_forward_dev", "re_qmat_matvec_ex_dev", "re_rmsnorm_dev", "re_rope_dev", "re_kv_append_dev",
           "re_attention_dev", "re_add_dev", "re_swiglu_dev", "re_argmax_dev", "re_embed_dev", "re_pos_add_dev",
           "re_ffn_create", "re_ffn_destroy", "re_ffn_forward_dev", "re_attention_work_bytes",
           "re_qkv_rope_append_dev", "re_decode_advance_dev",
           "re_qmat_create_stacked", "re_qmat_count", "re_qmat_matvec_stacked_dev", "re_moe_router_logits_dev",
           "re_moe_route_dev", "re_moe_forward_routed_dev", "re_moe_layer_dev",
           "re_gguf_open", "re_gguf_close", "re_gguf_version", "re_gguf_kv_count", "re_gguf_tensor_count",
           "re_gguf_alignment", "re_gguf_data_offset", "re_gguf_data_start", "re_gguf_kv", "re_gguf_get_int",
           "re_gguf_get_float", "re_gguf_get_str", "re_gguf_get_array", "re_gguf_tensor_info",
           "re_gguf_find_tensor", "re_gguf_tensor_data", "re_qmat_from_gguf", "re_moe_from_gguf",
           "re_quantize_q8_act", "re_quantize_q8_act_dev", "re_qmat_matmul_i8", "re_qmat_matmul_i8_dev",
           "re_attention_decode_dev", "re_qmat_gemv_plan", "re_qmat_matmul_noalloc_dev", "re_moe_set_shared",
           "re_rope_table_dev", "re_moe_route_group_dev", "re_moe_layer_group_dev")
GEMV_KERNELS = {0: "split", 1: "rows", 2: "tile", 3: "dense"}


class RehipError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


_lib = None
_sz = C.c_size_t
_vp = C.c_void_p


def lib() -> C.CDLL:
    """Load librehip.so (built by `make -C rusty-engine_amd`)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RehipError(RE_ERR_ARG, f"{LIB_PATH} is not built (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        L.re_init.restype = C.c_int
        L.re_last_error.restype = C.c_char_p
        L.re_version.restype = C.c_char_p
        L.re_row_bytes.argtypes = [C.c_uint32, _sz, C.POINTER(_sz)]
        L.re_tiled_bytes.argtypes = [C.c_uint32, _sz, _sz, C.POINTER(_sz)]
        L.re_repack.argtypes = [C.c_uint32, _vp, _sz, _sz, _sz, _vp, _sz]
        L.re_qmat_create.argtypes = [C.c_uint32, _vp, _sz, _sz, _sz, C.POINTER(_vp)]
        L.re_qmat_destroy.argtypes = [_vp]
        L.re_qmat_destroy.restype = None
        for f in ("re_qmat_rows", "re_qmat_cols"):
            getattr(L, f).argtypes = [_vp]
            getattr(L, f).restype = _sz
        L.re_qmat_type.argtypes = [_vp]
        L.re_qmat_type.restype = C.c_uint32
        L.re_qmat_matvec.argtypes = [_vp, _vp, _vp]
        L.re_qmat_matmul.argtypes = [_vp, _vp, _sz, _vp, C.c_int]
        L.re_qmat_matvec_dev.argtypes = [_vp, _vp, _vp, _vp]
        L.re_qmat_matmul_dev.argtypes = [_vp, _vp, _sz, _vp, C.c_int, _vp]
        L.re_qmat_dequant_dev.argtypes = [_vp, _vp, _vp]
        L.re_dequant.argtypes = [C.c_uint32, _vp, _sz, _vp, _sz]
        L.re_moe_create.argtypes = [C.c_uint32, _vp, _sz, C.c_uint32, _vp, _sz, C.c_uint32, _vp, _sz,
                                    _sz, _sz, _sz, C.POINTER(_vp)]
        L.re_moe_destroy.argtypes = [_vp]
        L.re_moe_destroy.restype = None
        L.re_moe_forward.argtypes = [_vp, _vp, _sz, _sz, _vp, _vp, _vp, C.c_int]
        L.re_moe_forward_dev.argtypes = [_vp, _vp, _sz, _sz, _vp, _vp, _vp, C.c_int, _vp]
        L.re_moe_set_shared.argtypes = [_vp, C.c_uint32, _vp, _sz, C.c_uint32, _vp, _sz, C.c_uint32, _vp, _sz, _sz]
        L.re_moe_router_logits_dev.argtypes = [_vp, _vp, _sz, _sz, _sz, _vp, _vp]
        L.re_moe_route_dev.argtypes = [_vp, _sz, _sz, _sz, C.c_int, _vp, _vp, _vp]
        L.re_moe_forward_routed_dev.argtypes = [_vp, _vp, _sz, _sz, _vp, _vp, _vp, C.c_int, _vp]
        L.re_moe_layer_dev.argtypes = [_vp, _vp, _sz, _vp, _sz, C.c_int, _vp, C.c_int, _vp]
        L.re_moe_route_group_dev.argtypes = [_vp, _sz, _sz, _sz, C.c_int, _vp, _sz, _sz, _sz, _vp, _vp, _vp]
        L.re_moe_layer_group_dev.argtypes = [_vp, _vp, _sz, _vp, _sz, C.c_int, _vp, _sz, _sz, _sz, _vp, C.c_int, _vp]
        L.re_qmat_create_stacked.argtypes = [C.c_uint32, _vp, _sz, _sz, _sz, _sz, C.POINTER(_vp)]
        L.re_qmat_count.argtypes = [_vp]
        L.re_qmat_count.restype = _sz
        L.re_qmat_matvec_stacked_dev.argtypes = [_vp, _sz, _sz, _vp, _sz, _vp, _sz, _vp]
        L.re_qmat_matvec_ex_dev.argtypes = [_vp, _vp, _vp, C.c_float, _vp, _vp, _vp, _vp]
        L.re_rmsnorm_dev.argtypes = [_vp, _vp, _sz, _sz, C.c_float, _vp, _vp]
        L.re_rope_dev.argtypes = [_vp, _sz, _sz, _sz, C.c_float, _vp, C.c_int, _vp]
        L.re_kv_append_dev.argtypes = [_vp, _vp, _sz, _sz, _vp, _vp, _sz, _vp, _vp]
        L.re_attention_work_bytes.argtypes = [_sz, _sz, _sz, _sz]
        L.re_attention_work_bytes.restype = _sz
        L.re_attention_dev.argtypes = [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _vp, _vp, _sz, _vp, _vp]
        L.re_qkv_rope_append_dev.argtypes = [_vp, _sz, _vp, _sz, _vp, _sz, _vp, _vp, _vp, _sz, _sz, _sz, _sz,
                                             C.c_float, _vp, _vp, _vp, _vp, _sz, _vp]
        L.re_decode_advance_dev.argtypes = [_vp, _vp, _vp, C.c_int, _vp, _sz, _vp]
        L.re_add_dev.argtypes = [_vp, _vp, _sz, _sz, _vp, _vp]
        L.re_swiglu_dev.argtypes = [_vp, _vp, _vp, _sz, _vp]
        L.re_argmax_dev.argtypes = [_vp, _sz, _vp, _vp]
        L.re_embed_dev.argtypes = [_vp, _sz, _sz, _vp, _sz, _vp, _vp]
        L.re_pos_add_dev.argtypes = [_vp, C.c_int, _vp]
        L.re_ffn_create.argtypes = [_vp, _vp, C.POINTER(_vp)]
        L.re_ffn_destroy.argtypes = [_vp]
        L.re_ffn_destroy.restype = None
        L.re_ffn_forward_dev.argtypes = [_vp, _vp, _vp, C.c_float, _vp, _vp]
        L.re_gguf_open.argtypes = [C.c_char_p, C.POINTER(_vp)]
        L.re_gguf_close.argtypes = [_vp]
        L.re_gguf_close.restype = None
        for f, r in (("re_gguf_version", C.c_uint32), ("re_gguf_kv_count", _sz), ("re_gguf_tensor_count", _sz),
                     ("re_gguf_alignment", C.c_uint64), ("re_gguf_data_offset", _sz), ("re_gguf_data_start", _sz)):
            getattr(L, f).argtypes = [_vp]
            getattr(L, f).restype = r
        L.re_gguf_kv.argtypes = [_vp, _sz, C.POINTER(C.c_char_p), C.POINTER(C.c_uint32)]
        L.re_gguf_get_int.argtypes = [_vp, C.c_char_p, C.POINTER(C.c_int64)]
        L.re_gguf_get_float.argtypes = [_vp, C.c_char_p, C.POINTER(C.c_double)]
        L.re_gguf_get_str.argtypes = [_vp, C.c_char_p, C.POINTER(_vp), C.POINTER(_sz)]
        L.re_gguf_get_array.argtypes = [_vp, C.c_char_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64)]
        L.re_gguf_tensor_info.argtypes = [_vp, _sz, C.POINTER(C.c_char_p), C.POINTER(C.c_uint32),
                                          C.POINTER(C.c_uint32), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]
        L.re_gguf_find_tensor.argtypes = [_vp, C.c_char_p, C.POINTER(_sz)]
        L.re_gguf_tensor_data.argtypes = [_vp, _sz, C.POINTER(_vp), C.POINTER(_sz)]
        L.re_qmat_from_gguf.argtypes = [_vp, C.c_char_p, _sz, _sz, C.POINTER(_vp)]
        L.re_attention_decode_dev.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, C.c_float, _vp, _vp, _vp,
                                              _vp, _sz, _vp, _sz, _vp, _vp]
        L.re_rope_table_dev.argtypes = [C.c_float, _sz, _sz, _vp, _vp]
        L.re_quantize_q8_act.argtypes = [_vp, _sz, _sz, _vp, _vp]
        L.re_quantize_q8_act_dev.argtypes = [_vp, _sz, _sz, _vp, _vp, _vp]
        L.re_qmat_matmul_i8.argtypes = [_vp, _vp, _vp, _sz, _vp]
        L.re_qmat_matmul_i8_dev.argtypes = [_vp, _vp, _vp, _sz, _vp, _vp]
        L.re_moe_from_gguf.argtypes = [_vp, C.c_char_p, C.c_char_p, C.c_char_p, _sz, _sz, _sz, C.POINTER(_vp)]
        L.re_qmat_gemv_plan.argtypes = [_vp, _sz] + [C.POINTER(C.c_int)] * 4
        L.re_qmat_matmul_noalloc_dev.argtypes = [_vp, _vp, _sz, _vp, C.c_int, _vp]
        _lib = L
    return _lib


def _check(rc: int) -> None:
    if rc != RE_OK:
        raise RehipError(rc, lib().re_last_error().decode())


def _u8(a) -> np.ndarray:
    if isinstance(a, (bytes, bytearray, memoryview)):
        return np.frombuffer(a, np.uint8)
    return np.ascontiguousarray(a, np.uint8).reshape(-1)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).reshape(-1)


def init() -> None:
    _check(lib().re_init())


def version() -> str:
    return lib().re_version().decode()


def row_bytes(ggml_type: int, n: int) -> int:
    out = _sz()
    _check(lib().re_row_bytes(ggml_type, n, C.byref(out)))
    return out.value


def tiled_bytes(ggml_type: int, m: int, n: int) -> int:
    out = _sz()
    _check(lib().re_tiled_bytes(ggml_type, m, n, C.byref(out)))
    return out.value


def repack(ggml_type: int, data, m: int, n: int) -> np.ndarray:
    """Host-side repack into the GPU tiled layout (no GPU needed)."""
    src = _u8(data)
    out = np.empty(tiled_bytes(ggml_type, m, n), np.uint8)
    _check(lib().re_repack(ggml_type, src.ctypes.data, src.size, m, n, out.ctypes.data, out.size))
    return out


def dequant(ggml_type: int, data) -> np.ndarray:
    """GPU dequant of a flat block stream (quant::dequant, src/quant.rs:363)."""
    src = _u8(data)
    qk, bb = GEOM.get(ggml_type, (1, DENSE_TYPES.get(ggml_type, 1)))
    n = src.size // bb * qk if ggml_type in GEOM or ggml_type in DENSE_TYPES else 0
    out = np.empty(max(n, 1), np.float32)
    _check(lib().re_dequant(ggml_type, src.ctypes.data, src.size, out.ctypes.data, n))
    return out[:n]


def _dev_ptr(t) -> int:
    """Device address of a device buffer: a rehip.hip.DeviceBuffer (or a view with a `ptr`), or
    an integer address."""
    return int(t) if isinstance(t, int) else int(t.ptr)


def _stream_ptr(stream) -> int | None:
    """HIP stream handle of a rehip.hip.Stream, an integer handle, or None (the default stream)."""
    if stream is None:
        return None
    return int(stream) if isinstance(stream, int) else int(stream.handle)


class QMat:
    """GPU-resident weight matrix W[m x n] (src/qmat.rs:30-42): quant blocks in the tiled layout,
    or F32/F16/BF16 elements row-major."""

    def __init__(self, handle: int, ggml_type: int, m: int, n: int):
        self._h = C.c_void_p(handle)
        self.ggml_type, self.m, self.n = ggml_type, m, n

    @classmethod
    def from_bytes(cls, ggml_type: int, data, m: int, n: int) -> "QMat":
        src = _u8(data)
        h = _vp()
        _check(lib().re_qmat_create(ggml_type, src.ctypes.data, src.size, m, n, C.byref(h)))
        return cls(h.value, ggml_type, m, n)

    @classmethod
    def from_f32(cls, data, m: int, n: int) -> "QMat":
        """QMat::from_f32 (qmat.rs:45-49): a row-major f32 matrix, products in f32."""
        w = np.ascontiguousarray(data, np.float32).reshape(-1)
        if w.size != m * n:
            raise ValueError("QMat::from_f32: shape mismatch")
        return cls.from_bytes(F32, w.view(np.uint8), m, n)

    @classmethod
    def from_bytes_stacked(cls, ggml_type: int, data, m: int, n: int, count: int) -> "QMat":
        """`count` matrices of m x n, their GGUF bytes one after the other."""
        src = _u8(data)
        h = _vp()
        _check(lib().re_qmat_create_stacked(ggml_type, src.ctypes.data, src.size, m, n, count, C.byref(h)))
        return cls(h.value, ggml_type, m, n)

    @classmethod
    def from_gguf(cls, model: "Gguf", name: str, m: int, n: int) -> "QMat":
        """QMat::from_model (qmat.rs:310-330): tensor `name` (dims [n, m], or [n, m, count] for a
        stack) straight from the mapped file to the device, repacked there."""
        h = _vp()
        _check(lib().re_qmat_from_gguf(model._h, name.encode(), m, n, C.byref(h)))
        t = model.tensor(name)
        return cls(h.value, t.ggml_type, m, n)

    def count(self) -> int:
        return lib().re_qmat_count(self._h)

    def matvec_stacked_dev(self, first: int, count: int, x_dev, x_stride: int, y_dev, y_stride: int,
                           stream=None) -> None:
        """y_b = W_b x_b for matrices first .. first + count - 1, one launch (strides in floats)."""
        _check(lib().re_qmat_matvec_stacked_dev(self._h, first, count, _dev_ptr(x_dev), x_stride, _dev_ptr(y_dev),
                                                y_stride, _stream_ptr(stream)))

    def gemv_plan(self, count: int = 1) -> dict:
        """Launch shape of the GEMV over `count` matrices of the stack (re_qmat_gemv_plan): kernel
        ("tile", "rows", "split" or "dense"), rows per workgroup, waves, half-block streaming."""
        v = [C.c_int() for _ in range(4)]
        _check(lib().re_qmat_gemv_plan(self._h, count, *[C.byref(x) for x in v]))
        return {"kernel": GEMV_KERNELS[v[0].value], "rows_per_group": v[1].value, "waves": v[2].value,
                "half": bool(v[3].value)}

    def rows(self) -> int:
        return lib().re_qmat_rows(self._h)

    def cols(self) -> int:
        return lib().re_qmat_cols(self._h)

    def matvec(self, x) -> np.ndarray:
        xv = _f32(x)
        if xv.size != self.n:
            raise RehipError(RE_ERR_SIZE, f"matvec: x has {xv.size} values, want {self.n}")
        y = np.empty(self.m, np.float32)
        _check(lib().re_qmat_matvec(self._h, xv.ctypes.data, y.ctypes.data))
        return y

    def matmul(self, x, rows: int, mode: int = MODE_BF16) -> np.ndarray:
        xv = _f32(x)
        if xv.size != rows * self.n:
            raise RehipError(RE_ERR_SIZE, f"matmul: X has {xv.size} values, want {rows}x{self.n}")
        y = np.empty(max(rows * self.m, 1), np.float32)
        _check(lib().re_qmat_matmul(self._h, xv.ctypes.data, rows, y.ctypes.data, mode))
        return y[:rows * self.m]

    # device-resident variants (rehip.hip device buffers and streams)
    def matvec_dev(self, x_dev, y_dev, stream=None) -> None:
        _check(lib().re_qmat_matvec_dev(self._h, _dev_ptr(x_dev), _dev_ptr(y_dev), _stream_ptr(stream)))

    def matvec_ex_dev(self, x_dev, y_dev, norm_w=None, eps=0.0, add=None, best=None, stream=None) -> None:
        """y = W rmsnorm(x) + add; each piece optional (see re_qmat_matvec_ex_dev). `best` folds the
        greedy argmax of y into a device uint64 (cleared by decode_advance_dev)."""
        _check(lib().re_qmat_matvec_ex_dev(self._h, _dev_ptr(x_dev), _p(norm_w), eps, _p(add), _dev_ptr(y_dev),
                                           _p(best), _stream_ptr(stream)))

    def matmul_dev(self, x_dev, rows: int, y_dev, mode: int = MODE_BF16, stream=None) -> None:
        _check(lib().re_qmat_matmul_dev(self._h, _dev_ptr(x_dev), rows, _dev_ptr(y_dev), mode,
                                        _stream_ptr(stream)))

    def matmul_noalloc_dev(self, x_dev, rows: int, y_dev, mode: int = MODE_BF16, stream=None) -> None:
        """matmul_dev that allocates nothing (K-split partials in the library's static scratch)."""
        _check(lib().re_qmat_matmul_noalloc_dev(self._h, _dev_ptr(x_dev), rows, _dev_ptr(y_dev), mode,
                                                _stream_ptr(stream)))

    def matmul_i8(self, scales, qs, rows: int) -> np.ndarray:
        """matvec/matmul_q8_0_i8 (kernel.rs:145-166) of a Q8_0 matrix against quantized activation
        rows (scales rows x n/32 f32, qs rows x n int8, as quantize_q8_act returns them)."""
        sc = _f32(scales)
        q = np.ascontiguousarray(qs, np.int8).reshape(-1)
        if sc.size != rows * (self.n // 32) or q.size != rows * self.n:
            raise RehipError(RE_ERR_SIZE, f"matmul_i8: want {rows} rows of {self.n} quantized values")
        y = np.empty(max(rows * self.m, 1), np.float32)
        _check(lib().re_qmat_matmul_i8(self._h, sc.ctypes.data, q.ctypes.data, rows, y.ctypes.data))
        return y[:rows * self.m]

    def matmul_i8_dev(self, scales_dev, qs_dev, rows: int, y_dev, stream=None) -> None:
        _check(lib().re_qmat_matmul_i8_dev(self._h, _dev_ptr(scales_dev), _dev_ptr(qs_dev), rows, _dev_ptr(y_dev),
                                           _stream_ptr(stream)))

    def dequant_dev(self, out_dev, stream=None) -> None:
        _check(lib().re_qmat_dequant_dev(self._h, _dev_ptr(out_dev), _stream_ptr(stream)))

    def close(self) -> None:
        if self._h:
            lib().re_qmat_destroy(self._h)
            self._h = C.c_void_p(0)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- device-resident transformer steps (src/forward.rs, src/infer.rs) --------------------------
def _p(b):
    return _dev_ptr(b) if b is not None else None


def rmsnorm_dev(x, w, rows, d, eps, out, stream=None):
    _check(lib().re_rmsnorm_dev(_p(x), _p(w), rows, d, eps, _p(out), _stream_ptr(stream)))


def rope_dev(x, rows, heads, head_dim, theta, pos, pos_offset=0, stream=None):
    _check(lib().re_rope_dev(_p(x), rows, heads, head_dim, theta, _p(pos), pos_offset, _stream_ptr(stream)))


def kv_append_dev(k, v, rows, kv_dim, kcache, vcache, max_seq, pos, stream=None):
    _check(lib().re_kv_append_dev(_p(k), _p(v), rows, kv_dim, _p(kcache), _p(vcache), max_seq, _p(pos),
                                  _stream_ptr(stream)))


GATE_SOFTMAX, GATE_SIGMOID, GATE_GROUP, GATE_NOAUX_TC = 0, 1, 2, 3


def moe_router_logits_dev(x, router_w, tokens, hidden, n_experts, logits, stream=None):
    _check(lib().re_moe_router_logits_dev(_p(x), _p(router_w), tokens, hidden, n_experts, _p(logits),
                                          _stream_ptr(stream)))


def moe_route_dev(logits, tokens, n_experts, top_k, gate, ids, weights, stream=None):
    _check(lib().re_moe_route_dev(_p(logits), tokens, n_experts, top_k, gate, _p(ids), _p(weights),
                                  _stream_ptr(stream)))


def moe_route_group_dev(logits, tokens, n_experts, top_k, gate, bias, bias_len, n_groups, top_k_group, ids,
                        weights, stream=None):
    """route_group (GATE_GROUP) / route_noaux_tc (GATE_NOAUX_TC) of moe.rs:126-268 on the device;
    bias: None or a device buffer of bias_len f32; top_k_group None or 0 = every group."""
    _check(lib().re_moe_route_group_dev(_p(logits), tokens, n_experts, top_k, gate, _p(bias), bias_len if bias else 0,
                                        n_groups, top_k_group or 0, _p(ids), _p(weights), _stream_ptr(stream)))


def attention_work_bytes(rows, n_heads, head_dim, max_seq) -> int:
    return int(lib().re_attention_work_bytes(rows, n_heads, head_dim, max_seq))


def attention_dev(q, kcache, vcache, rows, n_heads, n_kv_heads, head_dim, max_seq, pos, ctx, work=None,
                  work_bytes=0, stream=None):
    _check(lib().re_attention_dev(_p(q), _p(kcache), _p(vcache), rows, n_heads, n_kv_heads, head_dim, max_seq,
                                  _p(pos), _p(work), work_bytes, _p(ctx), _stream_ptr(stream)))


def qkv_rope_append_dev(q, ldq, k, ldk, v, ldv, bq, bk, bv, rows, n_heads, n_kv_heads, head_dim, theta, pos, qout,
                        kcache, vcache, max_seq, stream=None):
    _check(lib().re_qkv_rope_append_dev(_p(q), ldq, _p(k), ldk, _p(v), ldv, _p(bq), _p(bk), _p(bv), rows, n_heads,
                                        n_kv_heads, head_dim, theta, _p(pos), _p(qout), _p(kcache), _p(vcache),
                                        max_seq, _stream_ptr(stream)))


def attention_decode_dev(q, k, v, bq, bk, bv, n_heads, n_kv_heads, head_dim, theta, pos, kcache, vcache, max_seq,
                         work, work_bytes, ctx, stream=None, rope=None):
    """One decode row: q/k/v bias + RoPE + cache append folded into the key-split attention
    (re_attention_decode_dev); `rope`: None, or a rope_table_dev table with max_seq rows."""
    _check(lib().re_attention_decode_dev(_p(q), _p(k), _p(v), _p(bq), _p(bk), _p(bv), n_heads, n_kv_heads, head_dim,
                                         theta, _p(rope), _p(pos), _p(kcache), _p(vcache), max_seq, _p(work),
                                         work_bytes, _p(ctx), _stream_ptr(stream)))


def rope_table_dev(theta, head_dim, rows, table, stream=None):
    """(cos, sin) of every NeoX rotation pair at positions 0 .. rows - 1 into `table`
    (rows * head_dim floats; re_rope_table_dev)."""
    _check(lib().re_rope_table_dev(theta, head_dim, rows, _p(table), _stream_ptr(stream)))


def decode_advance_dev(best, tok, pos, delta, hist=None, hist_len=0, stream=None):
    _check(lib().re_decode_advance_dev(_p(best), _p(tok), _p(pos), delta, _p(hist), hist_len, _stream_ptr(stream)))


def add_dev(a, b, n, nb, out, stream=None):
    _check(lib().re_add_dev(_p(a), _p(b), n, nb, _p(out), _stream_ptr(stream)))


def swiglu_dev(g, u, h, n, stream=None):
    _check(lib().re_swiglu_dev(_p(g), _p(u), _p(h), n, _stream_ptr(stream)))


def argmax_dev(x, n, idx, stream=None):
    _check(lib().re_argmax_dev(_p(x), n, _p(idx), _stream_ptr(stream)))


def embed_dev(table, n_vocab, d, tok, rows, out, stream=None):
    _check(lib().re_embed_dev(_p(table), n_vocab, d, _p(tok), rows, _p(out), _stream_ptr(stream)))


def pos_add_dev(pos, delta, stream=None):
    _check(lib().re_pos_add_dev(_p(pos), delta, _stream_ptr(stream)))


class Ffn:
    """A gate/up pair read side by side: h = silu(gate x) * (up x) for one row in one launch."""

    def __init__(self, gate: "QMat", up: "QMat"):
        h = _vp()
        _check(lib().re_ffn_create(gate._h, up._h, C.byref(h)))
        self._h = h
        self._keep = (gate, up)

    def forward_dev(self, x_dev, h_dev, norm_w=None, eps=0.0, stream=None) -> None:
        _check(lib().re_ffn_forward_dev(self._h, _dev_ptr(x_dev), _p(norm_w), eps, _dev_ptr(h_dev),
                                        _stream_ptr(stream)))

    def close(self) -> None:
        if self._h:
            lib().re_ffn_destroy(self._h)
            self._h = C.c_void_p(0)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class MoeExperts:
    """All experts of one MoE layer resident on the GPU (gate/up inter x hidden, down hidden x inter)."""

    @classmethod
    def from_gguf(cls, model: "Gguf", gate: str, up: str, down: str, n_experts: int, hidden: int,
                  inter: int) -> "MoeExperts":
        """The layer's stacked expert tensors (ffn_{gate,up,down}_exps, model.rs:372-389) uploaded
        from the mapped file and repacked on the device."""
        h = _vp()
        _check(lib().re_moe_from_gguf(model._h, gate.encode(), up.encode(), down.encode(), n_experts, hidden, inter,
                                      C.byref(h)))
        self = cls.__new__(cls)
        self._h = h
        self.n_experts, self.hidden, self.inter = n_experts, hidden, inter
        return self

    def __init__(self, gate_type, gate, up_type, up, down_type, down, n_experts, hidden, inter):
        g, u, d = _u8(gate), _u8(up), _u8(down)
        h = _vp()
        _check(lib().re_moe_create(gate_type, g.ctypes.data, g.size, up_type, u.ctypes.data, u.size,
                                   down_type, d.ctypes.data, d.size, n_experts, hidden, inter, C.byref(h)))
        self._h = h
        self.n_experts, self.hidden, self.inter = n_experts, hidden, inter

    def set_shared(self, gate_type, gate, up_type, up, down_type, down, inter: int) -> None:
        """Shared expert (moe.rs:380-385): down(silu(gate x) * up x) added to every token's routed sum
        by every forward call; gate/up inter x hidden, down hidden x inter."""
        g, u, d = _u8(gate), _u8(up), _u8(down)
        self._shared = (g, u, d)
        _check(lib().re_moe_set_shared(self._h, gate_type, g.ctypes.data, g.size, up_type, u.ctypes.data, u.size,
                                       down_type, d.ctypes.data, d.size, inter))

    def clear_shared(self) -> None:
        _check(lib().re_moe_set_shared(self._h, 0, None, 0, 0, None, 0, 0, None, 0, 0))
        self._shared = None

    def forward(self, x, tokens: int, top_k: int, ids, weights, mode: int = MODE_BF16) -> np.ndarray:
        xv = _f32(x)
        idv = np.ascontiguousarray(ids, np.uint32).reshape(-1)
        wv = _f32(weights)
        if xv.size != tokens * self.hidden or idv.size != tokens * top_k or wv.size != tokens * top_k:
            raise RehipError(RE_ERR_SIZE, "moe forward: shape mismatch")
        out = np.empty(max(tokens * self.hidden, 1), np.float32)
        _check(lib().re_moe_forward(self._h, xv.ctypes.data, tokens, top_k, idv.ctypes.data, wv.ctypes.data,
                                    out.ctypes.data, mode))
        return out[:tokens * self.hidden]

    def forward_dev(self, x_dev, tokens, top_k, ids, weights, out_dev, mode=MODE_BF16, stream=None) -> None:
        idv = np.ascontiguousarray(ids, np.uint32).reshape(-1)
        wv = _f32(weights)
        _check(lib().re_moe_forward_dev(self._h, _dev_ptr(x_dev), tokens, top_k, idv.ctypes.data,
                                        wv.ctypes.data, _dev_ptr(out_dev), mode, _stream_ptr(stream)))

    def forward_routed_dev(self, x_dev, tokens, top_k, ids_dev, weights_dev, out_dev, mode=MODE_BF16,
                           stream=None) -> None:
        """Expert FFN with device-resident routing (ids int32, weights f32: tokens x top_k)."""
        _check(lib().re_moe_forward_routed_dev(self._h, _dev_ptr(x_dev), tokens, top_k, _dev_ptr(ids_dev),
                                               _dev_ptr(weights_dev), _dev_ptr(out_dev), mode, _stream_ptr(stream)))

    def layer_dev(self, x_dev, tokens, router_w_dev, top_k, gate, out_dev, mode=MODE_BF16, stream=None) -> None:
        """Router logits, top-k routing and the expert FFN, all on the device (moe.rs:360-388)."""
        _check(lib().re_moe_layer_dev(self._h, _dev_ptr(x_dev), tokens, _dev_ptr(router_w_dev), top_k, gate,
                                      _dev_ptr(out_dev), mode, _stream_ptr(stream)))

    def layer_group_dev(self, x_dev, tokens, router_w_dev, top_k, gate, bias_dev, bias_len, n_groups, top_k_group,
                        out_dev, mode=MODE_BF16, stream=None) -> None:
        """Router logits, bias-corrected group routing (GATE_GROUP / GATE_NOAUX_TC) and the expert
        FFN on the device."""
        _check(lib().re_moe_layer_group_dev(self._h, _dev_ptr(x_dev), tokens, _dev_ptr(router_w_dev), top_k, gate,
                                            _p(bias_dev), bias_len if bias_dev else 0, n_groups, top_k_group or 0,
                                            _dev_ptr(out_dev), mode, _stream_ptr(stream)))

    def close(self) -> None:
        if self._h:
            lib().re_moe_destroy(self._h)
            self._h = C.c_void_p(0)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- int8 activations (src/kernel.rs:70-166) ---------------------------------------------------
def quantize_q8_act(x, rows: int = 1):
    """Q8Activation::from_f32 on the GPU for `rows` rows of n values: (scales f32 rows x n/32,
    qs int8 rows x n)."""
    xv = _f32(x)
    n = xv.size // max(rows, 1)
    sc = np.empty(max(rows * (n // 32), 1), np.float32)
    qs = np.empty(max(rows * n, 1), np.int8)
    _check(lib().re_quantize_q8_act(xv.ctypes.data, rows, n, sc.ctypes.data, qs.ctypes.data))
    return sc[: rows * (n // 32)], qs[: rows * n]


def quantize_q8_act_dev(x_dev, rows: int, n: int, scales_dev, qs_dev, stream=None) -> None:
    _check(lib().re_quantize_q8_act_dev(_dev_ptr(x_dev), rows, n, _dev_ptr(scales_dev), _dev_ptr(qs_dev),
                                        _stream_ptr(stream)))


# ---- GGUF files (src/gguf.rs, src/loader.rs) ----------------------------------------------------
GGUF_VALUE_KINDS = ("U8", "I8", "U16", "I16", "U32", "I32", "F32", "Bool", "Str", "Array", "U64", "I64", "F64")


class TensorEntry:
    """One row of the tensor-info table (gguf.rs TensorEntry): name, dims, ggml type, byte offset."""

    def __init__(self, name: str, dims: list, ggml_type: int, offset: int):
        self.name, self.dims, self.ggml_type, self.offset = name, dims, ggml_type, offset

    def numel(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n

    def __repr__(self) -> str:
        return f"TensorEntry({self.name!r}, dims={self.dims}, type={self.ggml_type}, offset={self.offset})"


class Gguf:
    """A GGUF model file mapped read-only (MmapModel, loader.rs:25-130) with its parsed header
    (GgufFile, gguf.rs:120-160). Tensor bytes are views into the mapping; they stay valid while
    this object is open."""

    def __init__(self, path):
        h = _vp()
        _check(lib().re_gguf_open(os.fsencode(path), C.byref(h)))
        self._h = h
        L = lib()
        self.version = L.re_gguf_version(h)
        self.n_kv = L.re_gguf_kv_count(h)
        self.n_tensors = L.re_gguf_tensor_count(h)
        self.data_offset = L.re_gguf_data_offset(h)
        self.data_start = L.re_gguf_data_start(h)
        self.tensors = [self._info(i) for i in range(self.n_tensors)]
        self._by_name = {}
        for t in self.tensors:
            self._by_name.setdefault(t.name, t)

    def _info(self, i: int) -> TensorEntry:
        name, ty, nd = C.c_char_p(), C.c_uint32(), C.c_uint32()
        dims, off = (C.c_uint64 * 8)(), C.c_uint64()
        _check(lib().re_gguf_tensor_info(self._h, i, C.byref(name), C.byref(ty), C.byref(nd), dims, C.byref(off)))
        return TensorEntry(name.value.decode("utf-8", "replace"), [int(dims[d]) for d in range(nd.value)],
                           ty.value, off.value)

    def alignment(self) -> int:
        return lib().re_gguf_alignment(self._h)

    def keys(self) -> list:
        out = []
        for i in range(self.n_kv):
            k, kind = C.c_char_p(), C.c_uint32()
            _check(lib().re_gguf_kv(self._h, i, C.byref(k), C.byref(kind)))
            out.append((k.value.decode("utf-8", "replace"), GGUF_VALUE_KINDS[kind.value]))
        return out

    def get(self, key: str):
        """The first value under `key`: int, float, str, or ("Array", element kind, count);
        None when absent (gguf.rs:139-141)."""
        kinds = dict(self.keys())
        kind = kinds.get(key)
        if kind is None:
            return None
        L, k = lib(), key.encode()
        if kind == "Str":
            p, n = _vp(), _sz()
            _check(L.re_gguf_get_str(self._h, k, C.byref(p), C.byref(n)))
            return C.string_at(p.value, n.value).decode("utf-8", "replace") if n.value else ""
        if kind in ("F32", "F64"):
            v = C.c_double()
            _check(L.re_gguf_get_float(self._h, k, C.byref(v)))
            return v.value
        if kind == "Array":
            ek, cnt = C.c_uint32(), C.c_uint64()
            _check(L.re_gguf_get_array(self._h, k, C.byref(ek), C.byref(cnt)))
            return ("Array", GGUF_VALUE_KINDS[ek.value], cnt.value)
        v = C.c_int64()
        _check(L.re_gguf_get_int(self._h, k, C.byref(v)))
        return bool(v.value) if kind == "Bool" else v.value

    def tensor(self, name: str) -> TensorEntry:
        t = self._by_name.get(name)
        if t is None:
            raise RehipError(RE_ERR_ARG, f"tensor '{name}' not found")
        return t

    def tensor_bytes(self, name: str) -> np.ndarray:
        """Read-only uint8 view of the tensor's bytes in the mapping (loader.rs:95-101)."""
        i = _sz()
        _check(lib().re_gguf_find_tensor(self._h, name.encode(), C.byref(i)))
        p, n = _vp(), _sz()
        _check(lib().re_gguf_tensor_data(self._h, i.value, C.byref(p), C.byref(n)))
        if n.value == 0:
            return np.empty(0, np.uint8)
        a = np.ctypeslib.as_array((C.c_uint8 * n.value).from_address(p.value))
        a.flags.writeable = False
        return a

    def close(self) -> None:
        if self._h:
            lib().re_gguf_close(self._h)
            self._h = _vp(0)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
