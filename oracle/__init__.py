"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY. The oracle restates platinoff/rusty-engine's quantized matmul
arithmetic in C (oracle.c) so the HIP product can be checked against it; it is imported by
tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg, never by the product
package under rusty-engine_amd/.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

# GGML type codes (src/quant.rs:75-88)
F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 6, 8, 12, 13, 14, 30
QUANT_TYPES = (Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K)
TYPE_NAMES = {Q4_0: "Q4_0", Q5_0: "Q5_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K"}
# (elements per block, bytes per block)
GEOM = {Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176),
        Q6_K: (256, 210)}

ORC_OK, ORC_ERR_TYPE, ORC_ERR_SIZE, ORC_ERR_ARG = 0, 1, 2, 3


class OracleError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code
        self.message = message


def build(force: bool = False) -> None:
    """Compile liboracle.so with the Makefile beside this file."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)


_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_sz = C.c_size_t


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.orc_last_error.restype = C.c_char_p
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_block_info.argtypes = [C.c_uint32, C.POINTER(_sz), C.POINTER(_sz)]
        L.orc_bytes_for_numel.argtypes = [C.c_uint32, _sz, C.POINTER(_sz)]
        L.orc_get_scale_min_k4.argtypes = [C.c_int, _u8p, C.POINTER(C.c_uint8), C.POINTER(C.c_uint8)]
        L.orc_dequant.argtypes = [C.c_uint32, C.c_void_p, _sz, C.c_void_p, C.POINTER(_sz)]
        L.orc_quantize_q8_0.argtypes = [_f32p, _sz, _u8p]
        L.orc_quantize_q4_0.argtypes = [_f32p, _sz, _u8p]
        L.orc_quantize_q8_act.argtypes = [_f32p, _sz, _f32p, C.c_void_p]
        L.orc_dot_q8_0_i8.argtypes = [_u8p, _sz, _f32p, C.c_void_p]
        L.orc_dot_q8_0_i8.restype = C.c_float
        L.orc_matmul_q8_0_i8.argtypes = [_u8p, _sz, _sz, _f32p, C.c_void_p, _sz, _f32p]
        L.orc_dot.argtypes = [C.c_uint32, _u8p, _sz, _f32p]
        L.orc_dot.restype = C.c_float
        L.orc_matvec.argtypes = [C.c_uint32, _u8p, _sz, _sz, _f32p, _f32p]
        L.orc_dot_f32.argtypes = [_f32p, _f32p, _sz]
        L.orc_dot_f32.restype = C.c_float
        L.orc_dot_seq.argtypes = [_f32p, _f32p, _sz]
        L.orc_dot_seq.restype = C.c_float
        L.orc_matmul_reuse.argtypes = [C.c_uint32, _u8p, _sz, _sz, _f32p, _sz, _sz, _sz, _sz, _sz, _f32p]
        L.orc_matmul.argtypes = [C.c_uint32, _u8p, _sz, _sz, _f32p, _sz, _f32p]
        L.orc_matmul_blocks.argtypes = [C.c_uint32, _u8p, _sz, _sz, _f32p, _sz, _sz, _f32p]
        L.orc_qmat_row_bytes.argtypes = [C.c_uint32, _sz, C.POINTER(_sz)]
        L.orc_qmat_matvec.argtypes = [C.c_uint32, _u8p, _sz, _sz, _sz, _f32p, _f32p]
        L.orc_qmat_matmul.argtypes = [C.c_uint32, _u8p, _sz, _sz, _sz, _f32p, _sz, _f32p]
        L.orc_qmat_absdot.argtypes = [C.c_uint32, _u8p, _sz, _sz, _sz, _f32p, _sz, _f64p]
        L.orc_sigmoid.argtypes = [C.c_float]
        L.orc_sigmoid.restype = C.c_float
        L.orc_silu.argtypes = [C.c_float]
        L.orc_silu.restype = C.c_float
        L.orc_softmax_in_place.argtypes = [_f32p, _sz]
        L.orc_top_k.argtypes = [_f32p, _sz, _sz, _u32p, _f32p]
        L.orc_top_k.restype = _sz
        L.orc_top_k_sigmoid.argtypes = [_f32p, _sz, _sz, _u32p, _f32p]
        L.orc_top_k_sigmoid.restype = _sz
        for fn in (L.orc_route_group, L.orc_route_noaux_tc):
            fn.argtypes = [_f32p, _sz, C.c_void_p, _sz, _sz, _sz, _sz, _u32p, _f32p]
            fn.restype = _sz
        L.orc_moe_ffn.argtypes = [C.c_uint32, _u8p, _sz, C.c_uint32, _u8p, _sz, C.c_uint32, _u8p, _sz,
                                  _sz, _sz, _sz, _f32p, _sz, _sz, _u32p, _f32p, _f32p]
        L.orc_cpu_matmul.argtypes = [C.c_uint32, _u8p, _sz, _sz, _f32p, _sz, _f32p, C.c_int]
        L.orc_cpu_matvec.argtypes = [C.c_uint32, _u8p, _sz, _sz, _f32p, _f32p, C.c_int]
        L.orc_cpu_has_avx2.restype = C.c_int
        _lib = L
    return _lib


def _check(rc: int) -> None:
    if rc != ORC_OK:
        raise OracleError(rc, lib().orc_last_error().decode())


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(np.frombuffer(bytes(a), np.uint8) if isinstance(a, (bytes, bytearray)) else a,
                                dtype=np.uint8)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- quant.rs ---------------------------------------------------------------------------
def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(h)


def f16_to_f32_bits(h: int) -> int:
    return int(np.float32(lib().orc_f16_to_f32(h)).view(np.uint32))


def f32_to_f16(x: float) -> int:
    return lib().orc_f32_to_f16(x)


def block_info(t: int):
    e, b = _sz(), _sz()
    if lib().orc_block_info(t, C.byref(e), C.byref(b)) != ORC_OK:
        return None
    return e.value, b.value


def bytes_for_numel(t: int, numel: int):
    b = _sz()
    if lib().orc_bytes_for_numel(t, numel, C.byref(b)) != ORC_OK:
        return None
    return b.value


def get_scale_min_k4(j: int, q) -> tuple:
    sc, m = C.c_uint8(), C.c_uint8()
    lib().orc_get_scale_min_k4(j, _u8(q), C.byref(sc), C.byref(m))
    return sc.value, m.value


def dequant(t: int, data) -> np.ndarray:
    d = _u8(data)
    n = _sz()
    _check(lib().orc_dequant(t, d.ctypes.data, d.size, None, C.byref(n)))
    out = np.empty(n.value, np.float32)
    _check(lib().orc_dequant(t, d.ctypes.data, d.size, out.ctypes.data, C.byref(n)))
    return out


def quantize_q8_0(src) -> np.ndarray:
    s = _f32(src)
    out = np.empty(s.size // 32 * 34, np.uint8)
    _check(lib().orc_quantize_q8_0(s, s.size, out))
    return out


def quantize_q4_0(src) -> np.ndarray:
    s = _f32(src)
    out = np.empty(s.size // 32 * 18, np.uint8)
    _check(lib().orc_quantize_q4_0(s, s.size, out))
    return out


def quantize_q8_act(x):
    """Q8Activation::from_f32 (kernel.rs:88-105): (scales f32[n/32], qs i8[n])."""
    s = _f32(x)
    scales = np.empty(max(s.size // 32, 1), np.float32)
    qs = np.empty(max(s.size, 1), np.int8)
    _check(lib().orc_quantize_q8_act(s, s.size, scales, qs.ctypes.data))
    return scales[: s.size // 32], qs[: s.size]


def dot_q8_0_i8(row, scales, qs) -> float:
    """dot_q8_0_i8 (kernel.rs:123-142) over whole Q8_0 blocks."""
    r = _u8(row)
    sc = _f32(scales)
    q = np.ascontiguousarray(qs, np.int8).reshape(-1)
    return float(lib().orc_dot_q8_0_i8(r, r.size // 34, sc, q.ctypes.data))


def matmul_q8_0_i8(w, m: int, n: int, scales, qs, rows: int) -> np.ndarray:
    """matvec/matmul_q8_0_i8 (kernel.rs:145-166): rows x m."""
    ww = _u8(w)
    sc = _f32(scales)
    q = np.ascontiguousarray(qs, np.int8).reshape(-1)
    out = np.empty(max(rows * m, 1), np.float32)
    _check(lib().orc_matmul_q8_0_i8(ww, m, n, sc, q.ctypes.data, rows, out))
    return out[: rows * m]


# ---- kernel.rs ----------------------------------------------------------------------------
def dot(t: int, row, x) -> float:
    r, xv = _u8(row), _f32(x)
    qk, bb = GEOM[t]
    nb = r.size // bb
    assert xv.size >= nb * qk
    return lib().orc_dot(t, r, nb, xv)


def matvec(t: int, w, m: int, n: int, x) -> np.ndarray:
    out = np.empty(m, np.float32)
    _check(lib().orc_matvec(t, _u8(w), m, n, _f32(x), out))
    return out


def dot_f32(a, b) -> float:
    a, b = _f32(a), _f32(b)
    return lib().orc_dot_f32(a, b, a.size)


def dot_seq(a, b) -> float:
    a, b = _f32(a), _f32(b)
    return lib().orc_dot_seq(a, b, a.size)


def matmul_reuse(t, w, m, n, x, rows, tile=96, group=4, w_rows=2, r_block=1024) -> np.ndarray:
    out = np.empty(rows * m, np.float32)
    _check(lib().orc_matmul_reuse(t, _u8(w), m, n, _f32(x), rows, tile, group, w_rows, r_block, out))
    return out


def matmul(t, w, m, n, x, rows) -> np.ndarray:
    out = np.empty(rows * m, np.float32)
    _check(lib().orc_matmul(t, _u8(w), m, n, _f32(x), rows, out))
    return out


def matmul_blocks(t, w, m, n, x, rows, tile=96) -> np.ndarray:
    out = np.empty(rows * m, np.float32)
    _check(lib().orc_matmul_blocks(t, _u8(w), m, n, _f32(x), rows, tile, out))
    return out


# ---- QMat semantics (padded rows allowed) ------------------------------------------------
def qmat_row_bytes(t: int, n: int) -> int:
    rb = _sz()
    _check(lib().orc_qmat_row_bytes(t, n, C.byref(rb)))
    return rb.value


def qmat_matvec(t, w, m, n, x) -> np.ndarray:
    w = _u8(w)
    out = np.empty(m, np.float32)
    _check(lib().orc_qmat_matvec(t, w, w.size, m, n, _f32(x), out))
    return out


def qmat_matmul(t, w, m, n, x, rows) -> np.ndarray:
    w = _u8(w)
    out = np.empty(rows * m, np.float32)
    _check(lib().orc_qmat_matmul(t, w, w.size, m, n, _f32(x), rows, out))
    return out


def qmat_absdot(t, w, m, n, x, rows) -> np.ndarray:
    """sum_k |w_rk x_k| per output, f64 (the scale of the f32-mode tolerance)."""
    w = _u8(w)
    out = np.empty(rows * m, np.float64)
    _check(lib().orc_qmat_absdot(t, w, w.size, m, n, _f32(x), rows, out))
    return out


# ---- moe.rs -------------------------------------------------------------------------------
def sigmoid(x: float) -> float:
    return lib().orc_sigmoid(x)


def silu(x: float) -> float:
    return lib().orc_silu(x)


def softmax(x) -> np.ndarray:
    v = _f32(x).copy()
    lib().orc_softmax_in_place(v, v.size)
    return v


def top_k(scores, k: int):
    s = _f32(scores)
    kk = min(k, s.size)
    ids = np.zeros(max(kk, 1), np.uint32)
    w = np.zeros(max(kk, 1), np.float32)
    n = lib().orc_top_k(s, s.size, k, ids, w)
    return ids[:n].copy(), w[:n].copy()


def top_k_sigmoid(scores, k: int):
    s = _f32(scores)
    kk = min(k, s.size)
    ids = np.zeros(max(kk, 1), np.uint32)
    w = np.zeros(max(kk, 1), np.float32)
    n = lib().orc_top_k_sigmoid(s, s.size, k, ids, w)
    return ids[:n].copy(), w[:n].copy()


def _route_groups(fn, logits, bias, n_groups: int, top_k: int, top_k_group):
    s = _f32(logits)
    b = None if bias is None else _f32(bias)
    kk = min(top_k, s.size)
    ids = np.zeros(max(kk, 1), np.uint32)
    w = np.zeros(max(kk, 1), np.float32)
    n = fn(s, s.size, None if b is None else b.ctypes.data, 0 if b is None else b.size, n_groups, top_k,
           0 if top_k_group is None else top_k_group, ids, w)
    return ids[:n].copy(), w[:n].copy()


def route_group(logits, bias, n_groups: int, top_k: int, top_k_group=None):
    """moe.rs:132-194: group score = the group's summed sigmoid(logit + bias); None = every group."""
    return _route_groups(lib().orc_route_group, logits, bias, n_groups, top_k, top_k_group)


def route_noaux_tc(logits, bias, n_groups: int, top_k: int, top_k_group=None):
    """moe.rs:196-268: group score = the sum of the group's two best sigmoid(logit + bias)."""
    return _route_groups(lib().orc_route_noaux_tc, logits, bias, n_groups, top_k, top_k_group)


def moe_ffn(gate_t, gate, up_t, up, down_t, down, n_experts, hidden, inter, x, tokens, k, ids,
            weights) -> np.ndarray:
    """Quantized expert FFN + routing-order combine for `tokens` tokens (moe.rs:288-388)."""
    gate, up, down = _u8(gate), _u8(up), _u8(down)
    out = np.empty(tokens * hidden, np.float32)
    _check(lib().orc_moe_ffn(gate_t, gate, gate.size // n_experts, up_t, up, up.size // n_experts,
                             down_t, down, down.size // n_experts, n_experts, hidden, inter,
                             _f32(x), tokens, k, np.ascontiguousarray(ids, np.uint32),
                             _f32(weights), out))
    return out


def moe_ffn_shared(gate_t, gate, up_t, up, down_t, down, n_experts, hidden, inter, x, tokens, k, ids,
                   weights, shared) -> np.ndarray:
    """moe_layer_forward with a shared expert (moe.rs:360-388): the routed sum of moe_ffn, then the
    shared expert's FFN (expert_ffn, moe.rs:286-300) added verbatim per element (moe.rs:380-385).
    shared = (gate_t, gate, up_t, up, down_t, down, inter). The shared FFN is moe_ffn over one
    expert with weight 1 (the routed combine then yields 0 + 1 * v = v exactly)."""
    routed = moe_ffn(gate_t, gate, up_t, up, down_t, down, n_experts, hidden, inter, x, tokens, k, ids, weights)
    sg_t, sg, su_t, su, sd_t, sd, sinter = shared
    own = moe_ffn(sg_t, sg, su_t, su, sd_t, sd, 1, hidden, sinter, x, tokens, 1, np.zeros(tokens, np.uint32),
                  np.ones(tokens, np.float32))
    return (routed + own).astype(np.float32)


# ---- CPU baseline -------------------------------------------------------------------------
def cpu_has_avx2() -> bool:
    return bool(lib().orc_cpu_has_avx2())


def cpu_matmul(t, w, m, n, x, rows, threads=0) -> np.ndarray:
    out = np.empty(rows * m, np.float32)
    _check(lib().orc_cpu_matmul(t, _u8(w), m, n, _f32(x), rows, out, threads))
    return out


def cpu_matvec(t, w, m, n, x, threads=0) -> np.ndarray:
    out = np.empty(m, np.float32)
    _check(lib().orc_cpu_matvec(t, _u8(w), m, n, _f32(x), out, threads))
    return out
