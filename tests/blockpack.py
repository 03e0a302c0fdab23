"""Independent GGUF block packers and the reference's deterministic test fixtures.

The packers go the other way from the dequantizers: they take the integer fields of a block
(scale bits, quants, sub-scales, mins) and lay them out in bytes following the ggml block
specification (documented in the reference at docs/research/ggml-blocks.md and quant.rs doc
comments). A dequantizer that reads a nibble, a high bit, a sub-scale or a scale offset from
the wrong place fails the encode -> decode round trip against the closed form computed from
the fields, so these pin the oracle rather than restate it.
"""
from __future__ import annotations

import numpy as np

F16_ONE = 0x3C00


def _le16(v: int) -> bytes:
    return int(v & 0xFFFF).to_bytes(2, "little")


def f16_value(h: int) -> float:
    """binary16 bits -> exact value, via numpy's float16 (an independent library routine)."""
    return float(np.array([h], np.uint16).view(np.float16)[0])


# ---- packers: fields -> block bytes --------------------------------------------------
def pack_q4_0(d16: int, q: np.ndarray) -> bytes:
    """q: 32 unsigned 4-bit quants; element j <- low nibble of byte j (j<16), j+16 <- high."""
    q = np.asarray(q, np.uint8)
    qs = (q[:16] & 15) | ((q[16:] & 15) << 4)
    return _le16(d16) + qs.astype(np.uint8).tobytes()


def pack_q5_0(d16: int, q: np.ndarray) -> bytes:
    """q: 32 unsigned 5-bit quants; 5th bit of element j is bit j of the u32 qh."""
    q = np.asarray(q, np.uint32)
    qh = 0
    for j in range(32):
        qh |= int((q[j] >> 4) & 1) << j
    qs = (q[:16] & 15) | ((q[16:] & 15) << 4)
    return _le16(d16) + qh.to_bytes(4, "little") + qs.astype(np.uint8).tobytes()


def pack_q8_0(d16: int, q: np.ndarray) -> bytes:
    return _le16(d16) + np.asarray(q, np.int8).tobytes()


def pack_scales_k4(sc: np.ndarray, mn: np.ndarray) -> bytes:
    """8 six-bit (scale, min) pairs -> the 12-byte K-quant scale array."""
    sc = [int(v) & 63 for v in sc]
    mn = [int(v) & 63 for v in mn]
    b = [0] * 12
    for j in range(4):
        b[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        b[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        b[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return bytes(b)


def pack_q4_k(d16: int, dmin16: int, sc, mn, q: np.ndarray) -> bytes:
    """q: 256 unsigned 4-bit quants. Sub-block s (32 elements) = elements 32s..32s+31; group g
    holds sub-blocks 2g (low nibbles of qs[32g..32g+32]) and 2g+1 (high nibbles)."""
    q = np.asarray(q, np.uint8)
    qs = np.zeros(128, np.uint8)
    for g in range(4):
        qs[32 * g:32 * g + 32] = (q[64 * g:64 * g + 32] & 15) | ((q[64 * g + 32:64 * g + 64] & 15) << 4)
    return _le16(d16) + _le16(dmin16) + pack_scales_k4(sc, mn) + qs.tobytes()


def pack_q5_k(d16: int, dmin16: int, sc, mn, q: np.ndarray) -> bytes:
    """q: 256 unsigned 5-bit quants; the 5th bit of sub-block s, lane l is bit s of qh[l]."""
    q = np.asarray(q, np.uint8)
    qs = np.zeros(128, np.uint8)
    qh = np.zeros(32, np.uint8)
    for g in range(4):
        lo, hi = q[64 * g:64 * g + 32], q[64 * g + 32:64 * g + 64]
        qs[32 * g:32 * g + 32] = (lo & 15) | ((hi & 15) << 4)
        qh |= ((lo >> 4) & 1) << (2 * g)
        qh |= ((hi >> 4) & 1) << (2 * g + 1)
    return _le16(d16) + _le16(dmin16) + pack_scales_k4(sc, mn) + qh.tobytes() + qs.tobytes()


def pack_q6_k(d16: int, sc: np.ndarray, q: np.ndarray) -> bytes:
    """q: 256 unsigned 6-bit quants (value q-32); sc: 16 int8 scales, one per 16 elements."""
    q = np.asarray(q, np.uint8)
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for h in range(2):
        base = 128 * h
        for l in range(32):
            a, b, c, e = q[base + l], q[base + l + 32], q[base + l + 64], q[base + l + 96]
            ql[64 * h + l] = (a & 15) | ((c & 15) << 4)
            ql[64 * h + l + 32] = (b & 15) | ((e & 15) << 4)
            qh[32 * h + l] = (a >> 4) | ((b >> 4) << 2) | ((c >> 4) << 4) | ((e >> 4) << 6)
    return ql.tobytes() + qh.tobytes() + np.asarray(sc, np.int8).tobytes() + _le16(d16)


# ---- closed forms: fields -> exact values ------------------------------------------------
def closed_q4_0(d16, q):
    return np.float32(np.float64(f16_value(d16)) * (np.asarray(q, np.float64) - 8))


def closed_q5_0(d16, q):
    return np.float32(np.float64(f16_value(d16)) * (np.asarray(q, np.float64) - 16))


def closed_q8_0(d16, q):
    return np.float32(np.float64(f16_value(d16)) * np.asarray(q, np.float64))


def closed_k(d16, dmin16, sc, mn, q):
    """y = d*sc*q - dmin*m per 32-element sub-block: exact in f64, then rounded once to f32
    (the reference's f32 statement rounds once: both products are exact)."""
    d, dm = np.float64(f16_value(d16)), np.float64(f16_value(dmin16))
    s = np.repeat(np.asarray(sc, np.float64), 32)
    m = np.repeat(np.asarray(mn, np.float64), 32)
    return (d * s * np.asarray(q, np.float64) - dm * m).astype(np.float32)


def closed_q6_k(d16, sc, q):
    d = np.float64(f16_value(d16))
    s = np.repeat(np.asarray(sc, np.float64), 16)
    return (d * s * (np.asarray(q, np.float64) - 32)).astype(np.float32)


# ---- the reference's deterministic fixture generators -------------------------------------
def q4_blocks(nb: int) -> bytes:
    """kernel.rs:2041-2051 (scale 1.0, bytes (bi*37 + j*13) % 256)."""
    out = bytearray()
    for bi in range(nb):
        out += _le16(F16_ONE) + bytes(((bi * 37 + j * 13) % 256) for j in range(16))
    return bytes(out)


def q8_blocks(nb: int) -> bytes:
    """kernel.rs:2053-2063."""
    out = bytearray()
    for bi in range(nb):
        out += _le16(F16_ONE) + bytes(((bi * 53 + j * 29) % 256) for j in range(32))
    return bytes(out)


def q5_blocks(nb: int) -> bytes:
    """kernel.rs:2066-2078 (qh = (bi * 2654435761 mod 2^32) ^ 0x3C0A5E7F)."""
    out = bytearray()
    for bi in range(nb):
        qh = ((bi * 2654435761) & 0xFFFFFFFF) ^ 0x3C0A5E7F
        out += _le16(F16_ONE) + qh.to_bytes(4, "little") + bytes(((bi * 41 + j * 17) % 256) for j in range(16))
    return bytes(out)


def k_blocks(kind: int, nb: int) -> bytes:
    """kernel.rs:2369-2392: kind 0 = Q4_K (144 B), 1 = Q5_K (176 B), 2 = Q6_K (210 B)."""
    nbytes = {0: 144, 1: 176}.get(kind, 210)
    out = bytearray()
    for bi in range(nb):
        blk = bytearray(nbytes)
        if kind != 2:
            blk[0:4] = bytes([0x00, 0x3C, 0x00, 0x3C])
        else:
            blk[nbytes - 2:nbytes] = bytes([0x00, 0x3C])
        for j in range(nbytes - 4):
            blk[4 + j] = (bi * 91 + j * 7) % 251
        out += blk
    return bytes(out)


def q8_blocks_qmat(m: int, n: int) -> bytes:
    """qmat.rs:370-381 (scale 1.0, i8 ((bi*31 + j*7) % 251) - 125)."""
    out = bytearray()
    for bi in range(m * n // 32):
        out += _le16(F16_ONE) + bytes((((bi * 31 + j * 7) % 251) - 125) & 0xFF for j in range(32))
    return bytes(out)
