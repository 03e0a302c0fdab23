"""Pins the oracle's dequantizers (src/quant.rs restatement).

Three kinds of check, none of which re-types the oracle's own formula:
- the reference's known-answer tests (quant.rs:459-756), ported value for value;
- the f16 widening against numpy's float16 conversion for all 65,536 patterns (quant.rs:476-499
  uses an f64 closed form for the same purpose);
- encode -> decode round trips: integer fields are packed into bytes by tests/blockpack.py
  (written from the ggml block layout) and must come back as the exact closed-form values.
"""
import numpy as np
import pytest

import oracle as O
from blockpack import (F16_ONE, closed_k, closed_q4_0, closed_q5_0, closed_q6_k, closed_q8_0,
                       pack_q4_0, pack_q4_k, pack_q5_0, pack_q5_k, pack_q6_k, pack_q8_0)


def le16(v):
    return int(v).to_bytes(2, "little")


# ---- quant.rs:459-472 ------------------------------------------------------------------
def test_f16_known_values():
    assert O.f16_to_f32(0x3C00) == 1.0
    assert O.f16_to_f32(0x4000) == 2.0
    assert O.f16_to_f32(0x3800) == 0.5
    assert O.f16_to_f32(0x0000) == 0.0
    assert O.f16_to_f32(0xC000) == -2.0
    assert np.isinf(O.f16_to_f32(0x7C00))
    assert O.f16_to_f32_bits(0x8000) == 0x80000000
    assert O.f16_to_f32(0x0001) == 2.0 ** -24
    assert O.f16_to_f32(0x03FF) == 1023.0 * 2.0 ** -24
    assert np.isnan(O.f16_to_f32(0x7E00))
    assert np.isnan(O.f16_to_f32(0xFE00))


# ---- quant.rs:476-499: every pattern, against an independent conversion ----------------------
def test_f16_all_patterns_bit_exact_against_numpy():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = O.dequant(O.F16, h.tobytes())
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # the f64 closed form the reference uses (quant.rs:478-489), for the non-NaN patterns
    sign = np.where(h >> 15, -1.0, 1.0)
    e = ((h >> 10) & 0x1F).astype(np.int64)
    f = (h & 0x3FF).astype(np.float64)
    v = np.where(e == 0, f / 1024.0 * 2.0 ** -14, (1 + f / 1024.0) * np.power(2.0, e - 15))
    v = np.where((e == 31) & (f == 0), np.inf, v)
    closed = (sign * v).astype(np.float32)
    assert np.array_equal(got[~nan].view(np.uint32), closed[~nan].view(np.uint32))


def test_f32_to_f16_round_trips_every_finite_pattern():
    # quant.rs:48-72 narrows by truncation, so every representable value must come back intact
    for h in range(65536):
        if (h >> 10) & 0x1F == 0x1F and h & 0x3FF:
            continue  # NaN payloads are quieted (0x7E00 | payload)
        assert O.f32_to_f16(O.f16_to_f32(h)) == h, hex(h)
    assert O.f32_to_f16(1e9) == 0x7C00 and O.f32_to_f16(-1e9) == 0xFC00
    assert O.f32_to_f16(1e-12) == 0x0000
    assert O.f32_to_f16(float("nan")) & 0x7E00 == 0x7E00


# ---- quant.rs:501-553 ------------------------------------------------------------------
def test_block_sizes_match_ggml():
    assert O.block_info(2) == (32, 18)
    assert O.block_info(8) == (32, 34)
    assert O.block_info(6) == (32, 22)
    assert O.block_info(12) == (256, 144)
    assert O.block_info(13) == (256, 176)
    assert O.block_info(14) == (256, 210)
    assert O.block_info(999) is None


def test_bytes_for_numel_block_math():
    assert O.bytes_for_numel(2, 64) == 36
    assert O.bytes_for_numel(0, 10) == 40
    assert O.bytes_for_numel(2, 33) is None


# ---- quant.rs:555-616 ------------------------------------------------------------------
def test_q4_0_split_half_and_offset():
    blk = bytearray(18)
    blk[0:2] = le16(0x3C00)
    blk[2] = 0x0F
    out = O.dequant(O.Q4_0, blk)
    assert out.size == 32
    assert out[0] == 7.0 and out[16] == -8.0 and out[1] == -8.0 and out[31] == -8.0


def test_q4_0_all_zero_nibbles_minus_eight():
    blk = bytearray(18)
    blk[0:2] = le16(0x3C00)
    assert np.all(O.dequant(O.Q4_0, blk) == -8.0)


def test_q8_0_signed_values():
    blk = bytearray(34)
    blk[0:2] = le16(0x3C00)
    blk[2] = 0x7F
    blk[3] = 0xFF
    out = O.dequant(O.Q8_0, blk)
    assert out.size == 32 and out[0] == 127.0 and out[1] == -1.0


def test_q5_0_values_and_5th_bit():
    blk = bytearray(22)
    blk[0:2] = le16(0x3C00)
    blk[6:22] = bytes([0x11] * 16)
    out = O.dequant(O.Q5_0, blk)
    assert out.size == 32 and np.all(out == -15.0)
    b2 = bytearray(22)
    b2[0:2] = le16(0x3C00)
    b2[2:6] = (1).to_bytes(4, "little")
    out2 = O.dequant(O.Q5_0, b2)
    assert out2[0] == 0.0 and out2[16] == -16.0
    b3 = bytearray(22)
    b3[0:2] = le16(0x3C00)
    b3[6] = 0xF0
    out3 = O.dequant(O.Q5_0, b3)
    assert out3[0] == -16.0 and out3[16] == -1.0


# ---- quant.rs:618-629 ------------------------------------------------------------------
def test_dequant_dispatch_lengths():
    for t, n in [(2, 17), (6, 21), (12, 143)]:
        with pytest.raises(O.OracleError):
            O.dequant(t, bytes(n))
    with pytest.raises(O.OracleError) as e:
        O.dequant(99, bytes(8))
    assert "no scalar dequant for ggml type 99" in e.value.message
    assert O.dequant(6, bytes(22)).size == 32
    ok = bytearray(18)
    ok[0:2] = le16(0x3C00)
    assert O.dequant(2, ok).size == 32
    assert O.dequant(12, bytes(144)).size == 256


# ---- quant.rs:631-678 ------------------------------------------------------------------
def test_q4_k_zero_block_all_zero():
    b = bytearray(144)
    b[0:2] = le16(0x3C00)
    out = O.dequant(O.Q4_K, b)
    assert out.size == 256 and np.all(out == 0.0)


def test_q4_k_uniform_scale_and_min():
    b = bytearray(144)
    b[0:2] = le16(0x3C00)
    b[2:4] = le16(0x3C00)
    b[4] = 2
    b[8] = 1
    b[16:144] = bytes([0x03] * 128)
    out = O.dequant(O.Q4_K, b)
    assert abs(out[0] - 5.0) < 1e-5 and abs(out[31] - 5.0) < 1e-5
    assert out[32] == 0.0


def test_q5_k_low_group():
    b = bytearray(176)
    b[0:2] = le16(0x3C00)
    b[4] = 1
    b[48:176] = bytes([0x03] * 128)
    out = O.dequant(O.Q5_K, b)
    assert out.size == 256 and abs(out[0] - 3.0) < 1e-5


def test_q6_k_signed_zero_bias():
    b = bytearray(210)
    b[208:210] = le16(0x3C00)
    b[192:208] = bytes([1] * 16)
    out = O.dequant(O.Q6_K, b)
    assert out.size == 256 and np.all(np.abs(out + 32.0) < 1e-5)


# ---- quant.rs:680-724 ------------------------------------------------------------------
def test_dequant_f32_roundtrips_le_bytes():
    data = np.array([1.5, -2.0, 0.125], "<f4").tobytes()
    assert list(O.dequant(0, data)) == [1.5, -2.0, 0.125]


def test_dequant_f16_uses_f16_to_f32():
    data = b"".join(le16(h) for h in [0x3C00, 0x4000, 0xCC00])
    assert list(O.dequant(1, data)) == [1.0, 2.0, -16.0]


def test_dequant_bf16_widens_by_left_shift():
    data = b"".join(le16(h) for h in [0x3F80, 0x3F00, 0xC000, 0x4452])
    assert list(O.dequant(30, data)) == [1.0, 0.5, -2.0, 840.0]
    with pytest.raises(O.OracleError) as e:
        O.dequant(30, bytes(3))
    assert e.value.message == "BF16 data len 3 not a multiple of 2"


def test_dequant_f32_rejects_partial_word():
    with pytest.raises(O.OracleError) as e:
        O.dequant(0, bytes(3))
    assert "F32" in e.value.message


# ---- quant.rs:726-756 ------------------------------------------------------------------
@pytest.mark.parametrize("kind", ["q8_0", "q4_0"])
def test_quantize_round_trip_parity(kind):
    div, levels = (7.0, 127.0) if kind == "q8_0" else (9.0, 7.0)
    src = ((np.arange(64, dtype=np.float32) - 32.0) / np.float32(div)).astype(np.float32)
    q = O.quantize_q8_0(src) if kind == "q8_0" else O.quantize_q4_0(src)
    assert q.size == 2 * (34 if kind == "q8_0" else 18)
    back = O.dequant(O.Q8_0 if kind == "q8_0" else O.Q4_0, q)
    for i in range(64):
        blk = src[(i // 32) * 32:(i // 32 + 1) * 32]
        d = np.float32(np.abs(blk).max()) / np.float32(levels)
        assert abs(src[i] - back[i]) <= d * 0.75 + 1e-6


# ---- encode -> decode round trips against closed forms -----------------------------------
RNG = np.random.default_rng(20260)


def rand_f16_finite(rng, n, scale):
    return (np.abs(rng.standard_normal(n)) * scale).astype(np.float16).view(np.uint16)


def test_roundtrip_q4_0():
    for _ in range(200):
        d = int(rand_f16_finite(RNG, 1, 0.01)[0])
        q = RNG.integers(0, 16, 32)
        assert np.array_equal(O.dequant(O.Q4_0, pack_q4_0(d, q)), closed_q4_0(d, q))


def test_roundtrip_q5_0():
    for _ in range(200):
        d = int(rand_f16_finite(RNG, 1, 0.01)[0])
        q = RNG.integers(0, 32, 32)
        assert np.array_equal(O.dequant(O.Q5_0, pack_q5_0(d, q)), closed_q5_0(d, q))


def test_roundtrip_q8_0():
    for _ in range(200):
        d = int(rand_f16_finite(RNG, 1, 0.01)[0])
        q = RNG.integers(-128, 128, 32)
        assert np.array_equal(O.dequant(O.Q8_0, pack_q8_0(d, q)), closed_q8_0(d, q))


def test_roundtrip_q4_k_and_scale_packing():
    for _ in range(100):
        d, dm = (int(v) for v in rand_f16_finite(RNG, 2, 1e-3))
        sc, mn = RNG.integers(0, 64, 8), RNG.integers(0, 64, 8)
        q = RNG.integers(0, 16, 256)
        blk = pack_q4_k(d, dm, sc, mn, q)
        for j in range(8):
            assert O.get_scale_min_k4(j, np.frombuffer(blk[4:16], np.uint8)) == (sc[j], mn[j])
        assert np.array_equal(O.dequant(O.Q4_K, blk), closed_k(d, dm, sc, mn, q))


def test_roundtrip_q5_k():
    for _ in range(100):
        d, dm = (int(v) for v in rand_f16_finite(RNG, 2, 1e-3))
        sc, mn = RNG.integers(0, 64, 8), RNG.integers(0, 64, 8)
        q = RNG.integers(0, 32, 256)
        assert np.array_equal(O.dequant(O.Q5_K, pack_q5_k(d, dm, sc, mn, q)), closed_k(d, dm, sc, mn, q))


def test_roundtrip_q6_k():
    for _ in range(100):
        d = int(rand_f16_finite(RNG, 1, 1e-3)[0])
        sc = RNG.integers(-128, 128, 16)
        q = RNG.integers(0, 64, 256)
        assert np.array_equal(O.dequant(O.Q6_K, pack_q6_k(d, sc, q)), closed_q6_k(d, sc, q))


def test_roundtrip_subnormal_and_signed_zero_scales():
    # f16 subnormal d widen exactly; a negative-zero d gives signed zeros
    for d in (0x0001, 0x03FF, 0x8000, 0x8001, 0x7BFF):
        q = RNG.integers(0, 16, 32)
        got = O.dequant(O.Q4_0, pack_q4_0(d, q))
        assert np.array_equal(got.view(np.uint32), closed_q4_0(d, q).view(np.uint32))
