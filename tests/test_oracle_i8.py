"""Pins the oracle's int8-activation path (Q8Activation::from_f32, dot_q8_0_i8,
matvec/matmul_q8_0_i8; src/kernel.rs:70-166) before it is trusted as the GPU's checker:
the reference's own tests on its fixtures (kernel.rs:2210-2326) plus closed forms that a
plausible slip fails (round-half-even instead of half-away, a reordered block sum, a
reassociated scale product, f64 accumulation, NaN/Inf handling)."""
import struct

import numpy as np

import oracle as O
from blockpack import q8_blocks


def q8_test_vector(n):
    """kernel.rs:2196-2198, in f32 arithmetic."""
    return np.arange(n, dtype=np.float32) * np.float32(0.037) - np.float32(7.0)


def dequant_activation(scales, qs):
    """kernel.rs:2202-2208."""
    return qs.astype(np.float32) * np.repeat(scales, 32)


def f16(v: float) -> bytes:
    return struct.pack("<e", v)


def block(d: float, ws) -> bytes:
    w = np.zeros(32, np.int8)
    w[: len(ws)] = ws
    return f16(d) + w.tobytes()


# ---- the reference's tests ---------------------------------------------------------------
def test_activation_roundtrip_error_is_bounded():
    x = q8_test_vector(96)
    sc, qs = O.quantize_q8_act(x)
    assert sc.size == 3 and qs.size == 96
    for b in range(3):
        blk = x[32 * b: 32 * b + 32]
        d = sc[b]
        assert abs(d - np.abs(blk).max() / np.float32(127)) < 1e-6
        assert np.all(np.abs(qs[32 * b: 32 * b + 32].astype(np.float32) * d - blk) <= d / 2 + 1e-6)


def test_zero_block_stays_zero():
    sc, qs = O.quantize_q8_act(np.zeros(64, np.float32))
    assert sc.tolist() == [0.0, 0.0] and not qs.any()


def test_i8_dot_matches_dequantized_activation_dot():
    a = q8_blocks(6)
    sc, qs = O.quantize_q8_act(q8_test_vector(len(a) // 34 * 32))
    got = O.dot_q8_0_i8(a, sc, qs)
    want = O.dot(8, a, dequant_activation(sc, qs))
    assert abs(got - want) / max(abs(want), 1.0) < 1e-3


def test_matvec_matches_float_matvec_and_matmul_is_rowwise():
    m, n, rows = 3, 64, 2
    w = q8_blocks(m * n // 32)
    sc, qs = O.quantize_q8_act(q8_test_vector(n))
    got = O.matmul_q8_0_i8(w, m, n, sc, qs, 1)
    want = O.matvec(8, w, m, n, dequant_activation(sc, qs))
    assert np.all(np.abs(got - want) / np.maximum(np.abs(want), 1.0) < 1e-3)
    x = q8_test_vector(rows * n)
    pairs = [O.quantize_q8_act(x[r * n:(r + 1) * n]) for r in range(rows)]
    allsc = np.concatenate([p[0] for p in pairs])
    allq = np.concatenate([p[1] for p in pairs])
    mm = O.matmul_q8_0_i8(w, m, n, allsc, allq, rows)
    rowwise = np.concatenate([O.matmul_q8_0_i8(w, m, n, s, q, 1) for s, q in pairs])
    assert np.array_equal(mm, rowwise)


# ---- closed forms -----------------------------------------------------------------------
def test_power_of_two_scale_is_exact():
    # amax = 127 * 2^-3: d = 2^-3 exactly and every value is a multiple of d
    q = np.arange(-127, 128, 8)[:32].astype(np.float32)
    q[0] = -127
    x = q * np.float32(0.125)
    sc, qs = O.quantize_q8_act(x)
    assert sc[0] == 0.125 and np.array_equal(qs, q.astype(np.int8))


def test_rounding_is_half_away_from_zero():
    x = np.zeros(32, np.float32)
    x[:8] = [127, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5]   # d = 1, inv = 1
    _, qs = O.quantize_q8_act(x)
    assert qs[:8].tolist() == [127, 3, -3, 1, -1, 2, -2, 127]


def test_nan_and_inf_inputs():
    x = np.zeros(64, np.float32)
    x[0], x[1], x[2] = np.nan, 63.5, -127.0          # NaN never wins the max; it quantizes to 0
    x[32], x[33] = np.inf, 5.0                        # d = inf, inv = 0: everything 0
    sc, qs = O.quantize_q8_act(x)
    assert sc[0] == 1.0 and qs[0] == 0 and qs[1] == 64 and qs[2] == -127
    assert np.isinf(sc[1]) and not qs[32:].any()


def test_single_block_dot_is_the_exact_product_for_power_of_two_scales():
    rng = np.random.default_rng(3)
    w = rng.integers(-128, 128, 32).astype(np.int8)
    q = rng.integers(-127, 128, 32).astype(np.int8)
    a = f16(0.125) + w.tobytes()
    isum = int(np.dot(w.astype(np.int64), q.astype(np.int64)))
    assert O.dot_q8_0_i8(a, np.array([2.0 ** -5], np.float32), q) == isum / 256.0


def test_blocks_accumulate_left_to_right_in_f32():
    # terms 2^24, 1, -2^24: left to right gives 0; any other order, or f64, gives 1
    a = block(1024.0, [64] * 4) + block(1.0, [1]) + block(1024.0, [-64] * 4)
    qs = np.zeros(96, np.int8)
    qs[0:4] = 64
    qs[32] = 1
    qs[64:68] = 64
    assert O.dot_q8_0_i8(a, np.ones(3, np.float32), qs) == 0.0
    assert O.dot_q8_0_i8(a[68:] + a[34:68] + a[:34], np.ones(3, np.float32),
                         np.concatenate([qs[64:], qs[32:64], qs[:32]])) == 1.0


def test_scale_product_associates_left():
    f32 = np.float32
    rng = np.random.default_rng(9)
    found = 0
    for _ in range(2000):
        isum = int(rng.integers(1, 30000))
        dw = float(np.float16(rng.uniform(0.01, 2.0)))
        dx = float(f32(rng.uniform(0.001, 1.0)))
        left = f32(f32(f32(isum) * f32(dw)) * f32(dx))
        right = f32(f32(isum) * f32(f32(dw) * f32(dx)))
        if left == right:
            continue
        w = np.zeros(32, np.int8)
        q = np.zeros(32, np.int8)
        # isum as a sum of exact products
        rest, j = isum, 0
        while rest:
            p = min(rest, 127 * 127)
            a_, b_ = 127, p // 127
            if b_ == 0:
                a_, b_ = 1, p
            w[j], q[j] = a_, b_
            rest -= a_ * b_
            j += 1
        assert int(np.dot(w.astype(int), q.astype(int))) == isum
        got = O.dot_q8_0_i8(f16(dw) + w.tobytes(), np.array([dx], np.float32), q)
        assert got == left and got != right
        found += 1
        if found == 5:
            break
    assert found == 5


def test_quantizer_matches_a_vectorised_restatement():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(32 * 500) * np.exp(rng.uniform(-8, 8, 32 * 500))).astype(np.float32)
    x[::97] = 0.0
    sc, qs = O.quantize_q8_act(x)
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    inv = np.where(d > 0, np.float32(1) / np.where(d > 0, d, 1), 0).astype(np.float32)
    r = (xb * inv[:, None]).astype(np.float32).astype(np.float64)
    rq = np.where(r >= 0, np.floor(r + 0.5), np.ceil(r - 0.5))
    assert np.array_equal(sc, d)
    assert np.array_equal(qs.reshape(-1, 32), np.clip(rq, -127, 127).astype(np.int8))
