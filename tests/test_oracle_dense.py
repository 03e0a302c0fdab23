"""Oracle pinning for unquantized weights: the F32/F16/BF16 arms of quant::dequant
(src/quant.rs:365-397) and QMat's no-fused-kernel product (qmat.rs:132, 146-151, 277-283:
dequant, then moe::matvec's sequential sum, moe.rs:271-277).

Pins: the reference's own known answers (quant.rs:700-723), numpy's IEEE half -> single
conversion over all 65536 bit patterns, the bf16 definition (top half of an f32), and brute
force sequential sums on small matrices; the product is also checked against an f64 product
whose error bound a transposed or dropped operand would break.
"""
import numpy as np
import pytest

import oracle as O

F32, F16, BF16 = 0, 1, 30


def test_bf16_known_answer():
    # quant.rs:703-716: 1.0, 0.5, -2.0 and the truncated f32 of 1234.5
    raw = np.array([0x3F80, 0x3F00, 0xC000, 0x4452], np.uint16).view(np.uint8)
    assert O.dequant(BF16, raw).tolist() == [1.0, 0.5, -2.0, 840.0]
    with pytest.raises(O.OracleError, match="^BF16 data len 3 not a multiple of 2$"):
        O.dequant(BF16, np.zeros(3, np.uint8))


def test_f32_and_f16_partial_words_rejected():
    with pytest.raises(O.OracleError, match="^F32 data len 3 not a multiple of 4$"):
        O.dequant(F32, np.zeros(3, np.uint8))
    with pytest.raises(O.OracleError, match="^F16 data len 5 not a multiple of 2$"):
        O.dequant(F16, np.zeros(5, np.uint8))


def test_f32_is_identity_on_bits():
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 2**32, 4096, dtype=np.uint64).astype(np.uint32)
    got = O.dequant(F32, bits.view(np.uint8)).view(np.uint32)
    assert np.array_equal(got, bits)                 # NaN payloads and -0.0 kept


def test_f16_all_patterns_match_ieee_widening():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.dequant(F16, h.view(np.uint8))
    want = h.view(np.float16).astype(np.float32)
    finite = ~np.isnan(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isnan(got[~finite]))
    # a NaN keeps its sign and its payload in the top mantissa bits
    g = got[~finite].view(np.uint32)
    hh = h[~finite].astype(np.uint32)
    assert np.array_equal(g >> 31, hh >> 15)
    assert np.array_equal((g >> 13) & 0x3FF, hh & 0x3FF)


def test_bf16_all_patterns_are_top_halves():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.dequant(BF16, h.view(np.uint8)).view(np.uint32)
    assert np.array_equal(got, h.astype(np.uint32) << 16)


def seq_matvec(w, x):
    """Brute-force moe::matvec: each row folds from -0.0 in element order, rounding every step."""
    out = np.empty(w.shape[0], np.float32)
    for r in range(w.shape[0]):
        s = np.float32(-0.0)
        for k in range(w.shape[1]):
            s = np.float32(s + np.float32(w[r, k] * x[k]))
        out[r] = s
    return out


@pytest.mark.parametrize("t", [F32, F16, BF16])
def test_qmat_product_is_sequential_sum(t):
    rng = np.random.default_rng(11 + t)
    m, n, rows = 7, 37, 3
    w32 = rng.standard_normal((m, n)).astype(np.float32)
    raw = {F32: w32.view(np.uint8),
           F16: w32.astype(np.float16).view(np.uint8),
           BF16: (w32.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)}[t].reshape(-1)
    w = O.dequant(t, raw).reshape(m, n)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    got = O.qmat_matmul(t, raw, m, n, x, rows).reshape(rows, m)
    for i in range(rows):
        assert np.array_equal(got[i].view(np.uint32), seq_matvec(w, x[i]).view(np.uint32))
    assert np.array_equal(O.qmat_matvec(t, raw, m, n, x[0]), got[0])
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    bound = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    assert np.all(np.abs(got - exact) <= n * 2.0 ** -24 * bound)
    assert O.qmat_row_bytes(t, n) == n * (4 if t == F32 else 2)
    assert np.allclose(O.qmat_absdot(t, raw, m, n, x, rows).reshape(rows, m), bound, rtol=1e-12)


def test_qmat_dense_rejects_wrong_size():
    with pytest.raises(O.OracleError, match="want 24"):
        O.qmat_matvec(BF16, np.zeros(22, np.uint8), 3, 4, np.zeros(4, np.float32))
