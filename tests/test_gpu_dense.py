"""Unquantized weights on the GPU: the F32/F16/BF16 arms of quant::dequant (src/quant.rs:365-397)
and QMat over them (QMat::F32 and the no-fused-kernel arms, src/qmat.rs:31-49, 128-151, 277-305),
through the C ABI, against the oracle.

Bars: dequant bit-exact (NaN payloads included); products |y - y_oracle| <= 2^-10 * sum_k |w_rk x_k|
per output (the oracle folds sequentially, the kernel per lane then over a fixed tree)."""
import numpy as np
import pytest

import ggufw as W
import oracle as O
import rehip
from rehip import hip

pytestmark = pytest.mark.gpu
B = hip.DeviceBuffer
F32_TOL = 2.0 ** -10
DENSE = [rehip.F32, rehip.F16, rehip.BF16]


def _raw(t, w32):
    if t == rehip.F32:
        return np.ascontiguousarray(w32, np.float32).view(np.uint8).reshape(-1)
    if t == rehip.F16:
        return w32.astype(np.float16).view(np.uint8).reshape(-1)
    return (np.ascontiguousarray(w32, np.float32).view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(-1)


def _check_product(got, t, raw, m, n, x, rows):
    want = O.qmat_matmul(t, raw, m, n, x, rows)
    absd = O.qmat_absdot(t, raw, m, n, x, rows)
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= F32_TOL * absd), f"max err/bound {np.max(err / (absd + 1e-30))}"


@pytest.mark.parametrize("t", [rehip.F16, rehip.BF16])
def test_dequant_every_half_pattern_bit_exact(t):
    raw = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.uint8)
    got = rehip.dequant(t, raw)
    assert np.array_equal(got.view(np.uint32), O.dequant(t, raw).view(np.uint32))


def test_dequant_f32_bits_kept():
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 2**32, 100003, dtype=np.uint64).astype(np.uint32)
    assert np.array_equal(rehip.dequant(rehip.F32, bits.view(np.uint8)).view(np.uint32), bits)


def test_dequant_partial_words_rejected():
    for t, name, k, want in [(rehip.F32, "F32", 7, 4), (rehip.F16, "F16", 3, 2), (rehip.BF16, "BF16", 3, 2)]:
        with pytest.raises(rehip.RehipError, match=f"] {name} data len {k} not a multiple of {want}$"):
            rehip.dequant(t, np.zeros(k, np.uint8))


def test_from_f32_matches_plain_matvec():
    # qmat.rs:337-345: quarters and small integers, so every sum is exact
    data = np.arange(12, dtype=np.float32) * 0.25 - 1.0
    q = rehip.QMat.from_f32(data, 3, 4)
    x = np.array([1.0, -2.0, 0.5, 3.0], np.float32)
    assert np.array_equal(q.matvec(x), O.qmat_matvec(rehip.F32, data.view(np.uint8), 3, 4, x))
    assert (q.rows(), q.cols()) == (3, 4)
    q.close()


@pytest.mark.parametrize("t", DENSE)
@pytest.mark.parametrize("m,n", [(1, 1), (70, 131), (896, 896), (5, 4864)])
def test_dense_matvec_matmul(t, m, n):
    rng = np.random.default_rng(m * 7 + n + t)
    raw = _raw(t, rng.standard_normal((m, n)).astype(np.float32))
    q = rehip.QMat.from_bytes(t, raw, m, n)
    assert q.ggml_type == t and (q.rows(), q.cols()) == (m, n)
    x = rng.standard_normal(n).astype(np.float32)
    got = q.matvec(x)
    _check_product(got, t, raw, m, n, x, 1)
    for rows in (2, 5, 15):
        xs = rng.standard_normal((rows, n)).astype(np.float32)
        for mode in (rehip.MODE_F32, rehip.MODE_BF16):     # below 16 rows: f32 products in either mode
            y = q.matmul(xs, rows, mode)
            _check_product(y, t, raw, m, n, xs, rows)
        # a row's output does not depend on the rows beside it, nor on the row-group size
        # (1 or 4 rows per workgroup)
        assert np.array_equal(q.matmul(xs[:1], 1, rehip.MODE_F32), q.matvec(xs[0]))
        assert np.array_equal(q.matmul(xs[:2], 2, rehip.MODE_F32), q.matmul(xs, rows, rehip.MODE_F32)[:2 * m])
    q.close()


@pytest.mark.parametrize("t", DENSE)
@pytest.mark.parametrize("m,n,rows", [(896, 896, 961), (130, 200, 16), (64, 4864, 65), (333, 96, 100),
                                      (896, 4864, 64)])
def test_dense_mfma_gemm(t, m, n, rows):
    """16 rows and up (n % 8 == 0): the MFMA GEMM (with K slices when it has few output tiles). f32
    mode (f32 MFMA) within 2^-10 sum|w x| of the oracle's sequential sum; bf16 mode (operands
    rounded to bf16) within 1e-2 of the norm of an f64 product; a row's outputs do not depend on the
    call's other activation rows."""
    rng = np.random.default_rng(m + n + rows + t)
    raw = _raw(t, rng.standard_normal((m, n)).astype(np.float32))
    q = rehip.QMat.from_bytes(t, raw, m, n)
    xs = rng.standard_normal((rows, n)).astype(np.float32)
    y = q.matmul(xs, rows, rehip.MODE_F32)
    _check_product(y, t, raw, m, n, xs, rows)
    exact = (xs.astype(np.float64) @ O.dequant(t, raw).astype(np.float64).reshape(m, n).T).reshape(-1)
    yb = q.matmul(xs, rows, rehip.MODE_BF16)
    assert np.linalg.norm(yb - exact) / np.linalg.norm(exact) <= 1e-2
    xs2 = xs.copy()
    xs2[1:] = rng.standard_normal((rows - 1, n)).astype(np.float32)
    for mode in (rehip.MODE_F32, rehip.MODE_BF16):
        full = q.matmul(xs, rows, mode)
        other = q.matmul(xs2, rows, mode)
        assert np.array_equal(other[:m], full[:m]), mode
    q.close()


@pytest.mark.parametrize("t", DENSE)
def test_dense_device_entry_points(t):
    rng = np.random.default_rng(40 + t)
    m, n = 96, 200
    raw = _raw(t, rng.standard_normal((m, n)).astype(np.float32))
    q = rehip.QMat.from_bytes(t, raw, m, n)
    x = rng.standard_normal(n).astype(np.float32)
    add = rng.standard_normal(m).astype(np.float32)
    dx, dy, da = B.from_array(x), B(m * 4), B.from_array(add)
    q.matvec_dev(dx, dy)
    hip.synchronize()
    plain = dy.download()
    assert np.array_equal(plain, q.matvec(x))
    q.matvec_ex_dev(dx, dy, add=da)
    hip.synchronize()
    assert np.array_equal(dy.download(), plain + add)        # one f32 add after the product
    # the RMS-norm prologue: re_rmsnorm_dev's normed x, then the plain product (bit for bit)
    nw = B.from_array((1 + 0.1 * rng.standard_normal(n)).astype(np.float32))
    dn = B(n * 4)
    rehip.rmsnorm_dev(dx, nw, 1, n, 1e-6, dn)
    q.matvec_dev(dn, dy)
    hip.synchronize()
    normed = dy.download()
    q.matvec_ex_dev(dx, dy, norm_w=nw, eps=1e-6, add=da)
    hip.synchronize()
    assert np.array_equal(dy.download(), normed + add)
    out = B(m * n * 4)
    q.dequant_dev(out)
    hip.synchronize()
    assert np.array_equal(out.download().view(np.uint32), O.dequant(t, raw).view(np.uint32))
    rows = 9
    xs = rng.standard_normal((rows, n)).astype(np.float32)
    dxs, dys = B.from_array(xs), B(rows * m * 4)
    q.matmul_dev(dxs, rows, dys, rehip.MODE_F32)
    hip.synchronize()
    assert np.array_equal(dys.download(), q.matmul(xs, rows, rehip.MODE_F32))
    q.close()


def test_dense_errors():
    w = np.zeros(6, np.float32)
    with pytest.raises(rehip.RehipError, match="needs 24 bytes, got 20"):
        rehip.QMat.from_bytes(rehip.F32, w.view(np.uint8)[:20], 2, 3)
    with pytest.raises(rehip.RehipError, match="not stacked"):
        rehip.QMat.from_bytes_stacked(rehip.BF16, np.zeros(24, np.uint8), 2, 3, 2)
    q = rehip.QMat.from_f32(w, 2, 3)
    with pytest.raises(rehip.RehipError):
        q.matmul_i8(np.zeros(0, np.float32), np.zeros(0, np.int8), 0)  # needs Q8_0
    q8 = rehip.QMat.from_bytes(rehip.Q8_0, np.zeros(2 * 34, np.uint8), 2, 32)
    d32 = rehip.QMat.from_f32(np.zeros(64, np.float32), 2, 32)
    with pytest.raises(rehip.RehipError, match="both quantized or both dense"):
        rehip.Ffn(q8, d32)
    q8.close()
    d32.close()
    q.close()


def test_dense_tensor_from_gguf(tmp_path):
    rng = np.random.default_rng(9)
    m, n = 33, 64
    w16 = rng.standard_normal((m, n)).astype(np.float16)
    p = tmp_path / "d.gguf"
    p.write_bytes(W.write([], [("w", [n, m], rehip.F16, w16.tobytes())]))
    f = rehip.Gguf(p)
    q = rehip.QMat.from_gguf(f, "w", m, n)
    x = rng.standard_normal(n).astype(np.float32)
    raw = w16.view(np.uint8).reshape(-1)
    assert np.array_equal(q.matvec(x), rehip.QMat.from_bytes(rehip.F16, raw, m, n).matvec(x))
    _check_product(q.matvec(x), rehip.F16, raw, m, n, x, 1)
    q.close()
    f.close()
