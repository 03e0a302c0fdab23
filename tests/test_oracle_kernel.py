"""Pins the oracle's fused dots, GEMV and GEMM driver (src/kernel.rs + src/qmat.rs restatement).

- the reference's own tests (kernel.rs:2080-2721, qmat.rs:337-399), ported with their fixtures
  and tolerances;
- brute force: every oracle product against an f64 dot of the (exact) dequantized values,
  within the f32 rounding bound n * 2^-24 * sum|w*x|;
- closed forms: a single non-zero weight selects one activation exactly.
"""
import numpy as np
import pytest

import oracle as O
from blockpack import k_blocks, q4_blocks, q5_blocks, q8_blocks, q8_blocks_qmat, pack_q8_0


def f64_dot(w_f32, x):
    return float(np.dot(np.asarray(w_f32, np.float64), np.asarray(x, np.float64)))


def lin(n, a, b):
    return (np.arange(n, dtype=np.float32) * np.float32(a) - np.float32(b)).astype(np.float32)


# ---- kernel.rs:2080-2117, 2329-2367: fused dot / matvec vs dequant -> dot --------------
def test_dot_q5_0_fused_matches_reference():
    a = q5_blocks(4)
    b = lin(len(a) // 22 * 32, 0.07, 20.0)
    assert abs(O.dot(O.Q5_0, a, b) - f64_dot(O.dequant(O.Q5_0, a), b)) < 1e-2


def test_matvec_q5_0_matches_f32_matvec():
    m, n = 3, 64
    w = q5_blocks(m * n // 32)
    x = lin(n, 0.15, 3.0)
    fused = O.matvec(O.Q5_0, w, m, n, x)
    ref = O.dequant(O.Q5_0, w).reshape(m, n).astype(np.float64) @ x.astype(np.float64)
    assert np.all(np.abs(fused - ref) < 1e-2)


def test_dot_q4_0_fused_matches_reference():
    a = q4_blocks(4)
    b = lin(len(a) // 18 * 32, 0.1, 30.0)
    assert abs(O.dot(O.Q4_0, a, b) - f64_dot(O.dequant(O.Q4_0, a), b)) < 1e-3


def test_dot_q8_0_fused_matches_reference():
    a = q8_blocks(4)
    b = lin(len(a) // 34 * 32, 0.05, 10.0)
    assert abs(O.dot(O.Q8_0, a, b) - f64_dot(O.dequant(O.Q8_0, a), b)) < 1e-2


@pytest.mark.parametrize("t,n", [(O.Q4_0, 64), (O.Q8_0, 32)])
def test_matvec_32_blocks_match_f32_matvec(t, n):
    m = 3 if t == O.Q4_0 else 2
    w = (q4_blocks if t == O.Q4_0 else q8_blocks)(m * n // 32)
    x = lin(n, 0.2 if t == O.Q4_0 else 0.3, 5.0 if t == O.Q4_0 else 3.0)
    fused = O.matvec(t, w, m, n, x)
    ref = O.dequant(t, w).reshape(m, n).astype(np.float64) @ x.astype(np.float64)
    assert np.all(np.abs(fused - ref) < 1e-2)


@pytest.mark.parametrize("kind,t", [(0, O.Q4_K), (1, O.Q5_K), (2, O.Q6_K)])
def test_dot_k_quant_fused_matches_reference(kind, t):
    a = k_blocks(kind, 3)
    b = lin(3 * 256, 0.01, 1.3)
    ref = f64_dot(O.dequant(t, a), b)
    assert abs(O.dot(t, a, b) - ref) <= abs(ref) * 1e-4 + 1e-4


def test_matvec_k_quants_match_f32_matvec():
    m, n = 2, 512
    x = lin(n, 0.002, 1.0)
    for kind, t in [(0, O.Q4_K), (1, O.Q5_K), (2, O.Q6_K)]:
        w = k_blocks(kind, m * n // 256)
        fused = O.matvec(t, w, m, n, x)
        ref = O.dequant(t, w).reshape(m, n).astype(np.float64) @ x.astype(np.float64)
        assert np.all(np.abs(fused - ref) <= np.abs(ref) * 1e-4 + 1e-4), kind


# ---- kernel.rs:2533-2584 ------------------------------------------------------------------
def test_matmul_matches_rowwise_matvec():
    m, n, rows = 5, 64, 3
    x = (((np.arange(rows * n) * 7) % 13).astype(np.float32) * np.float32(0.1) - np.float32(0.6)).astype(np.float32)

    def close(a, b):
        return a.shape == b.shape and np.all(np.abs(a - b) <= 1e-2 * (1.0 + np.abs(a)))

    for t, w in [(O.Q4_0, q4_blocks(m * n // 32)), (O.Q5_0, q5_blocks(m * n // 32)),
                 (O.Q8_0, q8_blocks(m * n // 32))]:
        rowwise = np.concatenate([O.matvec(t, w, m, n, x[r * n:(r + 1) * n]) for r in range(rows)])
        assert close(O.matmul(t, w, m, n, x, rows), rowwise)
    km, kn = 3, 256
    kx = (((np.arange(rows * kn) * 5) % 11).astype(np.float32) * np.float32(0.1) - np.float32(0.5)).astype(np.float32)
    q6 = k_blocks(2, km * kn // 256)
    rowwise = np.concatenate([O.matvec(O.Q6_K, q6, km, kn, kx[r * kn:(r + 1) * kn]) for r in range(rows)])
    assert close(O.matmul(O.Q6_K, q6, km, kn, kx, rows), rowwise)


# ---- kernel.rs:2607-2701: driver knobs are bit-identical ---------------------------------
def xpat(rows, n, mul, mod, a, b):
    return (((np.arange(rows * n) * mul) % mod).astype(np.float32) * np.float32(a) - np.float32(b)).astype(np.float32)


def test_matmul_activation_tiling_is_bit_identical():
    m, n, rows = 7, 64, 70
    x = xpat(rows, n, 11, 17, 0.05, 0.4)
    w = q5_blocks(m * n // 32)
    untiled = O.matmul_reuse(O.Q5_0, w, m, n, x, rows, tile=rows)
    for tile in [1, 3, 31, 32, 64, 128]:
        assert np.array_equal(O.matmul_reuse(O.Q5_0, w, m, n, x, rows, tile=tile), untiled), tile


def test_matmul_k_quant_tiling_is_bit_identical():
    m, n, rows = 5, 512, 397
    x = xpat(rows, n, 11, 19, 0.05, 0.4)
    for kind, t in [(0, O.Q4_K), (1, O.Q5_K), (2, O.Q6_K)]:
        w = k_blocks(kind, m * n // 256)
        base = O.matmul_reuse(t, w, m, n, x, rows, tile=96)
        for tile in [96, 256, 512, 128]:
            assert np.array_equal(O.matmul_reuse(t, w, m, n, x, rows, tile=tile), base), (t, tile)


def test_matmul_row_grouping_is_bit_identical():
    m, n, rows = 5, 64, 70
    x = xpat(rows, n, 7, 23, 0.04, 0.5)
    w = q5_blocks(m * n // 32)
    single = O.matmul_reuse(O.Q5_0, w, m, n, x, rows, group=1, w_rows=1)
    for group in [2, 3, 4, 6, 8]:
        assert np.array_equal(O.matmul_reuse(O.Q5_0, w, m, n, x, rows, group=group), single), group


@pytest.mark.parametrize("m,w_rows", [(5, 2), (9, 4)])
def test_matmul_weight_rows_is_bit_identical(m, w_rows):
    n, rows = 64, 70
    x = xpat(rows, n, 5, 19, 0.03, 0.4)
    w = q5_blocks(m * n // 32)
    one = O.matmul_reuse(O.Q5_0, w, m, n, x, rows, w_rows=1)
    assert np.array_equal(O.matmul_reuse(O.Q5_0, w, m, n, x, rows, w_rows=w_rows), one)
    assert np.array_equal(O.matmul(O.Q5_0, w, m, n, x, rows), one)


def test_matmul_weight_row_blocking_is_bit_identical():
    m, n, rows = 70, 96, 13
    x = xpat(rows, n, 11, 17, 0.05, 0.4)
    w = q5_blocks(m * n // 32)
    assert np.array_equal(O.matmul_reuse(O.Q5_0, w, m, n, x, rows),
                          O.matmul_reuse(O.Q5_0, w, m, n, x, rows, r_block=1))


def test_matmul_row_wise_accumulator_matches_block_wise():
    m, n, rows = 9, 896, 37
    x = xpat(rows, n, 13, 29, 0.03, 0.45)
    w = q5_blocks(m * n // 32)
    row = O.matmul_reuse(O.Q5_0, w, m, n, x, rows)
    block = O.matmul_blocks(O.Q5_0, w, m, n, x, rows)
    assert np.all(np.abs(row - block) <= 1e-4 * (1.0 + np.abs(block)))


# ---- brute force against f64 on seeded random blocks --------------------------------------
def random_rows(rng, t, m, n):
    qk, bb = O.GEOM[t]
    nb = (n + qk - 1) // qk
    raw = rng.integers(0, 256, (m * nb, bb), dtype=np.uint8)
    d = (np.abs(rng.standard_normal(m * nb)) * 0.01).astype(np.float16).view(np.uint8).reshape(-1, 2)
    if t == O.Q6_K:
        raw[:, 208:210] = d
    else:
        raw[:, 0:2] = d
        if t in (O.Q4_K, O.Q5_K):
            raw[:, 2:4] = d[::-1]
    return raw.reshape(-1)


@pytest.mark.parametrize("t", O.QUANT_TYPES)
@pytest.mark.parametrize("n", [256, 512, 896])
def test_qmat_products_within_f32_bound_of_f64(t, n):
    rng = np.random.default_rng(7 + t + n)
    m, rows = 19, 5
    w = random_rows(rng, t, m, n)
    x = rng.standard_normal(rows * n).astype(np.float32)
    qk, _ = O.GEOM[t]
    nb = (n + qk - 1) // qk
    deq = O.dequant(t, w).reshape(m, nb * qk)[:, :n].astype(np.float64)
    exact = x.reshape(rows, n).astype(np.float64) @ deq.T
    absd = np.abs(x.reshape(rows, n).astype(np.float64)) @ np.abs(deq).T
    assert np.allclose(O.qmat_absdot(t, w, m, n, x, rows).reshape(rows, m), absd, rtol=1e-12)
    bound = n * 2.0 ** -24 * absd + 1e-30
    mm = O.qmat_matmul(t, w, m, n, x, rows).reshape(rows, m)
    assert np.all(np.abs(mm - exact) <= bound)
    for r in range(rows):
        mv = O.qmat_matvec(t, w, m, n, x[r * n:(r + 1) * n])
        assert np.all(np.abs(mv - exact[r]) <= bound[r])


def test_single_weight_selects_one_activation_exactly():
    # Q8_0 row with one non-zero quant 3 at column 37 and d = 1: out = 3 * x[37] exactly
    n = 64
    q = np.zeros(n, np.int64)
    q[37] = 3
    w = pack_q8_0(0x3C00, q[:32]) + pack_q8_0(0x3C00, q[32:])
    x = np.random.default_rng(3).standard_normal(n).astype(np.float32)
    want = np.float32(3.0) * x[37]
    assert O.matvec(O.Q8_0, w, 1, n, x)[0] == want
    assert O.matmul(O.Q8_0, w, 1, n, x, 1)[0] == want


def test_dot_f32_order_and_tail():
    # 8-lane FMA accumulators + hsum; tails (n % 8) are plain mul+add
    rng = np.random.default_rng(11)
    for n in [1, 7, 8, 9, 64, 67, 896]:
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        exact = f64_dot(a, b)
        bound = n * 2.0 ** -24 * float(np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64)))
        assert abs(O.dot_f32(a, b) - exact) <= bound
    # integer-valued inputs are exact in every order
    a = np.arange(1, 20, dtype=np.float32)
    assert O.dot_f32(a, a) == float(np.sum(a.astype(np.int64) ** 2))


def test_unknown_type_is_an_error():
    with pytest.raises(O.OracleError):
        O.matvec(99, bytes(34), 1, 32, np.zeros(32, np.float32))
    with pytest.raises(O.OracleError):
        O.qmat_matvec(O.Q8_0, bytes(33), 1, 32, np.zeros(32, np.float32))


# ---- qmat.rs:383-399 + baseline == oracle ---------------------------------------------------
def test_pooled_matmul_is_bit_identical_to_serial():
    m, n, rows = 64, 4096, 8
    w = q8_blocks_qmat(m, n)
    x = (np.arange(rows * n, dtype=np.float32) * np.float32(0.0007) - np.float32(1.5)).astype(np.float32)
    serial = O.matmul(O.Q8_0, w, m, n, x, rows)
    if O.cpu_has_avx2():
        for th in (1, 3, 8):
            assert np.array_equal(O.cpu_matmul(O.Q8_0, w, m, n, x, rows, threads=th), serial)


@pytest.mark.parametrize("t", O.QUANT_TYPES)
def test_cpu_baseline_matches_oracle(t):
    if not O.cpu_has_avx2():
        pytest.skip("host has no AVX2+FMA")
    rng = np.random.default_rng(40 + t)
    m, n, rows = 70, 512, 11
    w = random_rows(rng, t, m, n)
    x = rng.standard_normal(rows * n).astype(np.float32)
    # the pooled GEMM keeps matmul_reuse's per-output order: bit-identical on both split axes
    assert np.array_equal(O.cpu_matmul(t, w, m, n, x, rows, threads=4), O.matmul(t, w, m, n, x, rows))
    big_rows = 6 * 1024 * 1024 // (4 * n) + 1      # crosses the 6 MiB X budget -> weight-row split
    xb = rng.standard_normal(big_rows * n).astype(np.float32)
    assert np.array_equal(O.cpu_matmul(t, w[:O.qmat_row_bytes(t, n) * 8], 8, n, xb, big_rows, threads=4),
                          O.matmul(t, w[:O.qmat_row_bytes(t, n) * 8], 8, n, xb, big_rows))
    mv = O.cpu_matvec(t, w, m, n, x[:n], threads=4)
    absd = O.qmat_absdot(t, w, m, n, x[:n], 1)
    assert np.all(np.abs(mv - O.matvec(t, w, m, n, x[:n])) <= 2 * n * 2.0 ** -24 * absd)


@pytest.mark.parametrize("t", O.QUANT_TYPES)
def test_cpu_baseline_gemv_row_split_is_deterministic(t):
    # qmat.rs:80-127: above 2^18 MACs the rows are split in ceil(m / threads) chunks; each row is
    # one quant_row_dot, so the result does not depend on the thread count
    if not O.cpu_has_avx2():
        pytest.skip("host has no AVX2+FMA")
    rng = np.random.default_rng(90 + t)
    m, n = 97, 4096
    assert m * n >= 1 << 18
    w = random_rows(rng, t, m, n)
    x = rng.standard_normal(n).astype(np.float32)
    one = O.cpu_matvec(t, w, m, n, x, threads=1)
    for th in (2, 3, 8):
        assert np.array_equal(O.cpu_matvec(t, w, m, n, x, threads=th), one)
    absd = O.qmat_absdot(t, w, m, n, x, 1)
    assert np.all(np.abs(one - O.matvec(t, w, m, n, x)) <= 2 * n * 2.0 ** -24 * absd)


@pytest.mark.parametrize("t", [O.Q4_K, O.Q5_K, O.Q6_K])
def test_cpu_baseline_padded_k_quant_rows(t):
    # K = 896 is not a multiple of 256: rows are stored as 4 whole super-blocks and only the
    # first 896 elements enter the dot (the padded-row rule of the QMat oracle)
    if not O.cpu_has_avx2():
        pytest.skip("host has no AVX2+FMA")
    rng = np.random.default_rng(70 + t)
    m, n, rows = 40, 896, 6
    w = random_rows(rng, t, m, n)
    assert w.size == m * O.qmat_row_bytes(t, n)
    x = rng.standard_normal(rows * n).astype(np.float32)
    got = O.cpu_matmul(t, w, m, n, x, rows, threads=3)
    absd = O.qmat_absdot(t, w, m, n, x, rows)
    assert np.all(np.abs(got - O.qmat_matmul(t, w, m, n, x, rows)) <= 2 * n * 2.0 ** -24 * absd)
    mv = O.cpu_matvec(t, w, m, n, x[:n], threads=3)
    assert np.all(np.abs(mv - O.qmat_matvec(t, w, m, n, x[:n])) <= 2 * n * 2.0 ** -24 * absd[:m])
