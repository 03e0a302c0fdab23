"""GPU parity of librehip against the CPU oracle, through the C ABI.

Bars (from the task's parity contract):
  - dequant: bit-exact with quant::dequant (src/quant.rs:363-453);
  - GEMV and f32-mode GEMM: |y - y_oracle| <= 2^-10 * sum_k |w_rk x_k| per output;
  - bf16-mode GEMM and MoE: ||y - y_oracle|| / ||y_oracle|| <= 1e-2.
Full-size shapes compare against an f64 product of the oracle-dequantized weights (the
dequantized values are exact, so this is the exact product up to f64 rounding).
"""
import numpy as np
import pytest

import oracle as O
import rehip
from blockpack import k_blocks, q4_blocks, q5_blocks, q8_blocks
from rehip import hip, synth

pytestmark = pytest.mark.gpu

F32_TOL = 2.0 ** -10
BF16_TOL = 1e-2


def qmat(t, w, m, n):
    return rehip.QMat.from_bytes(t, w, m, n)


def f64_product(t, w, m, n, x, rows):
    qk, _ = rehip.GEOM[t]
    nb = (n + qk - 1) // qk
    deq = O.dequant(t, w).reshape(m, nb * qk)[:, :n].astype(np.float64)
    xx = x.reshape(rows, n).astype(np.float64)
    return xx @ deq.T, np.abs(xx) @ np.abs(deq).T


# ---- dequant: bit-exact ---------------------------------------------------------------------
def random_blocks_all_scales(rng, t, nb):
    """Random block bytes whose f16 scales span normal, subnormal, zero and negative values."""
    qk, bb = rehip.GEOM[t]
    raw = rng.integers(0, 256, (nb, bb), dtype=np.uint8)
    h = rng.integers(0, 0x7C00, nb).astype(np.uint16)              # finite, any sign below
    h[::7] = rng.integers(0, 0x400, len(h[::7]))                      # subnormals
    h[::11] = 0
    h[1::3] |= 0x8000                                                 # negative scales
    hb = h.view(np.uint8).reshape(nb, 2)
    if t == rehip.Q6_K:
        raw[:, 208:210] = hb
    else:
        raw[:, 0:2] = hb
        if t in (rehip.Q4_K, rehip.Q5_K):
            raw[:, 2:4] = hb[::-1]
    return raw.reshape(-1)


@pytest.mark.parametrize("t", rehip.QUANT_TYPES)
def test_dequant_bit_exact_random_blocks(t):
    rng = np.random.default_rng(100 + t)
    data = random_blocks_all_scales(rng, t, 1000)
    want = O.dequant(t, data)
    got = rehip.dequant(t, data)
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t,data", [(rehip.Q4_0, q4_blocks(67)), (rehip.Q5_0, q5_blocks(67)),
                                    (rehip.Q8_0, q8_blocks(67)), (rehip.Q4_K, k_blocks(0, 9)),
                                    (rehip.Q5_K, k_blocks(1, 9)), (rehip.Q6_K, k_blocks(2, 9))],
                         ids=["q4_blocks", "q5_blocks", "q8_blocks", "k_blocks0", "k_blocks1", "k_blocks2"])
def test_dequant_bit_exact_reference_fixtures(t, data):
    assert np.array_equal(rehip.dequant(t, data).view(np.uint32), O.dequant(t, data).view(np.uint32))


def test_dequant_errors_mirror_reference():
    with pytest.raises(rehip.RehipError) as e:
        rehip.dequant(rehip.Q4_K, bytes(143))
    assert e.value.message == "Q4_K data len 143 not a multiple of 144"
    assert rehip.dequant(rehip.Q6_K, b"").size == 0


@pytest.mark.parametrize("t", rehip.QUANT_TYPES)
def test_resident_dequant_matches_flat_dequant(t):
    rng = np.random.default_rng(7 + t)
    m, n = 130, 896
    w = synth.weight_bytes(rng, t, m, n)
    q = qmat(t, w, m, n)
    out = hip.DeviceBuffer(m * n * 4)
    q.dequant_dev(out)
    hip.synchronize()
    qk, _ = rehip.GEOM[t]
    nb = (n + qk - 1) // qk
    want = O.dequant(t, w).reshape(m, nb * qk)[:, :n].reshape(-1)
    assert np.array_equal(out.download().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("io", ["0", "1", "2"])
def test_device_entry_points_match_host_entry_points(io, monkeypatch):
    """Host-pointer calls (re_qmat_matvec / re_qmat_matmul) give the device calls' bits whatever
    the transfer: pageable copies (REHIP_HOST_IO=0), pinned copies (1), or pinned x with y written
    by the kernels straight into pinned host memory (2, the default), including a split GEMV and
    a split-K GEMM whose reduce writes y."""
    monkeypatch.setenv("REHIP_HOST_IO", io)
    rng = np.random.default_rng(17)
    t, m, n, rows = rehip.Q4_K, 256, 1024, 33
    w = synth.weight_bytes(rng, t, m, n)
    x = synth.activations(rng, rows, n)
    q = qmat(t, w, m, n)
    dx = hip.DeviceBuffer.from_array(x)
    dy = hip.DeviceBuffer(rows * m * 4)
    s = hip.Stream()
    q.matmul_dev(dx, rows, dy, rehip.MODE_BF16, stream=s)
    s.synchronize()
    assert np.array_equal(dy.download(), q.matmul(x, rows, rehip.MODE_BF16))
    q.matvec_dev(dx, dy, stream=s)
    s.synchronize()
    assert np.array_equal(dy.download(count=m), q.matvec(x[:n]))
    q.close()
    for t, m, n, rows in [(rehip.Q6_K, 96, 14336, 1), (rehip.Q6_K, 896, 4864, 64), (rehip.Q5_0, 4864, 896, 1)]:
        w = synth.weight_bytes(rng, t, m, n)
        x = synth.activations(rng, rows, n)
        q = qmat(t, w, m, n)
        dx = hip.DeviceBuffer.from_array(x)
        dy = hip.DeviceBuffer(rows * m * 4)
        q.matmul_dev(dx, rows, dy, rehip.MODE_F32, stream=s)
        s.synchronize()
        assert np.array_equal(dy.download(), q.matmul(x, rows, rehip.MODE_F32)), (t, m, n, rows)
        if rows == 1:
            assert np.array_equal(dy.download(), q.matvec(x)), (t, m, n)
        q.close()
    s.destroy()


# ---- GEMV --------------------------------------------------------------------------------
GEMV_SHAPES = [(1, 256), (5, 512), (64, 256), (70, 896), (130, 1024), (896, 4864), (4864, 896),
               (96, 14336)]     # the last row is longer than one workgroup stages: split launch


@pytest.mark.parametrize("t", rehip.QUANT_TYPES)
@pytest.mark.parametrize("m,n", GEMV_SHAPES)
def test_gemv_parity(t, m, n):
    rng = np.random.default_rng(1000 * t + m + n)
    w = synth.weight_bytes(rng, t, m, n)
    x = synth.activations(rng, 1, n)
    got = qmat(t, w, m, n).matvec(x)
    want = O.qmat_matvec(t, w, m, n, x)
    absd = O.qmat_absdot(t, w, m, n, x, 1)
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= F32_TOL * absd), f"max err/bound {np.max(err / (absd + 1e-30))}"


@pytest.mark.parametrize("t", [rehip.Q5_0, rehip.Q8_0, rehip.Q4_K, rehip.Q6_K])
@pytest.mark.parametrize("rows_per_group", [64, 16, 8, 4])
@pytest.mark.parametrize("waves", [4, 8, 16])
def test_gemv_launch_shapes(t, rows_per_group, waves, monkeypatch):
    # every row-group / wave-count kernel variant on a ragged shape (3 tiles, last one partial)
    monkeypatch.setenv("REHIP_GEMV_ROWS", str(rows_per_group))
    monkeypatch.setenv("REHIP_GEMV_WAVES", str(waves))
    m, n = 150, 2560
    rng = np.random.default_rng(5000 + 10 * t + rows_per_group + waves)
    w = synth.weight_bytes(rng, t, m, n)
    x = synth.activations(rng, 1, n)
    q = qmat(t, w, m, n)
    got = q.matvec(x)
    want = O.qmat_matvec(t, w, m, n, x)
    absd = O.qmat_absdot(t, w, m, n, x, 1)
    assert np.all(np.abs(got.astype(np.float64) - want) <= F32_TOL * absd)
    assert np.array_equal(q.matvec(x), got)
    q.close()


def sparse_unit_rows(rng, t, m, n):
    """m rows of n elements of type t whose values are 0 except three +-1 quant steps per row:
    every other quant sits at the type's zero point (q = bias, or q = 0 with min 0). With such
    rows sum|w x| is a few |x| while sum(x) over each 16-element run is large, so a dot that
    carried the zero point through the products would cancel away the answer."""
    from blockpack import pack_q4_0, pack_q4_k, pack_q5_0, pack_q5_k, pack_q6_k, pack_q8_0
    qk, _ = rehip.GEOM[t]
    out = []
    for r in range(m):
        zero = {rehip.Q4_0: 8, rehip.Q5_0: 16, rehip.Q8_0: 0, rehip.Q6_K: 32}.get(t, 0)
        q = np.full(n, zero, np.int64)
        for j in rng.choice(n, 3, replace=False):
            q[j] = zero + (1 if t in (rehip.Q4_K, rehip.Q5_K) else int(rng.choice([-1, 1])))
        for b in range(n // qk):
            qb = q[b * qk:(b + 1) * qk]
            d16 = int(rng.integers(0x3400, 0x3C00))           # 0.25 .. 1
            if t == rehip.Q4_0:
                out.append(pack_q4_0(d16, qb))
            elif t == rehip.Q5_0:
                out.append(pack_q5_0(d16, qb))
            elif t == rehip.Q8_0:
                out.append(pack_q8_0(d16, qb))
            elif t == rehip.Q6_K:
                out.append(pack_q6_k(d16, rng.integers(1, 127, 16), qb))
            else:
                pk = pack_q4_k if t == rehip.Q4_K else pack_q5_k
                out.append(pk(d16, 0x3C00, rng.integers(1, 63, 8), np.zeros(8, np.int64), qb))
    return np.frombuffer(b"".join(out), np.uint8)


@pytest.mark.parametrize("t", rehip.QUANT_TYPES)
@pytest.mark.parametrize("rows_per_group", [0, 64, 4])
def test_gemv_sparse_unit_quants_within_bound(t, rows_per_group, monkeypatch):
    """The f32 bound |y - y_oracle| <= 2^-10 sum|w x| where sum|w x| is small against sum|x|:
    rows of zero-point quants with three unit steps, x = 4 + N(0, 1), K = 4096 (the planned
    kernel, the tile kernel and 4-row groups)."""
    if rows_per_group:
        monkeypatch.setenv("REHIP_GEMV_ROWS", str(rows_per_group))
    rng = np.random.default_rng(7100 + t + rows_per_group)
    m, n = 96, 4096
    w = sparse_unit_rows(rng, t, m, n)
    x = (4.0 + rng.standard_normal(n)).astype(np.float32)
    q = qmat(t, w, m, n)
    got = q.matvec(x)
    want = O.qmat_matvec(t, w, m, n, x)
    absd = O.qmat_absdot(t, w, m, n, x, 1)
    assert np.all(np.abs(got.astype(np.float64) - want) <= F32_TOL * absd)
    q.close()


def test_moe_identity_experts_exact_silu():
    """Q8_0 identity experts (d = 1, quant 1 on the diagonal, moe.rs:768-776 at hidden = inter =
    32): one token through gate, up, SwiGLU and down gives silu(1) to f32 accuracy."""
    from blockpack import pack_q8_0
    rows = []
    for r in range(32):
        qv = np.zeros(32, np.int64)
        qv[r] = 1
        rows.append(pack_q8_0(0x3C00, qv))
    ident = np.frombuffer(b"".join(rows), np.uint8)
    moe = rehip.MoeExperts(rehip.Q8_0, ident, rehip.Q8_0, ident, rehip.Q8_0, ident, 1, 32, 32)
    x = np.zeros(32, np.float32)
    x[0] = 1.0
    for mode in (rehip.MODE_F32, rehip.MODE_BF16):
        out = moe.forward(x, 1, 1, np.zeros(1, np.uint32), np.ones(1, np.float32), mode)
        assert abs(float(out[0]) - O.silu(1.0)) <= 2e-7 and np.all(out[1:] == 0), (mode, out[0])
    moe.close()


def test_gemv_reference_fixtures_match_scalar_kernels():
    # kernel.rs fixtures; the oracle's matvec is the reference's scalar GEMV
    for t, w, m, n in [(rehip.Q4_0, q4_blocks(3 * 64 // 32), 3, 64), (rehip.Q5_0, q5_blocks(3 * 64 // 32), 3, 64),
                       (rehip.Q8_0, q8_blocks(2), 2, 32), (rehip.Q4_K, k_blocks(0, 4), 2, 512),
                       (rehip.Q5_K, k_blocks(1, 4), 2, 512), (rehip.Q6_K, k_blocks(2, 4), 2, 512)]:
        x = (np.arange(n, dtype=np.float32) * np.float32(0.01) - np.float32(1.3)).astype(np.float32)
        got = qmat(t, w, m, n).matvec(x)
        want = O.matvec(t, w, m, n, x)
        assert np.all(np.abs(got - want) <= np.abs(want) * 1e-4 + 1e-4), t


def test_gemv_is_deterministic_and_equals_rows1_matmul():
    rng = np.random.default_rng(3)
    t, m, n = rehip.Q6_K, 896, 4864
    w = synth.weight_bytes(rng, t, m, n)
    x = synth.activations(rng, 1, n)
    q = qmat(t, w, m, n)
    a, b = q.matvec(x), q.matvec(x)
    assert np.array_equal(a, b)
    assert np.array_equal(q.matmul(x, 1, rehip.MODE_BF16), a)


@pytest.mark.parametrize("t,m,n,count", [(rehip.Q6_K, 896, 4864, 5), (rehip.Q4_K, 130, 896, 3),
                                         (rehip.Q8_0, 64, 14336, 2), (rehip.Q5_0, 4864, 896, 2)])
def test_stacked_gemv_equals_single_launches(t, m, n, count):
    """One launch over a stack of matrices against the oracle (f32 bound) and one launch per
    matrix (equal up to summation order: the stack's launch shape is planned for all of it),
    also with a shared x, a sub-range of the stack and, for K > 12288, the per-matrix split
    fallback."""
    rng = np.random.default_rng(m + n + count)
    ws = [synth.weight_bytes(rng, t, m, n) for _ in range(count)]
    st = rehip.QMat.from_bytes_stacked(t, np.concatenate(ws), m, n, count)
    assert st.count() == count
    singles = [qmat(t, w, m, n) for w in ws]
    xs = rng.standard_normal((count, n)).astype(np.float32)
    dx = hip.DeviceBuffer.from_array(xs)
    dy = hip.DeviceBuffer(count * (m + 3) * 4)
    st.matvec_stacked_dev(0, count, dx, n, dy, m + 3)
    hip.synchronize()
    got = dy.download(np.float32, count * (m + 3)).reshape(count, m + 3)[:, :m]
    for b in range(count):
        one = singles[b].matvec(xs[b])
        np.testing.assert_allclose(got[b], one, rtol=0, atol=1e-5 * np.abs(one).max())
        err = np.abs(got[b].astype(np.float64) - O.qmat_matvec(t, ws[b], m, n, xs[b]))
        assert np.all(err <= F32_TOL * O.qmat_absdot(t, ws[b], m, n, xs[b], 1)), b
    # shared x, matrices 1..count-1
    st.matvec_stacked_dev(1, count - 1, dx, 0, dy, m)
    hip.synchronize()
    got = dy.download(np.float32, (count - 1) * m).reshape(count - 1, m)
    for b in range(1, count):
        one = singles[b].matvec(xs[0])
        np.testing.assert_allclose(got[b - 1], one, rtol=0, atol=1e-5 * np.abs(one).max())
    with pytest.raises(rehip.RehipError):
        st.matvec_stacked_dev(1, count, dx, n, dy, m)
    st.close()
    for q in singles:
        q.close()


def test_lm_head_gemv_q8_0_full_size():
    rng = np.random.default_rng(305)
    t, m, n = rehip.Q8_0, 151936, 896
    w = synth.weight_bytes(rng, t, m, n)
    x = synth.activations(rng, 1, n)
    got = qmat(t, w, m, n).matvec(x)
    exact, absd = f64_product(t, w, m, n, x, 1)
    assert np.all(np.abs(got - exact[0]) <= F32_TOL * absd[0])


# ---- GEMM --------------------------------------------------------------------------------
GEMM_SHAPES = [(5, 256, 2), (70, 512, 3), (128, 896, 64), (200, 1024, 70), (896, 4864, 129), (300, 1024, 500)]


@pytest.mark.parametrize("t", rehip.QUANT_TYPES)
@pytest.mark.parametrize("m,n,rows", GEMM_SHAPES)
def test_gemm_parity_both_modes(t, m, n, rows):
    rng = np.random.default_rng(2000 * t + m + n + rows)
    w = synth.weight_bytes(rng, t, m, n)
    x = synth.activations(rng, rows, n)
    q = qmat(t, w, m, n)
    exact, absd = f64_product(t, w, m, n, x, rows)
    exact, absd = exact.reshape(-1), absd.reshape(-1)
    got32 = q.matmul(x, rows, rehip.MODE_F32)
    assert np.all(np.abs(got32 - exact) <= F32_TOL * absd)
    got16 = q.matmul(x, rows, rehip.MODE_BF16)
    assert np.linalg.norm(got16 - exact) / np.linalg.norm(exact) <= BF16_TOL
    if m * n * rows <= 1 << 22:
        want = O.qmat_matmul(t, w, m, n, x, rows)
        assert np.all(np.abs(got32 - want) <= F32_TOL * absd)


@pytest.mark.parametrize("t", rehip.QUANT_TYPES)
@pytest.mark.parametrize("tile,kg,splits", [(1, 1, 1), (1, 2, 1), (2, 1, 1), (3, 1, 1), (4, 1, 1), (3, 1, 2),
                                            (4, 1, 3), (1, 2, 3), (5, 1, 1), (5, 1, 3)])
def test_gemm_forced_tiles(t, tile, kg, splits, monkeypatch):
    # every tile / K-group / K-split instance in bf16 mode on a ragged shape: 300 weight rows (a
    # partial 128- and 256-row tile), 500 activation rows, K = 1280 (5 super-blocks)
    monkeypatch.setenv("REHIP_GEMM_TILE", str(tile))
    monkeypatch.setenv("REHIP_GEMM_KG", str(kg))
    monkeypatch.setenv("REHIP_GEMM_SPLITS", str(splits))
    m, n, rows = 300, 1280, 500
    rng = np.random.default_rng(7000 + 10 * t + tile)
    w = synth.weight_bytes(rng, t, m, n)
    x = synth.activations(rng, rows, n)
    q = qmat(t, w, m, n)
    exact, _ = f64_product(t, w, m, n, x, rows)
    exact = exact.reshape(-1)
    got = q.matmul(x, rows, rehip.MODE_BF16)
    assert np.linalg.norm(got - exact) / np.linalg.norm(exact) <= BF16_TOL
    assert np.array_equal(q.matmul(x, rows, rehip.MODE_BF16), got)
    q.close()


@pytest.mark.parametrize("t", rehip.QUANT_TYPES)
@pytest.mark.parametrize("tile,splits", [(1, 1), (2, 1), (1, 3), (2, 4)])
def test_gemm_f32_split_operand_tiles(t, tile, splits, monkeypatch):
    # f32 mode on bf16 MFMAs (split operands) at both tiles, whole K and K split over workgroups,
    # on a ragged shape (300 weight rows, 500 activation rows, K = 1280): the f32 bar, and the same
    # bits on a repeat
    monkeypatch.setenv("REHIP_GEMM_TILE", str(tile))
    monkeypatch.setenv("REHIP_GEMM_KG", "1")
    monkeypatch.setenv("REHIP_GEMM_SPLITS", str(splits))
    m, n, rows = 300, 1280, 500
    rng = np.random.default_rng(9100 + 10 * t + tile)
    w = synth.weight_bytes(rng, t, m, n)
    x = synth.activations(rng, rows, n)
    q = qmat(t, w, m, n)
    exact, absd = f64_product(t, w, m, n, x, rows)
    got = q.matmul(x, rows, rehip.MODE_F32)
    assert np.all(np.abs(got - exact.reshape(-1)) <= F32_TOL * absd.reshape(-1))
    assert np.array_equal(q.matmul(x, rows, rehip.MODE_F32), got)
    q.close()


@pytest.mark.parametrize("t", [rehip.Q4_0, rehip.Q8_0, rehip.Q4_K, rehip.Q6_K])
def test_gemm_large_tiles_ragged_edges(t):
    # 3136 weight rows (not a multiple of 128) x 2085 activation rows (not a multiple of 256):
    # enough tiles for the 128 x 256 bf16 tile and the 128 x 128 f32 tile, with partial edge tiles
    m, n, rows = 3136, 512, 2085
    rng = np.random.default_rng(77 + t)
    w = synth.weight_bytes(rng, t, m, n)
    x = synth.activations(rng, rows, n)
    q = qmat(t, w, m, n)
    exact, absd = f64_product(t, w, m, n, x, rows)
    exact, absd = exact.reshape(-1), absd.reshape(-1)
    got16 = q.matmul(x, rows, rehip.MODE_BF16)
    assert np.linalg.norm(got16 - exact) / np.linalg.norm(exact) <= BF16_TOL
    got32 = q.matmul(x, rows, rehip.MODE_F32)
    assert np.all(np.abs(got32 - exact) <= F32_TOL * absd)


@pytest.mark.parametrize("name,t,m,n,rows", [("C1 Q5_0 4864x896 N=961", rehip.Q5_0, 4864, 896, 961),
                                             ("C2 Q6_K 896x4864 N=961", rehip.Q6_K, 896, 4864, 961),
                                             ("C2 Q6_K 896x4864 N=64", rehip.Q6_K, 896, 4864, 64),
                                             ("C1 Q5_0 4864x896 N=64", rehip.Q5_0, 4864, 896, 64)])
def test_prefill_rows_full_size(name, t, m, n, rows):
    rng = np.random.default_rng((101 if t == rehip.Q5_0 else 201) + rows)
    w = synth.weight_bytes(rng, t, m, n)
    x = synth.activations(rng, rows, n)
    q = qmat(t, w, m, n)
    exact, absd = f64_product(t, w, m, n, x, rows)
    exact, absd = exact.reshape(-1), absd.reshape(-1)
    got16 = q.matmul(x, rows, rehip.MODE_BF16)
    assert np.linalg.norm(got16 - exact) / np.linalg.norm(exact) <= BF16_TOL
    got32 = q.matmul(x, rows, rehip.MODE_F32)
    assert np.all(np.abs(got32 - exact) <= F32_TOL * absd)
    assert np.array_equal(q.matmul(x, rows, rehip.MODE_BF16), got16)      # deterministic
    assert np.array_equal(q.matmul(x, rows, rehip.MODE_F32), got32)


# ---- MoE ---------------------------------------------------------------------------------
def moe_case(seed, E, hidden, inter, T, k, gt=rehip.Q4_K, dt=rehip.Q6_K):
    rng = np.random.default_rng(seed)
    gate = np.concatenate([synth.weight_bytes(rng, gt, inter, hidden) for _ in range(E)])
    up = np.concatenate([synth.weight_bytes(rng, gt, inter, hidden) for _ in range(E)])
    down = np.concatenate([synth.weight_bytes(rng, dt, hidden, inter) for _ in range(E)])
    x = synth.activations(rng, T, hidden)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    ids = np.zeros((T, k), np.uint32)
    wts = np.zeros((T, k), np.float32)
    for i in range(T):
        ids[i], wts[i] = O.top_k(logits[i], k)        # the reference router (moe.rs:75-93)
    return gate, up, down, x, ids.reshape(-1), wts.reshape(-1)


@pytest.mark.parametrize("T", [1, 5, 40])
def test_moe_grouped_ffn_parity(T):
    E, hidden, inter, k = 16, 512, 256, 4
    gate, up, down, x, ids, wts = moe_case(400 + T, E, hidden, inter, T, k)
    want = O.moe_ffn(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, down, E, hidden, inter, x, T, k, ids, wts)
    moe = rehip.MoeExperts(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, down, E, hidden, inter)
    for mode, tol in [(rehip.MODE_F32, 1e-4), (rehip.MODE_BF16, BF16_TOL)]:
        got = moe.forward(x, T, k, ids, wts, mode)
        rel = np.linalg.norm(got - want) / np.linalg.norm(want)
        assert rel <= tol, (mode, rel)


@pytest.mark.parametrize("T", [1, 3, 60])
def test_moe_mixed_types_and_padded_rows(T):
    # gate/up of different types (separate gate and up launches + SwiGLU), K-quant rows padded to
    # whole super-blocks (hidden 640, inter 384), decode-sized and batch-sized routing
    E, hidden, inter, k = 8, 640, 384, 2
    rng = np.random.default_rng(900 + T)
    gate = np.concatenate([synth.weight_bytes(rng, rehip.Q4_0, inter, hidden) for _ in range(E)])
    up = np.concatenate([synth.weight_bytes(rng, rehip.Q5_K, inter, hidden) for _ in range(E)])
    down = np.concatenate([synth.weight_bytes(rng, rehip.Q6_K, hidden, inter) for _ in range(E)])
    x = synth.activations(rng, T, hidden)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    ids = np.zeros((T, k), np.uint32)
    wts = np.zeros((T, k), np.float32)
    for i in range(T):
        ids[i], wts[i] = O.top_k(logits[i], k)
    ids, wts = ids.reshape(-1), wts.reshape(-1)
    want = O.moe_ffn(rehip.Q4_0, gate, rehip.Q5_K, up, rehip.Q6_K, down, E, hidden, inter, x, T, k, ids, wts)
    moe = rehip.MoeExperts(rehip.Q4_0, gate, rehip.Q5_K, up, rehip.Q6_K, down, E, hidden, inter)
    for mode, tol in [(rehip.MODE_F32, 1e-4), (rehip.MODE_BF16, BF16_TOL)]:
        got = moe.forward(x, T, k, ids, wts, mode)
        assert np.linalg.norm(got - want) / np.linalg.norm(want) <= tol, mode
        assert np.array_equal(moe.forward(x, T, k, ids, wts, mode), got)


def test_moe_qwen3_shape_t32():
    E, hidden, inter, k, T = 128, 2048, 768, 8, 32
    gate, up, down, x, ids, wts = moe_case(401, E, hidden, inter, T, k)
    want = O.moe_ffn(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, down, E, hidden, inter, x, T, k, ids, wts)
    moe = rehip.MoeExperts(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, down, E, hidden, inter)
    got = moe.forward(x, T, k, ids, wts, rehip.MODE_BF16)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) <= BF16_TOL
    got32 = moe.forward(x, T, k, ids, wts, rehip.MODE_F32)
    assert np.linalg.norm(got32 - want) / np.linalg.norm(want) <= 1e-4


@pytest.mark.parametrize("ids", [[3, 3], [3, 3, 5, 3], [1, 1, 1, 1], [6, 2, 0, 4]])
def test_moe_one_token_repeated_expert(ids):
    """One token whose routing names an expert more than once (rehip.h allows it): the expert
    gets several gathered rows, so the single-row gate/up tasks do not apply. Host-routed and
    device-routed calls against the oracle FFN."""
    E, hidden, inter, k = 8, 512, 256, len(ids)
    gate, up, down, x, _, _ = moe_case(950 + 10 * k + ids[0], E, hidden, inter, 1, k)
    idv = np.array(ids, np.uint32)
    wts = np.linspace(0.1, 0.4, k).astype(np.float32)
    want = O.moe_ffn(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, down, E, hidden, inter, x, 1, k, idv, wts)
    moe = rehip.MoeExperts(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, down, E, hidden, inter)
    dx, did, dw = (hip.DeviceBuffer.from_array(a) for a in (x, idv.astype(np.int32), wts))
    out = hip.DeviceBuffer(hidden * 4)
    for mode, tol in [(rehip.MODE_F32, 1e-4), (rehip.MODE_BF16, BF16_TOL)]:
        got = moe.forward(x, 1, k, idv, wts, mode)
        assert np.linalg.norm(got - want) / np.linalg.norm(want) <= tol, ("host", mode)
        moe.forward_routed_dev(dx, 1, k, did, dw, out, mode)
        hip.synchronize()
        got = out.download(np.float32, hidden)
        assert np.linalg.norm(got - want) / np.linalg.norm(want) <= tol, ("device", mode)
    moe.close()


def test_moe_rejects_bad_expert_id():
    E, hidden, inter = 2, 256, 256
    gate, up, down, x, ids, wts = moe_case(9, E, hidden, inter, 1, 1)
    moe = rehip.MoeExperts(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, down, E, hidden, inter)
    with pytest.raises(rehip.RehipError) as e:
        moe.forward(x, 1, 1, np.array([5], np.uint32), wts)
    assert e.value.code == rehip.RE_ERR_ARG
