"""Int8 activation path on the GPU (re_quantize_q8_act[_dev], re_qmat_matmul_i8[_dev]) against
the oracle's restatement of Q8Activation::from_f32 / dot_q8_0_i8 / matmul_q8_0_i8
(src/kernel.rs:70-166). The bar is bit-identity: the reference's integer path is exact per
block and folds blocks in order, and so does the MFMA kernel. Full-size shapes compare the
oracle on a sample of activation rows (each output row depends only on its own input row)."""
import numpy as np
import pytest

import oracle as O
import rehip
from blockpack import q8_blocks
from rehip import hip, synth

pytestmark = pytest.mark.gpu
B = hip.DeviceBuffer


def activations(rng, rows, n):
    x = (rng.standard_normal((rows, n)) * np.exp(rng.uniform(-6, 6, (rows, 1)))).astype(np.float32)
    x[:, 5::97] = 0.0
    if rows > 2:
        x[1, :32] = 0.0                                   # an all-zero block
        x[2, 32:64] = np.float32(127) * np.arange(32, dtype=np.float32) / 2   # half-way quotients
    return x.reshape(-1)


def oracle_rows(x, rows, n):
    sc, qs = [], []
    for r in range(rows):
        s, q = O.quantize_q8_act(x[r * n:(r + 1) * n])
        sc.append(s)
        qs.append(q)
    return np.concatenate(sc), np.concatenate(qs)


@pytest.mark.parametrize("rows,n", [(1, 32), (1, 896), (37, 896), (5, 4864), (961, 896)])
def test_quantize_bit_exact(rows, n):
    rng = np.random.default_rng(rows + n)
    x = activations(rng, rows, n)
    sc, qs = rehip.quantize_q8_act(x, rows)
    want_sc, want_qs = oracle_rows(x, rows, n)
    assert np.array_equal(sc.view(np.uint32), want_sc.view(np.uint32))
    assert np.array_equal(qs, want_qs)


def test_quantize_nan_and_inf_blocks():
    x = np.zeros(96, np.float32)
    x[0], x[1], x[2] = np.nan, 63.5, -127.0
    x[32], x[33] = np.inf, 5.0
    x[64:96] = np.float32(-np.inf)
    sc, qs = rehip.quantize_q8_act(x, 1)
    want_sc, want_qs = O.quantize_q8_act(x)
    assert np.array_equal(sc.view(np.uint32), want_sc.view(np.uint32))
    assert np.array_equal(qs, want_qs)


def test_reference_fixture_matvec_and_matmul():
    """kernel.rs:2299-2326 on the GPU: m = 3, n = 64, the q8_blocks fixture."""
    m, n = 3, 64
    w = np.frombuffer(q8_blocks(m * n // 32), np.uint8)
    x = np.arange(2 * n, dtype=np.float32) * np.float32(0.037) - np.float32(7.0)
    sc, qs = rehip.quantize_q8_act(x, 2)
    q = rehip.QMat.from_bytes(rehip.Q8_0, w, m, n)
    got = q.matmul_i8(sc, qs, 2)
    assert np.array_equal(got, O.matmul_q8_0_i8(w, m, n, sc, qs, 2))
    deq_x = qs[:n].astype(np.float32) * np.repeat(sc[:2], 32)
    flt = O.matvec(rehip.Q8_0, w, m, n, deq_x)
    assert np.all(np.abs(got[:m] - flt) / np.maximum(np.abs(flt), 1.0) < 1e-3)
    q.close()


# rows >= 64 blocks over few output tiles take the K-segmented kernel (the fold handed from wave
# to wave): (130, 2048, 33), (64, 2080, 5) with a one-block last round, (896, 4864, 7), and
# (64, 9600, 3) whose 300 blocks of scales are staged in two chunks
@pytest.mark.parametrize("m,n,rows", [(64, 32, 1), (130, 256, 1), (130, 256, 33), (256, 896, 961),
                                      (4864, 896, 1), (896, 4864, 7), (130, 2048, 33), (64, 2080, 5),
                                      (64, 9600, 3)])
def test_matmul_i8_bit_exact(m, n, rows):
    rng = np.random.default_rng(m + n + rows)
    w = synth.weight_bytes(rng, rehip.Q8_0, m, n)
    x = activations(rng, rows, n)
    sc, qs = O.quantize_q8_act(x)
    q = rehip.QMat.from_bytes(rehip.Q8_0, w, m, n)
    got = q.matmul_i8(sc, qs, rows)
    want = O.matmul_q8_0_i8(w, m, n, sc, qs, rows)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    q.close()


@pytest.mark.parametrize("m,n", [(4864, 896), (896, 4864)])
def test_matmul_i8_full_size_sampled_rows(m, n):
    """961 activation rows; the oracle on 6 of them, through the device entry points."""
    rows = 961
    rng = np.random.default_rng(m)
    w = synth.weight_bytes(rng, rehip.Q8_0, m, n)
    x = activations(rng, rows, n)
    q = rehip.QMat.from_bytes(rehip.Q8_0, w, m, n)
    xd, sd, qd, yd = B.from_array(x), B(rows * (n // 32) * 4), B(rows * n), B(rows * m * 4)
    rehip.quantize_q8_act_dev(xd, rows, n, sd, qd)
    q.matmul_i8_dev(sd, qd, rows, yd)
    hip.synchronize()
    y = yd.download().reshape(rows, m)
    sc = sd.download(np.float32)
    qs = qd.download(np.int8)
    for r in (0, 1, 2, 31, 32, 960):
        s_r, q_r = O.quantize_q8_act(x[r * n:(r + 1) * n])
        assert np.array_equal(sc[r * (n // 32):(r + 1) * (n // 32)], s_r) and np.array_equal(qs[r * n:(r + 1) * n], q_r)
        want = O.matmul_q8_0_i8(w, m, n, s_r, q_r, 1)
        assert np.array_equal(y[r].view(np.uint32), want.view(np.uint32)), r
    q.close()


def test_errors():
    rng = np.random.default_rng(1)
    q = rehip.QMat.from_bytes(rehip.Q4_K, synth.weight_bytes(rng, rehip.Q4_K, 64, 256), 64, 256)
    sc, qs = O.quantize_q8_act(np.ones(256, np.float32))
    with pytest.raises(rehip.RehipError) as e:
        q.matmul_i8(sc, qs, 1)
    assert e.value.code == rehip.RE_ERR_TYPE
    q.close()
    with pytest.raises(rehip.RehipError) as e:
        rehip.quantize_q8_act(np.ones(48, np.float32), 1)
    assert e.value.code == rehip.RE_ERR_SIZE
