"""GGUF tensors straight to the device (re_qmat_from_gguf / re_moe_from_gguf): the mapped bytes
are copied unchanged and repacked by a kernel. Checked bit-exact against the oracle's dequant
(quant.rs:363-453) through the resident dequant, and against matrices built from the same bytes
held in host memory (QMat::from_bytes, qmat.rs:52-59) through the GEMV; the error texts follow
QMat::from_model (qmat.rs:318-327)."""
import numpy as np
import pytest

import ggufw as W
import oracle as O
import rehip
from rehip import hip, synth

pytestmark = pytest.mark.gpu
B = hip.DeviceBuffer


def _model(tmp_path, tensors, kvs=(), alignment=32, name="w.gguf"):
    p = tmp_path / name
    p.write_bytes(W.write(list(kvs), tensors, alignment=alignment))
    return rehip.Gguf(p)


def _dequant_dev(q, m, n):
    out = B(m * n * 4)
    q.dequant_dev(out)
    hip.synchronize()
    return out.download()


def _oracle_rows(t, w, m, n):
    qk, _ = rehip.GEOM[t]
    nb = (n + qk - 1) // qk
    return O.dequant(t, w).reshape(m, nb * qk)[:, :n].reshape(-1)


@pytest.mark.parametrize("t", rehip.QUANT_TYPES)
@pytest.mark.parametrize("m,n", [(1, 256), (130, 1536), (64, 4864)])
def test_qmat_from_gguf_dequant_bit_exact(tmp_path, t, m, n):
    rng = np.random.default_rng(300 + t + m)
    w = synth.weight_bytes(rng, t, m, n)
    qk, _ = rehip.GEOM[t]
    # a leading f32 tensor moves the quant tensor off the start of the data section
    with _model(tmp_path, [("norm", [7], 0, bytes(28)), ("w", [n, m], t, w.tobytes())],
                kvs=[("general.alignment", W.U32, 64)], alignment=64) as f:
        assert f.tensor_bytes("w").tobytes() == w.tobytes()
        q = rehip.QMat.from_gguf(f, "w", m, n)
    got = _dequant_dev(q, m, n)
    assert np.array_equal(got.view(np.uint32), _oracle_rows(t, w, m, n).view(np.uint32))
    # the GEMV of the same bytes held in host memory gives the same bits
    x = synth.activations(rng, 1, n)
    q2 = rehip.QMat.from_bytes(t, w, m, n)
    assert np.array_equal(q.matvec(x), q2.matvec(x))
    q.close()
    q2.close()


def test_qmat_from_gguf_spans_upload_chunks(tmp_path):
    """A 36 MB Q8_0 matrix: two 32 MiB upload chunks, the second ending in a partial tile."""
    t, m, n = rehip.Q8_0, 8300, 4096
    rng = np.random.default_rng(5)
    w = synth.weight_bytes(rng, t, m, n)
    with _model(tmp_path, [("w", [n, m], t, w.tobytes())]) as f:
        q = rehip.QMat.from_gguf(f, "w", m, n)
    got = _dequant_dev(q, m, n)
    assert np.array_equal(got.view(np.uint32), _oracle_rows(t, w, m, n).view(np.uint32))
    q.close()


def test_stacked_tensor_becomes_stacked_qmat(tmp_path):
    t, m, n, E = rehip.Q4_K, 96, 512, 5
    rng = np.random.default_rng(11)
    mats = [synth.weight_bytes(rng, t, m, n) for _ in range(E)]
    with _model(tmp_path, [("exps", [n, m, E], t, np.concatenate(mats).tobytes())]) as f:
        q = rehip.QMat.from_gguf(f, "exps", m, n)
    assert q.count() == E
    x = synth.activations(rng, E, n)
    y = B(E * m * 4)
    q.matvec_stacked_dev(0, E, B.from_array(x), n, y, m)
    hip.synchronize()
    got = y.download().reshape(E, m)
    for e in range(E):
        want = rehip.QMat.from_bytes(t, mats[e], m, n).matvec(x[e * n:(e + 1) * n])
        deq = _oracle_rows(t, mats[e], m, n).reshape(m, n).astype(np.float64)
        bound = np.abs(deq) @ np.abs(x[e * n:(e + 1) * n].astype(np.float64))
        assert np.all(np.abs(got[e] - want) <= 2.0 ** -10 * bound + 1e-30), e
    q.close()


def test_moe_from_gguf_equals_moe_from_bytes(tmp_path):
    E, hidden, inter, T, k = 8, 512, 256, 6, 2
    rng = np.random.default_rng(21)
    gate = np.concatenate([synth.weight_bytes(rng, rehip.Q4_K, inter, hidden) for _ in range(E)])
    up = np.concatenate([synth.weight_bytes(rng, rehip.Q4_K, inter, hidden) for _ in range(E)])
    dn = np.concatenate([synth.weight_bytes(rng, rehip.Q6_K, hidden, inter) for _ in range(E)])
    tensors = [("blk.0.ffn_gate_exps.weight", [hidden, inter, E], rehip.Q4_K, gate.tobytes()),
               ("blk.0.ffn_up_exps.weight", [hidden, inter, E], rehip.Q4_K, up.tobytes()),
               ("blk.0.ffn_down_exps.weight", [inter, hidden, E], rehip.Q6_K, dn.tobytes())]
    with _model(tmp_path, tensors) as f:
        a = rehip.MoeExperts.from_gguf(f, *(t[0] for t in tensors), E, hidden, inter)
        with pytest.raises(rehip.RehipError) as e:    # down's dims checked against [inter, hidden, E]
            rehip.MoeExperts.from_gguf(f, tensors[0][0], tensors[1][0], tensors[0][0], E, hidden, inter)
        assert "dims are not" in e.value.message
    b = rehip.MoeExperts(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, dn, E, hidden, inter)
    x = synth.activations(rng, T, hidden)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32).reshape(-1)
    wts = rng.random(T * k).astype(np.float32)
    for mode in (rehip.MODE_F32, rehip.MODE_BF16):
        assert np.array_equal(a.forward(x, T, k, ids, wts, mode), b.forward(x, T, k, ids, wts, mode))
    a.close()
    b.close()


def test_from_model_errors(tmp_path):
    t, m, n = rehip.Q4_0, 64, 256
    w = synth.weight_bytes(np.random.default_rng(1), t, m, n)
    with _model(tmp_path, [("w", [n, m], t, w.tobytes())]) as f:
        with pytest.raises(rehip.RehipError) as e:
            rehip.QMat.from_gguf(f, "nope", m, n)
        assert e.value.message == "QMat: tensor 'nope' missing"
        with pytest.raises(rehip.RehipError) as e:
            rehip.QMat.from_gguf(f, "w", n, m)           # transposed shape
        assert e.value.code == rehip.RE_ERR_SIZE
    hdr = tmp_path / "hdr.gguf"
    hdr.write_bytes(W.synth_gguf())
    with rehip.Gguf(hdr) as f:
        with pytest.raises(rehip.RehipError) as e:
            rehip.QMat.from_gguf(f, "blk.0.ffn_gate_exps.weight", 512, 2048)
        assert e.value.message == "QMat: tensor 'blk.0.ffn_gate_exps.weight' bytes out of bounds"
