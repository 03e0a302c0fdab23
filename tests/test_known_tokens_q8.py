"""The reference's known-answer construction of tests/dense_gen.rs:64-259 (residual-only blocks,
token 2 embeds to [1, 2, 0, ...], output row 4 = [1, 1, 0, ...] dominates, a zero embedding makes
every logit 0 and the last index wins) restated with Q8_0 weights at a shape the device-resident
decoder covers (d_model 64, 2 heads of head_dim 32, d_ff 64, vocab 5, 2 layers). The known
answers follow from the construction alone, not from any implementation:
  * prefill([2]) picks 4: the final RMS-norm scales [1, 2, 0, ...] by a positive factor, row 4's
    logit is 3 times that factor, row 0's 0.1 times it, the others 0;
  * generate([2], 3) == [2, 4, 4, 4]: token 4 embeds to zeros, the residual stream stays zero,
    the RMS-norm of zero is zero, every logit is 0 and the largest index (4) wins
    (infer.rs:217-223).
Q8_0 holds every weight exactly (1 = 32/32, 2 = 64/32; 0.1 as 100 * f16(0.001)).
The CPU test checks the construction with the oracle-backed host decoder and that DeviceDecoder
refuses the reference's own F32 fixture (head_dim 2: the attention kernels take multiples of 4)
with a clear error; the GPU tests run the device-resident decoder and the HIP host-step path."""
import numpy as np
import pytest

import rehip
from rehip import qwen

D, FF, NV = 64, 64, 5


def q8_rows(rows: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Q8_0 bytes of integer quants rows (m x n, |q| <= 127) with one f16 scale per row."""
    m, n = rows.shape
    out = bytearray()
    for r in range(m):
        for b in range(n // 32):
            out += np.float16(scales[r]).tobytes()
            out += rows[r, 32 * b:32 * b + 32].astype(np.int8).tobytes()
    return np.frombuffer(bytes(out), np.uint8).copy()


def known_answer_model() -> qwen.ModelBytes:
    g = qwen.Geometry(d_model=D, n_heads=2, n_kv_heads=2, d_ff=FF, rope_freq_base=1e4, rms_eps=1e-6)
    zq = lambda m, n: q8_rows(np.zeros((m, n)), np.zeros(m))   # noqa: E731
    emb = np.zeros((NV, D))
    emb[2, 0], emb[2, 1] = 32, 64                     # [1, 2, 0, ...] at scale 1/32
    out = np.zeros((NV, D))
    out[4, 0] = out[4, 1] = 32                        # [1, 1, 0, ...]
    out[0, 0] = 100                                   # 0.1 at scale 0.001
    out_scales = np.array([0.001, 1 / 32, 1 / 32, 1 / 32, 1 / 32])
    kv = g.n_kv_heads * g.head_dim
    ones = np.ones(D, np.float32)
    blocks = [qwen.BlockBytes(q=zq(D, D), k=zq(kv, D), v=zq(kv, D), o=zq(D, D), gate=zq(FF, D), up=zq(FF, D),
                              down=zq(D, FF), attn_norm=ones, ffn_norm=ones, q_bias=np.zeros(D, np.float32),
                              k_bias=np.zeros(kv, np.float32), v_bias=np.zeros(kv, np.float32))
              for _ in range(2)]
    return qwen.ModelBytes(geom=g, n_vocab=NV, embed=q8_rows(emb, np.full(NV, 1 / 32)),
                           output=q8_rows(out, out_scales), output_norm=ones, blocks=blocks,
                           attn_type=rehip.Q8_0, ffn_type=rehip.Q8_0, down_type=rehip.Q8_0,
                           embed_type=rehip.Q8_0)


def host_generate(backend, prompt, n):
    r = qwen.DenseRunner(known_answer_model(), backend)
    dec = qwen.DenseDecoder(r, len(prompt) + n + 1)
    logits = dec.prefill(prompt)
    toks = list(prompt) + [qwen.argmax_last(logits)]
    for _ in range(n - 1):
        logits = dec.step(toks[-1])
        toks.append(qwen.argmax_last(logits))
    return toks


def test_construction_on_the_oracle_host_path():
    import test_qwen_gguf as T
    assert host_generate(T.OracleQMatBackend(), [2], 3) == [2, 4, 4, 4]


def test_device_decoder_refuses_the_dense_head_dim_2_fixture(tmp_path):
    # dense F32 weights are covered; head_dim 2 is not (the attention kernels take multiples of 4)
    import test_qwen_gguf as T
    path = tmp_path / "dense_gen.gguf"
    path.write_bytes(T.synth_dense_gguf())
    g = rehip.Gguf(path)
    mb = qwen.model_from_gguf(g)
    with pytest.raises(ValueError, match="head_dim"):
        qwen.DeviceDecoder(mb, max_seq=8)
    g.close()


@pytest.mark.gpu
def test_device_decoder_known_tokens():
    dd = qwen.DeviceDecoder(known_answer_model(), max_seq=8, mode=rehip.MODE_F32, prefill_rows=4)
    assert dd.generate([2], 3) == [4, 4, 4]
    dd.close()
    dd = qwen.DeviceDecoder(known_answer_model(), max_seq=8, mode=rehip.MODE_F32, prefill_rows=4)
    assert dd.prefill([2]) == 4
    lg = dd.logits()
    assert np.all(np.isfinite(lg)) and int(np.argmax(lg)) == 4 and lg[4] > lg[0] > 0
    for _ in range(3):
        assert dd.step() == 4
        assert np.all(dd.logits() == 0.0)
    dd.close()


@pytest.mark.gpu
def test_hip_host_step_known_tokens():
    assert host_generate(qwen.HipBackend(rehip.MODE_F32), [2], 3) == [2, 4, 4, 4]
