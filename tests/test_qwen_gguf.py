"""The reference's dense end-to-end fixture (tests/dense_gen.rs:64-259) through the host-step
decoder (rehip.qwen): a 2-layer qwen2 GGUF of F32 tensors (d_model 4, 2 heads, 2 KV heads,
d_ff 8, vocab 5) whose attention output and FFN projections are zero, so every block is
residual-only; token 2 embeds to [1, 2, 0, 0] and output row 4 = [1, 1, 0, 0] dominates.
Known answers from the reference's tests:
  * greedy([2]) == 4 and the logits are finite and repeatable (dense_gen.rs:194-222);
  * generate([2], 3) == [2, 4, 4, 4] (dense_gen.rs:224-238): after token 4 (a zero embedding)
    every logit is 0 and the last index among equal maxima wins;
  * the incremental decoder equals re-prefilling (dense_gen.rs:240-259).
The file is written with the GGUF writer (tests/gguf_writer.py), mapped by librehip's GGUF
reader (rehip.Gguf) and loaded by rehip.qwen.model_from_gguf. The CPU tests run the projections
on the oracle's QMat over F32 weights (oracle.qmat_matvec, the reference's sequential f32 sum);
the GPU test runs them through librehip (HipBackend)."""
import numpy as np
import pytest

import gguf_writer as W
import oracle as O
import rehip
from rehip import qwen

DM, NV, FF, NH, KV = 4, 5, 8, 4, 4


def synth_dense_gguf() -> bytes:
    """dense_gen.rs:64-190: tensors as (name, ggml dims [ne0, ne1], F32 values)."""
    f32 = lambda a: np.asarray(a, np.float32).tobytes()   # noqa: E731
    emb = np.zeros(DM * NV, np.float32)
    emb[2 * DM], emb[2 * DM + 1] = 1.0, 2.0
    out = np.zeros(DM * NV, np.float32)
    out[4 * DM] = out[4 * DM + 1] = 1.0
    out[0] = 0.1
    ones = np.ones(DM, np.float32)
    tensors = [("token_embd.weight", [DM, NV], 0, f32(emb)), ("output.weight", [DM, NV], 0, f32(out)),
               ("output_norm.weight", [DM], 0, f32(ones))]
    for i in range(2):
        p = f"blk.{i}."
        tensors += [(p + "attn_norm.weight", [DM], 0, f32(ones)),
                    (p + "attn_q.weight", [DM, NH], 0, f32(np.full(DM * NH, 0.3))),
                    (p + "attn_k.weight", [DM, KV], 0, f32(np.full(DM * KV, 0.2))),
                    (p + "attn_v.weight", [DM, KV], 0, f32(np.full(DM * KV, 0.1))),
                    (p + "attn_output.weight", [DM, NH], 0, f32(np.zeros(DM * NH))),
                    (p + "ffn_norm.weight", [DM], 0, f32(ones)),
                    (p + "ffn_gate.weight", [DM, FF], 0, f32(np.zeros(DM * FF))),
                    (p + "ffn_up.weight", [DM, FF], 0, f32(np.zeros(DM * FF))),
                    (p + "ffn_down.weight", [FF, DM], 0, f32(np.zeros(FF * DM)))]
    kvs = [("general.architecture", W.STR, "qwen2"), ("qwen2.embedding_length", W.U32, DM),
           ("qwen2.block_count", W.U32, 2), ("qwen2.attention.head_count", W.U32, 2),
           ("qwen2.attention.head_count_kv", W.U32, 2), ("qwen2.feed_forward_length", W.U32, FF),
           ("qwen2.vocab_size", W.U32, NV)]
    return W.write(kvs, tensors, alignment=32)


class OracleQMatBackend:
    """Projections on the oracle's QMat semantics (test infrastructure)."""
    name = "oracle"

    @staticmethod
    def dequant(ggml_type, data):
        return O.dequant(ggml_type, data)

    def make(self, ggml_type, data, m, n):
        data = np.ascontiguousarray(data, dtype=np.uint8)

        class _M:
            def matvec(self_, x):
                return O.qmat_matvec(ggml_type, data, m, n, x)

            def matmul(self_, x, rows):
                return O.qmat_matmul(ggml_type, data, m, n, x, rows)

        return _M()


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    path = tmp_path_factory.mktemp("dense_gen") / "dense_gen.gguf"
    path.write_bytes(synth_dense_gguf())
    g = rehip.Gguf(path)
    mb = qwen.model_from_gguf(g)
    yield mb
    g.close()


def test_model_config_from_gguf(model):
    g = model.geom
    assert (g.d_model, g.n_heads, g.n_kv_heads, g.d_ff, model.n_vocab, len(model.blocks)) == (4, 2, 2, 8, 5, 2)
    assert g.rope_freq_base == 10000.0 and abs(g.rms_eps - 1e-5) < 1e-12     # model.rs:237-238 defaults
    assert all(t == 0 for t in model.blocks[0].types.values())
    assert not model.blocks[1].q_bias.any()                                    # absent bias = none


def known_answers(runner):
    dec = qwen.DenseDecoder(runner, 8)
    logits = dec.prefill([2])
    assert logits.shape == (NV,) and np.all(np.isfinite(logits))
    assert qwen.argmax_last(logits) == 4                                       # dense_gen.rs:214
    assert np.array_equal(qwen.DenseDecoder(runner, 8).prefill([2]), logits)
    assert runner.generate([2], 3) == [2, 4, 4, 4]                             # dense_gen.rs:234
    full = runner.generate([2, 3], 5)
    assert [2, 3] + qwen.DenseDecoder(runner, 16).generate([2, 3], 5) == full  # dense_gen.rs:240-259


def test_dense_gen_known_tokens_cpu(model):
    known_answers(qwen.DenseRunner(model, OracleQMatBackend()))


@pytest.mark.gpu
def test_dense_gen_known_tokens_hip(model):
    for mode in (rehip.MODE_F32, rehip.MODE_BF16):
        r = qwen.DenseRunner(model, qwen.HipBackend(mode))
        known_answers(r)
        r.close()
