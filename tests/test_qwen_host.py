"""Host side of the dense decoder (rehip.qwen) on the CPU backend: the reference's forward.rs
and runner.rs tests restated (zeroed projections reduce a block to its residual, single-token
attention returns the value, incremental decode equals re-prefill), plus closed forms for the
host steps."""
import math

import numpy as np
import pytest

import oracle as O
from oracle.backend import CpuBackend
from rehip import qwen

TINY = qwen.Geometry(d_model=128, n_heads=4, n_kv_heads=2, d_ff=256, rope_freq_base=1e4, rms_eps=1e-5)


def test_rmsnorm_closed_form():
    x = np.array([[1.0, -2.0, 3.0, 0.5]], np.float32)
    w = np.array([1.0, 0.5, 2.0, -1.0], np.float32)
    inv = 1.0 / math.sqrt((1 + 4 + 9 + 0.25) / 4 + 1e-5)
    assert np.allclose(qwen.rmsnorm_rows(x, w, 1e-5)[0], x[0] * inv * w, rtol=1e-6)


def test_rope_matches_per_pair_rotation():
    # infer.rs:98-108 restated element by element
    d, base, heads = 8, 1e4, 2
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, heads * d)).astype(np.float32)
    cos, sin = qwen.rope_table(3, 5, d, base)
    got = qwen.rope_rows(x, heads, d, cos, sin)
    for r in range(3):
        pos = 5 + r
        for h in range(heads):
            v = x[r, h * d:(h + 1) * d]
            for i in range(d // 2):
                ang = pos * (1.0 / base ** (2 * i / d))
                c, s = math.cos(ang), math.sin(ang)
                assert abs(got[r, h * d + i] - (v[i] * c - v[i + d // 2] * s)) < 1e-4
                assert abs(got[r, h * d + i + d // 2] - (v[i + d // 2] * c + v[i] * s)) < 1e-4
    # position 0 is the identity
    c0, s0 = qwen.rope_table(1, 0, d, base)
    assert np.array_equal(qwen.rope_rows(x[:1], heads, d, c0, s0), x[:1])


def test_softmax_and_argmax_tie_rule():
    p = qwen.softmax_rows(np.array([[1.0, 2.0, -np.inf, 3.0]], np.float32))
    assert abs(p.sum() - 1) < 1e-6 and p[0, 2] == 0
    assert qwen.argmax_last(np.array([1, 5, 5, 2], np.float32)) == 2      # Iterator::max_by
    assert qwen.argmax_last(np.array([7], np.float32)) == 0


def test_single_position_attention_returns_value():
    # forward.rs:285-316: softmax over one key is 1, so each head's context is its GQA value
    g = TINY
    rng = np.random.default_rng(1)
    kv = g.n_kv_heads * g.head_dim
    q = rng.standard_normal((1, g.d_model)).astype(np.float32)
    kc = rng.standard_normal((4, kv)).astype(np.float32)
    vc = rng.standard_normal((4, kv)).astype(np.float32)
    ctx = qwen.attention(q, kc, vc, g, 0).reshape(g.n_heads, g.head_dim)
    for h in range(g.n_heads):
        kvh = h * g.n_kv_heads // g.n_heads
        assert np.array_equal(ctx[h], vc[0, kvh * g.head_dim:(kvh + 1) * g.head_dim])


def tiny_model(seed, zero=False):
    mb = qwen.synth_model(seed, TINY, n_layers=2, n_vocab=300)
    if zero:
        for b in mb.blocks:
            for f in ("q", "k", "v", "o", "gate", "up", "down"):
                getattr(b, f)[:] = 0
    return mb


@pytest.mark.skipif(not O.cpu_has_avx2(), reason="host has no AVX2+FMA")
def test_zeroed_projections_reduce_blocks_to_residual():
    mb = tiny_model(3, zero=True)
    be = CpuBackend(threads=2)
    r = qwen.DenseRunner(mb, be)
    dec = qwen.DenseDecoder(r, 16)
    prompt = [5, 17, 42]
    logits = dec.prefill(prompt)
    emb = O.dequant(mb.embed_type, mb.embed).reshape(mb.n_vocab, TINY.d_model)
    normed = qwen.rmsnorm_rows(emb[42], mb.output_norm, TINY.rms_eps).reshape(-1)
    want = O.cpu_matvec(mb.embed_type, mb.output, mb.n_vocab, TINY.d_model, normed, threads=2)
    assert np.array_equal(logits, want)


@pytest.mark.skipif(not O.cpu_has_avx2(), reason="host has no AVX2+FMA")
def test_incremental_decode_matches_reprefill():
    # runner.rs:190-282: the cached decoder produces the token stream of re-prefilling the
    # whole sequence every step
    mb = tiny_model(4)
    r = qwen.DenseRunner(mb, CpuBackend(threads=2))
    prompt = [3, 1, 4, 1, 5, 9, 2, 6]
    inc = qwen.DenseDecoder(r, 64).generate(prompt, 8)
    seq = list(prompt)
    ref = []
    for _ in range(8):
        t = qwen.argmax_last(qwen.DenseDecoder(r, 64).prefill(seq))
        ref.append(t)
        seq.append(t)
    assert inc == ref
