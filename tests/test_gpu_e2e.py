"""End-to-end greedy parity on a seeded random-init Qwen2.5-0.5B-shaped model (24 layers,
hidden 896, 14/2 heads, d_ff 4864, vocab 151936, Q4_K_M mix): a 961-token random prompt is
prefilled and 64 tokens are decoded greedily with every projection on the GPU (f32 GEMM/GEMV)
and, separately, on the reference-restated CPU kernels; the host steps (attention, norms, RoPE,
argmax) are shared. The token streams must be identical."""
import numpy as np
import pytest

import rehip
from oracle.backend import CpuBackend
from rehip import qwen

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model():
    return qwen.synth_model(501)


def run(mb, backend, prompt, steps):
    r = qwen.DenseRunner(mb, backend)
    dec = qwen.DenseDecoder(r, len(prompt) + steps)
    logits = dec.prefill(prompt)
    first = logits.copy()
    toks = [qwen.argmax_last(logits)]
    for _ in range(steps - 1):
        toks.append(qwen.argmax_last(dec.step(toks[-1])))
    if hasattr(r, "close"):
        r.close()
    return toks, first


def test_greedy_64_steps_match_cpu_path(model):
    prompt = np.random.default_rng(502).integers(0, model.n_vocab, 961)
    got, lg_gpu = run(model, qwen.HipBackend(rehip.MODE_F32), prompt, 64)
    want, lg_cpu = run(model, CpuBackend(), prompt, 64)
    # prefill logits agree to f32 accumulation differences
    assert np.max(np.abs(lg_gpu - lg_cpu)) <= 1e-3 * np.max(np.abs(lg_cpu))
    assert got == want, next(i for i, (a, b) in enumerate(zip(got, want)) if a != b)


def test_tiny_model_decode_matches_cpu_path():
    g = qwen.Geometry(d_model=256, n_heads=4, n_kv_heads=2, d_ff=512, rope_freq_base=1e4, rms_eps=1e-5)
    mb = qwen.synth_model(7, g, n_layers=3, n_vocab=1000)
    prompt = [1, 2, 3, 5, 8, 13, 21, 34, 55, 89]
    got, _ = run(mb, qwen.HipBackend(rehip.MODE_F32), prompt, 20)
    want, _ = run(mb, CpuBackend(), prompt, 20)
    assert got == want
