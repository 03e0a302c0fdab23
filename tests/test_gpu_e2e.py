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


GATE_STEPS = 24


@pytest.fixture(scope="module")
def cpu_reference(model):
    """The f32 CPU path (reference-restated kernels): prefill logits and GATE_STEPS greedy steps,
    with every position's logits."""
    prompt = np.random.default_rng(502).integers(0, model.n_vocab, 961)
    r = qwen.DenseRunner(model, CpuBackend())
    dec = qwen.DenseDecoder(r, len(prompt) + GATE_STEPS + 1)
    logits = [dec.prefill(prompt).copy()]
    toks = [qwen.argmax_last(logits[0])]
    for _ in range(GATE_STEPS):
        logits.append(dec.step(toks[-1]).copy())
        toks.append(qwen.argmax_last(logits[-1]))
    return prompt, toks, logits


def _gate_all(ref_logits, got_logits):
    res = [qwen.logit_profile_check(r, g) for r, g in zip(ref_logits, got_logits)]
    bad = [(i, c) for i, c in enumerate(res) if not c["ok"]]
    assert not bad, bad[:3]
    return res


def test_bf16_profile_gate_host_step_path(model, cpu_reference):
    # bf16 MFMA projections (HipBackend), host attention/norms, teacher-forced on the CPU path's
    # greedy tokens: every position passes the reference's profile gate against the f32 CPU logits
    prompt, toks, ref = cpu_reference
    r = qwen.DenseRunner(model, qwen.HipBackend(rehip.MODE_BF16))
    dec = qwen.DenseDecoder(r, len(prompt) + GATE_STEPS + 1)
    got = [dec.prefill(prompt).copy()]
    for t in toks[:GATE_STEPS]:
        got.append(dec.step(t).copy())
    r.close()
    res = _gate_all(ref, got)
    assert sum(c["decisive"] for c in res) >= 1   # the gate exercised the argmax condition


def test_bf16_profile_gate_device_decoder(model, cpu_reference):
    # the device-resident decoder in bf16 mode (bf16 MFMA prefill GEMMs, decode GEMVs): prefill and
    # GATE_STEPS teacher-forced decode steps, each position gated against the f32 CPU logits
    prompt, toks, ref = cpu_reference
    dd = qwen.DeviceDecoder(model, max_seq=len(prompt) + GATE_STEPS + 1, mode=rehip.MODE_BF16,
                            prefill_rows=len(prompt))
    dd.prefill(prompt)
    got = [dd.logits()]
    for t in toks[:GATE_STEPS]:
        dd.tok.upload(np.array([t], np.int32))      # force the CPU path's token
        dd.step()
        got.append(dd.logits())
    dd.close()
    _gate_all(ref, got)
