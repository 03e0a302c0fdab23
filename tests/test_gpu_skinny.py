"""The few-row dense GEMM (2..32 rows in bf16 mode, 2..64 in f32 mode; above that the tiled GEMM
runs: weights decoded in registers, one workgroup per 64-row tile and K slice, the split-K reduce in
slice order) against an f64 product of the oracle's exact
dequantization: bf16 mode within 1e-2 relative to norm, f32 mode (split bf16 operands) within
2^-10 * sum|w x| per output. Every type, ragged K (K-quant rows at K = 896), partial weight tiles,
one and many K slices, and a captured graph on a matrix never called before (one slice, no
allocation under capture)."""
import numpy as np
import pytest

import oracle as O
import rehip
from rehip import hip, synth

pytestmark = pytest.mark.gpu

TYPES = [rehip.Q4_0, rehip.Q5_0, rehip.Q8_0, rehip.Q4_K, rehip.Q5_K, rehip.Q6_K]


def f64_product(t, w, m, n, x, rows):
    qk, _ = rehip.GEOM[t]
    nb = (n + qk - 1) // qk
    deq = O.dequant(t, w).reshape(m, nb * qk)[:, :n].astype(np.float64)
    xx = x.reshape(rows, n).astype(np.float64)
    return (xx @ deq.T).reshape(-1), (np.abs(xx) @ np.abs(deq).T).reshape(-1)


def check(got, exact, absd, mode, what):
    if mode == rehip.MODE_F32:
        assert np.all(np.abs(got - exact) <= 2.0 ** -10 * absd), what
    else:
        assert np.linalg.norm(got - exact) / np.linalg.norm(exact) <= 1e-2, what


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("m,n,rows", [(896, 4864, 64), (896, 4864, 32), (200, 896, 17), (4864, 896, 2),
                                      (70, 2048, 33), (130, 512, 64), (64, 256, 5)])
def test_skinny_against_f64(t, m, n, rows):
    rng = np.random.default_rng(9300 + t + m + rows)
    w = synth.weight_bytes(rng, t, m, n)
    x = synth.activations(rng, rows, n)
    q = rehip.QMat.from_bytes(t, w, m, n)
    exact, absd = f64_product(t, w, m, n, x, rows)
    for mode in (rehip.MODE_BF16, rehip.MODE_F32):
        got = q.matmul(x, rows, mode)
        check(got, exact, absd, mode, (mode, m, n, rows))
        again = q.matmul(x, rows, mode)
        assert np.array_equal(got, again), "deterministic"
    q.close()


@pytest.mark.parametrize("mode,rows", [(rehip.MODE_BF16, 32), (rehip.MODE_F32, 64)])
def test_skinny_under_capture_on_a_fresh_matrix(mode, rows):
    # C2's shape plans 19 K slices; a never-called matrix under capture runs one slice
    t, m, n = rehip.Q6_K, 896, 4864
    rng = np.random.default_rng(9400)
    w = synth.weight_bytes(rng, t, m, n)
    x = synth.activations(rng, rows, n)
    exact, absd = f64_product(t, w, m, n, x, rows)
    q = rehip.QMat.from_bytes(t, w, m, n)
    dx = hip.DeviceBuffer.from_array(x)
    yg = hip.DeviceBuffer(rows * m * 4)
    s = hip.Stream()
    g = hip.Graph(s, lambda: q.matmul_dev(dx, rows, yg, mode, stream=s))
    for rep in range(3):
        g.launch()
        s.synchronize()
        check(yg.download(np.float32, rows * m), exact, absd, mode, rep)
        q.matmul(x[: 8 * n], 8, mode)        # eager work between replays
    g.destroy()
    s.destroy()
    q.close()
