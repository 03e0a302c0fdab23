"""re_qmat_matmul_noalloc_dev: the GEMM entry point that allocates nothing (K-split partials in
the library's static device scratch) against re_qmat_matmul_dev on the same inputs. Same plan,
kernels and summation order, so the bar is bit-identity (stricter than the bf16 1e-2 / f32
2^-10 * sum|w x| bars, which are checked against an f64 product as well).

Two calls in a row, the second with fewer rows, check that the shared scratch carries nothing
from one call into the next; a graph captured on a never-warmed matrix shows the split plan
runs under capture; a forced plan whose partials exceed the scratch fails cleanly."""
import numpy as np
import pytest

import oracle as O
import rehip
from rehip import hip, synth

pytestmark = pytest.mark.gpu


def f64_product(t, w, m, n, x, rows):
    qk, _ = rehip.GEOM[t]
    nb = (n + qk - 1) // qk
    deq = O.dequant(t, w).reshape(m, nb * qk)[:, :n].astype(np.float64)
    xx = x.reshape(rows, n).astype(np.float64)
    return xx @ deq.T, np.abs(xx) @ np.abs(deq).T


def both(q, x, rows, m, mode):
    dx = hip.DeviceBuffer.from_array(x)
    ya, yb = hip.DeviceBuffer(rows * m * 4), hip.DeviceBuffer(rows * m * 4)
    q.matmul_noalloc_dev(dx, rows, ya, mode)
    hip.synchronize()
    got = ya.download(np.float32, rows * m)
    q.matmul_dev(dx, rows, yb, mode)
    hip.synchronize()
    return got, yb.download(np.float32, rows * m)


@pytest.mark.parametrize("mode", [rehip.MODE_BF16, rehip.MODE_F32])
def test_noalloc_equals_matmul_dev_two_calls(mode):
    # Q6_K 896 x 4864: 961 rows (bf16: 128 x 256 tiles, 8 K splits, 27.6 MB of partials) then
    # 300 rows (64 x 64 tiles, K-groups and splits)
    t, m, n = rehip.Q6_K, 896, 4864
    rng = np.random.default_rng(7700 + mode)
    w = synth.weight_bytes(rng, t, m, n)
    q = rehip.QMat.from_bytes(t, w, m, n)
    for rows in (961, 300):
        x = synth.activations(rng, rows, n)
        got, want = both(q, x, rows, m, mode)
        assert np.array_equal(got, want), rows
        exact, absd = f64_product(t, w, m, n, x, rows)
        exact, absd = exact.reshape(-1), absd.reshape(-1)
        if mode == rehip.MODE_F32:
            assert np.all(np.abs(got - exact) <= 2.0 ** -10 * absd), rows
        else:
            assert np.linalg.norm(got - exact) / np.linalg.norm(exact) <= 1e-2, rows
    q.close()


def test_noalloc_under_graph_capture():
    # a fresh matrix, never called before: the captured graph runs the planned K split (the
    # allocating entry point would fall back to an unsplit launch under capture)
    t, m, n, rows = rehip.Q4_K, 896, 4864, 640
    rng = np.random.default_rng(7800)
    w = synth.weight_bytes(rng, t, m, n)
    x = synth.activations(rng, rows, n)
    q = rehip.QMat.from_bytes(t, w, m, n)
    dx = hip.DeviceBuffer.from_array(x)
    yg = hip.DeviceBuffer(rows * m * 4)
    s = hip.Stream()
    g = hip.Graph(s, lambda: q.matmul_noalloc_dev(dx, rows, yg, rehip.MODE_BF16, stream=s))
    ye = hip.DeviceBuffer(rows * m * 4)
    q.matmul_dev(dx, rows, ye, rehip.MODE_BF16)           # eager, the existing entry point
    hip.synchronize()
    want = ye.download(np.float32, rows * m)
    other = synth.activations(rng, 200, n)
    for rep in range(3):
        g.launch()
        s.synchronize()
        assert np.array_equal(yg.download(np.float32, rows * m), want), rep
        q.matmul(other, 200, rehip.MODE_BF16)             # eager work between replays
    g.destroy()
    s.destroy()
    q.close()


def test_noalloc_rejects_plans_beyond_the_scratch(monkeypatch):
    # 64 x 64 tiles with 19 K splits over 4000 rows: 19 * 4000 * 896 * 4 B of partials > 32 MiB
    monkeypatch.setenv("REHIP_GEMM_TILE", "1")
    monkeypatch.setenv("REHIP_GEMM_SPLITS", "19")
    t, m, n, rows = rehip.Q6_K, 896, 4864, 4000
    rng = np.random.default_rng(7900)
    q = rehip.QMat.from_bytes(t, synth.weight_bytes(rng, t, m, n), m, n)
    dx = hip.DeviceBuffer(rows * n * 4)
    dy = hip.DeviceBuffer(rows * m * 4)
    with pytest.raises(rehip.RehipError) as e:
        q.matmul_noalloc_dev(dx, rows, dy, rehip.MODE_BF16)
    assert e.value.code == rehip.RE_ERR_SIZE and "static scratch" in e.value.message
    q.close()


def test_noalloc_two_streams_without_host_sync():
    # two matrices whose split plans both use the scratch, called alternately on two streams with
    # no host synchronisation in between: each call waits for the other stream's previous call, so
    # every output equals the allocating entry point's
    t, m, n = rehip.Q6_K, 896, 4864
    rng = np.random.default_rng(8000)
    qa = rehip.QMat.from_bytes(t, synth.weight_bytes(rng, t, m, n), m, n)
    qb = rehip.QMat.from_bytes(t, synth.weight_bytes(rng, t, m, n), m, n)
    rows = (961, 512, 700, 961)
    xs = [hip.DeviceBuffer.from_array(synth.activations(rng, r, n)) for r in rows]
    ys = [hip.DeviceBuffer(r * m * 4) for r in rows]
    sa, sb = hip.Stream(), hip.Stream()
    for i, r in enumerate(rows):
        (qa if i % 2 == 0 else qb).matmul_noalloc_dev(xs[i], r, ys[i], rehip.MODE_BF16,
                                                      stream=sa if i % 2 == 0 else sb)
    sa.synchronize()
    sb.synchronize()
    for i, r in enumerate(rows):
        want = hip.DeviceBuffer(r * m * 4)
        (qa if i % 2 == 0 else qb).matmul_dev(xs[i], r, want, rehip.MODE_BF16)
        hip.synchronize()
        assert np.array_equal(ys[i].download(np.float32, r * m), want.download(np.float32, r * m)), i
    sa.destroy()
    sb.destroy()
    qa.close()
    qb.close()
