"""GEMV launch shapes against the oracle's GEMV (oracle.qmat_matvec, the reference's scalar
kernels kernel.rs:17-360 behind QMat::matvec qmat.rs:80-127), at the f32 bar
|y - y_oracle| <= 2^-10 * sum_k |w_rk x_k| per output.

Every test asserts the launch shape it meant to reach through re_qmat_gemv_plan, so a planner
change cannot silently move a case onto another kernel:
  * the headline launch of the benchmark: one batched tile-kernel launch (8 waves, half-block
    streaming) over a stack of >= 37 Q6_K 896 x 4864 matrices, distinct and shared x;
  * every tile-kernel instance (2 / 4 / 8 waves, whole- and half-block streaming) in all six
    quant types, single and stacked;
  * every row-group and wave variant, including K >= 4096;
  * the 151936 x 896 lm_head of the decode sweep in all six types.
"""
import numpy as np
import pytest

import oracle as O
import rehip
from rehip import hip, synth

pytestmark = pytest.mark.gpu
F32_TOL = 2.0 ** -10


def check_rows(t, w, m, n, x, got, label=""):
    want = O.qmat_matvec(t, w, m, n, x)
    absd = O.qmat_absdot(t, w, m, n, x, 1)
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= F32_TOL * absd), f"{label} max err/bound {np.max(err / (F32_TOL * absd + 1e-30))}"


def test_benchmark_launch_q6k_stack():
    """The benchmark's timed kernel: Q6_K 896 x 4864 (19 super-blocks per row), a stack large
    enough that the whole launch plans 64-row tiles (>= 512 tiles): gemv_tile_kernel with 8
    waves and half-block streaming, batch > 1."""
    t, m, n, count = rehip.Q6_K, 896, 4864, 40
    rng = np.random.default_rng(9001)
    ws = [synth.weight_bytes(rng, t, m, n) for _ in range(count)]
    st = rehip.QMat.from_bytes_stacked(t, np.concatenate(ws), m, n, count)
    assert st.gemv_plan(count) == {"kernel": "tile", "rows_per_group": 64, "waves": 8, "half": True}
    xs = synth.activations(rng, count, n).reshape(count, n)
    dx = hip.DeviceBuffer.from_array(xs)
    dy = hip.DeviceBuffer(count * m * 4)
    st.matvec_stacked_dev(0, count, dx, n, dy, m)            # distinct x per matrix
    hip.synchronize()
    got = dy.download(np.float32, count * m).reshape(count, m)
    for b in range(count):
        check_rows(t, ws[b], m, n, xs[b], got[b], f"distinct x, matrix {b}")
    st.matvec_stacked_dev(0, count, dx, 0, dy, m)            # one shared x (the benchmark's form)
    hip.synchronize()
    got = dy.download(np.float32, count * m).reshape(count, m)
    for b in range(count):
        check_rows(t, ws[b], m, n, xs[0], got[b], f"shared x, matrix {b}")
    again = hip.DeviceBuffer(count * m * 4)
    st.matvec_stacked_dev(0, count, dx, 0, again, m)
    hip.synchronize()
    assert np.array_equal(again.download(np.float32, count * m).reshape(count, m), got)   # deterministic
    st.close()


@pytest.mark.parametrize("t", rehip.QUANT_TYPES)
@pytest.mark.parametrize("waves", [2, 4, 8])
@pytest.mark.parametrize("n", [4864, 896, 512])
def test_tile_kernel_instances(t, waves, n, monkeypatch):
    """Forced 64-row tiles: every (type, waves, half) instance. For super-block types half-block
    streaming runs when a row has >= 2 * waves blocks: n = 4864 (19 blocks) always, n = 896
    (4 padded blocks) with 2 waves, n = 512 never. 150 rows: three tiles, the last partial."""
    monkeypatch.setenv("REHIP_GEMV_ROWS", "64")
    monkeypatch.setenv("REHIP_GEMV_WAVES", str(waves))
    m, count = 150, 3
    qk, _ = rehip.GEOM[t]
    kb = (n + qk - 1) // qk
    rng = np.random.default_rng(9100 + 7 * t + waves + n)
    ws = [synth.weight_bytes(rng, t, m, n) for _ in range(count)]
    q = rehip.QMat.from_bytes(t, ws[0], m, n)
    want_plan = {"kernel": "tile", "rows_per_group": 64, "waves": waves, "half": qk == 256 and kb >= 2 * waves}
    assert q.gemv_plan() == want_plan
    x = synth.activations(rng, count, n).reshape(count, n)
    got = q.matvec(x[0])
    check_rows(t, ws[0], m, n, x[0], got, "single")
    assert np.array_equal(q.matvec(x[0]), got)
    q.close()
    st = rehip.QMat.from_bytes_stacked(t, np.concatenate(ws), m, n, count)
    assert st.gemv_plan(count) == want_plan
    dx = hip.DeviceBuffer.from_array(x)
    dy = hip.DeviceBuffer(count * m * 4)
    st.matvec_stacked_dev(0, count, dx, n, dy, m)
    hip.synchronize()
    got = dy.download(np.float32, count * m).reshape(count, m)
    for b in range(count):
        check_rows(t, ws[b], m, n, x[b], got[b], f"stacked {b}")
    st.close()


@pytest.mark.parametrize("t", rehip.QUANT_TYPES)
@pytest.mark.parametrize("rows_per_group", [64, 16, 8, 4])
@pytest.mark.parametrize("waves", [2, 4, 8, 16])
@pytest.mark.parametrize("n", [2560, 4864])
def test_gemv_launch_shapes_all_types(t, rows_per_group, waves, n, monkeypatch):
    """Every row-group size and wave count on a ragged shape (3 tiles, the last partial), at a
    short and a long row. Row groups run 4 / 8 / 16 waves (a request for 2 runs 4); the tile
    kernel 2 / 4 / 8 (16 runs 8)."""
    monkeypatch.setenv("REHIP_GEMV_ROWS", str(rows_per_group))
    monkeypatch.setenv("REHIP_GEMV_WAVES", str(waves))
    m = 150
    rng = np.random.default_rng(9300 + 10 * t + rows_per_group + waves + n)
    w = synth.weight_bytes(rng, t, m, n)
    x = synth.activations(rng, 1, n)
    q = rehip.QMat.from_bytes(t, w, m, n)
    plan = q.gemv_plan()
    if rows_per_group == 64:
        assert plan["kernel"] == "tile" and plan["waves"] == min(waves, 8)
    else:
        assert plan["kernel"] == "rows" and plan["rows_per_group"] == rows_per_group
        assert plan["waves"] == max(waves, 4)
    got = q.matvec(x)
    check_rows(t, w, m, n, x, got)
    assert np.array_equal(q.matvec(x), got)
    q.close()


@pytest.mark.parametrize("t", rehip.QUANT_TYPES)
def test_lm_head_151936x896_all_types(t):
    """The decode sweep's lm_head in every type, as planned: 2374 tiles -> the tile kernel; the
    K-quants hold 4 padded super-blocks per row (2 waves, half blocks), the 32-blocks 28 blocks
    (7 steps of four: 4 waves)."""
    m, n = 151936, 896
    rng = np.random.default_rng(9500 + t)
    w = synth.weight_bytes(rng, t, m, n)
    x = synth.activations(rng, 1, n)
    q = rehip.QMat.from_bytes(t, w, m, n)
    qk, _ = rehip.GEOM[t]
    want_plan = ({"kernel": "tile", "rows_per_group": 64, "waves": 2, "half": True} if qk == 256 else
                 {"kernel": "tile", "rows_per_group": 64, "waves": 4, "half": False})
    assert q.gemv_plan() == want_plan
    check_rows(t, w, m, n, x, q.matvec(x))
    q.close()
