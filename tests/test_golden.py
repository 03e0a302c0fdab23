"""The committed fixtures (tests/golden/fixtures.npz, written by tests/golden/make_fixtures.py
from the oracle on the reference's deterministic fixture blocks, kernel.rs:2041-2078,
2369-2392, and seeded float matrices): the oracle must still reproduce them bit for bit (CPU),
and librehip must match them (GPU) -- dequant bit-exact, products within
2^-10 * sum_k |w_rk x_k| per output (bf16-mode GEMM: 1e-2 relative to norm)."""
import os

import numpy as np
import pytest

import oracle as O

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures.npz")
QUANT = (2, 6, 8, 12, 13, 14)
FLOAT = (0, 1, 30)
SHAPE = {t: (8, 512) for t in QUANT} | {t: (5, 96) for t in FLOAT}
ROWS = 3


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("t", QUANT + FLOAT)
def test_oracle_reproduces_fixtures(fx, t):
    m, n = SHAPE[t]
    w = fx[f"t{t}_w"]
    assert np.array_equal(O.dequant(t, w).view(np.uint32), fx[f"t{t}_deq"].view(np.uint32))
    assert np.array_equal(O.qmat_matvec(t, w, m, n, fx[f"t{t}_x"]).view(np.uint32), fx[f"t{t}_y"].view(np.uint32))
    ys = O.qmat_matmul(t, w, m, n, fx[f"t{t}_xs"], ROWS)
    assert np.array_equal(ys.view(np.uint32), fx[f"t{t}_ys"].view(np.uint32))


def _bound(deq, m, n, x):
    return np.abs(x.reshape(-1, n).astype(np.float64)) @ np.abs(deq.reshape(m, -1)[:, :n].astype(np.float64)).T


@pytest.mark.gpu
@pytest.mark.parametrize("t", QUANT + FLOAT)
def test_librehip_matches_fixtures(fx, t):
    import rehip
    m, n = SHAPE[t]
    w, deq = fx[f"t{t}_w"], fx[f"t{t}_deq"]
    assert np.array_equal(rehip.dequant(t, w).view(np.uint32), deq.view(np.uint32))
    q = rehip.QMat.from_bytes(t, w, m, n)
    x, xs = fx[f"t{t}_x"], fx[f"t{t}_xs"]
    y = q.matvec(x)
    assert np.all(np.abs(y - fx[f"t{t}_y"]) <= 2.0 ** -10 * _bound(deq, m, n, x).reshape(-1))
    ys = q.matmul(xs, ROWS, rehip.MODE_F32)
    assert np.all(np.abs(ys - fx[f"t{t}_ys"]) <= 2.0 ** -10 * _bound(deq, m, n, xs).reshape(-1))
    y16 = q.matmul(xs, ROWS, rehip.MODE_BF16)
    want = fx[f"t{t}_ys"].astype(np.float64)
    assert np.linalg.norm(y16 - want) / np.linalg.norm(want) <= 1e-2
    q.close()
