"""Writes tests/golden/fixtures.npz: restatement-generated vectors (the CPU oracle, not the
reference binary, which cannot be built here) on the reference's own deterministic fixture
blocks (kernel.rs:2041-2078, 2369-2392 generators, as tests/blockpack.py restates them) and on
seeded float matrices.

Per quant type: W (m = 8 rows x n = 512 of fixture blocks), its dequant (quant.rs:363-453),
x[n] with x_k = ((k * 7) % 23 - 11) / 16, the QMat matvec (qmat.rs:80) and a 3-row matmul
(qmat.rs:169) of X_rk = ((r * 5 + k * 3) % 19 - 9) / 8. Per float type (F32 / F16 / BF16): a
seeded 5 x 96 matrix, its dequant and the same products. Run from the repo root:
python tests/golden/make_fixtures.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

import oracle as O  # noqa: E402
from blockpack import k_blocks, q4_blocks, q5_blocks, q8_blocks  # noqa: E402

M, N, ROWS = 8, 512, 3


def fixture_weights(t: int) -> np.ndarray:
    nb32, nb256 = M * N // 32, M * N // 256
    raw = {2: q4_blocks(nb32), 6: q5_blocks(nb32), 8: q8_blocks(nb32), 12: k_blocks(0, nb256),
           13: k_blocks(1, nb256), 14: k_blocks(2, nb256)}[t]
    return np.frombuffer(raw, np.uint8).copy()


def inputs(n: int):
    k = np.arange(n)
    x = (((k * 7) % 23) - 11).astype(np.float32) / 16
    r = np.arange(ROWS)[:, None]
    xs = ((((r * 5 + k[None, :] * 3) % 19) - 9).astype(np.float32) / 8)
    return x, xs


def main() -> None:
    out = {}
    for t in (2, 6, 8, 12, 13, 14):
        w = fixture_weights(t)
        x, xs = inputs(N)
        out[f"t{t}_w"] = w
        out[f"t{t}_deq"] = O.dequant(t, w)
        out[f"t{t}_x"] = x
        out[f"t{t}_y"] = O.qmat_matvec(t, w, M, N, x)
        out[f"t{t}_xs"] = xs
        out[f"t{t}_ys"] = O.qmat_matmul(t, w, M, N, xs, ROWS)
    rng = np.random.default_rng(2024)
    m, n = 5, 96
    w32 = rng.standard_normal((m, n)).astype(np.float32)
    raws = {0: w32.view(np.uint8).reshape(-1), 1: w32.astype(np.float16).view(np.uint8).reshape(-1),
            30: (w32.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(-1)}
    for t, w in raws.items():
        x, xs = inputs(n)
        out[f"t{t}_w"] = w
        out[f"t{t}_deq"] = O.dequant(t, w)
        out[f"t{t}_x"] = x
        out[f"t{t}_y"] = O.qmat_matvec(t, w, m, n, x)
        out[f"t{t}_xs"] = xs
        out[f"t{t}_ys"] = O.qmat_matmul(t, w, m, n, xs, ROWS)
    np.savez_compressed(os.path.join(HERE, "fixtures.npz"), **out)


if __name__ == "__main__":
    main()
