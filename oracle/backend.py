"""The CPU matmul backend for the dense decoder: the oracle's pooled AVX2 kernels (the
reference's QMat::matvec / matmul restated, oracle/baseline.c) behind the same
`make` / `dequant` interface as rehip.qwen.HipBackend.

TEST/BENCH INFRASTRUCTURE ONLY: the parity tests and bench.py's CPU leg use it; the product
never imports it."""
import numpy as np

import oracle as O


class CpuBackend:
    name = "cpu"

    def __init__(self, threads: int = 0):
        self.threads = threads

    @staticmethod
    def dequant(ggml_type, data):
        return O.dequant(ggml_type, data)

    def make(self, ggml_type, data, m, n):
        th = self.threads
        data = np.ascontiguousarray(data, dtype=np.uint8)

        class _M:
            def rows(self_):
                return m

            def cols(self_):
                return n

            def matvec(self_, x):
                return O.cpu_matvec(ggml_type, data, m, n, x, threads=th)

            def matmul(self_, x, rows):
                return O.cpu_matmul(ggml_type, data, m, n, x, rows, threads=th)

        return _M()
