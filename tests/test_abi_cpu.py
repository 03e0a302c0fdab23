"""CPU-side checks of the C ABI library: it loads, exports exactly what include/rehip.h declares,
validates arguments before touching a GPU, and its host repack produces the documented tiled
layout. No compute call is made here."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import oracle as O
import rehip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def L():
    return rehip.lib()


def test_header_declares_exactly_the_exports(L):
    hdr = open(os.path.join(ROOT, "include", "rehip.h")).read()
    declared = set(re.findall(r"\b(re_[a-z_0-9]+)\s*\(", hdr))
    assert declared == set(rehip.EXPORTS)
    for name in declared:
        assert hasattr(L, name), name


def test_version_and_geometry(L):
    assert "gfx950" in rehip.version()
    for t, (qk, bb) in rehip.GEOM.items():
        assert rehip.row_bytes(t, 4864) == (4864 + qk - 1) // qk * bb
        assert rehip.row_bytes(t, 896) == O.qmat_row_bytes(t, 896)
    # 64-row tiles: 896 rows = 14 tiles; Q6_K 4864 = 19 super-blocks
    assert rehip.tiled_bytes(rehip.Q6_K, 896, 4864) == 14 * 19 * 64 * 210
    assert rehip.tiled_bytes(rehip.Q4_0, 5, 64) == 1 * 2 * 64 * 18


def test_argument_errors_need_no_gpu(L):
    h = C.c_void_p()
    buf = np.zeros(1000, np.uint8)
    assert L.re_qmat_create(99, buf.ctypes.data, 34, 1, 32, C.byref(h)) == rehip.RE_ERR_TYPE
    assert b"99" in L.re_last_error()
    assert L.re_qmat_create(rehip.Q8_0, buf.ctypes.data, 33, 1, 32, C.byref(h)) == rehip.RE_ERR_SIZE
    assert L.re_qmat_create(rehip.Q8_0, buf.ctypes.data, 34, 1, 48, C.byref(h)) == rehip.RE_ERR_SIZE
    assert L.re_qmat_create(rehip.Q8_0, None, 34, 1, 32, C.byref(h)) == rehip.RE_ERR_ARG
    out = np.zeros(64, np.float32)
    assert L.re_dequant(rehip.Q4_0, buf.ctypes.data, 17, out.ctypes.data, 0) == rehip.RE_ERR_SIZE
    assert L.re_last_error().decode() == "Q4_0 data len 17 not a multiple of 18"
    assert L.re_dequant(99, buf.ctypes.data, 8, out.ctypes.data, 0) == rehip.RE_ERR_TYPE
    assert L.re_last_error().decode() == "no scalar dequant for ggml type 99"


PLANES = {  # (offset, width) of each plane inside a block, in slab order
    rehip.Q4_0: [(2, 16), (0, 2)],
    rehip.Q5_0: [(6, 16), (2, 4), (0, 2)],
    rehip.Q8_0: [(2, 16), (18, 16), (0, 2)],
    rehip.Q4_K: [(16 * i, 16) for i in range(9)],
    rehip.Q5_K: [(16 * i, 16) for i in range(11)],
    rehip.Q6_K: [(16 * i, 16) for i in range(13)] + [(208, 2)],
}


@pytest.mark.parametrize("t", rehip.QUANT_TYPES)
@pytest.mark.parametrize("m,n", [(1, 256), (70, 512), (130, 896)])
def test_repack_is_the_documented_permutation(t, m, n):
    qk, bb = rehip.GEOM[t]
    kb = (n + qk - 1) // qk
    rng = np.random.default_rng(m + n + t)
    src = rng.integers(0, 256, m * kb * bb, dtype=np.uint8)
    out = rehip.repack(t, src, m, n)
    tiles = (m + 63) // 64
    assert out.size == tiles * kb * 64 * bb
    blocks = src.reshape(m, kb, bb)
    planes = PLANES[t]
    assert sum(w for _, w in planes) == bb
    for tile in range(tiles):
        for k in range(kb):
            slab = out[(tile * kb + k) * 64 * bb:(tile * kb + k + 1) * 64 * bb]
            base = 0
            for off, w in planes:
                plane = slab[base:base + 64 * w].reshape(64, w)
                rows = min(64, m - 64 * tile)
                assert np.array_equal(plane[:rows], blocks[64 * tile:64 * tile + rows, k, off:off + w])
                assert not plane[rows:].any()          # padding rows are zero
                base += 64 * w
    # a permutation plus zero padding: byte histogram matches
    assert np.array_equal(np.bincount(out, minlength=256)[1:], np.bincount(src, minlength=256)[1:])
