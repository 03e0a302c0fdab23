"""Device-resident transformer steps (librehip's re_*_dev layer entry points) against the host
restatements of the reference's steps (rehip.qwen: infer.rs:72-223, forward.rs:232-586), and the
device-resident decoder (one HIP graph per token) against the CPU-kernel decoder.

Tolerances: RMS-norm, RoPE, attention and the FFN pair are f32 with a different summation order
from numpy's, so they are compared at 2e-5 relative to the output scale (RoPE angles at
positions up to 2048 carry ~1e-4 rad of f32 rounding in both, hence 5e-4 there); argmax, the
embedding gather, the K/V append and the fused add are exact."""
import numpy as np
import pytest

import oracle as O
import rehip
from oracle.backend import CpuBackend
from rehip import hip, qwen

pytestmark = pytest.mark.gpu

B = hip.DeviceBuffer


def dev_i32(a):
    return B.from_array(np.asarray(a, np.int32))


def down(buf, n, dtype=np.float32):
    hip.synchronize()
    return buf.download(dtype, n)


@pytest.mark.parametrize("rows,d", [(1, 896), (7, 896), (3, 100), (2, 4096)])
def test_rmsnorm(rows, d):
    rng = np.random.default_rng(rows * 1000 + d)
    x = (rng.standard_normal((rows, d)) * 3).astype(np.float32)
    w = rng.standard_normal(d).astype(np.float32)
    out = B(rows * d * 4)
    rehip.rmsnorm_dev(B.from_array(x), B.from_array(w), rows, d, 1e-6, out)
    got = down(out, rows * d).reshape(rows, d)
    want = qwen.rmsnorm_rows(x, w, 1e-6)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5 * np.abs(want).max())


@pytest.mark.parametrize("rows,heads,hd,pos0,off", [(1, 14, 64, 0, 0), (1, 2, 64, 2047, 0), (9, 14, 64, 100, 3),
                                                    (4, 4, 128, 5, 0), (3, 1, 2, 0, 0)])
def test_rope(rows, heads, hd, pos0, off):
    rng = np.random.default_rng(heads * 7 + hd + pos0)
    x = rng.standard_normal((rows, heads * hd)).astype(np.float32)
    xb = B.from_array(x)
    rehip.rope_dev(xb, rows, heads, hd, 1e6, dev_i32([pos0]), off)
    got = down(xb, x.size).reshape(rows, -1)
    cos, sin = qwen.rope_table(rows, pos0 + off, hd, 1e6)
    want = qwen.rope_rows(x, heads, hd, cos, sin)
    np.testing.assert_allclose(got, want, rtol=0, atol=5e-4)


@pytest.mark.parametrize("hd,rows,base", [(64, 2048, 1e6), (128, 300, 1e4), (2, 5, 1e4)])
def test_rope_table(hd, rows, base):
    """re_rope_table_dev against the host (cos, sin) of the NeoX angles (forward.rs rope tables),
    interleaved per pair; its bits against the computed rotation are pinned by the decode
    attention test."""
    tab = B(rows * hd * 4)
    rehip.rope_table_dev(base, hd, rows, tab)
    got = down(tab, rows * hd).reshape(rows, hd // 2, 2)
    cos, sin = qwen.rope_table(rows, 0, hd, base)
    np.testing.assert_allclose(got[:, :, 0], cos, rtol=0, atol=5e-4)
    np.testing.assert_allclose(got[:, :, 1], sin, rtol=0, atol=5e-4)
    assert got[0, :, 0].tolist() == [1.0] * (hd // 2) and got[0, :, 1].tolist() == [0.0] * (hd // 2)


def test_kv_append_and_bounds():
    kv, max_seq = 128, 16
    rng = np.random.default_rng(3)
    kc, vc = B.from_array(np.zeros((max_seq, kv), np.float32)), B.from_array(np.zeros((max_seq, kv), np.float32))
    k = rng.standard_normal((5, kv)).astype(np.float32)
    v = rng.standard_normal((5, kv)).astype(np.float32)
    # rows 13..15 fit, rows 16 and 17 are past the cache and are dropped
    rehip.kv_append_dev(B.from_array(k), B.from_array(v), 5, kv, kc, vc, max_seq, dev_i32([13]))
    gk = down(kc, max_seq * kv).reshape(max_seq, kv)
    gv = down(vc, max_seq * kv).reshape(max_seq, kv)
    assert np.array_equal(gk[13:], k[:3]) and np.array_equal(gv[13:], v[:3])
    assert not gk[:13].any() and not gv[:13].any()


# rows < 8 take the per-(head, row) kernel; rows >= 8 with head_dim 64/128 the query-blocked one
# (block sizes: 4 rows for 7 heads per kv head, 32 rows for MHA, 1 row for 32 heads per kv head)
@pytest.mark.parametrize("rows,pos0,nh,nkv,hd", [(1, 0, 14, 2, 64), (1, 300, 14, 2, 64), (6, 0, 14, 2, 64),
                                                 (5, 40, 4, 4, 32), (3, 2000, 2, 1, 256), (33, 7, 8, 1, 128),
                                                 (8, 0, 14, 2, 64), (961, 0, 14, 2, 64), (100, 50, 8, 8, 128),
                                                 (37, 3, 32, 1, 64), (70, 10, 5, 5, 64), (9, 130, 6, 2, 64)])
def test_attention(rows, pos0, nh, nkv, hd):
    g = qwen.Geometry(d_model=nh * hd, n_heads=nh, n_kv_heads=nkv)
    max_seq = max(512, pos0 + rows + 3)
    rng = np.random.default_rng(rows + pos0 + nh)
    kvd = nkv * hd
    kc = np.zeros((max_seq, kvd), np.float32)
    vc = np.zeros((max_seq, kvd), np.float32)
    total = pos0 + rows
    kc[:total] = rng.standard_normal((total, kvd))
    vc[:total] = rng.standard_normal((total, kvd))
    q = (rng.standard_normal((rows, nh * hd)) * 2).astype(np.float32)
    want = qwen.attention(q, kc, vc, g, pos0)
    qd, kd, vd, pd = B.from_array(q), B.from_array(kc), B.from_array(vc), dev_i32([pos0])
    wb = rehip.attention_work_bytes(rows, nh, hd, max_seq)
    work = B.from_array(np.full(wb // 4, np.nan, np.float32))   # nothing unwritten may be read
    for use_work in (False, True):                  # few rows: one workgroup per row, or key splits
        ctx = B(rows * nh * hd * 4)
        rehip.attention_dev(qd, kd, vd, rows, nh, nkv, hd, max_seq, pd, ctx,
                            work=work if use_work else None, work_bytes=wb if use_work else 0)
        got = down(ctx, rows * nh * hd).reshape(rows, -1)
        np.testing.assert_allclose(got, want, rtol=0, atol=2e-5 * np.abs(want).max())
    with pytest.raises(rehip.RehipError):
        rehip.attention_dev(qd, kd, vd, rows, nh, nkv, hd, max_seq, pd, ctx, work=work, work_bytes=wb - 4)


def test_attention_split_skips_unwritten_cache_rows():
    """Cache rows past the visible position hold NaN: neither attention path may read them."""
    g = qwen.Geometry(d_model=14 * 64, n_heads=14, n_kv_heads=2)
    max_seq, pos0 = 1000, 300
    rng = np.random.default_rng(12)
    kc = np.full((max_seq, 128), np.nan, np.float32)
    vc = np.full((max_seq, 128), np.nan, np.float32)
    kc[:pos0 + 9] = rng.standard_normal((pos0 + 9, 128))
    vc[:pos0 + 9] = rng.standard_normal((pos0 + 9, 128))
    for rows in (1, 9):
        q = rng.standard_normal((rows, 14 * 64)).astype(np.float32)
        want = qwen.attention(q, kc, vc, g, pos0)
        wb = rehip.attention_work_bytes(rows, 14, 64, max_seq)
        ctx = B(rows * 14 * 64 * 4)
        rehip.attention_dev(B.from_array(q), B.from_array(kc), B.from_array(vc), rows, 14, 2, 64, max_seq,
                            dev_i32([pos0]), ctx, work=B.from_array(np.full(wb // 4, np.nan, np.float32)),
                            work_bytes=wb)
        got = down(ctx, rows * 14 * 64).reshape(rows, -1)
        assert np.isfinite(got).all()
        np.testing.assert_allclose(got, want, rtol=0, atol=2e-5 * np.abs(want).max())


@pytest.mark.parametrize("rows,nh,nkv,hd,pos0,fused", [(1, 14, 2, 64, 37, True), (5, 14, 2, 64, 0, False),
                                                       (3, 4, 4, 128, 10, True), (2, 2, 1, 256, 7, False)])
def test_qkv_rope_append(rows, nh, nkv, hd, pos0, fused):
    rng = np.random.default_rng(rows * 31 + hd)
    d, kv = nh * hd, nkv * hd
    max_seq = pos0 + rows + 4
    qkv = rng.standard_normal((rows, d + 2 * kv)).astype(np.float32)
    bq, bk, bv = (rng.standard_normal(n).astype(np.float32) for n in (d, kv, kv))
    kc, vc, qo = B(max_seq * kv * 4), B(max_seq * kv * 4), B(rows * d * 4)
    kc.zero()
    vc.zero()
    if fused:
        src = B.from_array(qkv)
        from rehip.qwen import _Offset
        args = (src, d + 2 * kv, _Offset(src, 4 * d), d + 2 * kv, _Offset(src, 4 * (d + kv)), d + 2 * kv)
    else:
        args = (B.from_array(qkv[:, :d]), d, B.from_array(qkv[:, d:d + kv]), kv, B.from_array(qkv[:, d + kv:]), kv)
    rehip.qkv_rope_append_dev(*args, B.from_array(bq), B.from_array(bk), B.from_array(bv), rows, nh, nkv, hd, 1e6,
                              dev_i32([pos0]), qo, kc, vc, max_seq)
    cos, sin = qwen.rope_table(rows, pos0, hd, 1e6)
    want_q = qwen.rope_rows((qkv[:, :d] + bq).astype(np.float32), nh, hd, cos, sin)
    want_k = qwen.rope_rows((qkv[:, d:d + kv] + bk).astype(np.float32), nkv, hd, cos, sin)
    np.testing.assert_allclose(down(qo, rows * d).reshape(rows, d), want_q, rtol=0, atol=5e-4)
    gk = down(kc, max_seq * kv).reshape(max_seq, kv)
    gv = down(vc, max_seq * kv).reshape(max_seq, kv)
    np.testing.assert_allclose(gk[pos0:pos0 + rows], want_k, rtol=0, atol=5e-4)
    assert np.array_equal(gv[pos0:pos0 + rows], (qkv[:, d + kv:] + bv).astype(np.float32))
    assert not gk[:pos0].any() and not gv[pos0 + rows:].any()


def test_decode_advance():
    keys = np.zeros(8, np.uint64)
    keys[5] = (0xC0400000 << 32) | 1234                                     # key of (3.0, 1234)
    keys[2] = (0xC0000000 << 32) | 4321                                     # key of (2.0, 4321)
    best = B.from_array(keys)
    tok, pos, hist = dev_i32([0]), dev_i32([10]), dev_i32(np.full(16, -1))
    rehip.decode_advance_dev(best, tok, pos, 1, hist, 16)
    assert int(down(tok, 1, np.int32)[0]) == 1234 and int(down(pos, 1, np.int32)[0]) == 11
    assert not down(best, 8, np.uint64).any()
    assert down(hist, 16, np.int32)[11] == 1234
    before = down(hist, 16, np.int32)
    rehip.decode_advance_dev(best, tok, pos, 10, hist, 16)                  # past the history: not stored
    assert int(down(pos, 1, np.int32)[0]) == 21 and np.array_equal(down(hist, 16, np.int32), before)


def test_add_and_bias():
    rng = np.random.default_rng(9)
    a = rng.standard_normal(7 * 96).astype(np.float32)
    b = rng.standard_normal(96).astype(np.float32)
    out = B(a.nbytes)
    rehip.add_dev(B.from_array(a), B.from_array(b), a.size, b.size, out)
    assert np.array_equal(down(out, a.size), (a.reshape(7, 96) + b).reshape(-1))
    with pytest.raises(rehip.RehipError):
        rehip.add_dev(B.from_array(a), B.from_array(b), a.size, 97, out)


@pytest.mark.parametrize("n", [1, 5, 1000, 151936])
def test_argmax_last_of_ties(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) - 5).astype(np.float32)        # all negative
    if n > 4:
        top = np.float32(x.max() + 1)
        x[[1, n // 2, n - 2]] = top                              # ties: the last index wins
    idx = dev_i32([-7])
    rehip.argmax_dev(B.from_array(x), n, idx)
    assert int(down(idx, 1, np.int32)[0]) == qwen.argmax_last(x)


def test_embed_gather_and_out_of_range():
    rng = np.random.default_rng(4)
    table = rng.standard_normal((50, 96)).astype(np.float32)
    toks = np.array([3, 0, 49, 50, -1, 3], np.int32)
    out = B(toks.size * 96 * 4)
    rehip.embed_dev(B.from_array(table), 50, 96, dev_i32(toks), toks.size, out)
    got = down(out, toks.size * 96).reshape(toks.size, 96)
    assert np.array_equal(got[[0, 1, 2, 5]], table[[3, 0, 49, 3]])
    assert not got[3].any() and not got[4].any()


def test_pos_add():
    p = dev_i32([5])
    rehip.pos_add_dev(p, 3)
    rehip.pos_add_dev(p, 961)
    assert int(down(p, 1, np.int32)[0]) == 969


def small_scale_bytes(t, m, n, seed):
    """Random blocks of a legacy type with a small f16 scale (outputs stay O(1))."""
    r = np.random.default_rng(seed)
    bb = {rehip.Q4_0: 18, rehip.Q5_0: 22, rehip.Q8_0: 34}[t]
    w = r.integers(0, 256, m * rehip.row_bytes(t, n), dtype=np.uint8).reshape(m, -1)
    w[:, 0::bb] = 0x00
    w[:, 1::bb] = 0x24
    return w.reshape(-1)


@pytest.mark.parametrize("t,m,n", [(rehip.Q4_K, 896, 896), (rehip.Q6_K, 896, 4864), (rehip.Q8_0, 64, 14336),
                                   (rehip.Q4_0, 130, 512), (rehip.Q8_0, 151936 // 8, 896)])
def test_matvec_ex(t, m, n):
    """add: the plain GEMV's sum plus `add` exactly, also in place; norm: the GEMV of the
    RMS-normalised row; best: the last index of the largest output (also on ties)."""
    rng = np.random.default_rng(m + n)
    if t in (rehip.Q4_K, rehip.Q6_K):
        w = qwen.conditioned_weight_bytes(rng, t, m, n, 1.0 / np.sqrt(n))
    else:
        w = small_scale_bytes(t, m, n, m + n)
    rb = rehip.row_bytes(t, n)
    w = w.reshape(m, rb)
    w[[m // 3, m - 1]] = w[m // 5]                  # identical rows: identical outputs (a tie)
    w = w.reshape(-1)
    q = rehip.QMat.from_bytes(t, w, m, n)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    nw = rng.standard_normal(n).astype(np.float32)
    add = rng.standard_normal(m).astype(np.float32)
    xb, yb, ab, nb = B.from_array(x), B(m * 4), B.from_array(add), B.from_array(nw)
    q.matvec_dev(xb, yb)
    plain = down(yb, m)
    q.matvec_ex_dev(xb, yb, add=ab)
    assert np.array_equal(down(yb, m), plain + add)
    q.matvec_ex_dev(xb, ab, add=ab)                               # y aliases add
    assert np.array_equal(down(ab, m), plain + add)
    # norm in the prologue vs an explicit RMS-norm, then the same GEMV
    q.matvec_ex_dev(xb, yb, norm_w=nb, eps=1e-6)
    normed = qwen.rmsnorm_rows(x[None, :], nw, 1e-6)[0]
    q.matvec_dev(B.from_array(normed), ab)
    ref = down(ab, m)
    # both are f32 GEMVs of the same normalised row: each within 2^-10 * sum|w x| of the exact one
    bound = 2.0 ** -10 * O.qmat_absdot(t, w, m, n, normed, 1)
    assert np.all(np.abs(down(yb, m).astype(np.float64) - ref) <= 2 * bound)
    # argmax folded into the stores; make row m//5 (and its copies) the maximum
    best = B.from_array(np.zeros(8, np.uint64))
    bias = np.zeros(m, np.float32)
    bias[[m // 5, m // 3, m - 1]] = np.abs(plain).max() + 10
    q.matvec_ex_dev(xb, yb, add=B.from_array(bias), best=best)
    y = down(yb, m)
    key = int(down(best, 8, np.uint64).max())
    assert key & 0xffffffff == qwen.argmax_last(y) == m - 1
    best.upload(np.zeros(8, np.uint64))
    q.matvec_ex_dev(xb, yb, best=best)
    assert int(down(best, 8, np.uint64).max()) & 0xffffffff == qwen.argmax_last(down(yb, m))
    q.close()


@pytest.mark.parametrize("t,inter,hidden", [(rehip.Q4_K, 4864, 896), (rehip.Q8_0, 100, 256), (rehip.Q5_0, 48, 512)])
def test_ffn_pair(t, inter, hidden):
    rng = np.random.default_rng(inter)
    if t in (rehip.Q4_K, rehip.Q8_0):
        g = qwen.conditioned_weight_bytes(rng, t, inter, hidden, 1.0 / np.sqrt(hidden))
        u = qwen.conditioned_weight_bytes(rng, t, inter, hidden, 1.0 / np.sqrt(hidden))
    else:
        def small(seed):
            r = np.random.default_rng(seed)
            w = r.integers(0, 256, inter * rehip.row_bytes(t, hidden), dtype=np.uint8).reshape(inter, -1)
            w[:, 0::22] = 0x00
            w[:, 1::22] = 0x24
            return w.reshape(-1)
        g, u = small(1), small(2)
    G, U = rehip.QMat.from_bytes(t, g, inter, hidden), rehip.QMat.from_bytes(t, u, inter, hidden)
    f = rehip.Ffn(G, U)
    x = rng.standard_normal(hidden).astype(np.float32)
    h = B(inter * 4)
    f.forward_dev(B.from_array(x), h)
    got = down(h, inter)
    want = qwen.silu(G.matvec(x)) * U.matvec(x)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5 * np.abs(want).max())
    nw = rng.standard_normal(hidden).astype(np.float32)
    f.forward_dev(B.from_array(x), h, norm_w=B.from_array(nw), eps=1e-6)
    xn = qwen.rmsnorm_rows(x[None, :], nw, 1e-6)[0]
    want = qwen.silu(G.matvec(xn)) * U.matvec(xn)
    np.testing.assert_allclose(down(h, inter), want, rtol=0, atol=2e-5 * np.abs(want).max())
    f.close()
    G.close()
    U.close()


def cpu_tokens(mb, prompt, steps, backend=None):
    r = qwen.DenseRunner(mb, backend or CpuBackend())
    dec = qwen.DenseDecoder(r, len(prompt) + steps)
    logits = dec.prefill(prompt)
    first = logits.copy()
    toks = [qwen.argmax_last(logits)]
    for _ in range(steps - 1):
        toks.append(qwen.argmax_last(dec.step(toks[-1])))
    return toks, first


TINY = qwen.Geometry(d_model=256, n_heads=4, n_kv_heads=2, d_ff=512, rope_freq_base=1e4, rms_eps=1e-5)


def dense_model(seed, geom, n_layers, n_vocab):
    """Seeded random weights stored unquantized: F16 attention, BF16 gate/up, F32 down, embedding
    and lm_head (entries N(0, 1/K), embedding/output 0.1 N(0, 1))."""
    rng = np.random.default_rng(seed)

    def raw(t, m, n, std):
        w = (rng.standard_normal((m, n)) * std).astype(np.float32)
        if t == rehip.F32:
            return w.view(np.uint8).reshape(-1)
        if t == rehip.F16:
            return w.astype(np.float16).view(np.uint8).reshape(-1)
        return (w.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(-1)
    d, kv, ff = geom.d_model, geom.n_kv_heads * geom.head_dim, geom.d_ff
    wd, wf = 1.0 / np.sqrt(d), 1.0 / np.sqrt(ff)
    A, F, D = rehip.F16, rehip.BF16, rehip.F32
    blocks = [qwen.BlockBytes(q=raw(A, d, d, wd), k=raw(A, kv, d, wd), v=raw(A, kv, d, wd), o=raw(A, d, d, wd),
                              gate=raw(F, ff, d, wd), up=raw(F, ff, d, wd), down=raw(D, d, ff, wf),
                              attn_norm=(1 + 0.1 * rng.standard_normal(d)).astype(np.float32),
                              ffn_norm=(1 + 0.1 * rng.standard_normal(d)).astype(np.float32),
                              q_bias=(0.1 * rng.standard_normal(d)).astype(np.float32),
                              k_bias=(0.1 * rng.standard_normal(kv)).astype(np.float32),
                              v_bias=(0.1 * rng.standard_normal(kv)).astype(np.float32))
              for _ in range(n_layers)]
    return qwen.ModelBytes(geom, n_vocab, raw(D, n_vocab, d, 0.1), raw(D, n_vocab, d, 0.1),
                           (1 + 0.1 * rng.standard_normal(d)).astype(np.float32), blocks,
                           attn_type=A, ffn_type=F, down_type=D, embed_type=D, output_type=D)


@pytest.mark.parametrize("use_graph", [False, True])
def test_device_decoder_dense_weights_match_cpu_path(use_graph):
    """Unquantized weights through the device-resident decoder (the dense GEMV with its norm and
    argmax, the dense gate/up pair, the dense MFMA GEMM in the f32 prefill) against the greedy
    tokens of the oracle's QMat (the CPU kernels cover the quantized types only)."""
    import test_qwen_gguf as T
    mb = dense_model(11, TINY, n_layers=3, n_vocab=1000)
    prompt = list(np.random.default_rng(12).integers(0, 1000, 40))      # 40 rows: the MFMA GEMM
    want, lg = cpu_tokens(mb, prompt, 20, T.OracleQMatBackend())          # the oracle's dense QMat
    dd = qwen.DeviceDecoder(mb, max_seq=80, prefill_rows=40, use_graph=use_graph)
    first = dd.prefill(prompt)
    np.testing.assert_allclose(dd.logits(), lg, rtol=0, atol=1e-4 * np.abs(lg).max())
    got = [first] + [dd.step() for _ in range(19)]
    dd.close()
    assert got == want


@pytest.mark.parametrize("use_graph", [False, True])
def test_device_decoder_tiny_matches_cpu_path(use_graph):
    mb = qwen.synth_model(7, TINY, n_layers=3, n_vocab=1000)
    prompt = [1, 2, 3, 5, 8, 13, 21, 34, 55, 89]
    want, lg = cpu_tokens(mb, prompt, 20)
    dd = qwen.DeviceDecoder(mb, max_seq=64, prefill_rows=16, use_graph=use_graph)
    first = dd.prefill(prompt)
    np.testing.assert_allclose(dd.logits(), lg, rtol=0, atol=1e-4 * np.abs(lg).max())
    got = [first] + [dd.step() for _ in range(19)]
    dd.close()
    assert got == want
    dd = qwen.DeviceDecoder(mb, max_seq=64, prefill_rows=16, use_graph=use_graph)
    assert dd.generate(prompt, 20) == want            # back-to-back replays, history read at the end
    dd.close()
    with pytest.raises(ValueError):
        qwen.DeviceDecoder(mb, max_seq=8, prefill_rows=16).prefill(prompt)


def test_device_decoder_qwen_shape_64_steps_match_cpu_path():
    """Qwen2.5-0.5B shape, Q4_K_M mix, 961-token prompt, 64 greedy tokens: the device-resident
    decoder (GPU attention/norms/RoPE/argmax, graph-replayed steps) against the CPU kernels."""
    mb = qwen.synth_model(501)
    prompt = np.random.default_rng(502).integers(0, mb.n_vocab, 961)
    want, lg = cpu_tokens(mb, prompt, 64)
    dd = qwen.DeviceDecoder(mb, max_seq=1040, prefill_rows=961)
    got = [dd.prefill(prompt)]
    assert np.max(np.abs(dd.logits() - lg)) <= 1e-3 * np.max(np.abs(lg))
    got += [dd.step() for _ in range(31)]
    dd.replay(32)
    got += dd.history(961 + 32, 32)
    dd.close()
    assert got == want, next(i for i, (a, b) in enumerate(zip(got, want)) if a != b)


@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("nh,nkv,hd,pos0,bias", [(14, 2, 64, 0, True), (14, 2, 64, 37, True), (14, 2, 64, 127, False),
                                                 (14, 2, 64, 128, True), (4, 4, 128, 300, True),
                                                 (2, 1, 256, 511, True), (14, 2, 64, 512, True),
                                                 (3, 1, 68, 77, True)])
def test_attention_decode_equals_epilogue_then_attention(nh, nkv, hd, pos0, bias, rope):
    """re_attention_decode_dev (q|k|v epilogue folded into the split attention) against
    re_qkv_rope_append_dev + re_attention_dev on the same raw projection row: identical context
    and caches, including the split boundary (position 128), the last cache row and a position
    past the cache (nothing stored, the old keys attended). With `rope` the decode reads its
    cosines and sines from re_rope_table_dev's table (rotation in registers), so the bit equality
    also pins the table against the computed rotation; a position past the table computes them,
    and head_dim 68 (not a multiple of 8) keeps the computing kernel."""
    max_seq = 512
    rng = np.random.default_rng(pos0 + nh)
    kvd = nkv * hd
    # rows not yet written hold NaN (a fresh cache is not cleared): no lane may fold them in
    kc0 = np.full((max_seq, kvd), np.nan, np.float32)
    vc0 = np.full((max_seq, kvd), np.nan, np.float32)
    n_old = min(pos0, max_seq)
    kc0[:n_old] = rng.standard_normal((n_old, kvd))
    vc0[:n_old] = rng.standard_normal((n_old, kvd))
    qkv = rng.standard_normal(nh * hd + 2 * kvd).astype(np.float32)
    bq = (0.1 * rng.standard_normal(nh * hd)).astype(np.float32) if bias else None
    bk = (0.1 * rng.standard_normal(kvd)).astype(np.float32) if bias else None
    bv = (0.1 * rng.standard_normal(kvd)).astype(np.float32) if bias else None
    dq = B.from_array(qkv)
    kd, vd = nh * hd * 4, (nh * hd + kvd) * 4
    bqd, bkd, bvd = [B.from_array(b) if b is not None else None for b in (bq, bk, bv)]
    pd = dev_i32([pos0])
    wb = rehip.attention_work_bytes(1, nh, hd, max_seq)
    theta = 10000.0
    # reference path: epilogue kernel, then attention
    kc_a, vc_a = B.from_array(kc0), B.from_array(vc0)
    qb, ctx_a = B(nh * hd * 4), B(nh * hd * 4)
    ld = nh * hd + 2 * kvd
    rehip.qkv_rope_append_dev(dq, ld, qwen._Offset(dq, kd), ld, qwen._Offset(dq, vd), ld, bqd, bkd, bvd, 1, nh, nkv, hd, theta, pd,
                              qb, kc_a, vc_a, max_seq)
    rehip.attention_dev(qb, kc_a, vc_a, 1, nh, nkv, hd, max_seq, pd, ctx_a,
                        work=B.from_array(np.full(wb // 4, np.nan, np.float32)), work_bytes=wb)
    # folded path
    kc_b, vc_b = B.from_array(kc0), B.from_array(vc0)
    ctx_b = B(nh * hd * 4)
    tab = None
    if rope:
        tab = B(max_seq * hd * 4)
        rehip.rope_table_dev(theta, hd, max_seq, tab)
    rehip.attention_decode_dev(dq, qwen._Offset(dq, kd), qwen._Offset(dq, vd), bqd, bkd, bvd, nh, nkv, hd, theta, pd, kc_b, vc_b,
                               max_seq, B.from_array(np.full(wb // 4, np.nan, np.float32)), wb, ctx_b, rope=tab)
    a, b = down(ctx_a, nh * hd), down(ctx_b, nh * hd)
    assert np.isfinite(b).all()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(down(kc_a, max_seq * kvd).view(np.uint32), down(kc_b, max_seq * kvd).view(np.uint32))
    assert np.array_equal(down(vc_a, max_seq * kvd).view(np.uint32), down(vc_b, max_seq * kvd).view(np.uint32))
