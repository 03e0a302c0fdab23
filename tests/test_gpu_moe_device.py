"""MoE layer with the routing on the device (row F3): router logits, top-k routing and the
expert grouping run as kernels, so a layer needs no host round trip.

Bars: the chosen expert ids equal the oracle router's (moe.rs:75-118, restated in the oracle)
exactly, including ties (lower index first); routing weights agree to f32 rounding of expf
(parity of libm exp is unpinned: 1e-6 relative); the device-routed expert FFN equals the
host-routed one (re_moe_forward_dev) bit for bit when both take the same path, and the full
layer matches the oracle's f64-free restatement within the MoE bars (f32 1e-4, bf16 1e-2
relative to norm)."""
import numpy as np
import pytest

import oracle as O
import rehip
from rehip import hip, synth

pytestmark = pytest.mark.gpu
B = hip.DeviceBuffer


def down(buf, n, dtype=np.float32):
    hip.synchronize()
    return buf.download(dtype, n)


@pytest.mark.parametrize("T,E,k", [(1, 128, 8), (37, 128, 8), (5, 16, 4), (3, 1000, 16), (2, 8, 8)])
@pytest.mark.parametrize("gate", [rehip.GATE_SOFTMAX, rehip.GATE_SIGMOID])
def test_route_matches_oracle_router(T, E, k, gate):
    rng = np.random.default_rng(T * 31 + E + gate)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[0, 3] = logits[0, 7] = logits[0].max() + 1        # a tie at the top: index 3 first
    if T > 1:
        logits[1, :] = 0.25                                  # all equal: experts 0..k-1 in order
    ids, w = B(T * k * 4), B(T * k * 4)
    rehip.moe_route_dev(B.from_array(logits), T, E, k, gate, ids, w)
    gi = down(ids, T * k, np.int32).reshape(T, k)
    gw = down(w, T * k).reshape(T, k)
    for t in range(T):
        oi, ow = (O.top_k if gate == rehip.GATE_SOFTMAX else O.top_k_sigmoid)(logits[t], k)
        assert np.array_equal(gi[t], np.asarray(oi, np.int32)), t
        np.testing.assert_allclose(gw[t], ow, rtol=1e-6, atol=1e-7)
    assert list(gi[0, :2]) == [3, 7]


@pytest.mark.parametrize("T,H,E", [(7, 2048, 128), (37, 2048, 61), (512, 1024, 128), (9, 2046, 20)])
def test_router_logits_matvec(T, H, E):
    # the tiled kernel (one and eight tokens per workgroup, a partial expert group) and the
    # per-expert kernel (rows not a whole number of float4)
    rng = np.random.default_rng(3 + T)
    x = rng.standard_normal((T, H)).astype(np.float32)
    w = (rng.standard_normal((E, H)) / 45).astype(np.float32)
    out = B(T * E * 4)
    rehip.moe_router_logits_dev(B.from_array(x), B.from_array(w), T, H, E, out)
    got = down(out, T * E).reshape(T, E)
    want = x.astype(np.float64) @ w.astype(np.float64).T
    bound = 2.0 ** -20 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T)
    assert np.all(np.abs(got - want) <= bound)


def moe_case(seed, E, hidden, inter, T, k, gt=rehip.Q4_K, dt=rehip.Q6_K):
    rng = np.random.default_rng(seed)
    gate = np.concatenate([synth.weight_bytes(rng, gt, inter, hidden) for _ in range(E)])
    up = np.concatenate([synth.weight_bytes(rng, gt, inter, hidden) for _ in range(E)])
    down_ = np.concatenate([synth.weight_bytes(rng, dt, hidden, inter) for _ in range(E)])
    x = synth.activations(rng, T, hidden)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    return gate, up, down_, x, logits


@pytest.mark.parametrize("T,E,k,gt,dt", [(64, 16, 4, rehip.Q4_K, rehip.Q6_K), (300, 32, 4, rehip.Q4_K, rehip.Q6_K),
                                         (200, 8, 2, rehip.Q8_0, rehip.Q5_0)])
def test_grouped_gemm_bf16_activations_bit_identical(T, E, k, gt, dt, monkeypatch):
    """bf16 mode of the grouped expert GEMMs: activation rows rounded to bf16 up front and h
    written as bf16 by SwiGLU (REHIP_MOE_XB=1, the default), with gate and up as two launches
    or as one fused launch (REHIP_MOE_PAIR), give the same bits as rounding each tile while
    staging it (REHIP_MOE_XB=0), host- and device-routed."""
    hidden, inter = 512, 256
    gate, up, down_, x, logits = moe_case(950 + T + E, E, hidden, inter, T, k, gt, dt)
    ids = np.zeros((T, k), np.int32)
    wts = np.zeros((T, k), np.float32)
    for t in range(T):
        ids[t], wts[t] = O.top_k(logits[t], k)
    moe = rehip.MoeExperts(gt, gate, gt, up, dt, down_, E, hidden, inter)
    xd = B.from_array(x)
    idd, wd = B.from_array(ids.reshape(-1)), B.from_array(wts.reshape(-1))
    res = {}
    # f32 rows staged per tile; bf16 rows with gate and up apart; bf16 rows with the fused pair
    monkeypatch.setenv("REHIP_MOE_QMMA", "0")       # the LDS-staged grouped GEMMs
    for xb, pair in (("0", "0"), ("1", "0"), ("1", "1")):
        monkeypatch.setenv("REHIP_MOE_XB", xb)
        monkeypatch.setenv("REHIP_MOE_PAIR", pair)
        out = B(T * hidden * 4)
        moe.forward_routed_dev(xd, T, k, idd, wd, out, rehip.MODE_BF16)
        res[xb + pair] = (down(out, T * hidden),
                          moe.forward(x, T, k, ids.reshape(-1).astype(np.uint32), wts.reshape(-1), rehip.MODE_BF16))
    for key in ("10", "11"):
        assert np.array_equal(res["00"][0], res[key][0]), key
        assert np.array_equal(res["00"][1], res[key][1]), key
    res["1"] = res["11"]
    want = O.moe_ffn(gt, gate, gt, up, dt, down_, E, hidden, inter, x, T, k,
                     ids.reshape(-1).astype(np.uint32), wts.reshape(-1))
    assert np.linalg.norm(res["1"][1] - want) / np.linalg.norm(want) <= 1e-2
    moe.close()


@pytest.mark.parametrize("T,E,k", [(1, 16, 4), (5, 16, 4), (40, 16, 4), (3, 128, 8), (300, 32, 4)])
def test_forward_routed_equals_host_routed(T, E, k, monkeypatch):
    """Device grouping/tasks vs the host planner (REHIP_MOE_HOST_GROUP=1: the host-routed call
    groups on the host instead of handing its ids to the device planner): the same kernels over
    the same rows, so the outputs are identical whenever both pick the same path (GEMV for few
    rows per expert, grouped GEMM otherwise)."""
    monkeypatch.setenv("REHIP_MOE_HOST_GROUP", "1")
    hidden, inter = 512, 256
    gate, up, down_, x, logits = moe_case(900 + T + E, E, hidden, inter, T, k)
    ids = np.zeros((T, k), np.int32)
    wts = np.zeros((T, k), np.float32)
    for t in range(T):
        ids[t], wts[t] = O.top_k(logits[t], k)
    moe = rehip.MoeExperts(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter)
    xd = B.from_array(x)
    idd, wd = B.from_array(ids.reshape(-1)), B.from_array(wts.reshape(-1))
    pairs = T * k
    touched = len(set(ids.reshape(-1).tolist()))
    same_path = (pairs <= 4 * touched) == (pairs <= 2 * E)
    want_oracle = O.moe_ffn(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter, x, T, k,
                            ids.reshape(-1).astype(np.uint32), wts.reshape(-1))
    for mode, tol in [(rehip.MODE_F32, 1e-4), (rehip.MODE_BF16, 1e-2)]:
        out = B(T * hidden * 4)
        moe.forward_routed_dev(xd, T, k, idd, wd, out, mode)
        got = down(out, T * hidden)
        host = moe.forward(x, T, k, ids.reshape(-1).astype(np.uint32), wts.reshape(-1), mode)
        if same_path:
            assert np.array_equal(got, host), mode
        rel = np.linalg.norm(got - want_oracle) / np.linalg.norm(want_oracle)
        assert rel <= tol, (mode, rel)
    moe.close()


@pytest.mark.parametrize("T,E,k", [(1023, 520, 8), (1024, 520, 8), (257, 1, 1), (96, 3, 2)])
def test_device_planner_extremes(T, E, k, monkeypatch):
    """The device planner at its limits: 8184 and 8192 (token, expert) pairs (every wave's
    segment full, ten-bit expert ids), one expert, and a pair count that is not a multiple of 64.
    Device-routed equals host-routed with the host planner (REHIP_MOE_HOST_GROUP=1) bit for bit
    (both take the grouped GEMM path here)."""
    monkeypatch.setenv("REHIP_MOE_HOST_GROUP", "1")
    hidden, inter = 256, 256
    gate, up, down_, x, logits = moe_case(7000 + T + E, E, hidden, inter, T, k)
    ids = np.argsort(-logits, axis=1, kind="stable")[:, :k].astype(np.int32)
    wts = np.random.default_rng(T).uniform(0.1, 1.0, (T, k)).astype(np.float32)
    moe = rehip.MoeExperts(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter)
    xd, idd, wd = B.from_array(x), B.from_array(ids.reshape(-1)), B.from_array(wts.reshape(-1))
    for mode in (rehip.MODE_F32, rehip.MODE_BF16):
        out = B(T * hidden * 4)
        moe.forward_routed_dev(xd, T, k, idd, wd, out, mode)
        got = down(out, T * hidden)
        host = moe.forward(x, T, k, ids.reshape(-1).astype(np.uint32), wts.reshape(-1), mode)
        assert np.array_equal(got, host), mode
    moe.close()


@pytest.mark.parametrize("T,E,k,hidden,inter", [(32, 128, 8, 2048, 768), (5, 16, 4, 512, 256), (300, 32, 4, 512, 256),
                                                (2, 8, 8, 256, 256)])
def test_host_routed_hands_ids_to_device_planner(T, E, k, hidden, inter):
    """A host-routed call of up to 2048 (token, expert) pairs uploads its ids and weights and runs
    the device-routed launches: bit for bit the device-routed result, over repeated calls (the
    pinned staging reused), in both modes; and within tolerance of the oracle."""
    gate, up, down_, x, logits = moe_case(3300 + T + E, E, hidden, inter, T, k)
    ids = np.argsort(-logits, axis=1, kind="stable")[:, :k].astype(np.int32)
    wts = np.random.default_rng(T + 5).uniform(0.1, 1.0, (T, k)).astype(np.float32)
    moe = rehip.MoeExperts(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter)
    xd, idd, wd = B.from_array(x), B.from_array(ids.reshape(-1)), B.from_array(wts.reshape(-1))
    want = O.moe_ffn(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter, x, T, k,
                     ids.reshape(-1).astype(np.uint32), wts.reshape(-1))
    for mode, tol in [(rehip.MODE_F32, 1e-4), (rehip.MODE_BF16, 1e-2)]:
        out = B(T * hidden * 4)
        moe.forward_routed_dev(xd, T, k, idd, wd, out, mode)
        routed = down(out, T * hidden)
        for _ in range(3):
            host = moe.forward(x, T, k, ids.reshape(-1).astype(np.uint32), wts.reshape(-1), mode)
            assert np.array_equal(host.view(np.uint32), routed.view(np.uint32)), mode
        rel = np.linalg.norm(host - want) / np.linalg.norm(want)
        assert rel <= tol, (mode, rel)
    moe.close()


def test_host_routed_large_batch_then_small():
    """More (token, expert) pairs than the device planner takes (8192), which only the host-routed
    call serves, then a small call on the same experts (staging buffers already grown); against
    the oracle (f32 1e-4, bf16 1e-2 relative to norm)."""
    E, hidden, inter, k = 16, 256, 256, 8
    for T in (1040, 7):
        gate, up, down_, x, logits = moe_case(5000 + T, E, hidden, inter, T, k)
        ids = np.zeros((T, k), np.uint32)
        wts = np.zeros((T, k), np.float32)
        for t in range(T):
            ids[t], wts[t] = O.top_k(logits[t], k)
        if T == 1040:
            moe = rehip.MoeExperts(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter)
            g0, u0, d0 = gate, up, down_
        want = O.moe_ffn(rehip.Q4_K, g0, rehip.Q4_K, u0, rehip.Q6_K, d0, E, hidden, inter, x, T, k,
                         ids.reshape(-1), wts.reshape(-1))
        for mode, tol in [(rehip.MODE_F32, 1e-4), (rehip.MODE_BF16, 1e-2)]:
            got = moe.forward(x, T, k, ids.reshape(-1), wts.reshape(-1), mode)
            rel = np.linalg.norm(got - want) / np.linalg.norm(want)
            assert rel <= tol, (T, mode, rel)
    moe.close()


@pytest.mark.parametrize("T,k,rows", [(3, 2, [[1, 9], [2, 3], [-1, 4]]), (1, 4, [[5, -1, 9, 2]]),
                                      (1, 8, [[7, 0, 8, 3, 3, -5, 1, 6]])])
def test_forward_routed_skips_out_of_range_ids(T, k, rows):
    """Pairs whose expert id is outside [0, n_experts) add nothing (the grouped path and the
    one-token path alike)."""
    E, hidden, inter = 8, 256, 128
    gate, up, down_, x, logits = moe_case(77, E, hidden, inter, T, k)
    ids = np.array(rows, np.int32)
    wts = np.full((T, k), 0.5, np.float32)
    moe = rehip.MoeExperts(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter)
    out = B(T * hidden * 4)
    moe.forward_routed_dev(B.from_array(x), T, k, B.from_array(ids.reshape(-1)), B.from_array(wts.reshape(-1)), out,
                           rehip.MODE_F32)
    got = down(out, T * hidden).reshape(T, hidden)
    # only the valid pairs: as if the invalid ones had weight 0 (routed to any expert)
    ids_ok = np.where((ids >= 0) & (ids < E), ids, 0).astype(np.uint32)
    w_ok = np.where((ids >= 0) & (ids < E), wts, 0.0).astype(np.float32)
    want = O.moe_ffn(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter, x, T, k,
                     ids_ok.reshape(-1), w_ok.reshape(-1)).reshape(T, hidden)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-4 * np.abs(want).max())
    moe.close()


@pytest.mark.parametrize("T,E,k", [(1, 32, 4), (5, 32, 8), (40, 16, 4), (129, 32, 8), (300, 64, 4)])
@pytest.mark.parametrize("gate", [rehip.GATE_SOFTMAX, rehip.GATE_SIGMOID])
def test_moe_layer_equals_route_then_forward(T, E, k, gate):
    """The layer entry point equals router logits -> route -> forward_routed run as separate
    calls, bit for bit."""
    hidden, inter = 512, 256
    gate_b, up, down_, x, _ = moe_case(5000 + T + E + gate, E, hidden, inter, T, k)
    rw = (np.random.default_rng(5100 + T).standard_normal((E, hidden)) / np.sqrt(hidden)).astype(np.float32)
    moe = rehip.MoeExperts(rehip.Q4_K, gate_b, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter)
    xd, rwd = B.from_array(x), B.from_array(rw)
    logits, ids, w = B(T * E * 4), B(T * k * 4), B(T * k * 4)
    for mode in (rehip.MODE_F32, rehip.MODE_BF16):
        a, b = B(T * hidden * 4), B(T * hidden * 4)
        moe.layer_dev(xd, T, rwd, k, gate, a, mode)
        rehip.moe_router_logits_dev(xd, rwd, T, hidden, E, logits)
        rehip.moe_route_dev(logits, T, E, k, gate, ids, w)
        moe.forward_routed_dev(xd, T, k, ids, w, b, mode)
        assert np.array_equal(down(a, T * hidden), down(b, T * hidden)), mode
    moe.close()


@pytest.mark.parametrize("T", [1, 32])
@pytest.mark.parametrize("gate", [rehip.GATE_SOFTMAX, rehip.GATE_SIGMOID])
def test_moe_layer_qwen3_shape(T, gate):
    """Qwen3-30B-A3B-like layer: hidden 2048, 128 experts, top-8, Q4_K gate/up, Q6_K down; the
    router weights are f32 (moe.rs:367). Against the oracle router on the same f32 logits and
    the oracle FFN."""
    E, hidden, inter, k = 128, 2048, 768, 8
    gate_b, up, down_, x, _ = moe_case(4000 + T, E, hidden, inter, T, k)
    rng = np.random.default_rng(4100 + T)
    rw = (rng.standard_normal((E, hidden)) / np.sqrt(hidden)).astype(np.float32)
    moe = rehip.MoeExperts(rehip.Q4_K, gate_b, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter)
    out = B(T * hidden * 4)
    xd, rwd = B.from_array(x), B.from_array(rw)
    logits = B(T * E * 4)
    rehip.moe_router_logits_dev(xd, rwd, T, hidden, E, logits)
    lg = down(logits, T * E).reshape(T, E)
    ids = np.zeros((T, k), np.uint32)
    wts = np.zeros((T, k), np.float32)
    for t in range(T):
        ids[t], wts[t] = (O.top_k if gate == rehip.GATE_SOFTMAX else O.top_k_sigmoid)(lg[t], k)
    want = O.moe_ffn(rehip.Q4_K, gate_b, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter, x, T, k,
                     ids.reshape(-1), wts.reshape(-1))
    for mode, tol in [(rehip.MODE_F32, 1e-4), (rehip.MODE_BF16, 1e-2)]:
        moe.layer_dev(xd, T, rwd, k, gate, out, mode)
        got = down(out, T * hidden)
        rel = np.linalg.norm(got - want) / np.linalg.norm(want)
        assert rel <= tol, (mode, rel)
    moe.close()


def test_moe_qwen3_shape_t512_host_and_device_routed():
    """C4 at its largest batch: 512 tokens x top-8 = 4096 (token, expert) pairs over 128
    experts (grouped GEMM tasks, the fused bf16 gate/up pair, the device plan). Device routing
    picks the oracle router's experts exactly; host-routed and device-routed FFNs both match the
    oracle (f32 1e-4, bf16 1e-2 relative to norm)."""
    E, hidden, inter, k, T = 128, 2048, 768, 8, 512
    gate_b, up, down_, x, _ = moe_case(4512, E, hidden, inter, T, k)
    rng = np.random.default_rng(4612)
    rw = (rng.standard_normal((E, hidden)) / np.sqrt(hidden)).astype(np.float32)
    moe = rehip.MoeExperts(rehip.Q4_K, gate_b, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter)
    xd, rwd = B.from_array(x), B.from_array(rw)
    logits, dids, dw = B(T * E * 4), B(T * k * 4), B(T * k * 4)
    rehip.moe_router_logits_dev(xd, rwd, T, hidden, E, logits)
    lg = down(logits, T * E).reshape(T, E)
    ids = np.zeros((T, k), np.uint32)
    wts = np.zeros((T, k), np.float32)
    for t in range(T):
        ids[t], wts[t] = O.top_k(lg[t], k)
    rehip.moe_route_dev(logits, T, E, k, rehip.GATE_SOFTMAX, dids, dw)
    assert np.array_equal(down(dids, T * k, np.int32).reshape(T, k), ids.astype(np.int32))
    want = O.moe_ffn(rehip.Q4_K, gate_b, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter, x, T, k,
                     ids.reshape(-1), wts.reshape(-1))
    out = B(T * hidden * 4)
    for mode, tol in [(rehip.MODE_F32, 1e-4), (rehip.MODE_BF16, 1e-2)]:
        got = moe.forward(x, T, k, ids.reshape(-1), wts.reshape(-1), mode)
        rel = np.linalg.norm(got - want) / np.linalg.norm(want)
        assert rel <= tol, ("host-routed", mode, rel)
        moe.layer_dev(xd, T, rwd, k, rehip.GATE_SOFTMAX, out, mode)
        got = down(out, T * hidden)
        rel = np.linalg.norm(got - want) / np.linalg.norm(want)
        assert rel <= tol, ("device-routed", mode, rel)
    moe.close()


@pytest.mark.parametrize("T", [1, 5, 300])
def test_shared_expert_every_forward_path(T):
    """Shared expert (moe.rs:380-385): set on the experts, it is added after the routed sum by the
    host-routed, device-routed and whole-layer calls alike; against the oracle's routed sum plus
    shared FFN (f32 1e-4, bf16 1e-2 relative to norm), with its own width (inter 384 beside 256).
    Cleared, the calls give the routed sum alone again."""
    E, hidden, inter, sinter, k = 16, 512, 256, 384, 4
    gate_b, up, down_, x, _ = moe_case(5100 + T, E, hidden, inter, T, k)
    rng = np.random.default_rng(5200 + T)
    sg = synth.weight_bytes(rng, rehip.Q4_K, sinter, hidden)
    su = synth.weight_bytes(rng, rehip.Q4_K, sinter, hidden)
    sd = synth.weight_bytes(rng, rehip.Q8_0, hidden, sinter)
    rw = (rng.standard_normal((E, hidden)) / np.sqrt(hidden)).astype(np.float32)
    moe = rehip.MoeExperts(rehip.Q4_K, gate_b, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter)
    xd, rwd = B.from_array(x), B.from_array(rw)
    logits, dids, dw = B(T * E * 4), B(T * k * 4), B(T * k * 4)
    rehip.moe_router_logits_dev(xd, rwd, T, hidden, E, logits)
    lg = down(logits, T * E).reshape(T, E)
    ids = np.zeros((T, k), np.uint32)
    wts = np.zeros((T, k), np.float32)
    for t in range(T):
        ids[t], wts[t] = O.top_k(lg[t], k)
    rehip.moe_route_dev(logits, T, E, k, rehip.GATE_SOFTMAX, dids, dw)
    shared = (rehip.Q4_K, sg, rehip.Q4_K, su, rehip.Q8_0, sd, sinter)
    want = O.moe_ffn_shared(rehip.Q4_K, gate_b, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter, x, T, k,
                            ids.reshape(-1), wts.reshape(-1), shared)
    routed = O.moe_ffn(rehip.Q4_K, gate_b, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter, x, T, k,
                       ids.reshape(-1), wts.reshape(-1))
    moe.set_shared(*shared)
    out = B(T * hidden * 4)
    for mode, tol in [(rehip.MODE_F32, 1e-4), (rehip.MODE_BF16, 1e-2)]:
        got = {"host": moe.forward(x, T, k, ids.reshape(-1), wts.reshape(-1), mode)}
        moe.forward_routed_dev(xd, T, k, dids, dw, out, mode)
        got["routed"] = down(out, T * hidden)
        moe.layer_dev(xd, T, rwd, k, rehip.GATE_SOFTMAX, out, mode)
        got["layer"] = down(out, T * hidden)
        for name, g in got.items():
            rel = np.linalg.norm(g - want) / np.linalg.norm(want)
            assert rel <= tol, (name, mode, rel)
        assert np.array_equal(got["routed"], got["layer"]), mode
    moe.clear_shared()
    got = moe.forward(x, T, k, ids.reshape(-1), wts.reshape(-1), rehip.MODE_F32)
    assert np.linalg.norm(got - routed) / np.linalg.norm(routed) <= 1e-4
    moe.close()


QMMA_CASES = [(5, 16, 4, rehip.Q4_K, rehip.Q6_K), (40, 16, 4, rehip.Q4_K, rehip.Q6_K),
              (300, 32, 4, rehip.Q4_K, rehip.Q6_K), (64, 16, 2, rehip.Q5_K, rehip.Q5_K),
              (64, 16, 2, rehip.Q8_0, rehip.Q4_0), (70, 8, 2, rehip.Q5_0, rehip.Q8_0),
              (33, 4, 4, rehip.Q6_K, rehip.Q4_K)]


@pytest.mark.parametrize("T,E,k,gt,dt", QMMA_CASES)
def test_register_decoded_grouped_gemm(T, E, k, gt, dt, monkeypatch):
    """bf16 mode, more than one token: the grouped expert GEMMs with register-decoded weights
    (moe_qmma.hip), host- and device-routed, with 32-row chunks (few rows per expert) and 64-row
    chunks (ragged: 33, 40, 70 rows per expert and more), against the oracle at the bf16 bar. Where
    the path they replace is the LDS-staged grouped GEMM (many rows per expert), its operands are
    the same bf16 values, so the two agree to f32 summation order (1e-4 relative to norm: an
    ulp-level difference of a gate/up sum can flip the bf16 rounding of h); with few rows per
    expert the replaced path is the f32 expert GEMV."""
    hidden, inter = 512, 320
    gate, up, down_, x, logits = moe_case(990 + T + E + gt, E, hidden, inter, T, k, gt, dt)
    ids = np.zeros((T, k), np.int32)
    wts = np.zeros((T, k), np.float32)
    for t in range(T):
        ids[t], wts[t] = O.top_k(logits[t], k)
    moe = rehip.MoeExperts(gt, gate, gt, up, dt, down_, E, hidden, inter)
    xd = B.from_array(x)
    idd, wd = B.from_array(ids.reshape(-1)), B.from_array(wts.reshape(-1))
    res = {}
    for q in ("0", "1"):
        monkeypatch.setenv("REHIP_MOE_QMMA", q)
        out = B(T * hidden * 4)
        moe.forward_routed_dev(xd, T, k, idd, wd, out, rehip.MODE_BF16)
        res[q] = (moe.forward(x, T, k, ids.reshape(-1).astype(np.uint32), wts.reshape(-1), rehip.MODE_BF16),
                  down(out, T * hidden))
    want = O.moe_ffn(gt, gate, gt, up, dt, down_, E, hidden, inter, x, T, k,
                     ids.reshape(-1).astype(np.uint32), wts.reshape(-1))
    touched = len(np.unique(ids))
    many = {"host-routed": T * k > 4 * touched, "device-routed": T * k > 2 * E}
    for i, name in enumerate(("host-routed", "device-routed")):
        a, b = res["0"][i], res["1"][i]
        if many[name]:
            assert np.linalg.norm(b - a) / np.linalg.norm(a) <= 1e-4, name
        assert np.linalg.norm(b - want) / np.linalg.norm(want) <= 1e-2, name
    moe.close()



QMMA_FORCED_TYPES = [(rehip.Q4_K, rehip.Q6_K), (rehip.Q5_K, rehip.Q4_K), (rehip.Q6_K, rehip.Q5_K),
                     (rehip.Q4_0, rehip.Q8_0), (rehip.Q5_0, rehip.Q4_0), (rehip.Q8_0, rehip.Q5_0)]


@pytest.mark.parametrize("gt,dt", QMMA_FORCED_TYPES)
@pytest.mark.parametrize("ks,xl", [("2", None), ("2", "0"), ("1", "1")])
def test_qmma_forced_wave_split_and_staging(gt, dt, ks, xl, monkeypatch):
    """The register-decoded expert GEMMs with 64-row tasks (300 tokens over 16 experts; an
    expert's ragged last chunk runs the one-tile body) under the launch overrides: K split over
    two waves of a task (REHIP_QMMA_KS=2) with the down projection's activations staged in LDS
    (the stage copy runs four chunks ahead, two of a wave's groups for the 32-element block
    types), the same with staging off, and staging forced onto the gate/up pair. Host- and
    device-routed against the oracle at the bf16 bar."""
    T, E, k, hidden, inter = 300, 16, 4, 512, 320
    gate, up, down_, x, logits = moe_case(1234 + gt + 7 * dt, E, hidden, inter, T, k, gt, dt)
    ids = np.zeros((T, k), np.int32)
    wts = np.zeros((T, k), np.float32)
    for t in range(T):
        ids[t], wts[t] = O.top_k(logits[t], k)
    moe = rehip.MoeExperts(gt, gate, gt, up, dt, down_, E, hidden, inter)
    monkeypatch.setenv("REHIP_MOE_QMMA", "1")
    monkeypatch.setenv("REHIP_QMMA_KS", ks)
    if xl:
        monkeypatch.setenv("REHIP_QMMA_XL", xl)
    out = B(T * hidden * 4)
    moe.forward_routed_dev(B.from_array(x), T, k, B.from_array(ids.reshape(-1)), B.from_array(wts.reshape(-1)),
                           out, rehip.MODE_BF16)
    got = {"device-routed": down(out, T * hidden),
           "host-routed": moe.forward(x, T, k, ids.reshape(-1).astype(np.uint32), wts.reshape(-1), rehip.MODE_BF16)}
    want = O.moe_ffn(gt, gate, gt, up, dt, down_, E, hidden, inter, x, T, k,
                     ids.reshape(-1).astype(np.uint32), wts.reshape(-1))
    for name, g in got.items():
        assert np.linalg.norm(g - want) / np.linalg.norm(want) <= 1e-2, name
    moe.close()


@pytest.mark.parametrize("gt,dt", QMMA_FORCED_TYPES)
@pytest.mark.parametrize("T", [300, 40])
def test_qmma_half_tile_waves_bit_identical(gt, dt, T, monkeypatch):
    """Two 32-row waves per expert task sharing one LDS staging of the activation rows
    (REHIP_QMMA_H=1: lanes 0-31 of a wave decode one run of a chunk, lanes 32-63 the other; each
    wave copies half of every stage) give the same bits as whole-tile tasks with the same
    staging: every output sums the same MFMA products in the same order. 300 tokens over 16
    experts make 64-row tasks with ragged last chunks, 40 tokens 32-row ones; host- and
    device-routed, and against the oracle."""
    E, k, hidden, inter = 16, 4, 512, 320
    gate, up, down_, x, logits = moe_case(4321 + T + gt + 7 * dt, E, hidden, inter, T, k, gt, dt)
    ids = np.zeros((T, k), np.int32)
    wts = np.zeros((T, k), np.float32)
    for t in range(T):
        ids[t], wts[t] = O.top_k(logits[t], k)
    moe = rehip.MoeExperts(gt, gate, gt, up, dt, down_, E, hidden, inter)
    xd = B.from_array(x)
    idd, wd = B.from_array(ids.reshape(-1)), B.from_array(wts.reshape(-1))
    monkeypatch.setenv("REHIP_MOE_QMMA", "1")
    monkeypatch.setenv("REHIP_QMMA_KS", "1")
    monkeypatch.setenv("REHIP_QMMA_XL", "1")
    res = {}
    for h in ("0", "1"):
        monkeypatch.setenv("REHIP_QMMA_H", h)
        out = B(T * hidden * 4)
        moe.forward_routed_dev(xd, T, k, idd, wd, out, rehip.MODE_BF16)
        res[h] = (moe.forward(x, T, k, ids.reshape(-1).astype(np.uint32), wts.reshape(-1), rehip.MODE_BF16),
                  down(out, T * hidden))
    want = O.moe_ffn(gt, gate, gt, up, dt, down_, E, hidden, inter, x, T, k,
                     ids.reshape(-1).astype(np.uint32), wts.reshape(-1))
    for i, name in enumerate(("host-routed", "device-routed")):
        a, b = res["0"][i], res["1"][i]
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), name
        assert np.linalg.norm(b - want) / np.linalg.norm(want) <= 1e-2, name
    moe.close()
