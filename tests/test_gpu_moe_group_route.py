"""Bias-corrected group routing on the device (re_moe_route_group_dev: route_group and
route_noaux_tc of moe.rs:126-268) and the layer that uses it (re_moe_layer_group_dev).

Bars: the expert ids equal the oracle's (oracle.route_group / route_noaux_tc, pinned on the CPU
by the reference's tests, the top_k_sigmoid reduction and a brute force) exactly, ties included;
weights to f32 rounding of expf (1e-6 relative, as the other device routers); slots past the
eligible experts hold id -1 and weight 0; the layer matches the oracle FFN on the oracle's routing
of the device's f32 logits (f32 1e-4, bf16 1e-2 relative to norm)."""
import numpy as np
import pytest

import oracle as O
import rehip
from rehip import hip, synth

pytestmark = pytest.mark.gpu
B = hip.DeviceBuffer
ROUTERS = {rehip.GATE_GROUP: O.route_group, rehip.GATE_NOAUX_TC: O.route_noaux_tc}


def down(buf, n, dtype=np.float32):
    hip.synchronize()
    return buf.download(dtype, n)


@pytest.mark.parametrize("gate", [rehip.GATE_GROUP, rehip.GATE_NOAUX_TC])
@pytest.mark.parametrize("T,E,k,ng,tkg,bias_len", [
    (64, 128, 8, 8, 4, 128),      # Qwen3-30B-A3B-like: 128 experts, top-8
    (33, 256, 8, 8, 4, 256),      # DeepSeek-V3-like: 256 experts in 8 groups, 4 eligible
    (17, 10, 4, 3, 1, 0),         # ragged groups (4, 3, 3): one group holds fewer than k experts
    (9, 64, 6, 1, None, 64),      # one group: every expert eligible
    (5, 1000, 16, 12, 5, 700),    # a short bias (entries past 700 count as 0), ragged groups
    (3, 8, 2, 2, 1, 0),           # the reference's own 8-expert, 2-group example (moe.rs:690-711)
])
def test_group_route_matches_oracle(gate, T, E, k, ng, tkg, bias_len):
    rng = np.random.default_rng(6000 + T + E + gate)
    # quantised logits: many equal scores, so ties inside and across groups are exercised
    logits = (np.round(rng.standard_normal((T, E)) * 2) / 2).astype(np.float32)
    if (E, ng) == (8, 2):
        logits[0] = [5.0, 2.0, -9.0, -9.0, 0.0, 0.0, 0.0, 0.0]
    bias = (np.round(rng.standard_normal(bias_len) * 4) / 8).astype(np.float32) if bias_len else None
    ids, w = B(T * k * 4), B(T * k * 4)
    rehip.moe_route_group_dev(B.from_array(logits), T, E, k, gate, B.from_array(bias) if bias is not None else None,
                              bias_len, ng, tkg, ids, w)
    gi = down(ids, T * k, np.int32).reshape(T, k)
    gw = down(w, T * k).reshape(T, k)
    for t in range(T):
        oi, ow = ROUTERS[gate](logits[t], bias, ng, k, tkg)
        n = len(oi)
        assert np.array_equal(gi[t, :n], np.asarray(oi, np.int32)), (t, gi[t], oi)
        np.testing.assert_allclose(gw[t, :n], ow, rtol=1e-6, atol=1e-7)
        assert np.all(gi[t, n:] == -1) and np.all(gw[t, n:] == 0.0), t
    if (E, ng) == (8, 2):
        assert gi[0, 0] == (0 if gate == rehip.GATE_NOAUX_TC else 4)
    if (E, ng, tkg) == (10, 3, 1):
        assert (gi == -1).any()           # some token's best group held only 3 experts


@pytest.mark.parametrize("T", [1, 32])
@pytest.mark.parametrize("gate", [rehip.GATE_GROUP, rehip.GATE_NOAUX_TC])
def test_moe_layer_group_qwen3_shape(T, gate):
    """Qwen3-30B-A3B-like layer with group routing (8 groups, 4 eligible, a per-expert bias):
    against the oracle router on the device's f32 logits and the oracle FFN."""
    E, hidden, inter, k, ng, tkg = 128, 2048, 768, 8, 8, 4
    rng = np.random.default_rng(6100 + T + gate)
    gate_b = np.concatenate([synth.weight_bytes(rng, rehip.Q4_K, inter, hidden) for _ in range(E)])
    up = np.concatenate([synth.weight_bytes(rng, rehip.Q4_K, inter, hidden) for _ in range(E)])
    down_ = np.concatenate([synth.weight_bytes(rng, rehip.Q6_K, hidden, inter) for _ in range(E)])
    x = synth.activations(rng, T, hidden)
    rw = (rng.standard_normal((E, hidden)) / np.sqrt(hidden)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.3).astype(np.float32)
    moe = rehip.MoeExperts(rehip.Q4_K, gate_b, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter)
    xd, rwd, bd = B.from_array(x), B.from_array(rw), B.from_array(bias)
    logits = B(T * E * 4)
    rehip.moe_router_logits_dev(xd, rwd, T, hidden, E, logits)
    lg = down(logits, T * E).reshape(T, E)
    ids = np.zeros((T, k), np.uint32)
    wts = np.zeros((T, k), np.float32)
    for t in range(T):
        ids[t], wts[t] = ROUTERS[gate](lg[t], bias, ng, k, tkg)
    want = O.moe_ffn(rehip.Q4_K, gate_b, rehip.Q4_K, up, rehip.Q6_K, down_, E, hidden, inter, x, T, k,
                     ids.reshape(-1), wts.reshape(-1))
    out = B(T * hidden * 4)
    for mode, tol in [(rehip.MODE_F32, 1e-4), (rehip.MODE_BF16, 1e-2)]:
        moe.layer_group_dev(xd, T, rwd, k, gate, bd, E, ng, tkg, out, mode)
        got = down(out, T * hidden)
        rel = np.linalg.norm(got - want) / np.linalg.norm(want)
        assert rel <= tol, (mode, rel)
    moe.close()


def test_group_route_rejects_bad_arguments():
    lg = B(4 * 8 * 4)
    ids, w = B(4 * 4), B(4 * 4)
    with pytest.raises(rehip.RehipError):
        rehip.moe_route_group_dev(lg, 1, 8, 2, rehip.GATE_SOFTMAX, None, 0, 2, 1, ids, w)   # not a group gate
    with pytest.raises(rehip.RehipError):
        rehip.moe_route_group_dev(lg, 1, 2000, 2, rehip.GATE_GROUP, None, 0, 2, 1, ids, w)  # > 1024 experts
