"""Pins the oracle's router and expert FFN (src/moe.rs restatement).

The reference's own tests (moe.rs:624-801) are ported; its 2x2 f32 identity experts become
32x32 Q8_0 identity experts (d = 1, quant 1 on the diagonal), which dequantize exactly to the
identity, so the reference's closed forms (silu(1), 2*silu(1), ...) still apply. A brute-force
f64 evaluation of the whole layer pins the batched path on random experts.
"""
import math

import numpy as np

import oracle as O
from blockpack import pack_q8_0

EPS = 1e-5


def test_softmax_sums_to_one():
    assert abs(float(np.sum(O.softmax([1.0, 2.0, 3.0]))) - 1.0) < EPS


def test_top_k_picks_largest_and_renormalizes():
    ids, w = O.top_k([0.1, 0.9, 0.2, 0.8], 2)
    assert list(ids) == [1, 3] and abs(float(w.sum()) - 1.0) < EPS


def test_top_k_clamps_when_k_exceeds_experts():
    assert len(O.top_k([0.5, 0.4], 8)[0]) == 2
    assert len(O.top_k([], 2)[0]) == 0


def test_top_k_ties_keep_index_order():
    # Rust's sort_by is stable: equal scores keep ascending index order
    ids, w = O.top_k([1.0, 3.0, 3.0, 1.0, 3.0], 4)
    assert list(ids) == [1, 2, 4, 0]
    assert np.allclose(w[:3], w[0]) and w[3] < w[0]


def test_sigmoid_silu_basics():
    assert abs(O.sigmoid(0.0) - 0.5) < EPS
    assert O.sigmoid(10.0) > 0.999
    assert abs(O.silu(0.0)) < EPS
    assert abs(O.silu(1.0) - 1.0 / (1.0 + math.exp(-1.0))) < EPS


def test_sigmoid_router_renormalizes_to_one():
    ids, w = O.top_k_sigmoid([1.0, 5.0, 2.0, 4.0], 2)
    assert list(ids) == [1, 3] and abs(float(w.sum()) - 1.0) < EPS


def test_top_k_weights_are_softmax_of_chosen_logits():
    rng = np.random.default_rng(5)
    s = rng.standard_normal(128).astype(np.float32)
    ids, w = O.top_k(s, 8)
    order = np.argsort(-s.astype(np.float64), kind="stable")[:8]
    assert list(ids) == list(order)
    e = np.exp(s[order].astype(np.float64) - s[order].max())
    assert np.allclose(w, e / e.sum(), rtol=1e-6, atol=1e-7)


def q8_identity(scale_q: int, n: int = 32) -> bytes:
    """n x n Q8_0 matrix with d = 1 and quant `scale_q` on the diagonal."""
    rows = []
    for r in range(n):
        q = np.zeros(n, np.int64)
        q[r] = scale_q
        rows.append(b"".join(pack_q8_0(0x3C00, q[b * 32:(b + 1) * 32]) for b in range(n // 32)))
    return b"".join(rows)


def test_expert_ffn_pipeline_identity():
    # hidden = inter = 32, identity projections: out = silu(x) * x componentwise (moe.rs:768-776)
    e = q8_identity(1)
    x = np.zeros(32, np.float32)
    x[0] = 1.0
    out = O.moe_ffn(O.Q8_0, e, O.Q8_0, e, O.Q8_0, e, 1, 32, 32, x, 1, 1, [0], [1.0])
    assert abs(out[0] - O.silu(1.0)) < EPS and np.all(np.abs(out[1:]) < EPS)


def test_moe_layer_routes_to_best_expert():
    # expert1 has down = 2*I and wins the router: out = [2*silu(1), 0, ...] (moe.rs:784-796)
    ident, double = q8_identity(1), q8_identity(2)
    gate = ident + ident
    down = ident + double
    logits = np.array([0.0, 10.0], np.float32)      # router_w @ hidden, as in the reference test
    ids, w = O.top_k(logits, 1)
    assert list(ids) == [1] and w[0] == 1.0
    x = np.zeros(32, np.float32)
    x[0] = 1.0
    out = O.moe_ffn(O.Q8_0, gate, O.Q8_0, gate, O.Q8_0, down, 2, 32, 32, x, 1, 1, ids, w)
    assert abs(out[0] - 2.0 * O.silu(1.0)) < EPS and np.all(np.abs(out[1:]) < EPS)


def test_moe_layer_adds_shared_expert():
    # expert 0 wins (sigmoid top-1, weight 1) -> [silu(1), 0, ...]; the identity shared expert adds
    # its own FFN output -> [2*silu(1), 0, ...] (moe.rs:788-800)
    ident = q8_identity(1)
    two = ident + ident
    ids, w = O.top_k_sigmoid(np.array([10.0, 0.0], np.float32), 1)
    assert list(ids) == [0] and w[0] == 1.0
    x = np.zeros(32, np.float32)
    x[0] = 1.0
    out = O.moe_ffn_shared(O.Q8_0, two, O.Q8_0, two, O.Q8_0, two, 2, 32, 32, x, 1, 1, ids, w,
                           (O.Q8_0, ident, O.Q8_0, ident, O.Q8_0, ident, 32))
    assert abs(out[0] - 2.0 * O.silu(1.0)) < EPS and np.all(np.abs(out[1:]) < EPS)


def test_shared_expert_is_added_after_the_routed_sum():
    # combine (moe.rs:306-345): out = sum_j w_j routed_j, then + shared; the shared term is the
    # expert FFN of every token on its own, with its own width
    rng = np.random.default_rng(19)
    E, hidden, inter, sinter, T, k = 4, 64, 32, 96, 3, 2

    def rnd(m, n):
        raw = rng.integers(0, 256, (m * n // 32, 34), dtype=np.uint8)
        raw[:, 0:2] = (np.abs(rng.standard_normal(m * n // 32)) * 0.02).astype(np.float16).view(np.uint8).reshape(-1, 2)
        return raw.reshape(-1)

    gate, up = rnd(E * inter, hidden), rnd(E * inter, hidden)
    dn = rnd(E * hidden, inter)
    sg, su, sd = rnd(sinter, hidden), rnd(sinter, hidden), rnd(hidden, sinter)
    x = rng.standard_normal(T * hidden).astype(np.float32)
    ids = np.concatenate([rng.permutation(E)[:k] for _ in range(T)]).astype(np.uint32)
    w = rng.random(T * k).astype(np.float32)
    routed = O.moe_ffn(O.Q8_0, gate, O.Q8_0, up, O.Q8_0, dn, E, hidden, inter, x, T, k, ids, w)
    got = O.moe_ffn_shared(O.Q8_0, gate, O.Q8_0, up, O.Q8_0, dn, E, hidden, inter, x, T, k, ids, w,
                           (O.Q8_0, sg, O.Q8_0, su, O.Q8_0, sd, sinter))
    SG = O.dequant(O.Q8_0, sg).reshape(sinter, hidden).astype(np.float64)
    SU = O.dequant(O.Q8_0, su).reshape(sinter, hidden).astype(np.float64)
    SD = O.dequant(O.Q8_0, sd).reshape(hidden, sinter).astype(np.float64)
    for t in range(T):
        xt = x[t * hidden:(t + 1) * hidden].astype(np.float64)
        g, u = SG @ xt, SU @ xt
        want = SD @ (g / (1.0 + np.exp(-g)) * u) + routed[t * hidden:(t + 1) * hidden]
        scale = np.abs(want).max() + 1e-3
        assert np.all(np.abs(got[t * hidden:(t + 1) * hidden] - want) <= 1e-4 * scale), t


def test_moe_ffn_matches_f64_brute_force():
    rng = np.random.default_rng(9)
    E, hidden, inter, T, k = 6, 64, 96, 5, 3

    def rnd(m, n):
        raw = rng.integers(0, 256, (m * n // 32, 34), dtype=np.uint8)
        raw[:, 0:2] = (np.abs(rng.standard_normal(m * n // 32)) * 0.02).astype(np.float16).view(np.uint8).reshape(-1, 2)
        return raw.reshape(-1)

    gate = np.concatenate([rnd(inter, hidden) for _ in range(E)])
    up = np.concatenate([rnd(inter, hidden) for _ in range(E)])
    down = np.concatenate([rnd(hidden, inter) for _ in range(E)])
    x = rng.standard_normal(T * hidden).astype(np.float32)
    ids = np.concatenate([rng.permutation(E)[:k] for _ in range(T)]).astype(np.uint32)
    w = rng.random(T * k).astype(np.float32)
    out = O.moe_ffn(O.Q8_0, gate, O.Q8_0, up, O.Q8_0, down, E, hidden, inter, x, T, k, ids, w)
    G = O.dequant(O.Q8_0, gate).reshape(E, inter, hidden).astype(np.float64)
    U = O.dequant(O.Q8_0, up).reshape(E, inter, hidden).astype(np.float64)
    D = O.dequant(O.Q8_0, down).reshape(E, hidden, inter).astype(np.float64)
    for t in range(T):
        xt = x[t * hidden:(t + 1) * hidden].astype(np.float64)
        want = np.zeros(hidden)
        for j in range(k):
            e = ids[t * k + j]
            g, u = G[e] @ xt, U[e] @ xt
            a = g / (1.0 + np.exp(-g)) * u
            want += float(w[t * k + j]) * (D[e] @ a)
        scale = np.abs(want).max() + 1e-3
        assert np.all(np.abs(out[t * hidden:(t + 1) * hidden] - want) <= 1e-4 * scale), t
