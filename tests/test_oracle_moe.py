"""Pins the oracle's router and expert FFN (src/moe.rs restatement).

The reference's own tests (moe.rs:624-801) are ported; its 2x2 f32 identity experts become
32x32 Q8_0 identity experts (d = 1, quant 1 on the diagonal), which dequantize exactly to the
identity, so the reference's closed forms (silu(1), 2*silu(1), ...) still apply. A brute-force
f64 evaluation of the whole layer pins the batched path on random experts.
"""
import math

import numpy as np
import pytest

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


# ---- bias-corrected group routers (moe.rs:126-268) ----------------------------------------------
EPS = 1e-5


def test_route_group_restricts_to_best_group():           # moe.rs:675-686
    ids, w = O.route_group([0.0, 0.0, 0.0, 5.0, 4.0, 3.0], None, 2, 2, 1)
    assert len(ids) == 2 and all(3 <= i <= 5 for i in ids)
    assert abs(w.sum() - 1.0) < EPS


def test_route_noaux_tc_uses_top2_group_score_not_group_sum():   # moe.rs:688-701
    logits = [5.0, 2.0, -9.0, -9.0, 0.0, 0.0, 0.0, 0.0]
    ids, w = O.route_noaux_tc(logits, None, 2, 1, 1)
    assert ids[0] == 0 and abs(w[0] - 1.0) < EPS
    ids, _ = O.route_group(logits, None, 2, 1, 1)
    assert 4 <= ids[0] <= 7


def test_route_noaux_tc_renormalizes_top_k():             # moe.rs:703-712
    ids, w = O.route_noaux_tc([5.0, 2.0, -9.0, -9.0, 0.0, 0.0, 0.0, 0.0], None, 2, 2, 1)
    assert list(ids) == [0, 1] and abs(w.sum() - 1.0) < EPS


def test_route_noaux_tc_empty_input():                    # moe.rs:714-717
    assert O.route_noaux_tc([], None, 2, 1, 1)[0].size == 0
    assert O.route_group([], None, 2, 1, 1)[0].size == 0


@pytest.mark.parametrize("router", [O.route_group, O.route_noaux_tc])
@pytest.mark.parametrize("n,ng,k", [(128, 8, 8), (64, 1, 6), (256, 8, 8), (10, 3, 4)])
def test_every_group_eligible_is_top_k_sigmoid(router, n, ng, k):
    # top_k_group None (and = ng) keeps every expert: the selection and the weights are those of
    # top_k_sigmoid (moe.rs:97-117), bit for bit, ties included (quantised logits)
    rng = np.random.default_rng(500 + n + ng)
    logits = (np.round(rng.standard_normal(n) * 4) / 4).astype(np.float32)
    want = O.top_k_sigmoid(logits, k)
    for tkg in (None, ng):
        got = router(logits, None, ng, k, tkg)
        assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1]), tkg


@pytest.mark.parametrize("router", [O.route_group, O.route_noaux_tc])
def test_bias_is_added_to_the_logits(router):
    # sigmoid(logit + bias[i]): passing the bias equals passing logits + bias (same f32 sum);
    # entries past the bias's length count as 0 (bias.get(i).unwrap_or(0.0))
    rng = np.random.default_rng(510)
    logits = rng.standard_normal(128).astype(np.float32)
    bias = (rng.standard_normal(128) * 0.5).astype(np.float32)
    a = router(logits, bias, 8, 8, 4)
    b = router((logits + bias).astype(np.float32), None, 8, 8, 4)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    short = bias[:40]
    a = router(logits, short, 8, 8, 4)
    b = router(logits, np.concatenate([short, np.zeros(88, np.float32)]), 8, 8, 4)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def brute_force_route(logits, n_groups, k, tkg, top2):
    """Independent restatement by sets and numpy's stable argsort: group i * ng // n; group score
    = sum (route_group) or sum of the two best (route_noaux_tc) of the oracle's sigmoid scores;
    the tkg best groups (ties to the lower group) are eligible; the k best eligible experts (ties
    to the lower index)."""
    n = len(logits)
    sc = np.array([O.sigmoid(float(x)) for x in logits], np.float32)
    ng = max(1, min(n_groups, n))
    grp = np.arange(n) * ng // n
    gs = []
    for g in range(ng):
        v = sc[grp == g]
        if top2:
            v = np.sort(v)[::-1][:2]
        acc = np.float32(0.0)
        for x in (v if top2 else sc[grp == g]):
            acc = np.float32(acc + x)
        gs.append(acc)
    gs = np.array(gs, np.float32)
    order = np.argsort(-gs, kind="stable")
    allowed = set(order[:min(tkg, ng)].tolist())
    cand = np.array([i for i in range(n) if grp[i] in allowed])
    pick = cand[np.argsort(-sc[cand], kind="stable")][:min(k, len(cand))]
    return pick


@pytest.mark.parametrize("top2", [False, True])
@pytest.mark.parametrize("n,ng,k,tkg", [(128, 8, 8, 4), (256, 8, 8, 4), (10, 3, 4, 1), (96, 12, 6, 3),
                                        (8, 4, 4, 1)])
def test_group_routing_matches_brute_force(top2, n, ng, k, tkg):
    rng = np.random.default_rng(520 + n + ng + 7 * top2)
    for trial in range(20):
        # quantised logits: equal scores (ties) inside and across groups
        logits = (np.round(rng.standard_normal(n) * 2) / 2).astype(np.float32)
        ids, w = (O.route_noaux_tc if top2 else O.route_group)(logits, None, ng, k, tkg)
        want = brute_force_route(logits, ng, k, tkg, top2)
        assert list(ids) == list(want), (trial, list(ids), list(want))
        assert abs(float(w.sum()) - 1.0) < EPS
    # fewer eligible experts than k: (8 experts, 4 groups of 2, one group) -> 2 results
    if (n, ng, tkg) == (8, 4, 1):
        assert len(want) == 2
