"""MoE experts whose rows are too long for the grouped expert GEMV's LDS staging (a task stages 4
activation rows of K floats plus their per-16 sums and the wave partials: K = 8192 fits 160 KiB,
K = 9216 does not). Past that edge every batch size must take the grouped GEMM paths instead
(moe_gemv_fits), including the one-token path. The down projection's K is the intermediate
size, so inter = 8192 (fits), 9216 and 14336 (Mixtral-like) straddle the edge; T = 1 and 4 in
both modes against the oracle's expert FFN (f32 1e-4, bf16 1e-2 relative to norm)."""
import numpy as np
import pytest

import oracle as O
import rehip
from rehip import synth

pytestmark = pytest.mark.gpu

E, H, K = 4, 512, 2


@pytest.fixture(scope="module", params=[8192, 9216, 14336])
def experts(request):
    inter = request.param
    rng = np.random.default_rng(9100 + inter)
    gate = np.concatenate([synth.weight_bytes(rng, rehip.Q4_K, inter, H) for _ in range(E)])
    up = np.concatenate([synth.weight_bytes(rng, rehip.Q4_K, inter, H) for _ in range(E)])
    down = np.concatenate([synth.weight_bytes(rng, rehip.Q6_K, H, inter) for _ in range(E)])
    moe = rehip.MoeExperts(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, down, E, H, inter)
    yield inter, (gate, up, down), moe
    moe.close()


@pytest.mark.parametrize("tokens", [1, 4])
def test_long_expert_rows_match_oracle(experts, tokens):
    inter, (gate, up, down), moe = experts
    rng = np.random.default_rng(9200 + tokens + inter)
    ids, wts, _ = synth.router(rng, tokens, E, K)
    x = synth.activations(rng, tokens, H)
    want = O.moe_ffn(rehip.Q4_K, gate, rehip.Q4_K, up, rehip.Q6_K, down, E, H, inter, x, tokens, K,
                     ids.reshape(-1), wts.reshape(-1))
    for mode, tol in [(rehip.MODE_F32, 1e-4), (rehip.MODE_BF16, 1e-2)]:
        got = moe.forward(x, tokens, K, ids, wts, mode)
        rel = np.linalg.norm(got - want) / np.linalg.norm(want)
        assert rel <= tol, (inter, tokens, mode, rel)
