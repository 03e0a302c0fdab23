"""Dense Qwen2-architecture decoder over a pluggable quantized-matmul backend.

This restates the reference's dense runner (src/runner.rs:105-282) and transformer block
(src/forward.rs:100-586) on the host, with every projection going through a backend object
that exposes `matvec(x)` / `matmul(x, rows)` like `QMat` (src/qmat.rs:80, 169):

  * `HipBackend` routes each projection through librehip (`rehip.QMat`), which is the drop-in
    the reference would make in `QMat::Quant`;
  * any other object with `make(ggml_type, bytes, m, n)` returning such a matrix and
    `dequant(ggml_type, bytes)` can be passed in (the measurement and parity code passes the
    CPU kernels this way).

Attention, RMS-norm, RoPE, SwiGLU and argmax stay on the host, as in the reference's
configuration for this workload. They are vectorised numpy restatements of:
  rmsnorm            infer.rs:72-82    x * (1 / sqrt(mean(x^2) + eps)) * w
  rope (NeoX)        infer.rs:90-139   angle = pos * base^(-2i/d); (x0 c - x1 s, x1 c + x0 s)
  attention          forward.rs:232-277, 437-470   softmax(q.k / sqrt(hd)) over 0..=pos, p.v
  softmax            moe.rs:61-72      exp(x - max) / sum (no division when the sum is 0)
  silu / swiglu      moe.rs:44-51, 280-283         g * (1 / (1 + exp(-g))) * u
  argmax             infer.rs:217-223  the last index among equal maxima (Iterator::max_by)
  decoder            runner.rs:205-282 batched prefill that fills rotated K/V, then one
                                       position per step over the cache.
Sums inside these host steps use numpy's order, not the reference's sequential f32 order;
both backends share this host code, so a greedy comparison between them isolates the matmuls.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import MODE_F32, Q4_K, Q6_K, Q8_0, QMat, dequant
from . import synth


@dataclass(frozen=True)
class Geometry:
    """forward.rs:17-55."""
    d_model: int = 896
    n_heads: int = 14
    n_kv_heads: int = 2
    d_ff: int = 4864
    rope_freq_base: float = 1e6
    rms_eps: float = 1e-6

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads


QWEN25_05B = Geometry()
QWEN25_05B_LAYERS = 24
QWEN25_05B_VOCAB = 151936


class HipBackend:
    """Projections on the GPU through librehip; `mode` selects bf16 MFMA or f32 GEMM."""

    name = "hip"

    def __init__(self, mode: int = MODE_F32):
        self.mode = mode

    @staticmethod
    def dequant(ggml_type: int, data: np.ndarray) -> np.ndarray:
        return dequant(ggml_type, data)

    def make(self, ggml_type: int, data: np.ndarray, m: int, n: int):
        q = QMat.from_bytes(ggml_type, data, m, n)
        mode = self.mode

        class _M:
            def rows(self_):
                return m

            def cols(self_):
                return n

            def matvec(self_, x):
                return q.matvec(x)

            def matmul(self_, x, rows):
                return q.matmul(x, rows, mode)

            def close(self_):
                q.close()

        return _M()


# ---- host steps ---------------------------------------------------------------------------
def rmsnorm_rows(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = x.reshape(-1, w.size)
    ms = np.einsum("ij,ij->i", x, x, dtype=np.float32) / np.float32(w.size)
    inv = np.float32(1.0) / np.sqrt(ms + np.float32(eps), dtype=np.float32)
    return (x * inv[:, None] * w[None, :]).astype(np.float32)


def rope_freqs(d: int, base: float) -> np.ndarray:
    i = np.arange(d // 2, dtype=np.float32)
    return (np.float32(1.0) / np.power(np.float32(base), np.float32(2.0) * i / np.float32(d))).astype(np.float32)


def rope_table(seq: int, pos_start: int, d: int, base: float):
    f = rope_freqs(d, base)
    ang = (np.arange(pos_start, pos_start + seq, dtype=np.float32)[:, None] * f[None, :]).astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rope_rows(x: np.ndarray, heads: int, hd: int, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """NeoX rotate-half of a (seq, heads * hd) buffer with per-row (cos, sin) tables."""
    v = x.reshape(-1, heads, hd)
    half = hd // 2
    x0, x1 = v[:, :, :half], v[:, :, half:]
    c, s = cos[:, None, :], sin[:, None, :]
    out = np.empty_like(v)
    out[:, :, :half] = x0 * c - x1 * s
    out[:, :, half:] = x1 * c + x0 * s
    return out.reshape(x.shape)


def softmax_rows(s: np.ndarray) -> np.ndarray:
    mx = np.max(s, axis=-1, keepdims=True)
    e = np.exp(s - mx).astype(np.float32)
    tot = np.sum(e, axis=-1, keepdims=True, dtype=np.float32)
    return np.where(tot != 0, e / np.where(tot != 0, tot, 1), e).astype(np.float32)


def attention(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, g: Geometry, pos_start: int) -> np.ndarray:
    """Causal GQA attention of `seq` rotated query rows at positions pos_start.. over the cache
    rows 0..pos_start+seq (forward.rs:232-277)."""
    hd, nh, nkv = g.head_dim, g.n_heads, g.n_kv_heads
    seq = q.shape[0] // (nh * hd) if q.ndim == 1 else q.shape[0]
    q = q.reshape(seq, nh, hd)
    total = pos_start + seq
    k = kc[:total].reshape(total, nkv, hd)
    v = vc[:total].reshape(total, nkv, hd)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    ctx = np.empty((seq, nh, hd), np.float32)
    grp = nh // nkv                       # query heads h with h * nkv // nh == kv are contiguous
    rows = 128                            # query rows per pass: temporaries stay cache-sized
    for kv in range(nkv):
        qg = np.ascontiguousarray(q[:, kv * grp:(kv + 1) * grp, :].transpose(1, 0, 2))   # grp, seq, hd
        kt = np.ascontiguousarray(k[:, kv, :].T)
        vv = np.ascontiguousarray(v[:, kv, :])
        for r0 in range(0, seq, rows):
            r1 = min(seq, r0 + rows)
            end = pos_start + r1                           # keys 0..end-1 cover every row here
            s = np.matmul(qg[:, r0:r1, :], kt[:, :end]) * scale                             # grp, r, end
            if r1 - r0 > 1 or end > pos_start + r0 + 1:
                later = np.arange(end)[None, :] > (pos_start + np.arange(r0, r1))[:, None]
                s[:, later] = -np.inf
            p = softmax_rows(s)
            ctx[r0:r1, kv * grp:(kv + 1) * grp, :] = np.matmul(p, vv[:end]).transpose(1, 0, 2)
    return ctx.reshape(seq, nh * hd)


def silu(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):      # exp(-x) = inf for x < -88 gives silu = -0, as in f32
        return (x * (np.float32(1.0) / (np.float32(1.0) + np.exp(-x)))).astype(np.float32)


def argmax_last(logits: np.ndarray) -> int:
    """Index of the maximum; among equal maxima the last one (infer.rs:217-223)."""
    mx = np.max(logits)
    return int(np.flatnonzero(logits == mx)[-1])


# the reference's logit-profile gate (tests/qwen35_parity.rs:45-52)
LOGIT_TOL = 0.75    # nats: |(got - max got) - (ref - max ref)| over the reference's top-5
TIE_FLOOR = 0.5     # nats: the reference's top1 - top2 margin from which the argmax must agree


def logit_profile_check(ref: np.ndarray, got: np.ndarray, top: int = 5, tol: float = LOGIT_TOL,
                        tie_floor: float = TIE_FLOOR) -> dict:
    """The profile gate of tests/qwen35_parity.rs:12-20, 45-52 for one position: for each of the
    reference's `top` tokens, the gap of `got`'s logit to `got`'s maximum must match the gap of
    the reference's logit to the reference's maximum within `tol` (a logit gap equals the
    log-softmax gap); the argmax must agree where the reference's top-1 leads its top-2 by at
    least `tie_floor`. Returns the worst gap deviation, whether the argmax was required and
    matched, and `ok`."""
    ref = np.asarray(ref, np.float64)
    got = np.asarray(got, np.float64)
    order = np.argsort(-ref, kind="stable")[:top]
    dev = np.abs((got[order] - got.max()) - (ref[order] - ref.max()))
    margin = float(ref[order[0]] - ref[order[1]])
    decisive = margin >= tie_floor
    same = argmax_last(got) == argmax_last(ref)
    worst = float(dev.max())
    return {"worst_gap_dev": worst, "margin": margin, "decisive": bool(decisive), "argmax_same": bool(same),
            "ok": bool(worst <= tol and (same or not decisive))}


# ---- weights ------------------------------------------------------------------------------
@dataclass
class BlockBytes:
    """One block's tensors: projection bytes (GGUF blocks, or F32/F16/BF16 elements) and f32 norm
    and bias vectors. `types` names the ggml type of a projection whose type differs from the
    model-wide one (a real Q4_K_M file mixes types per tensor)."""
    q: np.ndarray
    k: np.ndarray
    v: np.ndarray
    o: np.ndarray
    gate: np.ndarray
    up: np.ndarray
    down: np.ndarray
    attn_norm: np.ndarray
    ffn_norm: np.ndarray
    q_bias: np.ndarray
    k_bias: np.ndarray
    v_bias: np.ndarray
    types: dict = field(default_factory=dict)


@dataclass
class ModelBytes:
    geom: Geometry
    n_vocab: int
    embed: np.ndarray          # Q8_0 token_embd bytes, n_vocab x d_model
    output: np.ndarray         # Q8_0 output (lm_head) bytes, n_vocab x d_model
    output_norm: np.ndarray
    blocks: list
    attn_type: int = Q4_K
    ffn_type: int = Q4_K
    down_type: int = Q6_K
    embed_type: int = Q8_0
    output_type: int | None = None     # None: the embedding's type
    eos_token_id: int | None = None


# standard deviation of one block's (scale-free) value, d = 1: Q4_K sc*q - 7.5*m with sc, m
# uniform in 0..63 and q in 0..15 (zero mean); Q6_K sc*(q - 32) with sc in -64..63, q in 0..63;
# Q8_0 qs uniform in -128..127
_UNIT_STD = {Q4_K: 257.2, Q6_K: 682.4, Q8_0: 73.9}


def conditioned_weight_bytes(rng: np.random.Generator, t: int, m: int, n: int, std: float) -> np.ndarray:
    """Random GGUF block bytes (synth.weight_bytes) whose f16 scales are re-drawn as
    |N(0,1)| * std / unit_std(t), so the dequantized weights have about zero mean and the given
    standard deviation (Q4_K: dmin = 7.5 d cancels the mean of d*sc*q)."""
    raw = synth.weight_bytes(rng, t, m, n)
    qk, bb = {Q4_K: (256, 144), Q6_K: (256, 210), Q8_0: (32, 34)}[t]
    blocks = raw.reshape(-1, bb)
    nb = blocks.shape[0]
    d = (np.abs(rng.standard_normal(nb)) * (std / _UNIT_STD[t])).astype(np.float16)
    if t == Q4_K:
        blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        blocks[:, 2:4] = (d.astype(np.float32) * 7.5).astype(np.float16).view(np.uint8).reshape(nb, 2)
    elif t == Q6_K:
        blocks[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    else:
        blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    return raw


def synth_model(seed: int, geom: Geometry = QWEN25_05B, n_layers: int = QWEN25_05B_LAYERS,
                n_vocab: int = QWEN25_05B_VOCAB) -> ModelBytes:
    """Seeded random-init weights of the Q4_K_M mix: Q4_K attention and gate/up, Q6_K down,
    Q8_0 embedding and output (untied: a tied random model locks onto one token). Projection weights have about zero mean and standard deviation
    1/sqrt(K) (activations stay of order one through the layers), embedding entries 0.1; norm
    weights are 1 + N(0, 0.1^2), q/k/v biases N(0, 0.1^2)."""
    rng = np.random.default_rng(seed)
    d, kv, ff = geom.d_model, geom.n_kv_heads * geom.head_dim, geom.d_ff
    wd, wf = 1.0 / np.sqrt(d), 1.0 / np.sqrt(ff)
    blocks = []
    for _ in range(n_layers):
        blocks.append(BlockBytes(
            q=conditioned_weight_bytes(rng, Q4_K, d, d, wd), k=conditioned_weight_bytes(rng, Q4_K, kv, d, wd),
            v=conditioned_weight_bytes(rng, Q4_K, kv, d, wd), o=conditioned_weight_bytes(rng, Q4_K, d, d, wd),
            gate=conditioned_weight_bytes(rng, Q4_K, ff, d, wd), up=conditioned_weight_bytes(rng, Q4_K, ff, d, wd),
            down=conditioned_weight_bytes(rng, Q6_K, d, ff, wf),
            attn_norm=(1 + 0.1 * rng.standard_normal(d)).astype(np.float32),
            ffn_norm=(1 + 0.1 * rng.standard_normal(d)).astype(np.float32),
            q_bias=(0.1 * rng.standard_normal(d)).astype(np.float32),
            k_bias=(0.1 * rng.standard_normal(kv)).astype(np.float32),
            v_bias=(0.1 * rng.standard_normal(kv)).astype(np.float32)))
    embed = conditioned_weight_bytes(rng, Q8_0, n_vocab, d, 0.1)
    output = conditioned_weight_bytes(rng, Q8_0, n_vocab, d, 0.1)
    output_norm = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    return ModelBytes(geom, n_vocab, embed, output, output_norm, blocks)


def _f32_vector(g, name: str) -> np.ndarray:
    """An F32 / F16 / BF16 vector tensor widened to f32 (norm weights and biases)."""
    t = g.tensor(name)
    raw = np.asarray(g.tensor_bytes(name))
    if t.ggml_type == 0:
        return raw.view(np.float32).copy()
    if t.ggml_type == 1:
        return raw.view(np.float16).astype(np.float32)
    if t.ggml_type == 30:
        return (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    raise ValueError(f"tensor '{name}' of ggml type {t.ggml_type} is not a float vector")


def model_from_gguf(g) -> ModelBytes:
    """A dense model from a GGUF file (rehip.Gguf) as DenseRunner::from_model loads it
    (runner.rs:46-101, model.rs:122-240): hyper-parameters under `<arch>.` or `general.` keys
    (head_count_kv defaults to head_count, vocab_size to the tokenizer's token count, rope base
    to 10000, RMS eps to 1e-5); per block attn_norm, attn_q/k/v/output, ffn_norm, ffn_gate/up/down
    and the optional attn_q/k/v biases (absent = zero); output_norm (or norm), output. Projection
    bytes are views of the mapping, typed per tensor."""
    arch = g.get("general.architecture")
    if not isinstance(arch, str):
        raise ValueError("missing general.architecture")

    def key(suffix, dflt=None, required=False):
        for k in (f"{arch}.{suffix}", f"general.{suffix}"):
            v = g.get(k)
            if v is not None:
                return v
        if required:
            raise ValueError(f"missing required key '{arch}.{suffix}'")
        return dflt

    n_heads = int(key("attention.head_count", required=True))
    d_model = int(key("embedding_length", required=True))
    n_layers = int(key("block_count", required=True))
    d_ff = key("feed_forward_length")
    if d_ff is None:
        d_ff = key("expert_feed_forward_length", required=True)
    n_kv = int(key("attention.head_count_kv", n_heads))
    tokens = g.get("tokenizer.ggml.tokens")
    n_vocab = int(key("vocab_size", tokens[2] if isinstance(tokens, tuple) else 0))
    geom = Geometry(d_model=d_model, n_heads=n_heads, n_kv_heads=n_kv, d_ff=int(d_ff),
                    rope_freq_base=float(key("rope.freq_base", 10000.0)),
                    rms_eps=float(key("attention.layer_norm_rms_epsilon", 1e-5)))
    kv = n_kv * geom.head_dim

    def bias(name, n):
        try:
            g.tensor(name)
        except Exception:
            return np.zeros(n, np.float32)
        return _f32_vector(g, name)

    names = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate",
             "up": "ffn_up", "down": "ffn_down"}
    blocks = []
    for i in range(n_layers):
        p = f"blk.{i}."
        proj = {f: np.asarray(g.tensor_bytes(p + t + ".weight")) for f, t in names.items()}
        types = {f: g.tensor(p + t + ".weight").ggml_type for f, t in names.items()}
        blocks.append(BlockBytes(attn_norm=_f32_vector(g, p + "attn_norm.weight"),
                                 ffn_norm=_f32_vector(g, p + "ffn_norm.weight"),
                                 q_bias=bias(p + "attn_q.bias", d_model), k_bias=bias(p + "attn_k.bias", kv),
                                 v_bias=bias(p + "attn_v.bias", kv), types=types, **proj))
    try:
        output_norm = _f32_vector(g, "output_norm.weight")
    except Exception:
        output_norm = _f32_vector(g, "norm.weight")
    eos = g.get("tokenizer.ggml.eos_token_id")
    return ModelBytes(geom, n_vocab, np.asarray(g.tensor_bytes("token_embd.weight")),
                      np.asarray(g.tensor_bytes("output.weight")), output_norm, blocks,
                      embed_type=g.tensor("token_embd.weight").ggml_type,
                      output_type=g.tensor("output.weight").ggml_type,
                      eos_token_id=None if eos is None else int(eos))


class _Block:
    def __init__(self, b: BlockBytes, mb: ModelBytes, backend):
        g = mb.geom
        d, kv, ff = g.d_model, g.n_kv_heads * g.head_dim, g.d_ff
        ty = lambda f, dflt: b.types.get(f, dflt)   # noqa: E731
        self.q = backend.make(ty("q", mb.attn_type), b.q, d, d)
        self.k = backend.make(ty("k", mb.attn_type), b.k, kv, d)
        self.v = backend.make(ty("v", mb.attn_type), b.v, kv, d)
        self.o = backend.make(ty("o", mb.attn_type), b.o, d, d)
        self.gate = backend.make(ty("gate", mb.ffn_type), b.gate, ff, d)
        self.up = backend.make(ty("up", mb.ffn_type), b.up, ff, d)
        self.down = backend.make(ty("down", mb.down_type), b.down, d, ff)
        self.attn_norm, self.ffn_norm = b.attn_norm, b.ffn_norm
        self.q_bias, self.k_bias, self.v_bias = b.q_bias, b.k_bias, b.v_bias

    def mats(self):
        return (self.q, self.k, self.v, self.o, self.gate, self.up, self.down)


class DenseRunner:
    """runner.rs:11-120: the embedding table is dequantized once (the backend's bit-exact
    dequant); the output projection is a quantized matrix like the others."""

    def __init__(self, mb: ModelBytes, backend):
        self.geom = mb.geom
        self.n_vocab = mb.n_vocab
        self.embed = backend.dequant(mb.embed_type, mb.embed).reshape(mb.n_vocab, mb.geom.d_model)
        self.blocks = [_Block(b, mb, backend) for b in mb.blocks]
        self.output_norm = mb.output_norm
        out_t = mb.embed_type if mb.output_type is None else mb.output_type
        self.output = backend.make(out_t, mb.output, mb.n_vocab, mb.geom.d_model)
        self.eos_token_id = mb.eos_token_id

    def generate(self, prompt, max_new: int) -> list:
        """runner.rs:154-164: the prompt followed by up to max_new greedy tokens, each chosen by
        re-prefilling the whole sequence; stops at the end-of-sequence token."""
        seq = [int(t) for t in prompt]
        for _ in range(max_new):
            t = argmax_last(DenseDecoder(self, len(seq)).prefill(seq))
            if self.eos_token_id is not None and t == self.eos_token_id:
                break
            seq.append(t)
        return seq

    def close(self):
        for b in self.blocks:
            for m in b.mats():
                if hasattr(m, "close"):
                    m.close()
        if hasattr(self.output, "close"):
            self.output.close()


class DenseDecoder:
    """runner.rs:205-282: per-layer rotated K/V caches; batched prefill, then one position per
    step."""

    def __init__(self, runner: DenseRunner, max_seq: int):
        self.r = runner
        g = runner.geom
        kv = g.n_kv_heads * g.head_dim
        self.kc = [np.zeros((max_seq, kv), np.float32) for _ in runner.blocks]
        self.vc = [np.zeros((max_seq, kv), np.float32) for _ in runner.blocks]
        self.seq_len = 0

    def _block(self, l: int, blk: _Block, x: np.ndarray, seq: int, pos_start: int) -> np.ndarray:
        g = self.r.geom
        hd = g.head_dim
        d = g.d_model
        n = rmsnorm_rows(x, blk.attn_norm, g.rms_eps).reshape(-1)
        if seq == 1:
            q, k, v = blk.q.matvec(n), blk.k.matvec(n), blk.v.matvec(n)
        else:
            q, k, v = blk.q.matmul(n, seq), blk.k.matmul(n, seq), blk.v.matmul(n, seq)
        q = (q.reshape(seq, -1) + blk.q_bias).astype(np.float32)
        k = (k.reshape(seq, -1) + blk.k_bias).astype(np.float32)
        v = (v.reshape(seq, -1) + blk.v_bias).astype(np.float32)
        cos, sin = rope_table(seq, pos_start, hd, g.rope_freq_base)
        q = rope_rows(q, g.n_heads, hd, cos, sin)
        k = rope_rows(k, g.n_kv_heads, hd, cos, sin)
        self.kc[l][pos_start:pos_start + seq] = k
        self.vc[l][pos_start:pos_start + seq] = v
        ctx = attention(q, self.kc[l], self.vc[l], g, pos_start).reshape(-1)
        o = blk.o.matvec(ctx) if seq == 1 else blk.o.matmul(ctx, seq)
        y = (x.reshape(seq, d) + o.reshape(seq, d)).astype(np.float32)
        yn = rmsnorm_rows(y, blk.ffn_norm, g.rms_eps).reshape(-1)
        if seq == 1:
            gt, up = blk.gate.matvec(yn), blk.up.matvec(yn)
        else:
            gt, up = blk.gate.matmul(yn, seq), blk.up.matmul(yn, seq)
        act = (silu(gt) * up).astype(np.float32)
        dn = blk.down.matvec(act) if seq == 1 else blk.down.matmul(act, seq)
        return (y + dn.reshape(seq, d)).astype(np.float32)

    def _logits(self, last: np.ndarray) -> np.ndarray:
        g = self.r.geom
        normed = rmsnorm_rows(last, self.r.output_norm, g.rms_eps).reshape(-1)
        return self.r.output.matvec(normed)

    def prefill(self, prompt) -> np.ndarray:
        prompt = np.asarray(prompt, dtype=np.int64)
        seq = prompt.size
        x = self.r.embed[prompt].astype(np.float32)
        pos_start = self.seq_len
        for l, blk in enumerate(self.r.blocks):
            x = self._block(l, blk, x, seq, pos_start)
        self.seq_len += seq
        return self._logits(x[-1])

    def step(self, tok: int) -> np.ndarray:
        x = self.r.embed[tok][None, :].astype(np.float32)
        pos = self.seq_len
        for l, blk in enumerate(self.r.blocks):
            x = self._block(l, blk, x, 1, pos)
        self.seq_len += 1
        return self._logits(x[0])

    def generate(self, prompt, max_new: int, on_token=None):
        """runner.rs:262-282 without an EOS token: prefill, then argmax / step."""
        logits = self.prefill(prompt)
        out = []
        for i in range(max_new):
            t = argmax_last(logits)
            out.append(t)
            if on_token:
                on_token(i, t)
            if i + 1 < max_new:
                logits = self.step(t)
        return out


class DeviceDecoder:
    """The dense decoder with every step on the GPU (row F1 of the hot-path plan): activations,
    rotated K/V caches, the position, the sampled token and the token history stay in HBM.

    Decode step (captured once as a HIP graph, replayed per token; 7 launches per layer):
      q|k|v GEMV over one fused q|k|v matrix with the attention RMS-norm in its prologue ->
      bias + RoPE + K/V-cache append -> key-split attention + combine -> o GEMV with the
      residual add -> gate/up GEMV pair with the FFN RMS-norm and SwiGLU -> down GEMV with the
      residual add; then the lm_head GEMV with the output norm and the greedy argmax folded into
      its stores, and one kernel that takes the token, advances the position and records the
      token. The host reads back 4 bytes per token (`step`) or nothing until the end (`replay`).
    Prefill (eager): the same with GEMMs over all prompt rows and MFMA flash attention.

    Same computation as `DenseDecoder` (runner.rs:205-282, forward.rs:347-586)."""

    def __init__(self, mb: ModelBytes, max_seq: int, mode: int = MODE_F32, prefill_rows: int = 1024,
                 use_graph: bool = True):
        from . import Ffn, attention_work_bytes, hip, rope_table_dev
        self._check_supported(mb)
        self.mb, self.mode, self.max_seq = mb, mode, max_seq
        self.use_graph = use_graph
        g = self.g = mb.geom
        d, hd = g.d_model, g.head_dim
        kv = g.n_kv_heads * hd
        self.kv = kv
        self.cap = max(1, prefill_rows)
        B = hip.DeviceBuffer
        self.blocks = []
        for b in mb.blocks:
            blk = dict(
                o=QMat.from_bytes(mb.attn_type, b.o, d, d),
                gate=QMat.from_bytes(mb.ffn_type, b.gate, g.d_ff, d),
                up=QMat.from_bytes(mb.ffn_type, b.up, g.d_ff, d),
                down=QMat.from_bytes(mb.down_type, b.down, d, g.d_ff),
                attn_norm=B.from_array(b.attn_norm), ffn_norm=B.from_array(b.ffn_norm),
                q_bias=B.from_array(b.q_bias), k_bias=B.from_array(b.k_bias), v_bias=B.from_array(b.v_bias),
                kc=B(max_seq * kv * 4), vc=B(max_seq * kv * 4))
            # q, k and v share their input: one fused matrix (rows q | k | v) when they share a type
            blk["qkv"] = QMat.from_bytes(mb.attn_type, np.concatenate([b.q, b.k, b.v]), d + 2 * kv, d)
            blk["ffn"] = Ffn(blk["gate"], blk["up"])
            self.blocks.append(blk)
        out_t = mb.output_type if mb.output_type is not None else mb.embed_type
        self.output = QMat.from_bytes(out_t, mb.output, mb.n_vocab, d)
        self.output_norm = B.from_array(mb.output_norm)
        self.embed = B.from_array(dequant(mb.embed_type, mb.embed))
        cap = self.cap
        self.x = B(cap * d * 4)
        self.n = B(cap * d * 4)
        self.qkv = B(cap * (d + 2 * kv) * 4)
        self.qb = B(cap * d * 4)
        self.ctx = B(cap * d * 4)
        self.ob = B(cap * g.d_ff * 4)       # o / down outputs of the prefill
        self.gb = B(cap * g.d_ff * 4)
        self.ub = B(cap * g.d_ff * 4)
        self.hb = B(cap * g.d_ff * 4)
        self.logits_buf = B(mb.n_vocab * 4)
        self.work_bytes = attention_work_bytes(8, g.n_heads, hd, max_seq)
        self.work = B(self.work_bytes)
        self.pos = B.from_array(np.zeros(1, np.int32))
        self.tok = B.from_array(np.zeros(1, np.int32))
        self.best = B.from_array(np.zeros(8, np.uint64))         # RE_ARGMAX_SLOTS
        self.hist = B.from_array(np.zeros(max_seq, np.int32))
        self.toks = B(cap * 4)
        self.stream = hip.Stream()
        # RoPE (cos, sin) of every position: the decode attention reads them instead of computing
        self.rope = B(max_seq * hd * 4)
        rope_table_dev(g.rope_freq_base, hd, max_seq, self.rope, self.stream)
        self.graph = None
        self.seq_len = 0

    @staticmethod
    def _check_supported(mb: ModelBytes) -> None:
        """The shapes and types the device-resident step covers, checked before anything is
        allocated: projections quantized (Q4_0/Q5_0/Q8_0/Q4_K/Q5_K/Q6_K, the fused norm / residual /
        SwiGLU / argmax epilogues) or dense (F32/F16/BF16: the norm and SwiGLU as launches of their
        own), one type for q, k and v (one fused matrix) and one for gate and up (one pair), rows a
        multiple of 32 elements, and head_dim a multiple of 4 up to 256 (the attention kernels).
        Raises ValueError naming what is outside."""
        from . import BF16, F16, F32, GEOM
        g = mb.geom
        if g.d_model % g.n_heads or g.head_dim % 4 or g.head_dim > 256 or g.n_heads % g.n_kv_heads:
            raise ValueError(f"DeviceDecoder: head_dim {g.d_model}/{g.n_heads} with {g.n_kv_heads} KV heads; the "
                             "attention kernels take head_dim a multiple of 4 up to 256 and whole query groups")
        if g.d_model % 32 or g.d_ff % 32:
            raise ValueError(f"DeviceDecoder: d_model {g.d_model} and d_ff {g.d_ff} must be multiples of 32")
        out_t = mb.output_type if mb.output_type is not None else mb.embed_type
        for name, t in (("attention", mb.attn_type), ("ffn", mb.ffn_type), ("down", mb.down_type),
                        ("embedding", mb.embed_type), ("output", out_t)):
            if t not in GEOM and t not in (F32, F16, BF16):
                raise ValueError(f"DeviceDecoder: the {name} weights are ggml type {t}, which has no GEMV kernel "
                                 "(Q4_0/Q5_0/Q8_0/Q4_K/Q5_K/Q6_K and F32/F16/BF16 only)")
        for i, b in enumerate(mb.blocks):
            if b.types:
                raise ValueError(f"DeviceDecoder: block {i} overrides tensor types {sorted(b.types)}; the device "
                                 "step takes one attention type (fused q|k|v) and one ffn type (paired gate/up)")

    # -- pieces ----------------------------------------------------------------------------
    def _qkv_post(self, blk, rows):
        from . import qkv_rope_append_dev
        g, d, kv = self.g, self.g.d_model, self.kv
        ld = d + 2 * kv
        qkv_rope_append_dev(self.qkv, ld, _Offset(self.qkv, 4 * d), ld, _Offset(self.qkv, 4 * (d + kv)), ld,
                            blk["q_bias"], blk["k_bias"], blk["v_bias"], rows, g.n_heads, g.n_kv_heads, g.head_dim,
                            g.rope_freq_base, self.pos, self.qb, blk["kc"], blk["vc"], self.max_seq, self.stream)

    def _decode_attention(self, blk):
        """One decode row: q|k|v epilogue and attention in one call (two kernels)."""
        from . import attention_decode_dev
        g, d, kv = self.g, self.g.d_model, self.kv
        attention_decode_dev(self.qkv, _Offset(self.qkv, 4 * d), _Offset(self.qkv, 4 * (d + kv)), blk["q_bias"],
                             blk["k_bias"], blk["v_bias"], g.n_heads, g.n_kv_heads, g.head_dim, g.rope_freq_base,
                             self.pos, blk["kc"], blk["vc"], self.max_seq, self.work, self.work_bytes, self.ctx,
                             self.stream, rope=self.rope)

    def _attention(self, blk, rows):
        from . import attention_dev
        g = self.g
        attention_dev(self.qb, blk["kc"], blk["vc"], rows, g.n_heads, g.n_kv_heads, g.head_dim, self.max_seq,
                      self.pos, self.ctx, work=self.work if rows < 8 else None,
                      work_bytes=self.work_bytes if rows < 8 else 0, stream=self.stream)

    def _head_and_advance(self, last_row, delta):
        from . import decode_advance_dev
        self.output.matvec_ex_dev(last_row, self.logits_buf, norm_w=self.output_norm, eps=self.g.rms_eps,
                                  best=self.best, stream=self.stream)
        decode_advance_dev(self.best, self.tok, self.pos, delta, self.hist, self.max_seq, self.stream)

    def _step_body(self):
        """One decode position: token *tok at position *pos -> next token in *tok, *pos + 1."""
        from . import embed_dev
        g, s, eps = self.g, self.stream, self.g.rms_eps
        embed_dev(self.embed, self.mb.n_vocab, g.d_model, self.tok, 1, self.x, s)
        for blk in self.blocks:
            blk["qkv"].matvec_ex_dev(self.x, self.qkv, norm_w=blk["attn_norm"], eps=eps, stream=s)
            self._decode_attention(blk)
            blk["o"].matvec_ex_dev(self.ctx, self.x, add=self.x, stream=s)            # residual
            blk["ffn"].forward_dev(self.x, self.hb, norm_w=blk["ffn_norm"], eps=eps, stream=s)
            blk["down"].matvec_ex_dev(self.hb, self.x, add=self.x, stream=s)          # residual
        self._head_and_advance(self.x, 1)

    # -- API -------------------------------------------------------------------------------
    def prefill(self, prompt) -> int:
        """Batched prefill of the prompt (runner.rs:236-260); returns the first greedy token."""
        from . import add_dev, embed_dev, rmsnorm_dev, swiglu_dev
        g, s, m = self.g, self.stream, self.mode
        d = g.d_model
        prompt = np.asarray(prompt, np.int32)
        rows = prompt.size
        if not (0 < rows <= self.cap and self.seq_len + rows <= self.max_seq):
            raise ValueError(f"prefill of {rows} rows at position {self.seq_len} (cap {self.cap}, max_seq {self.max_seq})")
        if prompt.min() < 0 or prompt.max() >= self.mb.n_vocab:
            raise ValueError("prompt token outside the vocabulary")
        self.toks.upload(prompt)
        embed_dev(self.embed, self.mb.n_vocab, d, self.toks, rows, self.x, s)
        for blk in self.blocks:
            rmsnorm_dev(self.x, blk["attn_norm"], rows, d, g.rms_eps, self.n, s)
            blk["qkv"].matmul_dev(self.n, rows, self.qkv, m, stream=s)
            self._qkv_post(blk, rows)
            self._attention(blk, rows)
            blk["o"].matmul_dev(self.ctx, rows, self.ob, m, stream=s)
            add_dev(self.x, self.ob, rows * d, rows * d, self.x, s)
            rmsnorm_dev(self.x, blk["ffn_norm"], rows, d, g.rms_eps, self.n, s)
            blk["gate"].matmul_dev(self.n, rows, self.gb, m, stream=s)
            blk["up"].matmul_dev(self.n, rows, self.ub, m, stream=s)
            swiglu_dev(self.gb, self.ub, self.hb, rows * g.d_ff, s)
            blk["down"].matmul_dev(self.hb, rows, self.ob, m, stream=s)
            add_dev(self.x, self.ob, rows * d, rows * d, self.x, s)
        self._head_and_advance(_Offset(self.x, (rows - 1) * d * 4), rows)
        self.seq_len += rows
        self.stream.synchronize()
        return int(self.tok.download(np.int32, 1)[0])

    def _graph(self):
        from . import hip
        if self.graph is None:
            self.graph = hip.Graph(self.stream, self._step_body)
        return self.graph

    def step(self) -> int:
        """Decode the token in *tok at the next position; returns the following greedy token."""
        if self.seq_len >= self.max_seq:
            raise ValueError(f"decode past max_seq {self.max_seq}")
        if not self.use_graph:
            self._step_body()
        else:
            self._graph().launch()
        self.seq_len += 1
        self.stream.synchronize()
        return int(self.tok.download(np.int32, 1)[0])

    def replay(self, steps: int) -> None:
        """`steps` decode steps back to back with no host synchronisation in between (the token
        and position stay on the GPU; each token is recorded in the history); waits for the
        last one."""
        if self.seq_len + steps > self.max_seq:
            raise ValueError(f"decode past max_seq {self.max_seq}")
        for _ in range(steps):
            if self.use_graph:
                self._graph().launch()
            else:
                self._step_body()
        self.seq_len += steps
        self.stream.synchronize()

    def history(self, start: int, count: int) -> list:
        """Tokens recorded at positions start .. start + count - 1."""
        self.stream.synchronize()
        h = self.hist.download(np.int32, self.max_seq)
        return [int(t) for t in h[start:start + count]]

    def logits(self) -> np.ndarray:
        """The logits of the last position computed (downloaded)."""
        self.stream.synchronize()
        return self.logits_buf.download(np.float32, self.mb.n_vocab)

    def generate(self, prompt, max_new: int):
        """Prefill, then max_new - 1 graph replays back to back; the tokens come from the
        device history in one read at the end."""
        p0 = self.seq_len
        if p0 + len(prompt) + max_new > self.max_seq:
            raise ValueError(f"{len(prompt)} + {max_new} tokens from position {p0} exceed max_seq {self.max_seq}")
        self.prefill(prompt)
        if max_new > 1:
            self.replay(max_new - 1)
        return self.history(p0 + len(prompt), max_new)

    def close(self):
        if self.graph is not None:
            self.graph.destroy()
            self.graph = None
        for blk in self.blocks:
            blk["ffn"].close()
            for k in ("qkv", "o", "gate", "up", "down"):
                blk[k].close()
        self.output.close()
        self.stream.destroy()


class _Offset:
    """A device address inside a buffer (for passing a row of a larger buffer)."""

    def __init__(self, buf, byte_offset: int):
        self.ptr = buf.ptr + byte_offset
