"""Seeded synthetic GGUF weights and activations for the quantized matmul workloads.

Block bytes are uniform random (so every quant field is uniform), with finite scales stamped in,
as the reference's benches do (benches/quant.rs:42-63, benches/kquant.rs:40-50):
  - 32-element blocks (Q4_0/Q5_0/Q8_0): d = f16(|N(0,1)| * 0.01);
  - Q4_K/Q5_K: d and dmin = f16(|N(0,1)| * 1e-3), scale/min bytes and quants uniform;
  - Q6_K: d = f16(|N(0,1)| * 1e-3), int8 sub-scales uniform in [-64, 63], quants uniform.
Activations are f32 ~ N(0, 1). Generators are numpy PCG64 (`default_rng(seed)`).
"""
from __future__ import annotations

import numpy as np

from . import GEOM, Q4_K, Q5_K, Q6_K


def weight_bytes(rng: np.random.Generator, ggml_type: int, m: int, n: int) -> np.ndarray:
    """m rows of ceil(n/QK) blocks (rows padded to whole blocks when n % QK != 0)."""
    qk, bb = GEOM[ggml_type]
    nb = m * ((n + qk - 1) // qk)
    raw = rng.integers(0, 256, (nb, bb), dtype=np.uint8)
    if ggml_type in (Q4_K, Q5_K):
        d = (np.abs(rng.standard_normal((nb, 2))) * 1e-3).astype(np.float16)
        raw[:, 0:4] = d.view(np.uint8).reshape(nb, 4)
    elif ggml_type == Q6_K:
        raw[:, 192:208] = rng.integers(-64, 64, (nb, 16)).astype(np.int8).view(np.uint8)
        d = (np.abs(rng.standard_normal(nb)) * 1e-3).astype(np.float16)
        raw[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    else:
        d = (np.abs(rng.standard_normal(nb)) * 0.01).astype(np.float16)
        raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)


def activations(rng: np.random.Generator, rows: int, n: int) -> np.ndarray:
    return rng.standard_normal((rows, n), dtype=np.float32).reshape(-1)


def router(rng: np.random.Generator, tokens: int, n_experts: int, top_k: int):
    """Top-k softmax routing on f32 logits ~ N(0,1): the reference's top_k (moe.rs:75-93) —
    stable descending sort of the logits, softmax over the chosen ones. Returns (ids, weights,
    logits); ids/weights are tokens x top_k."""
    logits = rng.standard_normal((tokens, n_experts), dtype=np.float32)
    ids = np.empty((tokens, top_k), np.uint32)
    w = np.empty((tokens, top_k), np.float32)
    for t in range(tokens):
        order = np.argsort(-logits[t], kind="stable")[:top_k]
        s = logits[t, order]
        e = np.exp((s - s.max()).astype(np.float32)).astype(np.float32)
        ids[t] = order
        w[t] = e / np.float32(e.sum(dtype=np.float32))
    return ids, w, logits
