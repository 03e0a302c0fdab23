"""Decode GEMV sweep (N = 1) over the projections of a Qwen2.5-0.5B-shaped layer stack, in every
quant type: q/o 896x896, k/v 128x896, gate/up 4864x896, down 896x4864, lm_head 151936x896.

Each projection is timed as a HIP graph of back-to-back launches rotating over enough weight
copies (> 512 MiB) that the weights stream from HBM. Bytes are algorithmic: stored GGUF weight
bytes + f32 x + f32 y per launch.

    python -m rehip.sweep [--types Q4_K,Q6_K] [--launches 300] [--json out.json]
"""
from __future__ import annotations

import argparse
import json
import sys

import numpy as np

from . import GEOM, QMat, TYPE_NAMES, init
from . import hip, synth

PROJECTIONS = [("tiny", 64, 32), ("q", 896, 896), ("o", 896, 896), ("k", 128, 896), ("v", 128, 896),
               ("gate", 4864, 896), ("up", 4864, 896), ("down", 896, 4864), ("lm_head", 151936, 896)]
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0


def algorithmic_bytes(t: int, m: int, k: int) -> int:
    qk, bb = GEOM[t]
    return m * k * bb // qk + 4 * k + 4 * m


def time_gemv(t: int, m: int, k: int, launches: int, seed: int, rotate_bytes: int = 512 << 20):
    rng = np.random.default_rng(seed)
    w = synth.weight_bytes(rng, t, m, k)
    x = synth.activations(rng, 1, k)
    copies = max(2, int(np.ceil(rotate_bytes / w.size)))
    copies = min(copies, launches)
    qs = [QMat.from_bytes(t, w, m, k) for _ in range(copies)]
    dx = hip.DeviceBuffer.from_array(x)
    dy = hip.DeviceBuffer(m * 4)
    s = hip.Stream()
    g = hip.Graph(s, lambda: [qs[i % copies].matvec_dev(dx, dy, stream=s) for i in range(launches)])
    g.launch()
    s.synchronize()
    e0, e1 = hip.Event(), hip.Event()
    e0.record(s)
    g.launch()
    e1.record(s)
    e1.synchronize()
    us = e0.elapsed_ms(e1) * 1e3 / launches
    g.destroy()
    for q in qs:
        q.close()
    s.destroy()
    nbytes = algorithmic_bytes(t, m, k)
    return {"type": TYPE_NAMES[t], "m": m, "k": k, "us": us, "bytes": nbytes,
            "gbs": nbytes / (us * 1e-6) / 1e9, "frac_hbm": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "copies": copies}


GEMMS = [("C1 Q5_0 4864x896", 6, 4864, 896), ("C2 Q6_K 896x4864", 14, 896, 4864)]
BF16_PEAK_TFLOPS, F32_PEAK_TFLOPS = 2500.0, 157.3


def time_gemm(t: int, m: int, k: int, n: int, mode: int, launches: int, seed: int):
    rng = np.random.default_rng(seed)
    w = synth.weight_bytes(rng, t, m, k)
    x = synth.activations(rng, n, k)
    q = QMat.from_bytes(t, w, m, k)
    dx = hip.DeviceBuffer.from_array(x)
    dy = hip.DeviceBuffer(n * m * 4)
    s = hip.Stream()
    q.matmul_dev(dx, n, dy, mode, stream=s)     # eager first call sizes the split-K buffer
    s.synchronize()
    g = hip.Graph(s, lambda: [q.matmul_dev(dx, n, dy, mode, stream=s) for _ in range(launches)])
    g.launch()
    s.synchronize()
    e0, e1 = hip.Event(), hip.Event()
    e0.record(s)
    g.launch()
    e1.record(s)
    e1.synchronize()
    us = e0.elapsed_ms(e1) * 1e3 / launches
    g.destroy()
    q.close()
    s.destroy()
    flop = 2.0 * n * m * k
    tf = flop / (us * 1e-6) / 1e12
    peak = F32_PEAK_TFLOPS if mode == 1 else BF16_PEAK_TFLOPS
    return {"m": m, "k": k, "n": n, "mode": "f32" if mode == 1 else "bf16", "us": us, "tflops": tf,
            "frac_peak": tf / peak, "gbs": algorithmic_bytes(t, m, k) / (us * 1e-6) / 1e9}


def time_i8(m: int, k: int, n: int, launches: int, seed: int = 701):
    """Int8 activation path (kernel.rs:70-166): Q8_0 W[m x k] times n quantized activation rows,
    one launch of the i8 MFMA GEMM each (the quantize kernel timed apart), against the bf16 and
    f32 GEMMs on the same weights. Ops = 2 n m k."""
    from . import MODE_BF16, MODE_F32, Q8_0, quantize_q8_act_dev
    rng = np.random.default_rng(seed)
    w = synth.weight_bytes(rng, Q8_0, m, k)
    x = synth.activations(rng, n, k)
    q = QMat.from_bytes(Q8_0, w, m, k)
    dx = hip.DeviceBuffer.from_array(x)
    ds, dq, dy = hip.DeviceBuffer(n * (k // 32) * 4), hip.DeviceBuffer(n * k), hip.DeviceBuffer(n * m * 4)
    s = hip.Stream()

    def timed(body):
        body()
        s.synchronize()
        g = hip.Graph(s, lambda: [body() for _ in range(launches)])
        g.launch()
        s.synchronize()
        e0, e1 = hip.Event(), hip.Event()
        e0.record(s)
        g.launch()
        e1.record(s)
        e1.synchronize()
        g.destroy()
        return e0.elapsed_ms(e1) * 1e3 / launches

    us_q = timed(lambda: quantize_q8_act_dev(dx, n, k, ds, dq, stream=s))
    us_i8 = timed(lambda: q.matmul_i8_dev(ds, dq, n, dy, stream=s))
    us_bf16 = timed(lambda: q.matmul_dev(dx, n, dy, MODE_BF16, stream=s))
    us_f32 = timed(lambda: q.matmul_dev(dx, n, dy, MODE_F32, stream=s))
    q.close()
    s.destroy()
    ops = 2.0 * n * m * k
    return {"m": m, "k": k, "n": n, "us_quantize": us_q, "us_i8": us_i8, "tops_i8": ops / (us_i8 * 1e-6) / 1e12,
            "frac_int8_peak": ops / (us_i8 * 1e-6) / 1e12 / INT8_PEAK_TOPS, "us_bf16": us_bf16, "us_f32": us_f32,
            "gbs_i8": algorithmic_bytes(Q8_0, m, k) / (us_i8 * 1e-6) / 1e9}


MOE = {"n_experts": 128, "hidden": 2048, "inter": 768, "top_k": 8}


def time_moe(tokens: int, mode: int, reps: int, seed: int = 401):
    """Qwen3-30B-A3B-like expert FFN (config 4): Q4_K gate/up 768x2048, Q6_K down 2048x768 for
    128 experts, top-8 softmax routing of f32 N(0,1) logits. Times re_moe_forward_dev (host
    grouping + metadata upload + grouped GEMMs + SwiGLU + combine) per call."""
    import time as _time
    from . import MoeExperts, Q4_K, Q6_K
    E, H, I, k = MOE["n_experts"], MOE["hidden"], MOE["inter"], MOE["top_k"]
    rng = np.random.default_rng(seed)
    gate = np.concatenate([synth.weight_bytes(rng, Q4_K, I, H) for _ in range(E)])
    up = np.concatenate([synth.weight_bytes(rng, Q4_K, I, H) for _ in range(E)])
    down = np.concatenate([synth.weight_bytes(rng, Q6_K, H, I) for _ in range(E)])
    ids, wts, _ = synth.router(np.random.default_rng(seed + 1), tokens, E, k)
    x = synth.activations(np.random.default_rng(seed + 2), tokens, H)
    moe = MoeExperts(Q4_K, gate, Q4_K, up, Q6_K, down, E, H, I)
    dx = hip.DeviceBuffer.from_array(x)
    dy = hip.DeviceBuffer(tokens * H * 4)
    s = hip.Stream()
    moe.forward_dev(dx, tokens, k, ids, wts, dy, mode, stream=s)
    s.synchronize()
    t0 = _time.perf_counter()
    for _ in range(reps):
        moe.forward_dev(dx, tokens, k, ids, wts, dy, mode, stream=s)
    s.synchronize()
    us = (_time.perf_counter() - t0) / reps * 1e6
    # the same FFN with the routing on the device (ids/weights resident), and the whole layer
    # (f32 router matvec + top-k + FFN), each as a replayed graph of `reps` calls
    did = hip.DeviceBuffer.from_array(np.asarray(ids, np.int32))
    dw = hip.DeviceBuffer.from_array(np.asarray(wts, np.float32))
    rw = hip.DeviceBuffer.from_array((np.random.default_rng(seed + 3).standard_normal((E, H)) / np.sqrt(H))
                                     .astype(np.float32))
    e0, e1 = hip.Event(), hip.Event()

    def graph_us(fn):
        fn()
        s.synchronize()
        g = hip.Graph(s, lambda: [fn() for _ in range(reps)])
        g.launch()
        s.synchronize()
        e0.record(s)
        g.launch()
        e1.record(s)
        e1.synchronize()
        g.destroy()
        return e0.elapsed_ms(e1) * 1e3 / reps

    us_routed = graph_us(lambda: moe.forward_routed_dev(dx, tokens, k, did, dw, dy, mode, stream=s))
    from . import GATE_SOFTMAX
    us_layer = graph_us(lambda: moe.layer_dev(dx, tokens, rw, k, GATE_SOFTMAX, dy, mode, stream=s))
    moe.close()
    s.destroy()
    hit = len(np.unique(ids))
    per_expert = (gate.size + up.size + down.size) // E
    nbytes = hit * per_expert + 2 * tokens * H * 4
    flop = 2.0 * tokens * k * 3 * H * I
    return {"tokens": tokens, "pairs": tokens * k, "experts_hit": int(hit), "mode": "f32" if mode == 1 else "bf16",
            "us": us, "bytes": int(nbytes), "gbs": nbytes / (us * 1e-6) / 1e9,
            "frac_hbm": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, "tflops": flop / (us * 1e-6) / 1e12,
            "us_device_routed": us_routed, "gbs_device_routed": nbytes / (us_routed * 1e-6) / 1e9,
            "us_layer_device": us_layer}


def time_decode(prompt_len: int, steps: int, mode: int, seed: int = 501, use_graph: bool = True):
    """DeviceDecoder on the Qwen2.5-0.5B-shaped model: prefill, then `steps` graph replays back to
    back (the token never leaves the GPU), then `steps` replays with a token read-back each."""
    import time

    from . import qwen
    mb = qwen.synth_model(seed)
    prompt = np.random.default_rng(seed + 1).integers(0, mb.n_vocab, prompt_len)
    print(f"decode: model ready, prompt {prompt_len}, graph {use_graph}", flush=True)
    dd = qwen.DeviceDecoder(mb, max_seq=prompt_len + 2 * steps + 1, mode=mode, prefill_rows=prompt_len,
                            use_graph=use_graph)
    dd.prefill(prompt[:16])
    dd.close()
    dd = qwen.DeviceDecoder(mb, max_seq=prompt_len + 2 * steps + 1, mode=mode, prefill_rows=prompt_len,
                            use_graph=use_graph)
    print("decode: weights resident", flush=True)
    t0 = time.perf_counter()
    dd.prefill(prompt)
    t1 = time.perf_counter()
    print("decode: prefill done", flush=True)
    dd.step()                                    # graph capture
    t2 = time.perf_counter()
    print("decode: first step done", flush=True)
    if use_graph:
        dd.replay(steps)
    else:
        for _ in range(steps):
            dd.step()
    t3 = time.perf_counter()
    for _ in range(steps - 1):
        dd.step()
    t4 = time.perf_counter()
    dd.close()
    return {"prompt": prompt_len, "steps": steps, "mode": "bf16" if mode == 0 else "f32",
            "prefill_ms": 1e3 * (t1 - t0), "capture_ms": 1e3 * (t2 - t1),
            "step_us_device": 1e6 * (t3 - t2) / steps, "step_us_readback": 1e6 * (t4 - t3) / (steps - 1)}


def time_load(layers: int, workdir: str, seed: int = 601, variant_env=None):
    """GGUF ingest: a file of `layers` Qwen3-30B-A3B-shaped MoE layers (128 experts, hidden 2048,
    inter 768; Q4_K gate/up, Q6_K down: 309 MB a layer) is written, mapped and uploaded expert
    stack by expert stack (map -> pinned chunk -> device -> repack kernel). The file is in the page
    cache (just written), so this is the map-to-HBM rate, not a disk read; each pass maps the file
    afresh and pays its page faults. Beside it: a plain
    pageable hipMemcpy of the same bytes (the bus rate the upload is bound by) and the host repack
    (the same permutation on one CPU core)."""
    import os
    import time

    from . import MoeExperts, Gguf, Q4_K, Q6_K, repack
    import gguf_writer as W  # noqa: F401 (tests/gguf_writer.py)
    variant_env = variant_env or {}
    E, hidden, inter = 128, 2048, 768
    rng = np.random.default_rng(seed)
    per = {Q4_K: inter * hidden // 256 * 144 * E, Q6_K: hidden * inter // 256 * 210 * E}
    gu = rng.integers(0, 256, per[Q4_K], dtype=np.uint8).tobytes()
    dn = rng.integers(0, 256, per[Q6_K], dtype=np.uint8).tobytes()
    tensors = []
    for layer in range(layers):
        p = f"blk.{layer}."
        tensors += [(p + "ffn_gate_exps.weight", [hidden, inter, E], Q4_K, gu),
                    (p + "ffn_up_exps.weight", [hidden, inter, E], Q4_K, gu),
                    (p + "ffn_down_exps.weight", [inter, hidden, E], Q6_K, dn)]
    path = os.path.join(workdir, "load_bench.gguf")
    with open(path, "wb") as f:
        f.write(W.write([("general.architecture", W.STR, "qwen3moe")], tensors))
    total = layers * (2 * len(gu) + len(dn))
    print(f"load: wrote {total / 1e9:.2f} GB of expert tensors", flush=True)
    t0 = time.perf_counter()
    g = Gguf(path)
    t1 = time.perf_counter()
    g.close()

    def upload_all():
        # a fresh mapping each time: its pages fault in as the upload touches them
        ta = time.perf_counter()
        g = Gguf(path)
        moes = []
        for layer in range(layers):
            p = f"blk.{layer}."
            moes.append(MoeExperts.from_gguf(g, p + "ffn_gate_exps.weight", p + "ffn_up_exps.weight",
                                             p + "ffn_down_exps.weight", E, hidden, inter))
        tb = time.perf_counter()
        for m in moes:
            m.close()
        g.close()
        return tb - ta

    variants = {}
    for name, env in variant_env.items():
        old = {k: os.environ.get(k) for k in env}
        os.environ.update(env)
        variants[name] = total / upload_all() / 1e9
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
        print(f"load: {name} {variants[name]:.2f} GB/s", flush=True)
    t2 = time.perf_counter()
    up_s = upload_all()
    buf = hip.DeviceBuffer(len(gu))
    src = np.frombuffer(gu, np.uint8)
    buf.upload(src)
    t3 = time.perf_counter()
    for _ in range(3):
        buf.upload(src)
    t4 = time.perf_counter()
    g = Gguf(path)
    view = g.tensor_bytes("blk.0.ffn_gate_exps.weight")
    t7 = time.perf_counter()
    buf.upload(view)                             # pageable copy straight from a fresh mapping
    t8 = time.perf_counter()
    del view
    g.close()
    buf.free()
    one = gu[: per[Q4_K] // E]
    t5 = time.perf_counter()
    repack(Q4_K, one, inter, hidden)
    t6 = time.perf_counter()
    os.remove(path)
    return {"layers": layers, "bytes": total, "open_ms": 1e3 * (t1 - t0), "upload_s": up_s,
            "gbs": total / up_s / 1e9, "variants": variants, "memcpy_pageable_gbs": 3 * len(gu) / (t4 - t3) / 1e9,
            "memcpy_from_map_gbs": len(gu) / (t8 - t7) / 1e9,
            "host_repack_gbs": len(one) / (t6 - t5) / 1e9}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--types", default="Q4_0,Q5_0,Q8_0,Q4_K,Q5_K,Q6_K")
    ap.add_argument("--launches", type=int, default=300)
    ap.add_argument("--only", default="", help="comma list of projection names")
    ap.add_argument("--json", default="")
    ap.add_argument("--gemm", action="store_true", help="time the prefill GEMMs instead")
    ap.add_argument("--moe", action="store_true", help="time the MoE expert FFN (config 4) instead")
    ap.add_argument("--rows", default="64,961", help="GEMM activation-row counts")
    ap.add_argument("--modes", default="bf16,f32", help="GEMM modes")
    ap.add_argument("--decode", action="store_true", help="time the device-resident decoder instead")
    ap.add_argument("--prompt", type=int, default=961, help="decoder prompt length")
    ap.add_argument("--steps", type=int, default=128, help="decoder steps")
    ap.add_argument("--no-graph", action="store_true", help="decoder steps launched eagerly")
    ap.add_argument("--i8", action="store_true", help="time the int8 activation GEMM instead")
    ap.add_argument("--load", type=int, default=0, help="time GGUF ingest of this many MoE layers instead")
    ap.add_argument("--workdir", default="/tmp", help="where --load writes its GGUF file")
    ap.add_argument("--load-variants", default="", help="name:ENV=v,ENV=v;... upload settings timed first")
    args = ap.parse_args(argv)
    init()
    if args.i8:
        rows = []
        for m, k in ((4864, 896), (896, 4864)):
            for n in (int(v) for v in args.rows.split(",") if v):
                r = time_i8(m, k, n, launches=50 if n > 64 else 200)
                rows.append(r)
                print(f"i8 Q8_0 {m}x{k} N={n:4d}: quantize {r['us_quantize']:7.2f} us | i8 GEMM {r['us_i8']:8.2f} us "
                      f"{r['tops_i8']:7.1f} TOP/s ({100 * r['frac_int8_peak']:4.1f}% of int8) "
                      f"{r['gbs_i8']:7.1f} GB/s | bf16 {r['us_bf16']:8.2f} us | f32 {r['us_f32']:8.2f} us", flush=True)
        if args.json:
            with open(args.json, "w") as f:
                json.dump(rows, f, indent=1)
        return 0
    if args.load:
        venv = {}
        for spec in filter(None, args.load_variants.split(";")):
            name, _, kv = spec.partition(":")
            venv[name] = dict(item.split("=", 1) for item in kv.split(",") if item)
        r = time_load(args.load, args.workdir, variant_env=venv)
        print(f"load {r['layers']} layers {r['bytes'] / 1e9:.2f} GB: open {r['open_ms']:.2f} ms, map -> HBM "
              f"{r['upload_s']:.3f} s = {r['gbs']:.2f} GB/s | pageable hipMemcpy {r['memcpy_pageable_gbs']:.2f} GB/s "
              f"(from a fresh mapping {r['memcpy_from_map_gbs']:.2f} GB/s) | host repack (1 core) "
              f"{r['host_repack_gbs']:.2f} GB/s", flush=True)
        if args.json:
            with open(args.json, "w") as f:
                json.dump(r, f, indent=1)
        return 0
    if args.decode:
        for mode in [{"bf16": 0, "f32": 1}[v] for v in args.modes.split(",") if v]:
            r = time_decode(args.prompt, args.steps, mode, use_graph=not args.no_graph)
            print(f"decode prompt={r['prompt']} {r['mode']:4s} prefill {r['prefill_ms']:8.2f} ms "
                  f"capture {r['capture_ms']:7.2f} ms step {r['step_us_device']:8.1f} us (device) "
                  f"{r['step_us_readback']:8.1f} us (with read-back)", flush=True)
        return 0
    only = set(filter(None, args.only.split(",")))
    if args.moe:
        rows = []
        for tokens in (1, 32, 512):
            for mode in (0, 1):
                r = time_moe(tokens, mode, reps=50 if tokens < 512 else 20)
                rows.append(r)
                print(f"MoE T={tokens:4d} pairs={r['pairs']:5d} experts={r['experts_hit']:3d} {r['mode']:4s} "
                      f"{r['us']:9.1f} us {r['gbs']:8.1f} GB/s ({100 * r['frac_hbm']:5.1f}% of HBM) "
                      f"{r['tflops']:7.2f} TFLOP/s | device-routed {r['us_device_routed']:8.1f} us "
                      f"{r['gbs_device_routed']:8.1f} GB/s ({100 * r['gbs_device_routed'] / HBM_PEAK_GBS:5.1f}%) "
                      f"| layer incl. router {r['us_layer_device']:8.1f} us", flush=True)
        if args.json:
            with open(args.json, "w") as f:
                json.dump(rows, f, indent=1)
        return 0
    if args.gemm:
        rows = []
        ns = [int(v) for v in args.rows.split(",") if v]
        modes = [{"bf16": 0, "f32": 1}[v] for v in args.modes.split(",") if v]
        for name, t, m, k in GEMMS:
            if only and not any(o in name for o in only):
                continue
            for n in ns:
                for mode in modes:
                    r = time_gemm(t, m, k, n, mode, max(20, args.launches // 10), seed=101 + n)
                    r["name"] = name
                    rows.append(r)
                    print(f"{name:18s} N={n:4d} {r['mode']:4s} {r['us']:9.2f} us {r['tflops']:8.2f} TFLOP/s "
                          f"({100 * r['frac_peak']:5.2f}% of {r['mode']} peak)", flush=True)
        if args.json:
            with open(args.json, "w") as f:
                json.dump(rows, f, indent=1)
        return 0
    by_name = {v: k for k, v in TYPE_NAMES.items()}
    types = [by_name[s] for s in args.types.split(",") if s]
    rows = []
    for ti, t in enumerate(types):
        for pi, (name, m, k) in enumerate(PROJECTIONS):
            if only and name not in only:
                continue
            r = time_gemv(t, m, k, args.launches, seed=300 + 10 * pi + t)
            r["proj"] = name
            rows.append(r)
            print(f"{r['type']:5s} {name:8s} {m:6d}x{k:<5d} {r['us']:8.2f} us {r['gbs']:8.1f} GB/s "
                  f"({100 * r['frac_hbm']:5.1f}% of HBM)", flush=True)
    if args.json:
        with open(args.json, "w") as f:
            json.dump(rows, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
