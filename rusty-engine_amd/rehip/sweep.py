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


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--types", default="Q4_0,Q5_0,Q8_0,Q4_K,Q5_K,Q6_K")
    ap.add_argument("--launches", type=int, default=300)
    ap.add_argument("--only", default="", help="comma list of projection names")
    ap.add_argument("--json", default="")
    ap.add_argument("--gemm", action="store_true", help="time the prefill GEMMs instead")
    args = ap.parse_args(argv)
    init()
    if args.gemm:
        rows = []
        for name, t, m, k in GEMMS:
            for n in (64, 961):
                for mode in (0, 1):
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
    only = set(filter(None, args.only.split(",")))
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
