"""Benchmark of the fused GGUF dequant-matmul on one MI355X.

Workload (the configuration the headline metric is quoted on): the Q6_K down projection
W[896 x 4864] (K = 4864, 256-element super-blocks of 210 B) with f32 activations X[N x 4864],
N = 1 (decode GEMV), 64 and 961 (prefill GEMM). Synthetic, seeded (numpy PCG64, seed 201 + N),
inputs resident in HBM before timing.

A "step" is one batched N = 1 GEMV launch over a stack of copies of W (> 512 MiB in all, so
every byte comes from HBM, not from the 256 MiB MALL): y_b = W_b x for every copy b, one
launch (re_qmat_matvec_stacked_dev). The timed region replays a HIP graph of `steps` such
launches. `value` = algorithmic bytes per launch (per copy: stored GGUF weight bytes + f32 x +
f32 y) / average launch time. A single 3.6 MB GEMV is bounded by the per-launch floor of a few
microseconds, not by HBM; its latency (one copy per launch, rotating over the copies) is
reported separately under "single_launch". The N = 961 and N = 64 GEMMs (bf16 MFMA mode) are
timed as graphs of single launches and reported under "gemm".

The CPU baseline is the oracle's restatement of the reference's pooled AVX2 kernels
(matmul_reuse + QMat split policy + persistent pool), timed on this host on a bounded sample.

Prints one JSON line.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "rusty-engine_amd"))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
F32_MFMA_PEAK_TFLOPS = 157.3
M, K = 896, 4864
MALL_BYTES = 256 << 20


def measured_traffic():
    """HBM bytes per batched GEMV launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE passes
    (profiles/gemv_q6k_896x4864_stacked_traffic.txt, copy-calibrated), or None."""
    path = os.path.join(ROOT, "profiles", "gemv_q6k_896x4864_stacked_traffic.txt")
    try:
        for line in open(path):
            if line.startswith("gemv_traffic_bytes_per_launch="):
                return int(line.split("=")[1].split()[0])
    except OSError:
        pass
    return None


def algorithmic_bytes(t, m, k, n):
    import rehip
    qk, bb = rehip.GEOM[t]
    return m * k // qk * bb + 4 * n * k + 4 * n * m


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--single-steps", type=int, default=2000, help="launches of the single-GEMV latency run")
    ap.add_argument("--gemm-steps", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="bound on the CPU-baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-e2e", action="store_true", help="skip the end-to-end decoder run")
    ap.add_argument("--e2e-steps", type=int, default=256, help="greedy decode steps of the end-to-end run")
    ap.add_argument("--e2e-cpu-steps", type=int, default=64,
                    help="decode steps of the CPU-matmul end-to-end run (parity and CPU tok/s)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="first run one 256 MiB device-to-device copy (calibrates profiler byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import rehip
    from rehip import hip, synth

    t = rehip.Q6_K
    rehip.init()
    stream = hip.Stream()
    if args.copy_probe:
        src, dst = hip.DeviceBuffer(256 << 20), hip.DeviceBuffer(256 << 20)
        hip.check(hip.hip().hipMemcpy(hip.C.c_void_p(dst.ptr), hip.C.c_void_p(src.ptr), 256 << 20, hip.D2D))
        hip.synchronize()
        src.free()
        dst.free()

    # ---- N = 1 GEMV: batched launches over a stack of weight copies ---------------------------
    rng = np.random.default_rng(201 + 1)
    w = synth.weight_bytes(rng, t, M, K)
    x1 = synth.activations(rng, 1, K)
    copies = int(np.ceil(2 * MALL_BYTES / w.size))
    stack = rehip.QMat.from_bytes_stacked(t, np.tile(w, copies), M, K, copies)
    dx = hip.DeviceBuffer.from_array(x1)
    dy = hip.DeviceBuffer(copies * M * 4)
    steps, warmup = args.steps, args.warmup

    def batched(n):
        for _ in range(n):
            stack.matvec_stacked_dev(0, copies, dx, 0, dy, M, stream=stream)

    e0, e1 = hip.Event(), hip.Event()

    def timed(fn_warm, fn_timed, n):
        gw = hip.Graph(stream, fn_warm)
        gt = hip.Graph(stream, fn_timed)
        gw.launch()
        stream.synchronize()
        e0.record(stream)
        gt.launch()
        e1.record(stream)
        e1.synchronize()
        gw.destroy()
        gt.destroy()
        return e0.elapsed_ms(e1) / n

    gemv_ms = timed(lambda: batched(warmup), lambda: batched(steps), steps)
    # parity spot check of the timed kernel against the oracle: every copy's output
    ys = dy.download(np.float32, copies * M).reshape(copies, M)
    import oracle
    y_ref = oracle.qmat_matvec(t, w, M, K, x1)
    absd = oracle.qmat_absdot(t, w, M, K, x1, 1)
    parity_ok = bool(np.all(np.abs(ys - y_ref[None, :]) <= 2.0 ** -10 * absd[None, :]))
    per_copy = algorithmic_bytes(t, M, K, 1)
    gemv_bytes = per_copy * copies
    gemv_gbs = gemv_bytes / (gemv_ms * 1e-3) / 1e9

    # single-launch latency: one copy per launch, rotating over the stack
    ns = args.single_steps

    def singles(n):
        for i in range(n):
            stack.matvec_stacked_dev(i % copies, 1, dx, 0, dy, M, stream=stream)

    single_ms = timed(lambda: singles(min(ns, 200)), lambda: singles(ns), ns)
    stack.close()

    # ---- N = 64 and N = 961 GEMM (bf16 MFMA) -----------------------------------------------------
    gemm = {}
    for n in (64, 961):
        rng = np.random.default_rng(201 + n)
        wn = synth.weight_bytes(rng, t, M, K)
        xn = synth.activations(rng, n, K)
        q = rehip.QMat.from_bytes(t, wn, M, K)
        dxn = hip.DeviceBuffer.from_array(xn)
        dyn = hip.DeviceBuffer(n * M * 4)
        gs = args.gemm_steps
        q.matmul_dev(dxn, n, dyn, rehip.MODE_BF16, stream=stream)     # sizes the split-K buffer
        stream.synchronize()
        g = hip.Graph(stream, lambda: [q.matmul_dev(dxn, n, dyn, rehip.MODE_BF16, stream=stream) for _ in range(gs)])
        g.launch()
        stream.synchronize()
        e0.record(stream)
        g.launch()
        e1.record(stream)
        e1.synchronize()
        ms = e0.elapsed_ms(e1) / gs
        g.destroy()
        flops = 2.0 * n * M * K
        nbytes = algorithmic_bytes(t, M, K, n)
        y = dyn.download()
        deq = oracle.dequant(t, wn).reshape(M, K).astype(np.float64)
        exact = (xn.reshape(n, K).astype(np.float64) @ deq.T).reshape(-1)
        rel = float(np.linalg.norm(y - exact) / np.linalg.norm(exact))
        gemm[f"n{n}"] = {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12, "gbs": nbytes / (ms * 1e-3) / 1e9,
                         "frac_bf16_peak": flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
                         "frac_hbm_peak": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                         "rel_err_vs_f64": rel, "flop": flops, "bytes": nbytes}
        q.close()

    # ---- CPU baseline (reference-restated pooled AVX2 kernels) on a bounded sample --------------
    cpu = None
    if not args.no_cpu and oracle.cpu_has_avx2():
        threads = int(os.environ.get("RE_THREADS", "0")) or min(os.cpu_count() or 1, 16)
        oracle.cpu_matvec(t, w, M, K, x1, threads)
        budget = args.cpu_seconds / 2
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget:
            oracle.cpu_matvec(t, w, M, K, x1, threads)
            reps += 1
        cpu_gemv_s = (time.perf_counter() - t0) / reps
        rng = np.random.default_rng(201 + 961)
        wn = synth.weight_bytes(rng, t, M, K)
        xn = synth.activations(rng, 961, K)
        oracle.cpu_matmul(t, wn, M, K, xn, 961, threads)
        reps2, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget:
            oracle.cpu_matmul(t, wn, M, K, xn, 961, threads)
            reps2 += 1
        cpu_gemm_s = (time.perf_counter() - t0) / reps2
        cpu = {"value": per_copy / cpu_gemv_s / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"Q6_K 896x4864: N=1 GEMV x{reps} ({cpu_gemv_s * 1e3:.3f} ms each), "
                         f"N=961 GEMM x{reps2} ({cpu_gemm_s * 1e3:.1f} ms each = "
                         f"{2.0 * 961 * M * K / cpu_gemm_s / 1e9:.1f} GFLOP/s)",
               "n961_gflops": 2.0 * 961 * M * K / cpu_gemm_s / 1e9}

    e2e = None if args.no_e2e else run_e2e(args, cpu_ok=not args.no_cpu and oracle.cpu_has_avx2())

    out = {
        "metric": "Q-matmul GB/s (N=1) & TFLOP/s (N=961) as % roofline; decode tok/s",
        "value": round(gemv_gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": gemv_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded PCG64 GGUF Q6_K blocks, finite f16 scales; X ~ N(0,1))",
        "config": {"workload": "Q6_K down projection W[896x4864], X[N x 4864] f32: N=1 GEMV batched over "
                               f"{copies} weight copies per launch (+ N=64/961 GEMM)",
                   "weight_copies_per_launch": copies, "graph_replay": True},
        "roofline": {"bound": "hbm", "achieved": round(gemv_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gemv_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "algorithmic_bytes_per_launch": gemv_bytes, "avg_launch_us": gemv_ms * 1e3},
        "single_launch": {"us": single_ms * 1e3, "gbs": per_copy / (single_ms * 1e-3) / 1e9,
                          "frac_hbm": per_copy / (single_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                          "note": "one 3.6 MB GEMV per launch, back to back in a graph: bounded by the "
                                  "per-launch floor, not HBM"},
        "gemm": gemm,
        "parity_ok": parity_ok and all(v["rel_err_vs_f64"] <= 1e-2 for v in gemm.values()),
        "cpu_baseline": cpu,
        "e2e": e2e,
    }
    if e2e and e2e.get("greedy_identical") is False:
        out["parity_ok"] = False
    print(json.dumps(out))


def run_e2e(args, cpu_ok):
    """Seeded random-init Qwen2.5-0.5B-shaped model (24 layers, Q4_K_M mix): 961-token prefill and
    greedy decode with every projection on the GPU (f32 mode), the host steps on the CPU; then the
    same with the reference-restated CPU kernels for the first e2e_cpu_steps tokens."""
    import rehip
    from rehip import qwen

    mb = qwen.synth_model(501)
    prompt = np.random.default_rng(502).integers(0, mb.n_vocab, 961)

    def decode(backend, steps):
        r = qwen.DenseRunner(mb, backend)
        dec = qwen.DenseDecoder(r, len(prompt) + steps)
        t0 = time.perf_counter()
        logits = dec.prefill(prompt)
        t1 = time.perf_counter()
        toks = [qwen.argmax_last(logits)]
        for _ in range(steps - 1):
            toks.append(qwen.argmax_last(dec.step(toks[-1])))
        t2 = time.perf_counter()
        if hasattr(r, "close"):
            r.close()
        return toks, t1 - t0, (steps - 1) / (t2 - t1) if steps > 1 else None

    def device_decode(steps, mode):
        """DeviceDecoder: everything on the GPU, one graph replay per token. Two rates: with a
        4-byte token read-back after every step, and with the steps replayed back to back (the
        tokens read from the device history at the end). The first step (which captures the
        graph) is in neither rate."""
        ms = len(prompt) + steps + 1
        dd = qwen.DeviceDecoder(mb, max_seq=ms, mode=mode, prefill_rows=len(prompt))
        dd.prefill(prompt[:32])                    # warm-up: GEMM scratch is allocated here
        dd.close()
        dd = qwen.DeviceDecoder(mb, max_seq=ms, mode=mode, prefill_rows=len(prompt))
        t0 = time.perf_counter()
        toks = [dd.prefill(prompt)]
        t1 = time.perf_counter()
        toks.append(dd.step())
        t2 = time.perf_counter()
        for _ in range(steps - 2):
            toks.append(dd.step())
        t3 = time.perf_counter()
        dd.close()
        dd = qwen.DeviceDecoder(mb, max_seq=ms, mode=mode, prefill_rows=len(prompt))
        dd.prefill(prompt)
        dd.step()
        t4 = time.perf_counter()
        dd.replay(steps - 2)
        t5 = time.perf_counter()
        replay_toks = dd.history(len(prompt), steps)
        dd.close()
        return toks, t1 - t0, (steps - 2) / (t3 - t2), (steps - 2) / (t5 - t4), replay_toks == toks

    dtoks, dpre_s, dtps, dtps_replay, replay_same = device_decode(args.e2e_steps, rehip.MODE_F32)
    _, dpre_bf16, _, _, _ = device_decode(3, rehip.MODE_BF16)
    toks, pre_s, tps = decode(qwen.HipBackend(rehip.MODE_F32), args.e2e_steps)
    res = {"model": "Qwen2.5-0.5B-shaped (24 layers, 896/14/2 heads, d_ff 4864, vocab 151936), Q4_K_M mix, "
                    "random init seed 501",
           "prompt_tokens": len(prompt), "decode_steps": args.e2e_steps, "matmul_mode": "f32",
           "prefill_s_hip": pre_s, "decode_tok_s_hip": tps,
           "host_steps": "attention/norm/RoPE/argmax on the host (numpy), projections through the backend",
           "device_resident": {"prefill_s": dpre_s, "prefill_s_bf16_gemm": dpre_bf16, "decode_tok_s": dtps,
                               "decode_tok_s_replay": dtps_replay,
                               "greedy_identical_to_host_step_path": dtoks == toks and replay_same,
                               "note": "attention, norms, RoPE, argmax and residuals on the GPU; one HIP graph "
                                       "replay per decode step; decode_tok_s reads the token back after every "
                                       "step, decode_tok_s_replay replays the steps back to back"}}
    if cpu_ok:
        from oracle.backend import CpuBackend
        n = min(args.e2e_cpu_steps, args.e2e_steps)
        ctoks, cpre_s, ctps = decode(CpuBackend(), n)
        res.update({"prefill_s_cpu": cpre_s, "decode_tok_s_cpu": ctps, "cpu_decode_steps": n,
                    "greedy_identical": ctoks == toks[:n] and ctoks == dtoks[:n], "greedy_compared_steps": n})
    return res


if __name__ == "__main__":
    main()
