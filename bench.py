"""Benchmark of the MI355X W4A16 hot path. Prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--layers 64] [--no-cpu]

Headline: the decode GEMV sweep of a full layer --
qkv (5120->7168), o (4096->5120), gate|up (5120->34816), down (17408->5120) --
over 64 layers of distinct synthetic weights (10.07 GiB of algorithmic bytes,
far beyond the 256 MB MALL). One step = one decoded token's body: all 256 GEMV
launches (M=1). value = algorithmic bytes / time (GB/s), inputs resident in HBM.

Also reported (in "extra"): config 1 (single 5120x5120 GEMV), config 3 (verify
M=9/12/16 over the same 64-layer sweep), config 4 (prefill GEMM TFLOPS at
M=512/1024/4096), config 5 (lm_head 248320x5120 + fused argmax, M=1/9), the
measured streaming-read HBM bandwidth, and the CPU baseline (the oracle's port
of the reference's host dequant+matmul) on a bounded sample.

Algorithmic bytes (4-bit zeros): K*N/2 + (K/128)*N*2 + (K/128)*N/2 + M*K*2 + M*N*2.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwen38-3090-cuda-server_amd"))

METRIC = "decode GEMV GB/s (% of HBM peak) per layer; prefill GEMM TFLOPS at M=4096"
HBM_PEAK_GBS = 8000.0          # MI355X published HBM3E bandwidth
BF16_PEAK_TFLOPS = 2500.0      # MI355X published dense bf16 MFMA
LAYER = (("qkv", 5120, 7168), ("o_proj", 4096, 5120), ("gate|up", 5120, 34816),
         ("down", 17408, 5120))


def alg_bytes(M: int, K: int, N: int, out: bool = True) -> int:
    G = K // 128
    return K * N // 2 + G * N * 2 + G * N // 2 + M * K * 2 + (M * N * 2 if out else M * 4)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Timer:
    """HIP events on the stream the kernels are launched on."""

    def __init__(self, torch):
        self.torch = torch
        self.stream = torch.cuda.current_stream()

    def event(self):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record(self.stream)
        return e


def make_weights(hip, torch, N, K, seed, tensor, tmp):
    """Generate one AWQ-layout tensor on the GPU and repack it."""
    qw, sc, zr = tmp
    G = K // 128
    q = qw[: K // 8 * N]
    s = sc[: G * N]
    z = zr[: G * N // 8]
    assert q.numel() == K // 8 * N and s.numel() == G * N and z.numel() == G * N // 8, \
        "generator staging buffers too small"
    hip.gen_awq_k(q, s, z, N, K, seed, tensor)
    w = hip.awq_alloc_fused(N, K)
    hip.awq_repack_awq_into(w, 0, q, s, z, N, hip.LAYOUT_AWQ_K)
    return w


def cpu_baseline(budget_s: float = 12.0):
    """Oracle port of the reference's host dequant+matmul on one decode layer (M=1)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc

    threads = orc.nthreads()
    layer = []
    for t, (name, K, N) in enumerate(LAYER):
        q, zp, s = orc.gen_weights(N, K, seed=0, tensor=100 + t)
        layer.append((K, N, orc.pack_ct(q, zp, s), orc.gen_x(1, K, seed=0, tensor=100 + t)))
        del q, zp, s
    byts = sum(alg_bytes(1, K, N) for K, N, _, _ in layer)
    reps, t0 = 0, time.perf_counter()
    while True:
        for K, N, packed, x in layer:
            orc.cpu_w4a16_matmul(x, *packed, N, K, threads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 200:
            break
    gbs = byts * reps / el / 1e9
    # prefill sample: M=64 rows of the gate projection (17408x5120), fp32 accumulate
    q, zp, s = orc.gen_weights(17408, 5120, seed=0, tensor=120)
    packed = orc.pack_ct(q, zp, s)
    x = orc.gen_x(64, 5120, seed=0, tensor=120)
    t1 = time.perf_counter()
    orc.cpu_w4a16_matmul(x, *packed, 17408, 5120, threads=threads)
    pf = 2.0 * 64 * 17408 * 5120 / (time.perf_counter() - t1) / 1e12
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"one decode layer (qkv, o, gate|up, down; M=1, 161 MiB) x {reps} "
                      f"repeats in {el:.1f} s, A0 tensors, fp32 accumulate",
            "prefill_tflops_m64_gate": round(pf, 4)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only-decode", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the W4A16 path is single-GPU; "
              "multi-GPU sharding is a design note, not a measured mode). Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import w4a16_hip as hip

    hip.lib()
    torch.cuda.set_device(0)
    T = Timer(torch)
    extra = {}

    # ---------------------------------------------------------------- inputs
    log("generating weights ...")
    # generator staging buffers sized for every (K, N) this run creates
    shapes = [(K, N) for _, K, N in LAYER] + [(5120, 5120), (5120, 248320), (5120, 17408),
                                               (17408, 5120)]
    kn = max(K * N for K, N in shapes)
    tmp = (torch.empty(kn // 8, dtype=torch.int32, device="cuda"),
           torch.empty(kn // 128, dtype=torch.int16, device="cuda"),
           torch.empty(kn // 1024, dtype=torch.int32, device="cuda"))
    layers = []
    for l in range(args.layers):
        layers.append([make_weights(hip, torch, N, K, 0, 8 * l + t, tmp)
                       for t, (_, K, N) in enumerate(LAYER)])
    scratch = hip.gemv_scratch_alloc(17408, 248320, 128, 16)
    xs = {}
    for K in (4096, 5120, 17408):
        x = torch.empty((16, K), dtype=torch.int16, device="cuda")
        hip.gen_bf16(x, 16 * K, 0, 1000 + K, 0)
        xs[K] = x
    ys = torch.empty((16, 34816), dtype=torch.int16, device="cuda")
    torch.cuda.synchronize()
    step_bytes = sum(alg_bytes(1, K, N) for _, K, N in LAYER) * args.layers

    def step(M=1, per_launch=None):
        for lw in layers:
            for (name, K, N), w in zip(LAYER, lw):
                if per_launch is not None:
                    e0 = torch.cuda.Event(enable_timing=True, external=True)
                    e0.record()
                if M == 1:
                    hip.gemv_w4a16(ys, w, xs[K], scratch)
                else:
                    hip.gemm_small_w4a16(ys, w, xs[K], M, scratch)
                if per_launch is not None:
                    e1 = torch.cuda.Event(enable_timing=True, external=True)
                    e1.record()
                    per_launch.append((name, e0, e1))

    def capture(fn):
        """One decode step as a hipGraph (the reference replays its decode step
        as a CUDA graph, src/model/model.cu:880-946): no host launch gaps."""
        fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        g.replay()
        torch.cuda.synchronize()
        return g

    def time_graph(g, iters):
        a = T.event()
        for _ in range(iters):
            g.replay()
        b = T.event()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / iters

    # ------------------------------------------------- headline: config 2
    g_step = capture(step)
    for _ in range(args.warmup):
        g_step.replay()
    torch.cuda.synchronize()
    e0 = T.event()
    for _ in range(args.steps):
        g_step.replay()
    e1 = T.event()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    value = step_bytes / (ms * 1e-3) / 1e9
    log(f"config2: {ms:.3f} ms/step, {value:.1f} GB/s")

    # per-launch kernel durations of the same sweep: timing events captured
    # around every launch inside a second graph
    per = {}
    try:
        rec = []
        g_prof = capture(lambda: step(per_launch=rec))
        rec_last = rec[-len(LAYER) * args.layers:]
        for _ in range(3):
            g_prof.replay()
            torch.cuda.synchronize()
            for name, a, b in rec_last:
                per.setdefault(name, []).append(a.elapsed_time(b))
        extra["kernel_timing"] = "HIP events captured around each launch in a graph"
    except Exception as exc:  # event nodes unsupported: per-shape graphs
        log(f"per-launch events in graph unavailable ({exc}); timing per-shape graphs")
        per = {}
        for li, (name, K, N) in enumerate(LAYER):
            g1 = capture(lambda: [hip.gemv_w4a16(ys, lw[li], xs[K], scratch) for lw in layers])
            t = time_graph(g1, 3)
            per[name] = [t / len(layers)] * len(layers)
        extra["kernel_timing"] = "per-shape graphs of 64 launches (includes inter-kernel gaps)"
    tot_ms, tot_bytes, launches = 0.0, 0, 0
    per_op = {}
    for name, K, N in LAYER:
        d = sum(per[name]) / len(per[name])
        b = alg_bytes(1, K, N)
        per_op[name] = {"K": K, "N": N, "us": round(d * 1e3, 2),
                        "GBps": round(b / (d * 1e-3) / 1e9, 1),
                        "splits": hip.gemv_choose_splits(N, K // 128)}
        tot_ms += sum(per[name])
        tot_bytes += b * len(per[name])
        launches += len(per[name])
    kernel_gbs = tot_bytes / (tot_ms * 1e-3) / 1e9
    extra["config2_per_projection"] = per_op
    extra["config2_launches_per_step"] = 4 * args.layers
    extra["config2_kernel_only_GBps"] = round(kernel_gbs, 1)

    # ---------------------------------------------------- HBM read microbench
    buf = torch.empty(4 << 30, dtype=torch.uint8, device="cuda")
    sink = torch.empty(8192, dtype=torch.int32, device="cuda")
    for _ in range(2):
        hip.stream_read(buf, buf.numel(), sink, 8192)
    a = T.event()
    for _ in range(5):
        hip.stream_read(buf, buf.numel(), sink, 8192)
    b = T.event()
    torch.cuda.synchronize()
    hbm = 5 * buf.numel() / (a.elapsed_time(b) * 1e-3) / 1e9
    del buf
    extra["measured_hbm_read_GBps"] = round(hbm, 1)
    extra["config2_frac_of_measured_hbm"] = round(value / hbm, 4)
    log(f"stream read {hbm:.1f} GB/s")

    if not args.only_decode:
        # ---------------------------------------------------------- config 1
        w1 = make_weights(hip, torch, 5120, 5120, 0, 9001, tmp)
        g1 = capture(lambda: [hip.gemv_w4a16(ys, w1, xs[5120], scratch) for _ in range(100)])
        us = time_graph(g1, 5) / 100 * 1e3
        extra["config1"] = {"us_per_call": round(us, 2),
                            "GBps": round(alg_bytes(1, 5120, 5120) / (us * 1e-6) / 1e9, 1),
                            "note": "13.6 MB, 100 calls in one graph: MALL-resident"}
        hip.awq_free(w1)

        # ---------------------------------------------------------- config 3
        c3 = {}
        for M in (9, 12, 16):
            gM = capture(lambda: step(M))
            msM = time_graph(gM, 5)
            byM = sum(alg_bytes(M, K, N) for _, K, N in LAYER) * args.layers
            c3[f"M{M}"] = {"ms_per_sweep": round(msM, 3), "GBps": round(byM / (msM * 1e-3) / 1e9, 1),
                           "x_of_M1": round(msM / ms, 3)}
            del gM
        extra["config3_verify"] = c3
        log(f"config3: {c3}")

        # ---------------------------------------------------------- config 5
        wl = make_weights(hip, torch, 248320, 5120, 0, 9002, tmp)
        idx = torch.empty(16, dtype=torch.int32, device="cuda")
        c5 = {}
        for M in (1, 9):
            g5 = capture(lambda: [hip.gemv_argmax_w4a16(idx, wl, xs[5120], M, scratch)
                                  for _ in range(10)])
            us = time_graph(g5, 3) / 10 * 1e3
            bts = alg_bytes(M, 5120, 248320, out=False)
            c5[f"M{M}"] = {"us_per_call": round(us, 2), "GBps": round(bts / (us * 1e-6) / 1e9, 1)}
            del g5
        extra["config5_lm_head_argmax"] = c5
        hip.awq_free(wl)
        log(f"config5: {c5}")

        # ---------------------------------------------------------- config 4
        c4 = {}
        A = torch.empty((4096, 17408), dtype=torch.int16, device="cuda")
        hip.gen_bf16(A, A.numel(), 0, 4242, 0)
        C = torch.empty((4096, 17408), dtype=torch.int16, device="cuda")
        prefill_kernel_ms = {}
        for name, K, N in (("gate", 5120, 17408), ("down", 17408, 5120)):
            wg = make_weights(hip, torch, N, K, 0, 9100 + K, tmp)
            for M in (512, 1024, 4096):
                hip.gemm_w4a16(C, wg, A, M)
                torch.cuda.synchronize()
                it = 10 if M == 4096 else 20
                a = T.event()
                for _ in range(it):
                    hip.gemm_w4a16(C, wg, A, M)
                b = T.event()
                torch.cuda.synchronize()
                msg = a.elapsed_time(b) / it
                tf = 2.0 * M * N * K / (msg * 1e-3) / 1e12
                c4[f"{name}_M{M}"] = {"ms": round(msg, 3), "TFLOPS": round(tf, 1),
                                      "frac_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4)}
                if M == 4096:
                    prefill_kernel_ms[name] = (msg, 2.0 * M * N * K)
            hip.awq_free(wg)
        extra["config4_prefill"] = c4
        fl = sum(v[1] for v in prefill_kernel_ms.values())
        tm = sum(v[0] for v in prefill_kernel_ms.values())
        pf_tf = fl / (tm * 1e-3) / 1e12
        extra["prefill_M4096_TFLOPS"] = round(pf_tf, 1)
        extra["roofline_prefill"] = {"bound": "mfma", "achieved": round(pf_tf, 1),
                                     "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                     "frac": round(pf_tf / BF16_PEAK_TFLOPS, 4), "traffic": None,
                                     "kernel": "k_gemm (M=4096, gate 17408x5120 + down 5120x17408)"}
        log(f"config4: {c4}")

    cpu = None if args.no_cpu else cpu_baseline()
    avg_bytes = tot_bytes / launches
    avg_ms = tot_ms / launches
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "BASELINE config 2: decode GEMV sweep, M=1, "
                               f"{args.layers} layers x (qkv 5120->7168, o 4096->5120, "
                               "gate|up 5120->34816, down 17408->5120), INT4 g128, "
                               "bf16 activations", "layers": args.layers,
                   "bytes_per_step": step_bytes, "weights": "W4A16 g128 (AWQ_K source, repacked)"},
        "roofline": {"bound": "hbm", "achieved": round(avg_bytes / (avg_ms * 1e-3) / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(avg_bytes / (avg_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": None,
                     "kernel": "k_skinny<0> (decode GEMV), avg over the sweep's 4 shapes",
                     "alg_bytes_per_launch": round(avg_bytes), "avg_launch_us": round(avg_ms * 1e3, 3)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
