"""Benchmark of the Q4_K / Q6_K MUL_MAT and MUL_MAT_ID path on one MI355X.

Headline (value): HBM GB/s of weight bytes of the batch-1 decode GEMV on the Q6_K output head
151936 x 2048 (255,252,480 weight bytes), one step = one MUL_MAT including the Q8_K quantization of
the activation, two weight copies alternated so no step finds its weights in the 256 MB MALL.
roofline: the GEMV kernel alone (activation already Q8_K), timed with HIP events on the stream it is
launched on, algorithmic bytes = weight bytes per launch.
cpu_baseline: the restated iqk AVX-512 VNNI CPU path (oracle/tq_cpu_baseline.c) on the host cores,
same weight bytes, Q8_K quantization included, median of calls within a bounded budget.
secondary: the other workloads (Q4_K GEMV 4096 x 4096 batch 1, attention projections, MUL_MAT_ID at
prefill sizes, MoE step and router, prefill, expert slot uploads from host memory).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4_K GEMV HBM GB/s (frac of peak) at batch 1; MoE MUL_MAT_ID µs/token"
PEAK_GBS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=2000)
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--moe-tokens", type=int, default=0, help="with --only moe: run just this token count")
    p.add_argument("--only", choices=["gemv", "copy", "moe", "prefill", "secondary", "slots"], default=None,
                   help="profiling runs: 'gemv' launches only the headline GEMV kernel (--steps times), "
                        "'copy' a plain 256 MiB device copy (--steps times) to scale the HBM byte counters")
    return p.parse_args()


def make_weights(ggml, torch, ty, k, n, copies, seed, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    out = []
    chunk = max(1, (1 << 27) // k)  # quantize in slices of ~512 MB of fp32
    for c in range(copies):
        raw = torch.empty(n * ty.row_size(k), dtype=torch.uint8, device=dev)
        rb = ty.row_size(k)
        for r0 in range(0, n, chunk):
            r1 = min(n, r0 + chunk)
            src = torch.randn((r1 - r0, k), generator=g, device=dev) * 0.02
            raw[r0 * rb:r1 * rb] = ggml.quantize(ty, src, r1 - r0, k)
            del src
        out.append(ggml.QTensor(ty, (k, n), raw))
    return out


def time_launches(torch, fn, n_launch, reps=3):
    """Average duration of one launch of fn(i) over n_launch back-to-back launches, with events on
    the current stream; the best of reps runs."""
    best = float("inf")
    for _ in range(reps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for i in range(n_launch):
            fn(i)
        e.record()
        e.synchronize()
        best = min(best, s.elapsed_time(e) * 1e3 / n_launch)
    return best


def time_graph(torch, fn, per_graph, replays=20):
    """Average µs per call of fn(i) captured per_graph times in a HIP graph and replayed."""
    for i in range(per_graph):  # warm (and allocate any workspace) outside the capture
        fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(per_graph):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(replays):
        g.replay()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) * 1e3 / (replays * per_graph)


def cpu_baseline(O, np, raw_np, ty_id, k, n, x_np, budget_s):
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or min(16, os.cpu_count() or 1)
    threads = max(1, min(threads, os.cpu_count() or threads))
    q8 = np.zeros(O.row_size(O.TYPE_Q8_K, k), dtype=np.uint8)
    y = np.zeros(n, dtype=np.float32)
    with O.Baseline(threads) as bl:
        for _ in range(3):
            bl.mul_mat(ty_id, raw_np, n, k, x_np, q8, y, use_iqk=True)
        times = []
        t_end = time.perf_counter() + budget_s
        while len(times) < 64 and (time.perf_counter() < t_end or len(times) < 5):
            t0 = time.perf_counter()
            bl.mul_mat(ty_id, raw_np, n, k, x_np, q8, y, use_iqk=True)
            times.append(time.perf_counter() - t0)
        iqk = bl.iqk
    med = statistics.median(times)
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            cpu_model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    return med, threads, len(times), iqk, cpu_model, y


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 (multi-GPU sharding is "
                                   "described in DESIGN.md, not built)"}))
        sys.exit(2)
    import numpy as np
    import torch
    from tetraeder_amd import ggml, _lib
    if not os.path.exists(_lib.LIB_PATH):
        from tetraeder_amd import build as tq_build
        tq_build.build()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"device {torch.cuda.get_device_name(dev)}; {_lib.lib().tq_version().decode()}")
    if args.only == "copy":
        a = torch.empty(1 << 26, dtype=torch.float32, device=dev)
        b = torch.empty_like(a)
        a.fill_(1.0)
        for _ in range(args.steps):
            b.copy_(a)
        torch.cuda.synchronize()
        log(f"copied {args.steps} x 256 MiB")
        return
    if args.only == "moe":
        print(json.dumps(bench_moe(ggml, torch, np, dev, tokens=(args.moe_tokens,) if args.moe_tokens else None)))
        return
    if args.only == "secondary":
        print(json.dumps(bench_secondary(ggml, torch, dev)))
        return
    if args.only == "slots":
        print(json.dumps(bench_slots(ggml, torch, dev)))
        return
    if args.only == "prefill":
        print(json.dumps(bench_prefill(ggml, torch, dev, only=os.environ.get("TQ_BENCH_PROFILE") == "1")))
        return

    # ---- headline: Q6_K output head 151936 x 2048, batch 1 ----
    ty, k, n = ggml.Type.Q6_K, 2048, 151936
    wbytes = n * ty.row_size(k)
    W = make_weights(ggml, torch, ty, k, n, 2, seed=1, dev=dev)
    x = torch.randn((1, k), generator=torch.Generator(device=dev).manual_seed(2), device=dev)
    out = torch.empty((1, n), device=dev)
    ws = torch.empty(ggml.mul_mat_workspace_size(W[0], x), dtype=torch.uint8, device=dev)
    step = lambda i: ggml.mul_mat(W[i & 1], x, out=out, workspace=ws)  # noqa: E731
    if args.only == "gemv":
        xq = ggml.QTensor(ggml.Type.Q8_K, (k, 1), ggml.quantize_q8_K(x).view(-1))
        for i in range(args.steps):
            ggml.mul_mat(W[i & 1], xq, out=out)
        torch.cuda.synchronize()
        log(f"ran {args.steps} GEMV launches")
        return
    log("headline warmup")
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    value = wbytes / (ms_per_step * 1e-3) / 1e9
    log(f"headline {ms_per_step * 1e3:.2f} us/step, {value:.1f} GB/s")

    # the GEMV kernel alone: activation already Q8_K, events on the launch stream
    xq = ggml.QTensor(ggml.Type.Q8_K, (k, 1), ggml.quantize_q8_K(x).view(-1))
    gemv = lambda i: ggml.mul_mat(W[i & 1], xq, out=out)  # noqa: E731
    kern_us = time_launches(torch, gemv, 400)
    kern_us_graph = time_graph(torch, gemv, 64)
    kern_us = min(kern_us, kern_us_graph)
    achieved = wbytes / (kern_us * 1e-6) / 1e9
    log(f"gemv kernel {kern_us:.2f} us -> {achieved:.1f} GB/s")

    # HBM bytes per launch: rocprofv3 FETCH_SIZE + WRITE_SIZE of this kernel, each scaled by what the
    # counter reads for a plain copy of known size (the profile summary next to traffic.json says how)
    traffic = None
    traffic_ratio = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        rec = json.load(open(tpath)).get("gemv_q6_K_151936x2048_m1")
        if rec:
            traffic = int(rec["bytes"])
            traffic_ratio = round(traffic / wbytes, 4)

    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O
        log("cpu baseline")
        raw_np = W[0].data.cpu().numpy()
        x_np = x.cpu().numpy().reshape(-1)
        med, threads, calls, iqk, cpu_model, y_cpu = cpu_baseline(O, np, raw_np, ty.id, k, n, x_np, args.cpu_seconds)
        y_gpu = ggml.mul_mat(W[0], x).cpu().numpy().reshape(-1)
        agree = float(np.abs(y_gpu - y_cpu).max() / np.abs(y_cpu).max())
        cpu = {"value": round(wbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads,
               "kind": "port", "sample": f"full 151936x2048 Q6_K GEMV incl. Q8_K quantize, median of {calls} calls "
                                         f"({'AVX-512 VNNI iqk restatement' if iqk else 'scalar vec_dot: no AVX-512 VNNI'}"
                                         f"; {cpu_model}); max |gpu-cpu| = {agree:.1e} of the largest",
               "us_per_op": round(med * 1e6, 1)}
        log(f"cpu {cpu['value']} GB/s on {threads} threads")
    del W, ws
    torch.cuda.empty_cache()

    secondary = {}
    moe = {}
    if not args.no_secondary:
        moe = bench_moe(ggml, torch, np, dev)
        secondary["moe_step"] = moe
        secondary.update(bench_secondary(ggml, torch, dev))
        secondary["prefill"] = bench_prefill(ggml, torch, dev)
        secondary["expert_slot_upload"] = bench_slots(ggml, torch, dev, moe)

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic: weights N(0,0.02) quantized on device, activations N(0,1)",
        "config": {"workload": "MUL_MAT Q6_K output head 151936x2048, batch 1 (Q8_K quantize + GEMV), "
                               "2 rotated weight copies", "n": n, "k": k, "batch": 1, "weight_bytes": wbytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic,
                     "traffic_over_algorithmic": traffic_ratio,
                     "kernel": "k_gemv_dma<q6_K,1 col>", "kernel_us": round(kern_us, 2)},
        "cpu_baseline": cpu,
        "moe_mul_mat_id_us_per_token": {t: v["us_per_token"] for t, v in moe.items()},
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)


MOE_EXPERT_BYTES = 2 * 884736 + 1290240  # gate + up Q4_K [2048 x 768] + down Q6_K [768 x 2048]


def moe_ids(np, tokens, seed, n_expert=128, used=8, neg_frac=0.1):
    """top-8 of softmax over N(0,1) router logits, then neg_frac of the id slots set to -1."""
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((tokens, n_expert)).astype(np.float32)
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :used].astype(np.int32)
    ids[rng.random(ids.shape) < neg_frac] = -1
    return ids


def bench_moe(ggml, torch, np, dev, layers=4, routings=8, tokens=None):
    """The MoE expert FFN step (gate, up, swiglu, down) at Qwen3-30B-A3B shapes: 128 experts, n_embd
    2048, n_ff 768, gate/up Q4_K, down Q6_K, top-8 with 10% -1. Steps rotate over `layers` weight copies
    (4 x 392 MB) and `routings` seeded id sets, captured in a HIP graph; the roofline bytes are the
    unique valid experts of each step's ids. us_per_step_summed: the same step through sum_experts
    (moe_ffn_sum, [n_embd, T] out); router_us: the router ahead of it (moe_router)."""
    n_embd, n_ff, E = 2048, 768, 128
    L = []
    for l in range(layers):
        L.append(tuple(make_weights(ggml, torch, ty, k, n * E, 1, seed=100 + 3 * l + i, dev=dev)[0]
                       for i, (ty, k, n) in enumerate(((ggml.Type.Q4_K, n_embd, n_ff), (ggml.Type.Q4_K, n_embd, n_ff),
                                                       (ggml.Type.Q6_K, n_ff, n_embd)))))
    L = [tuple(ggml.QTensor(w.type, (w.ne[0], w.ne[1] // E, E), w.data) for w in lw) for lw in L]
    res = {}
    for T in tokens or (1, 2, 4, 8, 16):
        ids_np = [moe_ids(np, T, seed=1000 * T + r) for r in range(routings)]
        uniq = [len(set(int(e) for e in x.reshape(-1) if e >= 0)) for x in ids_np]
        ids = [torch.from_numpy(x).to(dev) for x in ids_np]
        x = torch.randn((T, 1, n_embd), device=dev)
        out = torch.empty((T, 8, n_embd), device=dev)
        ws = torch.empty(max(1, ggml.moe_ffn_workspace_size(L[0][0], x, ids[0])), dtype=torch.uint8, device=dev)
        n = layers * routings
        step = lambda i: ggml.moe_ffn(*L[i % layers], x, ids[(i // layers) % routings], out=out, workspace=ws)  # noqa
        us = time_graph(torch, step, n)
        # the same step through sum_experts (moe_ffn: the slots summed in the same launch)
        out_sum = torch.empty((T, n_embd), device=dev)
        step_sum = lambda i: ggml.moe_ffn_sum(*L[i % layers], x, ids[(i // layers) % routings], out=out_sum,  # noqa
                                              workspace=ws)
        us_sum = time_graph(torch, step_sum, n)
        mean_bytes = sum(uniq[(i // layers) % routings] for i in range(n)) / n * MOE_EXPERT_BYTES
        gbs = mean_bytes / us / 1e3
        res[str(T)] = {"us_per_step": round(us, 2), "us_per_step_summed": round(us_sum, 2), "us_per_token": round(us / T, 2),
                       "unique_experts": round(mean_bytes / MOE_EXPERT_BYTES, 2),
                       "weight_MB": round(mean_bytes / 1e6, 2), "GBps": round(gbs, 1),
                       "frac": round(gbs / PEAK_GBS, 4)}
        # the router ahead of the step (rms_norm, the F32 gate_inp logits, softmax, top-8, weights)
        gate_inp = torch.randn((E, n_embd), device=dev) * 0.02
        norm = torch.ones(n_embd, device=dev)
        x2 = x.view(T, n_embd)
        wsr = torch.empty(max(1, ggml.moe_router_workspace_size(gate_inp, x2)), dtype=torch.uint8, device=dev)
        res[str(T)]["router_us"] = round(time_graph(torch, lambda i: ggml.moe_router(x2, norm, gate_inp, 1e-6, 8,
                                                                                      workspace=wsr), 16), 2)
        log(f"moe T={T}: {res[str(T)]}")
    del L
    torch.cuda.empty_cache()
    return res


def bench_slots(ggml, torch, dev, moe=None):
    """Expert slot uploads (copy_expert_slots) at Qwen3-30B-A3B shapes: the 8 experts of a decode token
    (3,059,712 B each: the gate, up and down slabs) from pinned host memory into 8 device slots, on the
    kernel engine (workgroups reading host memory over PCIe) and on the copy engines (one
    hipMemcpyAsync per slab, as ggml_backend_tensor_set issues them), set against the same experts in
    HBM: their share of the measured 1-token step and their bytes at the 8 TB/s peak."""
    n_embd, n_ff, n_host, n_dev = 2048, 768, 16, 8
    host, slots = [], []
    for ty, k, n in ((ggml.Type.Q4_K, n_embd, n_ff), (ggml.Type.Q4_K, n_embd, n_ff), (ggml.Type.Q6_K, n_ff, n_embd)):
        slab = ty.row_size(k) * n
        buf = torch.empty(slab * n_host, dtype=torch.uint8, pin_memory=True)
        buf.copy_(torch.randint(0, 256, (slab * n_host,), dtype=torch.uint8))
        host.append(ggml.QTensor(ty, (k, n, n_host), buf))
        slots.append(ggml.QTensor(ty, (k, n, n_dev), torch.empty(slab * n_dev, dtype=torch.uint8, device=dev)))
    res = {"experts_per_call": n_dev, "bytes_per_call": n_dev * MOE_EXPERT_BYTES}
    for name, engine in (("kernel", ggml.COPY_KERNEL), ("dma", ggml.COPY_DMA)):
        def call(i, engine=engine):
            first = (i % 2) * n_dev  # alternate between the two halves of the host slots
            ggml.copy_expert_slots(host, slots, range(first, first + n_dev), range(n_dev), engine=engine)
        us = time_launches(torch, call, 20)
        res[name] = {"us_per_call": round(us, 1), "us_per_expert": round(us / n_dev, 2),
                     "GBps": round(n_dev * MOE_EXPERT_BYTES / us / 1e3, 2)}
    res["hbm_peak_us_per_expert"] = round(MOE_EXPERT_BYTES / PEAK_GBS / 1e3, 3)
    if moe and "1" in moe:
        res["step_us_per_expert_T1"] = round(moe["1"]["us_per_step"] / moe["1"]["unique_experts"], 2)
    log(f"slots: {res}")
    del host, slots
    return res


PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA


def bench_prefill(ggml, torch, dev, only=False):
    """Dense prefill GEMMs (hidden 4096, FFN 12288): Q4_K gate/up [4096 -> 12288] and Q6_K down
    [12288 -> 4096] at M = 512 and 2048 activation rows. op = MUL_MAT with the F32 activations (Q8_K
    pass included); kernel = the MFMA kernel alone on pre-quantized activations. int ops = 2 M N K."""
    res = {}
    shapes = (("gate_up", ggml.Type.Q4_K, 4096, 12288), ("down", ggml.Type.Q6_K, 12288, 4096))
    for name, ty, k, n in shapes:
        W = make_weights(ggml, torch, ty, k, n, 2, seed=k + n, dev=dev)
        for m in (512, 2048):
            x = torch.randn((m, k), device=dev)
            out = torch.empty((m, n), device=dev)
            ws = torch.empty(ggml.mul_mat_workspace_size(W[0], x), dtype=torch.uint8, device=dev)
            xq = ggml.QTensor(ggml.Type.Q8_K, (k, m), ggml.quantize_q8_K(x).view(-1))
            if only:
                for i in range(20):
                    ggml.mul_mat(W[i & 1], xq, out=out)
                torch.cuda.synchronize()
                continue
            op_us = time_launches(torch, lambda i: ggml.mul_mat(W[i & 1], x, out=out, workspace=ws), 20)
            kern_us = time_launches(torch, lambda i: ggml.mul_mat(W[i & 1], xq, out=out), 20)
            ops = 2.0 * m * n * k
            res[f"{name}_{ty.name}_{k}x{n}_m{m}"] = {
                "op_us": round(op_us, 1), "kernel_us": round(kern_us, 1),
                "kernel_TOPS": round(ops / kern_us / 1e6, 1),
                "mfma_frac": round(ops / kern_us / 1e6 / PEAK_INT8_TOPS, 4),
                "op_TOPS": round(ops / op_us / 1e6, 1)}
            log(f"prefill {name} m={m}: {res[f'{name}_{ty.name}_{k}x{n}_m{m}']}")
            del x, out, ws, xq
        del W
        torch.cuda.empty_cache()
    return res


def bench_secondary(ggml, torch, dev):
    res = {}
    # Q4_K 4096 x 4096 batch 1: 64 rotated copies (604 MB > 2 x MALL), graph-replayed
    ty, k, n = ggml.Type.Q4_K, 4096, 4096
    copies = 64
    W = make_weights(ggml, torch, ty, k, n, copies, seed=3, dev=dev)
    x = torch.randn((1, k), device=dev)
    out = torch.empty((1, n), device=dev)
    ws = torch.empty(ggml.mul_mat_workspace_size(W[0], x), dtype=torch.uint8, device=dev)
    xq = ggml.QTensor(ggml.Type.Q8_K, (k, 1), ggml.quantize_q8_K(x).view(-1))
    wb = n * ty.row_size(k)
    op_us = time_graph(torch, lambda i: ggml.mul_mat(W[i % copies], x, out=out, workspace=ws), copies)
    kern_us = time_graph(torch, lambda i: ggml.mul_mat(W[i % copies], xq, out=out), copies)
    res["q4_K_gemv_4096x4096_m1"] = {"op_us": round(op_us, 2), "gemv_kernel_us": round(kern_us, 2),
                                     "gemv_GBps": round(wb / kern_us / 1e3, 1),
                                     "gemv_frac": round(wb / kern_us / 1e3 / PEAK_GBS, 4),
                                     "op_GBps": round(wb / op_us / 1e3, 1)}
    log(f"q4_K 4096x4096: {res['q4_K_gemv_4096x4096_m1']}")
    del W, ws
    # the same kernels at a bandwidth-bound size: Q4_K 151936 x 2048 at batch 1 (175 MB, two copies
    # alternated) and the Q6_K head at batch 4, kernel alone (activations already Q8_K)
    for label, tyb, k, n, m in (("q4_K", ggml.Type.Q4_K, 2048, 151936, 1), ("q6_K", ggml.Type.Q6_K, 2048, 151936, 4)):
        W = make_weights(ggml, torch, tyb, k, n, 2, seed=5 + m, dev=dev)
        x = torch.randn((m, k), device=dev)
        out = torch.empty((m, n), device=dev)
        xq = ggml.QTensor(ggml.Type.Q8_K, (k, m), ggml.quantize_q8_K(x).view(-1))
        wb = n * tyb.row_size(k)
        kern_us = min(time_launches(torch, lambda i: ggml.mul_mat(W[i & 1], xq, out=out), 200),
                      time_graph(torch, lambda i: ggml.mul_mat(W[i & 1], xq, out=out), 32))
        key = f"{label}_gemv_{n}x{k}_m{m}"
        res[key] = {"gemv_kernel_us": round(kern_us, 2), "gemv_GBps": round(wb / kern_us / 1e3, 1),
                    "gemv_frac": round(wb / kern_us / 1e3 / PEAK_GBS, 4)}
        log(f"{key}: {res[key]}")
        del W
    torch.cuda.empty_cache()
    # attention projections (Q4_K), decode batch 1, 4, 16, 32; 16 rotated layer copies
    shapes = (("q", 2048, 4096), ("k", 2048, 512), ("v", 2048, 512), ("o", 4096, 2048))
    copies = 16
    for name, k, n in shapes:
        W = make_weights(ggml, torch, ty, k, n, copies, seed=n + k, dev=dev)
        wb = n * ty.row_size(k)
        for m in (1, 4, 16, 32):
            x = torch.randn((m, k), device=dev)
            out = torch.empty((m, n), device=dev)
            ws = torch.empty(ggml.mul_mat_workspace_size(W[0], x), dtype=torch.uint8, device=dev)
            us = time_graph(torch, lambda i: ggml.mul_mat(W[i % copies], x, out=out, workspace=ws), copies)
            res[f"attn_{name}_proj_{k}x{n}_m{m}"] = {"op_us": round(us, 2), "GBps": round(wb / us / 1e3, 1)}
        del W
        log(f"attn {name}: " + ", ".join(f"m{m} {res[f'attn_{name}_proj_{k}x{n}_m{m}']['op_us']}us" for m in (1, 4, 16, 32)))
    torch.cuda.empty_cache()
    # MUL_MAT_ID at prefill sizes: gate Q4_K [2048 -> 768] x 128 experts, top-8 of 512 and 2048 tokens
    E, k, n = 128, 2048, 768
    w = make_weights(ggml, torch, ty, k, n * E, 1, seed=3, dev=dev)[0]
    w = ggml.QTensor(w.type, (k, n, E), w.data)
    import numpy as np
    for T in (512, 2048):
        ids = torch.from_numpy(moe_ids(np, T, seed=T)).to(dev)
        x = torch.randn((T, 1, k), device=dev)
        out = torch.empty((T, 8, n), device=dev)
        ws = torch.empty(max(1, ggml.mul_mat_id_workspace_size(w, x, ids)), dtype=torch.uint8, device=dev)
        us = time_graph(torch, lambda i: ggml.mul_mat_id(w, x, ids, out=out, workspace=ws), 4)
        valid = int((ids >= 0).sum().item())
        res[f"mul_mat_id_q4_K_2048x768x128_T{T}"] = {"op_us": round(us, 1),
                                                     "int_TOPS": round(2 * valid * n * k / us / 1e6, 1)}
        log(f"mul_mat_id T={T}: {res[f'mul_mat_id_q4_K_2048x768x128_T{T}']}")
    del w
    torch.cuda.empty_cache()
    return res


if __name__ == "__main__":
    main()
