"""Benchmark of the Q4_K / Q6_K MUL_MAT and MUL_MAT_ID path on one MI355X.

Headline (value): HBM GB/s of weight bytes of the batch-1 Q4_K decode GEMV the metric names, a
4096 x 4096 MUL_MAT (9,437,184 weight bytes; the shape of the reference's single-matmul CPU benchmark),
one step = one MUL_MAT of an F32 activation column (the Q8_K quantization runs inside the GEMV
workgroups: one launch per step). 64 weight copies (604 MB, more than twice the 256 MB MALL) rotate, so
every step reads its weights from HBM. The K timed steps are one HIP graph of K launches (the reference
replays decode ranges as graphs, patches 0005/0006; a host-issued launch from Python costs more than
the kernel), replayed once untimed, then timed between two stream synchronizations.
roofline: weight bytes / the mean kernel duration over the timed region (HIP events on the stream the
graph runs on; one kernel per step, so it is the per-step time including the dispatch gap between
graph nodes); `kernel_us_best` is the best of three more replays, reported apart. `traffic` comes
from the FETCH_SIZE / WRITE_SIZE profile of this kernel in profiles/traffic.json and is given only when
that profile was taken on the sources this run was built from (their hash is compared).
cpu_baseline: the restated iqk AVX-512 VNNI CPU path (oracle/tq_cpu_baseline.c) on the host cores,
same weight bytes, Q8_K quantization included, weight copies rotated; cpu_baselines: one line per
workload (Q4_K 4096 x 4096, Q6_K head, attention projections, the MoE MUL_MAT_ID step, prefill).
secondary: the other workloads (Q6_K head at batch 1 and 4, attention projections, q/k/v as backend
nodes sharing one Q8_K pass, MUL_MAT_ID at prefill sizes and its expert-parallel rank shares, the MoE
step and router, prefill, slot uploads).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4_K GEMV HBM GB/s (frac of peak) at batch 1; MoE MUL_MAT_ID µs/token"
PEAK_GBS = 8000.0
HEAD_COPIES = 64  # 64 x 9.4 MB = 604 MB > 2 x the 256 MB MALL


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=5000)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--cpu-seconds", type=float, default=4.0, help="CPU budget per baseline line")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--moe-tokens", type=int, default=0, help="with --only moe: run just this token count")
    p.add_argument("--cols", type=int, default=1, help="with --only head: activation columns (decode batch)")
    p.add_argument("--only", choices=["gemv", "head", "copy", "moe", "prefill", "secondary", "slots", "ranks", "cpu"],
                   default=None,
                   help="profiling runs: 'gemv' replays the headline graph of --steps Q4_K 4096 x 4096 launches, "
                        "'head' launches the Q6_K head GEMV kernel --steps times, 'copy' a plain 256 MiB device "
                        "copy (--steps times) to scale the HBM byte counters")
    return p.parse_args()


def source_hash():
    """sha1 over the HIP sources and headers libtq.so is built from (names and bytes, sorted)."""
    h = hashlib.sha1()
    csrc = os.path.join(ROOT, "tetraeder_amd", "csrc")
    for name in sorted(os.listdir(csrc)):
        if name.endswith((".hip", ".h")):
            h.update(name.encode())
            with open(os.path.join(csrc, name), "rb") as f:
                h.update(f.read())
    with open(os.path.join(ROOT, "include", "tq.h"), "rb") as f:
        h.update(f.read())
    return h.hexdigest()[:12]


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


def capture(torch, fn, n):
    """A HIP graph of fn(0) .. fn(n-1), warmed (any workspace allocated) outside the capture and
    replayed once untimed."""
    for i in range(min(n, 64)):
        fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    return g


def time_replay(torch, g, calls):
    """µs per call of one replay of graph g holding `calls` calls (events on the replay stream)."""
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    g.replay()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) * 1e3 / calls


def time_graph(torch, fn, per_graph, replays=20):
    """Average µs per call of fn(i) captured per_graph times in a HIP graph and replayed."""
    g = capture(torch, fn, per_graph)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(replays):
        g.replay()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) * 1e3 / (replays * per_graph)


# ---------------------------------------------------------------------------------------------------
# CPU baseline: the restated iqk path (oracle/tq_cpu_baseline.c) on the host cores


def cpu_env():
    """Threads the baseline may use (the affinity mask, capped by the cgroup's cpu.max quota) and what
    the host is: nproc, CPU model, AVX-512 flags."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = os.cpu_count() or 1
    quota = None
    for path in ("/sys/fs/cgroup/cpu.max",):
        try:
            q, per = open(path).read().split()[:2]
            if q != "max":
                quota = int(q) / int(per)
        except (OSError, ValueError):
            pass
    if quota is None:
        try:
            q = int(open("/sys/fs/cgroup/cpu/cpu.cfs_quota_us").read())
            per = int(open("/sys/fs/cgroup/cpu/cpu.cfs_period_us").read())
            if q > 0:
                quota = q / per
        except (OSError, ValueError):
            pass
    threads = affinity if quota is None else max(1, min(affinity, int(math.floor(quota + 1e-9))))
    model, flags = "", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and not model:
                    model = line.split(":", 1)[1].strip()
                elif line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    isa = sorted(f for f in flags if f.startswith("avx512") and f in ("avx512f", "avx512bw", "avx512dq", "avx512vl",
                                                                       "avx512_vnni", "avx512vnni"))
    return {"threads": threads, "affinity": affinity, "cgroup_quota_cpus": quota, "nproc": os.cpu_count(),
            "cpu": model, "isa": isa}


def cpu_median(call, budget_s, max_calls=100000, min_calls=5):
    """3 warm-up calls, then the median of calls within budget_s (at least min_calls)."""
    for i in range(3):
        call(i)
    times = []
    t_end = time.perf_counter() + budget_s
    i = 0
    while len(times) < max_calls and (time.perf_counter() < t_end or len(times) < min_calls):
        t0 = time.perf_counter()
        call(i)
        times.append(time.perf_counter() - t0)
        i += 1
    return statistics.median(times), len(times)


def cpu_baselines(ggml, torch, np, dev, env, budget_s):
    """One line per workload, each on the same weight bytes the GPU reads (copied to host memory) with
    the copies rotated so the reads come from DRAM, Q8_K quantization included. Returns (lines,
    the Q4_K 4096 x 4096 line, its GPU/CPU agreement)."""
    from oracle import oracle as O
    lines = []
    threads = env["threads"]
    with O.Baseline(threads) as bl:
        how = "AVX-512 VNNI iqk restatement" if bl.iqk else "scalar vec_dot (no AVX-512 VNNI on this host)"

        def line(config, workload, value, unit, us, calls, sample, **extra):
            d = {"config": config, "device": "cpu", "workload": workload, "value": value, "unit": unit,
                 "median_us_per_op": round(us, 2), "calls": calls, "threads": threads, "cpu": env["cpu"],
                 "isa": env["isa"], "nproc": env["nproc"], "kind": "port", "path": how, "sample": sample}
            d.update(extra)
            lines.append(d)
            log(f"cpu {workload}: {value} {unit} ({us:.1f} us/op, {calls} calls)")
            return d

        # 1. Q4_K 4096 x 4096, batch 1, 16 host copies of the GPU's weight bytes (151 MB)
        ty, k, n = ggml.Type.Q4_K, 4096, 4096
        W = make_weights(ggml, torch, ty, k, n, 16, seed=1, dev=dev)
        host = [w.data.cpu().numpy() for w in W]
        x = torch.randn((1, k), generator=torch.Generator(device=dev).manual_seed(2), device=dev)
        x_np = x.cpu().numpy().reshape(-1)
        q8 = np.zeros(O.row_size(O.TYPE_Q8_K, k), dtype=np.uint8)
        y = np.zeros(n, dtype=np.float32)
        med, calls = cpu_median(lambda i: bl.mul_mat(ty.id, host[i % 16], n, k, x_np, q8, y), budget_s)
        y_gpu = ggml.mul_mat(W[0], x).cpu().numpy().reshape(-1)
        bl.mul_mat(ty.id, host[0], n, k, x_np, q8, y)
        agree = float(np.abs(y_gpu - y).max() / np.abs(y).max())
        wb = n * ty.row_size(k)
        first = line(1, "MUL_MAT Q4_K 4096x4096 batch 1", round(wb / med / 1e9, 3), "GB/s", med * 1e6, calls,
                     f"the full op, 16 rotated weight copies; max |gpu-cpu| = {agree:.1e} of the largest")
        del W, host

        # 2. Q6_K head 151936 x 2048 at batch 1 and 4, 2 copies
        ty, k, n = ggml.Type.Q6_K, 2048, 151936
        W = make_weights(ggml, torch, ty, k, n, 2, seed=1, dev=dev)
        host = [w.data.cpu().numpy() for w in W]
        wb = n * ty.row_size(k)
        for m in (1, 4):
            xm = np.random.default_rng(2 + m).standard_normal((m, k)).astype(np.float32).reshape(-1)
            q8 = np.zeros(m * O.row_size(O.TYPE_Q8_K, k), dtype=np.uint8)
            y = np.zeros(m * n, dtype=np.float32)
            med, calls = cpu_median(lambda i: bl.mul_mat(ty.id, host[i & 1], n, k, xm, q8, y), budget_s / 2)
            line(2, f"MUL_MAT Q6_K 151936x2048 batch {m}", round(wb / med / 1e9, 3), "GB/s", med * 1e6, calls,
                 "the full op, 2 rotated weight copies (255 MB each)", batch=m)
        del W, host

        # 3. attention projections q, k, v, o (Q4_K) of one layer at batch 1 and 32, 16 layer copies
        shapes = (("q", 2048, 4096), ("k", 2048, 512), ("v", 2048, 512), ("o", 4096, 2048))
        ty = ggml.Type.Q4_K
        layers = [[make_weights(ggml, torch, ty, kk, nn, 1, seed=100 * li + j, dev=dev)[0].data.cpu().numpy()
                   for j, (_, kk, nn) in enumerate(shapes)] for li in range(16)]
        wb = sum(nn * ty.row_size(kk) for _, kk, nn in shapes)
        for m in (1, 32):
            xs = {kk: np.random.default_rng(kk + m).standard_normal((m, kk)).astype(np.float32).reshape(-1)
                  for kk in (2048, 4096)}
            q8s = {kk: np.zeros(m * O.row_size(O.TYPE_Q8_K, kk), dtype=np.uint8) for kk in (2048, 4096)}
            ys = [np.zeros(m * nn, dtype=np.float32) for _, _, nn in shapes]

            def layer(i):
                lw = layers[i % 16]
                for j, (_, kk, nn) in enumerate(shapes):
                    bl.mul_mat(ty.id, lw[j], nn, kk, xs[kk], q8s[kk], ys[j])
            med, calls = cpu_median(layer, budget_s / 2)
            line(3, f"attention q/k/v/o projections (Q4_K) batch {m}", round(wb / med / 1e9, 3), "GB/s", med * 1e6,
                 calls, "q 2048->4096, k and v 2048->512, o 4096->2048 in sequence, 16 rotated layer copies",
                 batch=m)
        del layers

        # 4. the MoE MUL_MAT_ID step (gate, up: Q4_K 2048->768; down: Q6_K 768->2048; 128 experts, top-8,
        # 10% -1) at 1 and 16 tokens; 4 layer copies and 8 seeded routings rotated, so the experts read
        # change from call to call (crates/ggml-sys/tests/expert_matmul.rs:65-109 rotates them likewise)
        n_embd, n_ff, E = 2048, 768, 128
        L = []
        for li in range(4):
            L.append([make_weights(ggml, torch, tyw, kk, nn * E, 1, seed=100 + 3 * li + i, dev=dev)[0].data.cpu().numpy()
                      for i, (tyw, kk, nn) in enumerate(((ggml.Type.Q4_K, n_embd, n_ff), (ggml.Type.Q4_K, n_embd, n_ff),
                                                         (ggml.Type.Q6_K, n_ff, n_embd)))])
        for T in (1, 16):
            idss = [moe_ids(np, T, seed=1000 * T + r) for r in range(8)]
            xb = np.random.default_rng(T).standard_normal((T, n_embd)).astype(np.float32)
            q8g = np.zeros(O.row_size(O.TYPE_Q8_K, n_embd), dtype=np.uint8)
            q8d = np.zeros(8 * O.row_size(O.TYPE_Q8_K, n_ff), dtype=np.uint8)
            g = np.zeros((T, 8, n_ff), np.float32)
            u = np.zeros((T, 8, n_ff), np.float32)
            o = np.zeros((T, 8, n_embd), np.float32)

            def step(i):
                lw = L[i % 4]
                ids = idss[(i // 4) % 8]
                for t in range(T):
                    bl.mul_mat_id(ggml.Type.Q4_K.id, lw[0], n_ff * 144 * (n_embd // 256), n_ff, n_embd, xb[t], ids[t],
                                  q8g, g[t])
                    bl.mul_mat_id(ggml.Type.Q4_K.id, lw[1], n_ff * 144 * (n_embd // 256), n_ff, n_embd, xb[t], ids[t],
                                  q8g, u[t])
                    act = (g[t] / (1.0 + np.exp(-g[t])) * u[t]).astype(np.float32)
                    bl.mul_mat_id(ggml.Type.Q6_K.id, lw[2], n_embd * 210 * (n_ff // 256), n_embd, n_ff, act, ids[t],
                                  q8d, o[t])
            med, calls = cpu_median(step, budget_s / 2)
            uniq = statistics.mean(len(set(int(e) for e in x.reshape(-1) if e >= 0)) for x in idss)
            wbytes = uniq * MOE_EXPERT_BYTES
            line(4, f"MoE MUL_MAT_ID step (gate, up, swiglu, down) T={T}", round(med * 1e6 / T, 2), "us/token",
                 med * 1e6, calls, "per token: gate and up MUL_MAT_ID of its 8 slots, swiglu (numpy), down; "
                 "4 layer copies x 8 routings rotated", tokens=T, unique_experts=round(uniq, 2),
                 unique_expert_GBps=round(wbytes / med / 1e9, 3))
        del L

        # 5. prefill GEMMs at M = 512: a bounded sample of 16 columns per call (the one-column kernel per
        # column, as the CPU path runs it), scaled to int ops per second
        for name, ty, k, n in (("gate_up", ggml.Type.Q4_K, 4096, 12288), ("down", ggml.Type.Q6_K, 12288, 4096)):
            wh = make_weights(ggml, torch, ty, k, n, 1, seed=k + n, dev=dev)[0].data.cpu().numpy()
            m = 16
            xm = np.random.default_rng(k).standard_normal((m, k)).astype(np.float32).reshape(-1)
            q8 = np.zeros(m * O.row_size(O.TYPE_Q8_K, k), dtype=np.uint8)
            y = np.zeros(m * n, dtype=np.float32)
            med, calls = cpu_median(lambda i: bl.mul_mat(ty.id, wh, n, k, xm, q8, y), budget_s / 2, min_calls=3)
            tops = 2.0 * m * n * k / med / 1e12
            line(5, f"prefill {name} {ty.name} {k}->{n}", round(tops, 4), "TOPS (int)", med * 1e6, calls,
                 f"{m} of the M = 512 columns per call, scaled: {round(med * 512 / m * 1e3, 2)} ms per M = 512 op",
                 est_ms_m512=round(med * 512 / m * 1e3, 2))
            del wh
    return lines, first


# ---------------------------------------------------------------------------------------------------


def headline(ggml, torch, dev, steps, warmup, only_profile=False):
    """The Q4_K 4096 x 4096 batch-1 MUL_MAT, 64 rotated weight copies, as a graph of `steps` launches."""
    ty, k, n = ggml.Type.Q4_K, 4096, 4096
    wbytes = n * ty.row_size(k)
    W = make_weights(ggml, torch, ty, k, n, HEAD_COPIES, seed=1, dev=dev)
    x = torch.randn((1, k), generator=torch.Generator(device=dev).manual_seed(2), device=dev)
    out = torch.empty((1, n), device=dev)
    assert ggml.mul_mat_workspace_size(W[0], x) == 0  # one launch, nothing allocated
    step = lambda i: ggml.mul_mat(W[i % HEAD_COPIES], x, out=out)  # noqa: E731
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    g = capture(torch, step, steps)
    if only_profile:
        g.replay()
        torch.cuda.synchronize()
        return None
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    g.replay()
    e.record()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / steps
    kern_us = s.elapsed_time(e) * 1e3 / steps
    best = min(time_replay(torch, g, steps) for _ in range(3))
    res = {"wbytes": wbytes, "ms_per_step": ms_per_step, "kernel_us": kern_us, "kernel_us_best": best}
    del g, W
    torch.cuda.empty_cache()
    return res


def traffic_record(key, wbytes):
    """(bytes, ratio, note) of the FETCH_SIZE + WRITE_SIZE profile of `key` when it was taken on these
    sources, else (None, None, why)."""
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(tpath):
        return None, None, "no traffic profile"
    rec = json.load(open(tpath)).get(key)
    if not rec:
        return None, None, "no traffic profile for this kernel"
    here = source_hash()
    if rec.get("source_hash") != here:
        return None, None, f"traffic profile taken on sources {rec.get('source_hash')}, this build is {here}"
    return int(rec["bytes"]), round(int(rec["bytes"]) / wbytes, 4), f"profiles/traffic.json ({key}, sources {here})"


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
        raise SystemExit(f"{_lib.LIB_PATH} is missing: build it first (python -m tetraeder_amd.build)")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"device {torch.cuda.get_device_name(dev)}; {_lib.lib().tq_version().decode()}; sources {source_hash()}")
    if args.only == "copy":
        a = torch.empty(1 << 26, dtype=torch.float32, device=dev)
        b = torch.empty_like(a)
        a.fill_(1.0)
        for _ in range(args.steps):
            b.copy_(a)
        torch.cuda.synchronize()
        log(f"copied {args.steps} x 256 MiB")
        return
    if args.only == "gemv":
        headline(ggml, torch, dev, args.steps, args.warmup, only_profile=True)
        log(f"replayed a graph of {args.steps} Q4_K 4096x4096 GEMV launches")
        return
    if args.only == "head":
        ty, k, n, m = ggml.Type.Q6_K, 2048, 151936, args.cols
        W = make_weights(ggml, torch, ty, k, n, 2, seed=1, dev=dev)
        x = torch.randn((m, k), generator=torch.Generator(device=dev).manual_seed(2), device=dev)
        out = torch.empty((m, n), device=dev)
        xq = ggml.QTensor(ggml.Type.Q8_K, (k, m), ggml.quantize_q8_K(x).view(-1))
        for i in range(args.steps):
            ggml.mul_mat(W[i & 1], xq, out=out)
        torch.cuda.synchronize()
        log(f"ran {args.steps} Q6_K head MUL_MAT launches at {m} columns")
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
    if args.only == "ranks":
        print(json.dumps(bench_rank_shares(ggml, torch, np, dev)))
        return
    if args.only == "prefill":
        print(json.dumps(bench_prefill(ggml, torch, dev, only=os.environ.get("TQ_BENCH_PROFILE") == "1")))
        return
    if args.only == "cpu":
        env = cpu_env()
        lines, _ = cpu_baselines(ggml, torch, np, dev, env, args.cpu_seconds)
        print(json.dumps({"cpu_env": env, "cpu_baselines": lines}))
        return

    # ---- headline: Q4_K 4096 x 4096, batch 1 ----
    log("headline")
    h = headline(ggml, torch, dev, args.steps, args.warmup)
    wbytes = h["wbytes"]
    value = wbytes / (h["ms_per_step"] * 1e-3) / 1e9
    achieved = wbytes / (h["kernel_us"] * 1e-6) / 1e9
    log(f"headline {h['ms_per_step'] * 1e3:.3f} us/step = {value:.1f} GB/s; kernel {h['kernel_us']:.3f} us (mean), "
        f"{h['kernel_us_best']:.3f} us (best replay)")
    traffic, traffic_ratio, traffic_src = traffic_record("gemv_q4_K_4096x4096_m1", wbytes)

    cpu, lines, env = None, None, None
    if not args.no_cpu:
        env = cpu_env()
        log(f"cpu baselines on {env['threads']} threads ({env['cpu']})")
        lines, first = cpu_baselines(ggml, torch, np, dev, env, args.cpu_seconds)
        cpu = {"value": first["value"], "unit": "GB/s", "cores": env["threads"], "kind": "port",
               "sample": f"{first['workload']}: {first['sample']}; median of {first['calls']} calls "
                         f"({first['path']}; {env['cpu']}; nproc {env['nproc']}, affinity {env['affinity']}, "
                         f"cgroup quota {env['cgroup_quota_cpus']} CPUs; {', '.join(env['isa']) or 'no AVX-512'})",
               "us_per_op": first["median_us_per_op"]}

    secondary = {}
    moe = {}
    if not args.no_secondary:
        moe = bench_moe(ggml, torch, np, dev)
        secondary["moe_step"] = moe
        secondary.update(bench_secondary(ggml, torch, dev))
        secondary["mul_mat_id_rank_shares_T512"] = bench_rank_shares(ggml, torch, np, dev)
        secondary["prefill"] = bench_prefill(ggml, torch, dev)
        secondary["expert_slot_upload"] = bench_slots(ggml, torch, dev, moe)

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(h["ms_per_step"], 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic: weights N(0,0.02) quantized on device, activations N(0,1)",
        "config": {"workload": "MUL_MAT Q4_K 4096x4096, batch 1 (F32 activation, Q8_K inside the GEMV, one "
                               "launch per step), 64 rotated weight copies, graph of K launches",
                   "n": 4096, "k": 4096, "batch": 1, "weight_bytes": wbytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic,
                     "traffic_over_algorithmic": traffic_ratio, "traffic_source": traffic_src,
                     "kernel": "k_gemv_dma<Q4_K, 1 col, 64 lanes per row>",
                     "kernel_us": round(h["kernel_us"], 3), "kernel_us_best": round(h["kernel_us_best"], 3),
                     "frac_best": round(wbytes / (h["kernel_us_best"] * 1e-6) / 1e9 / PEAK_GBS, 4),
                     "source_hash": source_hash()},
        "cpu_baseline": cpu,
        "cpu_baselines": lines,
        "cpu_env": env,
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
    # the Q6_K output head 151936 x 2048 (255 MB, two copies alternated) at batch 1 and 4: the whole
    # MUL_MAT (F32 activations) and the kernel alone on Q8_K activations, mean per launch over 400
    # back-to-back launches; Q4_K at the same bandwidth-bound size (175 MB) at batch 1 and 4
    for label, tyb, k, n, m in (("q6_K", ggml.Type.Q6_K, 2048, 151936, 1), ("q6_K", ggml.Type.Q6_K, 2048, 151936, 4),
                                ("q4_K", ggml.Type.Q4_K, 2048, 151936, 1), ("q4_K", ggml.Type.Q4_K, 2048, 151936, 4)):
        W = make_weights(ggml, torch, tyb, k, n, 2, seed=5 + m, dev=dev)
        x = torch.randn((m, k), device=dev)
        out = torch.empty((m, n), device=dev)
        ws = torch.empty(max(1, ggml.mul_mat_workspace_size(W[0], x)), dtype=torch.uint8, device=dev)
        xq = ggml.QTensor(ggml.Type.Q8_K, (k, m), ggml.quantize_q8_K(x).view(-1))
        wb = n * tyb.row_size(k)
        op_us = time_launches(torch, lambda i: ggml.mul_mat(W[i & 1], x, out=out, workspace=ws), 400, reps=1)
        kern_us = time_launches(torch, lambda i: ggml.mul_mat(W[i & 1], xq, out=out), 400, reps=1)
        key = f"{label}_gemv_{n}x{k}_m{m}"
        res[key] = {"op_us": round(op_us, 2), "op_GBps": round(wb / op_us / 1e3, 1),
                    "gemv_kernel_us": round(kern_us, 2), "gemv_GBps": round(wb / kern_us / 1e3, 1),
                    "gemv_frac": round(wb / kern_us / 1e3 / PEAK_GBS, 4)}
        log(f"{key}: {res[key]}")
        del W, ws
    torch.cuda.empty_cache()
    ty = ggml.Type.Q4_K
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
    # q, k, v of one layer as a run of backend nodes (one Q8_K pass shared from 4 columns) against three
    # separate calls; 48 rotated layer copies (288 MB, past the MALL), graphs on the backend's stream
    from tetraeder_amd import backend as B
    copies = 48
    Wl = [[make_weights(ggml, torch, ty, 2048, n, 1, seed=c * 3 + j, dev=dev)[0] for j, n in enumerate((4096, 512, 512))]
          for c in range(copies)]
    stream = torch.cuda.Stream()
    be = B.Backend.gpu(0, stream=stream)
    qkv = {}
    for m in (1, 4, 16, 32):
        x = torch.randn((m, 2048), device=dev)
        lists = [[B.mul_mat(w, x) for w in Wl[c]] for c in range(copies)]
        be.reserve([nd for l in lists for nd in l])
        for l in lists:
            be.compute_async(l)
        be.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for l in lists:
                be.compute_async(l)
        outs = [[nd.out for nd in l] for l in lists]
        ws = torch.empty(max(1, max(ggml.mul_mat_workspace_size(w, x) for w in Wl[0])), dtype=torch.uint8, device=dev)

        def sep(i):
            for w, o in zip(Wl[i % copies], outs[i % copies]):
                ggml.mul_mat(w, x, out=o, workspace=ws)

        t_sep = time_graph(torch, sep, copies)
        with torch.cuda.stream(stream):
            g.replay()
            torch.cuda.synchronize()
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record(stream)
            for _ in range(20):
                g.replay()
            t1.record(stream)
            t1.synchronize()
        t_be = t0.elapsed_time(t1) * 1e3 / (20 * copies)
        qkv[f"m{m}"] = {"backend_us": round(t_be, 2), "separate_calls_us": round(t_sep, 2)}
        del g, lists, outs
    be.close()
    res["attn_qkv_2048x4096_512_512_backend"] = qkv
    log(f"attn qkv backend vs separate calls: {qkv}")
    del Wl
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
    # and the down projections: Q6_K [768 -> 2048] x 128 experts, one activation row per slot
    k, n = 768, 2048
    w = make_weights(ggml, torch, ggml.Type.Q6_K, k, n * E, 1, seed=4, dev=dev)[0]
    w = ggml.QTensor(w.type, (k, n, E), w.data)
    for T in (512, 2048):
        ids = torch.from_numpy(moe_ids(np, T, seed=T)).to(dev)
        x = torch.randn((T, 8, k), device=dev)
        out = torch.empty((T, 8, n), device=dev)
        ws = torch.empty(max(1, ggml.mul_mat_id_workspace_size(w, x, ids)), dtype=torch.uint8, device=dev)
        us = time_graph(torch, lambda i: ggml.mul_mat_id(w, x, ids, out=out, workspace=ws), 4)
        valid = int((ids >= 0).sum().item())
        key = f"mul_mat_id_q6_K_768x2048x128_T{T}"
        res[key] = {"op_us": round(us, 1), "int_TOPS": round(2 * valid * n * k / us / 1e6, 1)}
        log(f"mul_mat_id down T={T}: {res[key]}")
    del w
    torch.cuda.empty_cache()
    return res


def rank_share_ids(np, tokens, seed, n_expert=128, used=8):
    """The routings of the reference's expert-parallel timing (crates/ggml-sys/tests/mul_mat_id_skip.rs:
    301-406): `used` distinct experts per token drawn uniformly (partial Fisher-Yates, :64-84); rank 0 of
    g holds experts 0 .. 128/g - 1; skip_g: the other ranks' slots are -1; remap_g: each remote slot takes
    the lowest local expert the token does not use yet; random_neg90: 90% of the slots -1."""
    rng = np.random.default_rng(seed)

    def draw(neg_pct):
        ids = np.zeros((tokens, used), dtype=np.int32)
        for t in range(tokens):
            pool = np.arange(n_expert)
            for j in range(used):
                pick = j + int(rng.integers(n_expert - j))
                pool[j], pool[pick] = pool[pick], pool[j]
                ids[t, j] = -1 if rng.integers(100) < neg_pct else pool[j]
        return ids
    routed = draw(0)
    cases = {}
    for g in (1, 2, 4, 8):
        local = n_expert // g
        cases[f"skip_g{g}"] = np.where(routed < local, routed, -1).astype(np.int32)
        if g > 1:
            remap = routed.copy()
            for t in range(tokens):
                free = [e for e in range(local) if e not in remap[t]]
                for j in range(used):
                    if remap[t, j] >= local:
                        remap[t, j] = free.pop(0)
            cases[f"remap_g{g}"] = remap
    cases["random_neg90"] = draw(90)
    return cases


def bench_rank_shares(ggml, torch, np, dev, tokens=512):
    """MUL_MAT_ID Q4_K gate shape (2048 -> 768, 128 experts, top-8) at 512 tokens for the reference's
    expert-parallel cases (skip_g1/2/4/8, remap_g2/4/8, random_neg90; mul_mat_id_skip.rs:301-406,
    published on an RTX 3090 in bench/results/20261116gpu5/gpu-smoke5/mul_mat_id_skip.json). One op =
    the whole MUL_MAT_ID of F32 activations (Q8_K pass and routing included); 4 weight copies (452 MB,
    more than the MALL) rotate; µs per op = mean over 10 replays of a graph of 8 ops."""
    E, k, n = 128, 2048, 768
    ty = ggml.Type.Q4_K
    copies = [ggml.QTensor(ty, (k, n, E), w.data) for w in make_weights(ggml, torch, ty, k, n * E, 4, seed=77, dev=dev)]
    x = torch.from_numpy(np.random.default_rng(78).uniform(-1, 1, (tokens, 1, k)).astype(np.float32)).to(dev)
    out = torch.empty((tokens, 8, n), device=dev)
    res = {}
    for name, ids_np in rank_share_ids(np, tokens, seed=79).items():
        ids = torch.from_numpy(ids_np).to(dev)
        ws = torch.empty(max(1, ggml.mul_mat_id_workspace_size(copies[0], x, ids)), dtype=torch.uint8, device=dev)
        us = time_graph(torch, lambda i: ggml.mul_mat_id(copies[i % 4], x, ids, out=out, workspace=ws), 8, replays=10)
        valid = int((ids_np >= 0).sum())
        experts = len(set(int(e) for e in ids_np.reshape(-1) if e >= 0))
        res[name] = {"ms": round(us / 1e3, 4), "valid_slots": valid, "experts": experts,
                     "int_TOPS": round(2 * valid * n * k / us / 1e6, 1),
                     "weight_GBps": round(experts * n * ty.row_size(k) / us / 1e3, 1)}
        log(f"rank share {name}: {res[name]}")
    del copies
    torch.cuda.empty_cache()
    ref = {"skip_g1": 0.5855, "skip_g2": 0.3309, "remap_g2": 0.3725, "skip_g4": 0.2230, "remap_g4": 0.2907,
           "skip_g8": 0.1694, "remap_g8": 0.2351, "random_neg90": 0.5984}
    res["reference_rtx3090_ms"] = ref
    res["checks"] = {"skip_g8_below_0.75_skip_g1": res["skip_g8"]["ms"] < 0.75 * res["skip_g1"]["ms"],
                     **{f"skip_g{g}_below_remap_g{g}": res[f"skip_g{g}"]["ms"] < res[f"remap_g{g}"]["ms"]
                        for g in (2, 4, 8)}}
    return res


if __name__ == "__main__":
    main()
