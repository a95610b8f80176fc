#!/usr/bin/env python3
"""MoE-layer benchmark of libfmx on one MI355X.

A step is one MoE-layer forward (router, top-k, gate/up + SwiGLU, down,
top-k weighted combine, gated shared expert) over one batch of tokens
already resident in HBM. Steps cycle over `--layers` copies of the layer's
weights (distinct HBM addresses, 24 by default like a 24-layer model) so that
the weights stream from HBM rather than the 256 MB last-level cache, and run
as captured HIP graphs. Every graph is replayed before the clock starts; the
K timed steps are repeated `--trials` times and the median trial is reported.
Prints ONE JSON line.

Headline workload: Qwen1.5-MoE-A2.7B-shape MoE block, decode batch 8 (seed
2). The same invocation measures the other single-GPU MoE-layer configs
(`--configs`, default all: Qwen1.5 decode batch 1 and 4, prefill 512;
Qwen3-30B-A3B decode batch 1 and 8, prefill 1024), each with its own
roofline, under "configs".

Per-stage timing: graphs of the first j kernel stages of every layer give
each stage's marginal time inside the layer (HIP events on the stream the
kernels run on, each timed section queued behind a spin kernel and
whole-layer graph replays so that it never waits for the host's launches
and runs at the layer's own clocks); the dominant kernel's
average duration (the stages it runs, together) gives the roofline figure.
The same command under `rocprofv3 --kernel-trace --stats` gives the
per-kernel averages that the summaries under profiles/ quote.

`--copy-calibration MIB` instead runs a plain device copy of MIB MiB five
times (for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import subprocess
import sys
import time

METRIC = "MoE-layer tok/s; decode HBM GB/s and prefill MFMA % on 1 MI355X"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
ROOT = os.path.dirname(os.path.abspath(__file__))
HEADLINE = "qwen15_decode_b8"
# the other single-GPU MoE-layer configurations of the benchmark
CONFIGS = ["qwen15_decode_b1", "qwen15_decode_b4", "qwen15_prefill_512", "qwen3_decode_b1",
           "qwen3_decode_b8", "qwen3_prefill_1024"]


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


_SLEEP_CYCLES_PER_MS = None


def gpu_lead(stream, ms: float = 20.0) -> None:
    """Queues about `ms` milliseconds of GPU work on `stream` as ONE bounded
    spin kernel (torch.cuda._sleep, calibrated once with HIP events), so
    that the launches the host queues after it are in place before the GPU
    reaches them: one kernel costs the host one launch, also under a tracing
    profiler that makes every launch slow."""
    global _SLEEP_CYCLES_PER_MS
    import torch

    with torch.cuda.stream(stream):
        if _SLEEP_CYCLES_PER_MS is None:
            torch.cuda._sleep(1000)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            torch.cuda._sleep(10_000_000)
            e1.record(stream)
            torch.cuda.synchronize()
            _SLEEP_CYCLES_PER_MS = 10_000_000 / max(e0.elapsed_time(e1), 1e-3)
        torch.cuda._sleep(int(min(ms * _SLEEP_CYCLES_PER_MS, 2e9)))


def cpu_model() -> str:
    """lscpu's model name, with its family / model / stepping numbers (a
    virtual machine's CPU may name only the product line)."""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        f = {}
        for ln in out.splitlines():
            if ":" in ln:
                k, v = ln.split(":", 1)
                f.setdefault(k.strip(), v.strip())
        if "Model name" in f:
            ids = ", ".join(f"{k.lower()} {f[k]}" for k in ("CPU family", "Model", "Stepping") if f.get(k))
            return f["Model name"] + (f" ({ids})" if ids else "")
    except OSError:
        pass
    return platform.processor() or "unknown"


def host_threads() -> int:
    """Threads this process may use: its CPU affinity, capped by the
    OMP_NUM_THREADS share the environment gives it."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def load_traffic(workload: str, stage: str):
    """HBM bytes per launch of a stage's kernel from the committed rocprofv3
    --pmc summary (profiles/traffic_<workload>.json), if there is one."""
    p = os.path.join(ROOT, "profiles", f"traffic_{workload}.json")
    try:
        with open(p) as f:
            d = json.load(f)
        return d.get("stages", {}).get(stage)
    except (OSError, ValueError):
        return None


def cpu_baseline(wl, y_gpu, inds_gpu, seconds: float):
    """The CPU oracle (C restatement of the reference's MLX CPU semantics,
    fp32 accumulation) timed on this host on a bounded sample of the same
    workload, at 1 thread and at the host's thread share; and, as the
    checker, the GPU output of the timed config against the oracle's."""
    sys.path.insert(0, ROOT)
    import numpy as np

    from flashmlx_amd import workloads as W
    from oracle import oracle as O

    O.build()
    hi = W.host_inputs(wl)
    q = O.quantize
    m = wl.model
    cfg = dict(hidden=m["hidden"], n_experts=m["n_experts"], top_k=m["top_k"], inter=m["inter"],
               shared_inter=m["shared_inter"], norm_topk=m["norm_topk"])
    rq = q if wl.router_quant else (lambda a: a)
    w = dict(router_w=rq(hi.router_w), router_bias=hi.router_bias, gate=q(hi.gate), up=q(hi.up),
             down=q(hi.down))
    if m["shared_inter"]:
        w.update(shared_gate=q(hi.shared_gate), shared_up=q(hi.shared_up),
                 shared_down=q(hi.shared_down), shared_expert_gate_w=rq(hi.shared_expert_gate_w))
    T = wl.tokens
    per_call = T if T <= 16 else 16
    tokens = None if per_call == T else list(range(per_call))
    nproc = host_threads()

    def timed(threads, secs):
        O.set_threads(threads)
        O.moe_block(cfg, w, hi.x, O.ACC_A, tokens=tokens)  # warm-up
        n, t0 = 0, time.perf_counter()
        while True:
            O.moe_block(cfg, w, hi.x, O.ACC_A, tokens=tokens)
            n += 1
            el = time.perf_counter() - t0
            if el >= secs:
                return n, el

    n1, e1 = timed(1, seconds / 2)
    nn, en = timed(nproc, seconds / 2)
    model = cpu_model()
    # parity of the timed config's GPU output (all rows) against the oracle
    O.set_threads(nproc)
    ry, rinds, _ = O.moe_block(cfg, w, hi.x, O.ACC_A)
    g = O.bf16_to_f32(y_gpu).astype(np.float64)
    r = O.bf16_to_f32(ry).astype(np.float64)
    d = np.abs(g - r)
    parity = {
        "vs": "CPU oracle, fp32 accumulation (mode A)",
        "rows": int(T),
        "max_abs": float(d.max()),
        "mean_rel": float((d / np.maximum(np.abs(r), 1e-6)).mean()),
        "rel_l2": float(np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30)),
        "within_rtol_2e-2_atol_1e-2": bool((d <= 1e-2 + 2e-2 * np.abs(r)).all()),
        "routing_bitexact": bool(np.array_equal(inds_gpu, rinds)),
    }
    sample = (f"oracle MoE-layer calls x {per_call} tokens ({'all' if tokens is None else 'first'} of {T}; "
              f"routing over all {T}), fp32 accumulate, on {model}: {nn} calls in {en:.1f}s on {nproc} "
              f"OpenMP threads, {n1} calls in {e1:.1f}s on 1 thread")
    return {
        "value": round(nn * per_call / en, 3),
        "unit": "tok/s",
        "cores": nproc,
        "kind": "port",
        "sample": sample,
        "short_sample": f"oracle MoE block, {per_call}-token calls",
        "single_thread_value": round(n1 * per_call / e1, 3),
        "cpu_model": model,
        "nproc": os.cpu_count(),
    }, parity


def copy_calibration(mib: int) -> None:
    import torch

    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "launches": 5}), flush=True)


def build_layers(wl, R: int, pack: bool):
    """R copies of one layer's weights at distinct addresses (the MLX-layout
    expert arrays released after packing), and x."""
    import torch

    from flashmlx_amd import workloads as W
    from flashmlx_amd.moe import MoEBlock, MoEWeights, QWeight

    block0, x = W.device_block(wl, W.DeviceSynth(wl), pack=pack, drop_mlx=pack)

    def clone(v):
        if v is None:
            return None
        if isinstance(v, QWeight):
            return QWeight(v.w.clone(), v.scales.clone(), v.biases.clone())
        return v.clone()

    def clone_block(b):
        w = b.weights
        nw = MoEWeights(**{f: clone(getattr(w, f)) for f in (
            "router_w", "gate", "up", "down", "shared_gate", "shared_up", "shared_down",
            "shared_expert_gate_w", "router_logit_bias", "packed")})
        return MoEBlock(b.cfg, nw, max_tokens=wl.tokens, pack=False)

    blocks = [block0] + [clone_block(block0) for _ in range(R - 1)]
    torch.cuda.synchronize()
    return blocks, x


def measure(wl, R: int, K: int, Wm: int, trials: int, profile_steps: int, pack: bool = True):
    """Times K steps (layer forwards, cycling over R weight copies) `trials`
    times after Wm warm-up steps; per-stage times from partial-forward
    graphs; the dominant kernel's roofline figure."""
    import torch

    from flashmlx_amd import workloads as W

    m, T = wl.model, wl.tokens
    log(f"workload {wl.key}: {R} layer copies")
    blocks, x = build_layers(wl, R, pack)
    y = torch.empty_like(x)
    per_layer = sum(t.numel() * t.element_size() for t in blocks[0].weight_tensors())

    # reference output (eager) and routing statistics
    blocks[0].forward_into(x, y)
    torch.cuda.synchronize()
    y_ref = y.clone()
    r = blocks[0].routing()
    offs = r["expert_offsets"].cpu().numpy().astype("int64")
    U = int((offs[1:] > offs[:-1]).sum())
    inds = r["inds"].cpu().numpy().view("uint32").copy()

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())

    def capture(fn):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            fn()
        return g

    with torch.cuda.stream(stream):
        for b in blocks:  # warm every layer eagerly before capture
            b.forward_into(x, y)
    torch.cuda.synchronize()

    def run_layers(n):
        for i in range(n):
            blocks[i % R].forward_into(x, y)

    graphs = {R: capture(lambda: run_layers(R))}
    for rem in {K % R, Wm % R} - {0}:
        graphs[rem] = capture(lambda rem=rem: run_layers(rem))
    # every graph that will be timed is replayed before the clock starts, and
    # every replay must reproduce the eager result
    for g in graphs.values():
        with torch.cuda.stream(stream):
            g.replay()
        torch.cuda.synchronize()
    for _ in range(3):
        with torch.cuda.stream(stream):
            graphs[R].replay()
        torch.cuda.synchronize()
        if not torch.equal(y, y_ref):
            raise RuntimeError("graph replay output differs from the eager output")
        with torch.cuda.stream(stream):
            blocks[0].forward_into(x, y)
        torch.cuda.synchronize()

    def run_steps(n):
        with torch.cuda.stream(stream):
            for _ in range(n // R):
                graphs[R].replay()
            if n % R:
                graphs[n % R].replay()

    run_steps(Wm)
    torch.cuda.synchronize()
    times = []
    t0 = time.perf_counter()
    for _ in range(trials):
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        ev0.record(stream)
        run_steps(K)
        ev1.record(stream)
        torch.cuda.synchronize()
        times.append(ev0.elapsed_time(ev1))
    wall = time.perf_counter() - t0
    ms_total = statistics.median(times)
    ms_step = ms_total / K
    tok_s = T * K / (ms_total / 1e3)

    # ---- per-stage timing: graphs of R layers that run only the first j
    # kernel stages; stage j's marginal time inside the layer is the
    # difference of consecutive graphs' times. Each timed section is queued
    # behind a 20 ms spin kernel, so that the host has queued the section's
    # kernels before the GPU reaches them (a graph of short kernels would
    # otherwise wait for the host's launches where launches are slow, under
    # a tracing profiler, and inflate its own stage at the next stage's
    # expense), and behind about 8 ms of whole-layer replays, which bring
    # the clocks back from the spin's one busy wave to the layer's own
    work = W.stage_work(m, T, U, wl.router_bias, packed=pack, router_quant=wl.router_quant)
    stages = [s[0] for s in work]
    reps = max(1, profile_steps // R)
    warm = max(2, int(8.0 / (R * ms_step)) + 1)
    cum = [0.0]
    host_ms = []
    for j in range(1, len(stages) + 1):
        gj = capture(lambda j=j: [blocks[i].forward_partial(x, y, j) for i in range(R)])
        with torch.cuda.stream(stream):
            gj.replay()
        torch.cuda.synchronize()
        tries = []
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            gpu_lead(stream)
            h0 = time.perf_counter()
            with torch.cuda.stream(stream):
                for _ in range(warm):
                    graphs[R].replay()
                e0.record(stream)
                for _ in range(reps):
                    gj.replay()
                e1.record(stream)
                host_ms.append((time.perf_counter() - h0) * 1e3)
            torch.cuda.synchronize()
            tries.append(e0.elapsed_time(e1) / (R * reps))
        cum.append(statistics.median(tries))
        del gj
    dur = [max(cum[j + 1] - cum[j], 1e-6) for j in range(len(stages))]
    stage_us = {s: round(dur[j] * 1e3, 2) for j, s in enumerate(stages)}
    log(f"{wl.key}: stage timing queued {max(host_ms):.2f} ms of launches at most behind a 20 ms spin; "
        f"stages add up to {cum[-1] * 1e3:.2f} us against {ms_step * 1e3:.2f} us per whole layer")

    # the dominant kernel of a whole forward: a kernel that runs several
    # stages as one grid takes their marginal times and work together
    groups = W.kernel_groups(m, T, packed=pack)
    gdur = [sum(dur[i] for i in idx) for _, idx in groups]
    dom = max(range(len(groups)), key=lambda q: gdur[q])
    name, idx = groups[dom]
    sbytes = sum(work[i][1] for i in idx)
    sflops = sum(work[i][2] for i in idx)
    path = W.forward_path(m, T, packed=pack)
    prefill = path != "decode"
    if prefill:
        achieved = sflops / (gdur[dom] * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4)}
    else:
        achieved = sbytes / (gdur[dom] * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4)}
    roof["traffic"] = load_traffic(wl.key, name)
    roof["stage"] = name
    roof["algorithmic_per_launch"] = sflops if prefill else sbytes
    roof["avg_launch_us"] = round(gdur[dom] * 1e3, 2)

    layer_bytes = W.algorithmic_bytes(m, T, U, wl.router_bias, wl.router_quant)
    layer_flops = W.flops(m, T)
    layer = {
        "unique_experts": U,
        "algorithmic_bytes": layer_bytes,
        "hbm_gbps": round(layer_bytes / (ms_step * 1e-3) / 1e9, 1),
        "hbm_frac": round(layer_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "tflops": round(layer_flops / (ms_step * 1e-3) / 1e12, 2),
        "mfma_frac": round(layer_flops / (ms_step * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
        "kernel_path": path,
        "stage_us": stage_us,
        "stage_bytes": {s: b for s, b, _ in work},
        "weight_bytes_per_copy": per_layer,
    }
    res = {
        "workload": f"{m['name']} MoE block, {wl.note}",
        "key": wl.key,
        "tokens": T,
        "seed": wl.seed,
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "steps": K,
        "warmup": Wm,
        "trials": trials,
        "ms_per_step": round(ms_step, 6),
        "us_per_layer": round(ms_step * 1e3, 2),
        "trial_ms": {"median": round(ms_total, 4), "min": round(min(times), 4),
                     "max": round(max(times), 4)},
        "roofline": roof,
        "layer": layer,
        "wall_s": round(wall, 3),
    }
    y_host = y_ref.view(torch.int16).cpu().numpy().view("uint16")
    del blocks, graphs, x, y, y_ref
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res, y_host, inds


# The Nemotron-H MoE block (30B-A3B layer shape: H 2688, 128 experts top-6,
# I 1856, shared 3712, routed_scaling_factor 2.5; random-init 4-bit weights,
# seed 16) at decode batch 1 and 8 and a 512-token prefill.
NH_CONFIGS = {"nh30b_decode_b1": 1, "nh30b_decode_b8": 8, "nh30b_prefill_512": 512}
NH_SEED = 16


def nh_bytes_flops(cfg, T: int, U: int):
    """Algorithmic HBM bytes and flops of one Nemotron-H layer forward of T
    tokens with U distinct experts selected: per expert grid {"fc1_grid",
    "fc2_grid"} the 4-bit weights it streams (0.5625 bytes per weight, the
    unpadded I and Is) and its products; the whole layer adds the router,
    the correction bias and x / y. The decode kernels (T <= 16) stream the
    shared up projection beside the router (D1), the prefill GEMMs in the
    fc1 grid; both run the shared down in the fc2 grid."""
    H, E, k = cfg.hidden_size, cfg.n_routed_experts, cfg.num_experts_per_tok
    I, Is = cfg.moe_intermediate_size, cfg.moe_shared_expert_intermediate_size
    wq = 0.5625
    routed, shared = U * I * H * wq, Is * H * wq
    grid_bytes = {"fc1_grid": int(routed + (0 if T <= 16 else shared)), "fc2_grid": int(routed + shared)}
    grid_flops = {g: 2 * T * k * I * H + 2 * T * Is * H for g in grid_bytes}
    layer_bytes = int(2 * (routed + shared) + E * H * 2 + E * 4 + 2 * T * H * 2)
    layer_flops = 2 * (2 * T * k * I * H + 2 * T * Is * H) + 2 * T * E * H
    return grid_bytes, grid_flops, layer_bytes, layer_flops


def measure_nh(key: str, T: int, R: int, K: int, Wm: int, trials: int, cpu_seconds: float):
    """Times K Nemotron-H layer forwards cycling over R copies of the packed
    weights (captured graphs), then each stage's kernels from stage events
    around eager forwards; the roofline of the dominant expert grid."""
    import numpy as np
    import torch

    from flashmlx_amd import nemotron as N
    from flashmlx_amd.moe import synth_normal_bf16_device

    cfg = N.NhMoEConfig()
    t0 = time.perf_counter()
    w0 = N.synthetic_nh_weights(cfg, NH_SEED)
    w0.pack(cfg)
    host = N.host_weights(w0) if cpu_seconds > 0 else None
    w0.drop_mlx_layout()
    blocks = [N.NhMoEBlock(cfg, w0, T)]
    for _ in range(R - 1):
        wi = N.NhMoEWeights(w0.gate_w, w0.correction_bias, None, None, packed=w0.packed.clone())
        blocks.append(N.NhMoEBlock(cfg, wi, T))
    x = synth_normal_bf16_device((T, cfg.hidden_size), NH_SEED, 7)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    log(f"{key}: {R} layer copies built in {time.perf_counter() - t0:.1f}s")
    blocks[0].forward_into(x, y)
    torch.cuda.synchronize()
    y_ref = y.clone()
    r = blocks[0].routing()
    inds = r["inds"].cpu().numpy().view("uint32").copy()
    U = int(np.unique(inds).size)

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for b in blocks:
            b.forward_into(x, y)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for b in blocks:
            b.forward_into(x, y)
    for _ in range(3):
        with torch.cuda.stream(stream):
            g.replay()
        torch.cuda.synchronize()
        if not torch.equal(y, y_ref):
            raise RuntimeError("graph replay output differs from the eager output")
    reps = max(1, K // R)
    with torch.cuda.stream(stream):
        for _ in range(max(1, Wm // R)):
            g.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(trials):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        with torch.cuda.stream(stream):
            for _ in range(reps):
                g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1))
    ms_total = statistics.median(times)
    ms_step = ms_total / (reps * R)

    # per-stage kernel times: graphs of R layers that run only the first j
    # kernel stages, each timed section queued behind a 20 ms spin kernel
    # (so that it never waits for the host's launches) and about 8 ms of
    # whole-layer replays (the clocks back to the layer's own); stage j's
    # marginal time inside the layer is the difference of consecutive
    # graphs' times
    names = ["router_sort", "fc1_grid", "fc2_grid", "combine"]
    sreps = max(1, 96 // R)
    warm = max(2, int(8.0 / (R * ms_step)) + 1)
    cum = [0.0]
    for j in range(1, len(names) + 1):
        gj = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gj, stream=stream):
            for b in blocks:
                b.forward_partial(x, y, j)
        with torch.cuda.stream(stream):
            gj.replay()
        torch.cuda.synchronize()
        tries = []
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            gpu_lead(stream)
            with torch.cuda.stream(stream):
                for _ in range(warm):
                    g.replay()
                e0.record(stream)
                for _ in range(sreps):
                    gj.replay()
                e1.record(stream)
            torch.cuda.synchronize()
            tries.append(e0.elapsed_time(e1) / (R * sreps))
        cum.append(statistics.median(tries))
        del gj
    stage_ms = {nm: max(cum[j + 1] - cum[j], 1e-6) for j, nm in enumerate(names)}
    grid_bytes, grid_flops, layer_bytes, layer_flops = nh_bytes_flops(cfg, T, U)
    dom = max(("fc1_grid", "fc2_grid"), key=lambda nm: stage_ms[nm])
    dur_s = stage_ms[dom] * 1e-3
    if T <= 16:
        ach = grid_bytes[dom] / dur_s / 1e9
        roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": load_traffic(key, dom),
                "algorithmic_per_launch": grid_bytes[dom]}
    else:
        ach = grid_flops[dom] / dur_s / 1e12
        roof = {"bound": "mfma", "achieved": round(ach, 2), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(ach / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": load_traffic(key, dom),
                "algorithmic_per_launch": grid_flops[dom]}
    # decode: D3's last contributors also form the combine, so the fc2 grid's
    # time includes it (the combine stage is then empty)
    roof["stage"] = dom + (" (D3, combine included)" if T <= 16 and dom == "fc2_grid" else "")
    roof["avg_launch_us"] = round(stage_ms[dom] * 1e3, 2)
    res = {
        "workload": (f"Nemotron-H MoE block (30B-A3B layer shape: H 2688, 128 experts top-6 sigmoid-routed "
                     f"with correction bias, I 1856, shared 3712, relu^2), {T} tokens, seed {NH_SEED}"),
        "kernel_path": "decode kernels D1-D3" if T <= 16 else "router + sort + prefill GEMMs + combine",
        "key": key,
        "tokens": T,
        "value": round(T / (ms_step * 1e-3), 1),
        "unit": "tok/s",
        "us_per_layer": round(ms_step * 1e3, 2),
        "steps": reps * R,
        "trials": trials,
        "roofline": roof,
        "layer": {"unique_experts": U, "algorithmic_bytes": layer_bytes,
                  "hbm_gbps": round(layer_bytes / (ms_step * 1e-3) / 1e9, 1),
                  "tflops": round(layer_flops / (ms_step * 1e-3) / 1e12, 2),
                  "stage_us": {nm: round(v * 1e3, 2) for nm, v in stage_ms.items()}},
    }
    log(f"{key}: {res['us_per_layer']} us/layer, {dom} {roof['achieved']} {roof['unit']}")
    if cpu_seconds > 0:
        res["cpu_baseline"] = nh_cpu_baseline(cfg, host, x, y_ref, inds, T, cpu_seconds)
    del blocks, g
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


def nh_cpu_baseline(cfg, host, x, y_gpu, inds_gpu, T: int, seconds: float):
    """The oracle's Nemotron-H block on this host on a bounded sample (the
    first token of the workload per call, fp32 accumulation), plus the GPU
    output's parity against it on up to 8 tokens."""
    sys.path.insert(0, ROOT)
    import numpy as np
    import torch

    from oracle import oracle as O

    O.build()
    oc = cfg.oracle_cfg()
    xh = x.view(torch.int16).cpu().numpy().view(np.uint16)
    nproc = host_threads()
    O.set_threads(nproc)
    O.nh_moe_block(oc, host, xh[:1], O.ACC_A)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        O.nh_moe_block(oc, host, xh[:1], O.ACC_A)
        n += 1
    el = time.perf_counter() - t0
    m = min(T, 8)
    ry, rinds, _ = O.nh_moe_block(oc, host, xh[:m], O.ACC_F64)
    g = O.bf16_to_f32(y_gpu.view(torch.int16).cpu().numpy().view(np.uint16)[:m]).astype(np.float64)
    rr = O.bf16_to_f32(ry).astype(np.float64)
    return {
        "value": round(n / el, 3),
        "unit": "tok/s",
        "cores": nproc,
        "kind": "port",
        "sample": (f"oracle Nemotron-H block on 1 token per call ({n} calls in {el:.1f}s, {nproc} OpenMP "
                   f"threads, fp32 accumulation) on {cpu_model()}"),
        "parity_rows": m,
        "parity_rel_l2": float(np.linalg.norm(g - rr) / max(np.linalg.norm(rr), 1e-30)),
        "routing_bitexact": bool(np.array_equal(inds_gpu[:m], rinds)),
    }


# The 24-layer Qwen1.5-MoE-A2.7B-shape decoder stack (random-init 4-bit
# weights, seed 5): a 256-token prompt, then 128 greedy tokens, at batch 1 and 4
STACK_CONFIGS = {"c4_stack_b1": 1, "c4_stack_b4": 4, "c4_stack_b8": 8}
STACK_PROMPT, STACK_NEW, STACK_SEED = 256, 128, 5


def stack_step_bytes(cfg, B: int, pos: int, unique_per_layer) -> int:
    """Algorithmic HBM bytes of one decode step of the stack: every layer's
    attention weights and its routed (unique) and shared experts' weights at
    0.5625 B per weight, router and norms, the KV cache read up to pos and
    written at pos, the lm_head, embedding rows and logits."""
    H, V, hd = cfg.hidden_size, cfg.vocab_size, cfg.hd
    nh, nkv = cfg.num_attention_heads, cfg.num_key_value_heads
    m = cfg.moe
    q = lambda n, k: n * k * 9 // 16  # noqa: E731
    exp = 3 * q(m.moe_intermediate_size, H)
    shared = 3 * q(m.shared_expert_intermediate_size, H) + H * 2 if m.shared_expert_intermediate_size else 0
    attn = q(cfg.n_qkv, H) + cfg.n_qkv * 2 + q(H, nh * hd)
    kv = B * 2 * nkv * hd * 2 * (pos + 2)
    layer = [attn + U * exp + shared + m.num_experts * H * 2 + 2 * H * 2 + kv for U in unique_per_layer]
    return int(sum(layer) + q(V, H) + B * H * 2 + B * V * 2 + H * 2)


def measure_stack(batches, trials: int, cpu_seconds: float):
    """Prefill of a 256-token prompt and 128 greedy tokens per sequence on
    the 24-layer stack, each as captured HIP graphs (one graph for the
    prefill and the first token, one for a decode step that reads the device
    cache offsets and advances them): the median of `trials` runs."""
    import numpy as np
    import torch

    from flashmlx_amd import model as M

    cfg = M.ModelConfig(max_position_embeddings=512)
    V = cfg.vocab_size
    t0 = time.perf_counter()
    w = M.synthetic_model(cfg, STACK_SEED, keep_mlx=cpu_seconds > 0)
    log(f"stack: 24-layer weights built in {time.perf_counter() - t0:.1f}s")
    rng = np.random.default_rng(STACK_SEED)
    res = {}
    solo = M.DecoderModel(cfg, w, 1, STACK_PROMPT + STACK_NEW, STACK_PROMPT)

    def alone(prompt):
        """Each prompt row generated on its own at batch 1 (eager)."""
        return torch.cat([solo.generate(prompt[b:b + 1].contiguous(), STACK_NEW)
                          for b in range(prompt.shape[0])])

    for B in batches:
        max_seq = STACK_PROMPT + STACK_NEW
        dm = M.DecoderModel(cfg, w, B, max_seq, B * STACK_PROMPT)
        prompt = torch.from_numpy(rng.integers(0, V, (B, STACK_PROMPT)).astype(np.int32)).cuda()
        logits = torch.empty((B, V), dtype=torch.bfloat16, device="cuda")
        tok = torch.empty((B, 1), dtype=torch.int32, device="cuda")
        offs = torch.full((B,), STACK_PROMPT, dtype=torch.int32, device="cuda")
        # eager reference generation and the routing of one decode step
        ref = dm.generate(prompt, STACK_NEW)
        rt = dm.routing_buffer(B)
        dm.forward(ref[:, :1].contiguous(), STACK_PROMPT, routing=rt)
        uniq = [int(np.unique(r.numpy()).size) for r in rt.cpu()]
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())

        def prefill():
            dm.forward_into(prompt, 0, logits)
            dm.greedy(logits, tok.view(-1))

        def step():
            dm.forward_into(tok, offs, logits)
            dm.greedy(logits, tok.view(-1), offs, 1)

        with torch.cuda.stream(stream):
            prefill()
            step()
        torch.cuda.synchronize()
        gp, gs = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
        with torch.cuda.graph(gp, stream=stream):
            prefill()
        with torch.cuda.graph(gs, stream=stream):
            step()
        pre, dec, last_ok = [], [], True
        for _ in range(trials + 1):
            offs.fill_(STACK_PROMPT)
            torch.cuda.synchronize()
            e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
            e0.record(stream)
            with torch.cuda.stream(stream):
                gp.replay()
                e1.record(stream)
                for _ in range(STACK_NEW - 1):
                    gs.replay()
                e2.record(stream)
            torch.cuda.synchronize()
            pre.append(e0.elapsed_time(e1))
            dec.append(e1.elapsed_time(e2))
            last_ok &= bool(torch.equal(tok.view(-1), ref[:, -1]))
        pre, dec = pre[1:], dec[1:]  # the first run warms the graphs
        pm, dmed = statistics.median(pre), statistics.median(dec)
        step_ms = dmed / (STACK_NEW - 1)
        pos = STACK_PROMPT + STACK_NEW // 2
        sb = stack_step_bytes(cfg, B, pos, uniq)
        res[f"c4_stack_b{B}"] = {
            "workload": (f"24-layer Qwen1.5-MoE-A2.7B-shape decoder stack, batch {B}: {STACK_PROMPT}-token "
                         f"prompt, {STACK_NEW} greedy tokens, seed {STACK_SEED}"),
            "value": round(B * (STACK_NEW - 1) / (dmed / 1e3), 1),
            "unit": "tok/s (decode)",
            "e2e_tok_s": round(B * STACK_NEW / ((pm + dmed) / 1e3), 1),
            "prefill_ms": round(pm, 3),
            "prefill_tok_s": round(B * STACK_PROMPT / (pm / 1e3), 1),
            "decode_ms_per_step": round(step_ms, 4),
            "trials": trials,
            "graph_tokens_equal_eager": last_ok,
            "roofline": {"bound": "hbm", "achieved": round(sb / (step_ms * 1e-3) / 1e9, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(sb / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                         "algorithmic_per_step": sb,
                         "note": f"unique experts per layer from the step at position {STACK_PROMPT}: "
                                 f"mean {np.mean(uniq):.1f}"},
        }
        log(f"stack B={B}: prefill {pm:.2f} ms, decode {step_ms * 1e3:.1f} us/step")
        res[f"c4_stack_b{B}"]["scheduler"] = measure_scheduler(
            cfg, w, prompt, ref if B == 1 else alone(prompt), max_seq)
        del dm, gp, gs
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    del solo
    if cpu_seconds > 0:
        res["c4_stack_b1"]["cpu_baseline"] = stack_cpu_baseline(cfg, w, cpu_seconds)
    return res


def measure_scheduler(cfg, w, prompt, alone, max_seq: int) -> dict:
    """The same B requests through the native server loop (BatchScheduler:
    batch-1 prefills into pool slots, then batched decode steps with a host
    round trip per step): wall-clock tok/s of the whole run, the decode
    steps' mean wall time once every request is admitted, and whether each
    request's tokens equal that prompt generated alone at batch 1 (`alone`
    [B, n] int32: the property the scheduler guarantees, since every decode
    kernel computes a row on its own for batches of up to 16)."""
    from flashmlx_amd import model as M

    B = prompt.shape[0]
    rows = prompt.cpu().numpy().tolist()
    sched = M.BatchScheduler(cfg, w, B, max_seq, STACK_PROMPT)
    out = {}
    runs = []
    for _ in range(2):  # the first run captures the decode graph
        ids = [sched.submit(r, STACK_NEW) for r in rows]
        toks = {i: [] for i in ids}
        t0 = time.perf_counter()
        steps = []
        while sched.has_work():
            ts = time.perf_counter()
            for rid, t in sched.step().items():
                toks[rid].extend(t)
            steps.append(time.perf_counter() - ts)
        wall = time.perf_counter() - t0
        sched.drain_completed()
        runs.append((wall, steps[1:], toks, ids))
    wall, dsteps, toks, ids = runs[-1]
    want = alone.cpu().numpy()
    out["tok_s"] = round(B * STACK_NEW / wall, 1)
    out["wall_ms"] = round(wall * 1e3, 2)
    out["decode_ms_per_step_wall"] = round(1e3 * sum(dsteps) / max(len(dsteps), 1), 4)
    out["tokens_equal_alone_b1"] = all(toks[i] == want[b].tolist() for b, i in enumerate(ids))
    sched.close()
    log(f"scheduler B={B}: {out['tok_s']} tok/s, decode step {out['decode_ms_per_step_wall']} ms wall")
    return out


def stack_cpu_baseline(cfg, w, seconds: float):
    """The oracle's DecoderStack (24 layers, fp32 accumulation) on this host:
    decode steps at batch 1 after an 8-token prompt, for about `seconds`."""
    sys.path.insert(0, ROOT)
    import numpy as np

    from flashmlx_amd import model as M
    from oracle import oracle as O

    O.build()
    hw = M.host_weights(cfg, w)
    nproc = host_threads()
    O.set_threads(nproc)
    st = O.DecoderStack(M.oracle_config(cfg, 64), hw, 1)
    ids = np.random.default_rng(STACK_SEED).integers(0, cfg.vocab_size, (1, 8))
    lg = st.forward(ids, 0)
    n, t0, pos = 0, time.perf_counter(), 8
    while time.perf_counter() - t0 < seconds and pos < 64:
        nxt = np.array([[int(np.argmax(O.bf16_to_f32(lg[0])))]])
        lg = st.forward(nxt, pos)
        pos += 1
        n += 1
    el = time.perf_counter() - t0
    return {"value": round(n / el, 3), "unit": "tok/s (decode, batch 1)", "cores": nproc, "kind": "port",
            "sample": f"oracle DecoderStack, 24 layers: {n} decode steps in {el:.1f}s after an 8-token "
                      f"prompt, on {cpu_model()}, {nproc} OpenMP threads"}


# The standalone operators (fmx_gather_qmm, fmx_quantized_matmul: the drop-in
# for switch_mlp's and shared_expert_mlp's MLX calls, model.cpp:703-721 and
# :741-747) at the Qwen1.5-MoE-A2.7B shapes, on the MLX layout (their general
# GEMM path). Decode cases stream their weights (GB/s), prefill cases are
# priced in flops (TFLOP/s).
def measure_ops(trials: int = 5, calls: int = 20) -> dict:
    import ctypes as C

    import torch

    from flashmlx_amd import _lib
    from flashmlx_amd import moe as Mo

    lib = _lib.load()
    H, E, I, Is, k = 2048, 60, 1408, 5632, 4
    w = Mo.synth_normal_bf16_device((E, I, H), 11, 60, 0.0, 0.02)
    gq, gs, gb = Mo.quantize(w)
    del w
    w = Mo.synth_normal_bf16_device((Is, H), 11, 61, 0.0, 0.02)
    sq, ss, sb = Mo.quantize(w)
    del w
    gen = torch.Generator().manual_seed(5)

    def graph_time(fn) -> float:
        """GPU us per call: a HIP graph of `calls` calls, replayed."""
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(3):
                fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(calls):
                fn()
        for _ in range(2):
            g.replay()
        torch.cuda.synchronize()
        ts = []
        for _ in range(trials):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            g.replay()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1000.0 / calls)
        return statistics.median(ts)

    def gather_case(x, rhs, sorted_idx: bool):
        ax, aw, asc, abi, ar = Mo._arr(x), Mo._packed(gq), Mo._arr(gs), Mo._arr(gb), Mo._index(rhs)
        shp = _lib.FmxArray()
        _lib.check(lib.fmx_gather_qmm_out_shape(C.byref(ax), C.byref(aw), None, C.byref(ar), 1, 64, 4,
                                                C.byref(shp)))
        out = torch.empty(Mo._shape(shp), dtype=torch.bfloat16, device="cuda")
        ao = Mo._arr(out)
        wsz = lib.fmx_gather_qmm_workspace_size(C.byref(ax), C.byref(aw), None, C.byref(ar))
        wbuf = torch.empty(max(wsz, 1), dtype=torch.uint8, device="cuda")
        return lambda: _lib.check(lib.fmx_gather_qmm(
            C.byref(ax), C.byref(aw), C.byref(asc), C.byref(abi), None, C.byref(ar), 1, 64, 4, b"affine",
            int(sorted_idx), C.byref(ao), wbuf.data_ptr(), wsz, Mo._stream())), (x, rhs, out, wbuf)

    def qmm_case(x):
        ax, aw, asc, abi = Mo._arr(x), Mo._packed(sq), Mo._arr(ss), Mo._arr(sb)
        shp = _lib.FmxArray()
        _lib.check(lib.fmx_quantized_matmul_out_shape(C.byref(ax), C.byref(aw), 1, 64, 4, C.byref(shp)))
        out = torch.empty(Mo._shape(shp), dtype=torch.bfloat16, device="cuda")
        ao = Mo._arr(out)
        wsz = lib.fmx_quantized_matmul_workspace_size(C.byref(ax), C.byref(aw))
        wbuf = torch.empty(max(wsz, 1), dtype=torch.uint8, device="cuda")
        return lambda: _lib.check(lib.fmx_quantized_matmul(
            C.byref(ax), C.byref(aw), C.byref(asc), C.byref(abi), 1, 64, 4, b"affine", C.byref(ao),
            wbuf.data_ptr(), wsz, Mo._stream())), (x, out, wbuf)

    def rand_x(shape):
        return torch.randn(shape, generator=gen).to(torch.bfloat16).cuda()

    res = {}
    # decode: switch_mlp's unsorted gate projection for 8 tokens x top-4
    B = 8
    inds = torch.stack([torch.randperm(E, generator=gen)[:k] for _ in range(B)]).to(torch.int32)
    fn, keep = gather_case(rand_x((B, 1, 1, 1, H)), inds.reshape(B, 1, k).cuda(), False)
    us = graph_time(fn)
    U = int(torch.unique(inds).numel())
    byts = U * I * H * 9 // 16 + B * H * 2 + B * k * I * 2
    res["gather_qmm_decode_b8"] = {"shape": f"x [8,1,1,1,{H}], w [{E},{I},{H}/8], rhs [8,1,{k}]", "us": round(us, 2),
                                   "algorithmic_bytes": byts, "GB_s": round(byts / us / 1e3, 1),
                                   "hbm_frac": round(byts / us / 1e3 / 8000.0, 4)}
    # prefill: the sorted call over 512 tokens x top-4 (rows already gathered)
    n = 512 * k
    rhs = torch.sort(torch.randint(0, E, (n,), generator=gen)).values.to(torch.int32)
    fn, keep2 = gather_case(rand_x((n, 1, H)), rhs.cuda(), True)
    us = graph_time(fn)
    fl = 2.0 * n * I * H
    res["gather_qmm_prefill_512"] = {"shape": f"x [{n},1,{H}] sorted, w [{E},{I},{H}/8]", "us": round(us, 2),
                                     "flops": fl, "TFLOP_s": round(fl / us / 1e6, 2),
                                     "mfma_frac": round(fl / us / 1e6 / 2500.0, 4)}
    for T, name in ((8, "quantized_matmul_decode_b8"), (512, "quantized_matmul_prefill_512")):
        fn, keep3 = qmm_case(rand_x((T, H)))
        us = graph_time(fn)
        if T <= 16:
            byts = Is * H * 9 // 16 + T * H * 2 + T * Is * 2
            res[name] = {"shape": f"x [{T},{H}], w [{Is},{H}/8]", "us": round(us, 2), "algorithmic_bytes": byts,
                         "GB_s": round(byts / us / 1e3, 1), "hbm_frac": round(byts / us / 1e3 / 8000.0, 4)}
        else:
            fl = 2.0 * T * Is * H
            res[name] = {"shape": f"x [{T},{H}], w [{Is},{H}/8]", "us": round(us, 2), "flops": fl,
                         "TFLOP_s": round(fl / us / 1e6, 2), "mfma_frac": round(fl / us / 1e6 / 2500.0, 4)}
        del keep3
    for key, v in res.items():
        log(f"op {key}: {v['us']} us")
    return {"workload": "standalone fmx_gather_qmm / fmx_quantized_matmul on the MLX layout, "
                        "Qwen1.5-MoE-A2.7B shapes, HIP graphs of 20 calls", "cases": res}


def _r(v, nd=4):
    return None if v is None else round(float(v), nd)


def compact_config(key: str, c: dict) -> dict:
    """The headline figures of one measured configuration as a flat object:
    throughput, per-layer (or per-step) time, the dominant kernel's roofline
    fraction with the figures it is computed from, and the check results."""
    if "cases" in c:  # the standalone operators
        return {k: {"us": v["us"], "frac": v.get("hbm_frac", v.get("mfma_frac")),
                    "bound": "hbm" if "hbm_frac" in v else "mfma"} for k, v in c["cases"].items()}
    rf = c.get("roofline", {})
    o = {"value": c.get("value"), "unit": c.get("unit")}
    if "decode_ms_per_step" in c:  # decoder stack
        sch = c.get("scheduler", {})
        o.update(decode_ms_per_step=c["decode_ms_per_step"], prefill_ms=c.get("prefill_ms"),
                 e2e_tok_s=c.get("e2e_tok_s"), frac=rf.get("frac"), achieved=rf.get("achieved"),
                 algorithmic_per_step=rf.get("algorithmic_per_step"),
                 graph_tokens_equal_eager=c.get("graph_tokens_equal_eager"),
                 sched_tok_s=sch.get("tok_s"), sched_tokens_equal_alone_b1=sch.get("tokens_equal_alone_b1"))
    else:
        ly = c.get("layer", {})
        o.update(us_per_layer=c.get("us_per_layer"), U=ly.get("unique_experts"), bound=rf.get("bound"),
                 frac=rf.get("frac"), achieved=rf.get("achieved"), stage=rf.get("stage"),
                 avg_launch_us=rf.get("avg_launch_us"), algorithmic_per_launch=rf.get("algorithmic_per_launch"),
                 traffic=rf.get("traffic"))
        if rf.get("bound") == "mfma" and "mfma_frac" in ly:
            o["layer_mfma_frac"] = ly["mfma_frac"]
        if "hbm_frac" in ly:
            o["layer_hbm_frac"] = ly["hbm_frac"]
    cb = c.get("cpu_baseline")
    if cb:
        o["cpu_tok_s"] = cb.get("value")
        if "parity_rel_l2" in cb:
            o["parity_rel_l2"] = _r(cb["parity_rel_l2"], 8)
            o["routing_bitexact"] = cb.get("routing_bitexact")
    return {k: v for k, v in o.items() if v is not None}


ROW_FIELDS = {
    "moe": "us/layer, kernel frac, layer frac (HBM decode, MFMA prefill), U",
    "stack": "ms/step, HBM frac, tok/s, tokens ok",
    "nemotron": "us/layer, frac, rel L2, routing exact",
    "ops": "us/call",
}


def config_row(c: dict):
    """A compact config record (compact_config) as the short array that
    ROW_FIELDS describes."""
    if "us_per_layer" not in c and "decode_ms_per_step" not in c:  # the standalone operators
        short = lambda k: k.replace("quantized_matmul", "qmm").replace("gather_qmm", "gqmm").replace(  # noqa: E731
            "_decode", "").replace("_prefill", "")
        return {short(k): v["us"] for k, v in c.items()}
    if "decode_ms_per_step" in c:
        return [c["decode_ms_per_step"], c.get("frac"), c["value"],
                bool(c.get("graph_tokens_equal_eager")) and bool(c.get("sched_tokens_equal_alone_b1"))]
    if "routing_bitexact" in c:
        return [c["us_per_layer"], c.get("frac"), _r(c.get("parity_rel_l2"), 6), bool(c["routing_bitexact"])]
    return [c["us_per_layer"], c.get("frac"), c.get("layer_mfma_frac", c.get("layer_hbm_frac")), c.get("U")]


def short_cpu(cpu):
    """The CPU baseline object of the printed line (the full one, with the
    single-thread figure and the sample's counts, goes to stderr)."""
    if not cpu:
        return cpu
    return {"value": cpu["value"], "unit": cpu["unit"], "cores": cpu["cores"], "kind": cpu["kind"],
            "sample": cpu["short_sample"], "single_thread_value": cpu["single_thread_value"]}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2400)
    ap.add_argument("--warmup", type=int, default=240)
    ap.add_argument("--trials", type=int, default=20, help="timed repetitions of --steps (median)")
    ap.add_argument("--workload", default=HEADLINE)
    ap.add_argument("--configs", default="all",
                    help="other MoE-layer configs measured in the same run: all, none or a comma list")
    ap.add_argument("--layers", type=int, default=24, help="weight copies cycled over")
    ap.add_argument("--profile-steps", type=int, default=96,
                    help="steps of each per-stage timing section (timed three times, median); small enough "
                         "that a section's launches fit the stream's queue behind the spin kernel")
    ap.add_argument("--cpu-seconds", type=float, default=16.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-pack", action="store_true",
                    help="MLX-layout weights only (no fmx_pack_expert_weights re-layout)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB")
    ap.add_argument("--stack", default="all",
                    help="decoder-stack configs measured in the same run: all, none or a comma list "
                         "(c4_stack_b1, c4_stack_b4, c4_stack_b8)")
    ap.add_argument("--stack-trials", type=int, default=5)
    ap.add_argument("--ops", default="all", choices=["all", "none"],
                    help="time the standalone fmx_gather_qmm / fmx_quantized_matmul")
    ap.add_argument("--detail", default="",
                    help="also write the full per-config results (stage times, bytes, samples) to this "
                         "JSON file; the printed line holds each config's headline figures")
    ap.add_argument("--nh", default="all",
                    help="Nemotron-H block configs measured in the same run: all, none or a comma list "
                         "(nh30b_decode_b1, nh30b_decode_b8, nh30b_prefill_512)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs the MoE layer on one GPU only (one GPU per "
                                   "box); run bench.py with --gpus 1",
                          "n_gpus": args.gpus}), flush=True)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return

    sys.path.insert(0, ROOT)
    import torch

    from flashmlx_amd import workloads as W

    torch.cuda.set_device(0)
    R = max(1, args.layers)
    pack = not args.no_pack
    wl = W.WORKLOADS[args.workload]
    K, Wm = args.steps, args.warmup
    head, y_head, inds_head = measure(wl, R, K, Wm, args.trials, args.profile_steps, pack)

    if args.configs == "all":
        keys = [k for k in CONFIGS if k != wl.key]
    elif args.configs == "none":
        keys = []
    else:
        keys = [k for k in args.configs.split(",") if k and k != wl.key]
    configs = {}
    for key in keys:
        c = W.WORKLOADS[key]
        # prefill steps are ~20x longer than decode steps: a tenth as many
        steps = K if c.tokens <= 16 else max(R, K // 10)
        warm = Wm if c.tokens <= 16 else max(R, Wm // 10)
        configs[key], _, _ = measure(c, R, steps, warm, args.trials, args.profile_steps, pack)

    skeys = list(STACK_CONFIGS) if args.stack == "all" else (
        [] if args.stack == "none" else [k for k in args.stack.split(",") if k])
    if skeys:
        stack = measure_stack([STACK_CONFIGS[k] for k in skeys], args.stack_trials,
                              0.0 if args.no_cpu_baseline else args.cpu_seconds)
        configs.update(stack)

    nkeys = list(NH_CONFIGS) if args.nh == "all" else (
        [] if args.nh == "none" else [k for k in args.nh.split(",") if k])
    for key in nkeys:
        T = NH_CONFIGS[key]
        steps = 480 if T <= 16 else 48
        configs[key] = measure_nh(key, T, 8, steps, max(8, steps // 10), 5,
                                  0.0 if args.no_cpu_baseline else min(args.cpu_seconds, 6.0))

    if args.ops == "all":
        configs["ops_qwen15"] = measure_ops()

    cpu, parity, full_cpu = None, None, None
    if not args.no_cpu_baseline:
        log("timing the CPU oracle")
        try:
            cpu, parity = cpu_baseline(wl, y_head, inds_head, args.cpu_seconds)
            full_cpu = cpu
        except Exception as e:  # noqa: BLE001
            log(f"CPU baseline failed: {e}")

    out = {
        "metric": METRIC,
        "value": head["value"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": Wm,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) bf16 x, N(0,0.02) weights quantized affine 4-bit g64",
        "config": {
            "workload": head["workload"],
            "key": wl.key,
            "tokens": wl.tokens,
            "seed": wl.seed,
            "layer_copies": R,
            "timing": f"HIP graphs, median of {args.trials} trials of {K} steps",
        },
        "roofline": head["roofline"],
        "cpu_baseline": short_cpu(cpu),
    }
    lay = head["layer"]
    out["layer"] = {"us": head["us_per_layer"], "U": lay["unique_experts"], "hbm_frac": lay["hbm_frac"]}
    if parity:
        out["parity"] = {"rel_l2": _r(parity["rel_l2"], 6), "max_abs": _r(parity["max_abs"], 6),
                         "within_tol": parity["within_rtol_2e-2_atol_1e-2"],
                         "routing_bitexact": parity["routing_bitexact"]}
    compact = {k: compact_config(k, c) for k, c in configs.items()}
    # every other config's headline figures as short arrays (fields in ROW_FIELDS), so that the
    # whole line stays within about 2 KB
    out["configs"] = {k: config_row(c) for k, c in compact.items()}
    out["config_fields"] = ROW_FIELDS
    if args.detail:
        full = dict(out, layer=head["layer"], trial_ms=head["trial_ms"], wall_s=head["wall_s"],
                    parity=parity, configs=configs, cpu_baseline_full=full_cpu)
        with open(args.detail, "w") as f:
            json.dump(full, f, indent=1)
        log(f"full results written to {args.detail}")
    for k, c in configs.items():  # every config's full record on stderr, one line each
        log(f"detail {k}: " + json.dumps(c))
    log("detail cpu_baseline: " + json.dumps(full_cpu))
    for k, c in compact.items():  # then a short line each
        log(f"summary {k}: " + json.dumps(c, separators=(",", ":")))
    print(json.dumps(out, separators=(",", ":")), flush=True)


if __name__ == "__main__":
    main()
