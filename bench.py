#!/usr/bin/env python3
"""MoE-layer benchmark of libfmx on one MI355X.

A step is one MoE-layer forward (router, top-k, gate/up + SwiGLU, down,
top-k weighted combine, gated shared expert) over one batch of tokens
already resident in HBM. Steps cycle over `--layers` copies of the layer's
weights (distinct HBM addresses, 24 by default like a 24-layer model) so that
the weights stream from HBM rather than the 256 MB last-level cache, and run
as a captured HIP graph. Prints ONE JSON line.

Default workload: Qwen1.5-MoE-A2.7B-shape MoE block, decode batch 8 (seed 2).
Other workloads: --workload (flashmlx_amd/workloads.py).

Per-stage timing: graphs of the first j kernel stages of every layer give
each stage's marginal time (HIP events on the stream the kernels run on);
the dominant kernel's average duration (the stages it runs, together) gives
the roofline figure. The same
command under `rocprofv3 --kernel-trace --stats` gives the per-kernel
averages that the summaries under profiles/ quote.

`--copy-calibration MIB` instead runs a plain device copy of MIB MiB five
times (for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import subprocess
import sys
import time

METRIC = "MoE-layer tok/s; decode HBM GB/s and prefill MFMA % on 1 MI355X"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
ROOT = os.path.dirname(os.path.abspath(__file__))


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        for ln in out.splitlines():
            if ln.startswith("Model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


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


def cpu_baseline(wl, seconds: float):
    """The CPU oracle (C restatement of the reference's MLX CPU semantics,
    fp32 accumulation) timed on this host on a bounded sample of the same
    workload."""
    sys.path.insert(0, ROOT)
    from flashmlx_amd import workloads as W
    from oracle import oracle as O

    O.build()
    hi = W.host_inputs(wl)
    q = O.quantize
    m = wl.model
    cfg = dict(hidden=m["hidden"], n_experts=m["n_experts"], top_k=m["top_k"], inter=m["inter"],
               shared_inter=m["shared_inter"], norm_topk=m["norm_topk"])
    w = dict(router_w=hi.router_w, router_bias=hi.router_bias, gate=q(hi.gate), up=q(hi.up),
             down=q(hi.down))
    if m["shared_inter"]:
        w.update(shared_gate=q(hi.shared_gate), shared_up=q(hi.shared_up),
                 shared_down=q(hi.shared_down), shared_expert_gate_w=hi.shared_expert_gate_w)
    T = wl.tokens
    # bounded sample: whole calls for small batches, a token slice for prefill
    per_call = T if T <= 16 else 16
    tokens = None if per_call == T else list(range(per_call))
    O.moe_block(cfg, w, hi.x, O.ACC_A, tokens=tokens)  # warm-up
    n = 0
    t0 = time.perf_counter()
    while True:
        O.moe_block(cfg, w, hi.x, O.ACC_A, tokens=tokens)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {
        "value": round(n * per_call / el, 3),
        "unit": "tok/s",
        "cores": O.get_threads(),
        "kind": "port",
        "sample": (f"{n} oracle MoE-layer calls x {per_call} tokens ({'all' if tokens is None else 'first'} "
                   f"of {T}; routing over all {T}) in {el:.1f}s, fp32 accumulate, "
                   f"{O.get_threads()} OpenMP threads on {cpu_model()}"),
    }


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


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2400)
    ap.add_argument("--warmup", type=int, default=240)
    ap.add_argument("--workload", default="qwen15_decode_b8")
    ap.add_argument("--layers", type=int, default=24, help="weight copies cycled over")
    ap.add_argument("--profile-steps", type=int, default=480, help="steps of the per-stage timing pass")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-pack", action="store_true",
                    help="MLX-layout weights only (no fmx_pack_expert_weights re-layout)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs the MoE layer on one GPU only; "
                                   "run bench.py with --gpus 1",
                          "n_gpus": args.gpus}), flush=True)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return

    sys.path.insert(0, ROOT)
    import torch

    from flashmlx_amd import workloads as W
    from flashmlx_amd.moe import MoEBlock, MoEWeights, QWeight

    wl = W.WORKLOADS[args.workload]
    m = wl.model
    T = wl.tokens
    torch.cuda.set_device(0)

    log(f"workload {wl.key}: generating inputs")
    hi = W.host_inputs(wl)
    block0, x = W.device_block(wl, hi, pack=not args.no_pack)
    del hi

    def clone_q(q):
        return QWeight(q.w.clone(), q.scales.clone(), q.biases.clone())

    def clone_block(b):
        w = b.weights
        nw = MoEWeights(router_w=w.router_w.clone(), gate=clone_q(w.gate), up=clone_q(w.up),
                        down=clone_q(w.down))
        if w.router_logit_bias is not None:
            nw.router_logit_bias = w.router_logit_bias.clone()
        if w.shared_gate is not None:
            nw.shared_gate, nw.shared_up, nw.shared_down = (clone_q(w.shared_gate), clone_q(w.shared_up),
                                                            clone_q(w.shared_down))
            nw.shared_expert_gate_w = w.shared_expert_gate_w.clone()
        if w.packed is not None:
            nw.packed = w.packed.clone()
        return MoEBlock(b.cfg, nw, max_tokens=T, pack=False)

    R = max(1, args.layers)
    blocks = [block0] + [clone_block(block0) for _ in range(R - 1)]
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    per_layer = sum(t.numel() * t.element_size() for t in blocks[0].weight_tensors())
    log(f"{R} layer copies, {R * per_layer / 2**30:.2f} GiB of weights")

    # reference output (eager) and routing statistics
    blocks[0].forward_into(x, y)
    torch.cuda.synchronize()
    y_ref = y.clone()
    r = blocks[0].routing()
    offs = r["expert_offsets"].cpu().numpy().astype("int64")
    U = int((offs[1:] > offs[:-1]).sum())

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

    K, Wm = args.steps, args.warmup
    graphs = {R: capture(lambda: run_layers(R))}
    for rem in {K % R, Wm % R} - {0}:
        graphs[rem] = capture(lambda rem=rem: run_layers(rem))
    # every replay must reproduce the eager result
    for _ in range(3):
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
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    run_steps(K)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_total = ev0.elapsed_time(ev1)
    ms_step = ms_total / K
    tok_s = T * K / (ms_total / 1e3)

    # ---- per-stage timing: graphs of R layers that run only the first j
    # kernel stages (j = 1..len(stages)); stage j's marginal time inside the layer is
    # the difference of consecutive graphs' times (HIP events on the kernels'
    # stream around each replay)
    work = W.stage_work(m, T, U, wl.router_bias, packed=not args.no_pack)
    stages = [s[0] for s in work]
    reps = max(1, args.profile_steps // R)
    cum = [0.0]
    ns = len(stages)
    for j in range(1, ns + 1):
        gj = capture(lambda j=j: [blocks[i].forward_partial(x, y, j) for i in range(R)])
        with torch.cuda.stream(stream):
            gj.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        with torch.cuda.stream(stream):
            for _ in range(reps):
                gj.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        cum.append(e0.elapsed_time(e1) / (R * reps))
        del gj
    dur = [max(cum[j + 1] - cum[j], 1e-6) for j in range(ns)]
    stage_us = {s: round(dur[j] * 1e3, 2) for j, s in enumerate(stages)}

    # the dominant kernel of a whole forward: a kernel that runs several
    # stages as one grid takes their marginal times and work together
    groups = W.kernel_groups(m, T, packed=not args.no_pack)
    gdur = [sum(dur[i] for i in idx) for _, idx in groups]
    dom = max(range(len(groups)), key=lambda q: gdur[q])
    name, idx = groups[dom]
    sbytes = sum(work[i][1] for i in idx)
    sflops = sum(work[i][2] for i in idx)
    path = W.forward_path(m, T, packed=not args.no_pack)
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

    layer_bytes = W.algorithmic_bytes(m, T, U, wl.router_bias)
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
    }

    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU oracle")
        try:
            cpu = cpu_baseline(wl, args.cpu_seconds)
        except Exception as e:  # noqa: BLE001
            log(f"CPU baseline failed: {e}")

    out = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": Wm,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) bf16 activations, N(0,0.02) weights quantized affine 4-bit g64",
        "config": {
            "workload": f"{m['name']} MoE block, {wl.note}",
            "key": wl.key,
            "tokens": T,
            "hidden": m["hidden"],
            "experts": m["n_experts"],
            "top_k": m["top_k"],
            "moe_intermediate": m["inter"],
            "shared_intermediate": m["shared_inter"],
            "seed": wl.seed,
            "layer_copies": R,
            "hip_graph": True,
            "parallelism": "single GPU",
        },
        "roofline": roof,
        "layer": layer,
        "wall_s": round(wall, 3),
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
