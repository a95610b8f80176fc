#!/usr/bin/env python3
"""MoE-layer benchmark of libfmx on one MI355X.

A step is one MoE-layer forward (router, sort, gate/up + SwiGLU, down,
top-k combine, gated shared expert) over one batch of tokens already
resident in HBM. Steps cycle over `--layers` copies of the layer's weights
(distinct HBM addresses, 24 by default like a 24-layer model) so that the
weights stream from HBM rather than the 256 MB last-level cache, and run as
a captured HIP graph. Prints ONE JSON line.

Default workload: Qwen1.5-MoE-A2.7B-shape MoE block, decode batch 8
(seed 2). Other workloads: --workload (see flashmlx_amd/workloads.py).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import subprocess
import sys
import time

METRIC = "MoE-layer tok/s; decode HBM GB/s and prefill MFMA % on 1 MI355X"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


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


def stage_bytes_flops(m, wl, U):
    """Algorithmic HBM bytes and FLOPs of each stage for one call."""
    H, E, I, Is, k = m["hidden"], m["n_experts"], m["inter"], m["shared_inter"], m["top_k"]
    T = wl.tokens
    pw = lambda n, kk: n * kk // 2 + 4 * n * (kk // 64)  # noqa: E731  packed weight bytes
    gu_b = U * 2 * pw(I, H) + (2 * pw(Is, H) if Is else 0) + T * H * 2 + T * k * I * 2 + T * Is * 2
    dn_b = U * pw(H, I) + (pw(H, Is) if Is else 0) + T * k * I * 2 + T * Is * 2 + T * k * H * 2 + T * H * 2
    rt_b = E * H * 2 + T * H * 2 + (H * 2 if Is else 0)
    cb_b = T * k * H * 2 + (T * H * 2 if Is else 0) + T * H * 2
    gu_f = 2 * T * k * 2 * H * I + (2 * T * 2 * H * Is if Is else 0)
    dn_f = 2 * T * k * H * I + (2 * T * H * Is if Is else 0)
    rt_f = 2 * T * H * (E + (1 if Is else 0))
    return {"router": (rt_b, rt_f), "gate_up": (gu_b, gu_f), "down": (dn_b, dn_f),
            "combine": (cb_b, 0)}


def load_traffic(workload: str, kernel_stage: str):
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 --pmc summary (profiles/traffic_<workload>.json), if present."""
    p = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                     f"traffic_{workload}.json")
    try:
        with open(p) as f:
            d = json.load(f)
        return d.get(kernel_stage)
    except (OSError, ValueError):
        return None


def cpu_baseline(wl, seconds: float):
    """The CPU oracle (C restatement of the reference's MLX CPU semantics,
    fp32 accumulation) timed on this host on the same workload."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
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
    ap.add_argument("--eager", action="store_true", help="no HIP graph")
    ap.add_argument("--no-pack", action="store_true",
                    help="MLX-layout weights only (no fmx_pack_expert_weights re-layout)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs the MoE layer on one GPU only; "
                                   "run bench.py with --gpus 1",
                          "n_gpus": args.gpus}), flush=True)
        sys.exit(2)

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import torch

    from flashmlx_amd import workloads as W
    from flashmlx_amd.moe import MoEBlock, MoEWeights, QWeight

    wl = W.WORKLOADS[args.workload]
    m = wl.model
    T = wl.tokens
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

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
    layer_bytes = sum(t.numel() * t.element_size() for q in (block0.weights.gate, block0.weights.up,
                                                            block0.weights.down)
                      for t in (q.w, q.scales, q.biases))
    log(f"{R} layer copies, {R * layer_bytes / 2**30:.2f} GiB of expert weights")

    # reference output (eager) and routing statistics
    blocks[0].forward_into(x, y)
    torch.cuda.synchronize()
    y_ref = y.clone()
    r = blocks[0].routing()
    offs = r["expert_offsets"].cpu().numpy().astype("int64")
    U = int((offs[1:] > offs[:-1]).sum())

    def run_layers(n0, n):
        for i in range(n0, n0 + n):
            blocks[i % R].forward_into(x, y)

    K, Wm = args.steps, args.warmup
    graphs = {}
    use_graph = not args.eager
    if use_graph:
        try:
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                run_layers(0, R)  # warm the stream before capture
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize()

            def capture(n):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    run_layers(0, n)
                return g

            graphs[R] = capture(R)
            if K % R:
                graphs[K % R] = capture(K % R)
            # every replay must equal the eager result
            for _ in range(3):
                graphs[R].replay()
                torch.cuda.synchronize()
                if not torch.equal(y, y_ref):
                    raise RuntimeError("graph replay output differs from eager output")
                blocks[0].forward_into(x, y)
                torch.cuda.synchronize()
        except Exception as e:  # noqa: BLE001
            log(f"graph capture unavailable ({e}); timing eager launches")
            use_graph = False
            graphs = {}

    def run_steps(n):
        if use_graph:
            for _ in range(n // R):
                graphs[R].replay()
            if n % R:
                g = graphs.get(n % R)
                if g is None:
                    run_layers(0, n % R)
                else:
                    g.replay()
        else:
            run_layers(0, n)

    run_steps(Wm)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    run_steps(K)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_total = ev0.elapsed_time(ev1)
    ms_step = ms_total / K
    tok_s = T * K / (ms_total / 1e3)

    # ---- per-stage timing pass (events between the kernels of each layer)
    stages = ["router", "gate_up", "down", "combine"]
    P = max(R, (args.profile_steps // R) * R)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(P)]
    for e5 in evs:
        for ev in e5:
            ev.record()
    torch.cuda.synchronize()
    # queue GPU work ahead so the profiled launches never wait for the host
    run_steps(K)
    th0 = time.perf_counter()
    for i in range(P):
        blocks[i % R].forward_profiled(x, y, evs[i])
    host_ms = (time.perf_counter() - th0) * 1e3
    torch.cuda.synchronize()
    dur = {s: 0.0 for s in stages}
    for e5 in evs:
        for j, s in enumerate(stages):
            dur[s] += e5[j].elapsed_time(e5[j + 1]) / P
    stage_us = {s: round(dur[s] * 1e3, 2) for s in stages}

    bf = stage_bytes_flops(m, wl, U)
    dom = max(("gate_up", "down"), key=lambda s: dur[s])
    prefill = T * m["top_k"] / m["n_experts"] >= 8
    if prefill:
        achieved = bf[dom][1] / (dur[dom] * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4)}
    else:
        achieved = bf[dom][0] / (dur[dom] * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4)}
    roof["kernel"] = f"qgemm_kernel ({dom})"
    roof["algorithmic_per_launch"] = bf[dom][1] if prefill else bf[dom][0]
    roof["avg_launch_us"] = round(dur[dom] * 1e3, 2)
    roof["traffic"] = load_traffic(wl.key, dom)

    layer_bytes_alg = W.algorithmic_bytes(m, T, U, wl.router_bias)
    layer_flops = W.flops(m, T)
    layer = {
        "unique_experts": U,
        "algorithmic_bytes": layer_bytes_alg,
        "hbm_gbps": round(layer_bytes_alg / (ms_step * 1e-3) / 1e9, 1),
        "hbm_frac": round(layer_bytes_alg / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "tflops": round(layer_flops / (ms_step * 1e-3) / 1e12, 2),
        "mfma_frac": round(layer_flops / (ms_step * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
        "stage_us": stage_us,
        # true when the host could not enqueue the profiled layers faster than
        # the queued work drained (stage times may then include idle gaps)
        "stage_timing_host_bound": bool(host_ms > ms_total + sum(dur.values()) * P),
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
            "hip_graph": use_graph,
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
