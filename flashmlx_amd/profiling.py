"""Summaries of rocprofv3 output for libfmx kernels.

  python -m flashmlx_amd.profiling trace  <kernel_stats.csv> --cmd "<command>"
      -> markdown table of per-kernel calls / average / min / max durations
  python -m flashmlx_amd.profiling traffic --fetch <csv> --write <csv>
         --copy-fetch <csv> --copy-write <csv> --copy-bytes N --workload KEY
      -> JSON of HBM bytes per launch of each MoE stage's kernel
  python -m flashmlx_amd.profiling eager KEY [--forwards N]
      -> N eager (not graph-captured) forwards of a workload's MoE block on
         packed weights, the program that counter passes (rocprofv3 --pmc)
         run under

FETCH_SIZE and WRITE_SIZE (KiB per dispatch) are scaled by what the same
counter reads for a plain device copy of known size (the factor that makes
the copy's reading equal its bytes), measured in the same pass.
"""
from __future__ import annotations

import argparse
import collections
import csv
import json
import re
import sys

# kernel name -> MoE stage (the four kernel stages of fmx_moe_block_forward)
STAGE_OF = [
    (r"dec_k1", "router+shared_gate_up"),
    (r"dec_k23", "gate_up+down+combine"),
    (r"dec_k2", "gate_up"),  # launched alone only by forwards that stop after gate/up
    (r"router_kernel|logits_kernel|topk_kernel|sort_kernel", "router+sort"),
    (r"pf_gemm<true", "gate_up"),
    (r"pf_gemm<false", "down"),
    (r"qgemm_kernel<true", "gate_up"),
    (r"qgemm_kernel<false", "down"),
    (r"combine_kernel", "combine"),
    # the decoder stack's kernels (fmx_model)
    (r"attn_split_kernel", "attention (single token)"),
    (r"attn_kernel", "attention (several tokens)"),
    (r"dense_dec_kernel<true", "q/k/v with input norm"),
    (r"dense_dec_kernel<false", "o_proj, lm_head"),
    (r"greedy_kernel", "argmax"),
    (r"rmsnorm_kernel", "norm"),
    # the Nemotron-H block's kernels
    (r"nh_d1", "router+shared_up (D1)"),
    (r"nh_d2", "fc1 (D2)"),
    (r"nh_d3", "fc2+combine (D3)"),
    (r"nh_combine_kernel", "combine"),
    # bench.py's timing lead: one bounded spin kernel queued before each
    # timed per-stage section
    (r"spin_kernel", "timing lead"),
]


def short_name(kernel: str) -> str:
    k = kernel.replace("(anonymous namespace)::", "")
    return re.sub(r"\(.*", "", k).replace("void ", "")


def stage_of(kernel: str):
    for pat, st in STAGE_OF:
        if re.search(pat, kernel):
            return st
    return None


def kernel_stats_md(path: str, cmd: str, top: int = 12) -> str:
    rows = list(csv.DictReader(open(path)))
    out = [f"Command: `{cmd}`", "",
           "| kernel | stage | calls | avg us | min us | max us |",
           "|---|---|---:|---:|---:|---:|"]
    for r in rows[:top]:
        name = r["Name"]
        short = short_name(name)[:60]
        out.append(f"| `{short}` | {stage_of(name) or '-'} | {r['Calls']} | "
                   f"{float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
                   f"{float(r['MaxNs']) / 1e3:.2f} |")
    return "\n".join(out) + "\n"


def counter_avgs(path: str) -> dict:
    d = collections.defaultdict(list)
    for r in csv.DictReader(open(path)):
        d[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in d.items()}


def copy_factor(path: str, copy_bytes: int) -> float:
    """bytes / (KiB reading x 1024) for the largest copy-kernel dispatch."""
    vals = [float(r["Counter_Value"]) for r in csv.DictReader(open(path))
            if "copy" in r["Kernel_Name"].lower()]
    if not vals:
        raise ValueError(f"no copy kernel in {path}")
    return copy_bytes / (max(vals) * 1024.0)


def traffic(fetch: str, write: str, copy_fetch: str, copy_write: str, copy_bytes: int,
            workload: str, cmds: dict) -> dict:
    ff = copy_factor(copy_fetch, copy_bytes)
    fw = copy_factor(copy_write, copy_bytes)
    fa, wa = counter_avgs(fetch), counter_avgs(write)
    stages = {}
    kernels = {}
    for k in fa:
        st = stage_of(k)
        if st is None:
            continue
        fb = fa[k] * 1024.0 * ff
        wb = wa.get(k, 0.0) * 1024.0 * fw
        kernels[short_name(k)] = {"fetch_bytes": round(fb), "write_bytes": round(wb)}
        stages[st] = stages.get(st, 0) + round(fb + wb)
    return {"workload": workload, "unit": "HBM bytes per launch", "fetch_scale": round(ff, 4),
            "write_scale": round(fw, 4), "stages": stages, "kernels": kernels, "commands": cmds}


def eager(key: str, n: int) -> None:
    import torch

    from . import workloads as W

    wl = W.WORKLOADS[key]
    block, x = W.device_block(wl, W.DeviceSynth(wl), pack=True, drop_mlx=True)
    y = torch.empty_like(x)
    for _ in range(n):
        block.forward_into(x, y)
    torch.cuda.synchronize()
    print(f"{n} eager forwards of {key}", flush=True)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="what", required=True)
    t = sub.add_parser("trace")
    t.add_argument("stats")
    t.add_argument("--cmd", required=True)
    c = sub.add_parser("traffic")
    for a in ("fetch", "write", "copy_fetch", "copy_write"):
        c.add_argument("--" + a.replace("_", "-"), required=True)
    c.add_argument("--copy-bytes", type=int, required=True)
    c.add_argument("--workload", required=True)
    c.add_argument("--cmd", action="append", default=[], help="name=command of a pass")
    e = sub.add_parser("eager")
    e.add_argument("key")
    e.add_argument("--forwards", type=int, default=6)
    a = ap.parse_args(argv)
    if a.what == "eager":
        eager(a.key, a.forwards)
    elif a.what == "trace":
        sys.stdout.write(kernel_stats_md(a.stats, a.cmd))
    else:
        cmds = dict(s.split("=", 1) for s in a.cmd)
        print(json.dumps(traffic(a.fetch, a.write, a.copy_fetch, a.copy_write, a.copy_bytes,
                                 a.workload, cmds), indent=1))


if __name__ == "__main__":
    main()
