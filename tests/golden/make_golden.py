"""Writes the golden fixtures under tests/golden/ from the CPU oracle.

For every MoE-layer workload (flashmlx_amd/workloads.py):
  inputs_sha256.json       SHA-256 of each synthetic input tensor (bf16 bytes)
  <workload>.npz           routing: inds [T,k], scores [T,k] (bf16 bits);
                           permutation: order, inv, src, idx [T*k], offsets [E+1];
                           tokens (the sampled rows) and y_rows [len(tokens), H]
                           (oracle accumulation mode A); row checksums of every
                           output row: row_sum, row_abs (sum of |y|), row_sq
                           (sum of y^2), float64 [T]; tiny workloads also keep
                           x and every output row.
Run: python tests/golden/make_golden.py [workload ...]
The fixtures are data (inputs and expected outputs); no reference code is
stored. Regenerate only when the oracle's definition of a result changes.
"""
from __future__ import annotations

import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from flashmlx_amd import workloads as W  # noqa: E402
from oracle import oracle as O  # noqa: E402

TENSORS = ("x", "router_w", "router_bias", "gate", "up", "down", "shared_gate", "shared_up",
           "shared_down", "shared_expert_gate_w")


def sample_tokens(T: int, n: int = 8) -> np.ndarray:
    if T <= 64:
        return np.arange(T)
    rng = np.random.default_rng(1234 + T)
    return np.unique(np.concatenate([[0, T - 1], rng.choice(np.arange(1, T - 1), n - 2, replace=False)]))


def tensor_sha(hi) -> dict:
    import hashlib
    out = {}
    for name in TENSORS:
        a = getattr(hi, name)
        if a is not None:
            out[name] = hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    return out


def make(key: str) -> dict:
    wl = W.WORKLOADS[key]
    hi = W.host_inputs(wl)
    m = wl.model
    cfg = dict(hidden=m["hidden"], n_experts=m["n_experts"], top_k=m["top_k"], inter=m["inter"],
               shared_inter=m["shared_inter"], norm_topk=m["norm_topk"])
    q = O.quantize
    rq = q if wl.router_quant else (lambda a: a)
    w = dict(router_w=rq(hi.router_w), router_bias=hi.router_bias, gate=q(hi.gate), up=q(hi.up),
             down=q(hi.down))
    if m["shared_inter"]:
        w.update(shared_gate=q(hi.shared_gate), shared_up=q(hi.shared_up),
                 shared_down=q(hi.shared_down), shared_expert_gate_w=rq(hi.shared_expert_gate_w))
    T = hi.x.shape[0]
    tokens = sample_tokens(T)
    y, inds, scores = O.moe_block(cfg, w, hi.x, O.ACC_A)
    order, inv, src, idx, offsets = O.moe_sort(inds, m["n_experts"])
    yf = O.bf16_to_f32(y).astype(np.float64)
    arrs = dict(inds=inds, scores=scores, order=order, inv=inv, src=src, idx=idx, offsets=offsets,
                tokens=tokens.astype(np.int64), y_rows=y[tokens], row_sum=yf.sum(1),
                row_abs=np.abs(yf).sum(1), row_sq=(yf * yf).sum(1))
    if m["name"].startswith("tiny"):
        arrs["x"] = hi.x
    np.savez_compressed(HERE / f"{key}.npz", **arrs)
    return tensor_sha(hi)


def main(keys) -> None:
    path = HERE / "inputs_sha256.json"
    shas = json.loads(path.read_text()) if path.exists() else {}
    for key in keys:
        shas[key] = make(key)
        print(f"{key}: ok", flush=True)
    path.write_text(json.dumps(dict(sorted(shas.items())), indent=1) + "\n")


if __name__ == "__main__":
    main(sys.argv[1:] or list(W.WORKLOADS))
