"""Committed golden fixtures (tests/golden/, written by make_golden.py).

CPU: the oracle and the seeded generator still reproduce every fixture
(input hashes, routing, permutation, sampled output rows).
GPU: libfmx's MoE block reproduces them: routing and permutation bit-exact,
output rows within the bf16 tolerance.
"""
from __future__ import annotations

import hashlib
import json
import pathlib

import numpy as np
import pytest

from helpers import assert_close, from_dev_bf16, from_dev_u32

GOLD = pathlib.Path(__file__).resolve().parent / "golden"
SHAS = json.loads((GOLD / "inputs_sha256.json").read_text())
KEYS = sorted(SHAS)
SMALL = ("x", "router_w", "router_bias", "shared_expert_gate_w")


def fixture(key):
    with np.load(GOLD / f"{key}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _small_inputs(wl):
    """x, router weights and biases without the (large) expert weights."""
    from flashmlx_amd import workloads as W
    m, s, T = wl.model, wl.seed, wl.tokens
    H, E = m["hidden"], m["n_experts"]
    out = dict(x=W._synth(T * H, s, W.S_X, 1.0).reshape(T, H),
               router_w=W._synth(E * H, s, W.S_ROUTER, W.W_STD).reshape(E, H))
    if wl.router_bias:
        out["router_bias"] = W._synth(E, s, W.S_RBIAS, 1.0)
    if m["shared_inter"]:
        out["shared_expert_gate_w"] = W._synth(H, s, W.S_SH_EGATE, W.W_STD).reshape(1, H)
    return out


def test_fixture_set_covers_every_workload():
    from flashmlx_amd import workloads as W
    assert KEYS == sorted(W.WORKLOADS)


@pytest.mark.parametrize("key", KEYS)
def test_oracle_reproduces_routing(oracle, fmx, key):
    from flashmlx_amd import workloads as W
    wl = W.WORKLOADS[key]
    g = fixture(key)
    small = _small_inputs(wl)
    for name, a in small.items():
        assert _sha(a) == SHAS[key][name], name
    m = wl.model
    _, _, inds, scores = oracle.router_topk(small["x"], small["router_w"], m["top_k"],
                                            m["norm_topk"], small.get("router_bias"))
    np.testing.assert_array_equal(inds, g["inds"])
    np.testing.assert_array_equal(scores, g["scores"])
    for name, a in zip(("order", "inv", "src", "idx", "offsets"), oracle.moe_sort(inds, m["n_experts"])):
        np.testing.assert_array_equal(a, g[name], err_msg=name)


@pytest.mark.parametrize("key", ["tiny_t5", "tiny_t40", "tiny_norm_t33", "qwen3_decode_b1"])
def test_oracle_reproduces_outputs(oracle, fmx, key):
    from flashmlx_amd import workloads as W
    from helpers import oracle_args
    wl = W.WORKLOADS[key]
    g = fixture(key)
    hi = W.host_inputs(wl)
    for name in SHAS[key]:
        assert _sha(getattr(hi, name)) == SHAS[key][name], name
    if "x" in g:
        np.testing.assert_array_equal(hi.x, g["x"])
    cfg, w = oracle_args(hi, wl.model, oracle.quantize)
    y, _, _ = oracle.moe_block(cfg, w, hi.x, oracle.ACC_A, tokens=g["tokens"])
    np.testing.assert_array_equal(y[g["tokens"]], g["y_rows"])


@pytest.mark.gpu
@pytest.mark.parametrize("key", KEYS)
def test_gpu_matches_fixture(gpu, fmx, key):
    from flashmlx_amd import workloads as W
    wl = W.WORKLOADS[key]
    g = fixture(key)
    hi = W.host_inputs(wl)
    block, xd = W.device_block(wl, hi)
    y = from_dev_bf16(block(xd))
    r = block.routing()
    np.testing.assert_array_equal(from_dev_u32(r["inds"]), g["inds"])
    np.testing.assert_array_equal(from_dev_bf16(r["scores"]), g["scores"])
    for name, dev in (("order", "order"), ("inv", "inv"), ("src", "src"), ("idx", "idx"),
                      ("offsets", "expert_offsets")):
        np.testing.assert_array_equal(from_dev_u32(r[dev]), g[name], err_msg=name)
    e = assert_close(y[g["tokens"]], g["y_rows"], f"{key} y")
    print(f"{key}: {len(g['tokens'])} rows vs fixture: {e}")
