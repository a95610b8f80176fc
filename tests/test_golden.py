"""Committed golden fixtures (tests/golden/, written by make_golden.py).

CPU: the oracle and the seeded generator still reproduce every fixture
(input hashes, routing, permutation, sampled output rows).
GPU: libfmx's MoE block reproduces them: routing and permutation bit-exact,
the sampled output rows within the bf16 tolerance and every row's checksums
within the bounds that tolerance implies.
"""
from __future__ import annotations

import hashlib
import json
import pathlib

import numpy as np
import pytest

from helpers import ATOL, RTOL, assert_close, bf16_to_f32, from_dev_bf16, from_dev_u32

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
    wr = oracle.quantize(small["router_w"]) if wl.router_quant else small["router_w"]
    _, _, inds, scores = oracle.router_topk(small["x"], wr, m["top_k"], m["norm_topk"],
                                            small.get("router_bias"))
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
    cfg, w = oracle_args(hi, wl.model, oracle.quantize, router_quant=wl.router_quant)
    y, _, _ = oracle.moe_block(cfg, w, hi.x, oracle.ACC_A, tokens=g["tokens"])
    np.testing.assert_array_equal(y[g["tokens"]], g["y_rows"])
    yf = bf16_to_f32(y[g["tokens"]]).astype(np.float64)
    np.testing.assert_array_equal(yf.sum(1), g["row_sum"][g["tokens"]])
    np.testing.assert_array_equal((yf * yf).sum(1), g["row_sq"][g["tokens"]])


def check_row_sums(got_u16, g, atol=ATOL, rtol=RTOL):
    """Every output row against the fixture's row checksums, within what the
    element-wise tolerance |y - r| <= atol + rtol |r| implies: the row sum
    within H atol + rtol sum|r|, the row's L2 norm within
    sqrt(H atol^2 + 2 atol rtol sum|r| + rtol^2 sum r^2)."""
    y = bf16_to_f32(got_u16).astype(np.float64)
    H = y.shape[1]
    ds = np.abs(y.sum(1) - g["row_sum"])
    assert (ds <= H * atol + rtol * g["row_abs"]).all(), ds.max()
    dn = np.abs(np.sqrt((y * y).sum(1)) - np.sqrt(g["row_sq"]))
    bound = np.sqrt(H * atol**2 + 2 * atol * rtol * g["row_abs"] + rtol**2 * g["row_sq"])
    assert (dn <= bound).all(), dn.max()
    return float(ds.max()), float(dn.max())


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
    ds, dn = check_row_sums(y, g)
    print(f"{key}: {len(g['tokens'])} rows vs fixture: {e}; all {y.shape[0]} row checksums within "
          f"tolerance (max |d sum| {ds:.3g}, max |d norm| {dn:.3g})")
