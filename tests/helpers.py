"""Test helpers: host<->device bf16 moves, error metrics, oracle argument packs."""
from __future__ import annotations

import numpy as np

# Parity bar for bf16 outputs, plus a tight relative
# bound that makes small-magnitude outputs meaningful.
RTOL = 2e-2
ATOL = 1e-2
REL_L2_MAX = 1e-2


def bf16_to_f32(h):
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_dev(a_u16, device="cuda"):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a_u16).view(np.int16)).to(device).view(torch.bfloat16)


def to_dev_u32(a, device="cuda"):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(device)


def from_dev_bf16(t):
    return t.contiguous().view(dtype=__import__("torch").int16).cpu().numpy().view(np.uint16)


def from_dev_u32(t):
    return t.contiguous().cpu().numpy().view(np.uint32)


def errors(got_u16, ref_u16):
    g = bf16_to_f32(got_u16).astype(np.float64)
    r = bf16_to_f32(ref_u16).astype(np.float64)
    d = np.abs(g - r)
    max_abs = float(d.max()) if d.size else 0.0
    mean_rel = float((d / np.maximum(np.abs(r), 1e-6)).mean()) if d.size else 0.0
    rel_l2 = float(np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30))
    return dict(max_abs=max_abs, mean_rel=mean_rel, rel_l2=rel_l2)


def assert_close(got_u16, ref_u16, what="", rtol=RTOL, atol=ATOL, rel_l2=REL_L2_MAX):
    g = bf16_to_f32(got_u16).astype(np.float64)
    r = bf16_to_f32(ref_u16).astype(np.float64)
    assert g.shape == r.shape, (what, g.shape, r.shape)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    bad = np.abs(g - r) > atol + rtol * np.abs(r)
    e = errors(got_u16, ref_u16)
    assert not bad.any(), f"{what}: {int(bad.sum())} elements outside rtol/atol; {e}"
    assert e["rel_l2"] <= rel_l2, f"{what}: relative L2 error {e['rel_l2']:.3g} > {rel_l2}; {e}"
    return e


def oracle_args(hi, model, quant, router_quant=False):
    """(cfg, weights) for oracle.moe_block from HostInputs and a quantizer;
    router_quant: the router and shared-expert gate quantized too."""
    cfg = dict(hidden=model["hidden"], n_experts=model["n_experts"], top_k=model["top_k"],
               inter=model["inter"], shared_inter=model["shared_inter"], norm_topk=model["norm_topk"])
    rq = quant if router_quant else (lambda a: a)
    w = dict(router_w=rq(hi.router_w), router_bias=hi.router_bias,
             gate=quant(hi.gate), up=quant(hi.up), down=quant(hi.down))
    if model["shared_inter"]:
        w.update(shared_gate=quant(hi.shared_gate), shared_up=quant(hi.shared_up),
                 shared_down=quant(hi.shared_down), shared_expert_gate_w=rq(hi.shared_expert_gate_w))
    return cfg, w


def assert_close_rows(got_u16, ref_u16, what="", rtol=RTOL, atol=ATOL, rel_l2=REL_L2_MAX):
    """assert_close for rows of the decoder stack's residual stream and
    logits: a value there is a chain of bf16-rounded sums (x + attn, + moe)
    whose addends can exceed the result, so an element's rounding error is
    bounded by the ulps of the row's large values, not of the element. The
    absolute tolerance of each row is max(atol, 2^-6 * max |row|) (two bf16
    ulps of the row's largest element); rtol and the relative L2 bound as in
    assert_close."""
    g = bf16_to_f32(got_u16).astype(np.float64)
    r = bf16_to_f32(ref_u16).astype(np.float64)
    assert g.shape == r.shape, (what, g.shape, r.shape)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    r2 = r.reshape(-1, r.shape[-1])
    row_atol = np.maximum(atol, 2.0 ** -6 * np.abs(r2).max(axis=1, keepdims=True))
    bad = np.abs(g.reshape(r2.shape) - r2) > row_atol + rtol * np.abs(r2)
    e = errors(got_u16, ref_u16)
    assert not bad.any(), f"{what}: {int(bad.sum())} elements outside the row tolerance; {e}"
    assert e["rel_l2"] <= rel_l2, f"{what}: relative L2 error {e['rel_l2']:.3g} > {rel_l2}; {e}"
    return e


# ---- float16 blocks (a float16 checkpoint, model.cpp:208-214)

def f16_bits(a):
    """fp16 bit patterns of values (one rounding from fp64)."""
    return np.asarray(a, np.float64).astype(np.float16).view(np.uint16)


def f16_vals(h):
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float64)


def f16_inputs(oracle, hi, model, router_quant=False):
    """(cfg, weights, x) for oracle.moe_block in float16 from HostInputs:
    x and the router rows converted, the experts (and a quantized router)
    quantized by the oracle with their bf16 scales and biases re-encoded as
    float16 (the same values)."""
    tof = lambda u: f16_bits(bf16_to_f32(u))  # noqa: E731
    q = lambda a: (lambda r: (r[0], tof(r[1]), tof(r[2])))(oracle.quantize(a))  # noqa: E731
    rq = q if router_quant else tof
    cfg = dict(hidden=model["hidden"], n_experts=model["n_experts"], top_k=model["top_k"],
               inter=model["inter"], shared_inter=model["shared_inter"], norm_topk=model["norm_topk"])
    w = dict(router_w=rq(hi.router_w), router_bias=None if hi.router_bias is None else tof(hi.router_bias),
             gate=q(hi.gate), up=q(hi.up), down=q(hi.down))
    if model["shared_inter"]:
        w.update(shared_gate=q(hi.shared_gate), shared_up=q(hi.shared_up), shared_down=q(hi.shared_down),
                 shared_expert_gate_w=rq(hi.shared_expert_gate_w))
    return cfg, w, tof(hi.x)
