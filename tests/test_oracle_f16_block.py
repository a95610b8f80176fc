"""Pins the oracle's float16 forms of the MoE block (a float16 checkpoint
runs the whole block in float16, model.cpp:208-214): the fp64 -> fp16 single
rounding and the fp16 sigmoid against numpy's correctly rounded conversions,
the router (exact logits rounded once, softmax probabilities, top-k on fp16
values, renormalisation) against numpy, and the block against a dense fp64
formula, where it is several times closer than the bf16 form of the same
block (a block that rounded in bf16 somewhere would not be), with planted
mistakes caught."""
from __future__ import annotations

import math

import numpy as np
import pytest


RNG = np.random.default_rng(20261202)


def _f16(a):
    return np.asarray(a, np.float64).astype(np.float16).view(np.uint16)


def _v(h):
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float64)


def test_f64_to_f16_single_rounding(oracle):
    """fp64 -> fp16 against numpy's double -> half conversion (one rounding):
    random values over the whole range and the subnormals, exact midpoints
    between neighbours (ties to even), values a hair off a midpoint (one
    rounding keeps the side a double rounding through fp32 would lose), the
    overflow edge, signed zeros."""
    lib = oracle.load()
    d = np.concatenate([
        RNG.standard_normal(20000) * np.exp2(RNG.integers(-30, 17, 20000)),
        np.array([0.0, -0.0, 65504.0, 65519.999, 65520.0, -65520.0, 2.0 ** -24, 2.0 ** -25,
                  3 * 2.0 ** -26, 2.0 ** -26])])
    h = RNG.integers(0, 0x7bff, 3000).astype(np.uint16)
    lo, hi = _v(h), _v(h + 1)
    mid = lo + (hi - lo) / 2
    d = np.concatenate([d, mid, mid + (hi - lo) * 2.0 ** -30, mid - (hi - lo) * 2.0 ** -30])
    with np.errstate(over="ignore"):
        ref = d.astype(np.float16).view(np.uint16)
    got = np.array([lib.orc_f64_to_f16(float(v)) for v in d], np.uint16)
    np.testing.assert_array_equal(got, ref)
    # the single rounding differs from a rounding through fp32 just above midpoints
    above = mid + (hi - lo) * 2.0 ** -30
    through32 = above.astype(np.float32).astype(np.float16).view(np.uint16)
    assert (through32 != ref[-2 * mid.size:-mid.size]).any()


def test_sigmoid_f16_all_inputs(oracle):
    """fp16(1 / (1 + e^-v)) for every finite fp16 v, against numpy fp64 and
    its correctly rounded conversion (differences only where the fp64 value
    sits on an fp16 midpoint to ~1e-15)."""
    lib = oracle.load()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    v = _v(bits)
    fin = np.isfinite(v)
    with np.errstate(over="ignore"):
        s = 1.0 / (1.0 + np.exp(-v[fin]))
    ref = s.astype(np.float16).astype(np.float64)
    got = np.array([lib.orc_sigmoid_f16(int(b)) for b in bits[fin]], np.float64)
    bad = np.flatnonzero(got != ref)
    for i in bad:
        lo, hi = sorted((got[i], ref[i]))
        assert abs(s[i] - (lo + hi) / 2) <= 1e-14 * max(s[i], 1e-300), (v[fin][i], got[i], ref[i])
    assert bad.size <= 4, bad.size


@pytest.mark.parametrize("norm", [False, True])
def test_router_f16_against_numpy(oracle, norm):
    """Logits are fp16 of the exact sum (math.fsum of the exact products);
    probabilities are within one fp16 ulp of numpy's fp64 softmax (equal for
    almost all); the selection is the full sort of the fp16 probabilities by
    (value desc, index asc); scores and their renormalisation follow the
    fp16 roundings. A planted mistake (bf16 probabilities) selects or scores
    differently."""
    T, E, H, k = 9, 60, 256, 4
    x = _f16(RNG.standard_normal((T, H)))
    wr = _f16(RNG.standard_normal((E, H)) * 0.05)
    lg, pr, inds, sc = oracle.router_topk(x, wr, k, norm, f16=True)
    xv, wv = _v(x), _v(wr)
    ref_lg = np.array([[math.fsum(xv[t] * wv[e]) for e in range(E)] for t in range(T)])
    np.testing.assert_array_equal(lg, _f16(ref_lg))
    lgv = _v(lg)
    ex = np.exp(lgv - lgv.max(1, keepdims=True))
    p = ex / ex.sum(1, keepdims=True)
    pv = _v(pr)
    ulp = np.spacing(p.astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(pv - p) <= ulp)
    assert (pr == _f16(p)).mean() > 0.99
    for t in range(T):
        order = sorted(range(E), key=lambda e: (-pv[t, e], e))
        np.testing.assert_array_equal(inds[t], order[:k])
        s = pv[t, order[:k]]
        if norm:
            den = _v(_f16(np.float32(s.astype(np.float32).sum())))
            want = _f16((s / den).astype(np.float32))
        else:
            want = _f16(s)
        np.testing.assert_array_equal(sc[t], want)
    # planted mistake: bf16 probabilities
    _, pr16, inds16, sc16 = oracle.router_topk(x, wr, k, norm)
    assert not np.array_equal(pr16, pr)


def _f16_inputs(oracle, wl):
    from flashmlx_amd import workloads as W
    from helpers import f16_inputs
    return f16_inputs(oracle, W.host_inputs(wl), wl.model)


def _nibbles(wq):
    """q of every element: nibble k % 8 of word k / 8."""
    wq = np.asarray(wq, np.uint32)
    q = (wq[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 15
    return q.reshape(*wq.shape[:-1], wq.shape[-1] * 8).astype(np.float64)


def _dense_f16(oracle, cfg, w, x, drop=None):
    """fp64 dense formula on the float16 values (routing from the f16 router)."""
    _, _, inds, scores = oracle.router_topk(x, w["router_w"], cfg["top_k"], cfg["norm_topk"],
                                            w.get("router_bias"), f16=True)
    deq = lambda t: np.repeat(_v(t[1]), 64, -1) * _nibbles(t[0]) + np.repeat(_v(t[2]), 64, -1)  # noqa: E731
    xf = _v(x)
    silu = lambda v: v / (1 + np.exp(-v))  # noqa: E731
    dg, du, dd = deq(w["gate"]), deq(w["up"]), deq(w["down"])
    y = np.zeros_like(xf)
    for t in range(x.shape[0]):
        for j, e in enumerate(inds[t]):
            g, u = dg[e] @ xf[t], du[e] @ xf[t]
            if drop == "swap":
                g, u = u, g
            y[t] += _v(scores[t, j]) * (dd[e] @ (silu(g) * u))
    if cfg["shared_inter"] and drop != "shared":
        sg, su, sd = deq(w["shared_gate"]), deq(w["shared_up"]), deq(w["shared_down"])
        gl = xf @ _v(w["shared_expert_gate_w"]).ravel()
        for t in range(x.shape[0]):
            y[t] += 1 / (1 + np.exp(-gl[t])) * (sd @ (silu(sg @ xf[t]) * (su @ xf[t])))
    return y


@pytest.mark.parametrize("key", ["tiny_t5", "tiny_norm_t33"])
def test_moe_block_f16_dense_formula(oracle, key):
    """The float16 block against the fp64 formula on its float16 inputs:
    within 5e-3 relative L2 (fp16 roundings), and at most a third of the
    bf16 block's error on the same values (fp16 keeps three more bits);
    planted mistakes (gate and up swapped, the shared expert dropped) are far
    off. The oracle's fp64 accumulation mode agrees with its fp32 mode."""
    from flashmlx_amd import workloads as W
    wl = W.WORKLOADS[key]
    cfg, w, x = _f16_inputs(oracle, wl)
    y, inds, _ = oracle.moe_block(dict(cfg, act_f16=True), w, x, oracle.ACC_A)
    ref = _dense_f16(oracle, cfg, w, x)
    got = _v(y)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel < 5e-3, rel
    for mistake in ("swap",) + (("shared",) if cfg["shared_inter"] else ()):
        bad = _dense_f16(oracle, cfg, w, x, drop=mistake)
        assert np.linalg.norm(got - bad) / np.linalg.norm(bad) > 5e-2, mistake
    # the same values in bf16 (exact: fp16 values of bf16 inputs), the bf16 block
    tob = lambda u: oracle.f32_to_bf16_array(_v(u).astype(np.float32))  # noqa: E731
    wb = {n: (tuple([v[0], tob(v[1]), tob(v[2])]) if isinstance(v, tuple) else (None if v is None else tob(v)))
          for n, v in w.items()}
    yb, indsb, _ = oracle.moe_block(cfg, wb, tob(x), oracle.ACC_A)
    relb = np.linalg.norm(oracle.bf16_to_f32(yb).astype(np.float64) - ref) / np.linalg.norm(ref)
    assert rel < relb / 3, (rel, relb)
    y64, _, _ = oracle.moe_block(dict(cfg, act_f16=True), w, x, oracle.ACC_F64)
    assert np.linalg.norm(_v(y64) - got) / np.linalg.norm(got) < 2e-3
