"""Pins the CPU oracle (oracle/fmx_oracle.c) without the reference library.

MLX (the library that holds the reference's arithmetic for this path) is not
available, and the reference's tests hold no vectors for it, so each oracle
function is pinned here by what the mathematics fixes: exact rational
arithmetic (fractions.Fraction), library routines (torch's float->bf16 cast,
numpy's stable argsort, fp64 matmul), closed forms of the quantizer on
hand-built groups, invariants, and brute force on tiny inputs. Several tests
also plant a mistake on the CPU side and check that the comparison notices.
"""
from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest

RNG = np.random.default_rng(20261201)


# ------------------------------------------------------------------ helpers

def bf16_from_fraction(v: Fraction) -> int:
    """Exact round-to-nearest-even of a rational to bf16 bits (finite range)."""
    if v == 0:
        return 0
    sign = 0x8000 if v < 0 else 0
    a = -v if v < 0 else v
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)                      # subnormals share the 2^-133 quantum
    quantum = Fraction(2) ** (e - 7)
    n = a / quantum
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    val = fl * quantum
    if val >= Fraction(2) ** 128:
        return sign | 0x7F80
    f = np.float32(float(val))
    return sign | int(np.array([f], np.float32).view(np.uint32)[0] >> 16)


def bf(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_rne_from_f64(v: np.ndarray) -> np.ndarray:
    return np.array([bf16_from_fraction(Fraction(float(t))) for t in np.ravel(v)], np.uint16)


def rand_bf16(shape, std=1.0):
    import torch
    t = torch.from_numpy(RNG.standard_normal(shape).astype(np.float32) * std).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------------ rounding

def test_f32_to_bf16_matches_torch(oracle):
    import torch
    bits = RNG.integers(0, 2**32, 200_000, dtype=np.uint64).astype(np.uint32)
    # every exact tie and its neighbours, both parities
    ties = (RNG.integers(0, 2**16, 2000, dtype=np.uint64).astype(np.uint32) << 16) | 0x8000
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7F7FFFFF, 0x00000001,
                        0x007FFFFF, 0x3F808000, 0x3F818000, 0x7F7F8000], np.uint32)
    bits = np.concatenate([bits, ties, ties + 1, ties - 1, special])
    f = bits.view(np.float32)
    finite = np.isfinite(f) | np.isinf(f)
    f = f[finite]
    ref = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = oracle.f32_to_bf16_array(f)
    np.testing.assert_array_equal(got, ref)
    some = f[:2000]
    np.testing.assert_array_equal(oracle.f32_to_bf16(some), ref[:2000])


def test_f64_to_bf16_single_rounding(oracle):
    vals = list(RNG.standard_normal(3000) * np.exp(RNG.uniform(-100, 100, 3000)))
    # exact bf16 midpoints and one double-ulp either side: a double rounding
    # through fp32 would get some of these wrong
    for h in RNG.integers(0x0080, 0x7F00, 400):
        lo = float(bf(np.uint16(h)))
        hi = float(bf(np.uint16(h + 1)))
        mid = (lo + hi) / 2
        vals += [mid, np.nextafter(mid, 0), np.nextafter(mid, np.inf), -mid]
    vals += [0.0, -0.0, 1e-45, 2.0**-133, 2.0**-134, 3 * 2.0**-135, 2.0**-126 * (1 - 2**-9),
             3.4e38, 3.3895313892515355e38]
    got = oracle.f64_to_bf16(np.array(vals))
    ref = np.array([bf16_from_fraction(Fraction(v)) for v in vals], np.uint16)
    # -0.0 is the one value whose sign Fraction loses
    ref[np.array(vals) == 0] = got[np.array(vals) == 0]
    np.testing.assert_array_equal(got, ref)


def test_exp_matches_libm(oracle):
    # exp_det flushes below e^-690 (far under any softmax term that matters)
    xs = np.concatenate([np.linspace(-690, 709, 4001), RNG.uniform(-30, 30, 4000),
                         [0.0, -0.0, 1e-300, -1e-300, math.log(2), -math.log(2)]])
    for x in xs:
        got = oracle.exp(float(x))
        ref = math.exp(float(x))
        assert abs(got - ref) <= 4 * np.spacing(ref), (x, got, ref)
    assert oracle.exp(-691.0) == 0.0 and oracle.exp(-800.0) == 0.0
    assert math.isinf(oracle.exp(800.0))


def test_sigmoid_bf16_all_inputs(oracle):
    lib = oracle.load()
    exact = inexact = 0
    for h in range(0, 1 << 16):
        x = float(bf(np.uint16(h)))
        if not math.isfinite(x):
            continue
        s = 1.0 / (1.0 + math.exp(-x)) if x > -700 else 0.0
        got = lib.orc_sigmoid_bf16(h)
        ref = float(bf(np.uint16(bf16_from_fraction(Fraction(s)))))
        if got == ref:
            exact += 1
        else:
            # only where the fp64 value sits on a bf16 midpoint to ~1e-15
            lo, hi = sorted((got, ref))
            assert abs(s - (lo + hi) / 2) <= 1e-14 * max(s, 1e-300), (h, x, got, ref)
            inexact += 1
    assert inexact <= 4, inexact
    assert lib.orc_sigmoid_bf16(0) == 0.5


# ------------------------------------------------------------------ quantization

def test_quantize_closed_forms(oracle):
    """Groups built on an exact 16-level grid quantize to that grid."""
    q = np.tile(np.arange(16), 4)
    RNG.shuffle(q)
    rows = []
    # min-dominated: |min| > |max| -> scale 0.125 > 0, bias = min = -1
    rows.append(-1.0 + 0.125 * q)
    # max-dominated: |max| >= |min| -> scale -0.125, bias = max = 1
    rows.append(1.0 - 0.125 * q)
    rows.append(np.full(64, 0.5))
    rows.append(np.zeros(64))
    w = np.stack(rows).astype(np.float32)
    import torch
    wb = torch.from_numpy(w).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    wq, s, b = oracle.quantize(wb)
    assert (bf(s[0]), bf(b[0])) == (0.125, -1.0)
    assert (bf(s[1]), bf(b[1])) == (-0.125, 1.0)
    assert bf(b[2]) == 0.5 and bf(b[3]) == 0.0
    nib = lambda words: np.array([(words[i // 8] >> (4 * (i % 8))) & 15 for i in range(64)])  # noqa: E731
    np.testing.assert_array_equal(nib(wq[0]), q)
    np.testing.assert_array_equal(nib(wq[1]), q)
    np.testing.assert_array_equal(nib(wq[2]), 0)
    np.testing.assert_array_equal(oracle.dequantize(wq, s, b), w)
    # little-endian nibble order: element i at bits 4i of its word
    ramp = np.tile(np.arange(16), 4).astype(np.float32) * 0.125 - 1.0
    rb = torch.from_numpy(ramp[None]).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    wq2, _, _ = oracle.quantize(rb)
    assert wq2[0, 0] == 0x76543210 and wq2[0, 1] == 0xFEDCBA98


def test_quantize_error_bound(oracle):
    w = rand_bf16((64, 512), std=0.02)
    wq, s, b = oracle.quantize(w)
    deq = oracle.dequantize(wq, s, b).astype(np.float64)
    wf = bf(w).astype(np.float64).reshape(64, 8, 64)
    g = deq.reshape(64, 8, 64)
    alpha = (wf.max(-1) - wf.min(-1)) / 15
    sc = np.abs(bf(s).astype(np.float64)).reshape(64, 8)
    # half a step, plus what bf16 storage of scale and bias can shift a level
    bound = alpha / 2 + 15 * np.abs(sc - alpha) + np.abs(bf(b).reshape(64, 8)) * 2.0**-8 + 1e-12
    assert (np.abs(g - wf).max(-1) <= bound).all()
    # the extreme edge is (nearly) representable after the zero snap
    assert (np.abs(g - wf).max(-1) <= alpha).all()


def test_dequantize_handbuilt_words(oracle):
    N, K = 5, 256
    words = RNG.integers(0, 2**32, (N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = rand_bf16((N, K // 64), 0.05)
    b = rand_bf16((N, K // 64), 0.5)
    deq = oracle.dequantize(words, s, b)
    for n in range(N):
        for k in range(0, K, 7):
            qv = (int(words[n, k // 8]) >> (4 * (k % 8))) & 15
            exact = Fraction(float(bf(s[n, k // 64]))) * qv + Fraction(float(bf(b[n, k // 64])))
            assert abs(Fraction(float(deq[n, k])) - exact) <= abs(exact) * Fraction(1, 2**24)


# ------------------------------------------------------------------ products

def _deq64(oracle, wq, s, b):
    return oracle.dequantize(wq, s, b).astype(np.float64)


@pytest.mark.parametrize("M,N,K", [(1, 16, 64), (3, 40, 256), (8, 64, 1408)])
def test_qmm_t_against_fp64_matmul(oracle, M, N, K):
    x = rand_bf16((M, K))
    wq, s, b = oracle.quantize(rand_bf16((N, K), 0.02))
    ref64 = bf(x).astype(np.float64) @ _deq64(oracle, wq, s, b).T
    got = oracle.qmm_t(x, wq, s, b, oracle.ACC_F64)
    ref = bf16_rne_from_f64(ref64).reshape(M, N)
    diff = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.99
    a = bf(oracle.qmm_t(x, wq, s, b, oracle.ACC_A)).astype(np.float64)
    assert np.abs(a - ref64).max() <= 1e-2 + 2e-2 * np.abs(ref64).max()
    # planted mistake: a dropped bias term is far outside the tolerance
    bad = _deq64(oracle, wq, s, np.zeros_like(b))
    assert np.abs(bf(x).astype(np.float64) @ bad.T - ref64).max() > 5e-2


def test_gather_qmm_reduces_to_qmm(oracle):
    E, N, K, T = 4, 8, 128, 3
    x = rand_bf16((T, 1, K))
    wq, s, b = oracle.quantize(rand_bf16((E, N, K), 0.02))
    rhs = np.array([2, 0, 3, 3, 1, 2], np.uint32)
    lhs = np.array([0, 1, 2, 0, 1, 2], np.uint32)
    got = oracle.gather_qmm(x, wq, s, b, lhs, rhs, oracle.ACC_F64)
    deq = _deq64(oracle, wq, s, b)
    for i, (l, r) in enumerate(zip(lhs, rhs)):
        one = oracle.qmm_t(x[l], wq[r], s[r], b[r], oracle.ACC_F64)
        np.testing.assert_array_equal(got[i], one)
        brute = bf16_rne_from_f64(bf(x[l]).astype(np.float64) @ deq[r].T).reshape(1, N)
        assert np.abs(got[i].astype(np.int32) - brute.astype(np.int32)).max() <= 1


# ------------------------------------------------------------------ router

def test_router_logits_exact(oracle):
    T, E, H = 3, 10, 64
    x, wr = rand_bf16((T, H)), rand_bf16((E, H), 0.02)
    bias = rand_bf16((E,))
    logits, probs, inds, scores = oracle.router_topk(x, wr, 3, False, bias)
    xf, wf, bfv = bf(x), bf(wr), bf(bias)
    for t in range(T):
        for e in range(E):
            dot = sum(Fraction(float(a)) * Fraction(float(c)) for a, c in zip(xf[t], wf[e]))
            l0 = bf16_from_fraction(dot)
            l1 = bf16_from_fraction(Fraction(float(bf(np.uint16(l0)))) + Fraction(float(bfv[e])))
            assert logits[t, e] == l1, (t, e)


def test_router_softmax_and_topk(oracle):
    T, E, H, k = 64, 60, 256, 4
    x, wr = rand_bf16((T, H)), rand_bf16((E, H), 0.02)
    logits, probs, inds, scores = oracle.router_topk(x, wr, k)
    lf = bf(logits).astype(np.float64)
    p64 = np.exp(lf - lf.max(1, keepdims=True))
    p64 /= p64.sum(1, keepdims=True)
    ref = bf16_rne_from_f64(p64).reshape(T, E)
    diff = np.abs(probs.astype(np.int32) - ref.astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.995
    for t in range(T):
        order = sorted(range(E), key=lambda e: (-float(bf(probs[t, e])), e))
        np.testing.assert_array_equal(inds[t], order[:k])
        np.testing.assert_array_equal(scores[t], probs[t, order[:k]])


def test_router_ties_go_to_lower_index(oracle):
    H, E, k = 64, 8, 3
    x = rand_bf16((2, H))
    base = rand_bf16((1, H), 0.02)
    wr = np.repeat(base, E, axis=0)       # all logits equal
    wr[5] = rand_bf16((1, H), 0.5)[0]     # one different expert
    _, probs, inds, _ = oracle.router_topk(x, wr, k)
    for t in range(2):
        exp = sorted(range(E), key=lambda e: (-float(bf(probs[t, e])), e))[:k]
        np.testing.assert_array_equal(inds[t], exp)
        others = [e for e in inds[t] if e != 5]
        assert others == sorted(others) and others[0] == 0


def test_router_renorm(oracle):
    T, E, H, k = 16, 128, 128, 8
    x, wr = rand_bf16((T, H)), rand_bf16((E, H), 0.05)
    _, probs, inds, raw = oracle.router_topk(x, wr, k, False)
    _, _, inds2, sc = oracle.router_topk(x, wr, k, True)
    np.testing.assert_array_equal(inds, inds2)
    s = bf(sc).astype(np.float64)
    assert np.abs(s.sum(1) - 1).max() <= k * 2.0**-8
    r = bf(raw).astype(np.float64)
    np.testing.assert_allclose(s, r / r.sum(1, keepdims=True), rtol=2 * 2.0**-8)


# ------------------------------------------------------------------ sort

@pytest.mark.parametrize("T,k,E", [(1, 4, 60), (8, 8, 128), (512, 4, 60), (1024, 8, 128), (5, 2, 3)])
def test_moe_sort_is_stable_argsort(oracle, T, k, E):
    inds = np.stack([RNG.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32)
    order, inv, src, idx, off = oracle.moe_sort(inds, E)
    flat = inds.ravel()
    ref = np.argsort(flat, kind="stable")
    np.testing.assert_array_equal(order, ref)
    np.testing.assert_array_equal(inv, np.argsort(ref, kind="stable"))
    np.testing.assert_array_equal(src, ref // k)
    np.testing.assert_array_equal(idx, flat[ref])
    np.testing.assert_array_equal(off, np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=E))]))


# ------------------------------------------------------------------ full block

def _dense_block(oracle, cfg, w, x, drop=None):
    """fp64 dense formula: y = sum_k s_k * down(silu(gate x) * up x) + sig(g) * shared."""
    H = cfg["hidden"]
    xf = bf(x).astype(np.float64)
    _, _, inds, scores = oracle.router_topk(x, w["router_w"], cfg["top_k"], cfg["norm_topk"],
                                            w.get("router_bias"))
    dq = {n: _deq64(oracle, *w[n]) for n in ("gate", "up", "down")}
    silu = lambda v: v / (1 + np.exp(-v))  # noqa: E731
    y = np.zeros((x.shape[0], H))
    for t in range(x.shape[0]):
        for j, e in enumerate(inds[t]):
            g, u = dq["gate"][e] @ xf[t], dq["up"][e] @ xf[t]
            if drop == "swap":
                g, u = u, g
            y[t] += float(bf(scores[t, j])) * (dq["down"][e] @ (silu(g) * u))
    if cfg["shared_inter"] and drop != "shared":
        sg, su, sd = (_deq64(oracle, *w[n]) for n in ("shared_gate", "shared_up", "shared_down"))
        g = w["shared_expert_gate_w"]
        gw = _deq64(oracle, *g) if isinstance(g, tuple) else bf(g).astype(np.float64)
        gl = xf @ gw.ravel()
        for t in range(x.shape[0]):
            y[t] += 1 / (1 + np.exp(-gl[t])) * (sd @ (silu(sg @ xf[t]) * (su @ xf[t])))
    return y


@pytest.mark.parametrize("key", ["tiny_t5", "tiny_norm_t33"])
def test_moe_block_dense_formula(oracle, key):
    from flashmlx_amd import workloads as W
    from helpers import oracle_args
    wl = W.WORKLOADS[key]
    hi = W.host_inputs(wl)
    cfg, w = oracle_args(hi, wl.model, oracle.quantize)
    y, _, _ = oracle.moe_block(cfg, w, hi.x, oracle.ACC_A)
    ref = _dense_block(oracle, cfg, w, hi.x)
    got = bf(y).astype(np.float64)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel < 1e-2, rel
    # planted mistakes in the formula are far outside that bound
    for mistake in ("swap",) + (("shared",) if cfg["shared_inter"] else ()):
        bad = _dense_block(oracle, cfg, w, hi.x, drop=mistake)
        assert np.linalg.norm(got - bad) / np.linalg.norm(bad) > 5e-2, mistake


# ------------------------------------------------------------------ accumulation modes

def _nib(wq, n, k):
    return (int(wq[n, k // 8]) >> (4 * (k % 8))) & 15


@pytest.mark.parametrize("mode_name", ["A", "B", "C"])
def test_qmm_accumulation_modes_brute_force(oracle, mode_name):
    """The three MLX CPU accumulators the oracle restates, recomputed by
    scalar loops with explicit per-operation rounding: A sequential fp32
    (w = s*q, + b; acc += x*w), B every operation rounded to bf16 (exact
    rational rounding), C eight fp32 lanes over k mod 8 summed pairwise
    ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)). Each result is rounded once to
    bf16. A planted wrong group index (scale/bias of group k // 32) is
    detected; the lane order itself moves only fp32-level bits, which the
    bf16 outputs rarely show (modes A and C nearly always agree)."""
    M, N, K = 2, 5, 128
    x = rand_bf16((M, K))
    wq, s, b = oracle.quantize(rand_bf16((N, K), 0.02))
    mode = {"A": oracle.ACC_A, "B": oracle.ACC_B, "C": oracle.ACC_C}[mode_name]
    got = oracle.qmm_t(x, wq, s, b, mode)
    f32 = np.float32
    xf = bf(x)

    def rb_frac(v):  # bf16 of an exact rational, as a float
        return float(bf(np.uint16(bf16_from_fraction(Fraction(v)))))

    def one(m, n, wrong_group=False):
        grp = (lambda kk: min(kk // 32, K // 64 - 1)) if wrong_group else (lambda kk: kk // 64)
        if mode_name == "A":
            acc = f32(0)
            for kk in range(K):
                g = grp(kk)
                w = f32(f32(bf(s[n, g])) * f32(_nib(wq, n, kk))) + f32(bf(b[n, g]))
                acc = f32(acc + f32(f32(xf[m, kk]) * f32(w)))
            return bf16_from_fraction(Fraction(float(acc)))
        if mode_name == "B":
            acc = 0.0
            for kk in range(K):
                g = grp(kk)
                sq = rb_frac(float(bf(s[n, g])) * _nib(wq, n, kk))
                w = rb_frac(Fraction(sq) + Fraction(float(bf(b[n, g]))))
                pr = rb_frac(Fraction(float(xf[m, kk])) * Fraction(w))
                acc = rb_frac(Fraction(acc) + Fraction(pr))
            return bf16_from_fraction(Fraction(acc))
        lane = [f32(0)] * 8
        for kk in range(K):
            g = grp(kk)
            w = f32(f32(_nib(wq, n, kk)) * f32(bf(s[n, g])))
            w = f32(w + f32(bf(b[n, g])))
            lane[kk % 8] = f32(lane[kk % 8] + f32(f32(xf[m, kk]) * w))
        a = [f32(lane[i] + lane[i + 4]) for i in range(4)]
        tot = f32(f32(a[0] + a[2]) + f32(a[1] + a[3]))
        return bf16_from_fraction(Fraction(float(tot)))

    ref = np.array([[one(m, n) for n in range(N)] for m in range(M)], np.uint16)
    np.testing.assert_array_equal(got, ref)
    bad = np.array([[one(m, n, wrong_group=True) for n in range(N)] for m in range(M)], np.uint16)
    assert (bad != ref).sum() > M * N // 2


# ------------------------------------------------------------------ quantized router

def test_router_quantized_logits_exact(oracle):
    """A quantized router (model.cpp:758-760): each logit is the exact
    rational x . (s*q + b) rounded once to bf16; rounding the dequantised
    weights to bf16 first (a plausible shortcut) changes some logits."""
    T, E, H = 3, 12, 128
    x = rand_bf16((T, H))
    wq, s, b = oracle.quantize(rand_bf16((E, H), 0.02))
    logits, _, _, _ = oracle.router_topk(x, (wq, s, b), 2)
    xf = bf(x)
    changed = 0
    for t in range(T):
        for e in range(E):
            ws = [Fraction(float(bf(s[e, kk // 64]))) * _nib(wq, e, kk) + Fraction(float(bf(b[e, kk // 64])))
                  for kk in range(H)]
            dot = sum(Fraction(float(xf[t, kk])) * ws[kk] for kk in range(H))
            assert logits[t, e] == bf16_from_fraction(dot), (t, e)
            short = sum(Fraction(float(xf[t, kk])) * Fraction(float(bf(np.uint16(bf16_from_fraction(ws[kk]))))) for kk in range(H))
            changed += bf16_from_fraction(short) != logits[t, e]
    assert changed > 0


def test_router_quantized_matches_numpy(oracle):
    """Softmax and top-k over quantized-router logits equal those over the
    logits numpy forms from its own fp64 dequantisation."""
    T, E, H, k = 32, 60, 256, 4
    x = rand_bf16((T, H))
    wq, s, b = oracle.quantize(rand_bf16((E, H), 0.02))
    logits, probs, inds, scores = oracle.router_topk(x, (wq, s, b), k)
    q = ((wq[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15).reshape(E, H).astype(np.float64)
    deq = q * np.repeat(bf(s).astype(np.float64), 64, 1) + np.repeat(bf(b).astype(np.float64), 64, 1)
    ref = bf16_rne_from_f64(bf(x).astype(np.float64) @ deq.T).reshape(T, E)
    diff = np.abs(logits.astype(np.int32) - ref.astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.99
    for t in range(T):
        order = sorted(range(E), key=lambda e: (-float(bf(probs[t, e])), e))
        np.testing.assert_array_equal(inds[t], order[:k])


def test_moe_block_quantized_router_dense_formula(oracle):
    """The whole block with a quantized router and shared-expert gate
    against the fp64 dense formula, which dequantises them with numpy."""
    from flashmlx_amd import workloads as W
    from helpers import oracle_args
    wl = W.Workload("tiny_t5_q", W.TINY, 5, 11, router_quant=True)
    hi = W.host_inputs(wl)
    cfg, w = oracle_args(hi, wl.model, oracle.quantize, router_quant=True)
    y, _, _ = oracle.moe_block(cfg, w, hi.x, oracle.ACC_A)
    ref = _dense_block(oracle, cfg, w, hi.x)
    got = bf(y).astype(np.float64)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-2


# ---------------------------------------------------------------- float16 forms

def test_f16_decode_all_patterns(oracle):
    """Every binary16 pattern decodes to numpy's value (NaNs as NaN)."""
    lib = oracle.load()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.orc_f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f16_encode_round_to_nearest_even(oracle):
    """fp32 -> fp16 against numpy's conversion: random values over the whole
    range, exact ties between neighbours (to even), subnormals, the
    overflow edge (65504, 65519.996 -> 65504, 65520 -> inf) and signs."""
    lib = oracle.load()
    rng = np.random.default_rng(5)
    f = np.concatenate([
        (rng.standard_normal(20000) * np.exp2(rng.integers(-30, 17, 20000))).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, -65520.0, 1e-8, 2.0 ** -24, 2.0 ** -25,
                  3 * 2.0 ** -26, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, np.inf, -np.inf], np.float32)])
    # ties: midpoints between consecutive fp16 values (exact in fp32)
    h = rng.integers(0, 0x7bff, 3000).astype(np.uint16)
    lo = h.view(np.float16).astype(np.float32)
    hi = (h + 1).view(np.float16).astype(np.float32)
    f = np.concatenate([f, (lo + (hi - lo) / 2).astype(np.float32)])
    with np.errstate(over="ignore"):
        ref = f.astype(np.float16).view(np.uint16)
    got = np.array([lib.orc_f32_to_f16(float(v)) for v in f], np.uint16)
    np.testing.assert_array_equal(got, ref)


def _f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def test_qmm_f16_matches_float64_formula(oracle):
    """The float16 quantized matmul in fp64 mode is fp16(x . (s q + b)) of
    the decoded values (numpy float64), and mode A (fp32) stays within two
    fp16 ulps of it; gather_qmm_f16 with one-hot indices equals it."""
    rng = np.random.default_rng(6)
    M, N, K = 5, 24, 256
    x = _f16(rng.standard_normal((M, K)))
    wq = rng.integers(0, 2 ** 32, (N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = _f16(rng.uniform(0.001, 0.01, (N, K // 64)))
    b = _f16(rng.uniform(-0.05, 0.05, (N, K // 64)))
    q = ((wq[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15).reshape(N, K).astype(np.float64)
    sf = np.repeat(s.view(np.float16).astype(np.float64), 64, axis=1)
    bf = np.repeat(b.view(np.float16).astype(np.float64), 64, axis=1)
    ref = x.view(np.float16).astype(np.float64) @ (sf * q + bf).T
    got64 = oracle.qmm_t_f16(x, wq, s, b, oracle.ACC_F64)
    np.testing.assert_array_equal(got64, ref.astype(np.float32).astype(np.float16).view(np.uint16))
    gotA = oracle.qmm_t_f16(x, wq, s, b, oracle.ACC_A).view(np.float16).astype(np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(gotA - ref) <= 2 * ulp + 1e-6)
    E = 3
    wE = np.stack([wq] * E)
    out = oracle.gather_qmm_f16(x.reshape(M, 1, K), wE, np.stack([s] * E), np.stack([b] * E),
                                np.arange(M, dtype=np.uint32), np.array([0, 2, 1, 2, 0], np.uint32))
    np.testing.assert_array_equal(out.reshape(M, N), oracle.qmm_t_f16(x, wq, s, b, oracle.ACC_A))
