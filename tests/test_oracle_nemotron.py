"""Pins the oracle's Nemotron-H MoE block (orc_nh_route, orc_nh_moe_block;
reference server/src/nemotron_h.cpp:1010-1111) by what the mathematics
fixes: the sigmoid against numpy, the selection against the top-k of the
logits (sigmoid is monotone), group-limited and biased selections on
constructed inputs whose answer is worked out by hand, the block against a
dense numpy fp64 formula on tiny shapes (with planted mistakes that the
comparison must notice), exact scaling, and relu's zeroing of negative
fc1 outputs."""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

from test_oracle import bf, bf16_from_fraction, rand_bf16

RNG = np.random.default_rng(20261202)


def _bf16_round64(v):
    return np.array([bf16_from_fraction(Fraction(float(t))) for t in np.ravel(v)],
                    np.uint16).reshape(np.shape(v))


def _ulp32(a):
    a = np.abs(np.asarray(a, np.float32))
    return np.spacing(a)


# ------------------------------------------------------------------ sigmoid

def test_sigmoid_f32_against_numpy(oracle):
    """fp32(sigmoid) of every bf16 logit in [-30, 30] within one fp32 ulp of
    numpy's fp64 sigmoid rounded to fp32; sigmoid(0) = 0.5 exactly and
    sigmoid(-l) = 1 - sigmoid(l) to an ulp."""
    u = np.arange(0, 0x10000, dtype=np.uint32).astype(np.uint16)
    v = bf(u)
    sel = np.isfinite(v) & (np.abs(v) <= 30)
    u, v = u[sel], v[sel]
    got = np.array([oracle.sigmoid_f32(int(h)) for h in u], np.float32)
    ref = (1.0 / (1.0 + np.exp(-v.astype(np.float64)))).astype(np.float32)
    assert np.all(np.abs(got - ref) <= _ulp32(ref)), np.max(np.abs(got - ref) / _ulp32(ref))
    assert oracle.sigmoid_f32(0) == 0.5
    one = np.float32(1.0)
    for h in (0x3f80, 0x4000, 0x3e00, 0x4120):
        s, sn = oracle.sigmoid_f32(h), oracle.sigmoid_f32(h | 0x8000)
        assert abs((one - np.float32(s)) - np.float32(sn)) <= _ulp32(s)


# ------------------------------------------------------------------ router

def _cfg(**kw):
    c = dict(hidden=256, n_experts=64, top_k=6, norm_topk=True, inter=128, shared_inter=0,
             n_group=1, topk_group=1, scaling=2.5)
    c.update(kw)
    return c


@pytest.mark.parametrize("norm", [False, True])
def test_route_topk_of_logits(oracle, norm):
    """Without groups or bias the selection is the top-k of the logits
    (sigmoid is strictly increasing on these bf16 values): numpy's fp64
    logits rounded exactly to bf16, then a (logit desc, index asc) sort.
    Scores are the sigmoids of the selected logits, renormalised to sum to
    the scaling factor when asked."""
    cfg = _cfg(norm_topk=norm)
    T, H, E, k = 8, cfg["hidden"], cfg["n_experts"], cfg["top_k"]
    x = rand_bf16((T, H))
    gw = rand_bf16((E, H), 0.05)
    logits, inds, scores = oracle.nh_route(cfg, x, gw)
    ref_lg = _bf16_round64(bf(x).astype(np.float64) @ bf(gw).astype(np.float64).T)
    assert np.array_equal(logits, ref_lg)
    lv = bf(ref_lg)
    for t in range(T):
        order = np.lexsort((np.arange(E), -lv[t]))[:k]
        assert np.array_equal(inds[t], order), (t, inds[t], order)
        sig = (1 / (1 + np.exp(-lv[t, order].astype(np.float64))))
        if norm:
            sig = sig / sig.sum()
            np.testing.assert_allclose(scores[t].sum(), cfg["scaling"], rtol=3e-7)
        np.testing.assert_allclose(scores[t], sig * cfg["scaling"], rtol=5e-7)


def test_route_correction_bias_selects_but_does_not_score(oracle):
    """A large correction bias on experts 5 and 7 puts them in slots 0 and 1
    for every token, while their scores stay the unbiased sigmoids of their
    logits (nemotron_h.cpp:1044); a planted mistake (scores from the biased
    values) would exceed 1."""
    cfg = _cfg(norm_topk=False, scaling=1.0, top_k=3)
    T, H, E = 6, cfg["hidden"], cfg["n_experts"]
    x = rand_bf16((T, H))
    gw = rand_bf16((E, H), 0.05)
    cb = np.zeros(E, np.float32)
    cb[5], cb[7] = 10.0, 5.0
    logits, inds, scores = oracle.nh_route(cfg, x, gw, cb)
    assert np.all(inds[:, 0] == 5) and np.all(inds[:, 1] == 7)
    for t in range(T):
        assert scores[t, 0] == np.float32(oracle.sigmoid_f32(int(logits[t, 5])))
        assert scores[t, 1] == np.float32(oracle.sigmoid_f32(int(logits[t, 7])))
        assert np.all(scores[t] < 1.0)


def _const_route(oracle, cb, **kw):
    """Route with x = 0: every logit is 0 and every sigmoid 0.5, so the
    selection scores are 0.5 + cb exactly."""
    E = cb.size
    cfg = _cfg(n_experts=E, hidden=128, **kw)
    x = np.zeros((1, 128), np.uint16)
    gw = rand_bf16((E, 128), 0.05)
    return oracle.nh_route(cfg, x, gw, cb.astype(np.float32))


def test_route_group_limit_constructed(oracle):
    """16 experts in 4 groups, 2 groups kept, top-3, selection scores (0.5 +
    bias, all dyadic): group sums of the two best are 1.625, 1.25, 1.4375, 1.0,
    so groups 0 and 2 stay and expert 4 (the best single expert, in group 1)
    is dropped: inds (1, 10, 0). Without the group limit: (4, 1, 10). Every
    selected score is 0.5 renormalised: 1/3 each, times the scaling."""
    cb = np.array([0.25, 0.375, 0, 0, 0.5, -0.25, -0.25, -0.25, 0.125, 0.125, 0.3125, 0,
                   0, 0, 0, 0], np.float32)
    _, inds, scores = _const_route(oracle, cb, top_k=3, n_group=4, topk_group=2, scaling=1.5)
    assert inds[0].tolist() == [1, 10, 0]
    third = np.float32(0.5) / (np.float32(1.5) + np.float32(1e-20))
    assert np.all(scores[0] == third * np.float32(1.5))
    _, inds1, _ = _const_route(oracle, cb, top_k=3, n_group=1)
    assert inds1[0].tolist() == [4, 1, 10]
    # every group kept: the same as no group limit
    _, inds4, _ = _const_route(oracle, cb, top_k=3, n_group=4, topk_group=4)
    assert inds4[0].tolist() == [4, 1, 10]


def test_route_group_limit_masked_zero_outranks_negative(oracle):
    """Masked experts get selection score 0, not -inf (nemotron_h.cpp:1037):
    with the kept group's scores all negative (-0.5) and the other group's
    lower still (-0.75), top-2 takes experts 8 and 9 of the masked group."""
    cb = np.concatenate([np.full(8, -1.0), np.full(8, -1.25)]).astype(np.float32)
    _, inds, _ = _const_route(oracle, cb, top_k=2, n_group=2, topk_group=1)
    assert inds[0].tolist() == [8, 9]


def test_route_group_ties_zero_lower_group(oracle):
    """Equal group scores: argpartition's (value asc, index asc) order puts
    the lower group first among the zeroed ones, so the higher group stays
    (the comparator that also sends top-k ties to the lower expert)."""
    cb = np.array([0.25, 0.25, 0, 0, 0.25, 0.25, 0, 0], np.float32)
    _, inds, _ = _const_route(oracle, cb, top_k=2, n_group=2, topk_group=1)
    assert inds[0].tolist() == [4, 5]


def _argpartition_route(sel, n_group, topk_group, k):
    """The group limit and top-k by numpy's ordering primitives: groups
    zeroed = the first n_group - topk_group in (group score asc, index asc)
    order (lexsort), experts chosen = the first k in (sel desc, index asc)."""
    E = sel.size
    G = E // n_group
    sel = sel.astype(np.float32).copy()
    if n_group > 1:
        top2 = np.sort(sel.reshape(n_group, G), axis=1)[:, -2:]
        gs = (top2[:, 1] + top2[:, 0]).astype(np.float32)
        zero = np.lexsort((np.arange(n_group), gs))[:n_group - topk_group]
        for g in zero:
            sel[g * G:(g + 1) * G] = 0.0
    return np.lexsort((np.arange(E), -sel))[:k]


@pytest.mark.parametrize("seed", range(6))
def test_route_group_limit_matches_argpartition_order(oracle, seed):
    """Many tied group scores (biases from a small dyadic set): the oracle's
    choice equals the comparator's, run by numpy's lexsort."""
    rng = np.random.default_rng(300 + seed)
    E, n_group = 32, 8
    for topk_group in (1, 3, 5, 7):
        cb = rng.choice(np.array([-0.25, 0.0, 0.125, 0.25], np.float32), E)
        _, inds, _ = _const_route(oracle, cb, top_k=4, n_group=n_group, topk_group=topk_group)
        sel = (np.float32(0.5) + cb).astype(np.float32)
        want = _argpartition_route(sel, n_group, topk_group, 4)
        assert inds[0].tolist() == want.tolist(), (topk_group, cb)


# ------------------------------------------------------------------ block

def _weights(oracle, cfg, seed_std=0.05, shared=True):
    E, H, I, Is = cfg["n_experts"], cfg["hidden"], cfg["inter"], cfg["shared_inter"]
    w = dict(gate_w=rand_bf16((E, H), seed_std),
             fc1=oracle.quantize(rand_bf16((E, I, H), 0.05)),
             fc2=oracle.quantize(rand_bf16((E, H, I), 0.05)))
    if shared and Is:
        w["shared_up"] = oracle.quantize(rand_bf16((Is, H), 0.05))
        w["shared_down"] = oracle.quantize(rand_bf16((H, Is), 0.05))
    return w


def _deq(oracle, t):
    return oracle.dequantize(*t).astype(np.float64)


def _dense(oracle, cfg, w, x, mistake=None):
    """fp64 dense formula: y = sum_j s_j fc2_e(relu(bf16(fc1_e x))^2) +
    shared(x), with the router's own choice and scores."""
    _, inds, scores = oracle.nh_route(cfg, x, w["gate_w"], w.get("cbias"))
    xf = bf(x).astype(np.float64)
    f1, f2 = _deq(oracle, w["fc1"]), _deq(oracle, w["fc2"])

    def act(h64):
        h = bf(_bf16_round64(h64)).astype(np.float64)
        if mistake == "relu":
            return np.maximum(h, 0)
        return np.maximum(h, 0) ** 2

    y = np.zeros((x.shape[0], cfg["hidden"]))
    for t in range(x.shape[0]):
        for j, e in enumerate(inds[t]):
            s = float(scores[t, j])
            if mistake == "unscaled":
                s /= cfg["scaling"]
            y[t] += s * (f2[e] @ act(f1[e] @ xf[t]))
    if cfg["shared_inter"] and mistake != "shared":
        su, sd = _deq(oracle, w["shared_up"]), _deq(oracle, w["shared_down"])
        for t in range(x.shape[0]):
            y[t] += sd @ act(su @ xf[t])
    return y


@pytest.mark.parametrize("groups", [(1, 1), (4, 2)])
def test_block_dense_formula(oracle, groups):
    """The block (both accumulation modes) against the dense fp64 formula:
    relative L2 within the bf16 output rounding; planted mistakes (relu for
    relu^2, the scaling dropped, the shared expert dropped) are far outside."""
    cfg = _cfg(hidden=128, n_experts=8, top_k=2, inter=128, shared_inter=128,
               n_group=groups[0], topk_group=groups[1])
    w = _weights(oracle, cfg)
    w["cbias"] = RNG.standard_normal(cfg["n_experts"]).astype(np.float32) * 0.05
    x = rand_bf16((5, cfg["hidden"]))
    ref = _dense(oracle, cfg, w, x)
    for mode in (oracle.ACC_F64, oracle.ACC_A):
        y, _, _ = oracle.nh_moe_block(cfg, w, x, mode)
        got = bf(y).astype(np.float64)
        rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert rel < 4e-3, (mode, rel)
    got = bf(oracle.nh_moe_block(cfg, w, x, oracle.ACC_F64)[0]).astype(np.float64)
    for mistake in ("relu", "unscaled", "shared"):
        bad = _dense(oracle, cfg, w, x, mistake)
        assert np.linalg.norm(got - bad) / np.linalg.norm(bad) > 5e-2, mistake


def test_block_scaling_is_exact(oracle):
    """Without a shared expert, routed_scaling_factor 2 doubles every output
    exactly (a power of two through fp32 products and sums and the bf16
    rounding)."""
    cfg = _cfg(hidden=128, n_experts=8, top_k=3, inter=128, shared_inter=0, scaling=1.0)
    w = _weights(oracle, cfg)
    x = rand_bf16((4, 128))
    y1, i1, s1 = oracle.nh_moe_block(cfg, w, x)
    y2, i2, s2 = oracle.nh_moe_block(dict(cfg, scaling=2.0), w, x)
    assert np.array_equal(i1, i2) and np.array_equal(s2, 2 * s1)
    assert np.array_equal(bf(y2), 2 * bf(y1))


def test_block_relu_zeroes_negative_fc1(oracle):
    """fc1 rows that dequantise to -0.5 everywhere (scale 0, bias -0.5) with
    a positive x give negative h, which relu zeroes: the routed experts then
    add nothing, so y does not depend on fc2 and equals the shared expert
    alone (the same call with the routed weights replaced)."""
    cfg = _cfg(hidden=128, n_experts=8, top_k=2, inter=128, shared_inter=128)
    w = _weights(oracle, cfg)
    wq, s, b = w["fc1"]
    neg = _bf16_round64(np.full(b.shape, -0.5))
    w["fc1"] = (wq, np.zeros_like(s), neg)
    x = _bf16_round64(np.abs(bf(rand_bf16((3, 128)))) + 0.01)
    y1, _, _ = oracle.nh_moe_block(cfg, w, x)
    w2 = dict(w, fc2=oracle.quantize(rand_bf16((8, 128, 128), 0.5)))
    y2, _, _ = oracle.nh_moe_block(cfg, w2, x)
    assert np.array_equal(y1, y2)
    assert np.any(y1 != 0)


def test_block_forced_choice(oracle):
    """The router's own choice given back reproduces the block bit for bit;
    another choice changes only the tokens whose choice changed."""
    cfg = _cfg(hidden=128, n_experts=8, top_k=2, inter=128, shared_inter=128)
    w = _weights(oracle, cfg)
    x = rand_bf16((4, 128))
    y, inds, scores = oracle.nh_moe_block(cfg, w, x)
    y2, inds2, scores2 = oracle.nh_moe_block(cfg, w, x, inds=inds)
    assert np.array_equal(y, y2) and np.array_equal(scores, scores2)
    alt = inds.copy()
    alt[2] = [(inds[2, 0] + 1) % 8, (inds[2, 1] + 3) % 8] if (inds[2, 0] + 1) % 8 != (inds[2, 1] + 3) % 8 \
        else [(inds[2, 0] + 1) % 8, (inds[2, 1] + 2) % 8]
    y3, _, _ = oracle.nh_moe_block(cfg, w, x, inds=alt)
    assert np.array_equal(np.delete(y3, 2, 0), np.delete(y, 2, 0))
    assert not np.array_equal(y3[2], y[2])
