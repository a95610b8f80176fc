"""Pins the decoder-stack functions of the CPU oracle (rms_norm, RoPE, scaled
dot-product attention, the layer composition) without the reference library.

Each function is checked against what the mathematics fixes: closed forms
(constant rows, position 0, one key, equal keys), invariants (power-of-two
scaling, rotation norms, composition of rotations, KV-cache consistency,
batch independence) and numpy fp64 restatements (x / rms * w, complex
rotation, softmax(QK^T)V, the whole stack on tiny shapes). Several tests
plant a mistake on the CPU side and check that the comparison notices.
"""
from __future__ import annotations

import numpy as np
import pytest

RNG = np.random.default_rng(20261202)


def bf(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_bf16(oracle, a):
    return oracle.f32_to_bf16_array(np.asarray(a, np.float32))


def ulps_bf16(a, b):
    """distance in bf16 ulps of two bf16 arrays (same sign region)"""
    ia = np.asarray(a, np.uint16).astype(np.int32)
    ib = np.asarray(b, np.uint16).astype(np.int32)
    sa = np.where(ia & 0x8000, -(ia & 0x7FFF), ia)
    sb = np.where(ib & 0x8000, -(ib & 0x7FFF), ib)
    return np.abs(sa - sb)


# ------------------------------------------------------------------ rms_norm

def test_rms_norm_constant_rows(oracle):
    """A constant row c has rms |c|: the normalised row is sign(c) (to within
    eps/(2c^2), far below half a bf16 ulp) and the output is +-w exactly."""
    H = 256
    w = to_bf16(oracle, RNG.standard_normal(H))
    for c in (2.0, -3.0, 0.5, 96.0):
        x = to_bf16(oracle, np.full((1, H), c))
        out = oracle.rms_norm(x, w, 1e-6)
        np.testing.assert_array_equal(bf(out[0]), np.sign(c) * bf(w))


def test_rms_norm_power_of_two_invariance(oracle):
    """With eps = 0, x * 2^k normalises to the same bits (every step scales
    exactly)."""
    x = to_bf16(oracle, RNG.standard_normal((5, 512)))
    w = to_bf16(oracle, RNG.standard_normal(512) * 0.5 + 1.0)
    ref = oracle.rms_norm(x, w, 0.0)
    for k in (-20, -3, 5, 40):
        xs = to_bf16(oracle, bf(x) * np.float32(2.0 ** k))
        np.testing.assert_array_equal(oracle.rms_norm(xs, w, 0.0), ref)


def test_rms_norm_matches_numpy(oracle):
    """x / sqrt(mean(x^2) + eps) * w in fp64, within the two bf16 roundings
    (normalised value, then the product with w); a planted mistake (sum
    instead of mean) is caught by the same comparison."""
    x = to_bf16(oracle, RNG.standard_normal((7, 2048)) * 3.0)
    w = to_bf16(oracle, RNG.standard_normal(2048) * 0.2 + 1.0)
    eps = 1e-6
    out = oracle.rms_norm(x, w, eps)
    xf = bf(x).astype(np.float64)
    ref = xf / np.sqrt((xf ** 2).mean(-1, keepdims=True) + np.float64(np.float32(eps))) * bf(w)
    rel = np.abs(bf(out) - ref) / np.maximum(np.abs(ref), 1e-30)
    assert rel.max() <= 2.0 ** -7, rel.max()
    wrong = xf / np.sqrt((xf ** 2).sum(-1, keepdims=True) + eps) * bf(w)
    assert (np.abs(bf(out) - wrong) / np.maximum(np.abs(wrong), 1e-30)).max() > 1.0


# ------------------------------------------------------------------ RoPE

def test_rope_table_matches_numpy(oracle):
    n_pos, hd, base = 300, 128, 1e6
    cs = oracle.rope_table(n_pos, hd, base)
    i = np.arange(hd // 2)
    th = np.arange(n_pos)[:, None] * np.power(base, -2.0 * i / hd)[None, :]
    np.testing.assert_allclose(cs[..., 0], np.cos(th), rtol=0, atol=2e-7)
    np.testing.assert_allclose(cs[..., 1], np.sin(th), rtol=0, atol=2e-7)


def test_rope_position_zero_is_identity(oracle):
    cs = oracle.rope_table(4, 64, 1e4)
    x = to_bf16(oracle, RNG.standard_normal((3, 4, 64)))
    np.testing.assert_array_equal(oracle.rope(x, [0, 0, 0], cs), x)


def test_rope_matches_complex_rotation(oracle):
    """Pairs (i, i + hd/2) rotate by p * base^(-2i/hd): (x1 + i x2) e^{i theta}
    in numpy complex128, within one bf16 ulp; the traditional pairing (2i,
    2i + 1) and a flipped sine, planted, are far off."""
    hd, base, n_pos = 128, 1e6, 400
    cs = oracle.rope_table(n_pos, hd, base)
    x = to_bf16(oracle, RNG.standard_normal((6, 3, hd)))
    pos = np.array([1, 7, 63, 255, 256, 399])
    out = oracle.rope(x, pos, cs)
    xf = bf(x).astype(np.float64)
    half = hd // 2
    th = pos[:, None, None] * np.power(base, -2.0 * np.arange(half) / hd)[None, None, :]
    z = (xf[..., :half] + 1j * xf[..., half:]) * np.exp(1j * th)
    ref = np.concatenate([z.real, z.imag], -1)
    got = bf(out).astype(np.float64)
    assert (np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-6).all()
    zt = (xf[..., 0::2] + 1j * xf[..., 1::2]) * np.exp(1j * th)
    trad = np.empty_like(xf)
    trad[..., 0::2], trad[..., 1::2] = zt.real, zt.imag
    assert np.abs(got - trad).max() > 0.5
    zf = (xf[..., :half] + 1j * xf[..., half:]) * np.exp(-1j * th)
    assert np.abs(got - np.concatenate([zf.real, zf.imag], -1)).max() > 0.5


def test_rope_preserves_pair_norms_and_composes(oracle):
    """|x'| = |x| per pair, and rotating by p1 then p2 equals rotating by
    p1 + p2 (within the roundings of each step)."""
    hd = 64
    cs = oracle.rope_table(64, hd, 1e4)
    x = to_bf16(oracle, RNG.standard_normal((4, 2, hd)))
    a = oracle.rope(x, [3, 3, 3, 3], cs)
    xf, af = bf(x).astype(np.float64), bf(a).astype(np.float64)
    h = hd // 2
    n0 = np.hypot(xf[..., :h], xf[..., h:])
    n1 = np.hypot(af[..., :h], af[..., h:])
    assert (np.abs(n1 - n0) <= n0 * 2.0 ** -7 + 1e-6).all()
    b = oracle.rope(a, [5, 5, 5, 5], cs)
    c = oracle.rope(x, [8, 8, 8, 8], cs)
    assert (np.abs(bf(b) - bf(c)) <= np.abs(bf(c)) * 2.0 ** -6 + 2e-2).all()


# ------------------------------------------------------------------ attention

def _cache(oracle, nkv, max_seq, hd, n):
    kc = np.zeros((nkv, max_seq, hd), np.uint16)
    vc = np.zeros_like(kc)
    kc[:, :n] = to_bf16(oracle, RNG.standard_normal((nkv, n, hd)))
    vc[:, :n] = to_bf16(oracle, RNG.standard_normal((nkv, n, hd)))
    return kc, vc


def test_sdpa_one_key_returns_its_value(oracle):
    """A query at position 0 sees key 0 only: out = v0 exactly."""
    kc, vc = _cache(oracle, 2, 8, 64, 1)
    q = to_bf16(oracle, RNG.standard_normal((1, 4, 64)))
    out = oracle.sdpa(q, kc, vc, 0, 0.125)
    for h in range(4):
        np.testing.assert_array_equal(out[0, h], vc[h // 2, 0])


def test_sdpa_equal_keys_average_values(oracle):
    """Equal keys give equal weights: the output is the mean of the values
    (fp64 mean rounded once)."""
    nkv, hd, n = 1, 32, 9
    kc, vc = _cache(oracle, nkv, 16, hd, n)
    kc[:, :n] = kc[:, :1]
    q = to_bf16(oracle, RNG.standard_normal((1, 1, hd)))
    out = oracle.sdpa(q, kc, vc, n - 1, 0.2)
    ref = bf(vc[0, :n]).astype(np.float64).mean(0)
    np.testing.assert_array_equal(out[0, 0], oracle.f64_to_bf16(ref))


@pytest.mark.parametrize("L,q_off,nh,nkv", [(1, 11, 4, 4), (5, 0, 4, 2), (6, 3, 6, 3), (1, 0, 2, 1)])
def test_sdpa_matches_numpy(oracle, L, q_off, nh, nkv):
    """softmax(q k^T * scale + causal mask) v in fp64 with the GQA mapping
    head h -> kv head h / (nh / nkv), within one bf16 ulp (2^-8 relative);
    a planted mistake (no causal mask) is caught."""
    hd, max_seq = 64, 32
    n = q_off + L
    kc, vc = _cache(oracle, nkv, max_seq, hd, n)
    q = to_bf16(oracle, RNG.standard_normal((L, nh, hd)))
    scale = float(np.float32(1 / np.sqrt(hd)))
    out = oracle.sdpa(q, kc, vc, q_off, scale)
    qf, kf, vf = (bf(a).astype(np.float64) for a in (q, kc, vc))
    ref = np.empty((L, nh, hd))
    nomask = np.empty_like(ref)
    for h in range(nh):
        g = h // (nh // nkv)
        s = qf[:, h] @ kf[g, :n].T * scale
        for l in range(L):
            for tgt, lim in ((ref, q_off + l + 1), (nomask, n)):
                p = np.exp(s[l, :lim] - s[l, :lim].max())
                tgt[l, h] = (p / p.sum()) @ vf[g, :lim]
    got = bf(out).astype(np.float64)
    assert (np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-6).all()
    if L > 1:
        assert np.abs(got - nomask).max() > 1e-2


def _numpy_attn(q, kc, vc, nk, scale, nkv):
    """fp64 softmax(q k^T * scale) v over keys 0 .. nk - 1 of one query."""
    qf, kf, vf = (bf(a).astype(np.float64) for a in (q, kc, vc))
    nh = q.shape[1]
    ref = np.empty((nh, q.shape[2]))
    for h in range(nh):
        g = h // (nh // nkv)
        s = kf[g, :nk] @ qf[0, h] * scale
        p = np.exp(s - s.max())
        ref[h] = (p / p.sum()) @ vf[g, :nk]
    return ref


def test_sdpa_split_one_key_and_equal_keys(oracle):
    """The split order keeps the closed forms: one key gives its value, equal
    keys the fp64 mean of the values (here over 5 ranges: 150 keys)."""
    kc, vc = _cache(oracle, 2, 8, 64, 1)
    q = to_bf16(oracle, RNG.standard_normal((1, 4, 64)))
    out = oracle.sdpa_split(q, kc, vc, 0, 0.125)
    for h in range(4):
        np.testing.assert_array_equal(out[0, h], vc[h // 2, 0])
    n = 150
    kc, vc = _cache(oracle, 1, 160, 32, n)
    kc[:, :n] = kc[:, :1]
    q = to_bf16(oracle, RNG.standard_normal((1, 1, 32)))
    out = oracle.sdpa_split(q, kc, vc, n - 1, 0.2)
    ref = bf(vc[0, :n]).astype(np.float64).mean(0)
    got = bf(out[0, 0]).astype(np.float64)
    assert (np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-6).all()


@pytest.mark.parametrize("nk", [1, 31, 32, 33, 65, 300, 481, 512, 513, 2500])
def test_sdpa_split_matches_numpy(oracle, nk):
    """At range-count boundaries (1 range up to 32 keys, 16 from 481) and
    with one key's score far above the rest in the first range (every other
    range's sums then carry f_s << 1): within one bf16 ulp of numpy's fp64
    softmax and of the four-quarter order. A planted mistake (the ranges'
    sums added without the exp(m_s - M) factors) is far off."""
    nh, nkv, hd = 4, 2, 64
    kc, vc = _cache(oracle, nkv, nk + 1, hd, nk)
    q = to_bf16(oracle, RNG.standard_normal((1, nh, hd)))
    kc[:, 0] = to_bf16(oracle, bf(q[0, 0]).astype(np.float64) * 3.0)  # a dominant early key
    scale = float(np.float32(1 / np.sqrt(hd)))
    out = oracle.sdpa_split(q, kc, vc, nk - 1, scale)
    ref = _numpy_attn(q, kc, vc, nk, scale, nkv)
    got = bf(out[0]).astype(np.float64)
    assert (np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-6).all()
    quart = bf(oracle.sdpa(q, kc, vc, nk - 1, scale)[0]).astype(np.float64)
    assert (np.abs(got - quart) <= np.abs(quart) * 2.0 ** -8 + 1e-6).all()
    if nk > 32:  # the planted mistake: unscaled range sums
        qf, kf, vf = (bf(a).astype(np.float64) for a in (q, kc, vc))
        S = min(16, (nk + 31) // 32)
        s = kf[0, :nk] @ qf[0, 0] * scale
        num = den = 0.0
        for r in range(S):
            j0, j1 = nk * r // S, nk * (r + 1) // S
            e = np.exp(s[j0:j1] - s[j0:j1].max())
            num, den = num + e @ vf[0, j0:j1], den + e.sum()
        assert np.abs(num / den - ref[0]).max() > 1e-2


# ------------------------------------------------------------------ the stack

TINY = dict(hidden=128, layers=2, heads=4, kv_heads=2, head_dim=32, vocab=96, eps=1e-6,
            theta=1e4, max_seq=24,
            moe=dict(hidden=128, n_experts=4, top_k=2, inter=64, shared_inter=64, norm_topk=False))


def _tiny_weights(oracle, cfg, seed=3):
    rng = np.random.default_rng(seed)
    H, nh, nkv, hd, V = cfg["hidden"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["vocab"]
    m = cfg["moe"]
    E, I, Is = m["n_experts"], m["inter"], m["shared_inter"]

    def b16(*shape, std=1.0, mean=0.0):
        return to_bf16(oracle, rng.standard_normal(shape) * std + mean)

    def q(*shape):
        return oracle.quantize(b16(*shape, std=0.05))

    layers = []
    for _ in range(cfg["layers"]):
        layers.append(dict(
            in_w=b16(H, std=0.1, mean=1.0), post_w=b16(H, std=0.1, mean=1.0),
            qkv=q((nh + 2 * nkv) * hd, H), qkv_bias=b16((nh + 2 * nkv) * hd, std=0.1),
            o=q(H, nh * hd),
            moe=dict(router_w=b16(E, H, std=0.05), gate=q(E, I, H), up=q(E, I, H), down=q(E, H, I),
                     shared_gate=q(Is, H), shared_up=q(Is, H), shared_down=q(H, Is),
                     shared_expert_gate_w=b16(1, H, std=0.05))))
    return dict(embed=b16(V, H), norm_w=b16(H, std=0.1, mean=1.0), lm_head=q(V, H), layers=layers)


def test_stack_cache_consistency(oracle):
    """Prefill of L tokens then one decode step gives the bits of a prefill
    of L + 1 tokens (cache offsets, RoPE positions and the causal mask agree),
    and a batch of two sequences gives each sequence's own bits."""
    w = _tiny_weights(oracle, TINY)
    ids = RNG.integers(0, TINY["vocab"], size=(2, 7))
    full = oracle.DecoderStack(TINY, w, 2).forward(ids, 0)
    st = oracle.DecoderStack(TINY, w, 2)
    st.forward(ids[:, :6], 0)
    np.testing.assert_array_equal(st.forward(ids[:, 6:], 6), full)
    for b in range(2):
        one = oracle.DecoderStack(TINY, w, 1).forward(ids[b:b + 1], 0)
        np.testing.assert_array_equal(one[0], full[b])


def _numpy_stack(oracle, cfg, w, ids, routing):
    """The stack in fp64 from the dequantised weights, with the oracle's expert
    choice per (layer, token) given (the router is pinned on its own)."""
    H, nh, nkv, hd = cfg["hidden"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    L = ids.shape[0]

    def deq(t):
        return oracle.dequantize(*t).astype(np.float64)

    def norm(x, g):
        return x / np.sqrt((x ** 2).mean(-1, keepdims=True) + cfg["eps"]) * bf(g)

    def rot(x, pos):
        half = hd // 2
        th = pos[:, None, None] * np.power(cfg["theta"], -2.0 * np.arange(half) / hd)
        z = (x[..., :half] + 1j * x[..., half:]) * np.exp(1j * th)
        return np.concatenate([z.real, z.imag], -1)

    def silu(g):
        return g / (1 + np.exp(-g))

    h = bf(w["embed"][ids]).astype(np.float64)
    pos = np.arange(L)
    for li, lw in enumerate(w["layers"]):
        n = norm(h, lw["in_w"])
        qkv = n @ deq(lw["qkv"]).T + bf(lw["qkv_bias"])
        q = rot(qkv[:, :nh * hd].reshape(L, nh, hd), pos)
        k = rot(qkv[:, nh * hd:(nh + nkv) * hd].reshape(L, nkv, hd), pos)
        v = qkv[:, (nh + nkv) * hd:].reshape(L, nkv, hd)
        att = np.empty((L, nh, hd))
        for hh in range(nh):
            g = hh // (nh // nkv)
            s = q[:, hh] @ k[:, g].T / np.sqrt(hd)
            s = np.where(np.tril(np.ones((L, L), bool)), s, -np.inf)
            p = np.exp(s - s.max(-1, keepdims=True))
            att[:, hh] = (p / p.sum(-1, keepdims=True)) @ v[:, g]
        h = h + att.reshape(L, nh * hd) @ deq(lw["o"]).T
        n2 = norm(h, lw["post_w"])
        mw = lw["moe"]
        xr = n2 @ bf(mw["router_w"]).astype(np.float64).T
        pr = np.exp(xr - xr.max(-1, keepdims=True))
        pr /= pr.sum(-1, keepdims=True)
        y = np.zeros_like(h)
        gw, uw, dw = deq(mw["gate"]), deq(mw["up"]), deq(mw["down"])
        for t in range(L):
            for e in routing[li][t]:
                a = silu(n2[t] @ gw[e].T) * (n2[t] @ uw[e].T)
                y[t] += pr[t, e] * (a @ dw[e].T)
        a = silu(n2 @ deq(mw["shared_gate"]).T) * (n2 @ deq(mw["shared_up"]).T)
        sg = 1 / (1 + np.exp(-(n2 @ bf(mw["shared_expert_gate_w"]).astype(np.float64).T)))
        y += sg * (a @ deq(mw["shared_down"]).T)
        h = h + y
    return norm(h, w["norm_w"]) @ deq(w["lm_head"]).T


def test_stack_matches_numpy_fp64(oracle):
    """All logits of a 2-layer tiny stack against the fp64 composition of
    model.cpp's ops (embed, norms, q/k/v with biases, RoPE, causal GQA
    attention, residuals, MoE with shared expert, final norm, lm_head): the
    bf16 roundings between ops leave a relative L2 error of a few 1e-3; a
    planted mistake (the post-attention residual dropped) is far off."""
    w = _tiny_weights(oracle, TINY)
    L = 9
    ids = RNG.integers(0, TINY["vocab"], size=(1, L))
    st = oracle.DecoderStack(TINY, w, 1)
    got = bf(st.forward(ids, 0, last_only=False)).astype(np.float64)
    routing = _oracle_routing(oracle, TINY, w, ids[0])
    ref = _numpy_stack(oracle, TINY, w, ids[0], routing)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel < 2e-2, rel
    bad = dict(w, layers=[dict(lw) for lw in w["layers"]])
    bad["layers"][0]["o"] = oracle.quantize(to_bf16(oracle, np.zeros((TINY["hidden"], 128))))
    ref_bad = _numpy_stack(oracle, TINY, bad, ids[0], routing)
    assert np.linalg.norm(got - ref_bad) / np.linalg.norm(ref_bad) > 5 * rel


def _oracle_routing(oracle, cfg, w, ids):
    """Expert choice of every (layer, token) along the oracle's forward."""
    nh, nkv, hd = cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    L = ids.shape[0]
    cs = oracle.rope_table(cfg["max_seq"], hd, cfg["theta"])
    scale = float(np.float32(1.0 / np.sqrt(hd)))
    h = np.ascontiguousarray(w["embed"][ids])
    pos = np.arange(L)
    out = []
    for lw in w["layers"]:
        n = oracle.rms_norm(h, lw["in_w"], cfg["eps"])
        qkv = oracle.bf16_add(oracle.qmm_t(n, *lw["qkv"]), lw["qkv_bias"][None, :])
        q = oracle.rope(qkv[:, :nh * hd].reshape(L, nh, hd), pos, cs)
        k = oracle.rope(qkv[:, nh * hd:(nh + nkv) * hd].reshape(L, nkv, hd), pos, cs)
        v = qkv[:, (nh + nkv) * hd:].reshape(L, nkv, hd)
        kc = np.zeros((nkv, cfg["max_seq"], hd), np.uint16)
        vc = np.zeros_like(kc)
        kc[:, :L], vc[:, :L] = k.transpose(1, 0, 2), v.transpose(1, 0, 2)
        att = oracle.sdpa(q, kc, vc, 0, scale)
        h = oracle.bf16_add(h, oracle.qmm_t(att.reshape(L, nh * hd), *lw["o"]))
        n2 = oracle.rms_norm(h, lw["post_w"], cfg["eps"])
        y, inds, _ = oracle.moe_block(cfg["moe"], lw["moe"], n2)
        out.append(inds)
        h = oracle.bf16_add(h, y)
    return out


def test_moe_block_routed(oracle):
    """moe_block with the expert choice given: its own choice reproduces
    moe_block's bits; another choice changes exactly the tokens it touches."""
    from flashmlx_amd.workloads import WORKLOADS, host_inputs
    import sys
    sys.path.insert(0, str(__import__("pathlib").Path(__file__).parent))
    from helpers import oracle_args
    wl = WORKLOADS["tiny_t5"]
    hi = host_inputs(wl)
    cfg, w = oracle_args(hi, wl.model, oracle.quantize)
    y, inds, scores = oracle.moe_block(cfg, w, hi.x)
    y2, inds2, scores2 = oracle.moe_block(cfg, w, hi.x, inds=inds)
    np.testing.assert_array_equal(y2, y)
    np.testing.assert_array_equal(scores2, scores)
    alt = inds.copy()
    alt[2, -1] = next(e for e in range(cfg["n_experts"]) if e not in inds[2])
    y3, _, _ = oracle.moe_block(cfg, w, hi.x, inds=alt)
    np.testing.assert_array_equal(np.delete(y3, 2, 0), np.delete(y, 2, 0))
    assert not np.array_equal(y3[2], y[2])
