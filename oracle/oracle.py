"""numpy binding of the CPU oracle (oracle/_build/libfmx_oracle.so).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and
bench.py's CPU-baseline leg, always as the checker or the CPU baseline,
never as the thing measured. Arrays are numpy: bf16 as uint16 bit patterns,
packed weights as uint32.
"""
from __future__ import annotations

import ctypes as C
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libfmx_oracle.so"

ACC_F64, ACC_A, ACC_B, ACC_C = 0, 1, 2, 3

_lib = None


def build(force: bool = False) -> pathlib.Path:
    """make in oracle/ (recompiles always with force=True)."""
    args = ["make", "-s", "-C", str(HERE)]
    if force:
        args.insert(2, "-B")
    subprocess.run(args, check=True)
    return LIB_PATH


class _Cfg(C.Structure):
    _fields_ = [
        ("hidden", C.c_int64),
        ("n_experts", C.c_int64),
        ("top_k", C.c_int),
        ("inter", C.c_int64),
        ("shared_inter", C.c_int64),
        ("norm_topk", C.c_int),
        ("group_size", C.c_int),
        ("bits", C.c_int),
        ("act_f16", C.c_int),
    ]


_vp = C.c_void_p


class _W(C.Structure):
    _fields_ = [(n, _vp) for n in (
        "router_w", "router_bias",
        "gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s", "down_b",
        "sh_gate_w", "sh_gate_s", "sh_gate_b", "sh_up_w", "sh_up_s", "sh_up_b",
        "sh_down_w", "sh_down_s", "sh_down_b", "sh_expert_gate_w",
        "router_s", "router_b", "sh_expert_gate_s", "sh_expert_gate_b")]


class _NhCfg(C.Structure):
    _fields_ = [
        ("hidden", C.c_int64),
        ("n_experts", C.c_int64),
        ("top_k", C.c_int),
        ("norm_topk", C.c_int),
        ("inter", C.c_int64),
        ("shared_inter", C.c_int64),
        ("n_group", C.c_int),
        ("topk_group", C.c_int),
        ("scaling", C.c_float),
        ("group_size", C.c_int),
        ("bits", C.c_int),
    ]


class _NhW(C.Structure):
    _fields_ = [(n, _vp) for n in (
        "gate_w", "cbias", "fc1_w", "fc1_s", "fc1_b", "fc2_w", "fc2_s", "fc2_b",
        "sh_up_w", "sh_up_s", "sh_up_b", "sh_down_w", "sh_down_s", "sh_down_b")]


def load() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        lib = C.CDLL(str(LIB_PATH))
        lib.orc_bf16_to_f32.restype = C.c_float
        lib.orc_bf16_to_f32.argtypes = [C.c_uint16]
        lib.orc_f32_to_bf16.restype = C.c_uint16
        lib.orc_f32_to_bf16.argtypes = [C.c_float]
        lib.orc_f64_to_bf16.restype = C.c_uint16
        lib.orc_f64_to_bf16.argtypes = [C.c_double]
        lib.orc_exp.restype = C.c_double
        lib.orc_exp.argtypes = [C.c_double]
        lib.orc_sigmoid_bf16.restype = C.c_float
        lib.orc_sigmoid_bf16.argtypes = [C.c_uint16]
        i64 = C.c_int64
        lib.orc_quantize.argtypes = [_vp, i64, i64, C.c_int, C.c_int, _vp, _vp, _vp]
        lib.orc_dequantize.argtypes = [_vp, _vp, _vp, i64, i64, C.c_int, C.c_int, _vp]
        lib.orc_qmm_t.argtypes = [_vp, i64, i64, _vp, _vp, _vp, i64, C.c_int, _vp]
        lib.orc_qmm_t_f16.argtypes = [_vp, i64, i64, _vp, _vp, _vp, i64, C.c_int, _vp]
        lib.orc_gather_qmm_f16.argtypes = [_vp, i64, i64, i64, _vp, _vp, _vp, i64, i64, _vp, _vp, i64,
                                           C.c_int, _vp]
        lib.orc_f16_to_f32.restype = C.c_float
        lib.orc_f16_to_f32.argtypes = [C.c_uint16]
        lib.orc_f32_to_f16.restype = C.c_uint16
        lib.orc_f32_to_f16.argtypes = [C.c_float]
        lib.orc_gather_qmm.argtypes = [_vp, i64, i64, i64, _vp, _vp, _vp, i64, i64, _vp, _vp, i64,
                                       C.c_int, _vp]
        lib.orc_router_topk.argtypes = [_vp, i64, i64, _vp, i64, _vp, C.c_int, C.c_int, _vp, _vp,
                                        _vp, _vp]
        lib.orc_router_topk_q.argtypes = [_vp, i64, i64, _vp, _vp, _vp, i64, _vp, C.c_int, C.c_int,
                                          _vp, _vp, _vp, _vp]
        lib.orc_router_topk_dt.argtypes = [_vp, i64, i64, _vp, _vp, _vp, i64, _vp, C.c_int, C.c_int,
                                           C.c_int, _vp, _vp, _vp, _vp]
        lib.orc_f64_to_f16.restype = C.c_uint16
        lib.orc_f64_to_f16.argtypes = [C.c_double]
        lib.orc_sigmoid_f16.restype = C.c_float
        lib.orc_sigmoid_f16.argtypes = [C.c_uint16]
        lib.orc_moe_sort.argtypes = [_vp, i64, C.c_int, i64, _vp, _vp, _vp, _vp, _vp]
        lib.orc_moe_block.argtypes = [C.POINTER(_Cfg), C.POINTER(_W), _vp, i64, C.c_int, _vp, i64,
                                      _vp, _vp, _vp]
        lib.orc_rms_norm.argtypes = [_vp, i64, i64, _vp, C.c_float, _vp]
        lib.orc_rope_table.argtypes = [i64, i64, C.c_double, _vp]
        lib.orc_rope_table.restype = None
        lib.orc_rope.argtypes = [_vp, i64, i64, i64, _vp, _vp]
        lib.orc_sdpa.argtypes = [_vp, i64, i64, i64, _vp, _vp, i64, i64, i64, C.c_float, _vp]
        lib.orc_sdpa_split.argtypes = [_vp, i64, i64, i64, _vp, _vp, i64, i64, i64, C.c_float, _vp]
        lib.orc_moe_block_routed.argtypes = [C.POINTER(_Cfg), C.POINTER(_W), _vp, i64, C.c_int, _vp,
                                             _vp, _vp]
        lib.orc_sigmoid_f32.restype = C.c_float
        lib.orc_sigmoid_f32.argtypes = [C.c_uint16]
        lib.orc_nh_route.argtypes = [C.POINTER(_NhCfg), _vp, i64, _vp, _vp, _vp, _vp, _vp]
        lib.orc_nh_moe_block.argtypes = [C.POINTER(_NhCfg), C.POINTER(_NhW), _vp, i64, C.c_int, _vp,
                                         _vp, _vp, _vp]
        lib.orc_set_threads.argtypes = [C.c_int]
        lib.orc_get_threads.restype = C.c_int
        _lib = lib
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dt):
    a = np.ascontiguousarray(a)
    assert a.dtype == dt, (a.dtype, dt)
    return a


def set_threads(n: int) -> None:
    load().orc_set_threads(n)


def get_threads() -> int:
    return load().orc_get_threads()


# ---------------------------------------------------------------- numerics

def f32_to_bf16(x) -> np.ndarray:
    lib = load()
    return np.array([lib.orc_f32_to_bf16(float(v)) for v in np.ravel(x)], dtype=np.uint16)


def f64_to_bf16(x) -> np.ndarray:
    lib = load()
    return np.array([lib.orc_f64_to_bf16(float(v)) for v in np.ravel(x)], dtype=np.uint16)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_array(a) -> np.ndarray:
    """Vectorised round-to-nearest-even float32 -> bf16 bits (same rule as
    orc_f32_to_bf16, checked against it in the tests)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def exp(r: float) -> float:
    return load().orc_exp(r)


# ---------------------------------------------------------------- ops

def quantize(w_bf16: np.ndarray, group_size=64, bits=4):
    w = _c(w_bf16, np.uint16)
    K = w.shape[-1]
    N = w.size // K
    wq = np.empty(w.shape[:-1] + (K // 8,), np.uint32)
    s = np.empty(w.shape[:-1] + (K // group_size,), np.uint16)
    b = np.empty_like(s)
    rc = load().orc_quantize(_p(w), N, K, group_size, bits, _p(wq), _p(s), _p(b))
    assert rc == 0, rc
    return wq, s, b


def dequantize(wq, s, b, group_size=64, bits=4) -> np.ndarray:
    wq, s, b = _c(wq, np.uint32), _c(s, np.uint16), _c(b, np.uint16)
    K = wq.shape[-1] * 8
    N = wq.size // (K // 8)
    out = np.empty(wq.shape[:-1] + (K,), np.float32)
    rc = load().orc_dequantize(_p(wq), _p(s), _p(b), N, K, group_size, bits, _p(out))
    assert rc == 0, rc
    return out


def qmm_t(x, wq, s, b, mode=ACC_A) -> np.ndarray:
    x, wq, s, b = _c(x, np.uint16), _c(wq, np.uint32), _c(s, np.uint16), _c(b, np.uint16)
    K = x.shape[-1]
    M = x.size // K
    N = wq.shape[-2]
    out = np.empty(x.shape[:-1] + (N,), np.uint16)
    rc = load().orc_qmm_t(_p(x), M, K, _p(wq), _p(s), _p(b), N, mode, _p(out))
    assert rc == 0, rc
    return out


def qmm_t_f16(x, wq, s, b, mode=ACC_A) -> np.ndarray:
    """quantized_matmul with float16 x, scales, biases and output (bit patterns as uint16)."""
    x, wq, s, b = _c(x, np.uint16), _c(wq, np.uint32), _c(s, np.uint16), _c(b, np.uint16)
    K = x.shape[-1]
    M = x.size // K
    N = wq.shape[-2]
    out = np.empty(x.shape[:-1] + (N,), np.uint16)
    rc = load().orc_qmm_t_f16(_p(x), M, K, _p(wq), _p(s), _p(b), N, mode, _p(out))
    assert rc == 0, rc
    return out


def gather_qmm_f16(x, wq, s, b, lhs, rhs, mode=ACC_A) -> np.ndarray:
    """gather_qmm with float16 x, scales, biases and output."""
    x, wq, s, b = _c(x, np.uint16), _c(wq, np.uint32), _c(s, np.uint16), _c(b, np.uint16)
    lhs, rhs = _c(lhs, np.uint32), _c(rhs, np.uint32)
    n_x, M, K = x.shape
    E, N = wq.shape[0], wq.shape[1]
    nb = lhs.size
    out = np.empty((nb, M, N), np.uint16)
    rc = load().orc_gather_qmm_f16(_p(x), n_x, M, K, _p(wq), _p(s), _p(b), E, N, _p(lhs), _p(rhs), nb,
                                   mode, _p(out))
    assert rc == 0, rc
    return out


def gather_qmm(x, wq, s, b, lhs, rhs, mode=ACC_A) -> np.ndarray:
    """x [n_x, M, K]; wq [E, N, K/8]; lhs/rhs flat, equal length nb -> [nb, M, N]."""
    x, wq, s, b = _c(x, np.uint16), _c(wq, np.uint32), _c(s, np.uint16), _c(b, np.uint16)
    lhs, rhs = _c(lhs, np.uint32), _c(rhs, np.uint32)
    n_x, M, K = x.shape
    E, N = wq.shape[0], wq.shape[1]
    nb = lhs.size
    out = np.empty((nb, M, N), np.uint16)
    rc = load().orc_gather_qmm(_p(x), n_x, M, K, _p(wq), _p(s), _p(b), E, N, _p(lhs), _p(rhs), nb,
                               mode, _p(out))
    assert rc == 0, rc
    return out


def router_topk(x, wr, k, norm_topk=False, logit_bias=None, f16=False):
    """-> logits [T,E], probs [T,E] (bf16 bits), inds [T,k] u32, scores [T,k] bf16.
    wr: bf16 [E, H], or a quantized (wq u32 [E, H/8], scales, biases) tuple.
    f16: every input and output in float16 instead (orc_router_topk_dt)."""
    x = _c(x, np.uint16)
    if isinstance(wr, tuple):
        wq, ws, wb = _c(wr[0], np.uint32), _c(wr[1], np.uint16), _c(wr[2], np.uint16)
    else:
        wq, ws, wb = _c(wr, np.uint16), None, None
    H = x.shape[-1]
    T = x.size // H
    E = wq.shape[0]
    lb = None if logit_bias is None else _c(logit_bias, np.uint16)
    logits = np.empty((T, E), np.uint16)
    probs = np.empty((T, E), np.uint16)
    inds = np.empty((T, k), np.uint32)
    scores = np.empty((T, k), np.uint16)
    rc = load().orc_router_topk_dt(_p(x), T, H, _p(wq), _p(ws), _p(wb), E, _p(lb), k,
                                   int(norm_topk), int(f16), _p(logits), _p(probs), _p(inds), _p(scores))
    assert rc == 0, rc
    return logits, probs, inds, scores


def moe_sort(inds, E):
    inds = _c(inds, np.uint32)
    T, k = inds.shape
    n = T * k
    order, inv, src, idx = (np.empty(n, np.uint32) for _ in range(4))
    offsets = np.empty(E + 1, np.uint32)
    rc = load().orc_moe_sort(_p(inds), T, k, E, _p(order), _p(inv), _p(src), _p(idx), _p(offsets))
    assert rc == 0, rc
    return order, inv, src, idx, offsets


def moe_block(cfg: dict, w: dict, x, mode=ACC_A, tokens=None, inds=None):
    """cfg keys: hidden, n_experts, top_k, inter, shared_inter, norm_topk,
    act_f16 (float16 activations, scales, biases and router: every array in
    and out is then fp16 bits; modes ACC_A and ACC_F64).
    w keys: router_w (bf16, or a quantized (wq, s, b) tuple), router_bias?,
    gate/up/down (wq, s, b) tuples, shared_gate/shared_up/shared_down tuples?,
    shared_expert_gate_w? (bf16 or a quantized tuple).
    Returns (y [T,H] with rows only for `tokens` filled when given, inds, scores).
    inds [T, k] given: that expert choice (orc_moe_block_routed), scores from
    this router's probabilities."""
    x = _c(x, np.uint16)
    H = cfg["hidden"]
    T = x.size // H
    k = cfg["top_k"]
    c = _Cfg(H, cfg["n_experts"], k, cfg["inter"], cfg.get("shared_inter", 0),
             int(cfg.get("norm_topk", False)), 64, 4, int(cfg.get("act_f16", False)))
    keep = []

    def ptr(a, dt):
        if a is None:
            return None
        a = _c(a, dt)
        keep.append(a)
        return a.ctypes.data

    ww = _W()
    r = w["router_w"]
    if isinstance(r, tuple):  # quantized router (wq, scales, biases)
        ww.router_w, ww.router_s, ww.router_b = (ptr(r[0], np.uint32), ptr(r[1], np.uint16),
                                                 ptr(r[2], np.uint16))
    else:
        ww.router_w = ptr(r, np.uint16)
    ww.router_bias = ptr(w.get("router_bias"), np.uint16)
    for nm, key in (("gate", "gate"), ("up", "up"), ("down", "down"),
                    ("sh_gate", "shared_gate"), ("sh_up", "shared_up"), ("sh_down", "shared_down")):
        t = w.get(key)
        if t is None:
            continue
        setattr(ww, nm + "_w", ptr(t[0], np.uint32))
        setattr(ww, nm + "_s", ptr(t[1], np.uint16))
        setattr(ww, nm + "_b", ptr(t[2], np.uint16))
    g = w.get("shared_expert_gate_w")
    if isinstance(g, tuple):  # quantized shared-expert gate
        ww.sh_expert_gate_w, ww.sh_expert_gate_s, ww.sh_expert_gate_b = (
            ptr(g[0], np.uint32), ptr(g[1], np.uint16), ptr(g[2], np.uint16))
    else:
        ww.sh_expert_gate_w = ptr(g, np.uint16)
    y = np.zeros((T, H), np.uint16)
    scores = np.empty((T, k), np.uint16)
    if inds is not None:
        inds = _c(np.asarray(inds, dtype=np.uint32).reshape(T, k), np.uint32)
        rc = load().orc_moe_block_routed(C.byref(c), C.byref(ww), _p(x), T, mode, _p(inds), _p(y),
                                         _p(scores))
        assert rc == 0, rc
        return y, inds, scores
    inds = np.empty((T, k), np.uint32)
    sub = None if tokens is None else np.ascontiguousarray(tokens, dtype=np.int64)
    rc = load().orc_moe_block(C.byref(c), C.byref(ww), _p(x), T, mode, _p(sub),
                              0 if sub is None else sub.size, _p(y), _p(inds), _p(scores))
    assert rc == 0, rc
    return y, inds, scores


# ---------------------------------------------------------------- decoder stack

def rms_norm(x, w, eps):
    x, w = _c(x, np.uint16), _c(w, np.uint16)
    H = x.shape[-1]
    out = np.empty_like(x)
    rc = load().orc_rms_norm(_p(x), x.size // H, H, _p(w), float(eps), _p(out))
    assert rc == 0, rc
    return out


def rope_table(n_pos: int, hd: int, base: float) -> np.ndarray:
    cs = np.empty((n_pos, hd // 2, 2), np.float32)
    load().orc_rope_table(n_pos, hd, float(base), _p(cs))
    return cs


def rope(x, pos, cs):
    """x [T, n_heads, hd] bf16 (a rotated copy is returned), pos [T]."""
    x = np.array(x, dtype=np.uint16, copy=True, order="C")
    pos = _c(np.asarray(pos, dtype=np.int64), np.int64)
    T, nh, hd = x.shape
    rc = load().orc_rope(_p(x), T, nh, hd, _p(pos), _p(_c(cs, np.float32)))
    assert rc == 0, rc
    return x


def sdpa(q, kc, vc, q_off: int, scale: float):
    """q [L, nh, hd]; kc/vc [nkv, max_seq, hd] of one sequence -> [L, nh, hd]."""
    q, kc, vc = _c(q, np.uint16), _c(kc, np.uint16), _c(vc, np.uint16)
    L, nh, hd = q.shape
    nkv, max_seq = kc.shape[0], kc.shape[1]
    out = np.empty_like(q)
    rc = load().orc_sdpa(_p(q), L, nh, hd, _p(kc), _p(vc), nkv, max_seq, q_off, float(scale),
                         _p(out))
    assert rc == 0, rc
    return out


def sdpa_split(q, kc, vc, q_off: int, scale: float):
    """sdpa in the key ranges of the single-token split kernel
    (fmx_oracle.c: orc_sdpa_split)."""
    q, kc, vc = _c(q, np.uint16), _c(kc, np.uint16), _c(vc, np.uint16)
    L, nh, hd = q.shape
    nkv, max_seq = kc.shape[0], kc.shape[1]
    out = np.empty_like(q)
    rc = load().orc_sdpa_split(_p(q), L, nh, hd, _p(kc), _p(vc), nkv, max_seq, q_off,
                               float(scale), _p(out))
    assert rc == 0, rc
    return out



def bf16_add(a, b) -> np.ndarray:
    """MLX add of two bf16 arrays: the fp32 sum rounded to bf16."""
    return f32_to_bf16_array(bf16_to_f32(a) + bf16_to_f32(b))


class DecoderStack:
    """LlamaModel::forward (server/src/model.cpp:1021-1033) over a KV cache:
    embed (:490-497, a bf16 table as the reference pre-dequantizes it at
    load, :214-224), per layer transformer_block (:891-911: input norm,
    attention :843-889 with q/k/v biases and RoPE, residual, post-attention
    norm, moe_block, residual), final norm and lm_head (:499-521).

    cfg: hidden, layers, heads, kv_heads, head_dim, vocab, eps, theta,
    max_seq, moe (moe_block's cfg dict). w: embed [V, H] bf16, norm_w,
    lm_head (wq, s, b), layers: list of dicts with in_w, post_w, qkv
    (wq, s, b) of the q;k;v rows, qkv_bias bf16 or None, o (wq, s, b), moe
    (moe_block's weight dict). B sequences share one cache offset per call.
    """

    def __init__(self, cfg: dict, w: dict, batch: int):
        self.cfg, self.w, self.B = cfg, w, batch
        c = cfg
        self.cs = rope_table(c["max_seq"], c["head_dim"], c["theta"])
        shape = (c["layers"], batch, c["kv_heads"], c["max_seq"], c["head_dim"])
        self.kc = np.zeros(shape, np.uint16)
        self.vc = np.zeros(shape, np.uint16)
        self.scale = float(np.float32(1.0 / np.sqrt(c["head_dim"])))

    def _router_margin(self, mw, x):
        """Per token, the relative gap between the k-th and the (k+1)-th
        largest router probability: where it is small, inputs that differ in
        the last bits can select another expert."""
        m = self.cfg["moe"]
        k, E = m["top_k"], m["n_experts"]
        if k >= E:
            return np.full(x.shape[0], np.inf)
        _, probs, _, _ = router_topk(x, mw["router_w"], k, m.get("norm_topk", False), mw.get("router_bias"))
        p = -np.sort(-bf16_to_f32(probs).astype(np.float64), axis=1)
        return (p[:, k - 1] - p[:, k]) / np.maximum(p[:, k - 1], 1e-300)

    def forward(self, ids, offset: int, last_only: bool = True, mode=ACC_A, return_hidden=False,
                routing=None):
        """ids [B, L] at cache positions offset.. -> logits [B, V] (last_only)
        or [B * L, V]; with return_hidden also the residual stream after the
        last layer [B * L, H]. self.last_margins [layers, B * L]: each
        token's router margin (_router_margin) in each layer; last_probs /
        last_inds: each layer's router probabilities and expert choice.
        routing (a list of [B * L, k] per layer): use that expert choice in
        each layer's MoE block (moe_block(inds=...))."""
        c, w = self.cfg, self.w
        ids = np.asarray(ids, dtype=np.int64)
        B, L = ids.shape
        H, nh, nkv, hd = c["hidden"], c["heads"], c["kv_heads"], c["head_dim"]
        h = np.ascontiguousarray(w["embed"][ids.reshape(-1)])
        pos = np.tile(np.arange(offset, offset + L, dtype=np.int64), B)
        margins = []
        self.last_probs, self.last_inds = [], []
        for li, lw in enumerate(w["layers"]):
            n = rms_norm(h, lw["in_w"], c["eps"])
            qkv = qmm_t(n, *lw["qkv"], mode=mode)
            if lw.get("qkv_bias") is not None:
                qkv = bf16_add(qkv, lw["qkv_bias"][None, :])
            q = qkv[:, :nh * hd].reshape(B * L, nh, hd)
            k = qkv[:, nh * hd:(nh + nkv) * hd].reshape(B * L, nkv, hd)
            v = qkv[:, (nh + nkv) * hd:].reshape(B * L, nkv, hd)
            q, k = rope(q, pos, self.cs), rope(k, pos, self.cs)
            att = np.empty((B * L, nh, hd), np.uint16)
            # single-token forwards: the split kernel's order (head sizes it takes)
            attn = sdpa_split if L == 1 and hd <= 128 and 64 % (hd // 8) == 0 else sdpa
            for b in range(B):
                rows = slice(b * L, (b + 1) * L)
                self.kc[li, b, :, offset:offset + L] = k[rows].transpose(1, 0, 2)
                self.vc[li, b, :, offset:offset + L] = v[rows].transpose(1, 0, 2)
                att[rows] = attn(q[rows], self.kc[li, b], self.vc[li, b], offset, self.scale)
            o = qmm_t(att.reshape(B * L, nh * hd), *lw["o"], mode=mode)
            h = bf16_add(h, o)
            n2 = rms_norm(h, lw["post_w"], c["eps"])
            y, inds, _ = moe_block(c["moe"], lw["moe"], n2, mode,
                                   inds=None if routing is None else routing[li])
            margins.append(self._router_margin(lw["moe"], n2))
            self.last_probs.append(router_topk(n2, lw["moe"]["router_w"], c["moe"]["top_k"],
                                               c["moe"].get("norm_topk", False),
                                               lw["moe"].get("router_bias"))[1])
            self.last_inds.append(inds)
            h = bf16_add(h, y)
        self.last_margins = np.stack(margins)
        hid = h
        if last_only:
            h = np.ascontiguousarray(h.reshape(B, L, H)[:, -1])
        n = rms_norm(h, w["norm_w"], c["eps"])
        logits = qmm_t(n, *w["lm_head"], mode=mode)
        return (logits, hid) if return_hidden else logits


# ---------------------------------------------------------------- Nemotron-H MoE block

def _nh_cfg(cfg: dict) -> _NhCfg:
    return _NhCfg(cfg["hidden"], cfg["n_experts"], cfg["top_k"], int(cfg.get("norm_topk", True)),
                  cfg["inter"], cfg.get("shared_inter", 0), cfg.get("n_group", 1),
                  cfg.get("topk_group", 1), float(cfg.get("scaling", 1.0)), 64, 4)


def sigmoid_f32(logit_bf16: int) -> float:
    return load().orc_sigmoid_f32(int(logit_bf16))


def nh_route(cfg: dict, x, gate_w, cbias=None):
    """Nemotron-H router (nemotron_h.cpp:1017-1050) -> logits [T, E] bf16 bits,
    inds [T, k] u32, scores [T, k] fp32. cbias: fp32 [E] or None."""
    x, gw = _c(x, np.uint16), _c(gate_w, np.uint16)
    H, E, k = cfg["hidden"], cfg["n_experts"], cfg["top_k"]
    T = x.size // H
    cb = None if cbias is None else _c(np.asarray(cbias, dtype=np.float32), np.float32)
    logits = np.empty((T, E), np.uint16)
    inds = np.empty((T, k), np.uint32)
    scores = np.empty((T, k), np.float32)
    c = _nh_cfg(cfg)
    rc = load().orc_nh_route(C.byref(c), _p(x), T, _p(gw), _p(cb), _p(logits), _p(inds), _p(scores))
    assert rc == 0, rc
    return logits, inds, scores


def nh_moe_block(cfg: dict, w: dict, x, mode=ACC_F64, inds=None):
    """Nemotron-H MoE block (nemotron_h.cpp:1010-1111). cfg keys: hidden,
    n_experts, top_k, norm_topk, inter, shared_inter, n_group, topk_group,
    scaling. w keys: gate_w (bf16 [E, H]), cbias (fp32 [E] or None), fc1, fc2,
    shared_up, shared_down ((wq, s, b) tuples; the shared ones optional).
    inds [T, k]: that expert choice. Returns (y [T, H] bf16, inds, scores fp32)."""
    x = _c(x, np.uint16)
    H, k = cfg["hidden"], cfg["top_k"]
    T = x.size // H
    keep = []

    def ptr(a, dt):
        if a is None:
            return None
        a = _c(a, dt)
        keep.append(a)
        return a.ctypes.data

    ww = _NhW()
    ww.gate_w = ptr(w["gate_w"], np.uint16)
    cb = w.get("cbias")
    ww.cbias = ptr(None if cb is None else np.asarray(cb, dtype=np.float32), np.float32)
    for nm, key in (("fc1", "fc1"), ("fc2", "fc2"), ("sh_up", "shared_up"), ("sh_down", "shared_down")):
        t = w.get(key)
        if t is None:
            continue
        setattr(ww, nm + "_w", ptr(t[0], np.uint32))
        setattr(ww, nm + "_s", ptr(t[1], np.uint16))
        setattr(ww, nm + "_b", ptr(t[2], np.uint16))
    c = _nh_cfg(cfg)
    y = np.zeros((T, H), np.uint16)
    inds_out = np.empty((T, k), np.uint32)
    scores = np.empty((T, k), np.float32)
    forced = None if inds is None else _c(np.asarray(inds, dtype=np.uint32).reshape(T, k), np.uint32)
    rc = load().orc_nh_moe_block(C.byref(c), C.byref(ww), _p(x), T, mode, _p(forced), _p(y),
                                 _p(inds_out), _p(scores))
    assert rc == 0, rc
    return y, inds_out, scores
