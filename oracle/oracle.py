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
    ]


_vp = C.c_void_p


class _W(C.Structure):
    _fields_ = [(n, _vp) for n in (
        "router_w", "router_bias",
        "gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s", "down_b",
        "sh_gate_w", "sh_gate_s", "sh_gate_b", "sh_up_w", "sh_up_s", "sh_up_b",
        "sh_down_w", "sh_down_s", "sh_down_b", "sh_expert_gate_w",
        "router_s", "router_b", "sh_expert_gate_s", "sh_expert_gate_b")]


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
        lib.orc_gather_qmm.argtypes = [_vp, i64, i64, i64, _vp, _vp, _vp, i64, i64, _vp, _vp, i64,
                                       C.c_int, _vp]
        lib.orc_router_topk.argtypes = [_vp, i64, i64, _vp, i64, _vp, C.c_int, C.c_int, _vp, _vp,
                                        _vp, _vp]
        lib.orc_router_topk_q.argtypes = [_vp, i64, i64, _vp, _vp, _vp, i64, _vp, C.c_int, C.c_int,
                                          _vp, _vp, _vp, _vp]
        lib.orc_moe_sort.argtypes = [_vp, i64, C.c_int, i64, _vp, _vp, _vp, _vp, _vp]
        lib.orc_moe_block.argtypes = [C.POINTER(_Cfg), C.POINTER(_W), _vp, i64, C.c_int, _vp, i64,
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


def router_topk(x, wr, k, norm_topk=False, logit_bias=None):
    """-> logits [T,E], probs [T,E] (bf16 bits), inds [T,k] u32, scores [T,k] bf16.
    wr: bf16 [E, H], or a quantized (wq u32 [E, H/8], scales, biases) tuple."""
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
    rc = load().orc_router_topk_q(_p(x), T, H, _p(wq), _p(ws), _p(wb), E, _p(lb), k,
                                  int(norm_topk), _p(logits), _p(probs), _p(inds), _p(scores))
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


def moe_block(cfg: dict, w: dict, x, mode=ACC_A, tokens=None):
    """cfg keys: hidden, n_experts, top_k, inter, shared_inter, norm_topk.
    w keys: router_w (bf16, or a quantized (wq, s, b) tuple), router_bias?,
    gate/up/down (wq, s, b) tuples, shared_gate/shared_up/shared_down tuples?,
    shared_expert_gate_w? (bf16 or a quantized tuple).
    Returns (y [T,H] with rows only for `tokens` filled when given, inds, scores)."""
    x = _c(x, np.uint16)
    H = cfg["hidden"]
    T = x.size // H
    k = cfg["top_k"]
    c = _Cfg(H, cfg["n_experts"], k, cfg["inter"], cfg.get("shared_inter", 0),
             int(cfg.get("norm_topk", False)), 64, 4)
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
    inds = np.empty((T, k), np.uint32)
    scores = np.empty((T, k), np.uint16)
    sub = None if tokens is None else np.ascontiguousarray(tokens, dtype=np.int64)
    rc = load().orc_moe_block(C.byref(c), C.byref(ww), _p(x), T, mode, _p(sub),
                              0 if sub is None else sub.size, _p(y), _p(inds), _p(scores))
    assert rc == 0, rc
    return y, inds, scores
