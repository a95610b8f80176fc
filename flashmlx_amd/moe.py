"""Python face of libfmx: the MoE hot path with the reference's operator names.

Mirrors the MLX calls of FlashMLX's MoE block (server/src/model.cpp:673-807):
`gather_qmm`, `quantized_matmul`, `quantize`, `dequantize`, and the fused
`MoEBlock` standing for LlamaModel::moe_block. torch tensors only carry device
memory and the current HIP stream into the C-ABI; every computation runs in
libfmx.so's HIP kernels.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import _lib
from ._lib import FMX_BF16, FMX_I32, FMX_U32, FmxArray, FmxMoEConfig, FmxMoEWeights, FmxQWeight

_DT = {torch.bfloat16: FMX_BF16, torch.float32: 1, torch.int32: FMX_I32, torch.float16: 4}
if hasattr(torch, "uint32"):
    _DT[torch.uint32] = FMX_U32


def _arr(t: Optional[torch.Tensor], code: Optional[int] = None) -> Optional[FmxArray]:
    if t is None:
        return None
    if not t.is_contiguous():
        raise ValueError("fmx arrays must be contiguous")
    a = FmxArray()
    a.data = t.data_ptr() if t.numel() else None
    a.dtype = code if code is not None else _DT[t.dtype]
    a.ndim = t.dim()
    for i, s in enumerate(t.shape):
        a.shape[i] = s
    return a


def _ref(a: Optional[FmxArray]):
    return C.byref(a) if a is not None else None


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _packed(t: torch.Tensor) -> FmxArray:
    if t.dtype not in (torch.int32, getattr(torch, "uint32", torch.int32)):
        raise TypeError("packed weights must be int32/uint32 tensors")
    return _arr(t, FMX_U32)


def _index(t: Optional[torch.Tensor]) -> Optional[FmxArray]:
    if t is None:
        return None
    if t.dtype == torch.int32:
        return _arr(t, FMX_I32)
    return _arr(t, FMX_U32)


def _shape(a: FmxArray) -> tuple:
    return tuple(a.shape[i] for i in range(a.ndim))


# --------------------------------------------------------------------- ops

def quantized_matmul(x, w, scales, biases, transpose=True, group_size=64, bits=4, mode="affine"):
    """mx::quantized_matmul (server/src/model.cpp:476-480, :741-747)."""
    lib = _lib.load()
    ax, aw = _arr(x), _packed(w)
    shp = FmxArray()
    _lib.check(lib.fmx_quantized_matmul_out_shape(C.byref(ax), C.byref(aw), int(transpose),
                                                  group_size, bits, C.byref(shp)))
    out = torch.empty(_shape(shp), dtype=x.dtype, device=x.device)
    ws = lib.fmx_quantized_matmul_workspace_size(C.byref(ax), C.byref(aw))
    wbuf = torch.empty(max(ws, 1), dtype=torch.uint8, device=x.device)
    _lib.check(lib.fmx_quantized_matmul(
        C.byref(ax), C.byref(aw), _ref(_arr(scales)), _ref(_arr(biases)), int(transpose),
        group_size, bits, mode.encode() if mode else None, C.byref(_arr(out)),
        wbuf.data_ptr(), ws, _stream()))
    return out


def gather_qmm(x, w, scales, biases, lhs_indices=None, rhs_indices=None, transpose=True,
               group_size=64, bits=4, mode="affine", sorted_indices=False):
    """mx::gather_qmm (server/src/model.cpp:703-721)."""
    lib = _lib.load()
    ax, aw = _arr(x), _packed(w)
    al, ar = _index(lhs_indices), _index(rhs_indices)
    shp = FmxArray()
    _lib.check(lib.fmx_gather_qmm_out_shape(C.byref(ax), C.byref(aw), _ref(al), _ref(ar),
                                            int(transpose), group_size, bits, C.byref(shp)))
    out = torch.empty(_shape(shp), dtype=x.dtype, device=x.device)
    ws = lib.fmx_gather_qmm_workspace_size(C.byref(ax), C.byref(aw), _ref(al), _ref(ar))
    wbuf = torch.empty(max(ws, 1), dtype=torch.uint8, device=x.device)
    _lib.check(lib.fmx_gather_qmm(
        C.byref(ax), C.byref(aw), _ref(_arr(scales)), _ref(_arr(biases)), _ref(al), _ref(ar),
        int(transpose), group_size, bits, mode.encode() if mode else None, int(sorted_indices),
        C.byref(_arr(out)), wbuf.data_ptr(), ws, _stream()))
    return out


def quantize(w, group_size=64, bits=4, mode="affine"):
    """mx::quantize(w) -> (wq uint32 as int32, scales bf16, biases bf16)."""
    lib = _lib.load()
    lead = tuple(w.shape[:-1])
    K = w.shape[-1]
    wq = torch.empty(lead + (K // 8,), dtype=torch.int32, device=w.device)
    s = torch.empty(lead + (K // group_size,), dtype=torch.bfloat16, device=w.device)
    b = torch.empty_like(s)
    _lib.check(lib.fmx_quantize(C.byref(_arr(w)), group_size, bits, mode.encode(),
                                C.byref(_arr(wq, FMX_U32)), C.byref(_arr(s)), C.byref(_arr(b)),
                                _stream()))
    return wq, s, b


def dequantize(wq, scales, biases, group_size=64, bits=4, mode="affine"):
    """mx::dequantize -> bf16."""
    lib = _lib.load()
    out = torch.empty(tuple(wq.shape[:-1]) + (wq.shape[-1] * 8,), dtype=torch.bfloat16,
                      device=wq.device)
    _lib.check(lib.fmx_dequantize(C.byref(_arr(wq, FMX_U32)), C.byref(_arr(scales)),
                                  C.byref(_arr(biases)), group_size, bits, mode.encode(),
                                  C.byref(_arr(out)), _stream()))
    return out


def moe_sort(inds: torch.Tensor, num_experts: int):
    """switch_mlp's sort (model.cpp:682-700): order, inv, src, idx, expert_offsets."""
    lib = _lib.load()
    T, k = inds.shape[0], inds.shape[-1]
    n = inds.numel()
    dev = inds.device
    outs = [torch.empty(n, dtype=torch.int32, device=dev) for _ in range(4)]
    offs = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    ws = lib.fmx_moe_sort_workspace_size(n // k, k, num_experts)
    wbuf = torch.empty(max(ws, 1), dtype=torch.uint8, device=dev)
    _lib.check(lib.fmx_moe_sort(inds.data_ptr(), n // k, k, num_experts,
                                *[o.data_ptr() for o in outs], offs.data_ptr(),
                                wbuf.data_ptr(), ws, _stream()))
    order, inv, src, idx = outs
    return order, inv, src, idx, offs


def synth_normal_bf16(n: int, seed: int, stream: int, mean: float = 0.0,
                      std: float = 1.0) -> np.ndarray:
    """Seeded bf16 normals (host, uint16 bit patterns); see fmx_synth.cpp."""
    lib = _lib.load()
    out = np.empty(n, dtype=np.uint16)
    _lib.check(lib.fmx_synth_normal_bf16(out.ctypes.data, n, seed, stream, mean, std))
    return out


def synth_normal_bf16_device(shape, seed: int, stream: int, mean: float = 0.0, std: float = 1.0,
                             device="cuda") -> torch.Tensor:
    """synth_normal_bf16 generated on the device (same values; see fmx_synth.hip)."""
    lib = _lib.load()
    out = torch.empty(shape, dtype=torch.bfloat16, device=device)
    _lib.check(lib.fmx_synth_normal_bf16_device(out.data_ptr(), out.numel(), seed, stream, mean, std,
                                                _stream()))
    return out


# --------------------------------------------------------------------- MoE block

@dataclass
class MoEConfig:
    """ModelConfig's MoE fields (server/include/flashmlx/model.h:40-53)."""
    hidden_size: int
    num_experts: int
    num_experts_per_tok: int
    moe_intermediate_size: int
    shared_expert_intermediate_size: int = 0
    norm_topk_prob: bool = False
    quant_bits: int = 4
    quant_group_size: int = 64
    # ModelConfig::activation_dtype (model.h:34): torch.bfloat16 or
    # torch.float16 (x, y, router rows, scales and biases all of it)
    activation_dtype: torch.dtype = torch.bfloat16

    def to_c(self) -> FmxMoEConfig:
        c = FmxMoEConfig()
        c.hidden_size = self.hidden_size
        c.num_experts = self.num_experts
        c.num_experts_per_tok = self.num_experts_per_tok
        c.norm_topk_prob = int(bool(self.norm_topk_prob))
        c.moe_intermediate_size = self.moe_intermediate_size
        c.shared_expert_intermediate_size = self.shared_expert_intermediate_size
        c.quant_bits = self.quant_bits
        c.quant_group_size = self.quant_group_size
        if self.activation_dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("activation_dtype must be torch.bfloat16 or torch.float16")
        c.activation_dtype = _lib.FMX_F16 if self.activation_dtype == torch.float16 else _lib.FMX_BF16
        return c


@dataclass
class QWeight:
    w: torch.Tensor       # int32 packed [.., N, K/8]
    scales: torch.Tensor  # bf16 [.., N, K/64]
    biases: torch.Tensor  # bf16 [.., N, K/64]

    def to_c(self) -> FmxQWeight:
        q = FmxQWeight()
        q.w, q.scales, q.biases = self.w.data_ptr(), self.scales.data_ptr(), self.biases.data_ptr()
        return q

    def tensors(self) -> list:
        return [self.w, self.scales, self.biases]


def _ptr(t) -> Optional[int]:
    return t.data_ptr() if t is not None else None


@dataclass
class MoEWeights:
    """MoEWeights (server/include/flashmlx/model.h:58-72), stacked over experts.

    The router and the shared-expert gate are a bf16 tensor or a QWeight
    (quantized, model.cpp:758-760 and :792-796). After pack(), the MLX-layout
    expert weights may be dropped (drop_mlx_layout): forwards read only the
    packed copy."""
    router_w: object                       # bf16 [E, H] or QWeight [E, H/8]
    gate: Optional[QWeight]                # [E, I, ..]
    up: Optional[QWeight]
    down: Optional[QWeight]                # [E, H, ..]
    shared_gate: Optional[QWeight] = None  # [Is, ..]
    shared_up: Optional[QWeight] = None
    shared_down: Optional[QWeight] = None
    shared_expert_gate_w: object = None    # bf16 [1, H] or QWeight [1, H/8]
    router_logit_bias: Optional[torch.Tensor] = None     # bf16 [E] (no reference counterpart)
    packed: Optional[torch.Tensor] = None  # uint8 blob from pack() (no reference counterpart)

    @property
    def device(self):
        r = self.router_w
        return (r.w if isinstance(r, QWeight) else r).device

    def to_c(self) -> FmxMoEWeights:
        w = FmxMoEWeights()
        if isinstance(self.router_w, QWeight):
            w.router_w = self.router_w.w.data_ptr()
            w.router_scales = self.router_w.scales.data_ptr()
            w.router_biases = self.router_w.biases.data_ptr()
        else:
            w.router_w = self.router_w.data_ptr()
        w.router_logit_bias = _ptr(self.router_logit_bias)
        for name in ("gate", "up", "down", "shared_gate", "shared_up", "shared_down"):
            q = getattr(self, name)
            if q is not None:
                setattr(w, name, q.to_c())
        g = self.shared_expert_gate_w
        if isinstance(g, QWeight):
            w.shared_expert_gate_w = g.w.data_ptr()
            w.shared_expert_gate_scales = g.scales.data_ptr()
            w.shared_expert_gate_biases = g.biases.data_ptr()
        elif g is not None:
            w.shared_expert_gate_w = g.data_ptr()
        if self.packed is not None:
            w.packed = self.packed.data_ptr()
            w.packed_bytes = self.packed.numel()
        return w

    def pack(self, cfg: "MoEConfig") -> None:
        """fmx_pack_expert_weights: the load-time re-layout that every forward
        then reads in place of the MLX-layout expert arrays."""
        lib = _lib.load()
        c = cfg.to_c()
        nbytes = lib.fmx_moe_packed_size(C.byref(c))
        if nbytes == 0:
            raise _lib.FmxError(_lib.FMX_ERR_UNSUPPORTED, "config cannot be packed")
        self.packed = None
        buf = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        w = self.to_c()
        _lib.check(lib.fmx_pack_expert_weights(C.byref(c), C.byref(w), buf.data_ptr(), nbytes,
                                               _stream()))
        self.packed = buf

    def drop_mlx_layout(self) -> None:
        """Releases the MLX-layout expert arrays once packed (the layer then
        holds its expert weights once)."""
        if self.packed is None:
            raise ValueError("pack() first: the MLX-layout arrays are the only copy")
        torch.cuda.current_stream().synchronize()  # the pack kernels have read them
        self.gate = self.up = self.down = None
        self.shared_gate = self.shared_up = self.shared_down = None


class MoEBlock:
    """LlamaModel::moe_block (server/src/model.cpp:750-807) on libfmx.

    Holds a device workspace for up to `max_tokens` tokens; calls on one
    MoEBlock must be ordered on one stream.
    """

    def __init__(self, cfg: MoEConfig, weights: MoEWeights, max_tokens: int = 1024,
                 device: Optional[torch.device] = None, pack: bool = True):
        self.lib = _lib.load()
        self.cfg = cfg
        self.weights = weights
        if pack and weights.packed is None and self.lib.fmx_moe_packed_size(C.byref(cfg.to_c())):
            weights.pack(cfg)
        self._c_cfg = cfg.to_c()
        self._c_w = weights.to_c()
        self.max_tokens = max_tokens
        self.ws_bytes = self.lib.fmx_moe_workspace_size(C.byref(self._c_cfg), max_tokens)
        if self.ws_bytes == 0:
            raise _lib.FmxError(_lib.FMX_ERR_ARG, "invalid MoE config or max_tokens")
        dev = device or weights.device
        self.workspace = torch.empty(self.ws_bytes, dtype=torch.uint8, device=dev)
        _lib.check(self.lib.fmx_moe_workspace_init(self.workspace.data_ptr(), self.ws_bytes, _stream()))
        self._last_T = 0

    def refresh(self) -> None:
        """Re-reads the weights' device pointers (after the weights changed,
        e.g. drop_mlx_layout)."""
        self._c_w = self.weights.to_c()

    def weight_tensors(self) -> list:
        """Every device tensor of the layer's weights (MLX layout and packed)."""
        w = self.weights
        ts = []
        for q in (w.router_w, w.gate, w.up, w.down, w.shared_gate, w.shared_up, w.shared_down,
                  w.shared_expert_gate_w, w.router_logit_bias, w.packed):
            if isinstance(q, QWeight):
                ts += q.tensors()
            elif q is not None:
                ts.append(q)
        return ts

    def forward_into(self, x: torch.Tensor, y: torch.Tensor) -> None:
        """y[T, H] = moe_block(x[T, H]) without allocating (graph-capturable)."""
        T = x.numel() // self.cfg.hidden_size
        _lib.check(self.lib.fmx_moe_block_forward(
            C.byref(self._c_cfg), C.byref(self._c_w), x.data_ptr(), T, y.data_ptr(),
            self.workspace.data_ptr(), self.ws_bytes, _stream()))
        self._last_T = T

    def forward_partial(self, x: torch.Tensor, y: torch.Tensor, n_stages: int) -> None:
        """forward_into that launches only the first n_stages (1..4) kernel
        stages: router, gate/up, down, combine (for per-stage timing)."""
        T = x.numel() // self.cfg.hidden_size
        _lib.check(self.lib.fmx_moe_block_forward_partial(
            C.byref(self._c_cfg), C.byref(self._c_w), x.data_ptr(), T, y.data_ptr(),
            self.workspace.data_ptr(), self.ws_bytes, _stream(), n_stages))
        self._last_T = T

    def forward_profiled(self, x: torch.Tensor, y: torch.Tensor, events) -> None:
        """forward_into that records 5 torch.cuda.Events at the stage
        boundaries (before the first kernel and after each of the four
        kernel stages)."""
        T = x.numel() // self.cfg.hidden_size
        for ev in events:  # torch creates an event's HIP handle at its first record
            if not ev.cuda_event:
                ev.record()
        arr = (C.c_void_p * 5)(*[ev.cuda_event for ev in events])
        _lib.check(self.lib.fmx_moe_block_forward_profiled(
            C.byref(self._c_cfg), C.byref(self._c_w), x.data_ptr(), T, y.data_ptr(),
            self.workspace.data_ptr(), self.ws_bytes, _stream(), arr))
        self._last_T = T

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if x.dtype != self.cfg.activation_dtype or not x.is_contiguous():
            raise ValueError(f"x must be a contiguous {self.cfg.activation_dtype} tensor [..., H]")
        y = torch.empty_like(x)
        self.forward_into(x, y)
        return y

    def status(self, clear: bool = False) -> int:
        """The workspace's status word after the queued forwards end (0, or
        _lib.FMX_STATUS_WAIT_TIMEOUT when a decode forward's bounded wait
        ran out and its products were written as NaN); clear resets it."""
        st = C.c_uint32()
        _lib.check(self.lib.fmx_moe_workspace_status(self.workspace.data_ptr(), self.ws_bytes,
                                                     C.byref(st), int(clear), _stream()))
        return st.value

    def routing(self) -> dict:
        """Views of the last forward's routing state inside the workspace."""
        T = self._last_T
        ptrs = [C.c_void_p() for _ in range(8)]
        _lib.check(self.lib.fmx_moe_workspace_routing(
            C.byref(self._c_cfg), T, self.workspace.data_ptr(), *[C.byref(p) for p in ptrs]))
        base = self.workspace.data_ptr()
        k, E = self.cfg.num_experts_per_tok, self.cfg.num_experts

        def view(p, n, dt, esz):
            off = p.value - base
            return self.workspace[off: off + n * esz].view(dt)

        return {
            "inds": view(ptrs[0], T * k, torch.int32, 4).view(T, k),
            "scores": view(ptrs[1], T * k, self.cfg.activation_dtype, 2).view(T, k),
            "probs": view(ptrs[2], T * E, self.cfg.activation_dtype, 2).view(T, E),
            "order": view(ptrs[3], T * k, torch.int32, 4),
            "inv": view(ptrs[4], T * k, torch.int32, 4),
            "src": view(ptrs[5], T * k, torch.int32, 4),
            "idx": view(ptrs[6], T * k, torch.int32, 4),
            "expert_offsets": view(ptrs[7], E + 1, torch.int32, 4),
        }


def router_topk(cfg: MoEConfig, x: torch.Tensor, router_w,
                logit_bias: Optional[torch.Tensor] = None, shared_expert_gate_w=None):
    """Router alone (model.cpp:757-775): (inds [T,k] int32, scores [T,k]
    bf16, probs [T,E] bf16), and with `shared_expert_gate_w` also the shared
    expert's gate sigmoid(x . wsg^T) [T] bf16 (:787-803). router_w and
    shared_expert_gate_w are bf16 tensors or QWeights (the quantized router
    of :758-760). With cfg.activation_dtype float16, every bf16 here is
    float16."""
    if isinstance(router_w, QWeight) or shared_expert_gate_w is not None:
        return _router_topk_ex(cfg, x, router_w, logit_bias, shared_expert_gate_w)
    lib = _lib.load()
    c = cfg.to_c()
    T = x.numel() // cfg.hidden_size
    k, E = cfg.num_experts_per_tok, cfg.num_experts
    inds = torch.empty(T, k, dtype=torch.int32, device=x.device)
    scores = torch.empty(T, k, dtype=cfg.activation_dtype, device=x.device)
    probs = torch.empty(T, E, dtype=cfg.activation_dtype, device=x.device)
    _lib.check(lib.fmx_moe_router_topk(
        C.byref(c), x.data_ptr(), T, router_w.data_ptr(),
        logit_bias.data_ptr() if logit_bias is not None else None,
        inds.data_ptr(), scores.data_ptr(), probs.data_ptr(), None, 0, _stream()))
    return inds, scores, probs


def _router_topk_ex(cfg: MoEConfig, x: torch.Tensor, router_w, logit_bias, shared_expert_gate_w):
    lib = _lib.load()
    c = cfg.to_c()
    T = x.numel() // cfg.hidden_size
    k, E = cfg.num_experts_per_tok, cfg.num_experts
    w = MoEWeights(router_w=router_w, gate=None, up=None, down=None,
                   shared_expert_gate_w=shared_expert_gate_w, router_logit_bias=logit_bias)
    cw = w.to_c()
    inds = torch.empty(T, k, dtype=torch.int32, device=x.device)
    scores = torch.empty(T, k, dtype=cfg.activation_dtype, device=x.device)
    probs = torch.empty(T, E, dtype=cfg.activation_dtype, device=x.device)
    sg = torch.empty(T, dtype=cfg.activation_dtype, device=x.device) if shared_expert_gate_w is not None else None
    _lib.check(lib.fmx_moe_router_topk_ex(
        C.byref(c), x.data_ptr(), T, C.byref(cw), inds.data_ptr(), scores.data_ptr(), probs.data_ptr(),
        _ptr(sg), None, 0, _stream()))
    return (inds, scores, probs) if sg is None else (inds, scores, probs, sg)
