"""NemotronHModel::moe_block (server/src/nemotron_h.cpp:1010-1111) on libfmx:
the sigmoid router with its correction bias and group limit, fc1 -> relu^2
-> fc2 over the selected experts, and the shared expert, in the HIP kernels
of libfmx.so (include/fmx_nemotron.h). torch tensors only carry device
memory and the current stream."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import _lib
from .moe import QWeight, quantize, synth_normal_bf16_device


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


@dataclass
class NhMoEConfig:
    """ModelConfig's Nemotron-H MoE fields (nemotron_h.cpp:245-258); the
    defaults are the shape of the 30B-A3B model's MoE layers."""
    hidden_size: int = 2688
    n_routed_experts: int = 128
    num_experts_per_tok: int = 6
    moe_intermediate_size: int = 1856
    moe_shared_expert_intermediate_size: int = 3712
    norm_topk_prob: bool = True
    n_group: int = 1
    topk_group: int = 1
    routed_scaling_factor: float = 2.5
    quant_bits: int = 4
    quant_group_size: int = 64

    def to_c(self) -> _lib.FmxNhMoEConfig:
        c = _lib.FmxNhMoEConfig()
        c.hidden_size = self.hidden_size
        c.n_routed_experts = self.n_routed_experts
        c.num_experts_per_tok = self.num_experts_per_tok
        c.norm_topk_prob = int(bool(self.norm_topk_prob))
        c.moe_intermediate_size = self.moe_intermediate_size
        c.moe_shared_expert_intermediate_size = self.moe_shared_expert_intermediate_size
        c.n_group = self.n_group
        c.topk_group = self.topk_group
        c.routed_scaling_factor = self.routed_scaling_factor
        c.quant_bits = self.quant_bits
        c.quant_group_size = self.quant_group_size
        return c

    def oracle_cfg(self) -> dict:
        return dict(hidden=self.hidden_size, n_experts=self.n_routed_experts,
                    top_k=self.num_experts_per_tok, norm_topk=self.norm_topk_prob,
                    inter=self.moe_intermediate_size,
                    shared_inter=self.moe_shared_expert_intermediate_size, n_group=self.n_group,
                    topk_group=self.topk_group, scaling=self.routed_scaling_factor)


@dataclass
class NhMoEWeights:
    """MoELayerWeights (nemotron_h.cpp:443-470). After pack(), the MLX-layout
    expert arrays may be dropped: forwards read only the packed copy."""
    gate_w: torch.Tensor                          # bf16 [E, H]
    correction_bias: Optional[torch.Tensor]       # fp32 [E] or None
    fc1: Optional[QWeight]                        # [E, I, H/8] ...
    fc2: Optional[QWeight]                        # [E, H, I/8] ...
    shared_up: Optional[QWeight] = None           # [Is, H/8] ...
    shared_down: Optional[QWeight] = None         # [H, Is/8] ...
    packed: Optional[torch.Tensor] = None

    def to_c(self) -> _lib.FmxNhMoEWeights:
        w = _lib.FmxNhMoEWeights()
        w.gate_w = self.gate_w.data_ptr()
        w.correction_bias = self.correction_bias.data_ptr() if self.correction_bias is not None else None
        for name in ("fc1", "fc2", "shared_up", "shared_down"):
            q = getattr(self, name)
            if q is not None:
                setattr(w, name, q.to_c())
        if self.packed is not None:
            w.packed = self.packed.data_ptr()
            w.packed_bytes = self.packed.numel()
        return w

    def pack(self, cfg: NhMoEConfig) -> None:
        """fmx_nh_pack_expert_weights (I and Is padded to 128 with zeros)."""
        lib = _lib.load()
        c = cfg.to_c()
        nbytes = lib.fmx_nh_moe_packed_size(C.byref(c))
        if nbytes == 0:
            raise _lib.FmxError(_lib.FMX_ERR_UNSUPPORTED, "config cannot be packed")
        self.packed = None
        buf = torch.empty(nbytes, dtype=torch.uint8, device=self.gate_w.device)
        w = self.to_c()
        _lib.check(lib.fmx_nh_pack_expert_weights(C.byref(c), C.byref(w), buf.data_ptr(), nbytes,
                                                  _stream()))
        self.packed = buf

    def drop_mlx_layout(self) -> None:
        if self.packed is None:
            raise ValueError("pack() first: the MLX-layout arrays are the only copy")
        torch.cuda.current_stream().synchronize()
        self.fc1 = self.fc2 = self.shared_up = self.shared_down = None


class NhMoEBlock:
    """NemotronHModel::moe_block on libfmx, with a workspace for up to
    `max_tokens` tokens; calls on one block are ordered on one stream."""

    def __init__(self, cfg: NhMoEConfig, weights: NhMoEWeights, max_tokens: int = 1024):
        self.lib = _lib.load()
        self.cfg, self.weights = cfg, weights
        if weights.packed is None:
            weights.pack(cfg)
        self._c_cfg = cfg.to_c()
        self._c_w = weights.to_c()
        ws = self.lib.fmx_nh_moe_workspace_size(C.byref(self._c_cfg), max_tokens)
        if ws == 0:
            _lib.check(_lib.FMX_ERR_ARG)
        self.workspace = torch.empty(ws, dtype=torch.uint8, device=weights.gate_w.device)
        _lib.check(self.lib.fmx_nh_moe_workspace_init(self.workspace.data_ptr(), ws, _stream()))
        self.max_tokens = max_tokens
        self._last_T = 0

    def forward_into(self, x: torch.Tensor, y: torch.Tensor) -> None:
        T = x.numel() // self.cfg.hidden_size
        if T > self.max_tokens:
            raise ValueError(f"{T} tokens > max_tokens {self.max_tokens}")
        _lib.check(self.lib.fmx_nh_moe_block_forward(
            C.byref(self._c_cfg), C.byref(self._c_w), x.data_ptr(), T, y.data_ptr(),
            self.workspace.data_ptr(), self.workspace.numel(), _stream()))
        self._last_T = T

    def forward_partial(self, x: torch.Tensor, y: torch.Tensor, n_stages: int) -> None:
        """forward_into that launches only the first n_stages (1..4) kernel
        stages: router + sort, fc1, fc2, combine (for per-stage timing)."""
        T = x.numel() // self.cfg.hidden_size
        if T > self.max_tokens:
            raise ValueError(f"{T} tokens > max_tokens {self.max_tokens}")
        _lib.check(self.lib.fmx_nh_moe_block_forward_partial(
            C.byref(self._c_cfg), C.byref(self._c_w), x.data_ptr(), T, y.data_ptr(),
            self.workspace.data_ptr(), self.workspace.numel(), _stream(), n_stages))
        self._last_T = T

    def forward_profiled(self, x: torch.Tensor, y: torch.Tensor, events) -> None:
        """forward_into recording 5 torch.cuda.Events at the stage
        boundaries (router+sort, fc1, fc2, combine)."""
        T = x.numel() // self.cfg.hidden_size
        for e in events:  # torch creates an event's HIP handle at its first record
            if not e.cuda_event:
                e.record()
        arr = (C.c_void_p * 5)(*[e.cuda_event for e in events])
        _lib.check(self.lib.fmx_nh_moe_block_forward_profiled(
            C.byref(self._c_cfg), C.byref(self._c_w), x.data_ptr(), T, y.data_ptr(),
            self.workspace.data_ptr(), self.workspace.numel(), _stream(), arr))
        self._last_T = T

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if x.dtype != torch.bfloat16 or not x.is_contiguous():
            raise ValueError("x must be a contiguous bf16 tensor [..., H]")
        y = torch.empty_like(x)
        self.forward_into(x, y)
        return y

    def routing(self) -> dict:
        """Views of the last forward's routing: inds [T, k] int32, scores
        [T, k] fp32, logits [T, E] bf16."""
        T, k, E = self._last_T, self.cfg.num_experts_per_tok, self.cfg.n_routed_experts
        ptrs = [C.c_void_p() for _ in range(3)]
        _lib.check(self.lib.fmx_nh_moe_workspace_routing(
            C.byref(self._c_cfg), T, self.workspace.data_ptr(), *[C.byref(p) for p in ptrs]))
        base = self.workspace.data_ptr()

        def view(p, n, dt, esz):
            off = p.value - base
            return self.workspace[off: off + n * esz].view(dt)

        return {
            "inds": view(ptrs[0], T * k, torch.int32, 4).view(T, k),
            "scores": view(ptrs[1], T * k, torch.float32, 4).view(T, k),
            "logits": view(ptrs[2], T * (E + 1), torch.bfloat16, 2).view(T, E + 1)[:, :E],
        }


# synth stream ids of the Nemotron-H weights
S_GATE, S_CBIAS, S_FC1, S_FC2, S_SH_UP, S_SH_DOWN = 40, 41, 42, 43, 44, 45


def synthetic_nh_weights(cfg: NhMoEConfig, seed: int, device="cuda", cbias_std: float = 0.05,
                         w_std: float = 0.02) -> NhMoEWeights:
    """Random-init weights of the config's shape, generated on the device:
    the router bf16 ~ N(0, w_std), the correction bias fp32 ~ N(0, cbias_std)
    (None when cbias_std is 0), fc1/fc2/shared ~ N(0, w_std) quantized affine
    4-bit g64 (MLX layout; pack() makes the packed copy)."""
    H, E, I, Is = (cfg.hidden_size, cfg.n_routed_experts, cfg.moe_intermediate_size,
                   cfg.moe_shared_expert_intermediate_size)

    def g(shape, stream, std=w_std):
        return synth_normal_bf16_device(shape, seed, stream, 0.0, std, device)

    def q(shape, stream):
        return QWeight(*quantize(g(shape, stream)))

    cb = g((E,), S_CBIAS, cbias_std).float() if cbias_std > 0 else None
    w = NhMoEWeights(gate_w=g((E, H), S_GATE), correction_bias=cb, fc1=q((E, I, H), S_FC1),
                     fc2=q((E, H, I), S_FC2))
    if Is:
        w.shared_up = q((Is, H), S_SH_UP)
        w.shared_down = q((H, Is), S_SH_DOWN)
    return w


def host_weights(w: NhMoEWeights) -> dict:
    """The weights as numpy arrays for the CPU oracle (oracle.nh_moe_block)."""
    def u16(t):
        return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    def qt(qw):
        return (qw.w.contiguous().cpu().numpy().view(np.uint32), u16(qw.scales), u16(qw.biases))

    out = dict(gate_w=u16(w.gate_w), fc1=qt(w.fc1), fc2=qt(w.fc2))
    out["cbias"] = None if w.correction_bias is None else w.correction_bias.cpu().numpy()
    if w.shared_up is not None:
        out["shared_up"], out["shared_down"] = qt(w.shared_up), qt(w.shared_down)
    return out
