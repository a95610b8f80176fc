"""MoE-layer workloads: model shapes, token counts, seeds, synthetic inputs.

Shapes follow the two MoE families the reference serves through
LlamaModel::moe_block (server/src/model.cpp:750-807; config fields
server/include/flashmlx/model.h:40-53):
  Qwen1.5-MoE-A2.7B: H 2048, 60 experts, top-4, I 1408, shared expert 5632
                     with a sigmoid gate, no top-k renormalisation;
  Qwen3-30B-A3B:     H 2048, 128 experts, top-8, I 768, no shared expert,
                     renormalised top-k scores.
Inputs are drawn from fmx_synth_normal_bf16 (one counter-based stream per
tensor), so every byte is a pure function of (seed, tensor, index).
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass, field
from typing import Dict, Optional

import numpy as np

QWEN15 = dict(name="qwen1.5-moe-a2.7b", hidden=2048, n_experts=60, top_k=4, inter=1408,
              shared_inter=5632, norm_topk=False)
QWEN3 = dict(name="qwen3-30b-a3b", hidden=2048, n_experts=128, top_k=8, inter=768,
             shared_inter=0, norm_topk=True)
# small shapes with the same structure, for tests that the CPU oracle must finish fast
TINY = dict(name="tiny", hidden=256, n_experts=8, top_k=2, inter=128, shared_inter=192,
            norm_topk=False)
TINY_NORM = dict(name="tiny-norm", hidden=320, n_experts=12, top_k=3, inter=192, shared_inter=0,
                 norm_topk=True)
# small shapes that the packed-weight kernels take (every K a multiple of 128);
# H = 384 leaves the down projection's last column group part-filled
SMALL = dict(name="small", hidden=384, n_experts=6, top_k=2, inter=256, shared_inter=256,
             norm_topk=False)
# the smallest shapes that the packed-weight decode kernels take (H a multiple
# of 512, the shared expert's down projection split four ways)
SMALL_DEC = dict(name="small-dec", hidden=512, n_experts=8, top_k=2, inter=256, shared_inter=512,
                 norm_topk=False)

# synth stream ids, one per tensor
S_X, S_ROUTER, S_RBIAS = 1, 2, 3
S_GATE, S_UP, S_DOWN = 10, 11, 12
S_SH_GATE, S_SH_UP, S_SH_DOWN, S_SH_EGATE = 20, 21, 22, 23

W_STD = 0.02


@dataclass(frozen=True)
class Workload:
    key: str
    model: dict
    tokens: int
    seed: int
    router_bias: bool = False
    note: str = ""
    # router and shared-expert gate quantized (affine 4-bit, group 64) like
    # every other linear, as in a checkpoint that quantizes them
    router_quant: bool = False


WORKLOADS: Dict[str, Workload] = {w.key: w for w in [
    Workload("qwen15_decode_b1", QWEN15, 1, 0, note="decode batch 1"),
    Workload("qwen15_decode_b4", QWEN15, 4, 1, note="decode batch 4"),
    Workload("qwen15_decode_b8", QWEN15, 8, 2, note="decode batch 8"),
    Workload("qwen15_prefill_512", QWEN15, 512, 3, router_bias=True,
             note="prefill 512 tokens, per-expert router logit bias ~ N(0,1)"),
    Workload("qwen3_decode_b1", QWEN3, 1, 4, note="decode batch 1"),
    Workload("qwen3_decode_b8", QWEN3, 8, 4, note="decode batch 8"),
    Workload("qwen15_decode_b16", QWEN15, 16, 6, router_bias=True,
             note="decode batch 16 (the largest decode batch), per-expert router logit bias ~ N(0,1)"),
    Workload("qwen3_decode_b16", QWEN3, 16, 7, note="decode batch 16 (up to 128 routed experts)"),
    Workload("qwen3_prefill_1024", QWEN3, 1024, 4, note="prefill 1024 tokens"),
    Workload("tiny_t5", TINY, 5, 11, note="tiny shapes, 5 tokens"),
    Workload("tiny_t40", TINY, 40, 12, router_bias=True, note="tiny shapes, 40 tokens, skewed"),
    Workload("tiny_norm_t33", TINY_NORM, 33, 13, note="tiny shapes, renormalised top-3"),
    Workload("small_t23", SMALL, 23, 14, router_bias=True,
             note="packable small shapes, 23 tokens (one pass per expert)"),
    Workload("small_t200", SMALL, 200, 15,
             note="packable small shapes, 200 tokens (experts over several passes)"),
    Workload("small_dec_t4", SMALL_DEC, 4, 16, note="small shapes on the decode kernels, 4 tokens"),
    Workload("qwen15_decode_b4_qrouter", QWEN15, 4, 21, router_quant=True,
             note="decode batch 4, quantized router and shared-expert gate"),
    Workload("small_t200_qrouter", SMALL, 200, 22, router_quant=True, router_bias=True,
             note="packable small shapes, 200 tokens, quantized router and shared-expert gate"),
]}


def _synth(n: int, seed: int, stream: int, std: float) -> np.ndarray:
    from .moe import synth_normal_bf16
    return synth_normal_bf16(n, seed, stream, 0.0, std)


@dataclass
class HostInputs:
    """bf16 bit patterns (uint16) of every input of one MoE-layer call."""
    x: np.ndarray                      # [T, H]
    router_w: np.ndarray               # [E, H]
    router_bias: Optional[np.ndarray]  # [E]
    gate: np.ndarray                   # [E, I, H]
    up: np.ndarray                     # [E, I, H]
    down: np.ndarray                   # [E, H, I]
    shared_gate: Optional[np.ndarray] = None   # [Is, H]
    shared_up: Optional[np.ndarray] = None     # [Is, H]
    shared_down: Optional[np.ndarray] = None   # [H, Is]
    shared_expert_gate_w: Optional[np.ndarray] = None  # [1, H]
    meta: dict = field(default_factory=dict)

    def sha256(self) -> str:
        h = hashlib.sha256()
        for name in ("x", "router_w", "router_bias", "gate", "up", "down", "shared_gate",
                     "shared_up", "shared_down", "shared_expert_gate_w"):
            a = getattr(self, name)
            if a is not None:
                h.update(name.encode())
                h.update(np.ascontiguousarray(a).tobytes())
        return h.hexdigest()


def host_inputs(wl: Workload, tokens: Optional[int] = None) -> HostInputs:
    m = wl.model
    T = wl.tokens if tokens is None else tokens
    H, E, I, Is = m["hidden"], m["n_experts"], m["inter"], m["shared_inter"]
    s = wl.seed
    hi = HostInputs(
        x=_synth(T * H, s, S_X, 1.0).reshape(T, H),
        router_w=_synth(E * H, s, S_ROUTER, W_STD).reshape(E, H),
        router_bias=_synth(E, s, S_RBIAS, 1.0) if wl.router_bias else None,
        gate=_synth(E * I * H, s, S_GATE, W_STD).reshape(E, I, H),
        up=_synth(E * I * H, s, S_UP, W_STD).reshape(E, I, H),
        down=_synth(E * H * I, s, S_DOWN, W_STD).reshape(E, H, I),
    )
    if Is:
        hi.shared_gate = _synth(Is * H, s, S_SH_GATE, W_STD).reshape(Is, H)
        hi.shared_up = _synth(Is * H, s, S_SH_UP, W_STD).reshape(Is, H)
        hi.shared_down = _synth(H * Is, s, S_SH_DOWN, W_STD).reshape(H, Is)
        hi.shared_expert_gate_w = _synth(H, s, S_SH_EGATE, W_STD).reshape(1, H)
    hi.meta = dict(workload=wl.key, model=m["name"], tokens=T, seed=s)
    return hi


# ------------------------------------------------------------------ device side

class DeviceSynth:
    """The tensors of HostInputs generated straight into device memory
    (fmx_synth_normal_bf16_device: the same values), for weight sets too
    large to build on the host."""

    def __init__(self, wl: Workload, device="cuda"):
        self.wl, self.device = wl, device

    def tensor(self, name: str):
        from .moe import synth_normal_bf16_device
        m, s, T = self.wl.model, self.wl.seed, self.wl.tokens
        H, E, I, Is = m["hidden"], m["n_experts"], m["inter"], m["shared_inter"]
        spec = dict(x=((T, H), S_X, 1.0), router_w=((E, H), S_ROUTER, W_STD),
                    router_bias=((E,), S_RBIAS, 1.0), gate=((E, I, H), S_GATE, W_STD),
                    up=((E, I, H), S_UP, W_STD), down=((E, H, I), S_DOWN, W_STD),
                    shared_gate=((Is, H), S_SH_GATE, W_STD), shared_up=((Is, H), S_SH_UP, W_STD),
                    shared_down=((H, Is), S_SH_DOWN, W_STD),
                    shared_expert_gate_w=((1, H), S_SH_EGATE, W_STD))[name]
        return synth_normal_bf16_device(spec[0], s, spec[1], 0.0, spec[2], self.device)

    def __getattr__(self, name):
        if name == "router_bias" and not self.wl.router_bias:
            return None
        if name.startswith("shared") and not self.wl.model["shared_inter"]:
            return None
        if name in ("x", "router_w", "router_bias", "gate", "up", "down", "shared_gate", "shared_up",
                    "shared_down", "shared_expert_gate_w"):
            return self.tensor(name)
        raise AttributeError(name)


def device_block(wl: Workload, hi, max_tokens: Optional[int] = None, device="cuda",
                 pack: bool = True, drop_mlx: bool = False):
    """Uploads the inputs (HostInputs, or DeviceSynth to generate them on the
    device), quantizes the weights on the GPU (fmx_quantize), packs them
    (fmx_pack_expert_weights) unless pack=False, and returns (MoEBlock,
    x_device). drop_mlx: release the MLX-layout expert arrays after packing
    (forwards read only the packed copy)."""
    import torch

    from .moe import MoEBlock, MoEConfig, MoEWeights, QWeight, quantize

    m = wl.model

    def up(a):
        if isinstance(a, torch.Tensor):
            return a
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(device).view(torch.bfloat16)

    def q(a):
        t = up(a)
        wq, s, b = quantize(t)
        del t
        return QWeight(wq, s, b)

    cfg = MoEConfig(hidden_size=m["hidden"], num_experts=m["n_experts"],
                    num_experts_per_tok=m["top_k"], moe_intermediate_size=m["inter"],
                    shared_expert_intermediate_size=m["shared_inter"],
                    norm_topk_prob=m["norm_topk"])
    rq = q if wl.router_quant else up
    w = MoEWeights(router_w=rq(hi.router_w), gate=q(hi.gate), up=q(hi.up), down=q(hi.down))
    if hi.router_bias is not None:
        w.router_logit_bias = up(hi.router_bias)
    if m["shared_inter"]:
        w.shared_gate, w.shared_up, w.shared_down = q(hi.shared_gate), q(hi.shared_up), q(hi.shared_down)
        w.shared_expert_gate_w = rq(hi.shared_expert_gate_w)
    block = MoEBlock(cfg, w, max_tokens=max_tokens or wl.tokens, pack=pack)
    if drop_mlx:
        w.drop_mlx_layout()
        block.refresh()
    return block, up(hi.x)


def algorithmic_bytes(m: dict, tokens: int, unique_experts: int, router_bias: bool = False,
                      router_quant: bool = False) -> int:
    """HBM bytes one MoE-layer call must move at minimum: the packed weights
    of every routed (unique) expert, the shared expert, the bf16 router and
    shared-gate rows, and the bf16 activations in and out."""
    H, E, I, Is = m["hidden"], m["n_experts"], m["inter"], m["shared_inter"]
    per_w = lambda n, k: n * k // 2 + 2 * 2 * n * (k // 64)  # noqa: E731
    expert = 2 * per_w(I, H) + per_w(H, I)
    shared = (2 * per_w(Is, H) + per_w(H, Is)) if Is else 0
    router = E * H * 2 + (E * 2 if router_bias else 0)
    sgate = H * 2 if Is else 0
    if router_quant:
        router = per_w(E, H) + (E * 2 if router_bias else 0)
        sgate = per_w(1, H) if Is else 0
    act = 2 * tokens * H * 2
    return unique_experts * expert + shared + router + sgate + act


def flops(m: dict, tokens: int) -> int:
    """Useful FLOPs of one call: routed experts (k per token), shared expert,
    router and shared-gate dot products."""
    H, E, I, Is, k = m["hidden"], m["n_experts"], m["inter"], m["shared_inter"], m["top_k"]
    f = 2 * tokens * k * 3 * H * I + 2 * tokens * H * E
    if Is:
        f += 2 * tokens * 3 * H * Is + 2 * tokens * H
    return f


def packed_bytes(n: int, k: int) -> int:
    """Bytes of an [n, k] weight at 4 bits per weight with a bf16 scale and
    bias per 64-group (0.5625 B per weight)."""
    return n * k // 2 + 2 * 2 * n * (k // 64)


def forward_path(m: dict, tokens: int, packed: bool = True) -> str:
    """The kernels fmx_moe_block_forward runs for this shape: "decode",
    "prefill" (packed-weight GEMMs) or "general" (asks the library:
    fmx_moe_forward_path)."""
    import ctypes as C

    from . import _lib
    from ._lib import FmxMoEConfig

    c = FmxMoEConfig()
    c.hidden_size, c.num_experts = m["hidden"], m["n_experts"]
    c.num_experts_per_tok, c.norm_topk_prob = m["top_k"], int(bool(m["norm_topk"]))
    c.moe_intermediate_size, c.shared_expert_intermediate_size = m["inter"], m["shared_inter"]
    c.quant_bits, c.quant_group_size = 4, 64
    r = _lib.load().fmx_moe_forward_path(C.byref(c), tokens, int(packed))
    if r < 0:
        _lib.check(-r)
    return {0: "general", 1: "decode", 2: "prefill"}[r]


def decode_path(m: dict, tokens: int, packed: bool = True) -> bool:
    """Whether fmx_moe_block_forward runs the decode kernels for this shape."""
    return forward_path(m, tokens, packed) == "decode"


def kernel_groups(m: dict, tokens: int, packed: bool = True) -> list:
    """The kernels of a whole forward as [(name, [stage indices of
    stage_work])]: on the decode path gate/up, down and combine run as one
    grid, so its time in the layer is the marginal time of those stages
    together; elsewhere each stage is its own kernel group."""
    if decode_path(m, tokens, packed):
        return [("router+shared_gate_up", [0]), ("gate_up+down+combine", [1, 2])]
    return [("router+sort", [0]), ("gate_up", [1]), ("down", [2]), ("combine", [3])]


def stage_work(m: dict, tokens: int, unique_experts: int, router_bias: bool = False,
               packed: bool = True, router_quant: bool = False) -> list:
    """Algorithmic work of each kernel stage of one MoE-layer call, in launch
    order: [(name, hbm_bytes, flops)]. Bytes are the weights the stage must
    read plus the activations it must read and write in HBM (the smallest
    traffic the stage's kernel can have); flops count the useful MACs x 2."""
    H, E, I, Is, k = m["hidden"], m["n_experts"], m["inter"], m["shared_inter"], m["top_k"]
    T, U = tokens, unique_experts
    pw = packed_bytes
    if router_quant:
        router_b = pw(E, H) + (E * 2 if router_bias else 0) + (pw(1, H) if Is else 0)
    else:
        router_b = E * H * 2 + (E * 2 if router_bias else 0) + (H * 2 if Is else 0)
    router_f = 2 * T * H * (E + (1 if Is else 0))
    x_b = T * H * 2
    h_b = T * k * I * 2
    hs_b = T * Is * 2
    d_b = T * k * H * 2
    sd_b = 4 * T * H * 4 if Is else 0
    y_b = T * H * 2
    gu_f = 2 * T * k * 2 * H * I
    sgu_f = 2 * T * 2 * H * Is
    dn_f = 2 * T * k * H * I
    sdn_f = 2 * T * H * Is
    if decode_path(m, T, packed):
        return [
            ("router+shared_gate_up", router_b + 2 * pw(Is, H) + x_b + T * (E + 1) * 2 + hs_b,
             router_f + sgu_f),
            ("gate_up", U * 2 * pw(I, H) + x_b + h_b, gu_f),
            ("down+combine", U * pw(H, I) + (pw(H, Is) if Is else 0) + h_b + hs_b + y_b, dn_f + sdn_f),
        ]
    return [
        ("router+sort", router_b + x_b + x_b, router_f),
        ("gate_up", U * 2 * pw(I, H) + 2 * pw(Is, H) + x_b + h_b + hs_b, gu_f + sgu_f),
        ("down", U * pw(H, I) + (pw(H, Is) if Is else 0) + h_b + hs_b + d_b + sd_b, dn_f + sdn_f),
        ("combine", d_b + sd_b + y_b, 0),
    ]
