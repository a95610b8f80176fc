"""The decoder stack around the MoE block (LlamaModel::forward for all-MoE
models, server/src/model.cpp:1021-1033) on libfmx.

`DecoderModel` holds the packed weights, a KV cache and a workspace and runs
fmx_model_forward: embedding, per layer RMSNorm -> attention (q/k/v with
biases, RoPE, cache, SDPA, o_proj) -> residual -> RMSNorm -> MoE block ->
residual, final RMSNorm, lm_head. `synthetic_model` builds random-init
4-bit weights of a given shape on the device (the Qwen1.5-MoE-A2.7B shape by
default), quantized with fmx_quantize and packed once.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import List, Optional

import torch

from . import _lib
from .moe import MoEConfig, MoEWeights, QWeight, dequantize, quantize, synth_normal_bf16_device


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


@dataclass
class ModelConfig:
    """ModelConfig (server/include/flashmlx/model.h:20-54) of an all-MoE
    decoder. Defaults: the Qwen1.5-MoE-A2.7B shape (hidden 2048, 24 layers,
    16 heads of 128, vocab 151936, rms_norm_eps 1e-6, rope_theta 1e6; its
    MoE block: 60 experts, top-4, I 1408, shared expert 5632)."""
    hidden_size: int = 2048
    num_hidden_layers: int = 24
    num_attention_heads: int = 16
    num_key_value_heads: int = 16
    head_dim: int = 0
    vocab_size: int = 151936
    max_position_embeddings: int = 4096
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    moe: MoEConfig = field(default_factory=lambda: MoEConfig(
        hidden_size=2048, num_experts=60, num_experts_per_tok=4, moe_intermediate_size=1408,
        shared_expert_intermediate_size=5632, norm_topk_prob=False))

    @property
    def hd(self) -> int:
        return self.head_dim or self.hidden_size // self.num_attention_heads

    @property
    def n_qkv(self) -> int:
        return (self.num_attention_heads + 2 * self.num_key_value_heads) * self.hd

    def to_c(self) -> _lib.FmxModelConfig:
        c = _lib.FmxModelConfig()
        for f in ("hidden_size", "num_hidden_layers", "num_attention_heads", "num_key_value_heads",
                  "head_dim", "vocab_size", "max_position_embeddings", "rms_norm_eps", "rope_theta"):
            setattr(c, f, getattr(self, f))
        c.moe = self.moe.to_c()
        return c


def pack_linear(parts: List[QWeight], K: int) -> torch.Tensor:
    """fmx_pack_linear: MLX-layout quantized matrices stacked by rows into
    the packed layout the decoder's projections read."""
    lib = _lib.load()
    rows = [p.w.shape[0] for p in parts]
    n = lib.fmx_packed_linear_size(sum(rows), K)
    if n == 0:
        raise _lib.FmxError(_lib.FMX_ERR_UNSUPPORTED, f"rows {rows}, K {K}")
    out = torch.empty(n, dtype=torch.uint8, device=parts[0].w.device)
    arr = (_lib.FmxQWeight * len(parts))(*[p.to_c() for p in parts])
    rr = (C.c_int64 * len(parts))(*rows)
    _lib.check(lib.fmx_pack_linear(arr, rr, len(parts), K, out.data_ptr(), n, _stream()))
    return out


@dataclass
class LayerWeights:
    """LlamaModel::LayerWeights (model.h:242-254) with the layer's MoEWeights."""
    input_norm_w: torch.Tensor
    post_norm_w: torch.Tensor
    qkv: torch.Tensor                    # packed q;k;v rows
    qkv_bias: Optional[torch.Tensor]     # bf16 [(nh + 2 nkv) hd] (q, k, v biases concatenated)
    o: torch.Tensor                      # packed [H, nh hd]
    moe: MoEWeights
    mlx: dict = field(default_factory=dict)  # MLX-layout QWeights kept on request (qkv, o)


@dataclass
class ModelWeights:
    embed: torch.Tensor                  # bf16 [V, H]
    norm_w: torch.Tensor
    lm_head: torch.Tensor                # packed [V, H]
    layers: List[LayerWeights]
    mlx: dict = field(default_factory=dict)  # MLX-layout lm_head kept on request


def c_weights(w):
    """(fmx_model_weights, the per-layer array it points to) for ModelWeights
    or a LoadedModel; keep both alive while the library may read them."""
    if isinstance(w, LoadedModel):
        return w.c_weights(), None
    layers = (_lib.FmxLayerWeights * len(w.layers))()
    for i, lw in enumerate(w.layers):
        L = layers[i]
        L.input_norm_w = lw.input_norm_w.data_ptr()
        L.post_norm_w = lw.post_norm_w.data_ptr()
        L.qkv = lw.qkv.data_ptr()
        L.qkv_bias = lw.qkv_bias.data_ptr() if lw.qkv_bias is not None else None
        L.o = lw.o.data_ptr()
        L.moe = lw.moe.to_c()
    c_w = _lib.FmxModelWeights()
    c_w.embed = w.embed.data_ptr()
    c_w.norm_w = w.norm_w.data_ptr()
    c_w.lm_head = w.lm_head.data_ptr()
    c_w.layers = layers
    return c_w, layers


class DecoderModel:
    """LlamaModel::forward (server/src/model.cpp:1021-1033) on libfmx, with
    a KV cache of `max_batch` sequences x `max_seq` positions and a workspace
    for forwards of up to `max_tokens` tokens."""

    def __init__(self, cfg: ModelConfig, w, max_batch: int, max_seq: int, max_tokens: int):
        """w: ModelWeights, or a LoadedModel (fmx_model_load)."""
        self.lib = _lib.load()
        self.cfg, self.w = cfg, w
        self._c_cfg = cfg.to_c()
        self.max_batch, self.max_seq = max_batch, max_seq
        dev = torch.device("cuda", torch.cuda.current_device())
        kv = self.lib.fmx_model_kv_cache_size(C.byref(self._c_cfg), max_batch, max_seq)
        ws = self.lib.fmx_model_workspace_size(C.byref(self._c_cfg), max_tokens)
        if kv == 0 or ws == 0:
            _lib.check(_lib.FMX_ERR_ARG)
        self.kv_cache = torch.zeros(kv, dtype=torch.uint8, device=dev)
        self.workspace = torch.empty(ws, dtype=torch.uint8, device=dev)
        self.ws_bytes = ws
        _lib.check(self.lib.fmx_model_workspace_init(C.byref(self._c_cfg), self.workspace.data_ptr(),
                                                     ws, _stream()))
        self._c_w, self._layers = c_weights(w)

    def kv_views(self):
        """(keys, values) as bf16 [layers, max_batch, nkv, max_seq, hd]."""
        c = self.cfg
        t = self.kv_cache.view(torch.bfloat16).view(c.num_hidden_layers, 2, self.max_batch,
                                                    c.num_key_value_heads, self.max_seq, c.hd)
        return t[:, 0], t[:, 1]

    def forward_into(self, ids: torch.Tensor, offset, logits: torch.Tensor, last_only: bool = True,
                     routing: Optional[torch.Tensor] = None):
        """ids int32 [B, L] (device); offset: an int, or a device int32 [B]
        tensor of per-sequence offsets. routing: an int32 [layers, B * L, k]
        device tensor that receives each layer's expert choice
        (fmx_model_forward_traced)."""
        B, L = ids.shape
        offs = offset.data_ptr() if isinstance(offset, torch.Tensor) else None
        off = 0 if offs is not None else int(offset)
        _lib.check(self.lib.fmx_model_forward_traced(
            C.byref(self._c_cfg), C.byref(self._c_w), ids.data_ptr(), B, L, off, offs,
            self.kv_cache.data_ptr(), self.max_batch, self.max_seq, int(last_only), logits.data_ptr(),
            self.workspace.data_ptr(), self.ws_bytes, _stream(),
            routing.data_ptr() if routing is not None else None))
        return logits

    def hidden(self, n_tokens: int) -> torch.Tensor:
        """The residual stream after the last layer of the latest forward
        (fmx_model_workspace_hidden), a bf16 [n_tokens, H] view."""
        p = C.c_void_p()
        _lib.check(self.lib.fmx_model_workspace_hidden(C.byref(self._c_cfg), n_tokens,
                                                       self.workspace.data_ptr(), C.byref(p)))
        off = p.value - self.workspace.data_ptr()
        H = self.cfg.hidden_size
        return self.workspace[off:off + n_tokens * H * 2].view(torch.bfloat16).view(n_tokens, H)

    def forward(self, ids: torch.Tensor, offset, last_only: bool = True,
                routing: Optional[torch.Tensor] = None) -> torch.Tensor:
        B, L = ids.shape
        shape = (B, self.cfg.vocab_size) if last_only else (B, L, self.cfg.vocab_size)
        logits = torch.empty(shape, dtype=torch.bfloat16, device=ids.device)
        return self.forward_into(ids, offset, logits, last_only, routing)

    def routing_buffer(self, n_tokens: int) -> torch.Tensor:
        """A device buffer for forward(routing=...): [layers, n_tokens, k] int32."""
        return torch.empty((self.cfg.num_hidden_layers, n_tokens, self.cfg.moe.num_experts_per_tok),
                           dtype=torch.int32, device=self.workspace.device)

    def greedy(self, logits: torch.Tensor, ids_out: torch.Tensor, offsets: Optional[torch.Tensor] = None,
               advance: int = 1) -> torch.Tensor:
        """fmx_greedy_next over logits [B, V]: ids_out [B] int32 (device);
        advances the device offsets when given."""
        B, V = logits.shape[0], logits.shape[-1]
        _lib.check(self.lib.fmx_greedy_next(
            logits.data_ptr(), B, V, logits.stride(0), ids_out.data_ptr(),
            offsets.data_ptr() if offsets is not None else None, advance, _stream()))
        return ids_out

    def generate(self, prompt: torch.Tensor, n_new: int) -> torch.Tensor:
        """Greedy decoding: prefill of prompt [B, L] at offset 0, then n_new
        tokens one step at a time. Returns int32 [B, n_new]."""
        B, L = prompt.shape
        out = torch.empty((B, n_new), dtype=torch.int32, device=prompt.device)
        ids = torch.empty((B, 1), dtype=torch.int32, device=prompt.device)
        logits = self.forward(prompt, 0)
        for i in range(n_new):
            self.greedy(logits, ids.view(-1))
            out[:, i] = ids.view(-1)
            if i + 1 < n_new:
                self.forward_into(ids, L + i, logits)
        return out


class BatchScheduler:
    """BatchScheduler (server/include/flashmlx/scheduler.h:37-99) on the
    native loop of fmx_sched.cpp: submit / step / has_work / drain_completed
    / active_count over a KV pool of n_slots slots of max_context positions.
    Greedy decoding only (temperature 0)."""

    def __init__(self, cfg: ModelConfig, w, n_slots: int, max_context: int, max_prompt: int,
                 prefix_cache: int = 0):
        """prefix_cache: entries of the prompt prefix cache (the reference
        keeps 32; 0 = off)."""
        self.lib = _lib.load()
        self.cfg, self.w = cfg, w
        self._c_cfg = cfg.to_c()
        self._c_w, self._layers = c_weights(w)
        self.n_slots = n_slots
        h = C.c_void_p()
        _lib.check(self.lib.fmx_scheduler_create(C.byref(self._c_cfg), C.byref(self._c_w), n_slots,
                                                 max_context, max_prompt, _stream(), C.byref(h)))
        self._h = h
        if prefix_cache:
            _lib.check(self.lib.fmx_scheduler_set_prefix_cache(h, prefix_cache))
        self._ids = (C.c_int64 * (2 * n_slots))()
        self._toks = (C.c_int32 * (2 * n_slots))()

    def close(self):
        if self._h:
            self.lib.fmx_scheduler_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def submit(self, prompt, max_tokens: int, temperature: float = 0.0) -> int:
        """Queues a request (prompt: a sequence of token ids); returns its id."""
        p = (C.c_int32 * len(prompt))(*[int(t) for t in prompt])
        rid = C.c_int64()
        _lib.check(self.lib.fmx_scheduler_submit(self._h, p, len(prompt), max_tokens,
                                                 float(temperature), C.byref(rid)))
        return rid.value

    def step(self) -> dict:
        """One iteration; {request id: [tokens generated in this step]}."""
        n = C.c_int64()
        _lib.check(self.lib.fmx_scheduler_step(self._h, self._ids, self._toks, 2 * self.n_slots,
                                               C.byref(n)))
        out: dict = {}
        for i in range(n.value):
            out.setdefault(self._ids[i], []).append(self._toks[i])
        return out

    def has_work(self) -> bool:
        return bool(self.lib.fmx_scheduler_has_work(self._h))

    def prefix_hits(self) -> int:
        return int(self.lib.fmx_scheduler_prefix_hits(self._h))

    def active_count(self) -> int:
        return int(self.lib.fmx_scheduler_active_count(self._h))

    def drain_completed(self) -> list:
        buf = (C.c_int64 * 256)()
        n = C.c_int64()
        out = []
        while True:
            _lib.check(self.lib.fmx_scheduler_drain_completed(self._h, buf, 256, C.byref(n)))
            out.extend(buf[i] for i in range(n.value))
            if n.value < 256:
                return out


# ------------------------------------------------------------------ synthetic weights

# synth stream ids: per layer 64 streams from LAYER_BASE * (layer + 1)
LAYER_BASE = 1000
S_EMBED, S_NORM, S_LM_HEAD = 1, 2, 3
S_IN_NORM, S_POST_NORM, S_Q, S_K, S_V, S_O, S_QB, S_KB, S_VB = 1, 2, 3, 4, 5, 6, 7, 8, 9
S_ROUTER, S_GATE, S_UP, S_DOWN, S_SH_GATE, S_SH_UP, S_SH_DOWN, S_SH_EGATE = 20, 21, 22, 23, 24, 25, 26, 27
W_STD = 0.02


def synthetic_model(cfg: ModelConfig, seed: int, device="cuda", keep_mlx: bool = False) -> ModelWeights:
    """Random-init weights of the config's shape, generated on the device
    (fmx_synth_normal_bf16_device): linears ~ N(0, 0.02) quantized affine
    4-bit g64 and packed; q/k/v biases ~ N(0, 0.1); norms ~ N(1, 0.1); the
    embedding ~ N(0, 0.02) quantized and dequantized to bf16 (the reference
    dequantizes its 4-bit table at load); the router and the shared-expert
    gate bf16 ~ N(0, 0.02). keep_mlx keeps the MLX-layout quantized arrays
    (for the CPU oracle)."""
    H, V, I, Is, E = (cfg.hidden_size, cfg.vocab_size, cfg.moe.moe_intermediate_size,
                      cfg.moe.shared_expert_intermediate_size, cfg.moe.num_experts)
    nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.hd

    def g(shape, stream, std=W_STD, mean=0.0):
        return synth_normal_bf16_device(shape, seed, stream, mean, std, device)

    def q(shape, stream):
        t = g(shape, stream)
        r = QWeight(*quantize(t))
        del t
        return r

    layers = []
    for li in range(cfg.num_hidden_layers):
        b = LAYER_BASE * (li + 1)
        qp, kp, vp = q((nh * hd, H), b + S_Q), q((nkv * hd, H), b + S_K), q((nkv * hd, H), b + S_V)
        op = q((H, nh * hd), b + S_O)
        bias = torch.cat([g((nh * hd,), b + S_QB, 0.1), g((nkv * hd,), b + S_KB, 0.1),
                          g((nkv * hd,), b + S_VB, 0.1)])
        moe = MoEWeights(router_w=g((E, H), b + S_ROUTER), gate=q((E, I, H), b + S_GATE),
                         up=q((E, I, H), b + S_UP), down=q((E, H, I), b + S_DOWN))
        if Is:
            moe.shared_gate, moe.shared_up = q((Is, H), b + S_SH_GATE), q((Is, H), b + S_SH_UP)
            moe.shared_down = q((H, Is), b + S_SH_DOWN)
            moe.shared_expert_gate_w = g((1, H), b + S_SH_EGATE)
        moe.pack(cfg.moe)
        lw = LayerWeights(input_norm_w=g((H,), b + S_IN_NORM, 0.1, 1.0),
                          post_norm_w=g((H,), b + S_POST_NORM, 0.1, 1.0),
                          qkv=pack_linear([qp, kp, vp], H), qkv_bias=bias,
                          o=pack_linear([op], nh * hd), moe=moe)
        if keep_mlx:
            lw.mlx = dict(qkv=QWeight(torch.cat([qp.w, kp.w, vp.w]), torch.cat([qp.scales, kp.scales, vp.scales]),
                                      torch.cat([qp.biases, kp.biases, vp.biases])), o=op)
        else:
            moe.drop_mlx_layout()
        layers.append(lw)
    et = QWeight(*quantize(g((V, H), S_EMBED)))
    embed = dequantize(et.w, et.scales, et.biases)
    lm = q((V, H), S_LM_HEAD)
    w = ModelWeights(embed=embed, norm_w=g((H,), S_NORM, 0.1, 1.0), lm_head=pack_linear([lm], H),
                     layers=layers)
    if keep_mlx:
        w.mlx = dict(lm_head=lm, embed=et)
    del et
    torch.cuda.synchronize()
    return w


def host_weights(cfg: ModelConfig, w: ModelWeights) -> dict:
    """The weights as numpy arrays in the CPU oracle's form (bf16 as uint16,
    quantized as (wq u32, scales, biases) tuples); needs keep_mlx=True."""
    import numpy as np

    def h16(t):
        return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    def hq(qw: QWeight):
        return (qw.w.contiguous().cpu().numpy().view(np.uint32), h16(qw.scales), h16(qw.biases))

    layers = []
    for lw in w.layers:
        m = lw.moe
        md = dict(router_w=h16(m.router_w), gate=hq(m.gate), up=hq(m.up), down=hq(m.down))
        if m.shared_gate is not None:
            md.update(shared_gate=hq(m.shared_gate), shared_up=hq(m.shared_up),
                      shared_down=hq(m.shared_down), shared_expert_gate_w=h16(m.shared_expert_gate_w))
        layers.append(dict(in_w=h16(lw.input_norm_w), post_w=h16(lw.post_norm_w), qkv=hq(lw.mlx["qkv"]),
                           qkv_bias=h16(lw.qkv_bias) if lw.qkv_bias is not None else None,
                           o=hq(lw.mlx["o"]), moe=md))
    return dict(embed=h16(w.embed), norm_w=h16(w.norm_w), lm_head=hq(w.mlx["lm_head"]), layers=layers)


def oracle_config(cfg: ModelConfig, max_seq: int) -> dict:
    """The CPU oracle's DecoderStack config for a ModelConfig."""
    m = cfg.moe
    return dict(hidden=cfg.hidden_size, layers=cfg.num_hidden_layers, heads=cfg.num_attention_heads,
                kv_heads=cfg.num_key_value_heads, head_dim=cfg.hd, vocab=cfg.vocab_size,
                eps=float(torch.tensor(cfg.rms_norm_eps, dtype=torch.float32)), theta=float(cfg.rope_theta),
                max_seq=max_seq,
                moe=dict(hidden=m.hidden_size, n_experts=m.num_experts, top_k=m.num_experts_per_tok,
                         inter=m.moe_intermediate_size, shared_inter=m.shared_expert_intermediate_size,
                         norm_topk=m.norm_topk_prob))


# ------------------------------------------------------------------ checkpoints

class LoadedModel:
    """Weights read from an MLX checkpoint directory by fmx_model_load (the
    library owns their device memory until close())."""

    def __init__(self, handle: int, cfg: ModelConfig):
        self.handle, self.cfg = handle, cfg
        self.lib = _lib.load()

    def c_weights(self):
        return self.lib.fmx_loaded_model_weights(self.handle).contents

    @property
    def device_bytes(self) -> int:
        return self.lib.fmx_loaded_model_device_bytes(self.handle)

    def close(self) -> None:
        if self.handle:
            self.lib.fmx_loaded_model_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 (interpreter shutdown)
            pass


def config_from_json(path: str) -> tuple:
    """fmx_model_config_from_json -> (ModelConfig, tie_word_embeddings)."""
    lib = _lib.load()
    c = _lib.FmxModelConfig()
    tie = C.c_int32()
    _lib.check(lib.fmx_model_config_from_json(str(path).encode(), C.byref(c), C.byref(tie)))
    m = c.moe
    cfg = ModelConfig(hidden_size=c.hidden_size, num_hidden_layers=c.num_hidden_layers,
                      num_attention_heads=c.num_attention_heads, num_key_value_heads=c.num_key_value_heads,
                      head_dim=c.head_dim, vocab_size=c.vocab_size,
                      max_position_embeddings=c.max_position_embeddings, rms_norm_eps=c.rms_norm_eps,
                      rope_theta=c.rope_theta,
                      moe=MoEConfig(hidden_size=m.hidden_size, num_experts=m.num_experts,
                                    num_experts_per_tok=m.num_experts_per_tok,
                                    moe_intermediate_size=m.moe_intermediate_size,
                                    shared_expert_intermediate_size=m.shared_expert_intermediate_size,
                                    norm_topk_prob=bool(m.norm_topk_prob), quant_bits=m.quant_bits,
                                    quant_group_size=m.quant_group_size))
    return cfg, bool(tie.value)


def load_checkpoint(path: str, cfg: Optional[ModelConfig] = None) -> LoadedModel:
    """fmx_model_load of an MLX checkpoint directory (config.json read when
    cfg is not given)."""
    import os
    lib = _lib.load()
    if cfg is None:
        cfg, _ = config_from_json(os.path.join(path, "config.json"))
    h = C.c_void_p()
    _lib.check(lib.fmx_model_load(str(path).encode(), C.byref(cfg.to_c()), C.byref(h), _stream()))
    return LoadedModel(h.value, cfg)


def write_safetensors(path: str, tensors: dict, metadata: Optional[dict] = None) -> None:
    """A safetensors file from {name: numpy array (uint16 for bf16, uint32,
    ...)}; uint16 arrays are written as BF16 (the MLX checkpoints' dtype)."""
    import json

    import numpy as np
    dt = {np.dtype(np.uint16): "BF16", np.dtype(np.uint32): "U32", np.dtype(np.float32): "F32",
          np.dtype(np.int32): "I32"}
    header, blobs, off = {}, [], 0
    for name in sorted(tensors):
        a = np.ascontiguousarray(tensors[name])
        b = a.tobytes()
        header[name] = {"dtype": dt[a.dtype], "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    if metadata:
        header["__metadata__"] = metadata
    h = json.dumps(header).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for b in blobs:
            f.write(b)


def save_checkpoint(cfg: ModelConfig, w: ModelWeights, path: str, shards: int = 2) -> None:
    """An MLX-format checkpoint of a synthetic model (keep_mlx=True): the
    per-expert arrays under the reference's key names
    (docs/superpowers/specs/2026-04-01-moe-support-design.md:138-151), with
    the "model." prefix, split over `shards` files, and its config.json."""
    import json
    import os

    import numpy as np

    def h(t):
        t = t.contiguous()
        if t.dtype == torch.bfloat16:
            return t.view(torch.int16).cpu().numpy().view(np.uint16)
        return t.cpu().numpy().view(np.uint32)

    def q(prefix, qw, out, idx=None):
        for part, t in (("weight", qw.w), ("scales", qw.scales), ("biases", qw.biases)):
            out[f"{prefix}.{part}"] = h(t if idx is None else t[idx])

    nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.hd
    out = {}
    for li, lw in enumerate(w.layers):
        p = f"model.layers.{li}"
        out[f"{p}.input_layernorm.weight"] = h(lw.input_norm_w)
        out[f"{p}.post_attention_layernorm.weight"] = h(lw.post_norm_w)
        qkv = lw.mlx["qkv"]
        r = [0, nh * hd, (nh + nkv) * hd, (nh + 2 * nkv) * hd]
        for i, name in enumerate(("q_proj", "k_proj", "v_proj")):
            q(f"{p}.self_attn.{name}", QWeight(qkv.w[r[i]:r[i + 1]], qkv.scales[r[i]:r[i + 1]],
                                               qkv.biases[r[i]:r[i + 1]]), out)
            if lw.qkv_bias is not None:
                out[f"{p}.self_attn.{name}.bias"] = h(lw.qkv_bias[r[i]:r[i + 1]])
        q(f"{p}.self_attn.o_proj", lw.mlx["o"], out)
        m = lw.moe
        if isinstance(m.router_w, QWeight):
            q(f"{p}.mlp.gate", m.router_w, out)
        else:
            out[f"{p}.mlp.gate.weight"] = h(m.router_w)
        for e in range(cfg.moe.num_experts):
            for name, qw in (("gate_proj", m.gate), ("up_proj", m.up), ("down_proj", m.down)):
                q(f"{p}.mlp.experts.{e}.{name}", qw, out, e)
        if m.shared_gate is not None:
            for name, qw in (("gate_proj", m.shared_gate), ("up_proj", m.shared_up), ("down_proj", m.shared_down)):
                q(f"{p}.mlp.shared_expert.{name}", qw, out)
            if isinstance(m.shared_expert_gate_w, QWeight):
                q(f"{p}.mlp.shared_expert_gate", m.shared_expert_gate_w, out)
            else:
                out[f"{p}.mlp.shared_expert_gate.weight"] = h(m.shared_expert_gate_w)
    q("model.embed_tokens", w.mlx["embed"], out)
    out["model.norm.weight"] = h(w.norm_w)
    q("lm_head", w.mlx["lm_head"], out)
    os.makedirs(path, exist_ok=True)
    names = sorted(out)
    for s in range(shards):
        part = {n: out[n] for n in names[s::shards]}
        write_safetensors(os.path.join(path, f"model-{s + 1:05d}-of-{shards:05d}.safetensors"), part,
                          {"format": "mlx"})
    mc = cfg.moe
    conf = dict(model_type="qwen2_moe", hidden_size=cfg.hidden_size, num_hidden_layers=cfg.num_hidden_layers,
                num_attention_heads=nh, num_key_value_heads=nkv, head_dim=hd, vocab_size=cfg.vocab_size,
                max_position_embeddings=cfg.max_position_embeddings, rms_norm_eps=cfg.rms_norm_eps,
                rope_theta=cfg.rope_theta, tie_word_embeddings=False, num_experts=mc.num_experts,
                num_experts_per_tok=mc.num_experts_per_tok, moe_intermediate_size=mc.moe_intermediate_size,
                shared_expert_intermediate_size=mc.shared_expert_intermediate_size,
                norm_topk_prob=mc.norm_topk_prob, quantization=dict(group_size=64, bits=4))
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(conf, f, indent=1)
