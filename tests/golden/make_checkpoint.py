"""Writes tests/golden/ckpt_tiny/: a one-layer Qwen2-MoE-style checkpoint in
the MLX format the reference loads (server/src/model.cpp:148-184, key names
of :214-224, :368-470 and :499-521), written by the `safetensors` library
(not by this package's own writer), and tests/golden/ckpt_tiny_logits.npz:
the CPU oracle's logits for a prompt and three decode steps on it.

Model: hidden 512, 4 heads on 1 kv head (head_dim 128) with q/k/v biases,
vocab 64, 4 experts top-2 (intermediate 128), a shared expert (128) with a
quantized sigmoid gate, a quantized router (mlp.gate.scales present, the
form of :758-760), quantized embedding and lm_head; every linear affine
4-bit group 64, quantized by the oracle's restatement of mx.quantize.

Run: python tests/golden/make_checkpoint.py
The fixture is data (weights, token ids, expected logits); no reference
code is stored.
"""
from __future__ import annotations

import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from oracle import oracle as O  # noqa: E402

OUT = HERE / "ckpt_tiny"
GOLDEN = HERE / "ckpt_tiny_logits.npz"
SEED = 2024
CONF = dict(model_type="qwen2_moe", architectures=["Qwen2MoeForCausalLM"], hidden_size=512,
            num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=1, vocab_size=64,
            max_position_embeddings=64, rms_norm_eps=1e-6, rope_theta=1000000.0, tie_word_embeddings=False,
            num_experts=4, num_experts_per_tok=2, moe_intermediate_size=128,
            shared_expert_intermediate_size=128, norm_topk_prob=False,
            quantization=dict(group_size=64, bits=4))
PROMPT_LEN, STEPS = 20, 3


def main() -> None:
    import torch
    from safetensors.torch import save_file

    rng = np.random.default_rng(SEED)
    c = CONF
    H, V, nh, nkv = c["hidden_size"], c["vocab_size"], c["num_attention_heads"], c["num_key_value_heads"]
    hd = H // nh
    E, I, Is = c["num_experts"], c["moe_intermediate_size"], c["shared_expert_intermediate_size"]

    def bf(shape, std, mean=0.0):
        return O.f32_to_bf16_array((rng.standard_normal(shape) * std + mean).astype(np.float32))

    def q(shape):
        return O.quantize(bf(shape, 0.02))

    tensors = {}

    def put_q(prefix, t):
        for part, a in zip(("weight", "scales", "biases"), t):
            tensors[f"{prefix}.{part}"] = a

    p = "model.layers.0"
    in_w, post_w = bf((H,), 0.1, 1.0), bf((H,), 0.1, 1.0)
    tensors[f"{p}.input_layernorm.weight"] = in_w
    tensors[f"{p}.post_attention_layernorm.weight"] = post_w
    qkv, biases = [], []
    for name, rows in (("q_proj", nh * hd), ("k_proj", nkv * hd), ("v_proj", nkv * hd)):
        t, b = q((rows, H)), bf((rows,), 0.1)
        put_q(f"{p}.self_attn.{name}", t)
        tensors[f"{p}.self_attn.{name}.bias"] = b
        qkv.append(t)
        biases.append(b)
    o = q((H, nh * hd))
    put_q(f"{p}.self_attn.o_proj", o)
    router = q((E, H))
    put_q(f"{p}.mlp.gate", router)
    experts = {n: [] for n in ("gate_proj", "up_proj", "down_proj")}
    for e in range(E):
        for name, shape in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
            t = q(shape)
            put_q(f"{p}.mlp.experts.{e}.{name}", t)
            experts[name].append(t)
    shared = {}
    for name, shape in (("gate_proj", (Is, H)), ("up_proj", (Is, H)), ("down_proj", (H, Is))):
        shared[name] = q(shape)
        put_q(f"{p}.mlp.shared_expert.{name}", shared[name])
    sgate = q((1, H))
    put_q(f"{p}.mlp.shared_expert_gate", sgate)
    embed = q((V, H))
    put_q("model.embed_tokens", embed)
    norm_w = bf((H,), 0.1, 1.0)
    tensors["model.norm.weight"] = norm_w
    lm = q((V, H))
    put_q("lm_head", lm)

    def to_torch(a):
        a = np.ascontiguousarray(a)
        if a.dtype == np.uint16:
            return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
        return torch.from_numpy(a)

    OUT.mkdir(exist_ok=True)
    for f in OUT.glob("*.safetensors"):
        f.unlink()
    names = sorted(tensors)
    for s in range(2):  # two shards, read in name order
        save_file({n: to_torch(tensors[n]) for n in names[s::2]},
                  str(OUT / f"model-{s + 1:05d}-of-00002.safetensors"), metadata={"format": "mlx"})
    (OUT / "config.json").write_text(json.dumps(CONF, indent=1) + "\n")

    # the oracle's decoder stack on the same arrays
    def cat(ts):
        return tuple(np.concatenate([t[i] for t in ts]) for i in range(3))

    def stack(ts):
        return tuple(np.stack([t[i] for t in ts]) for i in range(3))

    moe = dict(router_w=router, gate=stack(experts["gate_proj"]), up=stack(experts["up_proj"]),
               down=stack(experts["down_proj"]), shared_gate=shared["gate_proj"], shared_up=shared["up_proj"],
               shared_down=shared["down_proj"], shared_expert_gate_w=sgate)
    hw = dict(embed=O.f32_to_bf16_array(O.dequantize(*embed)), norm_w=norm_w, lm_head=lm,
              layers=[dict(in_w=in_w, post_w=post_w, qkv=cat(qkv), qkv_bias=np.concatenate(biases), o=o,
                           moe=moe)])
    oc = dict(hidden=H, layers=1, heads=nh, kv_heads=nkv, head_dim=hd, vocab=V,
              eps=float(np.float32(c["rms_norm_eps"])), theta=float(c["rope_theta"]), max_seq=32,
              moe=dict(hidden=H, n_experts=E, top_k=c["num_experts_per_tok"], inter=I, shared_inter=Is,
                       norm_topk=c["norm_topk_prob"]))
    st = O.DecoderStack(oc, hw, 1)
    prompt = rng.integers(0, V, (1, PROMPT_LEN))
    steps = rng.integers(0, V, (STEPS, 1, 1))
    prefill = st.forward(prompt, 0, last_only=False)
    dec = np.stack([st.forward(steps[i], PROMPT_LEN + i) for i in range(STEPS)])
    np.savez(GOLDEN, prompt=prompt.astype(np.int32), steps=steps.astype(np.int32), prefill_logits=prefill,
             step_logits=dec)
    print(f"wrote {OUT} ({sum(f.stat().st_size for f in OUT.iterdir())} bytes) and {GOLDEN}")


if __name__ == "__main__":
    main()
