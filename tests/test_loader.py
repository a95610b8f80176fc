"""The checkpoint loader's host side without a GPU: config.json parsing
with load_config's keys and defaults (server/src/model.cpp:111-140), and the
safetensors index (every *.safetensors file in name order, the "model."
prefix dropped, server/src/model.cpp:148-184), on files this test writes."""
import json

import numpy as np
import pytest


def _lib():
    from flashmlx_amd import _lib
    return _lib, _lib.load()


def test_config_from_json(fmx, tmp_path):
    from flashmlx_amd.model import config_from_json
    conf = dict(hidden_size=2048, num_hidden_layers=24, num_attention_heads=16, num_key_value_heads=16,
                vocab_size=151936, max_position_embeddings=8192, rms_norm_eps=1e-6, rope_theta=1000000.0,
                tie_word_embeddings=False, num_experts=60, num_experts_per_tok=4,
                moe_intermediate_size=1408, shared_expert_intermediate_size=5632, norm_topk_prob=False,
                quantization={"group_size": 64, "bits": 4}, architectures=["Qwen2MoeForCausalLM"],
                nested={"list": [1, 2.5e-3, "x", None, True]})
    p = tmp_path / "config.json"
    p.write_text(json.dumps(conf, indent=2))
    cfg, tie = config_from_json(str(p))
    assert (cfg.hidden_size, cfg.num_hidden_layers, cfg.num_attention_heads, cfg.num_key_value_heads) == (
        2048, 24, 16, 16)
    assert (cfg.vocab_size, cfg.max_position_embeddings, cfg.head_dim) == (151936, 8192, 0)
    assert cfg.rms_norm_eps == pytest.approx(1e-6) and cfg.rope_theta == 1e6 and tie is False
    m = cfg.moe
    assert (m.num_experts, m.num_experts_per_tok, m.moe_intermediate_size,
            m.shared_expert_intermediate_size, m.norm_topk_prob, m.quant_bits, m.quant_group_size) == (
        60, 4, 1408, 5632, False, 4, 64)
    # defaults of load_config when keys are missing
    p.write_text("{}")
    cfg, tie = config_from_json(str(p))
    assert (cfg.hidden_size, cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.vocab_size) == (
        4096, 32, 8, 128256)
    assert cfg.rope_theta == 10000.0 and tie is True and cfg.moe.quant_bits == 0
    p.write_text("{ not json")
    _l, lib = _lib()
    with pytest.raises(_l.FmxError):
        config_from_json(str(p))


def test_checkpoint_index(fmx, tmp_path):
    import ctypes as C

    from flashmlx_amd.model import write_safetensors
    _l, lib = _lib()
    a = np.arange(6, dtype=np.uint32).reshape(2, 3)
    b = np.arange(8, dtype=np.uint16)
    write_safetensors(str(tmp_path / "model-00001-of-00002.safetensors"), {"model.layers.0.w": a, "x": b})
    write_safetensors(str(tmp_path / "model-00002-of-00002.safetensors"), {"lm_head.scales": b[:4]})
    (tmp_path / "notes.txt").write_text("ignored")
    dt = C.create_string_buffer(8)
    shape = (C.c_int64 * 8)()
    nd = C.c_int32()
    assert lib.fmx_checkpoint_tensor(str(tmp_path).encode(), b"layers.0.w", dt, shape, C.byref(nd)) == 0
    assert dt.value == b"U32" and nd.value == 2 and list(shape[:2]) == [2, 3]
    assert lib.fmx_checkpoint_tensor(str(tmp_path).encode(), b"lm_head.scales", dt, shape, C.byref(nd)) == 0
    assert dt.value == b"BF16" and nd.value == 1 and shape[0] == 4
    assert lib.fmx_checkpoint_tensor(str(tmp_path).encode(), b"model.layers.0.w", dt, shape,
                                     C.byref(nd)) == _l.FMX_ERR_ARG
    assert b"no tensor" in lib.fmx_last_error()
    # a header whose offsets run past the file is refused
    bad = tmp_path / "zz.safetensors"
    hdr = json.dumps({"t": {"dtype": "U32", "shape": [4], "data_offsets": [0, 16]}}).encode()
    bad.write_bytes(len(hdr).to_bytes(8, "little") + hdr + b"\0" * 8)
    assert lib.fmx_checkpoint_tensor(str(tmp_path).encode(), b"x", dt, shape, C.byref(nd)) == _l.FMX_ERR_ARG
    assert b"inconsistent" in lib.fmx_last_error()


def test_safetensors_fixture_index(fmx):
    """The committed checkpoint written by the safetensors library
    (tests/golden/make_checkpoint.py): config.json parses with its keys,
    and the loader's index finds every tensor under the reference's names
    with the library's dtypes and shapes (the quantized router and shared
    gate included: mlp.gate.scales, mlp.shared_expert_gate.scales)."""
    import ctypes as C
    import pathlib

    from flashmlx_amd.model import config_from_json
    d = pathlib.Path(__file__).resolve().parent / "golden" / "ckpt_tiny"
    cfg, tie = config_from_json(str(d / "config.json"))
    assert (cfg.hidden_size, cfg.num_hidden_layers, cfg.num_attention_heads, cfg.num_key_value_heads,
            cfg.vocab_size) == (512, 1, 4, 1, 64) and tie is False
    assert (cfg.moe.num_experts, cfg.moe.num_experts_per_tok, cfg.moe.moe_intermediate_size,
            cfg.moe.shared_expert_intermediate_size, cfg.moe.quant_bits) == (4, 2, 128, 128, 4)
    _l, lib = _lib()
    dt = C.create_string_buffer(8)
    shape = (C.c_int64 * 8)()
    nd = C.c_int32()
    want = {"layers.0.mlp.gate.weight": ("U32", [4, 64]), "layers.0.mlp.gate.scales": ("BF16", [4, 8]),
            "layers.0.mlp.experts.3.down_proj.weight": ("U32", [512, 16]),
            "layers.0.mlp.shared_expert_gate.biases": ("BF16", [1, 8]),
            "layers.0.self_attn.k_proj.bias": ("BF16", [128]), "embed_tokens.scales": ("BF16", [64, 8]),
            "norm.weight": ("BF16", [512]), "lm_head.weight": ("U32", [64, 64])}
    for name, (dtype, shp) in want.items():
        assert lib.fmx_checkpoint_tensor(str(d).encode(), name.encode(), dt, shape, C.byref(nd)) == 0, name
        assert dt.value.decode() == dtype and list(shape[:nd.value]) == shp, (name, dt.value, shape[:nd.value])
