"""ctypes binding of libfmx.so (the C-ABI declared in include/fmx.h and
include/fmx_model.h).

This module only loads the library and declares its signatures. It raises
ImportError when libfmx.so is missing: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os
import pathlib

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libfmx.so"

FMX_OK = 0
FMX_ERR_ARG = 1
FMX_ERR_SHAPE = 2
FMX_ERR_DTYPE = 3
FMX_ERR_UNSUPPORTED = 4
FMX_ERR_WORKSPACE = 5
FMX_ERR_HIP = 6

FMX_BF16, FMX_F32, FMX_U32, FMX_I32, FMX_F16 = 0, 1, 2, 3, 4
MAX_NDIM = 8


class FmxArray(C.Structure):
    _fields_ = [
        ("data", C.c_void_p),
        ("dtype", C.c_int32),
        ("ndim", C.c_int32),
        ("shape", C.c_int64 * MAX_NDIM),
    ]


class FmxMoEConfig(C.Structure):
    _fields_ = [
        ("hidden_size", C.c_int64),
        ("num_experts", C.c_int64),
        ("num_experts_per_tok", C.c_int32),
        ("norm_topk_prob", C.c_int32),
        ("moe_intermediate_size", C.c_int64),
        ("shared_expert_intermediate_size", C.c_int64),
        ("quant_bits", C.c_int32),
        ("quant_group_size", C.c_int32),
        ("activation_dtype", C.c_int32),
    ]


class FmxQWeight(C.Structure):
    _fields_ = [("w", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p)]


class FmxMoEWeights(C.Structure):
    _fields_ = [
        ("router_w", C.c_void_p),
        ("router_logit_bias", C.c_void_p),
        ("gate", FmxQWeight),
        ("up", FmxQWeight),
        ("down", FmxQWeight),
        ("shared_gate", FmxQWeight),
        ("shared_up", FmxQWeight),
        ("shared_down", FmxQWeight),
        ("shared_expert_gate_w", C.c_void_p),
        ("packed", C.c_void_p),
        ("packed_bytes", C.c_size_t),
        ("router_scales", C.c_void_p),
        ("router_biases", C.c_void_p),
        ("shared_expert_gate_scales", C.c_void_p),
        ("shared_expert_gate_biases", C.c_void_p),
    ]


class FmxModelConfig(C.Structure):
    _fields_ = [
        ("hidden_size", C.c_int64),
        ("num_hidden_layers", C.c_int64),
        ("num_attention_heads", C.c_int64),
        ("num_key_value_heads", C.c_int64),
        ("head_dim", C.c_int64),
        ("vocab_size", C.c_int64),
        ("max_position_embeddings", C.c_int64),
        ("rms_norm_eps", C.c_float),
        ("rope_theta", C.c_float),
        ("moe", FmxMoEConfig),
    ]


class FmxLayerWeights(C.Structure):
    _fields_ = [
        ("input_norm_w", C.c_void_p),
        ("post_norm_w", C.c_void_p),
        ("qkv", C.c_void_p),
        ("qkv_bias", C.c_void_p),
        ("o", C.c_void_p),
        ("moe", FmxMoEWeights),
    ]


class FmxModelWeights(C.Structure):
    _fields_ = [
        ("embed", C.c_void_p),
        ("norm_w", C.c_void_p),
        ("lm_head", C.c_void_p),
        ("layers", C.POINTER(FmxLayerWeights)),
    ]


class FmxNhMoEConfig(C.Structure):
    _fields_ = [
        ("hidden_size", C.c_int64),
        ("n_routed_experts", C.c_int64),
        ("num_experts_per_tok", C.c_int32),
        ("norm_topk_prob", C.c_int32),
        ("moe_intermediate_size", C.c_int64),
        ("moe_shared_expert_intermediate_size", C.c_int64),
        ("n_group", C.c_int32),
        ("topk_group", C.c_int32),
        ("routed_scaling_factor", C.c_float),
        ("quant_bits", C.c_int32),
        ("quant_group_size", C.c_int32),
    ]


class FmxNhMoEWeights(C.Structure):
    _fields_ = [
        ("gate_w", C.c_void_p),
        ("correction_bias", C.c_void_p),
        ("fc1", FmxQWeight),
        ("fc2", FmxQWeight),
        ("shared_up", FmxQWeight),
        ("shared_down", FmxQWeight),
        ("packed", C.c_void_p),
        ("packed_bytes", C.c_size_t),
    ]


class FmxError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


STATUS_NAMES = {
    FMX_OK: "FMX_OK",
    FMX_ERR_ARG: "FMX_ERR_ARG",
    FMX_ERR_SHAPE: "FMX_ERR_SHAPE",
    FMX_ERR_DTYPE: "FMX_ERR_DTYPE",
    FMX_ERR_UNSUPPORTED: "FMX_ERR_UNSUPPORTED",
    FMX_ERR_WORKSPACE: "FMX_ERR_WORKSPACE",
    FMX_ERR_HIP: "FMX_ERR_HIP",
}

P = C.POINTER
_A = P(FmxArray)
_SIGS = {
    "fmx_abi_version": (C.c_int, []),
    "fmx_status_string": (C.c_char_p, [C.c_int]),
    "fmx_last_error": (C.c_char_p, []),
    "fmx_quantized_matmul_out_shape": (C.c_int, [_A, _A, C.c_int, C.c_int, C.c_int, _A]),
    "fmx_quantized_matmul_workspace_size": (C.c_size_t, [_A, _A]),
    "fmx_quantized_matmul": (
        C.c_int,
        [_A, _A, _A, _A, C.c_int, C.c_int, C.c_int, C.c_char_p, _A, C.c_void_p, C.c_size_t, C.c_void_p],
    ),
    "fmx_gather_qmm_out_shape": (C.c_int, [_A, _A, _A, _A, C.c_int, C.c_int, C.c_int, _A]),
    "fmx_gather_qmm_workspace_size": (C.c_size_t, [_A, _A, _A, _A]),
    "fmx_gather_qmm": (
        C.c_int,
        [_A, _A, _A, _A, _A, _A, C.c_int, C.c_int, C.c_int, C.c_char_p, C.c_int, _A,
         C.c_void_p, C.c_size_t, C.c_void_p],
    ),
    "fmx_quantize": (C.c_int, [_A, C.c_int, C.c_int, C.c_char_p, _A, _A, _A, C.c_void_p]),
    "fmx_dequantize": (C.c_int, [_A, _A, _A, C.c_int, C.c_int, C.c_char_p, _A, C.c_void_p]),
    "fmx_stack_experts": (C.c_int, [P(C.c_void_p), C.c_int64, C.c_size_t, C.c_void_p, C.c_void_p]),
    "fmx_moe_packed_size": (C.c_size_t, [P(FmxMoEConfig)]),
    "fmx_pack_expert_weights": (
        C.c_int, [P(FmxMoEConfig), P(FmxMoEWeights), C.c_void_p, C.c_size_t, C.c_void_p]),
    "fmx_moe_forward_path": (C.c_int, [P(FmxMoEConfig), C.c_int64, C.c_int]),
    "fmx_moe_workspace_size": (C.c_size_t, [P(FmxMoEConfig), C.c_int64]),
    "fmx_moe_workspace_init": (C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p]),
    "fmx_moe_workspace_status": (C.c_int, [C.c_void_p, C.c_size_t, P(C.c_uint32), C.c_int, C.c_void_p]),
    "fmx_set_decode_wait_limit": (C.c_int64, [C.c_int64]),
    "fmx_moe_block_forward": (
        C.c_int,
        [P(FmxMoEConfig), P(FmxMoEWeights), C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p,
         C.c_size_t, C.c_void_p],
    ),
    "fmx_moe_block_forward_profiled": (
        C.c_int,
        [P(FmxMoEConfig), P(FmxMoEWeights), C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p,
         C.c_size_t, C.c_void_p, P(C.c_void_p)],
    ),
    "fmx_moe_block_forward_noalloc": (
        C.c_int,
        [P(FmxMoEConfig), P(FmxMoEWeights), C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p],
    ),
    "fmx_moe_block_forward_partial": (
        C.c_int,
        [P(FmxMoEConfig), P(FmxMoEWeights), C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p,
         C.c_size_t, C.c_void_p, C.c_int],
    ),
    "fmx_moe_workspace_routing": (
        C.c_int,
        [P(FmxMoEConfig), C.c_int64, C.c_void_p] + [P(C.c_void_p)] * 8,
    ),
    "fmx_moe_router_topk": (
        C.c_int,
        [P(FmxMoEConfig), C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
         C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p],
    ),
    "fmx_moe_router_topk_ex": (
        C.c_int,
        [P(FmxMoEConfig), C.c_void_p, C.c_int64, P(FmxMoEWeights), C.c_void_p, C.c_void_p, C.c_void_p,
         C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p],
    ),
    "fmx_moe_sort_workspace_size": (C.c_size_t, [C.c_int64, C.c_int32, C.c_int64]),
    "fmx_moe_sort": (
        C.c_int,
        [C.c_void_p, C.c_int64, C.c_int32, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p,
         C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p],
    ),
    "fmx_synth_normal_bf16": (
        C.c_int, [C.c_void_p, C.c_int64, C.c_uint64, C.c_uint64, C.c_double, C.c_double]),
    "fmx_synth_normal_bf16_device": (
        C.c_int, [C.c_void_p, C.c_int64, C.c_uint64, C.c_uint64, C.c_double, C.c_double, C.c_void_p]),
    # decoder stack (include/fmx_model.h)
    "fmx_packed_linear_size": (C.c_size_t, [C.c_int64, C.c_int64]),
    "fmx_pack_linear": (
        C.c_int, [P(FmxQWeight), P(C.c_int64), C.c_int, C.c_int64, C.c_void_p, C.c_size_t, C.c_void_p]),
    "fmx_model_kv_cache_size": (C.c_size_t, [P(FmxModelConfig), C.c_int64, C.c_int64]),
    "fmx_model_workspace_size": (C.c_size_t, [P(FmxModelConfig), C.c_int64]),
    "fmx_model_workspace_init": (C.c_int, [P(FmxModelConfig), C.c_void_p, C.c_size_t, C.c_void_p]),
    "fmx_model_forward": (
        C.c_int,
        [P(FmxModelConfig), P(FmxModelWeights), C.c_void_p, C.c_int64, C.c_int64, C.c_int64,
         C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int, C.c_void_p, C.c_void_p, C.c_size_t,
         C.c_void_p],
    ),
    "fmx_model_forward_traced": (
        C.c_int,
        [P(FmxModelConfig), P(FmxModelWeights), C.c_void_p, C.c_int64, C.c_int64, C.c_int64,
         C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int, C.c_void_p, C.c_void_p, C.c_size_t,
         C.c_void_p, C.c_void_p],
    ),
    "fmx_model_forward_batched": (
        C.c_int,
        [P(FmxModelConfig), P(FmxModelWeights), C.c_void_p, C.c_int64, C.c_int64, C.c_int64,
         C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int, C.c_void_p, C.c_void_p,
         C.c_size_t, C.c_void_p, C.c_void_p],
    ),
    "fmx_model_workspace_hidden": (C.c_int, [P(FmxModelConfig), C.c_int64, C.c_void_p, P(C.c_void_p)]),
    "fmx_model_config_from_json": (C.c_int, [C.c_char_p, P(FmxModelConfig), P(C.c_int32)]),
    "fmx_checkpoint_tensor": (C.c_int, [C.c_char_p, C.c_char_p, C.c_char_p, P(C.c_int64), P(C.c_int32)]),
    "fmx_model_load": (C.c_int, [C.c_char_p, P(FmxModelConfig), P(C.c_void_p), C.c_void_p]),
    "fmx_loaded_model_weights": (P(FmxModelWeights), [C.c_void_p]),
    "fmx_loaded_model_device_bytes": (C.c_size_t, [C.c_void_p]),
    "fmx_loaded_model_free": (None, [C.c_void_p]),
    "fmx_greedy_next": (
        C.c_int,
        [C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p]),
    "fmx_rope_table": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_float, C.c_void_p]),
    "fmx_attention_decode": (
        C.c_int,
        [C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p,
         C.c_int64, C.c_void_p, C.c_float, C.c_void_p, C.c_void_p]),
    "fmx_scheduler_create": (
        C.c_int,
        [P(FmxModelConfig), P(FmxModelWeights), C.c_int64, C.c_int64, C.c_int64, C.c_void_p,
         P(C.c_void_p)]),
    "fmx_scheduler_submit": (
        C.c_int, [C.c_void_p, P(C.c_int32), C.c_int64, C.c_int64, C.c_float, P(C.c_int64)]),
    "fmx_scheduler_step": (
        C.c_int, [C.c_void_p, P(C.c_int64), P(C.c_int32), C.c_int64, P(C.c_int64)]),
    "fmx_scheduler_has_work": (C.c_int, [C.c_void_p]),
    "fmx_scheduler_active_count": (C.c_int64, [C.c_void_p]),
    "fmx_scheduler_drain_completed": (
        C.c_int, [C.c_void_p, P(C.c_int64), C.c_int64, P(C.c_int64)]),
    "fmx_scheduler_free": (None, [C.c_void_p]),
    "fmx_scheduler_set_prefix_cache": (C.c_int, [C.c_void_p, C.c_int64]),
    "fmx_scheduler_prefix_hits": (C.c_int64, [C.c_void_p]),
    "fmx_nh_moe_packed_size": (C.c_size_t, [P(FmxNhMoEConfig)]),
    "fmx_nh_pack_expert_weights": (
        C.c_int, [P(FmxNhMoEConfig), P(FmxNhMoEWeights), C.c_void_p, C.c_size_t, C.c_void_p]),
    "fmx_nh_moe_workspace_size": (C.c_size_t, [P(FmxNhMoEConfig), C.c_int64]),
    "fmx_nh_moe_workspace_init": (C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p]),
    "fmx_nh_moe_block_forward": (
        C.c_int, [P(FmxNhMoEConfig), P(FmxNhMoEWeights), C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p,
                  C.c_size_t, C.c_void_p]),
    "fmx_nh_moe_block_forward_profiled": (
        C.c_int, [P(FmxNhMoEConfig), P(FmxNhMoEWeights), C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p,
                  C.c_size_t, C.c_void_p, P(C.c_void_p)]),
    "fmx_nh_moe_block_forward_partial": (
        C.c_int, [P(FmxNhMoEConfig), P(FmxNhMoEWeights), C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p,
                  C.c_size_t, C.c_void_p, C.c_int]),
    "fmx_nh_moe_workspace_routing": (
        C.c_int, [P(FmxNhMoEConfig), C.c_int64, C.c_void_p, P(C.c_void_p), P(C.c_void_p), P(C.c_void_p)]),
}

FMX_STATUS_WAIT_TIMEOUT = 1

EXPORTED = tuple(_SIGS)

_lib = None


def load(path: os.PathLike | str | None = None) -> C.CDLL:
    """Loads libfmx.so once and declares every entry point's signature."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = pathlib.Path(path) if path else LIB_PATH
    if not p.exists():
        raise ImportError(
            f"{p} is missing: build it with `python -m flashmlx_amd.build` "
            "(the MoE path has no fallback)")
    lib = C.CDLL(str(p))
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def check(status: int) -> None:
    if status != FMX_OK:
        msg = load().fmx_last_error().decode(errors="replace")
        raise FmxError(status, msg)
