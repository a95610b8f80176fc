"""flashmlx_amd: MI355X-native MoE hot path of FlashMLX (router, token sort,
grouped 4-bit gather_qmm with SwiGLU, down + top-k combine, gated shared
expert), behind the C-ABI in include/fmx.h and built into libfmx.so."""
from ._lib import FmxError, load  # noqa: F401
from .moe import (  # noqa: F401
    MoEBlock,
    MoEConfig,
    MoEWeights,
    QWeight,
    dequantize,
    gather_qmm,
    moe_sort,
    quantize,
    quantized_matmul,
    router_topk,
    synth_normal_bf16,
    synth_normal_bf16_device,
)

__all__ = [
    "FmxError",
    "MoEBlock",
    "MoEConfig",
    "MoEWeights",
    "QWeight",
    "dequantize",
    "gather_qmm",
    "load",
    "moe_sort",
    "quantize",
    "quantized_matmul",
    "router_topk",
    "synth_normal_bf16",
    "synth_normal_bf16_device",
]
