"""fmx_moe_block_forward_noalloc: the MoE block forward whose workspace is
the library's fixed per-device scratch array (no allocation anywhere).
Its output equals fmx_moe_block_forward's on the same inputs, bit for bit,
on two calls in a row (the second smaller), on the decode kernels and on the
prefill GEMMs; a forward larger than the scratch is refused before any
launch."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from helpers import from_dev_bf16


def _noalloc(block, x, y):
    import torch
    from flashmlx_amd import _lib
    lib = _lib.load()
    T = x.numel() // block.cfg.hidden_size
    return lib.fmx_moe_block_forward_noalloc(C.byref(block._c_cfg), C.byref(block._c_w), x.data_ptr(), T,
                                             y.data_ptr(), torch.cuda.current_stream().cuda_stream)


def test_noalloc_refuses_oversize_forward(fmx):
    """A forward whose workspace exceeds the scratch returns
    FMX_ERR_UNSUPPORTED before any device call (runs without a GPU)."""
    from flashmlx_amd import MoEConfig
    from flashmlx_amd import _lib
    lib = _lib.load()
    cfg = MoEConfig(2048, 60, 4, 1408, 5632, False).to_c()
    assert lib.fmx_moe_workspace_size(C.byref(cfg), 512) > (8 << 20)
    w = _lib.FmxMoEWeights()
    buf = np.zeros(64, np.uint8)
    rc = lib.fmx_moe_block_forward_noalloc(C.byref(cfg), C.byref(w), buf.ctypes.data, 512,
                                           buf.ctypes.data, None)
    assert rc == _lib.FMX_ERR_UNSUPPORTED
    assert b"scratch" in lib.fmx_last_error()
    assert lib.fmx_moe_block_forward_noalloc(C.byref(cfg), C.byref(w), None, 0, None, None) == _lib.FMX_OK


@pytest.mark.gpu
@pytest.mark.parametrize("key,T0,T1", [("qwen15_decode_b16", 16, 5), ("qwen3_t64", 64, 20)])
def test_noalloc_matches_workspace_forward(gpu, fmx, key, T0, T1):
    import torch
    from flashmlx_amd import _lib
    from flashmlx_amd import workloads as W
    wl = W.WORKLOADS.get(key) or W.Workload(key, W.QWEN3, T0, 51)
    hi = W.host_inputs(wl)
    block, xd = W.device_block(wl, hi, max_tokens=T0)
    assert W.forward_path(wl.model, T0) == ("decode" if T0 <= 16 else "prefill")
    for T in (T0, T1):
        x = xd[:T].contiguous()
        ref = from_dev_bf16(block(x))
        y = torch.full_like(x, float("nan"))
        print(f"noalloc forward: {key} T={T}", flush=True)
        _lib.check(_noalloc(block, x, y))
        torch.cuda.synchronize()
        got = from_dev_bf16(y)
        np.testing.assert_array_equal(got, ref)
    # and once more at the first size: the scratch's counters were left at zero
    y = torch.empty_like(xd)
    _lib.check(_noalloc(block, xd, y))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev_bf16(y), from_dev_bf16(block(xd)))
