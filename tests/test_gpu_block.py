"""GPU parity of the fused MoE block (fmx_moe_block_forward) against the CPU
oracle on every MoE-layer workload: routing and permutation bit-exact and
every output row within the bf16 tolerance, plus invariants that hold at
full size."""
import numpy as np
import pytest

from helpers import assert_close, errors, from_dev_bf16, from_dev_u32, oracle_args

pytestmark = pytest.mark.gpu


def _run(wl_key, fmx, oracle, tokens=None, pack=True):
    from flashmlx_amd import workloads as W
    wl = W.WORKLOADS[wl_key]
    hi = W.host_inputs(wl)
    block, xd = W.device_block(wl, hi, pack=pack)
    y = block(xd)
    import torch
    torch.cuda.synchronize()
    return wl, hi, block, xd, y


CASES = [("tiny_t5", True), ("tiny_t5", False), ("tiny_t40", True), ("tiny_norm_t33", True),
         ("small_dec_t4", True), ("small_dec_t4", False),
         ("qwen15_decode_b1", True), ("qwen15_decode_b1", False), ("qwen15_decode_b4", True),
         ("small_t23", True), ("small_t200", True), ("small_t200", False),
         ("qwen15_decode_b8", True), ("qwen15_decode_b8", False), ("qwen15_prefill_512", True),
         ("qwen15_prefill_512", False),
         ("qwen3_decode_b1", True), ("qwen3_decode_b8", True), ("qwen3_decode_b8", False),
         ("qwen15_decode_b16", True), ("qwen3_decode_b16", True),
         ("qwen3_prefill_1024", True),
         ("qwen15_decode_b4_qrouter", True), ("qwen15_decode_b4_qrouter", False),
         ("small_t200_qrouter", True), ("small_t200_qrouter", False)]


# pack=True: forwards of at most 16 tokens run the packed-weight decode
# kernels, longer ones the packed-weight prefill GEMMs; pack=False keeps
# both on the MLX-layout grouped GEMM. Every output row is compared.
@pytest.mark.parametrize("wl_key,pack", CASES)
def test_block_parity(gpu, fmx, oracle, wl_key, pack):
    wl, hi, block, xd, y = _run(wl_key, fmx, oracle, pack=pack)
    m = wl.model
    T = hi.x.shape[0]
    cfg, w = oracle_args(hi, m, oracle.quantize, router_quant=wl.router_quant)
    ry, rinds, rscores = oracle.moe_block(cfg, w, hi.x, oracle.ACC_A)
    r = block.routing()
    np.testing.assert_array_equal(from_dev_u32(r["inds"]), rinds)
    np.testing.assert_array_equal(from_dev_bf16(r["scores"]), rscores)
    ro, rinv, rsrc, ridx, roff = oracle.moe_sort(rinds, m["n_experts"])
    np.testing.assert_array_equal(from_dev_u32(r["order"]), ro)
    np.testing.assert_array_equal(from_dev_u32(r["inv"]), rinv)
    np.testing.assert_array_equal(from_dev_u32(r["src"]), rsrc)
    np.testing.assert_array_equal(from_dev_u32(r["idx"]), ridx)
    np.testing.assert_array_equal(from_dev_u32(r["expert_offsets"]), roff)
    got = from_dev_bf16(y)
    e = assert_close(got, ry, f"{wl_key} y")
    print(f"{wl_key}: all {T} rows vs oracle(A): {e}")
    # report (not gate) the distance to the other MLX CPU accumulators the
    # oracle restates (modes B and C, each pinned in test_oracle.py)
    if T <= 8:
        sub = np.arange(min(T, 2))
        for mode, name in ((oracle.ACC_B, "B"), (oracle.ACC_C, "C")):
            yb, _, _ = oracle.moe_block(cfg, w, hi.x, mode, tokens=sub)
            print(f"  vs oracle({name}) tokens {sub.tolist()}: {errors(got[sub], yb[sub])}")


@pytest.mark.parametrize("wl_key", ["qwen15_decode_b8", "qwen15_prefill_512", "qwen3_decode_b8"])
def test_block_packed_only(gpu, fmx, oracle, wl_key):
    """With the MLX-layout expert arrays released after packing (the layer
    holds its expert weights once), both packed paths give the same bits."""
    import torch
    from flashmlx_amd import workloads as W
    wl = W.WORKLOADS[wl_key]
    hi = W.host_inputs(wl)
    block, xd = W.device_block(wl, hi)
    y1 = from_dev_bf16(block(xd))
    block2, xd2 = W.device_block(wl, hi, drop_mlx=True)
    w2 = block2.weights
    assert w2.gate is None and w2.shared_gate is None
    y2 = from_dev_bf16(block2(xd2))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y2, y1)


# Qwen1.5 shape at token counts between the named workloads: odd decode
# batches (partial 4-token slot words), both sides of the gate/up pairing
# threshold (one tile pair per workgroup up to 5 tokens, two from 6, where
# max_seg * I / 16 first reaches 2048 tile pairs: 24 * 88 = 2112) and 17,
# the smallest forward on the prefill GEMMs
@pytest.mark.parametrize("T", [3, 5, 6, 7, 12, 13, 15, 17])
def test_block_parity_token_sweep(gpu, fmx, oracle, T):
    import torch
    from flashmlx_amd import workloads as W
    wl = W.Workload(f"qwen15_t{T}", W.QWEN15, T, 100 + T, router_bias=T % 2 == 1)
    hi = W.host_inputs(wl)
    block, xd = W.device_block(wl, hi)
    y = block(xd)
    torch.cuda.synchronize()
    assert W.decode_path(wl.model, T) == (T <= 16)
    cfg, w = oracle_args(hi, wl.model, oracle.quantize)
    sub = np.arange(T)
    ry, rinds, rscores = oracle.moe_block(cfg, w, hi.x, oracle.ACC_A, tokens=sub)
    r = block.routing()
    np.testing.assert_array_equal(from_dev_u32(r["inds"]), rinds)
    np.testing.assert_array_equal(from_dev_bf16(r["scores"]), rscores)
    e = assert_close(from_dev_bf16(y), ry, f"qwen15 T={T} y")
    print(f"qwen15 T={T}: {e}")


@pytest.mark.parametrize("wl_key", ["qwen15_decode_b8", "qwen3_decode_b1"])
def test_block_decode_wait_guard(gpu, fmx, oracle, wl_key):
    """The down workgroups' bounded wait for their expert's gate/up tiles,
    made to give up at once from the host (fmx_set_decode_wait_limit(0)):
    every kernel still ends, the products come out NaN and the workspace's
    status word says so; with the default bound back and the word cleared,
    the next forward gives the normal output again."""
    import torch
    from flashmlx_amd import _lib
    from flashmlx_amd import workloads as W
    from helpers import bf16_to_f32
    lib = _lib.load()
    wl = W.WORKLOADS[wl_key]
    hi = W.host_inputs(wl)
    block, xd = W.device_block(wl, hi)
    y_ok = from_dev_bf16(block(xd))
    assert block.status() == 0
    assert lib.fmx_set_decode_wait_limit(0) == 1 << 21
    try:
        y_bad = block(xd)
        torch.cuda.synchronize()
    finally:
        lib.fmx_set_decode_wait_limit(-1)
    assert block.status(clear=True) == _lib.FMX_STATUS_WAIT_TIMEOUT
    assert np.isnan(bf16_to_f32(from_dev_bf16(y_bad))).all()
    assert block.status() == 0
    np.testing.assert_array_equal(from_dev_bf16(block(xd)), y_ok)
    assert block.status() == 0


@pytest.mark.parametrize("wl_key", ["qwen3_decode_b8", "qwen15_decode_b8"])
def test_block_deterministic_and_reusable(gpu, fmx, oracle, wl_key):
    """Same input twice -> identical bits; the workspace then serves a
    smaller call, whose rows equal the larger call's prefix rows (tokens are
    independent and x of T=1 is the first row of x of T=8). A 64-token call
    (eight copies of the 8 tokens; crosses the sort threshold and leaves the
    at-most-16-token kernels) gives the same bits for every copy, within the
    bf16 tolerance of the 8-token call (its accumulation order differs); an
    8-token call after it repeats the first call's bits."""
    import torch
    from flashmlx_amd import workloads as W
    wl = W.WORKLOADS[wl_key]
    hi = W.host_inputs(wl)
    block, xd = W.device_block(wl, hi, max_tokens=64)
    y1 = from_dev_bf16(block(xd))
    y2 = from_dev_bf16(block(xd))
    np.testing.assert_array_equal(y1, y2)
    y3 = from_dev_bf16(block(xd[:1].contiguous()))
    np.testing.assert_array_equal(y3[0], y1[0])
    xx = torch.cat([xd] * 8)
    y4 = from_dev_bf16(block(xx))
    for i in range(1, 8):
        np.testing.assert_array_equal(y4[8 * i: 8 * i + 8], y4[:8])
    assert_close(y4[:8], y1, "64-token call vs 8-token call")
    # back on the decode kernels after the prefill path: whatever counters
    # and flags either path uses are back at zero, so the bits repeat
    np.testing.assert_array_equal(from_dev_bf16(block(xd)), y1)


@pytest.mark.parametrize("wl_key", ["qwen15_decode_b8", "small_t23"])
def test_block_zero_tokens(gpu, fmx, oracle, wl_key):
    """A forward of zero tokens launches nothing and returns an empty y; the
    same workspace then serves a normal call with the same bits as before."""
    from flashmlx_amd import workloads as W
    wl = W.WORKLOADS[wl_key]
    hi = W.host_inputs(wl)
    block, xd = W.device_block(wl, hi)
    y1 = from_dev_bf16(block(xd))
    y0 = block(xd[:0].contiguous())
    assert tuple(y0.shape) == (0, xd.shape[1])
    np.testing.assert_array_equal(from_dev_bf16(block(xd)), y1)


def test_block_prefill_beyond_lds_sort(gpu, fmx, oracle):
    """A Qwen3-shape prefill of 4500 tokens (36,000 routed entries, more
    than the sort holds in LDS): routing and the sort bit-exact for every
    token, each row equal to the same token's row from two separate
    2250-token forwards, and 16 sampled rows within the bf16 tolerance of
    the oracle."""
    import torch
    from flashmlx_amd import workloads as W
    wl = W.Workload("qwen3_t4500", W.QWEN3, 4500, 41)
    hi = W.host_inputs(wl)
    block, xd = W.device_block(wl, hi)
    y = from_dev_bf16(block(xd))
    r = block.routing()
    inds = from_dev_u32(r["inds"])
    _, _, rinds, rscores = oracle.router_topk(hi.x, hi.router_w, 8, True)
    np.testing.assert_array_equal(inds, rinds)
    np.testing.assert_array_equal(from_dev_bf16(r["scores"]), rscores)
    ro, rinv, rsrc, ridx, roff = oracle.moe_sort(rinds, 128)
    np.testing.assert_array_equal(from_dev_u32(r["order"]), ro)
    np.testing.assert_array_equal(from_dev_u32(r["inv"]), rinv)
    np.testing.assert_array_equal(from_dev_u32(r["expert_offsets"]), roff)
    halves = [from_dev_bf16(block(xd[i * 2250:(i + 1) * 2250].contiguous())) for i in range(2)]
    torch.cuda.synchronize()
    assert_close(y, np.concatenate(halves), "4500-token forward vs two 2250-token forwards")
    cfg, w = oracle_args(hi, wl.model, oracle.quantize)
    sub = np.unique(np.linspace(0, 4499, 16).astype(np.int64))
    ry, _, _ = oracle.moe_block(cfg, w, hi.x, oracle.ACC_A, tokens=sub)
    e = assert_close(y[sub], ry[sub], "qwen3 t4500 sampled rows")
    print(f"qwen3 t4500: {e}")


# Prefill rows whose values leave fp16's range: one token's x scaled by 2^12
# (x below 65536, its SwiGLU outputs h far above) or by 2^17 (x itself above
# 65536). The GEMMs then take the exact bf16 path for that grid; every row,
# the scaled one included, is checked against the oracle.
@pytest.mark.parametrize("scale_exp", [12, 17])
def test_block_prefill_fp16_range(gpu, fmx, oracle, scale_exp):
    import dataclasses

    import torch
    from flashmlx_amd import workloads as W
    wl = W.WORKLOADS["small_t200"]
    hi = W.host_inputs(wl)
    x = hi.x.copy()
    row = (x[7].astype(np.uint32) << 16).view(np.float32) * np.float32(2.0 ** scale_exp)
    x[7] = (row.view(np.uint32) >> 16).astype(np.uint16)  # exact: a power-of-two scale
    hi = dataclasses.replace(hi, x=x)
    big = np.abs((x[7].astype(np.uint32) << 16).view(np.float32)).max()
    assert (big >= 65536) == (scale_exp == 17)
    block, xd = W.device_block(wl, hi)
    y = from_dev_bf16(block(xd))
    torch.cuda.synchronize()
    cfg, w = oracle_args(hi, wl.model, oracle.quantize)
    ry, rinds, _ = oracle.moe_block(cfg, w, hi.x, oracle.ACC_A)
    np.testing.assert_array_equal(from_dev_u32(block.routing()["inds"]), rinds)
    assert np.abs((ry[7].astype(np.uint32) << 16).view(np.float32)).max() >= 65536
    e = assert_close(y, ry, f"small_t200 with token 7 scaled by 2^{scale_exp}")
    print(f"fp16 range, 2^{scale_exp}: {e}")
