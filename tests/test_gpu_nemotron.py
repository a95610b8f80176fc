"""GPU parity of the Nemotron-H MoE block (fmx_nh_moe_block_forward,
reference server/src/nemotron_h.cpp:1010-1111) against the CPU oracle:
logits, expert choice and fp32 scores bit-exact; y within the bf16
tolerance. Shapes: tiny ones with groups, a correction bias and padded
intermediate sizes, the 30B-A3B MoE shape (H 2688, 128 experts top-6,
I 1856 and Is 3712 padded to whole 128-k units), inputs outside fp16's
range (the exact bf16 path of both GEMMs), and the empty forward."""
import numpy as np
import pytest

from helpers import assert_close_rows, bf16_to_f32, from_dev_bf16, to_dev

pytestmark = pytest.mark.gpu


def _x(shape, seed, scale=1.0):
    from flashmlx_amd.moe import synth_normal_bf16
    n = int(np.prod(shape))
    return synth_normal_bf16(n, seed, 7, 0.0, scale).reshape(shape)


def _run(cfg, w, x_host, max_tokens=None):
    import torch
    from flashmlx_amd.nemotron import NhMoEBlock
    T = x_host.shape[0]
    blk = NhMoEBlock(cfg, w, max_tokens or max(T, 1))
    y = blk(to_dev(x_host))
    r = blk.routing()
    torch.cuda.synchronize()
    return (from_dev_bf16(y), r["inds"].cpu().numpy().astype(np.uint32), r["scores"].cpu().numpy(),
            from_dev_bf16(r["logits"].contiguous()))


def _check(oracle, cfg, w, x, what):
    from flashmlx_amd import nemotron as N
    hw = N.host_weights(w)
    oc = cfg.oracle_cfg()
    y, inds, scores, logits = _run(cfg, w, x)
    ref_lg, ref_inds, ref_scores = oracle.nh_route(oc, x, hw["gate_w"], hw["cbias"])
    assert np.array_equal(logits, ref_lg), f"{what}: logits"
    assert np.array_equal(inds, ref_inds), f"{what}: expert choice"
    assert np.array_equal(scores.view(np.uint32), ref_scores.view(np.uint32)), f"{what}: scores"
    ref_y, _, _ = oracle.nh_moe_block(oc, hw, x, oracle.ACC_F64)
    # y = bf16(bf16(routed) + shared): the routed sum is rounded at its own
    # magnitude before the shared expert's output is added, so an element of
    # y is accurate to the ulps of the row's large values (row-scaled atol)
    e = assert_close_rows(y, ref_y, what)
    print(f"{what}: {e}")
    return e


@pytest.mark.parametrize("T", [1, 5, 40, 130])
def test_nh_tiny_groups_bias_padding(gpu, fmx, oracle, T):
    """16 experts in 4 groups (2 kept), top-4, renormalised, scaling 2.5, a
    correction bias; I = 192 and Is = 320 (packed as 256 and 384)."""
    from flashmlx_amd import nemotron as N
    cfg = N.NhMoEConfig(hidden_size=256, n_routed_experts=16, num_experts_per_tok=4,
                        moe_intermediate_size=192, moe_shared_expert_intermediate_size=320,
                        n_group=4, topk_group=2, routed_scaling_factor=2.5)
    w = N.synthetic_nh_weights(cfg, 11, w_std=0.05)
    _check(oracle, cfg, w, _x((T, 256), 100 + T), f"tiny T={T}")


@pytest.mark.parametrize("T", [1, 3, 16, 17])
def test_nh_decode_kernels_groups_bias_padding(gpu, fmx, oracle, T):
    """The decode kernels (T <= 16; 17 takes the prefill path): 32 experts in
    4 groups (2 kept), top-4, a correction bias, I = 192 and Is = 640 (packed
    as 256 and 640), H = 512."""
    from flashmlx_amd import nemotron as N
    cfg = N.NhMoEConfig(hidden_size=512, n_routed_experts=32, num_experts_per_tok=4,
                        moe_intermediate_size=192, moe_shared_expert_intermediate_size=640,
                        n_group=4, topk_group=2, routed_scaling_factor=1.5)
    w = N.synthetic_nh_weights(cfg, 17, w_std=0.05)
    _check(oracle, cfg, w, _x((T, 512), 500 + T), f"decode kernels T={T}")


@pytest.mark.parametrize("T", [1, 8, 16, 96])
def test_nh_30b_shape(gpu, fmx, oracle, T):
    """The Nemotron-H 30B-A3B MoE layer shape, no groups, no shared expert
    gate: decode batches and a short prefill."""
    from flashmlx_amd import nemotron as N
    cfg = N.NhMoEConfig()
    w = N.synthetic_nh_weights(cfg, 12)
    _check(oracle, cfg, w, _x((T, cfg.hidden_size), 200 + T), f"30B shape T={T}")


def test_nh_exact_path_outside_fp16(gpu, fmx, oracle):
    """x with values beyond fp16's range: fc1 runs on the exact bf16 path,
    and relu^2 of its large outputs (beyond 65504) sends fc2 there too."""
    from flashmlx_amd import nemotron as N
    cfg = N.NhMoEConfig(hidden_size=256, n_routed_experts=8, num_experts_per_tok=2,
                        moe_intermediate_size=128, moe_shared_expert_intermediate_size=128)
    w = N.synthetic_nh_weights(cfg, 13, w_std=0.05)
    x = _x((24, 256), 300, scale=3e4)
    assert np.abs(bf16_to_f32(x)).max() > 65536
    _check(oracle, cfg, w, x, "exact path")


def test_nh_no_shared_no_norm(gpu, fmx, oracle):
    """No shared expert, no renormalisation, k = 1."""
    from flashmlx_amd import nemotron as N
    cfg = N.NhMoEConfig(hidden_size=128, n_routed_experts=32, num_experts_per_tok=1,
                        moe_intermediate_size=64, moe_shared_expert_intermediate_size=0,
                        norm_topk_prob=False, routed_scaling_factor=1.0)
    w = N.synthetic_nh_weights(cfg, 14, cbias_std=0.0, w_std=0.05)
    _check(oracle, cfg, w, _x((20, 128), 400), "k=1 no shared")


def test_nh_empty_and_refusals(gpu, fmx):
    """T = 0 runs nothing; a forward without packed weights is refused."""
    import ctypes as C

    import torch
    from flashmlx_amd import _lib
    from flashmlx_amd import nemotron as N
    cfg = N.NhMoEConfig(hidden_size=128, n_routed_experts=8, num_experts_per_tok=2,
                        moe_intermediate_size=64, moe_shared_expert_intermediate_size=0)
    w = N.synthetic_nh_weights(cfg, 15)
    lib = _lib.load()
    c, cw = cfg.to_c(), w.to_c()
    assert lib.fmx_nh_moe_block_forward(C.byref(c), C.byref(cw), None, 0, None, None, 0, None) == 0
    x = torch.zeros(4, 128, dtype=torch.bfloat16, device="cuda")
    y = torch.empty_like(x)
    rc = lib.fmx_nh_moe_block_forward(C.byref(c), C.byref(cw), x.data_ptr(), 4, y.data_ptr(), None, 0,
                                      torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.FMX_ERR_ARG


@pytest.mark.parametrize("T", [3, 40])
def test_nh_partial_forwards_leave_the_block_consistent(gpu, fmx, T):
    """fmx_nh_moe_block_forward_partial: 4 stages give the whole forward's y
    bit for bit, and forwards cut after 1, 2 or 3 stages (as per-stage
    timing runs them) leave the workspace's counters and flags such that the
    next whole forward still gives the same bits (decode kernels at 3
    tokens, the prefill GEMMs at 40)."""
    import torch
    from flashmlx_amd import nemotron as N
    cfg = N.NhMoEConfig(hidden_size=512, n_routed_experts=32, num_experts_per_tok=4,
                        moe_intermediate_size=192, moe_shared_expert_intermediate_size=640,
                        n_group=4, topk_group=2, routed_scaling_factor=1.5)
    w = N.synthetic_nh_weights(cfg, 19, w_std=0.05)
    blk = N.NhMoEBlock(cfg, w, T)
    x = to_dev(_x((T, 512), 700 + T))
    y_ref = blk(x)
    y = torch.zeros_like(y_ref)
    blk.forward_partial(x, y, 4)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
    for n in (1, 2, 3, 2, 1):
        blk.forward_partial(x, y, n)
        y2 = blk(x)
        torch.cuda.synchronize()
        assert torch.equal(y2, y_ref), f"after a {n}-stage forward"
