"""GPU parity of the float16 MoE block (fmx_moe_config.activation_dtype =
FMX_F16: a float16 checkpoint runs the whole block in float16,
model.cpp:208-214) against the oracle's float16 form, on the decode kernels
(at most 16 tokens) and the prefill GEMMs: routing bit-exact, outputs within
a float16 tolerance, and several times closer to the float16 oracle than the
bf16 block of the same values is (a kernel that rounded in bf16 anywhere
would not be)."""
import numpy as np
import pytest

from helpers import f16_inputs, f16_vals, from_dev_bf16, from_dev_u32

pytestmark = pytest.mark.gpu

# fp16 keeps 11 significant bits: 5e-3 is about ten units in the last place
# of an output; the absolute floor covers outputs near zero (sums of terms
# whose own rounding errors are ~2^-11 of the larger terms)
RTOL_F16 = 5e-3
ATOL_F16 = 2.5e-3
REL_L2_F16 = 2e-3


def _dev16(a_u16):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a_u16).view(np.int16)).to("cuda").view(torch.float16)


def _dev32(a_u32):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a_u32, dtype=np.uint32).view(np.int32)).to("cuda")


def _block(wl, cfg, w):
    """A float16 MoEBlock on packed weights from the oracle's float16 inputs."""
    import torch
    from flashmlx_amd.moe import MoEBlock, MoEConfig, MoEWeights, QWeight

    def qw(t):
        return QWeight(_dev32(t[0]), _dev16(t[1]), _dev16(t[2]))

    def row(r):
        return qw(r) if isinstance(r, tuple) else _dev16(r)

    m = wl.model
    c = MoEConfig(hidden_size=m["hidden"], num_experts=m["n_experts"], num_experts_per_tok=m["top_k"],
                  moe_intermediate_size=m["inter"], shared_expert_intermediate_size=m["shared_inter"],
                  norm_topk_prob=m["norm_topk"], activation_dtype=torch.float16)
    mw = MoEWeights(router_w=row(w["router_w"]), gate=qw(w["gate"]), up=qw(w["up"]), down=qw(w["down"]))
    if w.get("router_bias") is not None:
        mw.router_logit_bias = _dev16(w["router_bias"])
    if m["shared_inter"]:
        mw.shared_gate, mw.shared_up, mw.shared_down = qw(w["shared_gate"]), qw(w["shared_up"]), qw(w["shared_down"])
        mw.shared_expert_gate_w = row(w["shared_expert_gate_w"])
    return MoEBlock(c, mw, max_tokens=wl.tokens)


def _close16(got, ref, what):
    g, r = f16_vals(got), f16_vals(ref)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    d = np.abs(g - r)
    rel = float(np.linalg.norm(g - r) / np.linalg.norm(r))
    bad = d > ATOL_F16 + RTOL_F16 * np.abs(r)
    assert not bad.any(), f"{what}: {int(bad.sum())} elements outside rtol/atol; max abs {d.max():.3g}, rel L2 {rel:.3g}"
    assert rel <= REL_L2_F16, f"{what}: relative L2 error {rel:.3g} > {REL_L2_F16}"
    return rel, float(d.max())


# decode kernels: small shapes, Qwen1.5 at batch 1 (the shared expert) and
# 8, Qwen3 at batch 8 (renormalised top-8, no shared expert), a quantized
# router; prefill GEMMs: small shapes with a logit bias, Qwen1.5 at 512
# tokens with a skewed router, a quantized router at 200 tokens, Qwen3 at
# 1024 tokens (renormalised)
CASES = ["small_dec_t4", "qwen15_decode_b1", "qwen15_decode_b8", "qwen3_decode_b8", "qwen15_decode_b4_qrouter",
         "small_t23", "qwen15_prefill_512", "small_t200_qrouter", "qwen3_prefill_1024"]


@pytest.mark.parametrize("wl_key", CASES)
def test_block_f16_parity(gpu, fmx, oracle, wl_key):
    import torch
    from flashmlx_amd import workloads as W
    wl = W.WORKLOADS[wl_key]
    hi = W.host_inputs(wl)
    cfg, w, x = f16_inputs(oracle, hi, wl.model, router_quant=wl.router_quant)
    path = W.forward_path(wl.model, wl.tokens)
    print(f"{wl_key}: {wl.tokens} tokens, {path} path", flush=True)
    assert path in ("decode", "prefill")
    block = _block(wl, cfg, w)
    y = block(_dev16(x))
    torch.cuda.synchronize()
    assert block.status() == 0
    ry, rinds, rscores = oracle.moe_block(dict(cfg, act_f16=True), w, x, oracle.ACC_A)
    r = block.routing()
    np.testing.assert_array_equal(from_dev_u32(r["inds"]), rinds)
    np.testing.assert_array_equal(from_dev_bf16(r["scores"]), rscores)  # fp16 bits
    got = from_dev_bf16(y)
    rel, mx = _close16(got, ry, f"{wl_key} y")
    # the bf16 block of the same values (fp16 values of bf16 inputs are
    # exact) is several times farther from the float16 result
    tob = lambda u: oracle.f32_to_bf16_array(f16_vals(u).astype(np.float32))  # noqa: E731
    wb = {n: ((v[0], tob(v[1]), tob(v[2])) if isinstance(v, tuple) else (None if v is None else tob(v)))
          for n, v in w.items()}
    sub = np.arange(min(wl.tokens, 8))
    yb, _, _ = oracle.moe_block(cfg, wb, tob(x), oracle.ACC_A, tokens=sub)
    yb16 = oracle.bf16_to_f32(yb[sub]).astype(np.float64)
    rsub = f16_vals(ry[sub])
    relb = float(np.linalg.norm(yb16 - rsub) / np.linalg.norm(rsub))
    relg = float(np.linalg.norm(f16_vals(got[sub]) - rsub) / np.linalg.norm(rsub))
    print(f"  rel L2 {rel:.3g}, max abs {mx:.3g}; rows {sub.tolist()}: {relg:.3g} vs bf16 block {relb:.3g}")
    assert relg < relb / 3, (relg, relb)


def test_block_f16_deterministic_and_batch_independent(gpu, fmx, oracle):
    """Two forwards give the same bits, and a token's output row is the same
    whether it runs alone or in a batch of 8 (decode) or 40 (prefill)."""
    import torch
    from flashmlx_amd import workloads as W
    wl = W.Workload("small_dec_f16_t40", W.SMALL_DEC, 40, 31, router_bias=True)
    hi = W.host_inputs(wl)
    cfg, w, x = f16_inputs(oracle, hi, wl.model)
    block = _block(wl, cfg, w)
    y40 = from_dev_bf16(block(_dev16(x)))
    y40b = from_dev_bf16(block(_dev16(x)))
    np.testing.assert_array_equal(y40b, y40)
    y8 = from_dev_bf16(block(_dev16(x[:8])))
    y1 = from_dev_bf16(block(_dev16(x[3:4])))
    torch.cuda.synchronize()
    # decode rows against each other bit for bit; prefill rows within the
    # float16 tolerance (its GEMMs round the weights to fp16 once)
    np.testing.assert_array_equal(y1[0], y8[3])
    _close16(y40[:8], y8, "prefill rows vs decode rows")


@pytest.mark.parametrize("T", [5, 40])
def test_router_f16_standalone(gpu, fmx, oracle, T):
    """fmx_moe_router_topk(_ex) with a float16 config: logits, probabilities
    and scores in fp16, bit-exact against the oracle's float16 router (the
    one-launch router at 5 tokens, the two-launch one at 40), and the shared
    gate's fp16 sigmoid."""
    import torch
    from flashmlx_amd.moe import MoEConfig, router_topk
    from helpers import f16_bits
    rng = np.random.default_rng(700 + T)
    H, E, k = 256, 60, 4
    x = f16_bits(rng.standard_normal((T, H)))
    wr = f16_bits(rng.standard_normal((E, H)) * 0.05)
    wsg = f16_bits(rng.standard_normal((1, H)) * 0.05)
    for norm in (False, True):
        c = MoEConfig(hidden_size=H, num_experts=E, num_experts_per_tok=k, moe_intermediate_size=128,
                      shared_expert_intermediate_size=128, norm_topk_prob=norm, activation_dtype=torch.float16)
        inds, sc, pr, sg = router_topk(c, _dev16(x), _dev16(wr), shared_expert_gate_w=_dev16(wsg))
        torch.cuda.synchronize()
        _, rpr, rinds, rsc = oracle.router_topk(x, wr, k, norm, f16=True)
        np.testing.assert_array_equal(from_dev_u32(inds), rinds)
        np.testing.assert_array_equal(from_dev_bf16(sc), rsc)
        np.testing.assert_array_equal(from_dev_bf16(pr), rpr)
        lg, _, _, _ = oracle.router_topk(x, wsg, 1, False, f16=True)
        want = np.array([oracle.load().orc_sigmoid_f16(int(v)) for v in lg[:, 0]], np.float64)
        np.testing.assert_array_equal(f16_vals(from_dev_bf16(sg)), want)


def test_block_f16_needs_packed_weights(gpu, fmx, oracle):
    """A float16 block without packed weights is refused (FMX_ERR_UNSUPPORTED),
    not run on the bf16 kernels."""
    import torch
    from flashmlx_amd import _lib
    from flashmlx_amd import workloads as W
    wl = W.WORKLOADS["small_dec_t4"]
    hi = W.host_inputs(wl)
    cfg, w, x = f16_inputs(oracle, hi, wl.model)
    block = _block(wl, cfg, w)
    block.weights.packed = None
    block.refresh()
    with pytest.raises(_lib.FmxError) as ei:
        block(_dev16(x))
    assert ei.value.status == _lib.FMX_ERR_UNSUPPORTED
    torch.cuda.synchronize()
