"""GPU parity of the single ops behind the C-ABI against the CPU oracle:
quantize/dequantize (bit-exact), quantized_matmul and gather_qmm (bf16
tolerance), router top-k and the expert sort (bit-exact)."""
import numpy as np
import pytest

from helpers import (assert_close, assert_close_rows, bf16_to_f32, from_dev_bf16, from_dev_u32, to_dev,
                     to_dev_u32)

pytestmark = pytest.mark.gpu


def _rand_bf16(rng, shape, std=1.0):
    from oracle import oracle as O
    return O.f32_to_bf16_array(rng.standard_normal(shape).astype(np.float32) * std)


@pytest.mark.parametrize("shape", [(4, 128), (3, 5, 256), (1408, 2048)])
def test_quantize_bitexact(gpu, fmx, oracle, shape):
    rng = np.random.default_rng(7)
    w = _rand_bf16(rng, shape, 0.02)
    if shape == (4, 128):  # edge groups: constant, all-negative, tiny range, zeros
        w[0, :64] = w[0, 0]
        w[1, :64] = np.abs(w[1, :64]) | 0x8000
        w[2, 64:] = 0
        w[3, :64] = 0x3f80  # 1.0
    wq, s, b = fmx.quantize(to_dev(w))
    rq, rs, rb = oracle.quantize(w)
    np.testing.assert_array_equal(from_dev_u32(wq), rq)
    np.testing.assert_array_equal(from_dev_bf16(s), rs)
    np.testing.assert_array_equal(from_dev_bf16(b), rb)


def test_dequantize_matches_oracle(gpu, fmx, oracle):
    rng = np.random.default_rng(8)
    w = _rand_bf16(rng, (64, 512), 0.02)
    rq, rs, rb = oracle.quantize(w)
    out = fmx.dequantize(to_dev_u32(rq), to_dev(rs), to_dev(rb))
    ref = oracle.f32_to_bf16_array(oracle.dequantize(rq, rs, rb))
    np.testing.assert_array_equal(from_dev_bf16(out), ref)


# fewer than 32 rows, and shapes outside whole 128-k units or 16-row tiles,
# run the grouped GEMM (exact dequantisation); more rows run the prefill
# GEMM on the MLX-layout weights (fp16 weights, within 2^-11 relative of
# exact)
@pytest.mark.parametrize("M,N,K", [(1, 64, 256), (3, 200, 1408), (16, 128, 2048),
                                   (37, 96, 768), (5, 2048, 5632), (17, 16, 128),
                                   (64, 256, 1024), (200, 512, 2048), (40, 200, 1408),
                                   (33, 64, 1344)])
def test_quantized_matmul(gpu, fmx, oracle, M, N, K):
    rng = np.random.default_rng(M * 1000 + N + K)
    x = _rand_bf16(rng, (M, K))
    w = _rand_bf16(rng, (N, K), 0.02)
    rq, rs, rb = oracle.quantize(w)
    out = fmx.quantized_matmul(to_dev(x), to_dev_u32(rq), to_dev(rs), to_dev(rb))
    got = from_dev_bf16(out)
    ref = oracle.qmm_t(x, rq, rs, rb, oracle.ACC_A)
    e = assert_close(got, ref, f"qmm M={M} N={N} K={K}")
    # also against the exact (fp64) value
    ref64 = oracle.qmm_t(x, rq, rs, rb, oracle.ACC_F64)
    e64 = assert_close(got, ref64, "qmm vs fp64")
    assert e64["max_abs"] <= 2 * np.abs(bf16_to_f32(ref64)).max() * 2 ** -8 + 1e-6, e64
    print(f"qmm M={M} N={N} K={K}: vs A {e}, vs f64 {e64}")


def test_quantized_matmul_prefill_fp16_overflow(gpu, fmx, oracle):
    """Rows holding values outside fp16's range take the exact bf16 path of
    the prefill GEMM (the copy kernel's flag); a second call on rows that fit
    takes the fp16 path again (the flag is cleared per call)."""
    rng = np.random.default_rng(23)
    M, N, K = 48, 128, 512
    w = _rand_bf16(rng, (N, K), 0.02)
    rq, rs, rb = oracle.quantize(w)
    x = _rand_bf16(rng, (M, K))
    big = x.copy()
    big[5, 17] = oracle.f32_to_bf16_array(np.array([1.0e5], np.float32))[0]
    big[40, 300] = oracle.f32_to_bf16_array(np.array([-7.0e4], np.float32))[0]
    # a row with a 1e5 element sums products up to ~5000 (fp32 ulp 2^-11
    # there) whose group sums cancel, so its elements are held to the row's
    # scale: two bf16 ulps of the row's largest output (assert_close_rows)
    for xi, what, check in ((big, "overflow rows", assert_close_rows), (x, "fp16 rows", assert_close)):
        out = fmx.quantized_matmul(to_dev(xi), to_dev_u32(rq), to_dev(rs), to_dev(rb))
        ref = oracle.qmm_t(xi, rq, rs, rb, oracle.ACC_A)
        check(from_dev_bf16(out), ref, f"qmm {what}")


def test_quantized_matmul_batch_dims(gpu, fmx, oracle):
    rng = np.random.default_rng(3)
    x = _rand_bf16(rng, (2, 3, 1, 256))
    w = _rand_bf16(rng, (64, 256), 0.02)
    rq, rs, rb = oracle.quantize(w)
    out = fmx.quantized_matmul(to_dev(x), to_dev_u32(rq), to_dev(rs), to_dev(rb))
    assert tuple(out.shape) == (2, 3, 1, 64)
    ref = oracle.qmm_t(x.reshape(-1, 256), rq, rs, rb, oracle.ACC_A).reshape(2, 3, 1, 64)
    assert_close(from_dev_bf16(out), ref, "qmm batch dims")


def _gather_case(rng, oracle, E, N, K, n_x, M):
    x = _rand_bf16(rng, (n_x, M, K))
    w = _rand_bf16(rng, (E, N, K), 0.02)
    rq, rs, rb = oracle.quantize(w)
    return x, rq, rs, rb


def test_gather_qmm_unsorted_decode_layout(gpu, fmx, oracle):
    """switch_mlp's unsorted call: x [B,L,1,1,H], rhs = inds [B,L,k] (model.cpp:681, :703)."""
    rng = np.random.default_rng(11)
    B, L, k, E, N, K = 2, 3, 4, 8, 128, 512
    x, rq, rs, rb = _gather_case(rng, oracle, E, N, K, B * L, 1)
    inds = np.stack([rng.permutation(E)[:k] for _ in range(B * L)]).astype(np.uint32).reshape(B, L, k)
    xd = to_dev(x.reshape(B, L, 1, 1, K))
    out = fmx.gather_qmm(xd, to_dev_u32(rq), to_dev(rs), to_dev(rb), rhs_indices=to_dev_u32(inds))
    assert tuple(out.shape) == (B, L, k, 1, N)
    lhs = np.repeat(np.arange(B * L, dtype=np.uint32), k)
    ref = oracle.gather_qmm(x, rq, rs, rb, lhs, inds.reshape(-1), oracle.ACC_A)
    assert_close(from_dev_bf16(out).reshape(-1, 1, N), ref, "gather unsorted")


def test_gather_qmm_sorted_layout(gpu, fmx, oracle):
    """switch_mlp's sorted call: x [Tk,1,H] gathered, rhs [Tk] (model.cpp:686-699)."""
    rng = np.random.default_rng(12)
    n, E, N, K = 70, 6, 96, 256
    x, rq, rs, rb = _gather_case(rng, oracle, E, N, K, n, 1)
    idx = np.sort(rng.integers(0, E, n)).astype(np.uint32)
    out = fmx.gather_qmm(to_dev(x), to_dev_u32(rq), to_dev(rs), to_dev(rb),
                         rhs_indices=to_dev_u32(idx), sorted_indices=True)
    assert tuple(out.shape) == (n, 1, N)
    ref = oracle.gather_qmm(x, rq, rs, rb, np.arange(n, dtype=np.uint32), idx, oracle.ACC_A)
    assert_close(from_dev_bf16(out), ref, "gather sorted")


# 12 rows (grouped GEMM) and 18 rows (prefill GEMM): x rows found through
# the broadcast lhs and the row within M on both
@pytest.mark.parametrize("M", [2, 3])
def test_gather_qmm_broadcast_and_m_rows(gpu, fmx, oracle, M):
    rng = np.random.default_rng(13)
    E, N, K, n_x = 5, 64, 256, 4
    x, rq, rs, rb = _gather_case(rng, oracle, E, N, K, n_x, M)
    lhs = np.array([[3], [0]], dtype=np.int32)          # [2,1]
    rhs = np.array([[4, 1, 1]], dtype=np.uint32)         # [1,3]
    import torch
    out = fmx.gather_qmm(to_dev(x), to_dev_u32(rq), to_dev(rs), to_dev(rb),
                         lhs_indices=torch.from_numpy(lhs).cuda(), rhs_indices=to_dev_u32(rhs))
    assert tuple(out.shape) == (2, 3, M, N)
    L = np.broadcast_to(lhs, (2, 3)).reshape(-1).astype(np.uint32)
    R = np.broadcast_to(rhs, (2, 3)).reshape(-1)
    ref = oracle.gather_qmm(x, rq, rs, rb, L, R, oracle.ACC_A)
    assert_close(from_dev_bf16(out).reshape(6, M, N), ref, "gather broadcast")


@pytest.mark.parametrize("T,k,E,N,K,big", [(75, 4, 16, 256, 1024, False), (300, 2, 8, 128, 512, False),
                                           (40, 4, 8, 128, 512, True)])
def test_gather_qmm_prefill_unsorted(gpu, fmx, oracle, T, k, E, N, K, big):
    """switch_mlp's prefill call (model.cpp:681, :703) at prefill sizes: the
    rows sorted by expert into passes of the prefill GEMM and scattered back
    to their (token, slot) output rows; a skewed expert choice leaves
    experts with no rows and others with several passes. big: one token's
    row scaled by 2^17 (values beyond fp16's range: the exact path), checked
    to two bf16 ulps of each output row's largest value."""
    rng = np.random.default_rng(T * k + E)
    x, rq, rs, rb = _gather_case(rng, oracle, E, N, K, T, 1)
    if big:
        row = bf16_to_f32(x[7]) * np.float32(2.0 ** 17)
        x[7] = oracle.f32_to_bf16_array(row)
    p = np.exp(-np.arange(E) / (E / 4.0))
    p /= p.sum()
    inds = np.stack([rng.choice(E, k, replace=False, p=p) for _ in range(T)]).astype(np.uint32)
    out = fmx.gather_qmm(to_dev(x.reshape(T, 1, 1, K)), to_dev_u32(rq), to_dev(rs), to_dev(rb),
                         rhs_indices=to_dev_u32(inds))
    assert tuple(out.shape) == (T, k, 1, N)
    lhs = np.repeat(np.arange(T, dtype=np.uint32), k)
    ref = oracle.gather_qmm(x, rq, rs, rb, lhs, inds.reshape(-1), oracle.ACC_A)
    check = assert_close_rows if big else assert_close
    check(from_dev_bf16(out).reshape(-1, 1, N), ref, "gather prefill")


@pytest.mark.parametrize("case", ["decode_8x4_unsorted", "prefill_2048_sorted"])
def test_gather_qmm_timed_shapes(gpu, fmx, oracle, case):
    """The calls the benchmark times, at their full size: switch_mlp's gate
    projection of the Qwen1.5-MoE-A2.7B shape (E 60, N 1408, K 2048) for 8
    tokens x top-4 unsorted (model.cpp:703, the grouped GEMM) and for 2048
    sorted rows (:686-706, the prefill GEMM in its MLX mode). Weights from
    the device generator and quantizer (the quantizer is bit-exact against
    the oracle's), copied to the host for the oracle. Every output row of
    the decode call and every 4th row of the prefill call (512 rows, all 60
    experts' segments) against the oracle; the whole prefill output finite."""
    import torch
    E, N, K, k = 60, 1408, 2048, 4
    w = fmx.synth_normal_bf16_device((E, N, K), 11, 60, 0.0, 0.02)
    wq, ws, wb = fmx.quantize(w)
    del w
    hq = wq.cpu().numpy().view(np.uint32)
    hs, hb = from_dev_bf16(ws), from_dev_bf16(wb)
    rng = np.random.default_rng(77)
    if case.startswith("decode"):
        B = 8
        x = _rand_bf16(rng, (B, 1, K))
        inds = np.stack([rng.permutation(E)[:k] for _ in range(B)]).astype(np.uint32)
        out = fmx.gather_qmm(to_dev(x.reshape(B, 1, 1, 1, K)), wq, ws, wb,
                             rhs_indices=to_dev_u32(inds.reshape(B, 1, k)))
        assert tuple(out.shape) == (B, 1, k, 1, N)
        ref = oracle.gather_qmm(x, hq, hs, hb, np.repeat(np.arange(B, dtype=np.uint32), k), inds.reshape(-1),
                                oracle.ACC_A)
        assert_close(from_dev_bf16(out).reshape(-1, 1, N), ref, "gather_qmm 8x4")
    else:
        n = 2048
        x = _rand_bf16(rng, (n, 1, K))
        idx = np.sort(rng.integers(0, E, n)).astype(np.uint32)
        out = fmx.gather_qmm(to_dev(x), wq, ws, wb, rhs_indices=to_dev_u32(idx), sorted_indices=True)
        assert tuple(out.shape) == (n, 1, N)
        assert bool(torch.isfinite(out.float()).all())
        rows = np.arange(0, n, 4, dtype=np.uint32)
        ref = oracle.gather_qmm(x, hq, hs, hb, rows, idx[rows], oracle.ACC_A)
        assert_close(from_dev_bf16(out)[rows], ref, "gather_qmm 2048 sorted")


def test_gather_qmm_defaults_one_hot(gpu, fmx, oracle):
    """No index arrays: out[e] = x[e] . W[e]^T, i.e. E independent quantized_matmuls."""
    rng = np.random.default_rng(14)
    E, N, K, M = 3, 48, 128, 2
    x, rq, rs, rb = _gather_case(rng, oracle, E, N, K, E, M)
    out = from_dev_bf16(fmx.gather_qmm(to_dev(x), to_dev_u32(rq), to_dev(rs), to_dev(rb)))
    for e in range(E):
        assert_close(out[e], oracle.qmm_t(x[e], rq[e], rs[e], rb[e], oracle.ACC_A), f"one-hot {e}")


def test_unsupported_arguments(gpu, fmx, oracle):
    rng = np.random.default_rng(15)
    x = _rand_bf16(rng, (1, 128))
    w = _rand_bf16(rng, (16, 128), 0.02)
    rq, rs, rb = oracle.quantize(w)
    args = (to_dev(x), to_dev_u32(rq), to_dev(rs), to_dev(rb))
    for kw in (dict(bits=8), dict(group_size=32), dict(transpose=False), dict(mode="mxfp4")):
        with pytest.raises(fmx.FmxError, match="UNSUPPORTED"):
            fmx.quantized_matmul(*args, **kw)


@pytest.mark.parametrize("T,E,k,norm,H,bias", [(1, 60, 4, False, 2048, False),
                                                (8, 128, 8, True, 2048, False),
                                                (77, 60, 4, False, 2048, True),
                                                (300, 128, 8, True, 512, False),
                                                (5, 1024, 16, True, 128, False)])
def test_router_bitexact(gpu, fmx, oracle, T, E, k, norm, H, bias):
    rng = np.random.default_rng(T + E + k)
    x = _rand_bf16(rng, (T, H))
    wr = _rand_bf16(rng, (E, H), 0.02)
    lb = _rand_bf16(rng, (E,)) if bias else None
    cfg = fmx.MoEConfig(hidden_size=H, num_experts=E, num_experts_per_tok=k,
                        moe_intermediate_size=64, norm_topk_prob=norm)
    inds, scores, probs = fmx.router_topk(cfg, to_dev(x), to_dev(wr),
                                          None if lb is None else to_dev(lb))
    _, rp, ri, rsc = oracle.router_topk(x, wr, k, norm, lb)
    np.testing.assert_array_equal(from_dev_bf16(probs), rp)
    np.testing.assert_array_equal(from_dev_u32(inds), ri)
    np.testing.assert_array_equal(from_dev_bf16(scores), rsc)


@pytest.mark.parametrize("T,E,k,norm,H,qr,qg", [(1, 60, 4, False, 2048, True, True),
                                                 (8, 60, 4, False, 2048, True, False),
                                                 (8, 128, 8, True, 2048, True, True),
                                                 (40, 60, 4, False, 2048, False, True),
                                                 (300, 128, 8, True, 512, True, True)])
def test_router_topk_ex_bitexact(gpu, fmx, oracle, T, E, k, norm, H, qr, qg):
    """fmx_moe_router_topk_ex: the router quantized (model.cpp:758-760) or
    bf16 (:762), and the shared-expert gate (:787-803) quantized or bf16.
    inds, scores and probs bit-exact against the oracle's router; the gate
    equals bf16(sigmoid(v)) of the oracle's exactly rounded logit v, with the
    sigmoid taken by numpy in float64."""
    rng = np.random.default_rng(1000 + T + E + k)
    x = _rand_bf16(rng, (T, H))
    wr = _rand_bf16(rng, (E, H), 0.02)
    wsg = _rand_bf16(rng, (1, H), 0.02)
    rq = oracle.quantize(wr) if qr else None
    gq = oracle.quantize(wsg) if qg else None
    cfg = fmx.MoEConfig(hidden_size=H, num_experts=E, num_experts_per_tok=k,
                        moe_intermediate_size=64, norm_topk_prob=norm)
    dev_r = fmx.QWeight(to_dev_u32(rq[0]), to_dev(rq[1]), to_dev(rq[2])) if qr else to_dev(wr)
    dev_g = fmx.QWeight(to_dev_u32(gq[0]), to_dev(gq[1]), to_dev(gq[2])) if qg else to_dev(wsg)
    inds, scores, probs, sg = fmx.router_topk(cfg, to_dev(x), dev_r, shared_expert_gate_w=dev_g)
    _, rp, ri, rsc = oracle.router_topk(x, rq if qr else wr, k, norm)
    np.testing.assert_array_equal(from_dev_bf16(probs), rp)
    np.testing.assert_array_equal(from_dev_u32(inds), ri)
    np.testing.assert_array_equal(from_dev_bf16(scores), rsc)
    glog, _, _, _ = oracle.router_topk(x, gq if qg else wsg, 1)
    v = bf16_to_f32(glog[:, 0]).astype(np.float64)
    want = oracle.f64_to_bf16(1.0 / (1.0 + np.exp(-v)))
    np.testing.assert_array_equal(from_dev_bf16(sg), want)
    # the bf16-router form through the same entry point equals fmx_moe_router_topk
    if not qr:
        i2, s2, p2 = fmx.router_topk(cfg, to_dev(x), to_dev(wr))
        np.testing.assert_array_equal(from_dev_u32(i2), from_dev_u32(inds))
        np.testing.assert_array_equal(from_dev_bf16(p2), from_dev_bf16(probs))


# (10001, 4, 60) and (8192, 8, 128): 40,004 and 65,536 entries, beyond the
# 32,768 keys the sort holds in LDS (the rest are re-read from memory)
@pytest.mark.parametrize("T,k,E", [(1, 4, 60), (8, 8, 128), (512, 4, 60), (1024, 8, 128),
                                   (33, 3, 5), (4096, 8, 128), (10001, 4, 60), (8192, 8, 128)])
def test_sort_bitexact(gpu, fmx, oracle, T, k, E):
    rng = np.random.default_rng(T * k + E)
    if T % 2:  # arbitrary keys, repeats allowed within a row
        inds = rng.integers(0, E, (T, k)).astype(np.uint32)
    else:      # distinct experts per token, skewed toward low ids
        p = np.exp(-np.arange(E) / (E / 6.0))
        p /= p.sum()
        inds = np.stack([rng.choice(E, k, replace=False, p=p) for _ in range(T)]).astype(np.uint32)
    order, inv, src, idx, offs = fmx.moe_sort(to_dev_u32(inds), E)
    ro, ri, rsrc, ridx, roff = oracle.moe_sort(inds, E)
    np.testing.assert_array_equal(from_dev_u32(order), ro)
    np.testing.assert_array_equal(from_dev_u32(inv), ri)
    np.testing.assert_array_equal(from_dev_u32(src), rsrc)
    np.testing.assert_array_equal(from_dev_u32(idx), ridx)
    np.testing.assert_array_equal(from_dev_u32(offs), roff)
    np.testing.assert_array_equal(ro, np.argsort(inds.reshape(-1), kind="stable"))


def test_empty_inputs(gpu, fmx, oracle):
    """Zero rows in, zero rows out, no error: quantized_matmul with M = 0 and
    gather_qmm with no index entries (MLX accepts empty arrays the same way)."""
    rng = np.random.default_rng(21)
    K, N, E = 256, 64, 4
    w = _rand_bf16(rng, (N, K), 0.02)
    rq, rs, rb = oracle.quantize(w)
    out = fmx.quantized_matmul(to_dev(np.zeros((0, K), np.uint16)), to_dev_u32(rq), to_dev(rs), to_dev(rb))
    assert tuple(out.shape) == (0, N)
    we = _rand_bf16(rng, (E, N, K), 0.02)
    eq, es, eb = oracle.quantize(we)
    out = fmx.gather_qmm(to_dev(np.zeros((0, 1, K), np.uint16)), to_dev_u32(eq), to_dev(es), to_dev(eb),
                         rhs_indices=to_dev_u32(np.zeros((0,), np.uint32)), sorted_indices=True)
    assert tuple(out.shape) == (0, 1, N)


def test_stack_experts(gpu, fmx, oracle):
    """fmx_stack_experts (mx::stack of per-expert arrays, model.cpp:396-404)
    places expert e's bytes at e * bytes, for every component of a layer."""
    import ctypes as C
    import torch
    from flashmlx_amd import _lib
    lib = _lib.load()
    rng = np.random.default_rng(31)
    E, N, K = 6, 40, 256
    per = [_rand_bf16(rng, (N, K), 0.02) for _ in range(E)]
    parts = [oracle.quantize(w) for w in per]
    for comp, dt in ((0, np.uint32), (1, np.uint16), (2, np.uint16)):
        devs = [to_dev_u32(p[comp]) if dt == np.uint32 else to_dev(p[comp]) for p in parts]
        nbytes = devs[0].numel() * devs[0].element_size()
        dst = torch.empty(E * nbytes, dtype=torch.uint8, device="cuda")
        ptrs = (C.c_void_p * E)(*[d.data_ptr() for d in devs])
        _lib.check(lib.fmx_stack_experts(ptrs, E, nbytes, dst.data_ptr(),
                                         torch.cuda.current_stream().cuda_stream))
        got = dst.cpu().numpy()
        ref = np.stack([p[comp] for p in parts]).view(np.uint8).reshape(-1)
        np.testing.assert_array_equal(got, ref)
    # a NULL source is an argument error
    ptrs = (C.c_void_p * 2)(devs[0].data_ptr(), None)
    assert lib.fmx_stack_experts(ptrs, 2, 16, dst.data_ptr(), None) == _lib.FMX_ERR_ARG


@pytest.mark.parametrize("n,seed,stream,mean,std", [(1 << 24, 2, 10, 0.0, 0.02), (1 << 20, 5, 1, 0.0, 1.0),
                                                    (100_003, 3, 3, 0.5, 0.02)])
def test_device_synth_matches_host(gpu, fmx, oracle, n, seed, stream, mean, std):
    """fmx_synth_normal_bf16_device writes the host generator's values (the
    bench and the decoder stack generate their multi-GB weight sets with it)."""
    import torch
    d = fmx.synth_normal_bf16_device((n,), seed, stream, mean, std)
    torch.cuda.synchronize()
    h = fmx.synth_normal_bf16(n, seed, stream, mean, std)
    np.testing.assert_array_equal(from_dev_bf16(d), h)


# ---------------------------------------------------------------- float16 activations

def _f16_case(rng, oracle, shape_w, shape_x):
    """float16 x and the oracle's quantization of w with its bf16 scales and
    biases re-encoded as float16 (the same values: bf16 values in fp16 range)."""
    w = _rand_bf16(rng, shape_w, 0.02)
    rq, rs, rb = oracle.quantize(w)
    to16 = lambda u: bf16_to_f32(u).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(shape_x).astype(np.float16).view(np.uint16)
    return x, rq, to16(rs), to16(rb)


def _to_dev_f16(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.float16)


def _f16_close(got_u16, ref_u16, what):
    g = got_u16.view(np.float16).astype(np.float64)
    r = ref_u16.view(np.float16).astype(np.float64)
    assert np.isfinite(g).all(), what
    bad = np.abs(g - r) > 1e-2 + 2e-2 * np.abs(r)
    assert not bad.any(), f"{what}: {int(bad.sum())} elements outside rtol/atol"
    l2 = np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30)
    assert l2 <= 1e-2, f"{what}: relative L2 {l2:.3g}"


@pytest.mark.parametrize("M,N,K", [(1, 64, 256), (5, 2048, 5632), (37, 96, 768), (512, 256, 1024)])
def test_quantized_matmul_f16(gpu, fmx, oracle, M, N, K):
    """float16 x, scales, biases and output (a float16 checkpoint's
    activations, model.cpp:208-214) against the oracle's float16 form; every
    row count runs the prefill GEMM in its float16 mode."""
    import torch
    rng = np.random.default_rng(M + N + K + 16)
    x, rq, s, b = _f16_case(rng, oracle, (N, K), (M, K))
    out = fmx.quantized_matmul(_to_dev_f16(x), to_dev_u32(rq), _to_dev_f16(s), _to_dev_f16(b))
    assert out.dtype == torch.float16
    got = out.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    _f16_close(got, oracle.qmm_t_f16(x, rq, s, b, oracle.ACC_A), f"qmm f16 M={M} N={N} K={K}")


@pytest.mark.parametrize("T,k,E,N,K", [(6, 4, 8, 128, 512), (75, 4, 16, 256, 1024)])
def test_gather_qmm_f16(gpu, fmx, oracle, T, k, E, N, K):
    import torch
    rng = np.random.default_rng(T * k + E + 16)
    x, rq, s, b = _f16_case(rng, oracle, (E, N, K), (T, 1, K))
    inds = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.uint32)
    out = fmx.gather_qmm(_to_dev_f16(x.reshape(T, 1, 1, K)), to_dev_u32(rq), _to_dev_f16(s), _to_dev_f16(b),
                         rhs_indices=to_dev_u32(inds))
    assert tuple(out.shape) == (T, k, 1, N) and out.dtype == torch.float16
    got = out.contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1, 1, N)
    ref = oracle.gather_qmm_f16(x, rq, s, b, np.repeat(np.arange(T, dtype=np.uint32), k), inds.reshape(-1),
                                oracle.ACC_A)
    _f16_close(got, ref, f"gather f16 T={T}")


def test_f16_shapes_outside_the_gemm(gpu, fmx, oracle):
    """float16 needs whole 128-k units and 16-row tiles: K % 128 == 64 is
    refused (no bfloat16 fallback for float16 operands); mixed dtypes too."""
    rng = np.random.default_rng(17)
    x, rq, s, b = _f16_case(rng, oracle, (64, 1344), (3, 1344))
    with pytest.raises(fmx.FmxError, match="UNSUPPORTED"):
        fmx.quantized_matmul(_to_dev_f16(x), to_dev_u32(rq), _to_dev_f16(s), _to_dev_f16(b))
    x, rq, s, b = _f16_case(rng, oracle, (64, 256), (3, 256))
    with pytest.raises(fmx.FmxError, match="DTYPE"):
        fmx.quantized_matmul(_to_dev_f16(x), to_dev_u32(rq), to_dev(np.zeros_like(s)), _to_dev_f16(b))
