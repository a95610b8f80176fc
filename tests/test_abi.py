"""The C-ABI library without a GPU: it loads, exports every entry point that
include/*.h declares, and its host-side logic (size queries, argument
validation, status strings, the seeded generator) behaves. No call here
launches a kernel."""
from __future__ import annotations

import ctypes as C
import pathlib
import re

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


def header_functions() -> list[str]:
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(re.findall(r"\b(fmx_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol(fmx):
    from flashmlx_amd import _lib
    lib = _lib.load()
    names = header_functions()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding declares a signature for each of them
    assert sorted(_lib.EXPORTED) == names


def test_missing_library_fails_loudly(tmp_path):
    from flashmlx_amd import _lib
    with pytest.raises(ImportError):
        _lib.load(tmp_path / "libfmx.so")


def test_status_strings_and_version(fmx):
    from flashmlx_amd import _lib
    lib = _lib.load()
    assert lib.fmx_abi_version() >= 1
    for code, name in _lib.STATUS_NAMES.items():
        assert lib.fmx_status_string(code).decode() == name
    assert lib.fmx_status_string(99).decode() == "FMX_ERR_UNKNOWN"


def _arr(shape, dtype, data=None):
    from flashmlx_amd import _lib
    a = _lib.FmxArray()
    a.data = data
    a.dtype = dtype
    a.ndim = len(shape)
    for i, s in enumerate(shape):
        a.shape[i] = s
    return a


def test_quantized_matmul_validation(fmx):
    """Arguments outside scope or inconsistent are rejected before any HIP call."""
    from flashmlx_amd import _lib
    lib = _lib.load()
    buf = np.zeros(1 << 16, np.uint8)
    p = (buf.ctypes.data + 255) // 256 * 256     # aligned host address; never dereferenced
    x, w = _arr([4, 256], _lib.FMX_BF16, p), _arr([64, 32], _lib.FMX_U32, p)
    s, b = _arr([64, 4], _lib.FMX_BF16, p), _arr([64, 4], _lib.FMX_BF16, p)
    out = _arr([4, 64], _lib.FMX_BF16, p)
    R = C.byref
    call = lambda **kw: lib.fmx_quantized_matmul(  # noqa: E731
        R(kw.get("x", x)), R(w), R(s), R(b), kw.get("t", 1), kw.get("g", 64), kw.get("bits", 4),
        kw.get("mode", b"affine"), R(out), None, 0, None)
    assert call(bits=8) == _lib.FMX_ERR_UNSUPPORTED
    assert b"bits=8" in lib.fmx_last_error()
    assert call(g=32) == _lib.FMX_ERR_UNSUPPORTED
    assert call(t=0) == _lib.FMX_ERR_UNSUPPORTED
    assert call(mode=b"mxfp4") == _lib.FMX_ERR_UNSUPPORTED
    assert call(x=_arr([4, 256], _lib.FMX_F32, p)) == _lib.FMX_ERR_DTYPE
    assert call(x=_arr([4, 128], _lib.FMX_BF16, p)) == _lib.FMX_ERR_SHAPE
    assert call(x=_arr([4, 256], _lib.FMX_BF16, p + 2)) == _lib.FMX_ERR_ARG
    o = _lib.FmxArray()
    assert lib.fmx_quantized_matmul_out_shape(R(_arr([2, 3, 256], 0, p)), R(w), 1, 64, 4, R(o)) == 0
    assert o.ndim == 3 and list(o.shape[:3]) == [2, 3, 64]


def test_gather_qmm_out_shape_broadcasts(fmx):
    from flashmlx_amd import _lib
    lib = _lib.load()
    x = _arr([5, 1, 1, 256], _lib.FMX_BF16)     # batch (5, 1), M = 1
    w = _arr([8, 96, 32], _lib.FMX_U32)
    rhs = _arr([5, 4], _lib.FMX_U32)
    o = _lib.FmxArray()
    rc = lib.fmx_gather_qmm_out_shape(C.byref(x), C.byref(w), None, C.byref(rhs), 1, 64, 4, C.byref(o))
    assert rc == 0, lib.fmx_last_error()
    assert list(o.shape[:o.ndim]) == [5, 4, 1, 96]


def test_moe_workspace_sizes(fmx):
    from flashmlx_amd import MoEConfig
    from flashmlx_amd import _lib
    lib = _lib.load()
    q15 = MoEConfig(2048, 60, 4, 1408, 5632, False).to_c()
    q3 = MoEConfig(2048, 128, 8, 768, 0, True).to_c()
    s1 = lib.fmx_moe_workspace_size(C.byref(q15), 1)
    s512 = lib.fmx_moe_workspace_size(C.byref(q15), 512)
    assert 0 < s1 < s512 < (1 << 31)
    assert lib.fmx_moe_workspace_size(C.byref(q3), 1024) > 0
    assert lib.fmx_moe_workspace_size(C.byref(q3), 65537) == 0        # above the token limit
    bad = MoEConfig(2048, 60, 4, 1408, 5632, False, quant_bits=8).to_c()
    assert lib.fmx_moe_workspace_size(C.byref(bad), 8) == 0
    odd = MoEConfig(2000, 60, 4, 1408, 5632, False).to_c()             # H not a multiple of 64
    assert lib.fmx_moe_workspace_size(C.byref(odd), 8) == 0
    topk = MoEConfig(2048, 8, 9, 1408, 0, False).to_c()                # k > E
    assert lib.fmx_moe_workspace_size(C.byref(topk), 8) == 0


def test_forward_path_per_shape(fmx):
    """Decode kernels up to 16 tokens on packed weights, the packed prefill
    GEMMs above, the MLX-layout GEMMs without packing or for shapes the
    packed layout cannot hold (a K that is not a multiple of 128)."""
    from flashmlx_amd import workloads as W
    assert W.forward_path(W.QWEN15, 1) == "decode"
    assert W.forward_path(W.QWEN15, 16) == "decode"
    assert W.forward_path(W.QWEN15, 17) == "prefill"
    assert W.forward_path(W.QWEN15, 512) == "prefill"
    assert W.forward_path(W.QWEN15, 512, packed=False) == "general"
    assert W.forward_path(W.QWEN3, 8) == "decode"
    assert W.forward_path(W.QWEN3, 1024) == "prefill"
    assert W.forward_path(W.SMALL, 23) == "prefill"
    assert W.forward_path(W.TINY, 40) == "general"        # shared_inter 192
    assert W.forward_path(W.TINY_NORM, 33) == "general"   # hidden 320


def test_synth_is_counter_based(fmx):
    """Each value is a pure function of (seed, stream, index): prefixes agree,
    streams and seeds differ, moments are those of N(mean, std)."""
    from flashmlx_amd import synth_normal_bf16
    a = synth_normal_bf16(1 << 20, 7, 3)
    b = synth_normal_bf16(1000, 7, 3)
    np.testing.assert_array_equal(a[:1000], b)
    assert not np.array_equal(synth_normal_bf16(1000, 7, 4), b)
    assert not np.array_equal(synth_normal_bf16(1000, 8, 3), b)
    f = (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    assert abs(f.mean()) < 5e-3 and abs(f.std() - 1) < 5e-3
    assert abs((np.abs(f) < 1).mean() - 0.6827) < 3e-3
    g = (synth_normal_bf16(1 << 18, 1, 1, 0.5, 0.02).astype(np.uint32) << 16).view(np.float32)
    assert abs(g.mean() - 0.5) < 1e-3 and abs(g.std() - 0.02) < 1e-3


def test_workload_bytes_match_published_figure():
    """Algorithmic bytes of one Qwen1.5 decode B=1 call with 4 unique experts:
    4 x 4,866,048 + 19,464,192 + 245,760 + 4,096 + 8,192 = 39,186,432."""
    from flashmlx_amd import workloads as W
    assert W.algorithmic_bytes(W.QWEN15, 1, 4) == 39_186_432
    assert W.algorithmic_bytes(W.QWEN3, 1, 8) == 21_766_144
    assert W.flops(W.QWEN15, 512) == 70_994_886_656
    assert W.flops(W.QWEN3, 1024) == 77_846_282_240


def test_zero_token_calls_need_no_buffers(fmx):
    """n_tokens = 0 runs nothing and returns FMX_OK even with NULL x / y /
    outputs (empty tensors have no storage); one token with a NULL x is an
    argument error, reported before any device call."""
    from flashmlx_amd import MoEConfig
    from flashmlx_amd import _lib
    lib = _lib.load()
    cfg = MoEConfig(2048, 60, 4, 1408, 5632, False).to_c()
    w = _lib.FmxMoEWeights()
    ws = (C.c_uint8 * 256)()
    fwd = lib.fmx_moe_block_forward
    assert fwd(C.byref(cfg), C.byref(w), None, 0, None, ws, 256, None) == _lib.FMX_OK
    assert fwd(C.byref(cfg), C.byref(w), None, 1, None, ws, 256, None) == _lib.FMX_ERR_ARG
    rt = lib.fmx_moe_router_topk
    assert rt(C.byref(cfg), None, 0, None, None, None, None, None, ws, 256, None) == _lib.FMX_OK
    assert rt(C.byref(cfg), None, 1, None, None, None, None, None, ws, 256, None) == _lib.FMX_ERR_ARG


def test_moe_workspace_size_nondecreasing(fmx):
    """A workspace sized for max_tokens serves every smaller forward: the
    size query never shrinks as the token count grows (the decode kernels'
    products are held for min(T, 16) tokens at every T)."""
    from flashmlx_amd import MoEConfig
    from flashmlx_amd import _lib
    lib = _lib.load()
    for cfg in (MoEConfig(2048, 60, 4, 1408, 5632, False), MoEConfig(2048, 128, 8, 768, 0, True),
                MoEConfig(512, 8, 2, 256, 512, False)):
        c = cfg.to_c()
        sizes = [lib.fmx_moe_workspace_size(C.byref(c), t)
                 for t in list(range(0, 65)) + [100, 512, 1024, 4096, 65536]]
        assert all(s > 0 for s in sizes)
        assert all(b >= a for a, b in zip(sizes, sizes[1:])), sizes


def test_decode_wait_limit_hook(fmx):
    """The bound of the decode kernels' wait: set, 0 (give up at once) and
    the default restored by a negative value; each call returns the bound
    it replaced. Host state only; status reads need no kernel either way."""
    from flashmlx_amd import _lib
    lib = _lib.load()
    default = 1 << 21
    assert lib.fmx_set_decode_wait_limit(5) == default
    assert lib.fmx_set_decode_wait_limit(0) == 5
    assert lib.fmx_set_decode_wait_limit(-1) == 0
    assert lib.fmx_set_decode_wait_limit(-1) == default
    st = C.c_uint32()
    assert lib.fmx_moe_workspace_status(None, 0, C.byref(st), 0, None) == _lib.FMX_ERR_ARG
    ws = (C.c_uint8 * 256)()
    assert lib.fmx_moe_workspace_status(ws, 256, C.byref(st), 0, None) == _lib.FMX_ERR_WORKSPACE


def test_packed_forward_arguments(fmx):
    """Packed forwards do not need the MLX-layout expert arrays, but the
    packed buffer must be 256-byte aligned and at least the config's packed
    size; a quantized router needs its biases. Each error is reported before
    any device call."""
    from flashmlx_amd import MoEConfig
    from flashmlx_amd import _lib
    lib = _lib.load()
    cfg = MoEConfig(2048, 60, 4, 1408, 5632, False).to_c()
    need = lib.fmx_moe_packed_size(C.byref(cfg))
    assert need > 0
    buf = np.zeros(1 << 16, np.uint8)
    p = (buf.ctypes.data + 255) // 256 * 256     # aligned host address; never dereferenced
    ws = np.zeros(1 << 16, np.uint8)
    wsp = (ws.ctypes.data + 255) // 256 * 256
    w = _lib.FmxMoEWeights()
    w.router_w = p
    w.shared_expert_gate_w = p
    w.packed = p
    w.packed_bytes = need - 256
    fwd = lib.fmx_moe_block_forward
    R = C.byref
    assert fwd(R(cfg), R(w), p, 1, p, wsp, 256, None) == _lib.FMX_ERR_WORKSPACE
    assert b"packed_bytes" in lib.fmx_last_error()
    w.packed_bytes = need
    w.packed = p + 16
    assert fwd(R(cfg), R(w), p, 1, p, wsp, 256, None) == _lib.FMX_ERR_ARG
    w.packed = p
    # a correctly described packed layer gets past validation without the
    # MLX-layout arrays: the next check is the (too small) workspace
    assert fwd(R(cfg), R(w), p, 1, p, wsp, 256, None) == _lib.FMX_ERR_WORKSPACE
    assert b"workspace" in lib.fmx_last_error()
    # quantized router: scales without biases is an argument error
    w.router_scales = p
    assert fwd(R(cfg), R(w), p, 1, p, wsp, 256, None) == _lib.FMX_ERR_ARG
    w.router_biases = p
    assert fwd(R(cfg), R(w), p, 1, p, wsp, 256, None) == _lib.FMX_ERR_WORKSPACE
    # unpacked forwards still need every expert array
    w.packed = None
    w.packed_bytes = 0
    assert fwd(R(cfg), R(w), p, 1, p, wsp, 256, None) == _lib.FMX_ERR_ARG
    assert b"expert weights" in lib.fmx_last_error()


def test_sort_limits(fmx):
    """The sort takes up to 2^22 entries and 1024 experts; a Qwen3 prefill
    of 65536 tokens (524,288 entries) fits, and gather_qmm states the same
    row limit."""
    from flashmlx_amd import _lib
    lib = _lib.load()
    assert lib.fmx_moe_sort_workspace_size(65536, 8, 128) > 0
    keys = np.zeros(16, np.uint32)   # host address; the calls below fail before using it
    k = keys.ctypes.data
    assert lib.fmx_moe_sort(k, 1, 8, 2048, None, None, None, None, None, None, 0, None) == \
        _lib.FMX_ERR_UNSUPPORTED
    assert lib.fmx_moe_sort(k, (1 << 22) // 8 + 1, 8, 128, None, None, None, None, None, None, 0,
                            None) == _lib.FMX_ERR_UNSUPPORTED
    assert b"limits" in lib.fmx_last_error()


def test_model_sizes_and_validation(fmx):
    """Decoder-stack entry points without a GPU: size queries for the
    Qwen1.5-MoE-A2.7B shape, packed sizes equal to MLX's 0.5625 bytes per
    weight, out-of-scope configs refused, and a forward with missing weights
    refused before any launch."""
    from flashmlx_amd import _lib
    from flashmlx_amd.model import ModelConfig
    lib = _lib.load()
    cfg = ModelConfig(max_position_embeddings=512)
    c = cfg.to_c()
    s1 = lib.fmx_model_workspace_size(C.byref(c), 1)
    s2 = lib.fmx_model_workspace_size(C.byref(c), 1028)
    assert 0 < s1 < s2
    assert lib.fmx_model_kv_cache_size(C.byref(c), 4, 384) == 24 * 2 * 4 * 16 * 384 * 128 * 2
    assert lib.fmx_packed_linear_size(6144, 2048) == 6144 * 2048 * 9 // 16
    assert lib.fmx_packed_linear_size(6144, 2000) == 0
    for bad in (ModelConfig(vocab_size=100), ModelConfig(num_key_value_heads=3),
                ModelConfig(max_position_embeddings=65536), ModelConfig(head_dim=100)):
        assert lib.fmx_model_workspace_size(C.byref(bad.to_c()), 1) == 0
    rc = lib.fmx_model_forward(C.byref(c), None, None, 1, 1, 0, None, None, 1, 1, 1, None, None, 0, None)
    assert rc == _lib.FMX_ERR_ARG
    w = _lib.FmxModelWeights()
    w.embed = w.norm_w = w.lm_head = 16
    w.layers = (_lib.FmxLayerWeights * 1)()
    # zero tokens: nothing runs
    assert lib.fmx_model_forward(C.byref(c), C.byref(w), None, 0, 5, 0, None, None, 1, 1, 1, None,
                                 None, 0, None) == _lib.FMX_OK
    # positions past the cache are refused on the host
    rc = lib.fmx_model_forward(C.byref(c), C.byref(w), 16, 1, 4, 380, None, 256, 1, 382, 1, 256,
                               256, 1 << 30, None)
    assert rc == _lib.FMX_ERR_SHAPE, lib.fmx_last_error()


def test_scheduler_validation(fmx):
    """Scheduler entry points without a GPU: pool shapes outside the limits
    and NULL handles are refused before any allocation."""
    from flashmlx_amd import _lib
    from flashmlx_amd.model import ModelConfig
    lib = _lib.load()
    c = ModelConfig(max_position_embeddings=512).to_c()
    w = _lib.FmxModelWeights()
    h = C.c_void_p()
    for n_slots, max_ctx, max_prompt in ((0, 64, 8), (257, 64, 8), (4, 8, 8), (4, 64, 0)):
        rc = lib.fmx_scheduler_create(C.byref(c), C.byref(w), n_slots, max_ctx, max_prompt, None, C.byref(h))
        assert rc == _lib.FMX_ERR_SHAPE, (n_slots, max_ctx, max_prompt)
        assert not h.value
    # a context beyond the attention kernel's cache limit
    rc = lib.fmx_scheduler_create(C.byref(c), C.byref(w), 4, 8192, 8, None, C.byref(h))
    assert rc == _lib.FMX_ERR_UNSUPPORTED
    assert lib.fmx_scheduler_create(None, C.byref(w), 4, 64, 8, None, C.byref(h)) == _lib.FMX_ERR_ARG
    assert lib.fmx_scheduler_has_work(None) == 0
    assert lib.fmx_scheduler_active_count(None) == 0
    n = C.c_int64()
    assert lib.fmx_scheduler_drain_completed(None, None, 0, C.byref(n)) == _lib.FMX_ERR_ARG
    p = (C.c_int32 * 1)(0)
    rid = C.c_int64()
    assert lib.fmx_scheduler_submit(None, p, 1, 1, 0.0, C.byref(rid)) == _lib.FMX_ERR_ARG
    ids = (C.c_int64 * 2)()
    toks = (C.c_int32 * 2)()
    assert lib.fmx_scheduler_step(None, ids, toks, 2, C.byref(n)) == _lib.FMX_ERR_ARG
    assert lib.fmx_scheduler_set_prefix_cache(None, 4) == _lib.FMX_ERR_ARG
    assert lib.fmx_scheduler_prefix_hits(None) == 0
    lib.fmx_scheduler_free(None)


def test_nemotron_sizes_and_validation(fmx):
    """Nemotron-H block entry points without a GPU: packed sizes with I and
    Is padded to whole 128-k units, configs outside the limits refused."""
    from flashmlx_amd import _lib
    from flashmlx_amd.nemotron import NhMoEConfig
    lib = _lib.load()
    cfg = NhMoEConfig()
    c = cfg.to_c()
    H, E, Ip, Isp = 2688, 128, 1920, 3712
    blocks = E * (Ip // 16) * (H // 128) + E * (H // 16) * (Ip // 128) + (Isp // 16) * (H // 128) \
        + (H // 16) * (Isp // 128)
    got = lib.fmx_nh_moe_packed_size(C.byref(c))
    assert blocks * 1152 <= got <= blocks * 1152 + 4 * 256
    assert 0 < lib.fmx_nh_moe_workspace_size(C.byref(c), 1) < lib.fmx_nh_moe_workspace_size(C.byref(c), 512)
    for bad in (NhMoEConfig(hidden_size=2700), NhMoEConfig(moe_intermediate_size=1850),
                NhMoEConfig(n_group=3), NhMoEConfig(n_group=4, topk_group=5),
                NhMoEConfig(num_experts_per_tok=17), NhMoEConfig(n_routed_experts=2048),
                NhMoEConfig(quant_bits=8), NhMoEConfig(n_group=128, topk_group=1)):
        assert lib.fmx_nh_moe_packed_size(C.byref(bad.to_c())) == 0
    w = _lib.FmxNhMoEWeights()
    assert lib.fmx_nh_moe_block_forward(C.byref(c), C.byref(w), None, 0, None, None, 0, None) == _lib.FMX_OK
    assert lib.fmx_nh_moe_block_forward(C.byref(c), None, None, 1, None, None, 0, None) == _lib.FMX_ERR_ARG
    for bad_n in (0, 5):
        assert lib.fmx_nh_moe_block_forward_partial(C.byref(c), C.byref(w), None, 0, None, None, 0, None,
                                                    bad_n) == _lib.FMX_ERR_ARG
    assert lib.fmx_nh_moe_block_forward_partial(C.byref(c), C.byref(w), None, 0, None, None, 0, None, 2) == _lib.FMX_OK
