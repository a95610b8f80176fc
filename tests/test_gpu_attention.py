"""Single-token decode attention (fmx_attention_decode: RoPE of q and the new
key, the KV-cache append and scaled dot-product attention over the cache,
model.cpp:874-884) against the oracle (orc_rope + orc_sdpa_split), at key
counts on both sides of every range-count boundary of the split kernel (one
range up to 32 keys, 16 from 481, ranges longer than one 32-key round
beyond 512), for MHA and GQA head layouts, with a dominant early key in
some sequences (the later ranges' sums then carry f_s << 1)."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import bf16_to_f32, from_dev_bf16, to_dev

pytestmark = pytest.mark.gpu

POSITIONS = [0, 1, 30, 31, 32, 33, 63, 64, 65, 299, 480, 481, 511, 512, 513, 700, 1535]


def _bf16(oracle, a):
    return oracle.f32_to_bf16_array(np.asarray(a, dtype=np.float32))


def _rand_bf16(rng, shape):
    """N(0, 1) samples truncated to bf16 (any bf16 values serve as inputs)."""
    return (rng.standard_normal(shape, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


@pytest.mark.parametrize("nh,nkv,hd", [(16, 16, 128), (4, 2, 64), (8, 1, 32)])
def test_attention_decode_matches_oracle(gpu, fmx, oracle, nh, nkv, hd):
    import torch
    from flashmlx_amd import _lib

    lib = _lib.load()
    rng = np.random.default_rng(nh * 1000 + hd)
    B, max_seq, theta = len(POSITIONS), 1536, 1e4
    width = (nh + 2 * nkv) * hd
    qkv = _rand_bf16(rng, (B, width))
    kc = _rand_bf16(rng, (B, nkv, max_seq, hd))
    vc = _rand_bf16(rng, (B, nkv, max_seq, hd))
    cs = oracle.rope_table(max_seq, hd, theta)
    rep = nh // nkv
    for b, p in enumerate(POSITIONS):  # key 0 of every kv group 3x its first q head, rotated
        if p >= 64 and b % 2 == 0:
            qr = oracle.rope(qkv[b, :nh * hd].reshape(1, nh, hd), [p], cs)[0]
            for g in range(nkv):
                kc[b, g, 0] = _bf16(oracle, 3.0 * bf16_to_f32(qr[g * rep]))
    scale = float(np.float32(1.0 / np.sqrt(hd)))

    stream = torch.cuda.current_stream().cuda_stream
    cs_d = torch.empty((max_seq, hd // 2, 2), dtype=torch.float32, device="cuda")
    _lib.check(lib.fmx_rope_table(cs_d.data_ptr(), max_seq, hd, theta, stream))
    np.testing.assert_array_equal(cs_d.cpu().numpy(), cs)  # the same fp64 formula, one rounding
    qkv_d, kc_d, vc_d = to_dev(qkv), to_dev(kc), to_dev(vc)
    offs = torch.tensor(POSITIONS, dtype=torch.int32, device="cuda")
    out_d = torch.empty((B, nh * hd), dtype=torch.bfloat16, device="cuda")
    _lib.check(lib.fmx_attention_decode(qkv_d.data_ptr(), B, nh, nkv, hd, cs_d.data_ptr(), kc_d.data_ptr(),
                                        vc_d.data_ptr(), max_seq, offs.data_ptr(), scale, out_d.data_ptr(),
                                        stream))
    torch.cuda.synchronize()
    out = from_dev_bf16(out_d)
    kc_g, vc_g = from_dev_bf16(kc_d), from_dev_bf16(vc_d)

    for b, p in enumerate(POSITIONS):
        q = qkv[b, :nh * hd].reshape(1, nh, hd)
        k = qkv[b, nh * hd:(nh + nkv) * hd].reshape(1, nkv, hd)
        v = qkv[b, (nh + nkv) * hd:].reshape(nkv, hd)
        qr = oracle.rope(q, [p], cs)
        kr = oracle.rope(k, [p], cs)[0]
        kref, vref = kc[b].copy(), vc[b].copy()
        kref[:, p], vref[:, p] = kr, v
        np.testing.assert_array_equal(kc_g[b, :, p], kr, err_msg=f"position {p}: cached key")
        np.testing.assert_array_equal(vc_g[b, :, p], v, err_msg=f"position {p}: cached value")
        want = oracle.sdpa_split(qr, kref, vref, p, scale).reshape(-1)
        got = out[b]
        if not np.array_equal(got, want):
            g, w = bf16_to_f32(got).astype(np.float64), bf16_to_f32(want).astype(np.float64)
            bad = np.flatnonzero(got != want)
            raise AssertionError(
                f"position {p} (nh {nh}, nkv {nkv}, hd {hd}): {bad.size} of {got.size} outputs differ "
                f"from the oracle, max abs {np.abs(g - w).max():.3g}, first at {bad[:8].tolist()}")
    # other cache positions untouched
    mask = np.ones((B, max_seq), bool)
    mask[np.arange(B), POSITIONS] = False
    np.testing.assert_array_equal(kc_g.transpose(0, 2, 1, 3)[mask], kc.transpose(0, 2, 1, 3)[mask])
    np.testing.assert_array_equal(vc_g.transpose(0, 2, 1, 3)[mask], vc.transpose(0, 2, 1, 3)[mask])


def test_attention_decode_rejects_unsupported(gpu, fmx):
    """Head sizes the split kernel does not take and caches beyond its LDS
    bound are refused, not computed."""
    from flashmlx_amd import _lib

    lib = _lib.load()
    assert lib.fmx_attention_decode(1, 1, 2, 1, 256, 1, 1, 1, 64, 1, 0.1, 1, None) == _lib.FMX_ERR_UNSUPPORTED
    assert lib.fmx_attention_decode(1, 1, 2, 1, 128, 1, 1, 1, 8192, 1, 0.1, 1, None) == _lib.FMX_ERR_UNSUPPORTED
    assert lib.fmx_attention_decode(1, 1, 3, 2, 128, 1, 1, 1, 64, 1, 0.1, 1, None) == _lib.FMX_ERR_SHAPE
