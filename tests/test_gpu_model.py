"""GPU parity of the decoder stack (fmx_model_forward) against the CPU
oracle's DecoderStack: logits and the residual stream after the last layer
within the bf16 tolerance, greedy tokens equal (or, where they differ, a
near-tie of the oracle's own logits), KV-cache and batch invariants, and the
24-layer Qwen1.5-MoE-A2.7B-shape stack end to end."""
import numpy as np
import pytest

from helpers import assert_close_rows as assert_close, bf16_to_f32, errors, from_dev_bf16

pytestmark = pytest.mark.gpu


def _tiny_cfg(**kw):
    from flashmlx_amd.model import ModelConfig
    from flashmlx_amd.moe import MoEConfig
    H = kw.pop("H", 512)
    moe = MoEConfig(hidden_size=H, num_experts=8, num_experts_per_tok=2, moe_intermediate_size=256,
                    shared_expert_intermediate_size=512, norm_topk_prob=False)
    base = dict(hidden_size=H, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                vocab_size=256, max_position_embeddings=64, moe=moe)
    base.update(kw)
    return ModelConfig(**base)


def _build(cfg, seed, B, max_seq, max_tokens):
    import torch
    from flashmlx_amd import model as M
    w = M.synthetic_model(cfg, seed, keep_mlx=True)
    dm = M.DecoderModel(cfg, w, B, max_seq, max_tokens)
    torch.cuda.synchronize()
    return w, dm


def _ids(rng, B, L, V):
    import torch
    a = rng.integers(0, V, size=(B, L)).astype(np.int32)
    return a, torch.from_numpy(a).cuda()


# tiny stacks: GQA (4 heads on 2 kv heads, hd 128) and MHA with hd 64
@pytest.mark.parametrize("kw", [dict(), dict(num_attention_heads=8, num_key_value_heads=8)])
def test_stack_tiny_matches_oracle(gpu, fmx, oracle, kw):
    """Prefill of 2 x 12 tokens (the prefill GEMMs and the MoE prefill path),
    then 3 decode steps (decode kernels), against the oracle: every logit of
    the prefill, the residual stream, and each step's logits."""
    import torch
    from flashmlx_amd import model as M
    cfg = _tiny_cfg(**kw)
    B, L, max_seq = 2, 12, 32
    w, dm = _build(cfg, 31, B, max_seq, B * L)
    hw = M.host_weights(cfg, w)
    st = oracle.DecoderStack(M.oracle_config(cfg, max_seq), hw, B)
    rng = np.random.default_rng(7)
    ids, ids_d = _ids(rng, B, L, cfg.vocab_size)
    lg = from_dev_bf16(dm.forward(ids_d, 0, last_only=False)).reshape(B * L, -1)
    hid = from_dev_bf16(dm.hidden(B * L))
    torch.cuda.synchronize()
    rl, rh = st.forward(ids, 0, last_only=False, return_hidden=True)
    e = assert_close(hid, rh, "prefill residual stream")
    e2 = assert_close(lg, rl, "prefill logits")
    print(f"tiny {kw}: hidden {e}, logits {e2}")
    for step in range(3):
        nxt, nxt_d = _ids(rng, B, 1, cfg.vocab_size)
        g = from_dev_bf16(dm.forward(nxt_d, L + step))
        torch.cuda.synchronize()
        r = st.forward(nxt, L + step)
        assert_close(g, r, f"decode step {step} logits")
    # the KV cache holds the oracle's keys and values (rotated keys)
    kc, vc = dm.kv_views()
    for li in range(cfg.num_hidden_layers):
        for b in range(B):
            n = L + 3
            got_k = from_dev_bf16(kc[li, b, :, :n].contiguous())
            got_v = from_dev_bf16(vc[li, b, :, :n].contiguous())
            assert_close(got_k, st.kc[li, b, :, :n], f"layer {li} seq {b} keys")
            assert_close(got_v, st.vc[li, b, :, :n], f"layer {li} seq {b} values")


def test_stack_tiny_single_sequence_decode(gpu, fmx, oracle):
    """One sequence (single-row decode steps: the q/k/v projection forms its
    input norm itself and the o projection adds the previous MoE output to
    the residual; attention in the split kernel's key ranges, a 70-token
    context spanning three ranges): each step's logits against the oracle, and
    the residual stream after a final prefill-path step."""
    import torch
    from flashmlx_amd import model as M
    cfg = _tiny_cfg(max_position_embeddings=128)
    B, L, max_seq = 1, 70, 80
    w, dm = _build(cfg, 33, B, max_seq, L)
    hw = M.host_weights(cfg, w)
    st = oracle.DecoderStack(M.oracle_config(cfg, max_seq), hw, B)
    rng = np.random.default_rng(9)
    ids, ids_d = _ids(rng, B, L, cfg.vocab_size)
    lg = from_dev_bf16(dm.forward(ids_d, 0))
    torch.cuda.synchronize()
    assert_close(lg, st.forward(ids, 0), "prefill logits")
    for step in range(4):
        nxt, nxt_d = _ids(rng, B, 1, cfg.vocab_size)
        g = from_dev_bf16(dm.forward(nxt_d, L + step))
        torch.cuda.synchronize()
        assert_close(g, st.forward(nxt, L + step), f"decode step {step} logits")


def test_stack_tiny_per_sequence_offsets(gpu, fmx, oracle):
    """Per-sequence device offsets (forward_heterogeneous): after a joint
    prefill, sequence 0 decodes at positions L, L+1, L+2 while sequence 1
    stays at L (its cache slot L rewritten each step); each matches its own
    oracle sequence. The device offsets advance through fmx_greedy_next."""
    import torch
    from flashmlx_amd import model as M
    cfg = _tiny_cfg()
    B, L, max_seq = 2, 10, 24
    w, dm = _build(cfg, 32, B, max_seq, B * L)
    hw = M.host_weights(cfg, w)
    oc = M.oracle_config(cfg, max_seq)
    rng = np.random.default_rng(8)
    ids, ids_d = _ids(rng, B, L, cfg.vocab_size)
    dm.forward(ids_d, 0)
    sts = [oracle.DecoderStack(oc, hw, 1) for _ in range(B)]
    for b in range(B):
        sts[b].forward(ids[b:b + 1], 0)
    offs = torch.tensor([L, L], dtype=torch.int32, device="cuda")
    pos = [L, L]
    tok = torch.empty(B, dtype=torch.int32, device="cuda")
    for step in range(3):
        nxt, nxt_d = _ids(rng, B, 1, cfg.vocab_size)
        g = dm.forward(nxt_d, offs)
        gh = from_dev_bf16(g)
        # advance sequence 0 only: ids are not used, the offsets are
        adv = torch.tensor([1, 0], dtype=torch.int32, device="cuda")
        dm.greedy(g, tok, offs, advance=1)
        offs -= 1 - adv
        torch.cuda.synchronize()
        for b in range(B):
            r = sts[b].forward(nxt[b:b + 1], pos[b])
            assert_close(gh[b:b + 1], r, f"step {step} seq {b}")
        pos[0] += 1
        assert offs.cpu().tolist() == pos


# The GPU and the oracle form the MoE block's input through different
# (equally valid) rounding orders, about 0.3 % apart, and the expert choice
# is discontinuous in it: where a router's k-th and (k+1)-th probabilities
# are within this relative gap, either choice is correct. The stack tests
# check that the GPU's choice is the oracle's top-k up to such near-ties, and
# then run the oracle with the GPU's choice (moe_block(inds=...)), so that
# every row can be compared.
TIE_MARGIN = 0.02


def _check_routing(gpu_inds, ref_probs, k):
    """Every expert the GPU chose and the oracle did not has an oracle
    probability within TIE_MARGIN of the oracle's k-th largest; returns the
    number of tokens whose expert set differs."""
    p = bf16_to_f32(ref_probs).astype(np.float64)
    kth = -np.sort(-p, axis=1)[:, k - 1]
    top = np.argsort(-p, axis=1, kind="stable")[:, :k]
    diff = 0
    for t in range(p.shape[0]):
        extra = set(gpu_inds[t].tolist()) - set(top[t].tolist())
        if extra:
            diff += 1
            for e in extra:
                assert p[t, e] >= kth[t] * (1 - TIE_MARGIN), (t, e, p[t, e], kth[t])
    return diff


def _near_tie_ok(ref_row, gpu_id, tol):
    r = bf16_to_f32(ref_row).astype(np.float64)
    return r[gpu_id] >= r.max() - tol


def test_stack_qwen15_two_layers(gpu, fmx, oracle):
    """The Qwen1.5-MoE-A2.7B shape (hidden 2048, 16 heads of 128, 60 experts
    top-4 with the shared expert, vocab 151936) cut to 2 layers, seed 5:
    prefill of 2 x 16 tokens, then 8 greedy steps on the GPU. Each layer's
    expert choice is the oracle's top-4 up to router near-ties; with that
    choice, every row of the residual stream and of the logits is within the
    bf16 tolerance of the oracle, and every greedy token is the oracle's
    argmax, or within 2 bf16 steps of the oracle's maximum logit (a near-tie
    of the logits, counted)."""
    import torch
    from flashmlx_amd import model as M
    cfg = M.ModelConfig(num_hidden_layers=2, max_position_embeddings=64)
    k = cfg.moe.num_experts_per_tok
    B, L, n_new, max_seq = 2, 16, 8, 32
    w, dm = _build(cfg, 5, B, max_seq, B * L)
    hw = M.host_weights(cfg, w)
    st = oracle.DecoderStack(M.oracle_config(cfg, max_seq), hw, B)
    rng = np.random.default_rng(5)
    prompt, prompt_d = _ids(rng, B, L, cfg.vocab_size)
    rt = dm.routing_buffer(B * L)
    lg = dm.forward(prompt_d, 0, last_only=False, routing=rt)
    hid = from_dev_bf16(dm.hidden(B * L))
    lg_h = from_dev_bf16(lg).reshape(B * L, -1)
    route = [r.numpy().view(np.uint32) for r in rt.cpu()]
    rl, rh = st.forward(prompt, 0, last_only=False, return_hidden=True, routing=route)
    flips = sum(_check_routing(route[li], st.last_probs[li], k) for li in range(cfg.num_hidden_layers))
    print("prefill hidden", assert_close(hid, rh, "prefill residual stream"))
    print("prefill logits", assert_close(lg_h, rl, "prefill logits"))
    last = lg.view(B, L, -1)[:, -1].contiguous()
    ref_last = rl.reshape(B, L, -1)[:, -1]
    tok = torch.empty(B, dtype=torch.int32, device="cuda")
    rt1 = dm.routing_buffer(B)
    logit_ties = 0
    for step in range(n_new):
        dm.greedy(last, tok)
        g_ids = tok.cpu().numpy()
        for b in range(B):
            o_id = int(np.argmax(bf16_to_f32(ref_last[b])))
            if g_ids[b] != o_id:
                tol = 2 * 2.0 ** (np.floor(np.log2(abs(bf16_to_f32(ref_last[b])).max())) - 7)
                assert _near_tie_ok(ref_last[b], g_ids[b], tol), (step, b, g_ids[b], o_id)
                logit_ties += 1
        if step + 1 == n_new:
            break
        last = dm.forward(tok.view(B, 1), L + step, routing=rt1)
        got = from_dev_bf16(last)
        route = [r.numpy().view(np.uint32) for r in rt1.cpu()]
        ref_last = st.forward(g_ids.reshape(B, 1), L + step, routing=route)
        flips += sum(_check_routing(route[li], st.last_probs[li], k) for li in range(cfg.num_hidden_layers))
        e = assert_close(got, ref_last, f"step {step} logits")
        print(f"step {step}: tokens {g_ids.tolist()} logits {e}")
    print(f"greedy: {B * n_new} tokens, {logit_ties} logit near-ties; {flips} router near-tie choices")
    assert logit_ties <= 2, logit_ties


def test_stack_qwen15_24_layers(gpu, fmx, oracle):
    """The full 24-layer Qwen1.5-MoE-A2.7B-shape stack (seed 5): a 256-token
    prompt at batch 1 and 4 then greedy decode steps; logits finite, a
    repeated forward gives the same bits, and the decode step's logits equal
    the last position of a prefill of the prompt plus that token within the
    row tolerance and 5 % relative L2: the two run different kernels (exact
    decode projections, fp16 prefill GEMMs) through 24 layers of bf16
    residual sums, and a router near-tie may go either way on either path."""
    import torch
    from flashmlx_amd import model as M
    cfg = M.ModelConfig(max_position_embeddings=512)
    L, max_seq = 256, 384
    w = M.synthetic_model(cfg, 5)
    rng = np.random.default_rng(55)
    for B in (1, 4):
        dm = M.DecoderModel(cfg, w, B, max_seq, B * (L + 1))
        prompt, prompt_d = _ids(rng, B, L, cfg.vocab_size)
        lg = dm.forward(prompt_d, 0)
        tok = torch.empty(B, dtype=torch.int32, device="cuda")
        dm.greedy(lg, tok)
        d1 = from_dev_bf16(dm.forward(tok.view(B, 1), L))
        d1b = from_dev_bf16(dm.forward(tok.view(B, 1), L))
        torch.cuda.synchronize()
        assert np.isfinite(bf16_to_f32(d1)).all()
        np.testing.assert_array_equal(d1, d1b)
        full = torch.cat([prompt_d, tok.view(B, 1)], 1).contiguous()
        dm2 = M.DecoderModel(cfg, w, B, max_seq, B * (L + 1))
        pf = from_dev_bf16(dm2.forward(full, 0))
        torch.cuda.synchronize()
        e = assert_close(d1, pf, f"B={B}: decode step vs prefill of {L + 1} tokens", rel_l2=5e-2)
        print(f"24 layers B={B}: decode vs prefill {e}")
        del dm, dm2
        torch.cuda.empty_cache()


@pytest.mark.parametrize("V", [151936, 1001])
def test_greedy_next(gpu, fmx, V):
    """fmx_greedy_next: the first of equal maxima (mx::argmax), NaN never
    chosen, an all-equal row gives 0, on the 16-byte path (V a multiple of 8)
    and the scalar one; the offsets advance."""
    import torch
    from flashmlx_amd import _lib
    rng = np.random.default_rng(V)
    B = 5
    x = torch.from_numpy(rng.standard_normal((B, V)).astype(np.float32)).to(torch.bfloat16)
    x[1, 77] = 9.0
    x[1, V - 5] = 9.0
    x[2, :] = 1.0
    x[3, 10] = float("nan")
    x[3, 11] = 20.0
    x[4, V - 1] = 30.0
    ids = torch.empty(B, dtype=torch.int32, device="cuda")
    offs = torch.arange(B, dtype=torch.int32, device="cuda")
    xd = x.cuda()
    lib = _lib.load()
    _lib.check(lib.fmx_greedy_next(xd.data_ptr(), B, V, V, ids.data_ptr(), offs.data_ptr(), 3,
                                   torch.cuda.current_stream().cuda_stream))
    got = ids.cpu().numpy()
    ref = x.float().numpy()
    assert got[0] == int(np.argmax(ref[0]))
    assert got[1] == 77 and got[2] == 0 and got[3] == 11 and got[4] == V - 1
    assert offs.cpu().tolist() == [3, 4, 5, 6, 7]


def test_checkpoint_safetensors_fixture_matches_oracle(gpu, fmx):
    """The committed checkpoint that the safetensors library wrote under the
    reference's key names (tests/golden/make_checkpoint.py: quantized
    router, quantized shared-expert gate, q/k/v biases, quantized embedding
    and lm_head), loaded by fmx_model_load: the prefill of a 20-token prompt
    (every position's logits: the prefill GEMMs and the MoE prefill path)
    and three decode steps (the decode kernels) against the CPU oracle's
    logits committed beside it."""
    import pathlib

    import torch
    from flashmlx_amd import model as M
    g = pathlib.Path(__file__).resolve().parent / "golden"
    ref = np.load(g / "ckpt_tiny_logits.npz")
    lm = M.load_checkpoint(str(g / "ckpt_tiny"))
    cfg = lm.cfg
    dm = M.DecoderModel(cfg, lm, 1, 32, 20)
    prompt = torch.from_numpy(ref["prompt"]).cuda()
    got = from_dev_bf16(dm.forward(prompt, 0, last_only=False)).reshape(20, -1)
    e = assert_close(got, ref["prefill_logits"], "fixture prefill logits")
    for i in range(ref["steps"].shape[0]):
        s = torch.from_numpy(ref["steps"][i]).cuda()
        assert_close(from_dev_bf16(dm.forward(s, 20 + i)), ref["step_logits"][i], f"fixture step {i} logits")
    torch.cuda.synchronize()
    print(f"safetensors fixture: prefill logits {e}")
    del dm
    lm.close()


def test_checkpoint_load_matches_memory(gpu, fmx, tmp_path):
    """A tiny stack written as an MLX checkpoint (per-expert arrays, "model."
    prefix, two shards, config.json) and read back by fmx_model_load gives
    the same logits, bit for bit, as the same weights built in memory, for a
    prefill and decode steps; the loaded layer holds its expert weights once
    (packed), not also in the MLX layout."""
    import torch
    from flashmlx_amd import model as M
    cfg = _tiny_cfg()
    B, L, max_seq = 2, 12, 32
    w, dm = _build(cfg, 33, B, max_seq, B * L)
    ck = tmp_path / "ckpt"
    M.save_checkpoint(cfg, w, str(ck))
    cfg2, tie = M.config_from_json(str(ck / "config.json"))
    assert not tie and cfg2.moe.quant_bits == 4 and cfg2.num_hidden_layers == cfg.num_hidden_layers
    lm = M.load_checkpoint(str(ck))
    dm2 = M.DecoderModel(cfg2, lm, B, max_seq, B * L)
    rng = np.random.default_rng(9)
    ids, ids_d = _ids(rng, B, L, cfg.vocab_size)
    a = from_dev_bf16(dm.forward(ids_d, 0, last_only=False))
    b = from_dev_bf16(dm2.forward(ids_d, 0, last_only=False))
    np.testing.assert_array_equal(a, b)
    for step in range(2):
        nxt, nxt_d = _ids(rng, B, 1, cfg.vocab_size)
        np.testing.assert_array_equal(from_dev_bf16(dm.forward(nxt_d, L + step)),
                                      from_dev_bf16(dm2.forward(nxt_d, L + step)))
    torch.cuda.synchronize()
    # device bytes: packed experts once per layer, attention and lm_head
    # packed, the bf16 embedding; no MLX-layout expert copy
    lib = M._lib.load()
    moe_packed = lib.fmx_moe_packed_size(M.C.byref(cfg.moe.to_c()))
    mlx_experts = sum(q.w.numel() * 4 + q.scales.numel() * 4 for q in (w.layers[0].moe.gate, w.layers[0].moe.up,
                                                                      w.layers[0].moe.down))
    assert lm.device_bytes < cfg.num_hidden_layers * (moe_packed + mlx_experts)
    print(f"loaded {lm.device_bytes} device bytes; packed MoE per layer {moe_packed}")
    lm.close()
