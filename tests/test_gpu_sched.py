"""GPU tests of the batched-decode server loop (fmx_sched.cpp, BatchScheduler
of server/src/scheduler.cpp): requests of different prompt lengths and
token budgets, joining while others decode, decoded together over the slots
of one KV pool, produce the same tokens as each request generated alone
(fmx_model_forward + greedy argmax, whose logits the decoder-stack tests hold
to the oracle)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _tiny_cfg():
    from flashmlx_amd.model import ModelConfig
    from flashmlx_amd.moe import MoEConfig
    moe = MoEConfig(hidden_size=512, num_experts=8, num_experts_per_tok=2, moe_intermediate_size=256,
                    shared_expert_intermediate_size=512, norm_topk_prob=False)
    return ModelConfig(hidden_size=512, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                       vocab_size=256, max_position_embeddings=64, moe=moe)


def _alone(cfg, w, prompt, n_new, max_ctx):
    import torch
    from flashmlx_amd import model as M
    dm = M.DecoderModel(cfg, w, 1, max_ctx, max(len(prompt), 1))
    p = torch.tensor([prompt], dtype=torch.int32, device="cuda")
    out = dm.generate(p, n_new).cpu().numpy()[0].tolist()
    torch.cuda.synchronize()
    return out


def _run(sched, requests, late, join_after):
    """Submits `requests`, steps, submits `late` after `join_after` steps,
    steps until no work is left; returns ({id: tokens}, {id: prompt index},
    max active count, completed ids)."""
    toks, index = {}, {}
    for i, (p, n) in enumerate(requests):
        index[sched.submit(p, n)] = i
    steps, max_active, completed = 0, 0, []
    while sched.has_work():
        for rid, t in sched.step().items():
            toks.setdefault(rid, []).extend(t)
        steps += 1
        max_active = max(max_active, sched.active_count())
        completed += sched.drain_completed()
        if steps == join_after:
            for j, (p, n) in enumerate(late):
                index[sched.submit(p, n)] = len(requests) + j
        assert steps < 200
    return toks, index, max_active, completed


def test_scheduler_matches_alone(gpu, fmx):
    """Three slots, seven requests: prompts of 1..20 tokens (the decode
    kernels below 17 prompt tokens, the prefill GEMMs above), budgets of 1..9
    tokens, three requests joining after two steps; each request's tokens
    equal the same request generated alone, every request completes once,
    and at most three are active at a time."""
    import torch
    from flashmlx_amd import model as M
    cfg = _tiny_cfg()
    w = M.synthetic_model(cfg, 41)
    rng = np.random.default_rng(3)
    mk = lambda L: rng.integers(0, cfg.vocab_size, size=L).tolist()
    requests = [(mk(5), 6), (mk(17), 3), (mk(1), 1), (mk(9), 9)]
    late = [(mk(20), 4), (mk(3), 7), (mk(12), 2)]
    max_ctx, max_prompt = 40, 20
    sched = M.BatchScheduler(cfg, w, 3, max_ctx, max_prompt)
    toks, index, max_active, completed = _run(sched, requests, late, 2)
    torch.cuda.synchronize()
    allr = requests + late
    assert sorted(completed) == sorted(index)
    assert max_active <= 3 and sched.active_count() == 0
    for rid, i in index.items():
        p, n = allr[i]
        ref = _alone(cfg, w, p, n, max_ctx)
        assert toks[rid] == ref, (i, len(p), n, toks[rid], ref)
    sched.close()


def test_scheduler_eight_slots(gpu, fmx):
    """Eight requests decoding together (batches of 8 through every decode
    kernel) on a 24-position context, then eight more reusing the freed
    slots: tokens equal each request alone."""
    import torch
    from flashmlx_amd import model as M
    cfg = _tiny_cfg()
    w = M.synthetic_model(cfg, 43)
    rng = np.random.default_rng(5)
    reqs = [(rng.integers(0, cfg.vocab_size, size=int(rng.integers(1, 13))).tolist(), int(rng.integers(3, 11)))
            for _ in range(16)]
    sched = M.BatchScheduler(cfg, w, 8, 24, 12)
    toks, index, max_active, completed = _run(sched, reqs[:8], reqs[8:], 3)
    torch.cuda.synchronize()
    assert max_active == 8 and sorted(completed) == sorted(index)
    for rid, i in index.items():
        p, n = reqs[i]
        assert toks[rid] == _alone(cfg, w, p, n, 24), (i, p, n)
    sched.close()


def test_scheduler_refusals(gpu, fmx):
    """Sampling, over-long prompts, budgets past the context and tokens
    outside the vocabulary are refused at submit; nothing is queued."""
    from flashmlx_amd import _lib
    from flashmlx_amd import model as M
    cfg = _tiny_cfg()
    w = M.synthetic_model(cfg, 47)
    sched = M.BatchScheduler(cfg, w, 2, 16, 8)
    cases = [(([1, 2], 3, 0.7), _lib.FMX_ERR_UNSUPPORTED), (([1] * 9, 2, 0.0), _lib.FMX_ERR_SHAPE),
             (([1] * 8, 9, 0.0), _lib.FMX_ERR_SHAPE), (([1, 256], 2, 0.0), _lib.FMX_ERR_ARG),
             (([1], 0, 0.0), _lib.FMX_ERR_SHAPE)]
    for (p, n, t), status in cases:
        with pytest.raises(_lib.FmxError) as e:
            sched.submit(p, n, t)
        assert e.value.status == status
    assert not sched.has_work()
    sched.close()


def _alone_split(cfg, w, prompt, n_new, max_ctx):
    """The prefix-cache path of a request run by hand: prefill of all but the
    last prompt token, the last one as a decode step, then greedy decoding."""
    import torch
    from flashmlx_amd import model as M
    dm = M.DecoderModel(cfg, w, 1, max_ctx, max(len(prompt), 1))
    p = torch.tensor([prompt], dtype=torch.int32, device="cuda")
    n = len(prompt)
    dm.forward(p[:, :-1].contiguous(), 0)
    logits = dm.forward(p[:, -1:].contiguous(), n - 1)
    ids = torch.empty((1, 1), dtype=torch.int32, device="cuda")
    out = []
    for i in range(n_new):
        dm.greedy(logits, ids.view(-1))
        out.append(int(ids.item()))
        if i + 1 < n_new:
            dm.forward_into(ids, n + i, logits)
    torch.cuda.synchronize()
    return out


def test_scheduler_prefix_cache(gpu, fmx):
    """With the prefix cache on, a repeated prompt is served from the cache
    (one hit; its tokens equal prefill of n-1 tokens + the last token as a
    decode step, the reference's cached path), new prompts are prefilled
    (tokens equal the request alone), and with one entry a third prompt
    evicts the first, whose repeat is then prefilled again."""
    import torch
    from flashmlx_amd import model as M
    cfg = _tiny_cfg()
    w = M.synthetic_model(cfg, 53)
    rng = np.random.default_rng(9)
    p1 = rng.integers(0, cfg.vocab_size, size=9).tolist()
    p2 = rng.integers(0, cfg.vocab_size, size=6).tolist()
    max_ctx = 32
    sched = M.BatchScheduler(cfg, w, 2, max_ctx, 12, prefix_cache=2)
    toks, index, _, _ = _run(sched, [(p1, 5), (p2, 4)], [(p1, 7)], 2)
    torch.cuda.synchronize()
    assert sched.prefix_hits() == 1
    by_i = {i: toks[rid] for rid, i in index.items()}
    assert by_i[0] == _alone(cfg, w, p1, 5, max_ctx)
    assert by_i[1] == _alone(cfg, w, p2, 4, max_ctx)
    assert by_i[2] == _alone_split(cfg, w, p1, 7, max_ctx)
    sched.close()
    # one entry: p1, then p2 (evicts p1), then p1 again is a miss
    sched = M.BatchScheduler(cfg, w, 1, max_ctx, 12, prefix_cache=1)
    toks, index, _, _ = _run(sched, [(p1, 3), (p2, 3), (p1, 4)], [], 0)
    torch.cuda.synchronize()
    assert sched.prefix_hits() == 0
    by_i = {i: toks[rid] for rid, i in index.items()}
    assert by_i[2] == _alone(cfg, w, p1, 4, max_ctx)
    sched.close()
