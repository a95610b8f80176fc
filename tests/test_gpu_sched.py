"""GPU tests of the batched-decode server loop (fmx_sched.cpp, BatchScheduler
of server/src/scheduler.cpp): requests of different prompt lengths and
token budgets, joining while others decode, decoded together over the slots
of one KV pool, produce the same tokens as each request generated alone
(fmx_model_forward + greedy argmax) and as the CPU oracle's DecoderStack
decoding each request alone."""
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


def _oracle_greedy(oracle, st, prompt, n):
    """Greedy tokens of the oracle's DecoderStack (the first largest bf16
    logit, as np.argmax), with each step's logits and the smallest router
    margin over the step's layers and tokens."""
    from helpers import bf16_to_f32
    lg = st.forward(np.array([prompt]), 0)
    toks, logits, margins, pos = [], [], [], len(prompt)
    for i in range(n):
        f = bf16_to_f32(lg[0]).astype(np.float64)
        toks.append(int(np.argmax(f)))
        logits.append(f)
        margins.append(float(st.last_margins.min()))
        if i + 1 < n:
            lg = st.forward(np.array([[toks[-1]]]), pos)
            pos += 1
    return toks, logits, margins


def test_scheduler_matches_oracle(gpu, fmx, oracle):
    """The scheduler's tokens against the CPU oracle's DecoderStack decoding
    each request alone: three slots, six requests with prompts of 1..20
    tokens (decode kernels and prefill GEMMs) and budgets of 1..8 tokens,
    three of them joining after two steps. Each request's tokens equal the
    oracle's, or agree up to a step where the oracle itself is at a near-tie
    (the GPU's token within four bf16 ulps of the oracle's largest logit, or
    a router margin below 2 % in the step that produced the logits: the
    GPU's other valid rounding order may then resolve it either way), after
    which the greedy chains are no longer comparable. At most one such
    near-tie over all requests."""
    import torch
    from flashmlx_amd import model as M
    cfg = _tiny_cfg()
    w = M.synthetic_model(cfg, 45, keep_mlx=True)
    max_ctx, max_prompt = 40, 20
    hw = M.host_weights(cfg, w)
    oc = M.oracle_config(cfg, max_ctx)
    rng = np.random.default_rng(11)
    mk = lambda L: rng.integers(0, cfg.vocab_size, size=L).tolist()
    requests = [(mk(4), 8), (mk(18), 5), (mk(1), 3)]
    late = [(mk(20), 6), (mk(7), 1), (mk(11), 7)]
    sched = M.BatchScheduler(cfg, w, 3, max_ctx, max_prompt)
    toks, index, _, completed = _run(sched, requests, late, 2)
    torch.cuda.synchronize()
    sched.close()
    allr = requests + late
    assert sorted(completed) == sorted(index)
    near_ties, compared = [], 0
    for rid, i in sorted(index.items(), key=lambda kv: kv[1]):
        p, n = allr[i]
        ref, logits, margins = _oracle_greedy(oracle, oracle.DecoderStack(oc, hw, 1), p, n)
        got = toks[rid]
        assert len(got) == n
        for step, (g, r) in enumerate(zip(got, ref)):
            if g == r:
                compared += 1
                continue
            f = logits[step]
            ulp = 2.0 ** (np.floor(np.log2(abs(f.max()))) - 7)
            gap = (f.max() - f[g]) / ulp
            assert gap <= 4 or margins[step] < 0.02, (i, step, g, r, gap, margins[step])
            near_ties.append((i, step, float(gap), margins[step]))
            break
    print(f"scheduler vs oracle: {compared} tokens equal, near-ties {near_ties}")
    assert len(near_ties) <= 1, near_ties
    assert compared >= 25


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


def test_scheduler_submit_from_another_thread(gpu, fmx):
    """submit, has_work and active_count from a second host thread while
    the main thread steps (the reference's Python threads feed the engine
    loop the same way): every request completes once, with the tokens of
    the request generated alone."""
    import threading
    import time

    import torch
    from flashmlx_amd import model as M
    cfg = _tiny_cfg()
    w = M.synthetic_model(cfg, 49)
    rng = np.random.default_rng(13)
    reqs = [(rng.integers(0, cfg.vocab_size, size=int(rng.integers(1, 15))).tolist(), int(rng.integers(2, 7)))
            for _ in range(10)]
    sched = M.BatchScheduler(cfg, w, 4, 24, 14)
    ids, seen_counts = {}, []
    first = sched.submit(*reqs[0])
    ids[first] = 0

    def feeder():
        for i in range(1, len(reqs)):
            time.sleep(0.002)
            ids[sched.submit(*reqs[i])] = i
            seen_counts.append((sched.has_work(), sched.active_count()))

    th = threading.Thread(target=feeder)
    th.start()
    toks, completed, t0 = {}, [], time.monotonic()
    while th.is_alive() or sched.has_work():
        assert time.monotonic() - t0 < 60
        if not sched.has_work():
            time.sleep(0.0005)  # the feeder is between submissions
            continue
        for rid, t in sched.step().items():
            toks.setdefault(rid, []).extend(t)
        completed += sched.drain_completed()
    th.join()
    completed += sched.drain_completed()
    torch.cuda.synchronize()
    assert sorted(completed) == sorted(ids) and len(ids) == len(reqs)
    assert len(seen_counts) == len(reqs) - 1 and all(0 <= a <= 4 for _, a in seen_counts)
    for rid, i in ids.items():
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
