"""End-to-end: LLM.generate with n-gram speculative decoding on a tiny random Qwen3.

Greedy speculative decoding must emit exactly the target model's argmax at every
position.  That is checked against a single causal prefill over each finished
sequence (paged prefill attention, q_len > 64), allowing disagreement only where
the top-2 logits are within bf16 noise."""
import numpy as np
import pytest
import torch
from transformers import Qwen3Config

from nanovllm import LLM, SamplingParams
from nanovllm.engine.sequence import Sequence
from nanovllm.spec.tree import depths
from nanovllm.utils.context import reset_context


def tiny_config(vocab=512, layers=2):
    cfg = Qwen3Config(hidden_size=512, intermediate_size=1024, num_hidden_layers=layers,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=128,
                      vocab_size=vocab, max_position_embeddings=4096, rms_norm_eps=1e-6,
                      tie_word_embeddings=False, attention_bias=False, hidden_act="silu")
    cfg.rope_theta = 1000000
    cfg.dtype = torch.bfloat16
    cfg.eos_token_id = -1
    return cfg


def prompts():
    rng = np.random.default_rng(0)
    out = []
    for n in (40, 200, 300, 777):
        motif = rng.integers(0, 512, size=12).tolist()
        out.append((motif * (n // 12 + 1))[:n])
    return out


def full_logits(llm, token_ids):
    """Logits of every position of one sequence via a causal paged prefill."""
    runner, bm = llm.model_runner, llm.scheduler.block_manager
    seq = Sequence(token_ids)
    bm.allocate(seq, 0)
    seq.num_cached_tokens = 0
    seq.num_scheduled_tokens = len(seq)
    try:
        input_ids, positions = runner.prepare_prefill([seq])
        with torch.inference_mode():
            hidden = runner.model(input_ids, positions)
            logits = runner.model.compute_logits(hidden).float().cpu()
    finally:
        reset_context()
        bm.deallocate(seq)
    return logits


@pytest.mark.gpu
def test_ngram_speculative_greedy_is_target_argmax(dev):
    llm = LLM("unused", hf_config=tiny_config(), num_kvcache_blocks=64,
              speculative_method="ngram", num_speculative_tokens=5, max_num_batched_tokens=4096,
              enforce_eager=True)
    ps = prompts()
    outs = llm.generate(ps, SamplingParams(temperature=0.0, max_tokens=48, ignore_eos=True),
                        use_tqdm=False)
    checked = mismatched = 0
    for p, o in zip(ps, outs):
        toks = o["token_ids"]
        assert len(toks) == 48
        logits = full_logits(llm, p + toks)
        for j, t in enumerate(toks):
            row = logits[len(p) + j - 1]
            top2 = torch.topk(row, 2).values
            checked += 1
            if int(row.argmax()) != t:
                mismatched += 1
                assert float(top2[0] - top2[1]) < 0.05, (j, t, int(row.argmax()))
    assert mismatched <= checked // 50
    steps = [s for s in llm.scheduler.running]  # all finished
    assert not steps


@pytest.mark.gpu
def test_ngram_speculative_sampling_runs_and_accepts(dev):
    llm = LLM("unused", hf_config=tiny_config(), num_kvcache_blocks=64,
              speculative_method="ngram", num_speculative_tokens=4, max_num_batched_tokens=4096,
              enforce_eager=True)
    ps = prompts()
    sps = [SamplingParams(temperature=t, max_tokens=40, ignore_eos=True) for t in (0.0, 0.6, 1.0, 0.0)]
    outs = llm.generate(ps, sps, use_tqdm=False)
    assert [len(o["token_ids"]) for o in outs] == [40] * 4
    assert all(0 <= t < 512 for o in outs for t in o["token_ids"])


@pytest.mark.gpu
def test_plain_decode_equals_argmax(dev):
    llm = LLM("unused", hf_config=tiny_config(), num_kvcache_blocks=64, max_num_batched_tokens=4096,
              enforce_eager=True)
    p = prompts()[1]
    out = llm.generate([p], SamplingParams(temperature=0.0, max_tokens=20, ignore_eos=True),
                       use_tqdm=False)[0]["token_ids"]
    logits = full_logits(llm, p + out)
    agree = sum(int(logits[len(p) + j - 1].argmax()) == t for j, t in enumerate(out))
    assert agree >= 19


def check_greedy_is_argmax(llm, ps, outs, n):
    checked = mismatched = 0
    for p, o in zip(ps, outs):
        toks = o["token_ids"]
        assert len(toks) == n
        logits = full_logits(llm, p + toks)
        for j, t in enumerate(toks):
            row = logits[len(p) + j - 1]
            top2 = torch.topk(row, 2).values
            checked += 1
            if int(row.argmax()) != t:
                mismatched += 1
                assert float(top2[0] - top2[1]) < 0.05, (j, t, int(row.argmax()))
    # every disagreement is a near-tie (above); the verify step and the one-pass
    # prefill add attention partials in different orders, so a few such flips occur
    assert mismatched <= max(2, checked // 25)


@pytest.mark.gpu
def test_eagle3_speculative_greedy_is_target_argmax(dev):
    """EAGLE-3 trees (top-8, depth 4, 16 nodes) on a 64-token vocabulary, where a
    random draft head still hits the target's argmax often enough to accept
    multi-token paths (tree compaction and the draft catch-up are exercised)."""
    V = 64
    llm = LLM("unused", hf_config=tiny_config(vocab=V, layers=6), num_kvcache_blocks=64,
              speculative_method="eagle3", num_speculative_tokens=15, eagle_topk=8, eagle_depth=4,
              max_num_batched_tokens=4096, enforce_eager=True)
    rng = np.random.default_rng(3)
    ps = [rng.integers(0, V, size=n).tolist() for n in (30, 257, 100, 513)]
    outs = llm.generate(ps, SamplingParams(temperature=0.0, max_tokens=40, ignore_eos=True),
                        use_tqdm=False)
    check_greedy_is_argmax(llm, ps, outs, 40)
    assert len(llm.model_runner.draft_states) == 0  # finished sequences drop their draft state
    hist = llm.model_runner.spec_stats["accepted_hist"]
    print("accepted-length histogram", dict(sorted(hist.items())), flush=True)
    assert sum(n for a, n in hist.items() if a >= 1) >= 5


@pytest.mark.gpu
def test_eagle3_graph_verify_greedy_is_target_argmax(dev):
    """The EAGLE-3 step (draft tree expansion, verify rows, the target's tree verify with
    the aux residual streams) replayed from one captured HIP graph per batch size, and
    the catch-up from its own, batches padded to the graph sizes: still the target's
    argmax."""
    V = 64
    llm = LLM("unused", hf_config=tiny_config(vocab=V, layers=6), num_kvcache_blocks=64,
              speculative_method="eagle3", num_speculative_tokens=15, eagle_topk=8, eagle_depth=4,
              max_num_batched_tokens=4096, enforce_eager=False, max_num_seqs=16,
              max_model_len=2048)
    assert list(llm.model_runner.graph_vars) == [16]
    assert sorted(llm.model_runner.eagle_graphs) == llm.model_runner.graph_bs
    rng = np.random.default_rng(3)
    ps = [rng.integers(0, V, size=n).tolist() for n in (30, 257, 100)]
    outs = llm.generate(ps, SamplingParams(temperature=0.0, max_tokens=40, ignore_eos=True),
                        use_tqdm=False)
    check_greedy_is_argmax(llm, ps, outs, 40)
    hist = llm.model_runner.spec_stats["accepted_hist"]
    print("accepted-length histogram", dict(sorted(hist.items())), flush=True)


@pytest.mark.gpu
def test_eagle3_draft_vocabulary_maps_to_target_ids(dev):
    """A draft head over a 64-token draft vocabulary whose d2t table scatters the draft
    ids over a 512-token target vocabulary: the tree tokens are target ids from the
    mapped set, and greedy output is still the target's argmax."""
    llm = LLM("unused", hf_config=tiny_config(vocab=512, layers=6), num_kvcache_blocks=64,
              speculative_method="eagle3", num_speculative_tokens=15, eagle_topk=4, eagle_depth=4,
              eagle_draft_vocab=64, max_num_batched_tokens=4096, enforce_eager=True)
    runner = llm.model_runner
    assert runner.draft.lm_head.weight.shape[0] == 64
    ids = torch.arange(64, device=runner.draft.d2t.device)
    runner.draft.d2t.copy_((ids * 7 + 3) % 512 - ids)
    mapped = set(((ids * 7 + 3) % 512).tolist())
    seen = set()
    orig = runner._eagle_tree

    def spy(*a):
        toks, parents, *rest = orig(*a)
        seen.update(toks.flatten().tolist())
        return (toks, parents, *rest)

    runner._eagle_tree = spy
    rng = np.random.default_rng(6)
    ps = [rng.integers(0, 512, size=n).tolist() for n in (40, 300)]
    outs = llm.generate(ps, SamplingParams(temperature=0.0, max_tokens=24, ignore_eos=True),
                        use_tqdm=False)
    check_greedy_is_argmax(llm, ps, outs, 24)
    assert seen and seen <= mapped


def greedy_continuation(llm, ids, n):
    ids = list(ids)
    out = []
    for _ in range(n):
        g = int(full_logits(llm, ids)[-1].argmax())
        out.append(g)
        ids.append(g)
    return out


@pytest.mark.gpu
def test_eagle3_deep_acceptance_is_lossless(dev):
    """The draft trees are built as usual, then the target's own greedy continuation is
    written onto an existing depth-3 branch of each tree (a non-chain path at BFS
    positions), so verification accepts multi-token paths: tree KV compaction and the
    draft head's multi-row catch-up must keep the output equal to plain greedy."""
    V = 64
    llm = LLM("unused", hf_config=tiny_config(vocab=V, layers=6), num_kvcache_blocks=96,
              speculative_method="eagle3", num_speculative_tokens=15, eagle_topk=4, eagle_depth=4,
              max_num_batched_tokens=4096, enforce_eager=True)
    runner = llm.model_runner
    orig = runner._eagle_tree

    def planted(seqs, ctx, block_tables, *more):
        toks, parents, *rest = orig(seqs, ctx, block_tables, *more)
        toks = toks.clone()
        par = parents.cpu().numpy()
        for b, seq in enumerate(seqs):
            d = depths(par[b])
            v = int(np.argmax(d >= 3)) if (d >= 3).any() else int(np.argmax(d))
            path = []
            while v > 0:
                path.append(v)
                v = int(par[b][v])
            path.reverse()
            for node, g in zip(path, greedy_continuation(llm, seq.token_ids, len(path))):
                toks[b, node - 1] = g
        return (toks, parents, *rest)

    runner._eagle_tree = planted
    rng = np.random.default_rng(5)
    ps = [rng.integers(0, V, size=n).tolist() for n in (64, 300)]
    outs = llm.generate(ps, SamplingParams(temperature=0.0, max_tokens=32, ignore_eos=True),
                        use_tqdm=False)
    check_greedy_is_argmax(llm, ps, outs, 32)
    hist = runner.spec_stats["accepted_hist"]
    print("accepted-length histogram", dict(sorted(hist.items())), flush=True)
    assert sum(n for a, n in hist.items() if a >= 2) >= 4


@pytest.mark.gpu
def test_eagle3_prefix_hits_need_the_next_token(dev):
    """EAGLE-3 with the prefix cache: the draft K/V row at a block's last position comes
    from the token after the block, so a prompt that shares a full block with a finished
    one but continues with another token must not hit it, and one that continues with
    the same token does.  Both generate the target's greedy output."""
    V = 64
    llm = LLM("unused", hf_config=tiny_config(vocab=V, layers=4), num_kvcache_blocks=64,
              speculative_method="eagle3", num_speculative_tokens=15, eagle_topk=8, eagle_depth=4,
              max_num_batched_tokens=4096, enforce_eager=True)
    rng = np.random.default_rng(11)
    base = rng.integers(0, V, size=300).tolist()
    other = list(base)
    other[256] = (base[256] + 1) % V
    sp = SamplingParams(temperature=0.0, max_tokens=24, ignore_eos=True)
    outs = llm.generate([base], sp, use_tqdm=False)
    bm = llm.scheduler.block_manager
    assert bm.can_allocate(Sequence(other)) == 0
    assert bm.can_allocate(Sequence(base[:280])) == 1
    ps = [other, base[:280]]
    outs = llm.generate(ps, sp, use_tqdm=False)
    check_greedy_is_argmax(llm, ps, outs, 24)


@pytest.mark.gpu
def test_eagle3_sampling_runs(dev):
    V = 64
    llm = LLM("unused", hf_config=tiny_config(vocab=V, layers=6), num_kvcache_blocks=64,
              speculative_method="eagle3", num_speculative_tokens=31, eagle_topk=8, eagle_depth=6,
              max_num_batched_tokens=300, enforce_eager=True)  # chunked prefill of the long prompt
    rng = np.random.default_rng(4)
    ps = [rng.integers(0, V, size=n).tolist() for n in (50, 700, 120)]
    sps = [SamplingParams(temperature=t, max_tokens=30, ignore_eos=True) for t in (1.0, 0.0, 0.7)]
    outs = llm.generate(ps, sps, use_tqdm=False)
    assert [len(o["token_ids"]) for o in outs] == [30] * 3
    assert all(0 <= t < V for o in outs for t in o["token_ids"])
    check_greedy_is_argmax(llm, ps[1:2], outs[1:2], 30)


@pytest.mark.gpu
@pytest.mark.parametrize("spec", ["none", "ngram"])
def test_graph_generate_is_target_argmax(dev, spec):
    """Verify / decode steps replayed from captured HIP graphs (padded batches)."""
    kw = dict(speculative_method="ngram", num_speculative_tokens=5) if spec == "ngram" else {}
    llm = LLM("unused", hf_config=tiny_config(), num_kvcache_blocks=64, enforce_eager=False,
              max_num_seqs=32, max_model_len=2048, max_num_batched_tokens=4096, **kw)
    assert llm.model_runner.graphs
    assert sorted(llm.model_runner.graph_vars) == ([1, 6] if spec == "ngram" else [1])
    ps = prompts()
    outs = llm.generate(ps, SamplingParams(temperature=0.0, max_tokens=24, ignore_eos=True),
                        use_tqdm=False)
    check_greedy_is_argmax(llm, ps, outs, 24)


@pytest.mark.gpu
def test_graph_replays_are_stable(dev):
    """Three replays of one padded batch, with eager forwards and synchronisations in
    between: every replay is bit-identical to the first and matches eager execution
    to bf16 accuracy."""
    llm = LLM("unused", hf_config=tiny_config(), num_kvcache_blocks=64, enforce_eager=False,
              max_num_seqs=32, max_model_len=2048, speculative_method="ngram",
              num_speculative_tokens=3)
    runner, bm = llm.model_runner, llm.scheduler.block_manager
    rng = np.random.default_rng(7)
    seqs = []
    for n in (100, 300, 257):
        seq = Sequence(rng.integers(0, 512, size=n).tolist())
        bm.allocate(seq, 0)
        bm.may_append(seq, 4)
        seq.num_cached_tokens = 0
        seq.num_scheduled_tokens = n
        seqs.append(seq)
    drafts = [[1, 2, 3], [], [7]]
    with torch.inference_mode():
        # prefill the prompts so every attended KV position holds the model's own keys
        # (the cache is allocated uninitialised)
        input_ids, positions = runner.prepare_prefill(seqs)
        runner.model(input_ids, positions)
        torch.cuda.synchronize()
        reset_context()
        outs = []
        for rep in range(3):
            input_ids, positions, T, _ = runner.prepare_decode(seqs, drafts)
            eager = runner.model(input_ids, positions).float()
            torch.cuda.synchronize()
            graph = runner.replay_graph(input_ids, positions).float().clone()
            torch.cuda.synchronize()
            reset_context()
            outs.append(graph)
            assert T == 4
            assert float((graph - eager).abs().max()) < 5e-2
        for o in outs[1:]:
            assert torch.equal(o, outs[0])
    for seq in seqs:
        bm.deallocate(seq)


@pytest.mark.gpu
def test_eagle3_draft_tree_graph_replays_are_stable(dev):
    """The captured EAGLE-3 step, replayed three times for four sequences (a captured
    batch size, no padding) with eager steps and synchronisations in between: every
    replay gives the eager expansion's tree, depths and masks, and the eager target
    verify's hidden states and aux streams of that tree, bit for bit."""
    V = 64
    llm = LLM("unused", hf_config=tiny_config(vocab=V, layers=2), num_kvcache_blocks=64,
              speculative_method="eagle3", num_speculative_tokens=15, eagle_topk=8, eagle_depth=4,
              max_num_batched_tokens=4096, enforce_eager=False, max_num_seqs=16,
              max_model_len=2048)
    runner, bm, cfg = llm.model_runner, llm.scheduler.block_manager, llm.model_runner.config
    assert 4 in runner.eagle_graphs
    g = torch.Generator(device="cuda").manual_seed(11)
    for cache in (runner.draft.self_attn.attn.k_cache, runner.draft.self_attn.attn.v_cache):
        cache.normal_(generator=g)
    rng = np.random.default_rng(12)
    k, rmax = cfg.eagle_topk, cfg.eagle_topk * (cfg.eagle_depth - 1)
    H = cfg.hf_config.hidden_size
    seqs = []
    for n in (60, 300, 257, 129):
        seq = Sequence(rng.integers(0, V, size=n).tolist())
        bm.allocate(seq, 0)
        bm.may_append(seq, rmax + 1)
        seqs.append(seq)
        lp = torch.sort(torch.rand(k, device="cuda", generator=g).log(), descending=True).values
        runner.draft_states.put(runner.draft_states.rows([seq.seq_id], create=True),
                                torch.randn(1, H, device="cuda", generator=g).to(torch.bfloat16),
                                torch.randint(0, V, (1, k), device="cuda", generator=g), lp[None])
    ctx = [len(seq) - 1 for seq in seqs]
    with torch.inference_mode():
        block_tables = runner.prepare_block_tables(seqs)
        feat, tok, lp = runner.draft_states.get(runner.draft_states.rows([s.seq_id for s in seqs]))
        ctx_d = torch.tensor(ctx, dtype=torch.int64, device="cuda")
        args = (tok, lp, feat, ctx_d, block_tables, cfg.max_model_len)
        T = 1 + cfg.num_speculative_tokens
        roots = torch.tensor([s.last_token for s in seqs], device="cuda")
        valid = torch.ones(len(seqs), dtype=torch.bool, device="cuda")
        gv = runner.graph_vars[T]
        for rep in range(3):
            eager = runner._expand_draft_tree(*args)
            tokens = torch.cat([roots.unsqueeze(1), eager[0]], dim=1)
            e_h, e_a = runner._verify_tree(tokens, eager[2], eager[3], ctx_d, block_tables, valid,
                                           cfg.max_model_len)
            e_h, e_a = e_h.clone(), e_a.clone()
            torch.cuda.synchronize()
            replay = runner._eagle_tree(seqs, ctx, block_tables)
            torch.cuda.synchronize()
            assert len(replay) == len(eager) == 4
            assert all(torch.equal(r, e) for r, e in zip(replay, eager)), f"replay {rep}"
            n = len(seqs) * T
            assert torch.equal(gv["outputs"][:n], e_h), f"replay {rep}: verify hidden states"
            assert torch.equal(gv["aux"][:n], e_a), f"replay {rep}: aux streams"
        e_par = eager[1]
        assert (e_par[:, 0] == -1).all() and (e_par[:, 1:] < torch.arange(1, 16, device="cuda")).all()
    for seq in seqs:
        runner.draft_states.drop(seq.seq_id)
        bm.deallocate(seq)


@pytest.mark.gpu
@pytest.mark.parametrize("eager", [True, False])
def test_eagle3_preemption_keeps_output_lossless(dev, eager):
    """A KV pool too small for every sequence's next page: sequences are preempted,
    re-prefilled and drafted again from their resident root-state rows (reused across
    the preemption).  Greedy output is still the target's argmax."""
    V = 64
    llm = LLM("unused", hf_config=tiny_config(vocab=V, layers=2), num_kvcache_blocks=9,
              speculative_method="eagle3", num_speculative_tokens=15, eagle_topk=4,
              eagle_depth=4, max_num_batched_tokens=4096, enforce_eager=eager,
              max_num_seqs=16, max_model_len=2048)
    sched = llm.scheduler
    preempted = []
    orig = sched.preempt

    def counting(seq):
        preempted.append(seq.seq_id)
        return orig(seq)

    sched.preempt = counting
    rng = np.random.default_rng(21)
    ps = [rng.integers(0, V, size=n).tolist() for n in (200, 230, 180, 240, 210)]
    outs = llm.generate(ps, SamplingParams(temperature=0.0, max_tokens=80, ignore_eos=True),
                        use_tqdm=False)
    print("preemptions", len(preempted), flush=True)
    assert preempted
    check_greedy_is_argmax(llm, ps, outs, 80)
    assert len(llm.model_runner.draft_states) == 0


@pytest.mark.gpu
def test_eagle3_catch_up_graph_matches_eager(dev):
    """The captured draft catch-up (depth + 1 rows per sequence, the rows past each
    accepted length padded) gives the eager padded catch-up's root states bit for bit,
    and those of the packed eager catch-up (exactly the accepted rows) within bf16
    noise."""
    V = 64
    llm = LLM("unused", hf_config=tiny_config(vocab=V, layers=2), num_kvcache_blocks=64,
              speculative_method="eagle3", num_speculative_tokens=15, eagle_topk=4, eagle_depth=4,
              max_num_batched_tokens=4096, enforce_eager=False, max_num_seqs=16,
              max_model_len=2048)
    runner, bm, cfg = llm.model_runner, llm.scheduler.block_manager, llm.model_runner.config
    assert sorted(runner.catchup_graphs) == runner.graph_bs
    g = torch.Generator(device="cuda").manual_seed(31)
    for cache in (runner.draft.self_attn.attn.k_cache, runner.draft.self_attn.attn.v_cache):
        cache.normal_(generator=g)
    T, D1 = 1 + cfg.num_speculative_tokens, cfg.eagle_depth + 1
    rng = np.random.default_rng(32)
    seqs = []
    for n in (60, 300, 257, 129):
        seq = Sequence(rng.integers(0, V, size=n).tolist())
        bm.allocate(seq, 0)
        bm.may_append(seq, cfg.verify_lookahead)
        seqs.append(seq)
    B = len(seqs)
    ctx = [len(s) - 1 for s in seqs]
    acc_h = [0, 2, 4, 1]
    path = torch.full((B, T), -1, dtype=torch.int32)
    out = torch.full((B, T), -1, dtype=torch.int32)
    for b, a in enumerate(acc_h):
        nodes = [0] + sorted(rng.choice(np.arange(1, T), size=a, replace=False).tolist())
        path[b, :a + 1] = torch.tensor(nodes, dtype=torch.int32)
        out[b, :a + 1] = torch.from_numpy(rng.integers(0, V, size=a + 1).astype(np.int32))
    with torch.inference_mode():
        aux = runner.graph_vars[T]["aux"]
        aux.normal_(generator=g)
        block_tables = runner.prepare_block_tables(seqs)
        ctx_d = torch.tensor(ctx, dtype=torch.int64, device="cuda")
        acc = torch.tensor(acc_h, dtype=torch.int32, device="cuda")
        path, out = path.cuda(), out.cuda()
        padded = [t.clone() for t in runner._catch_up_padded(
            acc.long(), path[:, :D1].long(), out[:, :D1].long(), ctx_d, block_tables, aux, T,
            cfg.max_model_len)]
        replays = []
        for _ in range(3):
            replays.append([t.clone() for t in runner._replay_catch_up(acc, path, out, ctx_d,
                                                                       block_tables)])
            torch.cuda.synchronize()
        packed = runner._catch_up_packed(acc, acc_h, path, out, ctx, ctx_d, block_tables,
                                         aux[:B * T], T)
        torch.cuda.synchronize()
    for rep, replay in enumerate(replays):
        assert all(torch.equal(r, e) for r, e in zip(replay, padded)), f"replay {rep}"
    f_p, _, lp_p = packed
    assert torch.allclose(f_p.float(), padded[0].float(), atol=5e-2, rtol=2e-2)
    assert torch.allclose(lp_p, padded[2], atol=5e-2)
    for seq in seqs:
        bm.deallocate(seq)
