"""Scheduler / BlockManager / Sequence with scripted tokens (no GPU): the reference's
one-token decode behaviour, and the verify step's multi-token accounting."""
import pytest
from transformers import Qwen3Config

from nanovllm.config import Config
from nanovllm.engine.block_manager import BlockManager, block_key
from nanovllm.engine.scheduler import Scheduler
from nanovllm.engine.sequence import Sequence, SequenceStatus
from nanovllm.sampling_params import SamplingParams

BS = 256
EOS = 7


def make_scheduler(num_blocks=16, spec=False, k=5, max_num_seqs=512):
    cfg = Config("unused", hf_config=Qwen3Config(max_position_embeddings=8192),
                 num_kvcache_blocks=num_blocks, max_num_seqs=max_num_seqs,
                 speculative_method="ngram" if spec else "none", num_speculative_tokens=k)
    cfg.eos = EOS
    Sequence.block_size = BS
    return Scheduler(cfg)


def prompt(n, start=100):
    return [start + (i % 50) for i in range(n)]


def run_prefill(s):
    seqs, is_prefill = s.schedule()
    assert is_prefill
    s.postprocess(seqs, [11] * len(seqs), True)
    return seqs


def test_one_token_decode_matches_reference_rules():
    s = make_scheduler()
    seq = Sequence(prompt(255), SamplingParams(max_tokens=10))
    s.add(seq)
    run_prefill(s)
    assert len(seq) == 256 and seq.num_cached_tokens == 255 and len(seq.block_table) == 1
    seqs, is_prefill = s.schedule()  # decode writes position 255: still block 0
    assert not is_prefill and len(seq.block_table) == 1
    s.postprocess(seqs, [12], False)
    assert len(seq) == 257 and seq.num_cached_tokens == 256
    seqs, _ = s.schedule()  # position 256 needs block 1 (reference: len % bs == 1)
    assert len(seq.block_table) == 2


def test_verify_lookahead_reserves_blocks_across_boundary():
    s = make_scheduler(spec=True, k=5)
    seq = Sequence(prompt(253), SamplingParams(max_tokens=100))
    s.add(seq)
    run_prefill(s)  # len 254, cached 253
    seqs, _ = s.schedule()  # rows at positions 253..258 -> blocks 0 and 1
    assert len(seq.block_table) == 2


def test_multi_token_append_and_cached_count():
    s = make_scheduler(spec=True, k=5)
    seq = Sequence(prompt(300), SamplingParams(max_tokens=100))
    s.add(seq)
    run_prefill(s)
    seqs, _ = s.schedule()
    s.postprocess(seqs, [[21, 22, 23, 24]], False)  # 3 accepted + next token
    assert seq.completion_token_ids == [11, 21, 22, 23, 24]
    assert seq.num_cached_tokens == len(seq) - 1 and seq.last_token == 24
    assert seq.num_accepted_draft == 3 and seq.num_verify_steps == 1


def test_eos_inside_accepted_path_truncates():
    s = make_scheduler(spec=True)
    seq = Sequence(prompt(50), SamplingParams(max_tokens=100))
    s.add(seq)
    run_prefill(s)
    seqs, _ = s.schedule()
    s.postprocess(seqs, [[21, EOS, 23, 24]], False)
    assert seq.is_finished and seq.completion_token_ids == [11, 21, EOS]
    assert not seq.block_table and s.is_finished()


def test_ignore_eos_and_max_tokens_mid_path():
    s = make_scheduler(spec=True)
    seq = Sequence(prompt(50), SamplingParams(max_tokens=3, ignore_eos=True))
    s.add(seq)
    run_prefill(s)
    seqs, _ = s.schedule()
    s.postprocess(seqs, [[EOS, 22, 23, 24]], False)
    assert seq.is_finished and seq.completion_token_ids == [11, EOS, 22]


def test_preemption_when_lookahead_does_not_fit():
    s = make_scheduler(num_blocks=3, spec=True, k=5)
    a = Sequence(prompt(254), SamplingParams(max_tokens=50))
    b = Sequence(prompt(254, 300), SamplingParams(max_tokens=50))
    s.add(a)
    s.add(b)
    seqs, _ = s.schedule()
    s.postprocess(seqs, [11, 11], True)  # each holds 1 block (255 tokens), 1 block free
    seqs, is_prefill = s.schedule()  # each needs a 2nd block for rows 254..259
    assert not is_prefill
    assert seqs == [a] and b.status == SequenceStatus.WAITING and not b.block_table
    assert len(a.block_table) == 2


def test_prefix_hashes_after_multi_token_steps():
    s = make_scheduler(spec=True, k=5)
    seq = Sequence(prompt(250), SamplingParams(max_tokens=100))
    s.add(seq)
    run_prefill(s)
    for step in range(3):
        seqs, _ = s.schedule()
        s.postprocess(seqs, [[30 + step, 31 + step, 32 + step]], False)
    # block 0 (positions 0..255) is complete and cached: its key names its tokens
    bm = s.block_manager
    b0 = seq.block_table[0]
    assert seq.num_cached_tokens >= 256
    assert bm.keys[b0] == block_key(seq.block(0)) and bm.contents[b0] == tuple(seq.block(0))
    # a new sequence with the same first 256 tokens hits the prefix cache
    twin = Sequence(seq.token_ids[:300], SamplingParams())
    assert bm.can_allocate(twin) == 1


def test_prefix_cache_reuse_release_and_eviction():
    """A released block stays a cache hit until it is handed out again; a hit on a
    free block takes it back, a hit on a held block shares it; the block released
    longest ago is reused first; content is compared, not only keys."""
    bm = BlockManager(4, BS)
    a = Sequence(list(range(600)))           # 3 blocks, 2 full blocks before the last
    bm.allocate(a, bm.can_allocate(a))
    assert bm.num_free_blocks == 1 and bm.can_allocate(a) == -1  # no hits, 3 > 1 free
    a.num_scheduled_tokens = 600
    bm.hash_blocks(a)                         # publishes blocks 0 and 1 (512 tokens)
    a.num_cached_tokens, a.num_scheduled_tokens = 600, 0
    b = Sequence(list(range(520)))
    assert bm.can_allocate(b) == 2           # shares 2 held blocks, needs 1 free
    bm.allocate(b, 2)
    assert b.block_table[:2] == a.block_table[:2] and b.num_cached_tokens == 512
    assert bm.refs[a.block_table[0]] == 2 and bm.num_free_blocks == 0
    held = list(a.block_table)
    bm.deallocate(a)
    bm.deallocate(b)
    assert bm.num_free_blocks == 4 and (bm.refs == 0).all()
    c = Sequence(list(range(513)))
    assert bm.can_allocate(c) == 2          # released blocks are still hits
    bm.allocate(c, 2)
    assert c.block_table[:2] == held[:2] and bm.num_free_blocks == 1
    # same key, different content: a collision is never a hit
    d = Sequence(list(range(300)))
    assert bm._cached_prefix(d) == [c.block_table[0]]
    bm.contents[c.block_table[0]] = (7,) * 256
    assert bm._cached_prefix(d) == []
    with pytest.raises(RuntimeError):
        bm.allocate(c, 0)                    # c already holds blocks


def test_draft_prefix_keys_cover_the_next_token():
    """EAGLE-3 drafting (key_next_token): the draft K/V row at a block's last position is
    computed from the token after the block, so a prefix hit needs that token to match
    too.  Two prompts sharing a full block but differing in the next token share nothing;
    with the same next token they share the block.  Without the flag the next token
    plays no part."""
    for flag, hits_diff in ((True, 0), (False, 1)):
        bm = BlockManager(8, BS, key_next_token=flag)
        a = Sequence(list(range(300)))
        bm.allocate(a, bm.can_allocate(a))
        a.num_scheduled_tokens = 300
        bm.hash_blocks(a)
        a.num_cached_tokens, a.num_scheduled_tokens = 300, 0
        diff = Sequence(list(range(256)) + [9999] + list(range(257, 300)))
        same = Sequence(list(range(290)))
        assert bm.can_allocate(diff) == hits_diff
        assert bm.can_allocate(same) == 1
    # a block's key is never formed before the token after it exists
    bm = BlockManager(8, BS, key_next_token=True)
    full = Sequence(list(range(2 * BS)))
    bm.allocate(full, 0)
    full.num_scheduled_tokens = 2 * BS
    bm.hash_blocks(full)                      # block 1's next token is not known yet
    assert len(full.block_hashes) == 1 and bm.keys[full.block_table[1]] is None
    with pytest.raises(ValueError):
        bm._keys_of(full, 2)


def test_eagle_prefill_publishes_the_prompt_end_block_after_sampling():
    """With EAGLE-3 the scheduler publishes a prefill's blocks after the sampled token
    joins the history, so a prompt that ends on a block boundary still publishes its
    last block (keyed with the sampled token)."""
    cfg = Config("unused", hf_config=Qwen3Config(max_position_embeddings=8192),
                 num_kvcache_blocks=16, speculative_method="eagle3", num_speculative_tokens=31)
    cfg.eos = EOS
    Sequence.block_size = BS
    s = Scheduler(cfg)
    assert s.block_manager.key_next_token
    a = Sequence(prompt(2 * BS), SamplingParams(max_tokens=8))
    s.add(a)
    run_prefill(s)                            # samples token 11 after the prompt
    bm = s.block_manager
    assert a.num_cached_tokens == 2 * BS and a.token_ids[-1] == 11
    assert all(bm.keys[b] is not None for b in a.block_table[:2])
    # a later prompt continuing with the same token hits both blocks, another does not
    assert bm.can_allocate(Sequence(prompt(2 * BS) + [11, 12])) == 2
    assert bm.can_allocate(Sequence(prompt(2 * BS) + [13, 12])) == 1


def test_chunked_prefill_fills_the_budget():
    """The token budget is filled: the last sequence admitted may take a chunk and
    stays at the head of the waiting queue until its prompt is cached."""
    cfg = Config("unused", hf_config=Qwen3Config(max_position_embeddings=8192),
                 num_kvcache_blocks=16, max_num_batched_tokens=1000)
    cfg.eos = EOS
    s = Scheduler(cfg)
    a, b = Sequence(prompt(600)), Sequence(prompt(700, 300))
    s.add(a)
    s.add(b)
    seqs, is_prefill = s.schedule()
    assert is_prefill and seqs == [a, b]
    assert a.num_scheduled_tokens == 600 and b.num_scheduled_tokens == 400
    s.postprocess(seqs, [11, 99], True)
    assert a.completion_token_ids == [11] and b.completion_token_ids == [] and b.num_cached_tokens == 400
    seqs, is_prefill = s.schedule()
    assert is_prefill and seqs == [b] and b.num_scheduled_tokens == 300
    s.postprocess(seqs, [12], True)
    assert b.completion_token_ids == [12] and list(s.running) == [a, b]


def test_preempted_sequence_is_recomputed():
    """A preempted sequence returns to the head of the waiting queue and its whole
    history (prompt and completion) is prefilled again."""
    s = make_scheduler(num_blocks=3, spec=True, k=5)
    a = Sequence(prompt(254), SamplingParams(max_tokens=50))
    b = Sequence(prompt(254, 300), SamplingParams(max_tokens=50))
    s.add(a)
    s.add(b)
    seqs, _ = s.schedule()
    s.postprocess(seqs, [11, 11], True)
    seqs, is_prefill = s.schedule()        # both need a 2nd block, one is free: b goes
    assert not is_prefill and seqs == [a] and b.status == SequenceStatus.WAITING
    s.postprocess(seqs, [[21]], False)
    assert len(b) == 255 and b.num_cached_tokens == 0 and not b.block_table
    seqs, is_prefill = s.schedule()
    assert is_prefill and seqs == [b] and b.num_scheduled_tokens == 255
    s.postprocess(seqs, [12], True)
    assert b.completion_token_ids == [11, 12] and list(s.running) == [a, b]


def test_blocks_needed_formula():
    bm = BlockManager(8, BS)
    seq = Sequence(list(range(256)))
    bm.allocate(seq, 0)
    assert len(seq.block_table) == 1
    seq.append_token(1)  # len 257: root at position 256
    assert bm.blocks_needed(seq, 1) == 1 and bm.blocks_needed(seq, 300) == 2
    with pytest.raises(AssertionError):
        Config("unused", hf_config=Qwen3Config(), tensor_parallel_size=2)


def test_slot_mapping_from_block_tables():
    """The verify step's slot mapping, computed from the padded block tables with
    tensor ops (run here on CPU tensors), equals page * block_size + offset for every
    position inside a sequence's table and is negative past its end."""
    import types

    import torch

    from nanovllm.engine.model_runner import ModelRunner

    r = types.SimpleNamespace(block_size=256)
    r._slots_of = lambda *a: ModelRunner._slots_of(r, *a)
    tables = [[5, 2, 9], [7], [3, 4]]
    bt = torch.full((3, 3), -1, dtype=torch.int32)
    for b, t in enumerate(tables):
        bt[b, :len(t)] = torch.tensor(t, dtype=torch.int32)
    start = torch.tensor([300, 10, 500])
    grid = ModelRunner._slot_grid(r, bt, start, 40)
    for b, t in enumerate(tables):
        for i in range(40):
            p = int(start[b]) + i
            want = t[p // 256] * 256 + p % 256 if p // 256 < len(t) else -1
            assert int(grid[b, i]) == want, (b, i)
    # packed rows (sequence, position) as in the draft catch-up
    seq_of = torch.tensor([0, 0, 2, 1, 2])
    pos = torch.tensor([511, 512, 511, 0, 767])
    got = ModelRunner._slots_of(r, bt, seq_of, pos).tolist()
    assert got == [2 * 256 + 255, 9 * 256, 4 * 256 + 255, 7 * 256, -1]
