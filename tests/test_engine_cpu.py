"""Scheduler / BlockManager / Sequence with scripted tokens (no GPU): the reference's
one-token decode behaviour, and the verify step's multi-token accounting."""
import pytest
from transformers import Qwen3Config

from nanovllm.config import Config
from nanovllm.engine.block_manager import BlockManager
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
    # block 0 (positions 0..255) is complete and cached: its hash names its tokens
    bm = s.block_manager
    blk = bm.blocks[seq.block_table[0]]
    assert seq.num_cached_tokens >= 256
    assert blk.hash == BlockManager.compute_hash(seq.block(0)) and blk.token_ids == seq.block(0)
    # a new sequence with the same first 256 tokens hits the prefix cache
    twin = Sequence(seq.token_ids[:300], SamplingParams())
    assert bm.can_allocate(twin) == 1


def test_blocks_needed_formula():
    bm = BlockManager(8, BS)
    seq = Sequence(list(range(256)))
    bm.allocate(seq, 0)
    assert len(seq.block_table) == 1
    seq.append_token(1)  # len 257: root at position 256
    assert bm.blocks_needed(seq, 1) == 1 and bm.blocks_needed(seq, 300) == 2
    with pytest.raises(AssertionError):
        Config("unused", hf_config=Qwen3Config(), tensor_parallel_size=2)
