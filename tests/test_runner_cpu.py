"""Host-side checks of the verify step's post-walk handling and of request admission
(no GPU): the model forward and the walk are replaced by scripted outputs.

The reference's step either returns its tokens or stops on an assert
(nanovllm/engine/model_runner.py:214-220, scheduler.py:71); here a walk whose
workgroups failed to meet writes accepted_len = -1, and the step must raise before
any of it is counted, handed to the scheduler or used as a draft root.
"""
import pytest
import torch
from transformers import Qwen3Config

from nanovllm.config import Config
from nanovllm.engine.llm_engine import LLMEngine
from nanovllm.engine.model_runner import ModelRunner
from nanovllm.engine.scheduler import Scheduler
from nanovllm.engine.sequence import Sequence
from nanovllm.sampling_params import SamplingParams

BS = 256


def make_config(max_model_len=4096, max_pos=8192, k=5):
    cfg = Config("unused", hf_config=Qwen3Config(max_position_embeddings=max_pos),
                 num_kvcache_blocks=32, max_model_len=max_model_len,
                 speculative_method="ngram", num_speculative_tokens=k)
    cfg.eos = -1
    Sequence.block_size = BS
    return cfg


def scripted_runner(acc, out_tokens, T):
    """A ModelRunner whose forward, drafter and walk are scripted: the n-gram verify
    path of ModelRunner.run runs unchanged around them."""
    B = len(acc)
    r = object.__new__(ModelRunner)
    r.draft = None
    r.spec_stats = {"verify_rows": 0, "accepted": 0, "accepted_hist": {}}
    r.gen = torch.Generator().manual_seed(0)

    class Proposer:
        def propose_seqs(self, ids, histories):
            return [[1] * (T - 1) for _ in ids]

    r.proposer = Proposer()
    r.prepare_decode = lambda seqs, drafts: (torch.zeros(B * T, dtype=torch.int64),
                                             torch.zeros(B * T, dtype=torch.int64), T,
                                             torch.full((B,), T, dtype=torch.int32))
    r.prepare_sample = lambda seqs: torch.ones(B)
    r.run_model = lambda ids, pos, is_prefill: torch.zeros(B * T, 16)
    r._chain = lambda n: (torch.arange(-1, n - 1, dtype=torch.int32), None)

    def rejection(logits, temps, q, tokens, parents, U, Uf, num_nodes=None):
        assert U.shape == (B, T) and Uf.shape == (B,)
        return (torch.zeros(B, T, dtype=torch.int32), torch.tensor(acc, dtype=torch.int32),
                torch.tensor(out_tokens, dtype=torch.int32), torch.zeros(B, dtype=torch.int32))

    r.rejection = rejection
    return r


def scheduled_decode(cfg, n=2):
    s = Scheduler(cfg)
    seqs = [Sequence([100 + i] * 40, SamplingParams(max_tokens=50, ignore_eos=True))
            for i in range(n)]
    for seq in seqs:
        s.add(seq)
    batch, is_prefill = s.schedule()
    assert is_prefill
    s.postprocess(batch, [11] * len(batch), True)
    batch, is_prefill = s.schedule()
    assert not is_prefill
    return s, batch


def test_verified_tokens_refuses_failed_rows():
    r = scripted_runner([0], [[0]], 2)
    with pytest.raises(RuntimeError, match="walk failed for 1 of 3"):
        r._verified_tokens([2, -1, 0], [[5, 6, 7], [-1, -1, -1], [9, -1, -1]])
    assert r.spec_stats == {"verify_rows": 0, "accepted": 0, "accepted_hist": {}}
    assert r._verified_tokens([2, 0], [[5, 6, 7], [9, -1, -1]]) == [[5, 6, 7], [9]]
    assert r.spec_stats["accepted"] == 2 and r.spec_stats["accepted_hist"] == {2: 1, 0: 1}


def test_sampled_tokens_refuse_failed_rows():
    assert ModelRunner._sampled([3, 0, 7]) == [3, 0, 7]
    assert ModelRunner._sampled([]) == []
    with pytest.raises(RuntimeError, match="sampler walk failed for 1 of 3"):
        ModelRunner._sampled([3, -1, 7])


def test_failed_walk_row_stops_the_engine_step():
    """A scripted walk output with a -1 row goes through LLMEngine.step ->
    ModelRunner.run (n-gram verify) -> the post-walk check, which raises; the
    scheduler's sequences are left as they were."""
    cfg = make_config()
    T = 1 + cfg.num_speculative_tokens
    sched, batch = scheduled_decode(cfg)
    eng = object.__new__(LLMEngine)
    eng.scheduler = sched
    eng.model_runner = scripted_runner([1, -1], [[21, 22] + [-1] * (T - 2), [-1] * T], T)
    lens = [len(seq) for seq in batch]
    with pytest.raises(RuntimeError, match="walk failed"):
        eng.step()
    assert [len(seq) for seq in batch] == lens
    assert all(seq.num_verify_steps == 0 for seq in batch)
    assert eng.model_runner.spec_stats["verify_rows"] == 0


def test_good_walk_rows_reach_the_scheduler():
    cfg = make_config()
    T = 1 + cfg.num_speculative_tokens
    sched, batch = scheduled_decode(cfg)
    runner = scripted_runner([2, 0], [[21, 22, 23] + [-1] * (T - 3), [31] + [-1] * (T - 1)], T)
    out = runner.run(batch, False)
    assert out == [[21, 22, 23], [31]]
    sched.postprocess(batch, out, False)
    assert batch[0].completion_token_ids == [11, 21, 22, 23]
    assert batch[1].completion_token_ids == [11, 31]


def test_scheduler_refuses_empty_or_negative_decode_tokens():
    cfg = make_config()
    for bad in ([], [-1], [5, -1]):
        sched, batch = scheduled_decode(cfg, n=1)
        with pytest.raises(RuntimeError, match="at least one token id"):
            sched.postprocess(batch, [bad], False)


def test_admission_bound_is_max_model_len():
    """Requests are admitted only if prompt + max_tokens fits max_model_len, the length
    the graphs' block tables and the n-gram history buffers are sized for."""
    cfg = make_config(max_model_len=2048)
    eng = object.__new__(LLMEngine)
    eng.config, eng.tokenizer = cfg, None
    eng.scheduler = Scheduler(cfg)
    eng._max_positions = cfg.hf_config.max_position_embeddings
    eng.add_request([1] * 1000, SamplingParams(max_tokens=1048))  # exactly 2048
    with pytest.raises(ValueError, match="max_model_len 2048"):
        eng.add_request([1] * 1000, SamplingParams(max_tokens=1049))
    with pytest.raises(ValueError, match="max_model_len"):
        eng.add_request([1] * 4000, SamplingParams(max_tokens=1000))
    # positions beyond the RoPE table are refused even when max_model_len allows them
    cfg2 = make_config(max_model_len=8192, max_pos=8192)
    eng2 = object.__new__(LLMEngine)
    eng2.config, eng2.tokenizer = cfg2, None
    eng2.scheduler = Scheduler(cfg2)
    eng2._max_positions = 8192
    with pytest.raises(ValueError, match="positions"):
        eng2.add_request([1] * 4000, SamplingParams(max_tokens=4192))
