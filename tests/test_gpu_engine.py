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
from nanovllm.utils.context import reset_context


def tiny_config():
    cfg = Qwen3Config(hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=128,
                      vocab_size=512, max_position_embeddings=4096, rms_norm_eps=1e-6,
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
              speculative_method="ngram", num_speculative_tokens=5, max_num_batched_tokens=4096)
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
              speculative_method="ngram", num_speculative_tokens=4, max_num_batched_tokens=4096)
    ps = prompts()
    sps = [SamplingParams(temperature=t, max_tokens=40, ignore_eos=True) for t in (0.0, 0.6, 1.0, 0.0)]
    outs = llm.generate(ps, sps, use_tqdm=False)
    assert [len(o["token_ids"]) for o in outs] == [40] * 4
    assert all(0 <= t < 512 for o in outs for t in o["token_ids"])


@pytest.mark.gpu
def test_plain_decode_equals_argmax(dev):
    llm = LLM("unused", hf_config=tiny_config(), num_kvcache_blocks=64, max_num_batched_tokens=4096)
    p = prompts()[1]
    out = llm.generate([p], SamplingParams(temperature=0.0, max_tokens=20, ignore_eos=True),
                       use_tqdm=False)[0]["token_ids"]
    logits = full_logits(llm, p + out)
    agree = sum(int(logits[len(p) + j - 1].argmax()) == t for j, t in enumerate(out))
    assert agree >= 19
