"""Offline engine: a Scheduler and one in-process ModelRunner on one GPU.

Keeps the reference's entry points (nanovllm/engine/llm_engine.py:15-90):
``LLMEngine(model, **config_kwargs)`` (unknown kwargs are ignored),
``add_request(prompt, sampling_params)``, ``step() -> (finished outputs,
num_tokens)`` with num_tokens > 0 for a prefill step and < 0 (minus the tokens
produced) for a decode step, ``is_finished()`` and
``generate(prompts, sampling_params, use_tqdm) -> [{"text", "token_ids"}]`` in
prompt order.  A verify step may produce several tokens per sequence.  Prompts may
be token-id lists; text prompts and decoded text need a tokenizer in the model
directory (random-init runs have none).
"""
import atexit
import os
from dataclasses import fields
from time import perf_counter

from nanovllm.config import Config
from nanovllm.engine.model_runner import ModelRunner
from nanovllm.engine.scheduler import Scheduler
from nanovllm.engine.sequence import Sequence
from nanovllm.sampling_params import SamplingParams

_CONFIG_FIELDS = frozenset(f.name for f in fields(Config))


def _load_tokenizer(model):
    if not (model and os.path.isdir(model)):
        return None
    if not any(os.path.exists(os.path.join(model, f))
               for f in ("tokenizer.json", "tokenizer_config.json")):
        return None
    from transformers import AutoTokenizer
    return AutoTokenizer.from_pretrained(model, use_fast=True)


class LLMEngine:

    def __init__(self, model, **kwargs):
        config = Config(model, **{k: v for k, v in kwargs.items() if k in _CONFIG_FIELDS})
        Sequence.block_size = config.kvcache_block_size
        self.tokenizer = _load_tokenizer(model)
        if self.tokenizer is not None:
            config.eos = self.tokenizer.eos_token_id
        elif config.eos == -1:
            config.eos = getattr(config.hf_config, "eos_token_id", None) or -1
        self.config = config
        self.model_runner = ModelRunner(config, 0)
        self.scheduler = Scheduler(config)
        # largest position a step may rotate: the RoPE table covers
        # max_position_embeddings positions
        self._max_positions = config.hf_config.max_position_embeddings
        atexit.register(self.exit)

    def exit(self):
        runner, self.model_runner = getattr(self, "model_runner", None), None
        if runner is not None:
            runner.call("exit")

    # ------------------------------------------------------------ requests
    def add_request(self, prompt: str | list[int], sampling_params: SamplingParams):
        if isinstance(prompt, str):
            if self.tokenizer is None:
                raise ValueError("text prompts need a tokenizer in the model directory")
            prompt = self.tokenizer.encode(prompt)
        # The engine is sized for max_model_len tokens per sequence (the graphs' block
        # tables, the n-gram history buffers), and every position a step writes
        # (prompt, completion, draft rows) must have a RoPE table entry.
        length = len(prompt) + sampling_params.max_tokens
        if length > self.config.max_model_len:
            raise ValueError(f"prompt of {len(prompt)} tokens + max_tokens "
                             f"{sampling_params.max_tokens} exceeds max_model_len "
                             f"{self.config.max_model_len}")
        span = length + self.config.verify_lookahead
        if span > self._max_positions:
            raise ValueError(f"prompt of {len(prompt)} tokens + max_tokens "
                             f"{sampling_params.max_tokens} + {self.config.verify_lookahead} "
                             f"draft rows exceeds the model's {self._max_positions} positions")
        seq = Sequence(prompt, sampling_params)
        self.scheduler.add(seq)
        return seq.seq_id

    def is_finished(self):
        return self.scheduler.is_finished()

    def step(self):
        seqs, is_prefill = self.scheduler.schedule()
        token_ids = self.model_runner.call("run", seqs, is_prefill)
        if is_prefill:
            num_tokens = sum(seq.num_scheduled_tokens for seq in seqs)
        else:
            num_tokens = -sum(1 if isinstance(t, int) else len(t) for t in token_ids)
        self.scheduler.postprocess(seqs, token_ids, is_prefill)
        finished = [seq for seq in seqs if seq.is_finished]
        for seq in finished:
            self.model_runner.drop_draft_state(seq.seq_id)
        return [(seq.seq_id, seq.completion_token_ids) for seq in finished], num_tokens

    # ------------------------------------------------------------ generate
    def generate(self, prompts, sampling_params, use_tqdm: bool = True):
        params = sampling_params if isinstance(sampling_params, list) \
            else [sampling_params] * len(prompts)
        if len(params) != len(prompts):
            raise ValueError("one SamplingParams per prompt (or a single one for all)")
        order = {self.add_request(p, sp): i for i, (p, sp) in enumerate(zip(prompts, params))}
        results = [None] * len(prompts)
        bar = None
        if use_tqdm:
            from tqdm.auto import tqdm
            bar = tqdm(total=len(prompts), desc="Generating", dynamic_ncols=True)
        rate = {"Prefill": 0, "Decode": 0}
        while not self.is_finished():
            t0 = perf_counter()
            done, num_tokens = self.step()
            rate["Prefill" if num_tokens > 0 else "Decode"] = int(abs(num_tokens) / (perf_counter() - t0))
            for seq_id, token_ids in done:
                results[order[seq_id]] = token_ids
            if bar is not None:
                bar.set_postfix({k: f"{v}tok/s" for k, v in rate.items()})
                bar.update(len(done))
        if bar is not None:
            bar.close()
        decode = self.tokenizer.decode if self.tokenizer is not None else (lambda ids: "")
        return [{"text": decode(ids), "token_ids": ids} for ids in results]
