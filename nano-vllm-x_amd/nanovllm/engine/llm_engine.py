"""LLMEngine, as in the reference (nanovllm/engine/llm_engine.py:15-90), driving one
GPU in-process.  ``step`` handles prefill and (speculative) decode; a verify step
returns several tokens per sequence.  Prompts may be token-id lists; text prompts
and decoded text need a tokenizer in the model directory."""
import atexit
import os
from dataclasses import fields
from time import perf_counter

from tqdm.auto import tqdm

from nanovllm.config import Config
from nanovllm.engine.model_runner import ModelRunner
from nanovllm.engine.scheduler import Scheduler
from nanovllm.engine.sequence import Sequence
from nanovllm.sampling_params import SamplingParams


class LLMEngine:

    def __init__(self, model, **kwargs):
        config_fields = {field.name for field in fields(Config)}
        config_kwargs = {k: v for k, v in kwargs.items() if k in config_fields}
        config = Config(model, **config_kwargs)
        Sequence.block_size = config.kvcache_block_size
        self.model_runner = ModelRunner(config, 0)
        self.tokenizer = None
        if model and os.path.isdir(model) and any(
                os.path.exists(os.path.join(model, f)) for f in ("tokenizer.json", "tokenizer_config.json")):
            from transformers import AutoTokenizer
            self.tokenizer = AutoTokenizer.from_pretrained(model, use_fast=True)
            config.eos = self.tokenizer.eos_token_id
        elif config.eos == -1:
            config.eos = getattr(config.hf_config, "eos_token_id", -1) or -1
        self.config = config
        self.scheduler = Scheduler(config)
        atexit.register(self.exit)

    def exit(self):
        if getattr(self, "model_runner", None) is not None:
            self.model_runner.call("exit")
            self.model_runner = None

    def add_request(self, prompt: str | list[int], sampling_params: SamplingParams):
        if isinstance(prompt, str):
            assert self.tokenizer is not None, "text prompts need a tokenizer in the model dir"
            prompt = self.tokenizer.encode(prompt)
        self.scheduler.add(Sequence(prompt, sampling_params))

    def step(self):
        seqs, is_prefill = self.scheduler.schedule()
        num_tokens = sum(seq.num_scheduled_tokens for seq in seqs) if is_prefill else -len(seqs)
        token_ids = self.model_runner.call("run", seqs, is_prefill)
        if not is_prefill:
            num_tokens = -sum(len(t) for t in token_ids)
        self.scheduler.postprocess(seqs, token_ids, is_prefill)
        outputs = [(seq.seq_id, seq.completion_token_ids) for seq in seqs if seq.is_finished]
        for seq in seqs:
            if seq.is_finished:
                self.model_runner.drop_draft_state(seq.seq_id)
        return outputs, num_tokens

    def is_finished(self):
        return self.scheduler.is_finished()

    def generate(self, prompts, sampling_params, use_tqdm: bool = True):
        pbar = tqdm(total=len(prompts), desc="Generating", dynamic_ncols=True, disable=not use_tqdm)
        if not isinstance(sampling_params, list):
            sampling_params = [sampling_params] * len(prompts)
        for prompt, sp in zip(prompts, sampling_params):
            self.add_request(prompt, sp)
        outputs = {}
        prefill_throughput = decode_throughput = 0.
        while not self.is_finished():
            t = perf_counter()
            output, num_tokens = self.step()
            if num_tokens > 0:
                prefill_throughput = num_tokens / (perf_counter() - t)
            else:
                decode_throughput = -num_tokens / (perf_counter() - t)
            pbar.set_postfix({"Prefill": f"{int(prefill_throughput)}tok/s",
                              "Decode": f"{int(decode_throughput)}tok/s"})
            for seq_id, token_ids in output:
                outputs[seq_id] = token_ids
                pbar.update(1)
        pbar.close()
        outputs = [outputs[seq_id] for seq_id in sorted(outputs.keys())]
        decode = self.tokenizer.decode if self.tokenizer is not None else (lambda ids: "")
        return [{"text": decode(token_ids), "token_ids": token_ids} for token_ids in outputs]
