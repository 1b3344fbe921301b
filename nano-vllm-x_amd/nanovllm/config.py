"""Config, as in the reference (nanovllm/config.py:6-25), plus speculative
decoding fields (unknown kwargs are filtered by LLMEngine as in
llm_engine.py:18-20, so the additions are backward compatible).  ``hf_config``
may be passed directly (a transformers config object) for checkpoint-free,
random-init runs; otherwise it is read from the local model directory."""
import os
from dataclasses import dataclass

from transformers import AutoConfig


@dataclass(slots=True)
class Config:
    model: str
    max_num_batched_tokens: int = 16384
    max_num_seqs: int = 512
    max_model_len: int = 4096
    gpu_memory_utilization: float = 0.9
    tensor_parallel_size: int = 1
    enforce_eager: bool = True
    hf_config: AutoConfig | None = None
    eos: int = -1
    kvcache_block_size: int = 256
    num_kvcache_blocks: int = -1
    # speculative decoding: "none" or "ngram"
    speculative_method: str = "none"
    num_speculative_tokens: int = 5
    ngram_max: int = 3
    ngram_min: int = 1
    seed: int = 0

    def __post_init__(self):
        assert self.kvcache_block_size % 256 == 0
        assert self.tensor_parallel_size == 1, "this build drives one GPU"
        assert self.speculative_method in ("none", "ngram")
        if self.hf_config is None:
            assert os.path.isdir(self.model)
            self.hf_config = AutoConfig.from_pretrained(self.model)
        self.max_model_len = min(self.max_model_len, self.hf_config.max_position_embeddings)

    @property
    def verify_lookahead(self) -> int:
        """KV positions a decode step writes per sequence (root + draft rows)."""
        return 1 if self.speculative_method == "none" else 1 + self.num_speculative_tokens
