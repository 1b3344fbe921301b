"""SamplingParams, as in the reference (nanovllm/sampling_params.py:4-11).

The reference forbids greedy sampling (:11); the verify path supports it, so
temperature 0 means greedy (argmax acceptance and argmax next token).
"""
from dataclasses import dataclass


@dataclass(slots=True)
class SamplingParams:
    temperature: float = 1.0
    max_tokens: int = 64
    ignore_eos: bool = False

    def __post_init__(self):
        assert self.temperature >= 0.0, "temperature must be >= 0 (0 = greedy)"
