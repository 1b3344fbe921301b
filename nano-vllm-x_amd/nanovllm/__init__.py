"""nano-vllm-x on MI355X: the speculative-decoding verify path as gfx950 HIP kernels
behind nano-vllm's interfaces (``from nanovllm import LLM, SamplingParams``)."""
from nanovllm.sampling_params import SamplingParams


def __getattr__(name):
    if name == "LLM":
        from nanovllm.llm import LLM
        return LLM
    raise AttributeError(name)


__all__ = ["LLM", "SamplingParams"]
