"""Per-forward side channel from the model runner to the attention layers.

Mirrors nanovllm/utils/context.py:5-27 of the reference (same fields and
functions); the verify step adds the draft-tree mask and the maximum context
length, both defaulting to "absent" so existing callers are unchanged.
"""
from dataclasses import dataclass

import torch


@dataclass(slots=True)
class Context:
    is_prefill: bool = False
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    # verify step: uint64 ancestor bitmask per query row (stored as int64), or None
    tree_mask: torch.Tensor | None = None
    # decode / verify step: q rows per sequence are cu_seqlens_q[b+1] - cu_seqlens_q[b]
    max_context_len: int = 0


_CONTEXT = Context()


def get_context():
    return _CONTEXT


def set_context(is_prefill, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=0, max_seqlen_k=0,
                slot_mapping=None, context_lens=None, block_tables=None, tree_mask=None,
                max_context_len=0):
    global _CONTEXT
    _CONTEXT = Context(is_prefill, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                       slot_mapping, context_lens, block_tables, tree_mask, max_context_len)


def reset_context():
    global _CONTEXT
    _CONTEXT = Context()
