"""N-gram prompt-lookup drafter on libnvx_spec.

The reference (nano-vllm 0.2.0) has no drafter; its input is the token history
``Sequence.token_ids`` (nanovllm/engine/sequence.py:21, :67-70).  Semantics are
those of transformers' PromptLookupCandidateGenerator.get_candidates
(generation/candidate_generator.py:1076-1096): for n = min(max_ngram, L-1) down
to min_ngram, the left-most earlier occurrence of the last n tokens with a
non-empty continuation wins and up to ``num_draft`` following tokens are proposed.
"""
import torch

from .. import _C


def ngram_propose(tokens: torch.Tensor, offsets: torch.Tensor, max_ngram: int = 3,
                  min_ngram: int = 1, num_draft: int = 5):
    """tokens int32 [sum L] (device); offsets int64 [B+1] (device).

    Returns (draft int32 [B, num_draft] padded with -1, draft_len int32 [B])."""
    if tokens.dtype != torch.int32 or offsets.dtype != torch.int64:
        raise ValueError("ngram_propose: tokens must be int32 and offsets int64")
    tokens, offsets = tokens.contiguous(), offsets.contiguous()
    B = offsets.numel() - 1
    draft = torch.empty(B, num_draft, dtype=torch.int32, device=offsets.device)
    draft_len = torch.empty(B, dtype=torch.int32, device=offsets.device)
    _C.require_cuda(tokens, offsets)
    _C.check(_C.lib().nvx_ngram_propose(_C.ptr(tokens), _C.ptr(offsets), B, min_ngram, max_ngram,
                                        num_draft, _C.ptr(draft), _C.ptr(draft_len),
                                        _C.stream_of(offsets)))
    return draft, draft_len


class NgramProposer:
    """Host-facing drafter: token histories (lists) in, draft token lists out."""

    def __init__(self, max_ngram=3, min_ngram=1, num_draft=5, device="cuda"):
        self.max_ngram, self.min_ngram, self.num_draft = max_ngram, min_ngram, num_draft
        self.device = torch.device(device)

    def propose(self, histories):
        lens = [len(h) for h in histories]
        offs = [0]
        for n in lens:
            offs.append(offs[-1] + n)
        flat = [t for h in histories for t in h]
        tokens = torch.tensor(flat, dtype=torch.int32, pin_memory=True).to(self.device, non_blocking=True)
        offsets = torch.tensor(offs, dtype=torch.int64, pin_memory=True).to(self.device, non_blocking=True)
        draft, dlen = ngram_propose(tokens, offsets, self.max_ngram, self.min_ngram, self.num_draft)
        draft, dlen = draft.cpu().tolist(), dlen.cpu().tolist()
        return [d[:n] for d, n in zip(draft, dlen)]
