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
    """Host-facing drafter: token histories (lists) in, draft token lists out.

    ``propose(histories)`` packs every history on each call.  ``propose_seqs(keys,
    histories)`` keeps each sequence's history resident on the device (one row of
    ``capacity`` tokens per sequence, keyed by ``keys``) and copies only the tokens
    appended since the previous call; ``drop(key)`` releases a finished sequence's
    row.  Histories must only grow between calls (as ``Sequence.token_ids`` does).
    """

    def __init__(self, max_ngram=3, min_ngram=1, num_draft=5, device="cuda", capacity=4096):
        self.max_ngram, self.min_ngram, self.num_draft = max_ngram, min_ngram, num_draft
        self.device = torch.device(device)
        self.capacity = capacity
        self._slot, self._known, self._free = {}, {}, []
        self._hist = None  # device int32 [rows, capacity]

    def _run(self, tokens, offsets):
        draft, dlen = ngram_propose(tokens, offsets, self.max_ngram, self.min_ngram, self.num_draft)
        draft, dlen = draft.cpu().tolist(), dlen.cpu().tolist()
        return [d[:n] for d, n in zip(draft, dlen)]

    def propose(self, histories):
        lens = [len(h) for h in histories]
        offs = [0]
        for n in lens:
            offs.append(offs[-1] + n)
        flat = [t for h in histories for t in h]
        tokens = torch.tensor(flat, dtype=torch.int32, pin_memory=True).to(self.device, non_blocking=True)
        offsets = torch.tensor(offs, dtype=torch.int64, pin_memory=True).to(self.device, non_blocking=True)
        return self._run(tokens, offsets)

    def _row(self, key):
        row = self._slot.get(key)
        if row is not None:
            return row
        if self._free:
            row = self._free.pop()
        else:
            row = len(self._slot)
            rows = 0 if self._hist is None else self._hist.shape[0]
            if row >= rows:  # grow the resident buffer (doubling)
                grown = torch.empty(max(2 * rows, 64), self.capacity, dtype=torch.int32,
                                    device=self.device)
                if self._hist is not None:
                    grown[:rows] = self._hist
                self._hist = grown
        self._slot[key] = row
        self._known[key] = 0
        return row

    def propose_seqs(self, keys, histories):
        rows, lens, new_vals, new_pos = [], [], [], []
        for key, h in zip(keys, histories):
            L = len(h)
            if L > self.capacity:
                raise ValueError(f"NgramProposer: history of {L} tokens exceeds the resident "
                                 f"capacity {self.capacity}")
            row = self._row(key)
            n0 = self._known[key]
            if L > n0:
                new_vals.extend(h[n0:])
                base = row * self.capacity
                new_pos.extend(range(base + n0, base + L))
                self._known[key] = L
            rows.append(row)
            lens.append(L)
        dev = self.device
        if new_vals:
            vals = torch.tensor(new_vals, dtype=torch.int32, pin_memory=True).to(dev, non_blocking=True)
            pos = torch.tensor(new_pos, dtype=torch.int64, pin_memory=True).to(dev, non_blocking=True)
            self._hist.view(-1).index_copy_(0, pos, vals)
        B, total = len(lens), sum(lens)
        lens_d = torch.tensor(lens, dtype=torch.int64, pin_memory=True).to(dev, non_blocking=True)
        rows_d = torch.tensor(rows, dtype=torch.int64, pin_memory=True).to(dev, non_blocking=True)
        offsets = torch.zeros(B + 1, dtype=torch.int64, device=dev)
        torch.cumsum(lens_d, 0, out=offsets[1:])
        # packed gather of the resident rows: flat index i belongs to sequence seq[i]
        seq = torch.repeat_interleave(torch.arange(B, device=dev), lens_d, output_size=total)
        col = torch.arange(total, device=dev) - offsets[:-1][seq]
        tokens = self._hist.view(-1)[rows_d[seq] * self.capacity + col]
        return self._run(tokens, offsets)

    def drop(self, key):
        row = self._slot.pop(key, None)
        if row is not None:
            self._known.pop(key, None)
            self._free.append(row)
