"""Oracle: n-gram prompt-lookup drafter (integer only).

Semantics follow transformers 5.15 ``PromptLookupCandidateGenerator.get_candidates``
(generation/candidate_generator.py:1076-1096), with ``max_length`` unbounded and
no logits processor / EOS cropping:

    for n = min(max_ngram, L-1) down to min_ngram:
        scan windows h[i:i+n] left to right; the first i with h[i:i+n] == h[L-n:L]
        and i+n < L wins; propose h[i+n : min(i+n+k, L)] and stop.
    no match -> no proposal.

The reference (nano-vllm 0.2.0) has no drafter; its input is
``Sequence.token_ids`` (nanovllm/engine/sequence.py:21, :67-70).

Pinned by: transformers' own routine at B=1 (tests/test_oracle_ngram.py),
brute force vs the vectorised form, and closed-form cases (no repeats -> empty,
planted copy -> exact continuation, match near the end -> truncated, L <= n).
"""
import numpy as np


def propose_one_bruteforce(h, max_ngram=3, min_ngram=1, k=5):
    """Literal restatement of candidate_generator.py:1076-1096 (pure Python)."""
    h = [int(x) for x in h]
    L = len(h)
    for n in range(min(max_ngram, L - 1), min_ngram - 1, -1):
        suffix = h[L - n:]
        for i in range(0, L - n + 1):
            if h[i:i + n] == suffix:
                s, e = i + n, min(i + n + k, L)
                if s < e:
                    return h[s:e]
    return []


def propose_one(h, max_ngram=3, min_ngram=1, k=5):
    """Vectorised form of the same rule.

    A window of size n that ends at e (exclusive, e = i + n) matches the suffix
    iff h[e-t] == h[L-t] for t = 1..n.  With ml(e) = length of that backward match
    (capped at max_ngram), size n matches at e iff ml(e) >= n, and the earliest
    window is the smallest such e.  Proposals need e <= L-1.
    """
    h = np.asarray(h, dtype=np.int64)
    L = h.shape[0]
    nmax = min(max_ngram, L - 1)
    if nmax < min_ngram:
        return []
    e = np.arange(L)  # candidate window ends, valid ones are 1..L-1
    ml = np.zeros(L, dtype=np.int64)
    alive = np.ones(L, dtype=bool)
    for t in range(1, nmax + 1):
        idx = e - t
        ok = alive & (idx >= 0) & (e <= L - 1)
        ok[ok] = h[idx[ok]] == h[L - t]
        alive = ok
        ml += alive
    for n in range(nmax, min_ngram - 1, -1):
        cand = np.nonzero((ml >= n) & (e >= n) & (e <= L - 1))[0]
        if cand.size:
            s = int(cand[0])
            return h[s:min(s + k, L)].tolist()
    return []


def ngram_propose(tokens, offsets, max_ngram=3, min_ngram=1, k=5):
    """Batched oracle over a packed CSR batch.

    tokens: int32 [sum L]; offsets: int64 [B+1].
    Returns (draft int32 [B, k] padded with -1, draft_len int32 [B]).
    """
    tokens = np.asarray(tokens)
    offsets = np.asarray(offsets, dtype=np.int64)
    B = offsets.shape[0] - 1
    draft = np.full((B, k), -1, dtype=np.int32)
    draft_len = np.zeros(B, dtype=np.int32)
    for b in range(B):
        p = propose_one(tokens[offsets[b]:offsets[b + 1]], max_ngram, min_ngram, k)
        draft[b, :len(p)] = p
        draft_len[b] = len(p)
    return draft, draft_len
