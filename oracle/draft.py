"""Oracle: draft-head top-k log-probabilities (float64 numpy).

TEST INFRASTRUCTURE ONLY (see the package docstring).

EAGLE-2 tree expansion (Li et al. 2024, arXiv:2406.16858, Sec. 4) grows every
frontier node by the k most likely tokens of the draft distribution, scored by
log-probability; EAGLE-3 (arXiv:2503.01840) keeps that expansion.  The reference
(nano-vllm 0.2.0) has no draft head, so no reference file is restated here; the
contract of ``nvx_topk_logprobs`` is the one of ``torch.log_softmax`` followed by
``torch.topk`` with a fixed tie rule:

* ``logprob[y] = (x[y] - max) - ln(sum_v exp(x[v] - max))``;
* tokens by descending logprob; equal values ordered by the lower token id.

Pinned in tests/test_oracle_draft.py against torch.log_softmax + torch.topk on
tie-free rows, closed forms (a constant row; a row with two levels), and a
brute-force Python sort of (value, token) pairs on small rows with many ties.
"""
import numpy as np


def topk_logprobs(logits, k):
    """logits [N, V] (any real dtype; bf16 values given as float32) -> (tokens int32
    [N, k], logprobs float64 [N, k])."""
    x = np.asarray(logits, dtype=np.float64)
    if x.ndim != 2 or not 1 <= k <= x.shape[1]:
        raise ValueError("topk_logprobs: logits must be [N, V] with 1 <= k <= V")
    m = x.max(axis=1, keepdims=True)
    lse = m + np.log(np.exp(x - m).sum(axis=1, keepdims=True))
    # stable sort of -x: descending values, equal values by ascending index
    order = np.argsort(-x, axis=1, kind="stable")[:, :k]
    return order.astype(np.int32), np.take_along_axis(x - lse, order, axis=1)
