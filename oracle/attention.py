"""Oracle: paged attention with an ancestor (tree) mask, float32 numpy.

Semantics restated from the reference decode call
``flash_attn_with_kvcache(q, k_cache, v_cache, cache_seqlens=context_lens,
block_table=block_tables, softmax_scale=scale, causal=True)``
(nanovllm/layers/attention.py:72-74) generalised from q_len = 1 to a draft tree:

* The K/V of the q_len query rows were stored first (attention.py:62-63), so
  ``context_lens[b]`` counts them; the rows occupy positions
  ``base = context_lens[b] - q_len`` .. ``context_lens[b] - 1``.
* Keys at positions ``< base`` are visible to every query.  Key ``base + m`` is
  visible to query node ``i`` iff bit ``m`` of ``tree_mask[row(i)]`` is set (the
  ancestors-or-self of node i); with no mask the rule is causal, ``m <= i``
  (flash-attn's bottom-right aligned causal mask).
* GQA: query head h reads KV head ``h // (Hq // Hkv)`` (nanovllm/models/qwen3.py:79-81);
  scores are scaled by ``scale`` (head_dim ** -0.5, qwen3.py:39).
* Cache layout [num_blocks, block_size, Hkv, D] and slot arithmetic as in
  ``oracle.kvcache.slot_of``.

Pinned by tests/test_oracle_attention.py: torch's scaled_dot_product_attention on
gathered K/V with an explicit boolean mask (library routine), a chain tree equals
the causal rule, q_len = 1 equals plain decode, and permuting physical pages
together with the block table leaves the output unchanged.
"""
import numpy as np

from .kvcache import slot_of


def tree_visible(q_len, ctx_len, tree_mask_rows):
    """Boolean [q_len, ctx_len] visibility matrix for one sequence."""
    base = ctx_len - q_len
    vis = np.zeros((q_len, ctx_len), dtype=bool)
    vis[:, :base] = True
    m = np.arange(q_len)
    if tree_mask_rows is None:
        vis[:, base:] = m[None, :] <= m[:, None]
    else:
        bits = np.asarray(tree_mask_rows, dtype=np.uint64)
        vis[:, base:] = ((bits[:, None] >> m[None, :].astype(np.uint64)) & np.uint64(1)).astype(bool)
    return vis


def paged_attention(q, k_cache, v_cache, block_tables, cu_seqlens_q, context_lens,
                    tree_mask, scale, block_size):
    """q: float32 [N, Hq, D]; caches: float32 [num_blocks, block_size, Hkv, D];
    tree_mask: uint64 [N] or None.  Returns float32 [N, Hq, D]."""
    q = np.asarray(q, dtype=np.float32)
    N, Hq, D = q.shape
    Hkv = k_cache.shape[2]
    G = Hq // Hkv
    kf = k_cache.reshape(-1, Hkv, D)
    vf = v_cache.reshape(-1, Hkv, D)
    out = np.zeros_like(q)
    for b in range(len(context_lens)):
        r0, r1 = int(cu_seqlens_q[b]), int(cu_seqlens_q[b + 1])
        ql, cl = r1 - r0, int(context_lens[b])
        if ql == 0:
            continue
        slots = slot_of(block_tables[b], np.arange(cl), block_size)
        K = kf[slots]  # [cl, Hkv, D]
        V = vf[slots]
        vis = tree_visible(ql, cl, None if tree_mask is None else tree_mask[r0:r1])
        for h in range(Hq):
            hk = h // G
            s = (q[r0:r1, h, :] @ K[:, hk, :].T) * np.float32(scale)  # [ql, cl]
            s = np.where(vis, s, -np.inf)
            s = s - s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            out[r0:r1, h, :] = p @ V[:, hk, :]
    return out
