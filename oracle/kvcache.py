"""Oracle: paged KV-cache slot arithmetic, slot scatter and accepted-path compaction.

Byte/index work, bit-exact.

* Cache layout per layer: [num_blocks, block_size, Hkv, D] (reference
  nanovllm/engine/model_runner.py:115); a token at position ``pos`` of a sequence
  lives in slot ``block_table[pos // block_size] * block_size + pos % block_size``
  (model_runner.py:151-161, :181).  One slot holds a row of Hkv*D elements.
* ``store_kvcache``: ``cache[slot_mapping[i]] = kv[i]``, slot -1 skipped
  (nanovllm/layers/attention.py:21-30).
* ``kv_compact``: after verification the tree rows stored at positions
  ctx..ctx+T-1 are moved so the accepted path becomes contiguous:
  ``row(ctx + d) <- row(ctx + path[d])`` for d = 1..accepted_len, for every layer,
  K and V.  All sources are read before any destination is written (a tree path is
  strictly increasing, so this equals an ascending sequential copy).

Pinned by brute-force index arithmetic in tests/test_oracle_kvcache.py and the
invariant that after compaction rows ctx..ctx+a equal the accepted nodes' rows.
"""
import numpy as np


def slot_of(block_table_row, pos, block_size):
    pos = np.asarray(pos, dtype=np.int64)
    bt = np.asarray(block_table_row, dtype=np.int64)
    return bt[pos // block_size] * block_size + pos % block_size


def store_kvcache(key, value, k_cache, v_cache, slot_mapping):
    """key/value: [N, Hkv, D]; caches: [num_blocks, block_size, Hkv, D] (modified in place)."""
    N = key.shape[0]
    kf = k_cache.reshape(-1, *k_cache.shape[2:])
    vf = v_cache.reshape(-1, *v_cache.shape[2:])
    for i in range(N):
        s = int(slot_mapping[i])
        if s == -1:
            continue
        kf[s] = key[i]
        vf[s] = value[i]


def kv_compact(k_caches, v_caches, block_tables, ctx_lens, path, accepted_len, block_size):
    """k_caches/v_caches: [L, num_blocks, block_size, Hkv, D] (modified in place).

    ctx_lens[b] is the number of cached tokens before the tree; path[b, d] the node
    accepted at depth d (path[b, 0] == 0); accepted_len[b] the number of accepted
    draft nodes."""
    L = k_caches.shape[0]
    for b in range(len(ctx_lens)):
        a = int(accepted_len[b])
        if a <= 0:
            continue
        ctx = int(ctx_lens[b])
        d = np.arange(1, a + 1)
        src = slot_of(block_tables[b], ctx + np.asarray(path[b][1:a + 1], np.int64), block_size)
        dst = slot_of(block_tables[b], ctx + d, block_size)
        for caches in (k_caches, v_caches):
            for l in range(L):
                flat = caches[l].reshape(-1, *caches.shape[3:])
                rows = flat[src].copy()
                flat[dst] = rows
