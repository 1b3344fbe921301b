"""Pins the KV-cache oracle: the reference's slot loops, -1 skip, compaction
invariant and the overlap case against a sequential ascending copy."""
import numpy as np

from oracle import kvcache as okv


def reference_prefill_slots(block_table, start, end, block_size):
    """The slot loop of nanovllm/engine/model_runner.py:151-161, as written there."""
    out = []
    start_block, end_block = start // block_size, (end + block_size - 1) // block_size
    for i in range(start_block, end_block):
        slot_start = block_table[i] * block_size
        if i == start_block:
            slot_start += start % block_size
        if i != end_block - 1:
            slot_end = block_table[i] * block_size + block_size
        else:
            slot_end = block_table[i] * block_size + end - i * block_size
        out.extend(range(slot_start, slot_end))
    return out


def test_slot_of_matches_reference_loops():
    rng = np.random.default_rng(0)
    for _ in range(200):
        bs = int(rng.choice([64, 256, 512]))
        nblk = int(rng.integers(1, 9))
        bt = rng.permutation(50)[:nblk]
        end = int(rng.integers(1, nblk * bs + 1))
        start = int(rng.integers(0, end))
        assert okv.slot_of(bt, np.arange(start, end), bs).tolist() == \
            reference_prefill_slots(bt, start, end, bs)
        # decode slot (model_runner.py:181): block_table[-1]*bs + last_block_num_tokens - 1
        n = int(rng.integers(1, nblk * bs + 1))
        nb = (n + bs - 1) // bs
        last = n - (nb - 1) * bs
        assert okv.slot_of(bt, n - 1, bs) == bt[nb - 1] * bs + last - 1


def test_store_skips_minus_one():
    k = np.arange(4 * 2 * 3, dtype=np.float32).reshape(4, 2, 3)
    kc = np.zeros((2, 4, 2, 3), np.float32)
    vc = np.zeros_like(kc)
    okv.store_kvcache(k, -k, kc, vc, np.array([5, -1, 0, 7]))
    flat = kc.reshape(-1, 2, 3)
    assert (flat[5] == k[0]).all() and (flat[0] == k[2]).all() and (flat[7] == k[3]).all()
    assert np.count_nonzero(flat.reshape(8, -1).any(1)) == 3


def sequential_compact(caches, bt, ctx, path, acc, bs):
    for b in range(len(ctx)):
        for d in range(1, acc[b] + 1):
            s = okv.slot_of(bt[b], ctx[b] + path[b][d], bs)
            t = okv.slot_of(bt[b], ctx[b] + d, bs)
            for l in range(caches.shape[0]):
                f = caches[l].reshape(-1, *caches.shape[3:])
                f[t] = f[s]


def test_compaction_equals_sequential_and_overlap():
    rng = np.random.default_rng(1)
    L, nblk, bs, H, D = 2, 6, 64, 2, 4
    kc = rng.normal(size=(L, nblk, bs, H, D)).astype(np.float32)
    vc = rng.normal(size=(L, nblk, bs, H, D)).astype(np.float32)
    bt = np.array([[3, 1, 4], [0, 5, 2]], np.int32)
    ctx = np.array([60, 10], np.int32)
    path = np.array([[0, 2, 3, 4, -1], [0, 1, 5, 9, 12]], np.int32)  # seq 0 overlaps
    acc = np.array([3, 4], np.int32)
    k1, v1 = kc.copy(), vc.copy()
    okv.kv_compact(k1, v1, bt, ctx, path, acc, bs)
    k2 = kc.copy()
    sequential_compact(k2, bt, ctx, path, acc, bs)
    np.testing.assert_array_equal(k1, k2)
    for b in range(2):  # invariant: accepted rows are now contiguous from ctx
        src = okv.slot_of(bt[b], ctx[b] + path[b, :acc[b] + 1], bs)
        dst = okv.slot_of(bt[b], ctx[b] + np.arange(acc[b] + 1), bs)
        np.testing.assert_array_equal(k1[:, :, :, :, :].reshape(L, -1, H, D)[:, dst],
                                      kc.reshape(L, -1, H, D)[:, src])
