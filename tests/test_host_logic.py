"""Host-side logic of the verify path: trees, masks, synthetic workloads."""
import numpy as np

from nanovllm.spec.tree import ancestor_masks, chain_parents, depths, random_tree
from nanovllm.utils.synthetic import (VerifyBatch, ngram_histories, pack_histories,
                                      paged_block_tables)


def test_random_tree_properties():
    rng = np.random.default_rng(0)
    for T, d in ((64, 8), (32, 6), (9, 8), (1, 0)):
        p = random_tree(T, d, rng)
        assert p[0] == -1 and all(0 <= p[i] < i for i in range(1, T))
        dep = depths(p)
        assert dep.max() == d
        # BFS order: depths are non-decreasing
        assert np.all(np.diff(dep) >= 0)


def test_ancestor_masks():
    p = np.array([-1, 0, 0, 1, 3, 2])
    m = ancestor_masks(p).view(np.uint64)
    assert [int(x) for x in m] == [0b1, 0b11, 0b101, 0b1011, 0b11011, 0b100101]
    c = ancestor_masks(chain_parents(64)).view(np.uint64)
    assert int(c[63]) == (1 << 64) - 1


def test_ngram_workload_copy_fraction():
    rng = np.random.default_rng(1)
    hist = ngram_histories(8, 1024, 4096, 151936, rng)
    assert all(1024 <= len(h) <= 4096 for h in hist)
    flat, offs = pack_histories(hist)
    assert offs[-1] == len(flat) and flat.dtype == np.int32


def test_verify_batch_layout():
    rng = np.random.default_rng(2)
    trees = [random_tree(8, 3, rng), random_tree(5, 2, rng)]
    vb = VerifyBatch([300, 12], trees, 256, rng)
    assert vb.cu_q.tolist() == [0, 8, 13]
    assert vb.context_lens.tolist() == [308, 17]
    # slots of the tree rows follow the block table
    for b in range(2):
        for i in range(vb.qlens[b]):
            pos = vb.ctx[b] + i
            s = vb.slot_mapping[vb.cu_q[b] + i]
            assert s == vb.bt[b][pos // 256] * 256 + pos % 256
    assert vb.positions[:8].tolist() == (300 + depths(trees[0])).tolist()
    bt, n = paged_block_tables([10, 600], 256, rng)
    assert n == 4 and sorted(bt[bt >= 0].tolist()) == [0, 1, 2, 3]
