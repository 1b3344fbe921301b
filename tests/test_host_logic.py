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
    """At least 30% of each history's positions are overwritten by copied spans, and
    the copies make prompt lookup find earlier matches: with random ids alone the
    drafter almost never proposes anything."""
    from oracle import ngram as ong
    rng = np.random.default_rng(1)
    hist, fracs = ngram_histories(8, 1024, 4096, 151936, rng, return_covered=True)
    assert all(1024 <= len(h) <= 4096 for h in hist)
    assert min(fracs) >= 0.30 and max(fracs) < 0.30 + 32 / 1024 + 1e-9
    flat, offs = pack_histories(hist)
    assert offs[-1] == len(flat) and flat.dtype == np.int32
    # proposals at many cut points: copied histories match often, fresh ids rarely
    def hit_rate(hs):
        hits = tries = 0
        for h in hs:
            for cut in range(64, len(h), 97):
                _, n = ong.ngram_propose(h[:cut], np.array([0, cut], np.int64), 3, 1, 5)
                hits += int(n[0] > 0)
                tries += 1
        return hits / tries
    fresh = [rng.integers(0, 151936, size=len(h)).astype(np.int32) for h in hist]
    assert hit_rate(hist) > 0.2 > 0.05 > hit_rate(fresh)


def test_walk_rows_counts_the_oracles_passes():
    """bench.walk_rows (the sampler's algorithmic-bytes count) equals the residual
    passes the oracle's walk makes, plus one target row for each walk that ends at a
    leaf (the final draw after a rejection reuses that rejection's residual)."""
    import bench
    from oracle import sampler as osamp
    rng = np.random.default_rng(5)
    B, T, V = 12, 16, 40
    parents = np.stack([random_tree(T, 4, rng) for _ in range(B)])
    P = rng.dirichlet(np.ones(V), size=(B, T)).astype(np.float32)
    Q = rng.dirichlet(np.ones(V), size=(B, T)).astype(np.float32)
    toks = rng.integers(0, V, size=(B, T)).astype(np.int32)
    U = rng.random((B, T)).astype(np.float32)
    Uf = rng.random(B).astype(np.float32)
    counts = {"rej": 0}
    orig = osamp._Residual.reject

    def counting(self, x):
        counts["rej"] += 1
        return orig(self, x)
    osamp._Residual.reject = counting
    try:
        path, acc, _, _ = osamp.rejection_sample_tree(P, Q, toks, parents, U, Uf, np.zeros(B, bool))
    finally:
        osamp._Residual.reject = orig
    path_acc = np.concatenate([acc[:, None], path], axis=1)
    p_rows, q_rows = bench.walk_rows(parents, path_acc)
    leaves = sum(int((parents[b] == path[b, acc[b]]).sum() == 0) for b in range(B))
    assert 0 < leaves < B
    assert q_rows == counts["rej"] and p_rows == counts["rej"] + leaves


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


def test_power_tool_parsing():
    """bench.py --workload power reads the socket power, shader clock and power cap from
    the JSON that amd-smi and rocm-smi print on the MI355X box (samples captured there;
    rocm-smi may put a warning line before its JSON)."""
    import bench
    amd = ('{\n    "gpu_data": [\n        {\n            "gpu": 0,\n            "power": {\n'
           '                "socket_power": {\n                    "value": 1398,\n'
           '                    "unit": "W"\n                },\n'
           '                "gfx_voltage": "N/A"\n            }\n        }\n    ]\n}\n')
    smi = ('WARNING: AMD GPU device(s) is/are in a low-power state. Check power '
           'control/runtime_status\n\n{"card0": {"mclk clock speed:": "(2000Mhz)", '
           '"mclk clock level:": "0", "sclk clock speed:": "(1667Mhz)", "sclk clock level:": "S", '
           '"Max Graphics Package Power (W)": "1400.0"}}\n')
    assert bench.parse_socket_power(amd) == 1398.0
    assert bench.parse_sclk(smi) == 1667.0
    assert bench.parse_power_cap(smi) == 1400.0
    for f in (bench.parse_socket_power, bench.parse_sclk, bench.parse_power_cap):
        assert f("") is None and f("N/A") is None
