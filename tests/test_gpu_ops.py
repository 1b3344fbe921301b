"""torch.ops.nvx.* on the GPU: each op equals the wrapper the engine calls (one launch
path), and torch.library.opcheck accepts the schema and the fake implementation."""
import numpy as np
import pytest
import torch

import nanovllm.ops  # noqa: F401
from nanovllm.layers.attention import tree_attention
from nanovllm.layers.sampler import (rejection_sample_tree, rejection_sample_tree_logits,
                                     rejection_sample_tree_logits_lazy, softmax_stats,
                                     temperature_softmax)
from nanovllm.spec.tree import random_tree
from nanovllm.utils.synthetic import VerifyBatch, randn_bf16

CHECKS = ("test_schema", "test_faketensor")


@pytest.mark.gpu
def test_tree_attention_op(dev):
    rng = np.random.default_rng(31)
    vb = VerifyBatch.random(3, (100, 700), 16, 4, 256, rng)
    g = torch.Generator().manual_seed(31)
    Hq, Hkv, D = 16, 8, 128
    kc = randn_bf16((vb.num_blocks, 256, Hkv, D), g).to(dev)
    vc = randn_bf16((vb.num_blocks, 256, Hkv, D), g).to(dev)
    q = randn_bf16((int(vb.cu_q[-1]), Hq, D), g).to(dev)
    t = lambda a, dt=torch.int32: torch.from_numpy(np.ascontiguousarray(a)).to(dev, dt)  # noqa
    args = (q, kc, vc, t(vb.bt), t(vb.cu_q), t(vb.context_lens), D ** -0.5,
            t(vb.masks, torch.int64), int(vb.qlens.max()), int(vb.context_lens.max()))
    assert torch.equal(torch.ops.nvx.tree_attention(*args), tree_attention(*args))
    torch.library.opcheck(torch.ops.nvx.tree_attention.default, args, test_utils=CHECKS)


@pytest.mark.gpu
def test_sampler_ops(dev):
    g = torch.Generator().manual_seed(32)
    B, T, V = 2, 8, 1000
    logits = (torch.randn(B * T, V, generator=g) * 2).to(torch.bfloat16).to(dev)
    temps = torch.full((B * T,), 0.8, device=dev)
    P = torch.ops.nvx.temperature_softmax(logits, temps)
    assert torch.equal(P, temperature_softmax(logits, temps))
    torch.library.opcheck(torch.ops.nvx.temperature_softmax.default, (logits, temps),
                          test_utils=CHECKS)
    rng = np.random.default_rng(32)
    parents = torch.from_numpy(np.stack([random_tree(T, 3, rng) for _ in range(B)])).to(dev)
    Q = torch.softmax(torch.randn(B, T, V, generator=g), -1).to(dev)
    toks = torch.randint(0, V, (B, T), generator=g, dtype=torch.int32).to(dev)
    U, Uf = torch.rand(B, T, generator=g).to(dev), torch.rand(B, generator=g).to(dev)
    args = (P.view(B, T, V), Q, toks, parents.to(torch.int32), U, Uf)
    got = torch.ops.nvx.rejection_sample_tree(*args)
    want = rejection_sample_tree(*args)
    assert all(torch.equal(a, b) for a, b in zip(got, want))
    torch.library.opcheck(torch.ops.nvx.rejection_sample_tree.default, args, test_utils=CHECKS)
    # the fused form the verify step uses: statistics pass, then the walk on the logits
    V2 = 1024
    lg = (torch.randn(B * T, V2, generator=g) * 2).to(torch.bfloat16).to(dev)
    st = torch.ops.nvx.softmax_stats(lg, temps)
    assert torch.equal(st, softmax_stats(lg, temps))
    torch.library.opcheck(torch.ops.nvx.softmax_stats.default, (lg, temps), test_utils=CHECKS)
    Pf = torch.ops.nvx.softmax_from_stats(lg, temps, st)
    torch.library.opcheck(torch.ops.nvx.softmax_from_stats.default, (lg, temps, st),
                          test_utils=CHECKS)
    Q2 = torch.softmax(torch.randn(B, T, V2, generator=g), -1).to(dev)
    toks2 = torch.randint(0, V2, (B, T), generator=g, dtype=torch.int32).to(dev)
    a2 = (lg, temps, st, Q2, toks2, parents.to(torch.int32), U, Uf)
    got = torch.ops.nvx.rejection_sample_tree_logits(*a2)
    assert all(torch.equal(a, b) for a, b in zip(got, rejection_sample_tree_logits(*a2)))
    want = rejection_sample_tree(Pf.view(B, T, V2), Q2, toks2, parents.to(torch.int32), U, Uf)
    assert all(torch.equal(a, b) for a, b in zip(got, want))
    torch.library.opcheck(torch.ops.nvx.rejection_sample_tree_logits.default, a2,
                          test_utils=CHECKS)
    a3 = (lg, temps, Q2, toks2, parents.to(torch.int32), U, Uf)
    lazy = torch.ops.nvx.rejection_sample_tree_logits_lazy(*a3)
    so = torch.full((B * T, 2), float("nan"), device=dev)
    direct = rejection_sample_tree_logits_lazy(*a3, stats_out=so)
    assert all(torch.equal(a, b) for a, b in zip(lazy[:4], direct[:4]))
    assert torch.equal(torch.isnan(lazy[4]), torch.isnan(so))
    vis = ~torch.isnan(so[:, 0])
    assert torch.equal(lazy[4][vis], so[vis])
    torch.library.opcheck(torch.ops.nvx.rejection_sample_tree_logits_lazy.default, a3,
                          test_utils=CHECKS)


@pytest.mark.gpu
def test_cache_ops_mutate_in_place(dev):
    g = torch.Generator().manual_seed(33)
    N, Hkv, D, nblk = 40, 8, 128, 4
    key, val = randn_bf16((N, Hkv, D), g).to(dev), randn_bf16((N, Hkv, D), g).to(dev)
    kc = torch.zeros(nblk, 256, Hkv, D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    slots = torch.randperm(nblk * 256, generator=g)[:N].to(torch.int32).to(dev)
    torch.ops.nvx.store_kvcache(key, val, kc, vc, slots)
    assert torch.equal(kc.view(-1, Hkv, D)[slots.long()], key)
    assert torch.equal(vc.view(-1, Hkv, D)[slots.long()], val)
    torch.library.opcheck(torch.ops.nvx.store_kvcache.default, (key, val, kc, vc, slots),
                          test_utils=CHECKS)
    # compaction: one sequence, context 100, tree rows at 100.., path 0 -> 3 -> 5
    bt = torch.tensor([[2, 0]], dtype=torch.int32, device=dev)
    ctx = torch.tensor([100], dtype=torch.int32, device=dev)
    path = torch.tensor([[0, 3, 5, -1]], dtype=torch.int32, device=dev)
    acc = torch.tensor([2], dtype=torch.int32, device=dev)
    k5, v5 = kc.clone().unsqueeze(0), vc.clone().unsqueeze(0)
    src = [2 * 256 + 100 + 3, 2 * 256 + 100 + 5]
    want_k = k5.view(-1, Hkv, D)[src].clone()
    torch.ops.nvx.kv_compact(k5, v5, bt, ctx, path, acc)
    assert torch.equal(k5.view(-1, Hkv, D)[[2 * 256 + 101, 2 * 256 + 102]], want_k)
    torch.library.opcheck(torch.ops.nvx.kv_compact.default, (k5, v5, bt, ctx, path, acc),
                          test_utils=CHECKS)


@pytest.mark.gpu
def test_ngram_op(dev):
    hist = np.array([5, 6, 7, 8, 9, 5, 6, 7], dtype=np.int32)
    toks = torch.from_numpy(hist).to(dev)
    offs = torch.tensor([0, len(hist)], dtype=torch.int64, device=dev)
    d, n = torch.ops.nvx.ngram_propose(toks, offs, 3, 1, 5)
    # the last three tokens (5 6 7) first occur at 0: propose what followed, up to 5 tokens
    assert int(n[0]) == 5 and d[0].tolist() == [8, 9, 5, 6, 7]
    torch.library.opcheck(torch.ops.nvx.ngram_propose.default, (toks, offs, 3, 1, 5),
                          test_utils=CHECKS)
