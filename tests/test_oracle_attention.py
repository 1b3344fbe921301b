"""Pins the attention oracle: torch SDPA golden vectors, live SDPA with an
explicit mask, chain == causal, single-query decode, page permutation, GQA."""
import os

import numpy as np
import torch

from nanovllm.spec.tree import chain_parents, random_tree
from nanovllm.utils.synthetic import VerifyBatch
from oracle import attention as oatt

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "attention_sdpa.npz")


def test_golden_sdpa():
    z = np.load(GOLDEN)
    out = oatt.paged_attention(z["q"].astype(np.float32), z["k_cache"].astype(np.float32),
                               z["v_cache"].astype(np.float32), z["block_tables"], z["cu_seqlens_q"],
                               z["context_lens"], z["tree_mask"].view(np.uint64),
                               z["q"].shape[2] ** -0.5, int(z["block_size"]))
    np.testing.assert_allclose(out, z["expected"], atol=2e-5)


def _case(seed, trees, ctx, Hq=8, Hkv=2, D=32, bs=64):
    rng = np.random.default_rng(seed)
    vb = VerifyBatch(ctx, trees, bs, rng)
    kc = rng.normal(size=(vb.num_blocks, bs, Hkv, D)).astype(np.float32)
    vc = rng.normal(size=(vb.num_blocks, bs, Hkv, D)).astype(np.float32)
    q = rng.normal(size=(int(vb.cu_q[-1]), Hq, D)).astype(np.float32)
    return vb, kc, vc, q


def test_live_sdpa_with_explicit_mask():
    rng = np.random.default_rng(0)
    trees = [random_tree(12, 4, rng), random_tree(3, 1, rng)]
    vb, kc, vc, q = _case(1, trees, [100, 7])
    D = q.shape[2]
    out = oatt.paged_attention(q, kc, vc, vb.bt, vb.cu_q, vb.context_lens,
                               vb.masks.view(np.uint64), D ** -0.5, 64)
    for b in range(vb.B):
        r0, r1 = vb.cu_q[b], vb.cu_q[b + 1]
        cl = vb.context_lens[b]
        pos = np.arange(cl)
        slots = vb.bt[b][pos // 64] * 64 + pos % 64
        K = torch.from_numpy(kc.reshape(-1, 2, D)[slots]).permute(1, 0, 2).repeat_interleave(4, 0)
        V = torch.from_numpy(vc.reshape(-1, 2, D)[slots]).permute(1, 0, 2).repeat_interleave(4, 0)
        mask = torch.from_numpy(oatt.tree_visible(r1 - r0, cl, vb.masks[r0:r1].view(np.uint64)))
        ref = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(q[r0:r1]).permute(1, 0, 2), K, V, attn_mask=mask, scale=D ** -0.5)
        np.testing.assert_allclose(out[r0:r1], ref.permute(1, 0, 2).numpy(), atol=1e-5)


def test_chain_mask_equals_causal():
    vb, kc, vc, q = _case(2, [chain_parents(9), chain_parents(30)], [50, 0])
    a = oatt.paged_attention(q, kc, vc, vb.bt, vb.cu_q, vb.context_lens, vb.masks.view(np.uint64),
                             0.2, 64)
    b = oatt.paged_attention(q, kc, vc, vb.bt, vb.cu_q, vb.context_lens, None, 0.2, 64)
    np.testing.assert_array_equal(a, b)


def test_single_query_is_plain_softmax_attention():
    vb, kc, vc, q = _case(3, [chain_parents(1)], [77], Hq=2, Hkv=2)
    out = oatt.paged_attention(q, kc, vc, vb.bt, vb.cu_q, vb.context_lens, None, 0.3, 64)
    pos = np.arange(78)
    slots = vb.bt[0][pos // 64] * 64 + pos % 64
    for h in range(2):
        K = kc.reshape(-1, 2, 32)[slots, h].astype(np.float64)
        V = vc.reshape(-1, 2, 32)[slots, h].astype(np.float64)
        s = K @ q[0, h].astype(np.float64) * 0.3
        w = np.exp(s - s.max())
        w /= w.sum()
        np.testing.assert_allclose(out[0, h], w @ V, atol=1e-5)


def test_page_permutation_invariance():
    rng = np.random.default_rng(4)
    vb, kc, vc, q = _case(4, [random_tree(10, 3, rng)] * 3, [130, 1, 64])
    a = oatt.paged_attention(q, kc, vc, vb.bt, vb.cu_q, vb.context_lens, vb.masks.view(np.uint64),
                             0.2, 64)
    perm = rng.permutation(vb.num_blocks)
    inv = np.argsort(perm)
    bt2 = np.where(vb.bt >= 0, inv[np.maximum(vb.bt, 0)], -1)
    b = oatt.paged_attention(q, kc[perm], vc[perm], bt2, vb.cu_q, vb.context_lens,
                             vb.masks.view(np.uint64), 0.2, 64)
    np.testing.assert_allclose(a, b, atol=1e-6)


def test_gqa_grouping():
    """Query head h reads KV head h // G: zeroing KV head 1's values zeroes
    exactly the outputs of query heads G..2G-1."""
    vb, kc, vc, q = _case(5, [chain_parents(4)], [20], Hq=8, Hkv=2)
    vc2 = vc.copy()
    vc2[:, :, 1] = 0
    out = oatt.paged_attention(q, kc, vc2, vb.bt, vb.cu_q, vb.context_lens, None, 0.2, 64)
    assert np.all(out[:, 4:] == 0) and np.all(np.abs(out[:, :4]).sum(-1) > 0)
