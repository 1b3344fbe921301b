"""Tree attention (HIP) vs the CPU oracle: within 2e-2 absolute in bf16."""
import numpy as np
import pytest
import torch

from nanovllm.layers.attention import tree_attention, Attention
from nanovllm.spec.tree import chain_parents, random_tree
from nanovllm.utils.context import set_context, reset_context
from nanovllm.utils.synthetic import VerifyBatch, randn_bf16
from oracle import attention as oatt

TOL = 2e-2


def run_case(dev, Hq, Hkv, ctx, trees, seed, block_size=256, causal=False):
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    vb = VerifyBatch(ctx, trees, block_size, rng)
    D = 128
    kc = randn_bf16((vb.num_blocks, block_size, Hkv, D), g)
    vc = randn_bf16((vb.num_blocks, block_size, Hkv, D), g)
    N = int(vb.cu_q[-1])
    q = randn_bf16((N, Hq, D), g)
    mask = None if causal else torch.from_numpy(vb.masks)
    print(f"[attn] Hq={Hq} Hkv={Hkv} B={vb.B} N={N} maxctx={int(vb.context_lens.max())} "
          f"causal={causal} seed={seed}", flush=True)
    o = tree_attention(q.to(dev), kc.to(dev), vc.to(dev), torch.from_numpy(vb.bt).to(dev),
                       torch.from_numpy(vb.cu_q).to(dev), torch.from_numpy(vb.context_lens).to(dev),
                       D ** -0.5, None if mask is None else mask.to(dev))
    ref = oatt.paged_attention(q.float().numpy(), kc.float().numpy(), vc.float().numpy(), vb.bt,
                               vb.cu_q, vb.context_lens,
                               None if causal else vb.masks.view(np.uint64), D ** -0.5, block_size)
    err = np.abs(o.cpu().float().numpy() - ref)
    assert np.isfinite(o.cpu().float().numpy()).all()
    assert err.max() < TOL, f"max abs err {err.max()}"
    return err.max()


@pytest.mark.gpu
@pytest.mark.parametrize("Hq,Hkv", [(16, 8), (32, 8), (8, 8), (4, 1)])
def test_small_trees(dev, Hq, Hkv):
    rng = np.random.default_rng(1)
    trees = [random_tree(t, d, rng) for t, d in ((8, 3), (32, 6), (1, 0), (17, 4))]
    run_case(dev, Hq, Hkv, [300, 64, 5, 1000], trees, seed=Hq * 10 + Hkv)


@pytest.mark.gpu
def test_chain_equals_causal(dev):
    rng = np.random.default_rng(2)
    ctx = [700, 129]
    trees = [chain_parents(6), chain_parents(20)]
    run_case(dev, 16, 8, ctx, trees, seed=3)
    run_case(dev, 16, 8, ctx, trees, seed=3, causal=True)


@pytest.mark.gpu
def test_decode_single_query(dev):
    rng = np.random.default_rng(4)
    ctx = list(rng.integers(1, 3000, size=37))
    run_case(dev, 32, 8, ctx, [chain_parents(1)] * 37, seed=5)


@pytest.mark.gpu
def test_tree64_block512(dev):
    rng = np.random.default_rng(6)
    trees = [random_tree(64, 8, rng) for _ in range(3)]
    run_case(dev, 32, 8, [2048, 100, 513], trees, seed=7, block_size=512)


@pytest.mark.gpu
@pytest.mark.parametrize("block_size", [64, 128, 192])
def test_small_pages(dev, block_size):
    """Pages of one, two and three 64-key chunks: the per-chunk page lookup and each
    KV split's window of pages at page sizes other than 256 (few sequences, so every
    item is split many ways; the 64-node tree takes the 8-wave workgroup)."""
    rng = np.random.default_rng(block_size)
    trees = [random_tree(64, 8, rng), chain_parents(1), random_tree(20, 5, rng)]
    run_case(dev, 32, 8, [1500, 4000, 77], trees, seed=block_size, block_size=block_size)


@pytest.mark.gpu
def test_long_context_full_batch(dev):
    """64 decode rows (a batch that alone fills the GPU, so the plan starts from one KV
    split) over 33-40K-token contexts in 64-token pages: more pages than one
    workgroup's page table holds, so the plan adds splits instead of refusing the
    launch.  Caches are drawn on the GPU; two sequences are checked against the oracle."""
    B, Hq, Hkv, D, bs = 64, 32, 8, 128, 64
    rng = np.random.default_rng(40)
    ctx = [int(c) for c in rng.integers(33000, 40000, size=B)]
    vb = VerifyBatch(ctx, [chain_parents(1)] * B, bs, rng)
    print(f"[attn] long contexts B={B} bs={bs} maxctx={int(vb.context_lens.max())}", flush=True)
    g = torch.Generator(device=dev).manual_seed(41)
    shape = (vb.num_blocks, bs, Hkv, D)
    kc = torch.randn(shape, generator=g, device=dev, dtype=torch.bfloat16)
    vc = torch.randn(shape, generator=g, device=dev, dtype=torch.bfloat16)
    q = torch.randn(B, Hq, D, generator=g, device=dev, dtype=torch.bfloat16)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    o = tree_attention(q, kc, vc, t(vb.bt), t(vb.cu_q), t(vb.context_lens), D ** -0.5, None)
    for b in (0, 37):
        L = int(vb.context_lens[b])
        npg = (L + bs - 1) // bs
        pages = torch.from_numpy(vb.bt[b, :npg].astype(np.int64)).to(dev)
        ref = oatt.paged_attention(q[b:b + 1].float().cpu().numpy(), kc[pages].float().cpu().numpy(),
                                   vc[pages].float().cpu().numpy(),
                                   np.arange(npg, dtype=np.int32)[None], np.array([0, 1], np.int32),
                                   np.array([L], np.int32), None, D ** -0.5, bs)
        assert np.abs(o[b:b + 1].float().cpu().numpy() - ref).max() < TOL


@pytest.mark.gpu
def test_causal_prefill_long_queries(dev):
    # prompt-style: q_len up to 300 with a cached prefix (multiple q-row chunks)
    run_case(dev, 16, 8, [0, 256, 40], [chain_parents(300), chain_parents(77),
                                         chain_parents(200)], seed=8, causal=True)


@pytest.mark.gpu
def test_causal_wave_plans_agree(dev):
    """Causal launches with at most 64 q rows per sequence and more than 128 rows per KV
    head run 8-wave workgroups; longer q (prefill) runs 4-wave workgroups, two per CU.
    The same prompt with q = 64 and q = 65 at 32/8 heads behind a cached prefix takes each
    path: both match the oracle, and the 64 shared tokens' outputs agree bit for bit
    (rows keep their 32-row waves and see the same chunks in the same order)."""
    Hq, Hkv, D, bs = 32, 8, 128, 256
    rng = np.random.default_rng(21)
    g = torch.Generator().manual_seed(21)
    vb = VerifyBatch([300, 190], [chain_parents(65), chain_parents(65)], bs, rng)
    kc = randn_bf16((vb.num_blocks, bs, Hkv, D), g)
    vc = randn_bf16((vb.num_blocks, bs, Hkv, D), g)
    q = randn_bf16((int(vb.cu_q[-1]), Hq, D), g)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    outs = {}
    for T in (65, 64):
        # the first T tokens of each sequence: the same cache, context shortened by 65 - T
        cu = np.array([0, T, 2 * T], dtype=np.int32)
        cl = (vb.context_lens - (65 - T)).astype(np.int32)
        qq = torch.cat([q[int(vb.cu_q[b]):int(vb.cu_q[b]) + T] for b in range(2)])
        o = tree_attention(qq.to(dev), kc.to(dev), vc.to(dev), t(vb.bt), t(cu), t(cl), D ** -0.5,
                           None)
        ref = oatt.paged_attention(qq.float().numpy(), kc.float().numpy(), vc.float().numpy(),
                                   vb.bt, cu, cl, None, D ** -0.5, bs)
        assert np.abs(o.cpu().float().numpy() - ref).max() < TOL, T
        outs[T] = o.cpu()
    shared = torch.cat([outs[65][0:64], outs[65][65:129]])
    assert torch.equal(shared, outs[64])


@pytest.mark.gpu
def test_config3_tree32_qwen3_0p6b(dev):
    """Qwen3-0.6B shape: 16 q heads, 8 KV heads, B=32, ctx U[1024,4096], 32-node
    depth-6 trees, pages scattered randomly (the split-KV path)."""
    rng = np.random.default_rng(0)
    ctx = rng.integers(1024, 4097, size=32)
    trees = [random_tree(32, 6, rng) for _ in range(32)]
    run_case(dev, 16, 8, ctx, trees, seed=0)


@pytest.mark.gpu
def test_config4_tree64_qwen3_8b_layer(dev):
    """Qwen3-8B shape, one layer: 32 q heads, 8 KV heads, B=64, ctx 2048, 64-node
    depth-8 trees (the single-split path)."""
    rng = np.random.default_rng(1)
    trees = [random_tree(64, 8, rng) for _ in range(64)]
    run_case(dev, 32, 8, [2048] * 64, trees, seed=1)


@pytest.mark.gpu
def test_config4_heads_short_context_mask(dev):
    """Qwen3-8B heads (32/8), 64-node depth-8 trees after only 0-64 cached tokens: the
    tree keys carry most of the softmax mass, so a wrong mask bit moves outputs by far
    more than the tolerance (at ctx 2048 the same error would be diluted to ~1e-3).
    32 sequences, so the 256-row items take the 8-wave workgroup as at config 4."""
    rng = np.random.default_rng(21)
    ctx = [int(c) for c in rng.integers(0, 65, size=32)]
    ctx[:3] = [0, 1, 64]
    trees = [random_tree(64, 8, rng) for _ in range(32)]
    run_case(dev, 32, 8, ctx, trees, seed=21)


@pytest.mark.gpu
def test_page_permutation_invariance(dev):
    rng = np.random.default_rng(9)
    g = torch.Generator().manual_seed(9)
    trees = [random_tree(16, 4, rng) for _ in range(4)]
    vb = VerifyBatch([500, 900, 33, 1500], trees, 256, rng)
    kc = randn_bf16((vb.num_blocks, 256, 8, 128), g)
    vc = randn_bf16((vb.num_blocks, 256, 8, 128), g)
    q = randn_bf16((int(vb.cu_q[-1]), 16, 128), g).to(dev)
    args = (torch.from_numpy(vb.cu_q).to(dev), torch.from_numpy(vb.context_lens).to(dev), 128 ** -0.5,
            torch.from_numpy(vb.masks).to(dev))
    o1 = tree_attention(q, kc.to(dev), vc.to(dev), torch.from_numpy(vb.bt).to(dev), *args)
    perm = rng.permutation(vb.num_blocks)
    inv = np.argsort(perm)
    kc2, vc2 = kc[torch.from_numpy(perm)], vc[torch.from_numpy(perm)]
    bt2 = np.where(vb.bt >= 0, inv[np.maximum(vb.bt, 0)], -1).astype(np.int32)
    o2 = tree_attention(q, kc2.to(dev), vc2.to(dev), torch.from_numpy(bt2).to(dev), *args)
    assert torch.equal(o1, o2)


@pytest.mark.gpu
def test_attention_module_store_then_attend(dev):
    """Attention.forward: store the tree rows, then attend (reference order,
    attention.py:62-74), driven through the Context side channel."""
    rng = np.random.default_rng(10)
    g = torch.Generator().manual_seed(10)
    trees = [random_tree(12, 4, rng) for _ in range(3)]
    vb = VerifyBatch([260, 31, 800], trees, 256, rng)
    Hq, Hkv, D = 16, 8, 128
    N = int(vb.cu_q[-1])
    kc = randn_bf16((vb.num_blocks, 256, Hkv, D), g)
    vc = randn_bf16((vb.num_blocks, 256, Hkv, D), g)
    q, k, v = randn_bf16((N, Hq, D), g), randn_bf16((N, Hkv, D), g), randn_bf16((N, Hkv, D), g)
    attn = Attention(Hq, D, D ** -0.5, Hkv)
    attn.k_cache, attn.v_cache = kc.to(dev), vc.to(dev)
    set_context(False, cu_seqlens_q=torch.from_numpy(vb.cu_q).to(dev),
                slot_mapping=torch.from_numpy(vb.slot_mapping).to(dev),
                context_lens=torch.from_numpy(vb.context_lens).to(dev),
                block_tables=torch.from_numpy(vb.bt).to(dev),
                tree_mask=torch.from_numpy(vb.masks).to(dev), max_seqlen_q=vb.T,
                max_context_len=int(vb.context_lens.max()))
    try:
        o = attn(q.to(dev), k.to(dev), v.to(dev))
    finally:
        reset_context()
    kf, vf = kc.float().numpy(), vc.float().numpy()
    kff, vff = kf.reshape(-1, Hkv, D), vf.reshape(-1, Hkv, D)
    kff[vb.slot_mapping] = k.float().numpy()
    vff[vb.slot_mapping] = v.float().numpy()
    ref = oatt.paged_attention(q.float().numpy(), kf, vf, vb.bt, vb.cu_q, vb.context_lens,
                               vb.masks.view(np.uint64), D ** -0.5, 256)
    assert np.abs(o.cpu().float().numpy() - ref).max() < TOL


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(8))
def test_random_shapes(dev, case):
    """Seeded sweep: GQA group sizes 1-16 (including 5, as 40 q / 8 KV heads), batches
    of 1-6, cached contexts of 0-12k tokens (tree keys only, partial last chunks, many
    KV splits), trees of 1-64 nodes; a few cases causal instead of tree-masked."""
    rng = np.random.default_rng(1000 + case)
    Hq, Hkv = [(40, 8), (64, 4), (8, 8), (32, 8), (20, 4), (16, 8), (48, 8), (16, 1)][case]
    B = int(rng.integers(1, 7))
    ctx = [int(rng.choice([0, rng.integers(1, 70), rng.integers(70, 3000), rng.integers(3000, 12000)]))
           for _ in range(B)]
    trees = [random_tree(int(t), int(min(t - 1, rng.integers(1, 10))), rng)
             for t in rng.integers(1, 65, size=B)]
    causal = case % 4 == 3
    if causal:
        trees = [chain_parents(len(t)) for t in trees]
    run_case(dev, Hq, Hkv, ctx, trees, seed=2000 + case, causal=causal)
