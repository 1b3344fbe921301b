"""store_kvcache and kv_compact (HIP) vs the CPU oracle: bit-exact."""
import numpy as np
import pytest
import torch

from nanovllm.layers.attention import store_kvcache
from nanovllm.spec.kv_compact import kv_compact
from nanovllm.spec.tree import random_tree
from nanovllm.utils.synthetic import paged_block_tables, slots_for
from oracle import kvcache as okv


@pytest.mark.gpu
@pytest.mark.parametrize("Hkv,D,dtype", [(8, 128, torch.bfloat16), (2, 64, torch.float32),
                                          (3, 5, torch.bfloat16)])
def test_store_kvcache(dev, Hkv, D, dtype):
    g = torch.Generator().manual_seed(D)
    rng = np.random.default_rng(D)
    nblk, bs, N = 6, 256, 300
    kc = torch.randn(nblk, bs, Hkv, D, generator=g).to(dtype)
    vc = torch.randn(nblk, bs, Hkv, D, generator=g).to(dtype)
    # key/value as column slices of a fused qkv row (reference qwen3.py:77-81 layout)
    qkv = torch.randn(N, (4 + 2) * Hkv * D, generator=g).to(dtype)
    k = qkv[:, 4 * Hkv * D:5 * Hkv * D].view(N, Hkv, D)
    v = qkv[:, 5 * Hkv * D:].view(N, Hkv, D)
    slots = rng.permutation(nblk * bs)[:N].astype(np.int32)
    slots[::7] = -1
    kd, vd = kc.to(dev), vc.to(dev)
    qkvd = qkv.to(dev)
    store_kvcache(qkvd[:, 4 * Hkv * D:5 * Hkv * D].view(N, Hkv, D),
                  qkvd[:, 5 * Hkv * D:].view(N, Hkv, D), kd, vd, torch.from_numpy(slots).to(dev))
    # the oracle moves raw bytes (uint8 views), so the check is bit-exact for any dtype
    kf, vf = kc.view(torch.uint8).numpy().copy(), vc.view(torch.uint8).numpy().copy()
    okv.store_kvcache(k.contiguous().view(torch.uint8).numpy(), v.contiguous().view(torch.uint8).numpy(),
                      kf, vf, slots)
    assert np.array_equal(kd.cpu().view(torch.uint8).numpy(), kf)
    assert np.array_equal(vd.cpu().view(torch.uint8).numpy(), vf)


@pytest.mark.gpu
def test_store_kvcache_asserts(dev):
    k = torch.zeros(4, 2, 8, dtype=torch.bfloat16, device=dev)
    cache = torch.zeros(2, 16, 2, 8, dtype=torch.bfloat16, device=dev)
    with pytest.raises(AssertionError):
        store_kvcache(k, k, cache, cache, torch.zeros(3, dtype=torch.int32, device=dev))


def compact_case(dev, B, L, T, depth, seed, block_size=256, Hkv=8, D=128):
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    print(f"[compact] B={B} L={L} T={T} depth={depth} Hkv={Hkv} D={D} seed={seed}", flush=True)
    ctx = rng.integers(1, 3000, size=B).astype(np.int32)
    bt, nblk = paged_block_tables(ctx + T, block_size, rng)
    kc = torch.randn(L, nblk, block_size, Hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(L, nblk, block_size, Hkv, D, generator=g).to(torch.bfloat16)
    path = np.full((B, depth + 1), -1, np.int32)
    acc = np.zeros(B, np.int32)
    for b in range(B):
        par = random_tree(T, depth, rng)
        leaf = int(rng.integers(0, T))
        chain = [leaf]
        while par[chain[-1]] >= 0:
            chain.append(int(par[chain[-1]]))
        chain = chain[::-1]
        path[b, :len(chain)] = chain
        acc[b] = len(chain) - 1
    if B > 1:  # overlap case: path[d'] == d for some d' < d
        path[0, :4] = [0, 2, 3, 4]
        acc[0] = 3
    kd, vd = kc.to(dev), vc.to(dev)
    kv_compact(kd, vd, torch.from_numpy(bt).to(dev), torch.from_numpy(ctx).to(dev),
               torch.from_numpy(path).to(dev), torch.from_numpy(acc).to(dev))
    kref, vref = kc.view(torch.uint8).numpy().copy(), vc.view(torch.uint8).numpy().copy()
    okv.kv_compact(kref, vref, bt, ctx, path, acc, block_size)
    assert np.array_equal(kd.cpu().view(torch.uint8).numpy(), kref)
    assert np.array_equal(vd.cpu().view(torch.uint8).numpy(), vref)
    # invariant: rows ctx..ctx+a now hold the accepted nodes' original rows
    for b in range(B):
        src = slots_for(bt[b], ctx[b] + path[b, :acc[b] + 1], block_size)
        dst = slots_for(bt[b], ctx[b] + np.arange(acc[b] + 1), block_size)
        ko = kc.view(L, -1, Hkv, D)[:, src]
        kn = kd.view(L, -1, Hkv, D)[:, dst].cpu()
        assert torch.equal(ko, kn)


@pytest.mark.gpu
def test_kv_compact_small(dev):
    compact_case(dev, B=8, L=3, T=16, depth=5, seed=1)


@pytest.mark.gpu
def test_kv_compact_config4_shape(dev):
    """64 sequences, 36 layers, 64-node depth-8 trees (Qwen3-8B verify step)."""
    compact_case(dev, B=64, L=36, T=64, depth=8, seed=2)


@pytest.mark.gpu
def test_kv_compact_deep_paths(dev):
    """Accepted paths of up to 30 rows: several 8-row gather/scatter groups in sequence."""
    compact_case(dev, B=6, L=2, T=40, depth=30, seed=3)


@pytest.mark.gpu
@pytest.mark.parametrize("Hkv,D", [(2, 64), (16, 256)])
def test_kv_compact_row_widths(dev, Hkv, D):
    """256-byte rows (fewer columns than threads) and 8 KiB rows (each thread moves
    several columns)."""
    compact_case(dev, B=5, L=2, T=24, depth=10, seed=4 + Hkv, Hkv=Hkv, D=D)
