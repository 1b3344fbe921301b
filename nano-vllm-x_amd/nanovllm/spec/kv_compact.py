"""Compaction of the accepted draft path's KV rows on libnvx_spec.

After verification the tree rows sit at positions ctx..ctx+T-1; the accepted path
[0, n1, n2, ...] must end at ctx, ctx+1, ctx+2, ...  This moves row(ctx + path[d])
to row(ctx + d) for d = 1..accepted_len, for every layer, K and V, with the
reference's slot formula (nanovllm/engine/model_runner.py:151-161, :181) and cache
layout (:115).  It generalises store_kvcache (nanovllm/layers/attention.py:21-30)
to a cache-resident source; the reference has no compaction.
"""
import torch

from .. import _C


def kv_compact(k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor,
               ctx_lens: torch.Tensor, path: torch.Tensor, accepted_len: torch.Tensor):
    """k_cache / v_cache: [L, num_blocks, block_size, Hkv, D] (a layer-stacked view such
    as ModelRunner.kv_cache[0] / [1]) or [num_blocks, block_size, Hkv, D] for one layer.
    block_tables int32 [B, max_blocks]; ctx_lens int32 [B] (cached tokens before the
    tree); path int32 [B, P] (path[:, 0] == 0); accepted_len int32 [B]."""
    if k_cache.dim() == 4:
        k_cache, v_cache = k_cache.unsqueeze(0), v_cache.unsqueeze(0)
    if k_cache.shape != v_cache.shape or k_cache.dim() != 5:
        raise ValueError("kv_compact: caches must be [L, num_blocks, block_size, Hkv, D]")
    L, nblk, bs, Hkv, D = k_cache.shape
    es = k_cache.element_size()
    if k_cache.stride(4) != 1 or k_cache.stride(3) != D or k_cache.stride(2) != Hkv * D \
            or k_cache.stride(1) != bs * Hkv * D or v_cache.stride() != k_cache.stride():
        raise ValueError("kv_compact: each layer of the caches must be contiguous")
    for name, t in (("block_tables", block_tables), ("ctx_lens", ctx_lens), ("path", path),
                    ("accepted_len", accepted_len)):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"kv_compact: {name} must be contiguous int32")
    _C.require_cuda(k_cache, v_cache, block_tables, ctx_lens, path, accepted_len)
    B = ctx_lens.numel()
    _C.check(_C.lib().nvx_kv_compact(
        _C.ptr(k_cache), _C.ptr(v_cache), k_cache.stride(0) * es, L, Hkv * D * es, bs,
        _C.ptr(block_tables), block_tables.shape[1], _C.ptr(ctx_lens), _C.ptr(path),
        path.shape[1], _C.ptr(accepted_len), B, _C.stream_of(k_cache)))
