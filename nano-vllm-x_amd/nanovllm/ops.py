"""torch custom ops (namespace ``nvx``) over the verify path's kernels.

The engine calls the Python wrappers directly, so its hot path does not go through the
dispatcher. These registrations give the same kernels a torch schema and fake (meta)
implementations: ``torch.ops.nvx.*`` can be traced with FakeTensor or ``torch.compile``
and checked with ``torch.library.opcheck``. Each op launches through the wrapper the
engine uses (one launch path, the same validation), on the current stream.

Importing this module registers the ops; ``nanovllm`` itself does not import it.
"""
from typing import Optional

import torch
from torch import Tensor

from .layers import attention as _attention
from .layers import sampler as _sampler
from .spec import kv_compact as _kv_compact
from .spec import ngram as _ngram


@torch.library.custom_op("nvx::store_kvcache", mutates_args=("k_cache", "v_cache"))
def store_kvcache(key: Tensor, value: Tensor, k_cache: Tensor, v_cache: Tensor,
                  slot_mapping: Tensor) -> None:
    """Scatter the step's K/V rows into the paged caches (reference attention.py:33-40)."""
    _attention.store_kvcache(key, value, k_cache, v_cache, slot_mapping)


@store_kvcache.register_fake
def _store_kvcache_fake(key, value, k_cache, v_cache, slot_mapping):
    return None


@torch.library.custom_op("nvx::tree_attention", mutates_args=())
def tree_attention(q: Tensor, k_cache: Tensor, v_cache: Tensor, block_tables: Tensor,
                   cu_seqlens_q: Tensor, context_lens: Tensor, scale: float,
                   tree_mask: Optional[Tensor] = None, max_seqlen_q: Optional[int] = None,
                   max_context_len: Optional[int] = None) -> Tensor:
    """Paged tree-masked attention (causal when tree_mask is None): bf16 [N, Hq, 128]."""
    return _attention.tree_attention(q, k_cache, v_cache, block_tables, cu_seqlens_q,
                                     context_lens, scale, tree_mask, max_seqlen_q,
                                     max_context_len)


@tree_attention.register_fake
def _tree_attention_fake(q, k_cache, v_cache, block_tables, cu_seqlens_q, context_lens, scale,
                         tree_mask=None, max_seqlen_q=None, max_context_len=None):
    return torch.empty_like(q)


@torch.library.custom_op("nvx::temperature_softmax", mutates_args=())
def temperature_softmax(logits: Tensor, temperatures: Tensor) -> Tensor:
    """fp32 softmax(logits / T) per row; rows with T = 0 keep their fp32 logits."""
    return _sampler.temperature_softmax(logits, temperatures)


@temperature_softmax.register_fake
def _temperature_softmax_fake(logits, temperatures):
    return logits.new_empty(logits.shape, dtype=torch.float32)


@torch.library.custom_op("nvx::topk_logprobs", mutates_args=())
def topk_logprobs(logits: Tensor, k: int) -> tuple[Tensor, Tensor]:
    """Top-k of log_softmax(logits) per row: (log-probs fp32 [N, k], tokens int64 [N, k])."""
    return _sampler.topk_logprobs(logits, k)


@topk_logprobs.register_fake
def _topk_logprobs_fake(logits, k):
    n = logits.shape[0]
    return (logits.new_empty((n, k), dtype=torch.float32),
            logits.new_empty((n, k), dtype=torch.int64))


@torch.library.custom_op("nvx::rejection_sample_tree", mutates_args=())
def rejection_sample_tree(target_probs: Tensor, draft_probs: Optional[Tensor], tokens: Tensor,
                          parents: Tensor, uniforms: Tensor, final_uniforms: Tensor,
                          greedy: Optional[Tensor] = None, num_nodes: Optional[Tensor] = None,
                          draft_mode: str = "stochastic"
                          ) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Tree (or chain) rejection sampling: int32 (path [B, T], accepted_len [B],
    out_tokens [B, T], next_token [B])."""
    return _sampler.rejection_sample_tree(target_probs, draft_probs, tokens, parents, uniforms,
                                          final_uniforms, greedy, num_nodes, draft_mode)


@rejection_sample_tree.register_fake
def _rejection_sample_tree_fake(target_probs, draft_probs, tokens, parents, uniforms,
                                final_uniforms, greedy=None, num_nodes=None,
                                draft_mode="stochastic"):
    B, T = target_probs.shape[0], target_probs.shape[1]
    i32 = dict(dtype=torch.int32)
    return (target_probs.new_empty((B, T), **i32), target_probs.new_empty((B,), **i32),
            target_probs.new_empty((B, T), **i32), target_probs.new_empty((B,), **i32))


@torch.library.custom_op("nvx::softmax_stats", mutates_args=())
def softmax_stats(logits: Tensor, temperatures: Tensor) -> Tensor:
    """Per-row (max * log2(e) / T, 1 / sum) of the temperature softmax: fp32 [N, 2]."""
    return _sampler.softmax_stats(logits, temperatures)


@softmax_stats.register_fake
def _softmax_stats_fake(logits, temperatures):
    return logits.new_empty((logits.shape[0], 2), dtype=torch.float32)


@torch.library.custom_op("nvx::softmax_from_stats", mutates_args=())
def softmax_from_stats(logits: Tensor, temperatures: Tensor, stats: Tensor) -> Tensor:
    """fp32 probabilities from the logits and their softmax_stats (the fused walk's values)."""
    return _sampler.softmax_from_stats(logits, temperatures, stats)


@softmax_from_stats.register_fake
def _softmax_from_stats_fake(logits, temperatures, stats):
    return logits.new_empty(logits.shape, dtype=torch.float32)


@torch.library.custom_op("nvx::rejection_sample_tree_logits", mutates_args=())
def rejection_sample_tree_logits(logits: Tensor, temperatures: Tensor, stats: Tensor,
                                 draft_probs: Optional[Tensor], tokens: Tensor, parents: Tensor,
                                 uniforms: Tensor, final_uniforms: Tensor,
                                 greedy: Optional[Tensor] = None, num_nodes: Optional[Tensor] = None,
                                 draft_mode: str = "stochastic"
                                 ) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """The tree walk on logits [B*T, V] + softmax_stats (the verify step's fused sampler):
    int32 (path [B, T], accepted_len [B], out_tokens [B, T], next_token [B])."""
    return _sampler.rejection_sample_tree_logits(logits, temperatures, stats, draft_probs, tokens,
                                                 parents, uniforms, final_uniforms, greedy,
                                                 num_nodes, draft_mode)


@rejection_sample_tree_logits.register_fake
def _rejection_sample_tree_logits_fake(logits, temperatures, stats, draft_probs, tokens, parents,
                                       uniforms, final_uniforms, greedy=None, num_nodes=None,
                                       draft_mode="stochastic"):
    B, T = tokens.shape
    i32 = dict(dtype=torch.int32)
    return (tokens.new_empty((B, T), **i32), tokens.new_empty((B,), **i32),
            tokens.new_empty((B, T), **i32), tokens.new_empty((B,), **i32))


@torch.library.custom_op("nvx::rejection_sample_tree_logits_lazy", mutates_args=())
def rejection_sample_tree_logits_lazy(logits: Tensor, temperatures: Tensor,
                                      draft_probs: Optional[Tensor], tokens: Tensor,
                                      parents: Tensor, uniforms: Tensor, final_uniforms: Tensor,
                                      greedy: Optional[Tensor] = None,
                                      num_nodes: Optional[Tensor] = None,
                                      draft_mode: str = "stochastic"
                                      ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """The tree walk on logits [B*T, V] computing the softmax statistics of the rows it
    visits (the verify step's sampler): int32 (path [B, T], accepted_len [B],
    out_tokens [B, T], next_token [B]) and fp32 stats [B*T, 2] (NaN on rows not
    visited)."""
    B, T = tokens.shape
    stats = torch.full((B * T, 2), float("nan"), dtype=torch.float32, device=logits.device)
    return _sampler.rejection_sample_tree_logits_lazy(logits, temperatures, draft_probs, tokens,
                                                      parents, uniforms, final_uniforms, greedy,
                                                      num_nodes, draft_mode, stats_out=stats)


@rejection_sample_tree_logits_lazy.register_fake
def _rejection_sample_tree_logits_lazy_fake(logits, temperatures, draft_probs, tokens, parents,
                                            uniforms, final_uniforms, greedy=None, num_nodes=None,
                                            draft_mode="stochastic"):
    B, T = tokens.shape
    i32 = dict(dtype=torch.int32)
    return (tokens.new_empty((B, T), **i32), tokens.new_empty((B,), **i32),
            tokens.new_empty((B, T), **i32), tokens.new_empty((B,), **i32),
            logits.new_empty((B * T, 2), dtype=torch.float32))


@torch.library.custom_op("nvx::kv_compact", mutates_args=("k_cache", "v_cache"))
def kv_compact(k_cache: Tensor, v_cache: Tensor, block_tables: Tensor, ctx_lens: Tensor,
               path: Tensor, accepted_len: Tensor) -> None:
    """Move the accepted path's KV rows to positions ctx..ctx+accepted_len, every layer."""
    _kv_compact.kv_compact(k_cache, v_cache, block_tables, ctx_lens, path, accepted_len)


@kv_compact.register_fake
def _kv_compact_fake(k_cache, v_cache, block_tables, ctx_lens, path, accepted_len):
    return None


@torch.library.custom_op("nvx::ngram_propose", mutates_args=())
def ngram_propose(tokens: Tensor, offsets: Tensor, max_ngram: int = 3, min_ngram: int = 1,
                  num_draft: int = 5) -> tuple[Tensor, Tensor]:
    """Prompt-lookup drafts: (draft int32 [B, num_draft] padded with -1, draft_len int32 [B])."""
    return _ngram.ngram_propose(tokens, offsets, max_ngram, min_ngram, num_draft)


@ngram_propose.register_fake
def _ngram_propose_fake(tokens, offsets, max_ngram=3, min_ngram=1, num_draft=5):
    B = offsets.shape[0] - 1
    return (offsets.new_empty((B, num_draft), dtype=torch.int32),
            offsets.new_empty((B,), dtype=torch.int32))
