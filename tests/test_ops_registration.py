"""torch.ops.nvx registrations: schemas and fake implementations (runs without a GPU:
FakeTensorMode traces the ops with device tensors that have no storage)."""
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import nanovllm.ops  # noqa: F401  (registers torch.ops.nvx.*)


def test_schemas_declare_the_mutated_caches():
    schemas = {n: str(getattr(torch.ops.nvx, n).default._schema)
               for n in ("store_kvcache", "kv_compact", "tree_attention", "temperature_softmax",
                         "topk_logprobs", "rejection_sample_tree", "ngram_propose",
                         "softmax_stats", "softmax_from_stats", "rejection_sample_tree_logits",
                         "rejection_sample_tree_logits_lazy")}
    import re
    for n in ("store_kvcache", "kv_compact"):
        assert re.search(r"Tensor\(\w+!\) k_cache", schemas[n]), schemas[n]
        assert re.search(r"Tensor\(\w+!\) v_cache", schemas[n]), schemas[n]
        assert schemas[n].count("!") == 2, schemas[n]
    for n in ("tree_attention", "temperature_softmax", "topk_logprobs", "rejection_sample_tree",
              "ngram_propose", "softmax_stats", "softmax_from_stats", "rejection_sample_tree_logits",
              "rejection_sample_tree_logits_lazy"):
        assert "!" not in schemas[n], schemas[n]
    assert "Tensor? tree_mask=None" in schemas["tree_attention"]
    assert "-> (Tensor, Tensor, Tensor, Tensor)" in schemas["rejection_sample_tree"]


def test_fake_shapes_at_the_verify_step():
    """Config-4 shapes (64 sequences x 64-node trees, 32/8 heads, 151,936-token vocab)."""
    with FakeTensorMode():
        dev = "cuda"
        B, T, Hq, Hkv, D, V = 64, 64, 32, 8, 128, 151936
        q = torch.empty(B * T, Hq, D, dtype=torch.bfloat16, device=dev)
        kc = torch.empty(600, 256, Hkv, D, dtype=torch.bfloat16, device=dev)
        i32 = lambda *s: torch.empty(*s, dtype=torch.int32, device=dev)  # noqa: E731
        o = torch.ops.nvx.tree_attention(q, kc, kc, i32(B, 9), i32(B + 1), i32(B), D ** -0.5,
                                         torch.empty(B * T, dtype=torch.int64, device=dev), T,
                                         2048 + T)
        assert o.shape == q.shape and o.dtype == torch.bfloat16 and o.device.type == "cuda"
        logits = torch.empty(B * T, V, dtype=torch.bfloat16, device=dev)
        P = torch.ops.nvx.temperature_softmax(logits, torch.empty(B * T, device=dev))
        assert P.shape == (B * T, V) and P.dtype == torch.float32
        path, acc, toks, nxt = torch.ops.nvx.rejection_sample_tree(
            P.view(B, T, V), P.view(B, T, V), i32(B, T), i32(B, T),
            torch.empty(B, T, device=dev), torch.empty(B, device=dev))
        assert (path.shape, acc.shape, toks.shape, nxt.shape) == ((B, T), (B,), (B, T), (B,))
        assert all(t.dtype == torch.int32 for t in (path, acc, toks, nxt))
        temps = torch.empty(B * T, device=dev)
        stats = torch.ops.nvx.softmax_stats(logits, temps)
        assert stats.shape == (B * T, 2) and stats.dtype == torch.float32
        assert torch.ops.nvx.softmax_from_stats(logits, temps, stats).shape == (B * T, V)
        outs = torch.ops.nvx.rejection_sample_tree_logits(
            logits, temps, stats, P.view(B, T, V), i32(B, T), i32(B, T),
            torch.empty(B, T, device=dev), torch.empty(B, device=dev))
        assert [o_.shape for o_ in outs] == [(B, T), (B,), (B, T), (B,)]
        outs = torch.ops.nvx.rejection_sample_tree_logits_lazy(
            logits, temps, P.view(B, T, V), i32(B, T), i32(B, T),
            torch.empty(B, T, device=dev), torch.empty(B, device=dev))
        assert [o_.shape for o_ in outs] == [(B, T), (B,), (B, T), (B,), (B * T, 2)]
        assert outs[4].dtype == torch.float32
        lp, tok = torch.ops.nvx.topk_logprobs(logits[:2048], 8)
        assert lp.shape == tok.shape == (2048, 8) and tok.dtype == torch.int64
        d, n = torch.ops.nvx.ngram_propose(i32(4000), torch.empty(B + 1, dtype=torch.int64,
                                                                    device=dev), 3, 1, 5)
        assert d.shape == (B, 5) and n.shape == (B,) and d.dtype == n.dtype == torch.int32
        caches = torch.empty(36, 600, 256, Hkv, D, dtype=torch.bfloat16, device=dev)
        assert torch.ops.nvx.kv_compact(caches, caches.clone(), i32(B, 9), i32(B), i32(B, 9),
                                        i32(B)) is None
        assert torch.ops.nvx.store_kvcache(q[:, :Hkv], q[:, :Hkv], kc, kc.clone(),
                                           i32(B * T)) is None
