"""The C ABI: the library loads, exports every function include/nvx_spec.h
declares, the ctypes binding covers them, and argument validation fails loudly
(no kernel is launched by these calls, so they run without a GPU)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nvx_spec.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:[\w\*\s]+?)\b(nvx_\w+)\s*\(", text, re.M)))


def test_header_declarations_are_bound():
    from nanovllm import _C
    names = declared()
    assert len(names) >= 10
    assert sorted(_C.EXPORTED) == names


def test_library_exports_every_symbol():
    from nanovllm import _C
    lib = _C.lib()
    for name in declared():
        assert hasattr(lib, name), name
    assert lib.nvx_version() >= 100


def test_validation_errors_are_reported():
    from nanovllm import _C
    lib = _C.lib()
    rc = lib.nvx_ngram_propose(None, None, 1, 1, 9, 5, None, None, None)
    assert rc == -1 and b"max_ngram" in lib.nvx_last_error()
    rc = lib.nvx_tree_attention(None, None, None, None, None, 1, None, None, None, 1, 1, 1, 1,
                                8, 8, 64, 256, 1.0, None, 0, None)
    assert rc == -1 and b"head_dim" in lib.nvx_last_error()
    rc = lib.nvx_rejection_sample_tree(None, 0, None, 0, 10, None, None, None, 65, None, None, None,
                                       0, 1, None, None, None, None, None, 0, None)
    assert rc == -1 and b"node_stride" in lib.nvx_last_error()
    # the walk's exchange workspace: 1280 bytes per sequence
    assert lib.nvx_rejection_walk_workspace_size(0) == 0
    assert lib.nvx_rejection_walk_workspace_size(1) == 1280
    assert lib.nvx_rejection_walk_workspace_size(64) == 64 * 1280
    h = ctypes.c_void_p(0x100000)  # non-null host addresses: refused before any launch
    rc = lib.nvx_rejection_sample_tree(h, 10, None, 0, 10, h, h, None, 1, h, h, None, 1, 2, h, h, h,
                                       h, h, 2000, None)
    assert rc == -1 and b"exchange workspace of 2560 bytes" in lib.nvx_last_error()
    with pytest.raises(RuntimeError, match="kv_compact"):
        _C.check(lib.nvx_kv_compact(None, None, 0, 1, 24, 256, None, 1, None, None, 9, None, 1, None))
    rc = lib.nvx_rejection_walk_max_width(0)
    assert rc == -1 and b"outside" in lib.nvx_last_error()
    prev = lib.nvx_rejection_walk_max_width(12)  # rounds down to 8
    assert lib.nvx_rejection_walk_max_width(prev) == 8
    rc = lib.nvx_topk_logprobs(None, _C.DTYPE_BF16, 64, 1, 64, 65, None, None, None)
    assert rc == -1 and b"k must be" in lib.nvx_last_error()
    rc = lib.nvx_topk_logprobs(None, _C.DTYPE_BF16, 100, 1, 100, 8, None, None, None)
    assert rc == -1 and b"multiples of 8" in lib.nvx_last_error()
    rc = lib.nvx_softmax_stats(None, _C.DTYPE_BF16, 100, None, None, 1, 100, None)
    assert rc == -1 and b"null pointer" in lib.nvx_last_error()
    # Non-null host addresses: each call is refused before anything is launched.
    rows, stats = ctypes.c_void_p(0x100000), ctypes.c_void_p(0x200004)
    rc = lib.nvx_softmax_stats(rows, _C.DTYPE_BF16, 128, rows, stats, 1, 128, None)
    assert rc == -1 and b"8-byte aligned" in lib.nvx_last_error()
    rc = lib.nvx_softmax_from_stats(rows, _C.DTYPE_BF16, 128, rows, stats, rows, 1, 128, None)
    assert rc == -1 and b"8-byte aligned" in lib.nvx_last_error()
    rc = lib.nvx_rejection_sample_tree_logits(None, _C.DTYPE_BF16, 64, None, None, None, 0, 64, None,
                                              None, None, 65, None, None, None, 1, 1, None, None,
                                              None, None, None, 0, None)
    assert rc == -1 and b"node_stride" in lib.nvx_last_error()


def test_workspace_size_plan():
    from nanovllm import _C
    lib = _C.lib()
    # one split per (seq, kv head) when the grid already fills the GPU: no workspace
    assert lib.nvx_tree_attention_workspace_size(64, 4096, 64, 2112, 32, 8, 128) == 0
    # few long sequences: split-KV partials (fp32 o + lse per split)
    ws = lib.nvx_tree_attention_workspace_size(2, 2, 1, 4096, 32, 8, 128)
    assert ws > 0 and ws % (2 * 32 * 129 * 4) == 0
    assert lib.nvx_tree_attention_workspace_size(2, 2, 1, 4096, 32, 8, 64) == 0
    # a full batch over contexts longer than one split's page table (511 chunks at
    # 64-token pages) still gets KV splits
    assert lib.nvx_tree_attention_workspace_size(64, 64, 1, 32704, 32, 8, 128) == 0
    ws = lib.nvx_tree_attention_workspace_size(64, 64, 1, 40000, 32, 8, 128)
    assert ws == 2 * 64 * 32 * 129 * 4


def test_ops_refuse_cpu_tensors():
    import torch
    from nanovllm.layers.sampler import temperature_softmax
    with pytest.raises(RuntimeError, match="GPU only"):
        temperature_softmax(torch.zeros(2, 8), torch.ones(2))
