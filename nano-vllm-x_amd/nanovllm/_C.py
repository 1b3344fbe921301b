"""ctypes binding of libnvx_spec.so (the C ABI declared in include/nvx_spec.h).

torch is imported first so the HIP runtime it bundles (libamdhip64.so.7) is the
one the library binds to; torch provides device memory and streams, every kernel
of the verify path lives in the library.  There is no fallback: if the library is
missing or fails to load, using any op raises.
"""
import ctypes
from ctypes import c_void_p, c_int32, c_int64, c_float, c_size_t, c_double, POINTER
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime before the library)

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libnvx_spec.so"

DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
TIMER_NGRAM, TIMER_STORE_KV, TIMER_KV_COMPACT, TIMER_TREE_ATTENTION, TIMER_SOFTMAX, \
    TIMER_REJECTION, TIMER_TOPK = range(7)

_SIGS = {
    "nvx_version": ([], c_int32),
    "nvx_last_error": ([], ctypes.c_char_p),
    "nvx_ngram_propose": ([c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p,
                           c_void_p, c_void_p], c_int32),
    "nvx_store_kvcache": ([c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p,
                           c_int32, c_int32, c_void_p], c_int32),
    "nvx_kv_compact": ([c_void_p, c_void_p, c_int64, c_int32, c_int32, c_int32, c_void_p, c_int32,
                        c_void_p, c_void_p, c_int32, c_void_p, c_int32, c_void_p], c_int32),
    "nvx_tree_attention_workspace_size": ([c_int32] * 7, c_size_t),
    "nvx_tree_attention": ([c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_void_p,
                            c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32,
                            c_int32, c_int32, c_int32, c_float, c_void_p, c_size_t, c_void_p],
                           c_int32),
    "nvx_tree_attention_noalloc_scratch_bytes": ([], c_size_t),
    "nvx_tree_attention_noalloc": ([c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32,
                                    c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32,
                                    c_int32, c_int32, c_int32, c_int32, c_int32, c_float,
                                    c_void_p], c_int32),
    "nvx_temperature_softmax": ([c_void_p, c_int32, c_int64, c_void_p, c_void_p, c_int32, c_int32,
                                 c_void_p], c_int32),
    "nvx_rejection_sample_tree": ([c_void_p, c_int64, c_void_p, c_int64, c_int32, c_void_p,
                                   c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p,
                                   c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p,
                                   c_void_p, c_size_t, c_void_p], c_int32),
    "nvx_rejection_walk_workspace_size": ([c_int32], c_size_t),
    "nvx_rmsnorm": ([c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32,
                     c_float, c_void_p], c_int32),
    "nvx_qk_norm_rope": ([c_void_p, c_int64, c_int32, c_int32, c_int32, c_void_p, c_void_p,
                          c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_void_p,
                          c_void_p, c_void_p, c_float, c_void_p], c_int32),
    "nvx_silu_mul": ([c_void_p, c_int64, c_void_p, c_int32, c_int32, c_void_p], c_int32),
    "nvx_softmax_stats": ([c_void_p, c_int32, c_int64, c_void_p, c_void_p, c_int32, c_int32,
                           c_void_p], c_int32),
    "nvx_softmax_from_stats": ([c_void_p, c_int32, c_int64, c_void_p, c_void_p, c_void_p, c_int32,
                                c_int32, c_void_p], c_int32),
    "nvx_rejection_sample_tree_logits": ([c_void_p, c_int32, c_int64, c_void_p, c_void_p, c_void_p,
                                          c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_int32,
                                          c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p,
                                          c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                          c_void_p], c_int32),
    "nvx_rejection_sample_tree_logits_lazy": ([c_void_p, c_int32, c_int64, c_void_p, c_void_p,
                                               c_void_p, c_int64, c_int32, c_void_p, c_void_p,
                                               c_void_p, c_int32, c_void_p, c_void_p, c_void_p,
                                               c_int32, c_int32, c_void_p, c_void_p, c_void_p,
                                               c_void_p, c_void_p, c_size_t, c_void_p], c_int32),
    "nvx_topk_logprobs": ([c_void_p, c_int32, c_int64, c_int32, c_int32, c_int32, c_void_p,
                           c_void_p, c_void_p], c_int32),
    "nvx_rejection_walk_max_width": ([c_int32], c_int32),
    "nvx_timing_enable": ([c_int32], c_int32),
    "nvx_timing_read": ([c_int32, POINTER(c_double), POINTER(c_int64)], c_int32),
    "nvx_timing_reset": ([], c_int32),
}

EXPORTED = tuple(_SIGS)

_lib = None


def lib():
    """Load (once) and return the library; raises if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
                f"g.build()'` (hipcc, gfx950). The verify path has no CPU fallback.")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in _SIGS.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        _lib = handle
    return _lib


def check(rc):
    if rc != 0:
        msg = lib().nvx_last_error().decode(errors="replace")
        raise RuntimeError(f"libnvx_spec: {msg} (code {rc})")


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else c_void_p(t.data_ptr())


def stream_of(t):
    return c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_cuda(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("libnvx_spec ops run on the GPU only: got a tensor on "
                               f"{t.device}")


def timing_enable(on=True):
    check(lib().nvx_timing_enable(1 if on else 0))


def timing_reset():
    check(lib().nvx_timing_reset())


def timing_read(kernel_id):
    ms, n = c_double(0), c_int64(0)
    check(lib().nvx_timing_read(kernel_id, ctypes.byref(ms), ctypes.byref(n)))
    return ms.value, n.value
