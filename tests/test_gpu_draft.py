"""Draft-head top-k log-probabilities (HIP, nvx_topk_logprobs) vs the CPU oracle.

Tokens must match exactly (ties to the lower token id); log-probabilities within
2e-5 + 1e-6*|ref| (fp32 sums over up to 152k terms)."""
import numpy as np
import pytest
import torch

from nanovllm.layers.sampler import topk_logprobs
from oracle import draft as odraft


def check(dev, logits, k):
    """logits: CPU tensor [N, V] (bf16 or fp32, possibly a strided view)."""
    print(f"[topk] N={logits.shape[0]} V={logits.shape[1]} k={k} dtype={logits.dtype} "
          f"stride={logits.stride(0)}", flush=True)
    lp, tok = topk_logprobs(logits.to(dev) if logits.is_contiguous() else
                            _strided_copy(logits, dev), k)
    etok, elp = odraft.topk_logprobs(logits.float().numpy(), k)
    assert tok.dtype == torch.int64 and lp.dtype == torch.float32
    assert tok.cpu().numpy().tolist() == etok.tolist()
    err = np.abs(lp.cpu().numpy() - elp)
    assert (err <= 2e-5 + 1e-6 * np.abs(elp)).all(), float(err.max())


def _strided_copy(view, dev):
    """Device tensor with the same row stride as the CPU view."""
    N, V = view.shape
    full = torch.zeros(N, view.stride(0), dtype=view.dtype)
    full[:, :V] = view
    return full.to(dev)[:, :V]


@pytest.mark.gpu
@pytest.mark.parametrize("N,k", [(3, 8), (40, 10)])
def test_qwen_vocab_bf16(dev, N, k):
    g = torch.Generator().manual_seed(N)
    x = (torch.randn(N, 151936, generator=g) * 3).to(torch.bfloat16)
    check(dev, x, k)


@pytest.mark.gpu
@pytest.mark.parametrize("N", [5, 1100])
@pytest.mark.parametrize("k", [1, 10, 64])
def test_heavy_ties_bf16(dev, N, k):
    """Few distinct values: the tie rule decides almost every slot."""
    g = torch.Generator().manual_seed(k * 7 + N)
    x = (torch.randint(0, 6, (N, 4096), generator=g) * 0.5).to(torch.bfloat16)
    check(dev, x, k)


@pytest.mark.gpu
@pytest.mark.parametrize("N", [7, 1030])
def test_fp32_padded_rows(dev, N):
    g = torch.Generator().manual_seed(N)
    full = torch.randn(N, 1012, generator=g) * 5
    check(dev, full[:, :1000], 16)


@pytest.mark.gpu
def test_masked_vocab(dev):
    """Most entries -inf (a masked vocabulary); k still within the finite ones."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(9, 8192, generator=g)
    x[torch.rand(9, 8192, generator=g) < 0.97] = float("-inf")
    check(dev, x.to(torch.bfloat16), 16)


@pytest.mark.gpu
def test_k_equals_vocab_and_monotone_rows(dev):
    g = torch.Generator().manual_seed(4)
    check(dev, torch.randn(6, 64, generator=g).to(torch.bfloat16), 64)
    ramp = torch.arange(16384, dtype=torch.float32)
    check(dev, torch.stack([ramp * 1e-3, -ramp * 1e-3, ramp.flip(0) * 1e-3]), 32)
    check(dev, torch.zeros(2, 2048), 8)


@pytest.mark.gpu
def test_empty_batch(dev):
    lp, tok = topk_logprobs(torch.zeros(0, 512, device=dev), 4)
    assert lp.shape == (0, 4) and tok.shape == (0, 4)
