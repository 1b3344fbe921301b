"""Pins the draft top-k oracle: torch on tie-free rows, closed forms, and a
brute-force sort with ties."""
import math

import numpy as np
import torch

from oracle import draft as odraft


def test_matches_torch_on_tie_free_rows():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 3001, generator=g, dtype=torch.float64) * 4
    for k in (1, 8, 64):
        tok, lp = odraft.topk_logprobs(x.numpy(), k)
        ev, ei = torch.topk(torch.log_softmax(x, dim=-1), k, dim=-1)
        assert tok.tolist() == ei.tolist()
        np.testing.assert_allclose(lp, ev.numpy(), rtol=0, atol=1e-12)


def test_constant_row_closed_form():
    V, k = 1000, 10
    tok, lp = odraft.topk_logprobs(np.full((2, V), 3.25, np.float32), k)
    assert tok.tolist() == [list(range(k))] * 2
    np.testing.assert_allclose(lp, -math.log(V), rtol=0, atol=1e-12)


def test_two_level_row_closed_form():
    # n entries at a, the rest at b < a: logprob(a) = -ln(n + (V - n) e^(b - a))
    V, n, a, b = 512, 3, 2.0, -1.5
    x = np.full((1, V), b)
    hot = [400, 7, 128]
    x[0, hot] = a
    tok, lp = odraft.topk_logprobs(x, 5)
    assert tok[0].tolist() == sorted(hot) + [0, 1]
    za = -math.log(n + (V - n) * math.exp(b - a))
    np.testing.assert_allclose(lp[0, :3], za, rtol=0, atol=1e-12)
    np.testing.assert_allclose(lp[0, 3:], za + (b - a), rtol=0, atol=1e-12)


def test_brute_force_with_ties():
    rng = np.random.default_rng(1)
    for _ in range(50):
        V = int(rng.integers(1, 40))
        k = int(rng.integers(1, V + 1))
        x = (rng.integers(-3, 4, size=(1, V)) * 0.5).astype(np.float32)
        tok, lp = odraft.topk_logprobs(x, k)
        pairs = sorted(((-float(v), i) for i, v in enumerate(x[0])))
        assert tok[0].tolist() == [i for _, i in pairs[:k]]
        z = sum(math.exp(float(v)) for v in x[0])
        for j, t in enumerate(tok[0]):
            assert abs(lp[0, j] - (float(x[0, t]) - math.log(z))) < 1e-12
