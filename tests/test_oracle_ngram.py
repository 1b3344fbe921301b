"""Pins the drafter oracle: transformers' routine (golden + live), brute force,
closed-form cases."""
import os

import numpy as np
import pytest

from oracle import ngram as ongram

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ngram_hf.npz")


def test_golden_transformers_prompt_lookup():
    z = np.load(GOLDEN)
    offs, eoffs = z["offsets"], z["expected_offsets"]
    for i, (max_n, k) in enumerate(z["params"]):
        h = z["tokens"][offs[i]:offs[i + 1]]
        exp = z["expected"][eoffs[i]:eoffs[i + 1]].tolist()
        assert ongram.propose_one(h, int(max_n), 1, int(k)) == exp, i
        assert ongram.propose_one_bruteforce(h, int(max_n), 1, int(k)) == exp, i


def test_live_transformers_prompt_lookup():
    torch = pytest.importorskip("torch")
    from transformers.generation.candidate_generator import PromptLookupCandidateGenerator
    rng = np.random.default_rng(5)
    for _ in range(150):
        L = int(rng.integers(1, 60))
        h = rng.integers(0, 4, size=L)
        max_n, k = int(rng.integers(1, 5)), int(rng.integers(1, 6))
        gen = PromptLookupCandidateGenerator(num_output_tokens=k, max_matching_ngram_size=max_n,
                                             max_length=L + 100)
        cand, _ = gen.get_candidates(torch.tensor([h.tolist()]))
        assert ongram.propose_one(h, max_n, 1, k) == cand[0, L:].tolist()


def test_vectorised_equals_bruteforce():
    rng = np.random.default_rng(1)
    for _ in range(500):
        L = int(rng.integers(0, 50))
        h = rng.integers(0, int(rng.integers(1, 6)), size=L)
        mx = int(rng.integers(1, 6))
        mn = int(rng.integers(1, mx + 1))
        k = int(rng.integers(1, 7))
        assert ongram.propose_one(h, mx, mn, k) == ongram.propose_one_bruteforce(h, mx, mn, k)


def test_closed_form_cases():
    assert ongram.propose_one(np.arange(100), 3, 1, 5) == []          # no repeats
    h = list(range(50)) + [10, 11, 12]                                  # planted copy
    assert ongram.propose_one(h, 3, 1, 5) == [13, 14, 15, 16, 17]
    h = [1, 2, 3, 9, 1, 2, 3]                                           # continuation hits the end
    assert ongram.propose_one(h, 3, 1, 5) == [9, 1, 2, 3]
    assert ongram.propose_one([5], 3, 1, 5) == []                       # L <= n
    assert ongram.propose_one([5, 5], 3, 1, 5) == [5]                   # n reduced to L-1
    assert ongram.propose_one([1, 2, 1, 3, 1], 3, 1, 2) == [2, 1]       # left-most 1-gram
    assert ongram.propose_one([1, 2, 1, 3, 1], 3, 2, 2) == []           # min_ngram excludes n=1


def test_batched_layout():
    hist = [np.array([1, 2, 3, 1, 2], np.int32), np.array([], np.int32), np.array([4, 4], np.int32)]
    offs = np.array([0, 5, 5, 7], np.int64)
    d, dl = ongram.ngram_propose(np.concatenate(hist), offs, 3, 1, 3)
    assert dl.tolist() == [3, 0, 1]
    assert d.tolist() == [[3, 1, 2], [-1, -1, -1], [4, -1, -1]]
