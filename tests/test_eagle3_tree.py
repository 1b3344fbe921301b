"""EAGLE-3 dynamic tree construction (host logic, CPU).

``expand_tree`` / ``select_tree`` are checked against a plain-loop restatement of
the EAGLE-2 procedure (top-k expansion of the k best frontier nodes per level,
then the T-1 best candidates by cumulative log-probability, ties to the earlier
candidate, relabelled in BFS order), driven by a deterministic fake draft head
whose output depends on the whole path (through the feature it passes on).
Scores are quantised so ties across parents occur and the tie rule is exercised.
"""
import numpy as np
import pytest
import torch

from nanovllm.spec.eagle3 import expand_tree, select_tree, tree_depths, tree_masks
from nanovllm.spec.tree import ancestor_masks, depths

V = 97


def fake_step(feat, tok):
    """Output feature of a draft row (deterministic, path dependent)."""
    return (feat * 1.37 + tok * 0.11) % 1.0


def fake_children(out_feat, k):
    """Top-k (tokens, log-probs, descending) after a row with output feature f."""
    base = int(out_feat * 1000)
    toks = [(base + 7 * j * j + 3 * j) % V for j in range(k)]
    # distinct tokens per row
    seen, out = set(), []
    for t in toks:
        while t in seen:
            t = (t + 1) % V
        seen.add(t)
        out.append(t)
    lps = [-0.25 * round(4 * (j * 0.5 + (out_feat * (j + 3)) % 0.5)) for j in range(k)]
    lps = sorted(lps, reverse=True)
    return out, lps


def brute_tree(root_tok, root_lp, root_feat, k, depth, T):
    # candidate: (token, score, parent, level, out_feat_if_expanded)
    cands = [dict(tok=int(t), score=float(l), parent=-1, level=1, feat_in=root_feat)
             for t, l in zip(root_tok, root_lp)]
    frontier = list(range(k))
    for level in range(1, depth):
        new = []
        for f in frontier:
            c = cands[f]
            of = fake_step(c["feat_in"], c["tok"])
            toks, lps = fake_children(of, k)
            for t, l in zip(toks, lps):
                new.append(dict(tok=t, score=np.float32(np.float32(c["score"]) + np.float32(l)),
                                parent=f, level=level + 1, feat_in=of))
        start = len(cands)
        cands += new
        ranked = sorted(range(len(new)), key=lambda i: (-new[i]["score"], i))[:k]
        frontier = [start + i for i in ranked]
    order = sorted(range(len(cands)), key=lambda c: (-cands[c]["score"], c))[:T - 1]
    order.sort(key=lambda c: (cands[c]["level"], c))
    node = {c: i + 1 for i, c in enumerate(order)}
    parents = [-1] + [0 if cands[c]["parent"] < 0 else node[cands[c]["parent"]] for c in order]
    return [cands[c]["tok"] for c in order], parents


def torch_draft_rows(k):
    def run(rows_tok, rows_feat, rows_mask, level):
        B, R = rows_tok.shape
        last_tok = rows_tok[:, R - k:]
        last_feat = rows_feat[:, R - k:, 0]
        out = fake_step(last_feat.double(), last_tok.double())
        tt = torch.empty(B, k, k, dtype=torch.long)
        ll = torch.empty(B, k, k, dtype=torch.float32)
        for b in range(B):
            for i in range(k):
                t, l = fake_children(float(out[b, i]), k)
                tt[b, i] = torch.tensor(t)
                ll[b, i] = torch.tensor(l)
        return (tt, ll), out.unsqueeze(-1)
    return run


@pytest.mark.parametrize("k,depth,T", [(4, 4, 16), (8, 6, 32), (3, 2, 10), (5, 1, 4)])
def test_expand_tree_matches_plain_loops(k, depth, T):
    rng = np.random.default_rng(k * 10 + depth)
    B = 3
    root_tok = torch.from_numpy(np.stack([rng.choice(V, k, replace=False) for _ in range(B)]))
    root_lp = torch.from_numpy(np.sort(-0.25 * rng.integers(0, 8, (B, k)), 1)[:, ::-1].copy()).float()
    root_feat = torch.from_numpy(rng.random((B, 1)))
    toks, parents = expand_tree(torch_draft_rows(k), root_tok, root_lp, root_feat, depth, T)
    for b in range(B):
        et, ep = brute_tree(root_tok[b].tolist(), root_lp[b].tolist(), float(root_feat[b, 0]),
                            k, depth, T)
        assert toks[b].tolist() == et
        assert parents[b].tolist() == ep
        p = parents[b].numpy()
        assert p[0] == -1 and all(p[i] < i for i in range(1, T))
        # depths / masks from the tree helpers agree with the numpy tree utilities
        assert tree_depths(parents[b:b + 1], depth)[0].tolist() == depths(p).tolist()
        assert tree_masks(parents[b:b + 1], depth)[0].tolist() == ancestor_masks(p).tolist()


def test_select_tree_tie_rule_and_closure():
    # candidates: level-1 a(0) b(1); children of a: c(2) d(3); child of b: e(4)
    tok = torch.tensor([[10, 11, 12, 13, 14]])
    score = torch.tensor([[-1.0, -1.0, -1.0, -2.0, -1.0]])   # ties everywhere
    parent = torch.tensor([[-1, -1, 0, 0, 1]])
    level = torch.tensor([[1, 1, 2, 2, 2]])
    t, p = select_tree(tok, score, parent, level, 5)
    # top-4 by (-score, index): a, b, c, e ; BFS: a, b, c, e
    assert t[0].tolist() == [10, 11, 12, 14]
    assert p[0].tolist() == [-1, 0, 0, 1, 2]
