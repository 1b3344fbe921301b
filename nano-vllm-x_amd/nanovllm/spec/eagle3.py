"""EAGLE-3 dynamic draft trees (EAGLE-2 tree construction, Li et al. 2024,
arXiv:2406.16858; EAGLE-3 draft inputs, arXiv:2503.01840).  Absent in the
reference, which decodes one token per step.

Per verify step and sequence with n committed tokens (the root t[n-1] at position
n-1 is not cached yet; the draft head's cache holds rows 0..n-2):

1. Level 1: the top-k tokens of the draft distribution left by the last draft row
   (row n-2 predicts t[n]); score = draft log-probability.
2. Level j -> j+1 (j < depth): the k frontier nodes of level j become draft rows at
   position n-2+j (token = the node, feature = its parent row's output feature, the
   root-level feature for level 1), attending to the cached rows and to their
   ancestors among the expanded rows (tree mask).  Each yields its top-k children,
   scored by cumulative log-probability; the k best of the k*k candidates form the
   next frontier.  Every level re-runs all expanded rows so the mask covers them.
3. The tree is the root plus the T-1 best candidates of all levels by score (ties
   to the earlier-created node).  Scores never increase along a path, so the set is
   closed under ancestors; nodes are relabelled in BFS order (parents[i] < i).

The target verifies the tree with delta-mode rejection sampling (top-k proposals
are deterministic); afterwards the draft head catches up on the accepted rows with
the target's features.  Everything here stays on the device (no host syncs).
"""
import torch


def select_tree(cand_tokens, cand_scores, cand_parent, cand_level, num_nodes):
    """Top-(num_nodes-1) candidates per sequence, relabelled in BFS order.

    cand_* [B, C] (C candidates in creation order; cand_parent indexes candidates,
    -1 = child of the root; levels start at 1).  Returns (tokens [B, num_nodes-1] of
    the chosen candidates in BFS order, parents [B, num_nodes] long with
    parents[:, 0] = -1 and node 0 the root)."""
    B, C = cand_scores.shape
    n = num_nodes - 1
    if n > C:
        raise ValueError(f"select_tree: {n} nodes requested from {C} candidates")
    dev = cand_scores.device
    # score descending, ties to the earlier candidate (stable sort)
    order = torch.sort(cand_scores, dim=1, descending=True, stable=True).indices[:, :n]
    # BFS order of the chosen set: by level, then by creation index
    key = cand_level.gather(1, order) * C + order
    order = order.gather(1, torch.sort(key, dim=1).indices)
    node_of = torch.full((B, C), -1, dtype=torch.long, device=dev)
    node_of.scatter_(1, order, torch.arange(1, n + 1, device=dev).expand(B, n).contiguous())
    par_c = cand_parent.gather(1, order)
    par_node = torch.where(par_c < 0, torch.zeros_like(par_c),
                           node_of.gather(1, par_c.clamp(min=0)))
    parents = torch.cat([torch.full((B, 1), -1, dtype=torch.long, device=dev), par_node], dim=1)
    return cand_tokens.gather(1, order), parents


def tree_depths(parents, max_depth):
    """Depth of every node, [B, T] long (root 0); max_depth bounds the iterations."""
    d = torch.zeros_like(parents)
    for _ in range(max_depth):
        d = torch.where(parents >= 0, d.gather(1, parents.clamp(min=0)) + 1, torch.zeros_like(d))
    return d


def tree_masks(parents, max_depth):
    """Ancestor-or-self bitmask per node, [B, T] int64 (bit m = node m).  Parents
    precede children, so max_depth rounds of "own | parent's" reach the fixed point."""
    B, T = parents.shape
    own = torch.bitwise_left_shift(torch.ones(1, T, dtype=torch.int64, device=parents.device),
                                   torch.arange(T, device=parents.device))
    own = own.expand(B, T)
    m = own.clone()
    for _ in range(max_depth):
        m = own | torch.where(parents >= 0, m.gather(1, parents.clamp(min=0)), torch.zeros_like(m))
    return m


def expand_tree(draft_rows, root_tokens, root_lp, root_feat, depth, num_nodes):
    """Build one draft tree per sequence.

    draft_rows(tokens [B, R], features [B, R, H], masks [B, R] int64, level) must run
    the draft head on the R = k * level expanded rows and return
    ((top-k tokens [B, k, k], top-k log-probs [B, k, k]) of the next token after each
    of the last k rows, the output features of the last k rows [B, k, H]).
    root_tokens / root_lp [B, k]: top-k of the distribution the last cached draft row
    predicts; root_feat [B, H]: that row's output feature.

    Returns (tree tokens [B, num_nodes-1] without the root, parents [B, num_nodes]).
    """
    B, k = root_tokens.shape
    dev = root_tokens.device
    H = root_feat.shape[-1]
    if k * max(depth - 1, 1) > 64:
        raise ValueError("expand_tree: topk * (depth - 1) expanded rows must fit a 64-row mask")
    cand_tok, cand_score = [root_tokens.long()], [root_lp.float()]
    cand_parent = [torch.full((B, k), -1, dtype=torch.long, device=dev)]
    cand_level = [torch.ones(B, k, dtype=torch.long, device=dev)]
    front_cand = torch.arange(k, device=dev).expand(B, k)
    front_score = cand_score[0]
    rows_tok = root_tokens.long()
    rows_feat = root_feat.unsqueeze(1).expand(B, k, H)
    one = torch.ones(1, dtype=torch.int64, device=dev)
    rows_mask = torch.bitwise_left_shift(one, torch.arange(k, device=dev)).expand(B, k)
    base = k
    for level in range(1, depth):
        (top_tok, top_lp), out_feat = draft_rows(rows_tok, rows_feat.contiguous(), rows_mask, level)
        child_score = (front_score.unsqueeze(2) + top_lp.float()).reshape(B, k * k)
        child_tok = top_tok.long().reshape(B, k * k)
        cand_tok.append(child_tok)
        cand_score.append(child_score)
        cand_parent.append(front_cand.unsqueeze(2).expand(B, k, k).reshape(B, k * k))
        cand_level.append(torch.full((B, k * k), level + 1, dtype=torch.long, device=dev))
        if level == depth - 1:
            break
        best = torch.sort(child_score, dim=1, descending=True, stable=True).indices[:, :k]
        src = best // k                                       # frontier slot of the parent
        parent_row = (level - 1) * k + src                    # its row index
        new_rows = level * k + torch.arange(k, device=dev)
        new_mask = torch.bitwise_left_shift(one, new_rows).expand(B, k) | \
            rows_mask.gather(1, parent_row)
        front_cand = base + best
        front_score = child_score.gather(1, best)
        rows_tok = torch.cat([rows_tok, child_tok.gather(1, best)], dim=1)
        rows_feat = torch.cat([rows_feat, out_feat.gather(1, src.unsqueeze(2).expand(B, k, H))], 1)
        rows_mask = torch.cat([rows_mask, new_mask], dim=1)
        base += k * k
    return select_tree(torch.cat(cand_tok, 1), torch.cat(cand_score, 1),
                       torch.cat(cand_parent, 1), torch.cat(cand_level, 1), num_nodes)
