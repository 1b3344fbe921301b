"""The tree-attention kernel's per-chunk visibility word against the oracle's per-key
visibility (no GPU).

The kernel (nano-vllm-x_amd/csrc/attention.hip, tree_attn_kernel, the phase_softmax
step) masks a 64-key chunk at positions pos0 .. pos0+63 with one 64-bit word per q
row, built from the row's tree-mask bits, the tree start base = context_len - q_len
and context_len; lane half g of a wave tests bit kt*32 + (j/4)*8 + 4g + j%4 for score
j of S tile kt.  A chunk is masked only if it reaches the first key some row of the
wave cannot see (the tree start with a tree mask; causal, one past the key of the
wave's first node), and a q-row chunk streams keys only up to key_end =
min(context_len, base + last node of its rows + 1).
This restates that logic on the host, bit for bit, and compares every key of every
chunk and row with oracle.attention.tree_visible (reference semantics: the
bottom-right causal decode of nanovllm/layers/attention.py:72-74 generalised to a
tree).  At long contexts the GPU parity tests cannot see a wrong mask bit (the tree
keys carry a few percent of the softmax mass), so this is where the word is pinned.
"""
import numpy as np

from nanovllm.spec.tree import ancestor_masks, chain_parents, random_tree
from oracle.attention import tree_visible

KC = 64
U64 = np.uint64
ALL = U64(0xFFFFFFFFFFFFFFFF)


def low_bits64(n):
    """Bits [0, n) set, n clamped to [0, 64] (the kernel's low_bits64)."""
    if n <= 0:
        return U64(0)
    if n >= 64:
        return ALL
    return U64((1 << n) - 1)


def kernel_word(mbits, node, base, ctxlen, pos0, use_tree):
    """vis64 of the kernel for one row and the chunk at pos0 (only called for chunks
    with pos0 + 64 > base, as in the kernel)."""
    off = base - pos0
    if use_tree:
        mb = U64(int(mbits) & 0xFFFFFFFFFFFFFFFF)
        if off >= 0:
            sh = U64(0) if off >= 64 else U64((int(mb) << off) & 0xFFFFFFFFFFFFFFFF)
        else:
            sh = U64(0) if off <= -64 else U64(int(mb) >> -off)
        vis = sh | low_bits64(off)
    else:
        vis = low_bits64(off + node + 1)
    return vis & low_bits64(ctxlen - pos0)


def kernel_chunk_visibility(mbits, node, wave_first_node, last_node, base, ctxlen, pos0,
                            use_tree):
    """Boolean [64] visibility of keys pos0 .. pos0+63 for one row as the kernel applies
    it: through the lane-half / tile / element mapping of the S accumulators, with
    keys past key_end never streamed."""
    key_end = max(0, min(ctxlen, base + last_node + 1))
    out = np.zeros(KC, dtype=bool)
    if pos0 >= key_end:  # the chunk is not streamed at all
        return out
    mask_from = base if use_tree else base + wave_first_node + 1
    if pos0 + KC > mask_from:
        word = kernel_word(mbits, node, base, ctxlen, pos0, use_tree)
    else:
        word = ALL
    for g in range(2):
        v = int(word) >> (4 * g)
        for kt in range(2):
            for j in range(16):
                bit = kt * 32 + (j >> 2) * 8 + (j & 3)
                key = kt * 32 + (j >> 2) * 8 + 4 * g + (j & 3)
                out[key] = bool((v >> bit) & 1)
    # keys past the streamed end are stale ring data: masked only if the word did
    keys = pos0 + np.arange(KC)
    assert not (out & (keys >= key_end)).any(), "a key past key_end would be visible"
    return out


def check_sequence(parents, ctx, G, W, use_tree):
    """Every row and every chunk of one sequence: tree of `parents` after ctx cached
    tokens, G query heads per KV head (row r is node r // G), W waves of 32 rows per
    q-row chunk (which set each row's wave and its chunk's last node)."""
    q_len = len(parents)
    ctxlen = ctx + q_len
    base = ctx
    masks = ancestor_masks(parents).view(np.uint64) if use_tree else None
    vis = tree_visible(q_len, ctxlen, masks)  # oracle, [q_len, ctxlen]
    nchunks = (ctxlen + KC - 1) // KC
    seen, cases = set(), 0
    for r in range(G * q_len):
        node = r // G
        row0 = (r // (W * 32)) * W * 32
        wave_first_node = (row0 + ((r - row0) // 32) * 32) // G
        last_node = min(q_len - 1, (row0 + W * 32 - 1) // G)
        if (node, wave_first_node, last_node) in seen:
            continue
        seen.add((node, wave_first_node, last_node))
        mb = int(masks[node]) if use_tree else 0
        for c in range(nchunks):
            pos0 = c * KC
            got = kernel_chunk_visibility(mb, node, wave_first_node, last_node, base, ctxlen,
                                          pos0, use_tree)
            want = np.zeros(KC, dtype=bool)
            hi = min(ctxlen, pos0 + KC)
            want[:hi - pos0] = vis[node, pos0:hi]
            assert np.array_equal(got, want), (node, pos0, ctx, q_len)
            cases += 1
    return cases


def test_word_matches_oracle_random_trees():
    """Random EAGLE-style trees (1-64 nodes) after 0-300 cached tokens, so chunks
    straddle the tree start, lie wholly inside the tree, and end past context_len;
    q-row chunks of 8-256 rows at 1-8 heads per KV head."""
    rng = np.random.default_rng(11)
    cases = 0
    for _ in range(700):
        T = int(rng.integers(1, 65))
        depth = int(rng.integers(1, min(T - 1, 10) + 1)) if T > 1 else 0
        parents = random_tree(T, depth, rng) if T > 1 else np.array([-1], np.int32)
        ctx = int(rng.integers(0, 300))
        G = int(rng.choice([1, 2, 4, 5, 8]))
        W = int(rng.choice([4, 8]))
        cases += check_sequence(parents, ctx, G, W, True)
    assert cases > 50000


def test_word_matches_oracle_causal():
    """No tree mask (decode and paged prefill): key base+m visible to row i iff m <= i,
    for q_len 1-300 over 0-300 cached tokens (prefill with no cached tokens included),
    several q-row chunks per sequence; only chunks that reach past the keys every row
    of the wave sees are masked."""
    rng = np.random.default_rng(12)
    for i in range(150):
        T = int(rng.integers(1, 301))
        ctx = 0 if i % 3 == 0 else int(rng.integers(0, 300))
        G = int(rng.choice([1, 2, 4, 5]))
        check_sequence(chain_parents(T), ctx, G, int(rng.choice([4, 8])), False)


def test_word_edge_offsets():
    """The word at every offset of a chunk against the tree start (off = base - pos0
    from -70 to 70) for masks with the top bit set, and context ends inside the chunk."""
    parents = random_tree(64, 8, np.random.default_rng(3))
    masks = ancestor_masks(parents).view(np.uint64)
    for ctx in list(range(0, 130)) + [191, 192, 193, 255, 256, 257]:
        check_sequence(parents, ctx, 4, 8, True)
    assert int(masks[63]) >> 63 == 1


def test_a_planted_mistake_is_caught():
    """A plausible bug -- the lane-half shift 4*g dropped -- fails the comparison."""
    parents = random_tree(32, 6, np.random.default_rng(5))
    masks = ancestor_masks(parents).view(np.uint64)
    vis = tree_visible(32, 100 + 32, masks)
    node, pos0, base, ctxlen = 20, 64, 100, 132
    word = kernel_word(int(masks[node]), node, base, ctxlen, pos0, True)
    wrong = np.zeros(KC, dtype=bool)
    for g in range(2):
        for kt in range(2):
            for j in range(16):
                bit = kt * 32 + (j >> 2) * 8 + (j & 3)
                key = kt * 32 + (j >> 2) * 8 + 4 * g + (j & 3)
                wrong[key] = bool((int(word) >> bit) & 1)  # no >> 4*g
    want = vis[node, pos0:pos0 + KC]
    assert not np.array_equal(wrong, want)
