"""Paged KV block pool with a content-addressed prefix cache, built around the
lookahead reservation of speculative verify steps.

A verify step writes the K/V of its draft-tree rows at positions len(seq)-1 ..
len(seq)+rows-2 before any of them is accepted, so a step reserves blocks for a
lookahead of ``rows`` positions (the reference reserves for one new position,
nanovllm/engine/block_manager.py:103-108; rows = 1 is that rule).

Pool state, per block id b:
  refs[b]      number of block tables holding b (numpy int32)
  keys[b]      prefix-cache key of the full block b holds, or None
  contents[b]  that block's token ids, compared on every cache hit so a key
               collision can never alias two different prefixes
Free blocks live in an insertion-ordered set: a released block keeps its key and
stays a prefix-cache hit until it is handed out again, and the block released
longest ago is handed out first.  A cache hit on a free block takes it out of the
set in O(1).

Keys chain block by block: key(i) = xxh3_64(int32 tokens of block i, seed=key(i-1)),
seed 0 for block 0, so equal keys name equal prefixes.  A sequence caches the keys
of its full blocks (``Sequence.block_hashes``); its history only grows, so they stay
valid across steps and preemptions.

With ``key_next_token`` (EAGLE-3 drafting) a block's key and content also cover the
token after the block: the draft K/V row at position p is computed from token p+1,
so the block's last draft row belongs to the prefix only together with that token.
A block is then published once that token is in the history.
"""
from collections import OrderedDict

import numpy as np
import xxhash

from nanovllm.engine.sequence import Sequence


def block_key(token_ids, parent_key: int = 0) -> int:
    """Prefix-cache key of a full block whose predecessor blocks have key parent_key."""
    return xxhash.xxh3_64_intdigest(np.asarray(token_ids, dtype=np.int32).tobytes(),
                                    seed=parent_key)


class BlockManager:

    def __init__(self, num_blocks: int, block_size: int, key_next_token: bool = False):
        if num_blocks <= 0 or block_size <= 0:
            raise ValueError("BlockManager: num_blocks and block_size must be positive")
        self.block_size = block_size
        self.key_next_token = key_next_token
        self.num_blocks = num_blocks
        self.refs = np.zeros(num_blocks, dtype=np.int32)
        self.keys: list[int | None] = [None] * num_blocks
        self.contents: list[tuple | None] = [None] * num_blocks
        self.index: dict[int, int] = {}
        self.free: OrderedDict[int, None] = OrderedDict.fromkeys(range(num_blocks))

    # ------------------------------------------------------------ pool state
    @property
    def num_free_blocks(self) -> int:
        return len(self.free)

    def _take(self, block_id: int | None = None) -> int:
        """Remove a block from the free set (the oldest one if none is named)."""
        if block_id is None:
            block_id, _ = self.free.popitem(last=False)
            self._forget(block_id)  # its content is about to be overwritten
        else:
            del self.free[block_id]
        self.refs[block_id] = 1
        return block_id

    def _forget(self, block_id: int):
        key = self.keys[block_id]
        if key is not None and self.index.get(key) == block_id:
            del self.index[key]
        self.keys[block_id] = None
        self.contents[block_id] = None

    def _release(self, block_id: int):
        self.refs[block_id] -= 1
        assert self.refs[block_id] >= 0, f"block {block_id} released more often than taken"
        if self.refs[block_id] == 0:
            self.free[block_id] = None

    # ---------------------------------------------------------- prefix cache
    def _content(self, seq: Sequence, i: int) -> list[int]:
        """What block i's key covers: its tokens, and with key_next_token the token after
        it (which the caller guarantees is in the history)."""
        toks = seq.block(i)
        if self.key_next_token:
            toks = toks + [seq.token_ids[(i + 1) * self.block_size]]
        return toks

    def _keyable(self, seq: Sequence) -> int:
        """Number of leading blocks whose key the history determines."""
        if self.key_next_token:
            return (len(seq) - 1) // self.block_size
        return len(seq) // self.block_size

    def _keys_of(self, seq: Sequence, num_full_blocks: int) -> list[int]:
        keys = seq.block_hashes
        if num_full_blocks > self._keyable(seq):
            raise ValueError(f"sequence {seq.seq_id}: the keys of {num_full_blocks} blocks need "
                             f"tokens past its {len(seq)}")
        for i in range(len(keys), num_full_blocks):
            keys.append(block_key(self._content(seq, i), keys[i - 1] if i else 0))
        return keys

    def _cached_prefix(self, seq: Sequence) -> list[int]:
        """Block ids caching the sequence's leading full blocks.  The block holding the
        last token is never taken from the cache, so a prefill computes at least one
        position (the one whose logits give the next token)."""
        candidates = (len(seq) - 1) // self.block_size
        hits = []
        for i, key in enumerate(self._keys_of(seq, candidates)[:candidates]):
            b = self.index.get(key)
            if b is None or self.contents[b] != tuple(self._content(seq, i)):
                break
            hits.append(b)
        return hits

    # ------------------------------------------------------------- prefill
    def can_allocate(self, seq: Sequence) -> int:
        """Number of leading blocks the prefix cache supplies, or -1 if the pool cannot
        hold the sequence now.  Hits on blocks other tables hold cost no free block."""
        hits = self._cached_prefix(seq)
        shared = sum(1 for b in hits if self.refs[b] > 0)
        return len(hits) if seq.num_blocks - shared <= len(self.free) else -1

    def allocate(self, seq: Sequence, num_cached_blocks: int):
        if seq.block_table:
            raise RuntimeError(f"sequence {seq.seq_id} already holds blocks")
        hits = self._cached_prefix(seq)[:num_cached_blocks]
        if len(hits) != num_cached_blocks:
            raise RuntimeError("prefix cache changed between can_allocate and allocate")
        for b in hits:
            if self.refs[b] == 0:
                self._take(b)
            else:
                self.refs[b] += 1
        seq.block_table = hits + [self._take() for _ in range(seq.num_blocks - len(hits))]
        seq.num_cached_tokens = len(hits) * self.block_size

    def deallocate(self, seq: Sequence):
        # last block first: the tail is the least shareable part, so it should be
        # the first to be handed out again
        for b in reversed(seq.block_table):
            self._release(b)
        seq.block_table = []
        seq.num_cached_tokens = 0

    # ------------------------------------------------------ decode / verify
    def blocks_needed(self, seq: Sequence, lookahead: int = 1) -> int:
        """New blocks a step writing `lookahead` rows from position len(seq)-1 needs."""
        last = len(seq) - 2 + lookahead
        return max(0, last // self.block_size + 1 - len(seq.block_table))

    def can_append(self, seq: Sequence, lookahead: int = 1) -> bool:
        return self.blocks_needed(seq, lookahead) <= len(self.free)

    def may_append(self, seq: Sequence, lookahead: int = 1):
        seq.block_table.extend(self._take() for _ in range(self.blocks_needed(seq, lookahead)))

    # ------------------------------------------------------------- publish
    def hash_blocks(self, seq: Sequence, num_cached_tokens: int | None = None):
        """Publish to the prefix cache every block that becomes full and cached when
        the sequence's cached length grows from seq.num_cached_tokens to
        num_cached_tokens (default: + seq.num_scheduled_tokens)."""
        if num_cached_tokens is None:
            num_cached_tokens = seq.num_cached_tokens + seq.num_scheduled_tokens
        first = seq.num_cached_tokens // self.block_size
        last = min(num_cached_tokens // self.block_size, self._keyable(seq))
        if last <= first:
            return
        keys = self._keys_of(seq, last)
        for i in range(first, last):
            b = seq.block_table[i]
            self.keys[b] = keys[i]
            self.contents[b] = tuple(self._content(seq, i))
            self.index[keys[i]] = b
