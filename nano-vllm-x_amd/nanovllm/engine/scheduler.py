"""Continuous-batching scheduler for prefill and speculative verify steps.

A step is either a prefill batch or a decode batch, never both (the reference's
split, nanovllm/engine/scheduler.py:25-73):

* prefill: waiting sequences are admitted in arrival order while the step's token
  budget (``max_num_batched_tokens``), ``max_num_seqs`` and the block pool allow.
  The budget is filled completely: the last sequence admitted may get only a chunk
  of its prompt and stays at the head of the waiting queue until the rest is cached.
* decode / verify: the running sequences (at most ``max_num_seqs``, in order) each
  reserve ``lookahead`` KV positions for the draft rows the step writes
  (``Config.verify_lookahead``; 1 for plain decode).  The reservations are planned
  for the whole batch first; while they do not fit in the pool, the running
  sequence admitted last is preempted (its blocks freed, it is recomputed from the
  head of the waiting queue later).
* postprocess: a decode step returns, per sequence, the accepted draft tokens and
  the recovered / bonus token; they are appended in path order and the stop rule
  (EOS unless ignore_eos, or max_tokens; reference scheduler.py:89) is applied per
  token.  Cached-token counts advance to len(seq) - 1 (the last token is the next
  step's root) and newly full blocks are published to the prefix cache.
"""
from collections import deque
from itertools import islice

from nanovllm.config import Config
from nanovllm.engine.block_manager import BlockManager
from nanovllm.engine.sequence import Sequence, SequenceStatus


class Scheduler:

    def __init__(self, config: Config):
        self.max_num_seqs = config.max_num_seqs
        self.max_num_batched_tokens = config.max_num_batched_tokens
        self.eos = config.eos
        self.block_size = config.kvcache_block_size
        self.lookahead = config.verify_lookahead
        # EAGLE-3's draft K/V row at position p depends on token p+1: prefix-cache keys
        # then cover the token after each block
        self.block_manager = BlockManager(config.num_kvcache_blocks, config.kvcache_block_size,
                                          key_next_token=config.speculative_method == "eagle3")
        self.waiting: deque[Sequence] = deque()
        self.running: deque[Sequence] = deque()

    def is_finished(self):
        return not self.waiting and not self.running

    def add(self, seq: Sequence):
        self.waiting.append(seq)

    def schedule(self) -> tuple[list[Sequence], bool]:
        batch = self._prefill_batch()
        if batch:
            return batch, True
        batch = self._decode_batch()
        if not batch:
            raise RuntimeError("scheduler: nothing can run (the KV pool is too small for one "
                               "sequence's next step)")
        return batch, False

    # ------------------------------------------------------------- prefill
    def _prefill_batch(self) -> list[Sequence]:
        bm = self.block_manager
        budget = self.max_num_batched_tokens
        batch = []
        while self.waiting and budget > 0 and len(batch) < self.max_num_seqs:
            seq = self.waiting[0]
            if not seq.block_table:
                hits = bm.can_allocate(seq)
                if hits < 0:
                    break  # the pool cannot hold it; running sequences free blocks first
                bm.allocate(seq, hits)
            todo = len(seq) - seq.num_cached_tokens
            seq.num_scheduled_tokens = min(todo, budget)
            budget -= seq.num_scheduled_tokens
            batch.append(seq)
            if seq.num_scheduled_tokens < todo:
                break  # a chunk: the rest of the prompt goes in later steps
            self.waiting.popleft()
            seq.status = SequenceStatus.RUNNING
            self.running.append(seq)
        return batch

    # -------------------------------------------------------------- decode
    def _decode_batch(self) -> list[Sequence]:
        bm = self.block_manager
        batch = list(islice(self.running, self.max_num_seqs))
        need = [bm.blocks_needed(seq, self.lookahead) for seq in batch]
        while batch and sum(need) > bm.num_free_blocks:
            victim = self.running.pop()
            if batch[-1] is victim:
                batch.pop()
                need.pop()
            self.preempt(victim)
        for seq, n in zip(batch, need):
            if n:
                bm.may_append(seq, self.lookahead)
        return batch

    def preempt(self, seq: Sequence):
        """Free the sequence's blocks and requeue it for recomputation."""
        self.block_manager.deallocate(seq)
        seq.status = SequenceStatus.WAITING
        seq.num_scheduled_tokens = 0
        self.waiting.appendleft(seq)

    # --------------------------------------------------------- postprocess
    def postprocess(self, seqs: list[Sequence], token_ids: list, is_prefill: bool):
        """token_ids[i] is an int (one token, as in the reference) or a list of the
        verify step's accepted draft tokens followed by the recovered/bonus token."""
        bm = self.block_manager
        for seq, new in zip(seqs, token_ids):
            new = [new] if isinstance(new, int) else list(new)
            if not is_prefill and (not new or min(new) < 0):
                # a step always yields at least the recovered / bonus token; -1 marks a
                # failed walk row, never a token
                raise RuntimeError(f"sequence {seq.seq_id}: a decode step must append at least "
                                   f"one token id >= 0 (got {new})")
            if is_prefill:
                cached = seq.num_cached_tokens + seq.num_scheduled_tokens
                seq.num_scheduled_tokens = 0
                if cached < len(seq):  # a prompt chunk: no token is sampled yet
                    bm.hash_blocks(seq, cached)
                    seq.num_cached_tokens = cached
                    continue
            else:
                seq.num_verify_steps += 1
                seq.num_accepted_draft += len(new) - 1
            seq.extend_until_stop(new, self.eos)
            if is_prefill:
                # published after the sampled token joins the history, so a block that
                # ends the prompt can carry the token after it in its key
                bm.hash_blocks(seq, cached)
                seq.num_cached_tokens = cached
            if seq.is_finished:
                bm.deallocate(seq)
                self.running.remove(seq)
            elif not is_prefill:
                # the root and the accepted rows are cached now; the last token is not
                cached = len(seq.token_ids) - 1
                if cached // self.block_size > seq.num_cached_tokens // self.block_size:
                    bm.hash_blocks(seq, cached)  # a block became full
                seq.num_cached_tokens = cached
