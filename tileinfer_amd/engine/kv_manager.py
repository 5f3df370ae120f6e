"""Block and prefix-sharing flow of a scheduler over the paged KV cache.

The parts of tileInfer's ``engine/scheduler.py`` that decide which physical blocks a sequence
holds, without its batching policy:

* admitting a new sequence (engine/scheduler.py:161-189): try the longest cached whole-block
  prefix; on a hit adopt those blocks (``share_blocks``), mark the matched tokens cached and
  allocate the rest; otherwise allocate everything. New tokens therefore never land in a shared
  block, so no copy-on-write is needed;
* a decode step's slot (engine/scheduler.py:93-108): ``can_append`` / ``may_append``;
* after a prefill chunk (engine/scheduler.py:243-250): record the prefix in the cache when the
  cached token count sits on a block boundary;
* teardown (engine/scheduler.py:50-62, 289-293): drop references; every block that becomes free
  evicts the prefix-cache entries that end in it.

One fix: the reference can match every block of a prompt whose length is a multiple of the block
size, leaving nothing to prefill, so the sequence is never scheduled (engine/scheduler.py:127-131).
Here a match is cut back by one block when it would cover the whole prompt.
"""
from __future__ import annotations

from typing import Callable

from .block_manager import BlockManager
from .prefix_cache import PrefixCache
from .sequence import Sequence


class PagedKVManager:
    def __init__(self, num_blocks: int, block_size: int, enable_prefix_caching: bool = True):
        self.block_size = block_size
        self.block_manager = BlockManager(num_blocks, block_size)
        self.prefix_cache = PrefixCache(block_size)
        self.enable_prefix_caching = enable_prefix_caching
        self.on_block_freed: Callable[[int], None] | None = None
        self.block_manager.on_block_freed = self._on_block_freed

    def _on_block_freed(self, block_id: int) -> None:
        self.prefix_cache.evict_block(block_id)
        if self.on_block_freed is not None:
            self.on_block_freed(block_id)

    def admit(self, seq: Sequence) -> bool:
        """Give a fresh sequence its blocks, sharing a cached prefix when one matches.

        Returns False (and changes nothing) when the pool cannot hold the sequence.
        """
        if seq.block_table:
            raise ValueError(f"sequence {seq.seq_id} already has blocks")
        bm = self.block_manager
        if self.enable_prefix_caching:
            matched, n = self.prefix_cache.find_longest_prefix(seq.token_ids)
            if matched and n >= seq.num_tokens:
                matched = matched[:-1]
                n -= self.block_size
            if matched and bm.num_free_blocks >= seq.num_blocks - len(matched):
                bm.share_blocks(seq, matched)
                seq.num_cached_tokens = n
                bm.allocate_extra(seq)
                return True
        if bm.can_allocate(seq):
            bm.allocate(seq)
            return True
        return False

    def can_append(self, seq: Sequence) -> bool:
        return self.block_manager.can_append(seq)

    def append_slot(self, seq: Sequence) -> None:
        """Make room for the newest token of a decoding sequence."""
        self.block_manager.may_append(seq)

    def finish_chunk(self, seq: Sequence, num_tokens: int) -> None:
        """Account a computed prefill chunk of ``num_tokens`` and record whole-block prefixes."""
        seq.num_cached_tokens += num_tokens
        seq.num_scheduled_tokens = 0
        if (self.enable_prefix_caching and seq.is_prefill and seq.num_cached_tokens > 0
                and seq.num_cached_tokens % self.block_size == 0):
            # Only tokens whose K/V has been written are recorded (the reference records every
            # whole block of the prompt, engine/scheduler.py:248, which its one-prefill-at-a-time
            # admission keeps from being matched early).
            self.prefix_cache.add(seq.token_ids[:seq.num_cached_tokens], seq.block_table)

    def free(self, seq: Sequence) -> list[int]:
        return self.block_manager.deallocate(seq)

    def shares_blocks(self, seqs: list[Sequence]) -> bool:
        """Whether any block of these sequences is held by more than one sequence: the decode
        hint ``kv_reuse`` (shared pages are then worth keeping in cache)."""
        blocks = self.block_manager.blocks
        return any(blocks[b].ref_count > 1 for s in seqs for b in s.block_table)
