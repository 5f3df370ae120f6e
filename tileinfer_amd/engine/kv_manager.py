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

Swapping (advertised by the reference, never implemented: engine/config.py:22,
engine/block_manager.py:29): ``swap_out`` moves a sequence's unshared blocks to slots of a pinned
host pool and frees them on the device; ``swap_in`` brings them back into fresh device blocks at
the same logical positions. Both return the ``(source, destination)`` pairs that
``tileinfer_amd.kernels.block_copy.swap_blocks`` executes; shared (prefix) blocks stay resident.
"""
from __future__ import annotations

from typing import Callable

from .block_manager import BlockManager
from .prefix_cache import PrefixCache
from .sequence import Sequence


class PagedKVManager:
    def __init__(self, num_blocks: int, block_size: int, enable_prefix_caching: bool = True,
                 num_host_blocks: int = 0):
        self.block_size = block_size
        self.block_manager = BlockManager(num_blocks, block_size)
        self.host_free: list[int] = list(range(num_host_blocks - 1, -1, -1))
        self.swapped: dict[int, list[tuple[int, int]]] = {}  # seq_id -> [(table index, host slot)]
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
        for _, slot in self.swapped.pop(seq.seq_id, []):
            self.host_free.append(slot)
        seq.block_table[:] = [b for b in seq.block_table if b >= 0]
        seq.table_changed()
        return self.block_manager.deallocate(seq)

    def swap_out(self, seq: Sequence, max_blocks: int | None = None) -> list[tuple[int, int]]:
        """Move up to ``max_blocks`` of the sequence's unshared blocks to host slots.

        Returns ``(device block, host slot)`` pairs to copy device -> host before the freed device
        blocks are reused (stream order does that when both run on one stream). The table keeps
        -1 at swapped positions until ``swap_in``. Raises if the host pool is too small.
        """
        if seq.seq_id in self.swapped:
            raise ValueError(f"sequence {seq.seq_id} is already swapped out")
        bm = self.block_manager
        todo = [i for i, b in enumerate(seq.block_table) if b >= 0 and bm.ref_counts[b] == 1]
        if max_blocks is not None:
            todo = todo[:max_blocks]
        if len(todo) > len(self.host_free):
            raise RuntimeError(f"host swap pool has {len(self.host_free)} free slots, "
                               f"{len(todo)} needed")
        pairs, record = [], []
        for i in todo:
            slot = self.host_free.pop()
            pairs.append((seq.block_table[i], slot))
            record.append((i, slot))
            bm.release(seq.block_table[i])
            seq.block_table[i] = -1
        if record:
            seq.table_changed()
        self.swapped[seq.seq_id] = record
        return pairs

    def can_swap_in(self, seq: Sequence) -> bool:
        return self.block_manager.num_free_blocks >= len(self.swapped.get(seq.seq_id, ()))

    def swap_in(self, seq: Sequence) -> list[tuple[int, int]]:
        """Give the sequence's swapped positions fresh device blocks.

        Returns ``(host slot, device block)`` pairs to copy host -> device before the sequence runs.
        """
        record = self.swapped.pop(seq.seq_id, [])
        if len(record) > self.block_manager.num_free_blocks:
            self.swapped[seq.seq_id] = record
            raise RuntimeError("not enough free device blocks to swap in")
        pairs = []
        for i, slot in record:
            bid = self.block_manager.allocate_block()
            seq.block_table[i] = bid
            pairs.append((slot, bid))
            self.host_free.append(slot)
        if record:
            seq.table_changed()
        return pairs

    def common_prefix_tokens(self, seqs: list[Sequence]) -> int:
        """Tokens at the start of every sequence held in the same physical blocks (whole blocks,
        as prefix caching shares them): the ``shared_prefix_tokens`` of a decode over this batch.
        0 for fewer than two sequences."""
        if len(seqs) < 2:
            return 0
        n = min(len(s.block_table) for s in seqs)
        first = seqs[0].block_table
        common = 0
        while common < n and first[common] >= 0 and all(s.block_table[common] == first[common]
                                                         for s in seqs[1:]):
            common += 1
        return common * self.block_size

    def shares_blocks(self, seqs: list[Sequence]) -> bool:
        """Whether any block of these sequences is held by more than one sequence: the decode
        hint ``kv_reuse`` (shared pages are then worth keeping in cache)."""
        refs = self.block_manager.ref_counts
        return any(b >= 0 and refs[b] > 1 for s in seqs for b in s.block_table)
