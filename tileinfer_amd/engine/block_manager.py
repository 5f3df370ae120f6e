"""Refcounted physical block pool: the allocation semantics of tileInfer's ``engine/block_manager.py``.

Kept identical to the reference so block ids come out in the same order
(engine/block_manager.py:26-117):
  * the free list starts as ``[n-1, ..., 1, 0]`` and is popped from the end, so a fresh pool hands
    out 0, 1, 2, ... and a freed block is the next one reused (LIFO);
  * ``share_blocks`` adopts prefix-cache blocks by bumping their reference count;
  * ``deallocate`` walks the table in reverse, frees blocks whose count reaches 0 and reports each
    through ``on_block_freed`` (used to evict prefix-cache entries).

One fix (the reference's ``may_append`` only allocates when ``len(seq) % block_size == 0``, which
misses the first decode token of a prompt whose length is a multiple of the block size,
engine/block_manager.py:107-117): ``may_append`` keeps that one-block-ahead trigger and also
allocates whenever the table holds fewer than ``len(seq)`` slots; ``can_append`` counts both.
"""
from __future__ import annotations

from typing import Callable

from .sequence import Sequence


class Block:
    __slots__ = ("block_id", "ref_count")

    def __init__(self, block_id: int):
        self.block_id = block_id
        self.ref_count = 0

    def reset(self) -> None:
        self.ref_count = 1


class BlockManager:
    """Pool of ``num_blocks`` KV blocks of ``block_size`` token slots each."""

    def __init__(self, num_blocks: int, block_size: int, swap_space_bytes: int = 0):
        if num_blocks < 0 or block_size <= 0:
            raise ValueError(f"bad pool: num_blocks={num_blocks}, block_size={block_size}")
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.swap_space_bytes = swap_space_bytes  # accepted for signature parity; unused
        self.blocks: list[Block] = [Block(i) for i in range(num_blocks)]
        self.free_block_ids: list[int] = list(range(num_blocks - 1, -1, -1))
        self.used_block_ids: set[int] = set()
        self.on_block_freed: Callable[[int], None] | None = None

    @property
    def num_free_blocks(self) -> int:
        return len(self.free_block_ids)

    def _allocate_block(self) -> int:
        if not self.free_block_ids:
            raise RuntimeError("KV block pool exhausted")
        block_id = self.free_block_ids.pop()
        block = self.blocks[block_id]
        assert block.ref_count == 0, f"block {block_id} on the free list with refs"
        block.reset()
        self.used_block_ids.add(block_id)
        return block_id

    def _deallocate_block(self, block_id: int) -> None:
        assert self.blocks[block_id].ref_count == 0
        self.used_block_ids.remove(block_id)
        self.free_block_ids.append(block_id)

    def can_allocate(self, seq: Sequence) -> bool:
        return self.num_free_blocks >= seq.num_blocks

    def allocate(self, seq: Sequence) -> None:
        """Give a fresh sequence all the blocks its tokens need."""
        if seq.block_table:
            raise ValueError(f"sequence {seq.seq_id} already has blocks")
        for _ in range(seq.num_blocks):
            seq.block_table.append(self._allocate_block())
        seq.num_cached_tokens = 0

    def share_blocks(self, seq: Sequence, block_ids: list[int]) -> None:
        """Adopt existing blocks (a prefix-cache hit): their K/V is already valid."""
        if seq.block_table:
            raise ValueError(f"sequence {seq.seq_id} already has blocks")
        for block_id in block_ids:
            if self.blocks[block_id].ref_count <= 0:
                raise ValueError(f"cannot share free block {block_id}")
        seq.block_table = list(block_ids)
        for block_id in block_ids:
            self.blocks[block_id].ref_count += 1

    def can_allocate_remaining(self, seq: Sequence) -> bool:
        return self.num_free_blocks >= seq.num_blocks - len(seq.block_table)

    def allocate_extra(self, seq: Sequence) -> None:
        """Allocate the blocks still needed to reach ``seq.num_blocks``."""
        while len(seq.block_table) < seq.num_blocks:
            seq.block_table.append(self._allocate_block())

    def deallocate(self, seq: Sequence) -> list[int]:
        """Drop the sequence's references; return the ids whose count reached 0 (freed)."""
        freed: list[int] = []
        for block_id in reversed(seq.block_table):
            block = self.blocks[block_id]
            block.ref_count -= 1
            if block.ref_count <= 0:
                block.ref_count = 0
                self._deallocate_block(block_id)
                freed.append(block_id)
                if self.on_block_freed is not None:
                    self.on_block_freed(block_id)
        seq.block_table.clear()
        return freed

    def allocate_block(self) -> int:
        """Take one free block (reference count 1); the caller places it in a table."""
        return self._allocate_block()

    def release(self, block_id: int) -> bool:
        """Drop one reference to ``block_id``; returns True when that freed it."""
        block = self.blocks[block_id]
        if block.ref_count <= 0:
            raise ValueError(f"block {block_id} is already free")
        block.ref_count -= 1
        if block.ref_count == 0:
            self._deallocate_block(block_id)
            if self.on_block_freed is not None:
                self.on_block_freed(block_id)
            return True
        return False

    def _blocks_needed_for_append(self, seq: Sequence) -> int:
        short = max(0, seq.num_blocks - len(seq.block_table))   # slots missing for len(seq) tokens
        ahead = 1 if len(seq) % self.block_size == 0 else 0     # the reference's early trigger
        return short + ahead

    def can_append(self, seq: Sequence) -> bool:
        """Whether the slot of the newest token (and the reference's look-ahead block) fits."""
        return self.num_free_blocks >= self._blocks_needed_for_append(seq)

    def may_append(self, seq: Sequence) -> None:
        """Make room for the newest token's K/V, allocating blocks as needed."""
        while len(seq.block_table) * self.block_size < len(seq):
            seq.block_table.append(self._allocate_block())
        if len(seq) % self.block_size == 0:
            seq.block_table.append(self._allocate_block())
