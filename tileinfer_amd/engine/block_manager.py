"""Physical KV block pool with reference counts (the role of tileInfer's ``engine/block_manager.py``).

State is two int32 arrays, the shape the device-side tables and a future GPU allocator want:

* ``ref_counts[num_blocks]`` -- how many block tables hold each block (0 = free);
* a free stack ``_stack[:_top]`` -- ids of the free blocks, the next one to hand out on top.

Observable behaviour matches the reference (engine/block_manager.py:26-117) so a block id sequence
is the same for the same calls:

* a fresh pool hands out 0, 1, 2, ... (the stack starts as ``n-1 .. 0`` with 0 on top);
* a released block goes back on top, so it is the next one reused (LIFO);
* releasing a table walks it from its last entry to its first, and each block whose count reaches
  0 is pushed and reported through ``on_block_freed`` in that order (prefix-cache eviction);
* ``share_blocks`` adopts live blocks (a prefix-cache hit) by raising their counts.

Two fixes. ``may_append``: the reference allocates only when ``len(seq) % block_size == 0``, one
token early, and so never gives the first decode token of a prompt whose length is a multiple of
the block size a slot (engine/block_manager.py:107-117); here it also allocates while the table
holds fewer slots than tokens, and ``can_append`` counts both. Releasing a block that is already
free, or an id outside ``[0, num_blocks)``, raises instead of corrupting the pool (numpy would
wrap a -1 to the last block). ``deallocate`` skips negative table entries: they are positions
that hold no device block (swapped out to host memory), the way the device tables mark them.
"""
from __future__ import annotations

from typing import Callable, NamedTuple

import numpy as np

from .sequence import Sequence


class Block(NamedTuple):
    """A read-only snapshot of one pool entry."""
    block_id: int
    ref_count: int


class _BlockView:
    """``pool.blocks[i]`` -> ``Block(i, ref_counts[i])`` (snapshots of the count array)."""

    __slots__ = ("_refs",)

    def __init__(self, refs: np.ndarray):
        self._refs = refs

    def __len__(self) -> int:
        return int(self._refs.shape[0])

    def __getitem__(self, block_id: int) -> Block:
        return Block(int(block_id), int(self._refs[block_id]))


class BlockManager:
    """Pool of ``num_blocks`` KV blocks of ``block_size`` token slots each."""

    def __init__(self, num_blocks: int, block_size: int, swap_space_bytes: int = 0):
        if num_blocks < 0 or block_size <= 0:
            raise ValueError(f"bad pool: num_blocks={num_blocks}, block_size={block_size}")
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.swap_space_bytes = swap_space_bytes  # accepted for signature parity; unused
        self.ref_counts = np.zeros(num_blocks, dtype=np.int32)
        self._stack = np.arange(num_blocks - 1, -1, -1, dtype=np.int32)
        self._top = num_blocks
        self.on_block_freed: Callable[[int], None] | None = None

    # -- views -------------------------------------------------------------------------------------

    @property
    def num_free_blocks(self) -> int:
        return self._top

    @property
    def free_block_ids(self) -> list[int]:
        """Free ids, bottom of the stack first (the last one is handed out next)."""
        return self._stack[:self._top].tolist()

    @property
    def used_block_ids(self) -> set[int]:
        return set(np.flatnonzero(self.ref_counts).tolist())

    @property
    def blocks(self) -> _BlockView:
        return _BlockView(self.ref_counts)

    def ref_count(self, block_id: int) -> int:
        return int(self.ref_counts[block_id])

    # -- the stack ---------------------------------------------------------------------------------

    def _take(self, n: int) -> list[int]:
        """Pop ``n`` ids off the stack (top first) with count 1 each."""
        if n > self._top:
            raise RuntimeError(f"KV block pool exhausted: {n} blocks wanted, {self._top} free")
        if n <= 0:
            return []
        ids = self._stack[self._top - n:self._top][::-1].copy()
        if self.ref_counts[ids].any():
            raise AssertionError("a block on the free stack has references")
        self.ref_counts[ids] = 1
        self._top -= n
        return ids.tolist()

    def _push_freed(self, ids: list[int]) -> None:
        """Return ids (count already 0) to the stack in the given order and report each one."""
        n = len(ids)
        if not n:
            return
        self._stack[self._top:self._top + n] = ids
        self._top += n
        if self.on_block_freed is not None:
            for block_id in ids:
                self.on_block_freed(block_id)

    def _check_ids(self, arr: np.ndarray) -> None:
        bad = (arr < 0) | (arr >= self.num_blocks)
        if bad.any():
            raise ValueError(f"block id {int(arr[bad][0])} is outside the pool "
                             f"[0, {self.num_blocks})")

    def _drop(self, ids: list[int]) -> list[int]:
        """Drop one reference per listing of each id, walking the list last to first; returns the
        ids that became free, in the order they go back on the stack."""
        if not ids:
            return []
        arr = np.asarray(ids[::-1], dtype=np.int64)
        self._check_ids(arr)
        uniq, mult = np.unique(arr, return_counts=True)
        short = self.ref_counts[uniq] < mult
        if short.any():
            raise ValueError(f"block {int(uniq[short][0])} is already free")
        np.subtract.at(self.ref_counts, arr, 1)
        if uniq.size == arr.size:
            freed = arr[self.ref_counts[arr] == 0].tolist()
        else:
            # An id listed twice is freed at its last listing in walk order.
            last = {int(b): i for i, b in enumerate(arr.tolist())}
            freed = sorted((b for b in last if self.ref_counts[b] == 0), key=last.__getitem__)
        self._push_freed(freed)
        return freed

    # -- sequences ---------------------------------------------------------------------------------

    def can_allocate(self, seq: Sequence) -> bool:
        return self._top >= seq.num_blocks

    def allocate(self, seq: Sequence) -> None:
        """Give a fresh sequence all the blocks its tokens need."""
        if seq.block_table:
            raise ValueError(f"sequence {seq.seq_id} already has blocks")
        seq.block_table = self._take(seq.num_blocks)
        seq.table_changed()
        seq.num_cached_tokens = 0

    def share_blocks(self, seq: Sequence, block_ids: list[int]) -> None:
        """Adopt live blocks (a prefix-cache hit): their K/V is already valid."""
        if seq.block_table:
            raise ValueError(f"sequence {seq.seq_id} already has blocks")
        arr = np.asarray(block_ids, dtype=np.int64)
        self._check_ids(arr)
        if arr.size and (self.ref_counts[arr] <= 0).any():
            bad = int(arr[self.ref_counts[arr] <= 0][0])
            raise ValueError(f"cannot share free block {bad}")
        np.add.at(self.ref_counts, arr, 1)
        seq.block_table = [int(b) for b in block_ids]
        seq.table_changed()

    def can_allocate_remaining(self, seq: Sequence) -> bool:
        return self._top >= seq.num_blocks - len(seq.block_table)

    def allocate_extra(self, seq: Sequence) -> None:
        """Allocate the blocks still needed to reach ``seq.num_blocks``."""
        seq.block_table.extend(self._take(max(0, seq.num_blocks - len(seq.block_table))))

    def deallocate(self, seq: Sequence) -> list[int]:
        """Drop the sequence's references; return the ids whose count reached 0 (freed).
        Negative entries (positions swapped out to host memory) hold no device block and are
        skipped."""
        freed = self._drop([b for b in seq.block_table if b >= 0])
        seq.block_table.clear()
        seq.table_changed()
        return freed

    def allocate_block(self) -> int:
        """Take one free block (reference count 1); the caller places it in a table."""
        return self._take(1)[0]

    def release(self, block_id: int) -> bool:
        """Drop one reference to ``block_id``; returns True when that freed it."""
        return bool(self._drop([block_id]))

    # -- decode growth -----------------------------------------------------------------------------

    def _blocks_needed_for_append(self, seq: Sequence) -> int:
        short = max(0, seq.num_blocks - len(seq.block_table))   # slots missing for len(seq) tokens
        ahead = 1 if len(seq) % self.block_size == 0 else 0     # the reference's early trigger
        return short + ahead

    def can_append(self, seq: Sequence) -> bool:
        """Whether the slot of the newest token (and the reference's look-ahead block) fits."""
        return self._top >= self._blocks_needed_for_append(seq)

    def may_append(self, seq: Sequence) -> None:
        """Make room for the newest token's K/V, allocating blocks as needed."""
        need = self._blocks_needed_for_append(seq)
        if need > self._top:
            raise RuntimeError(f"KV block pool exhausted: {need} blocks wanted, {self._top} free")
        seq.block_table.extend(self._take(need))
