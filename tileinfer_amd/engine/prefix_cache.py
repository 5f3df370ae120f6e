"""Whole-block prefix index over the paged KV cache (the role of tileInfer's ``engine/prefix_cache.py``).

What it promises (engine/prefix_cache.py:1-20, 51-118):

* a block of ``block_size`` tokens is reused only at the position where its K/V was computed, so
  an entry is keyed by the whole token prefix up to its block boundary, never by the block's own
  tokens alone (rotary positions make K/V position-dependent);
* ``find_longest_prefix`` returns the physical blocks of the longest recorded whole-block prefix;
* ``add`` records every whole-block boundary of a computed prefix, repeatably;
* ``evict_block`` forgets every recorded prefix that contains a block the pool just freed.

Design: a flat table of entries, one per recorded boundary. Entry ``e`` holds the physical block of
its own last ``block_size`` tokens (``_block[e]``) and its parent entry; the dictionary
``_index[(parent, tokens of the block)] -> e`` is the only lookup structure (parent ``-1`` is the
empty prefix), so a lookup of ``k`` blocks is ``k`` dictionary probes and the block chain of an
entry is the path of blocks from the first boundary down to it. A reverse index
``_by_block[block] -> entries`` finds the entries to forget when a block is freed; forgetting an
entry forgets its descendants (their chains pass through it), and forgotten entries are removed,
so every entry in the table is live and every live entry's ancestors are live.

When two sequences compute the same prefix into different blocks (both admitted before either
recorded it), the entry keeps the first recorded block: both hold the same K/V, and the first one
stays registered under exactly the block it names, so freeing either sequence evicts exactly the
entries that name its blocks. (The reference replaces the chain but keeps the reverse index on the
old block, so freeing the later sequence leaves an entry pointing at freed blocks.)

``max_entries`` (0 = no cap; the reference's scheduler runs without one, engine/scheduler.py:41)
bounds the table by forgetting the oldest recorded entries that have no descendants.
"""
from __future__ import annotations

from typing import Sequence as _Seq


class PrefixCache:
    """Maps token prefixes (whole blocks) to the physical blocks that hold their K/V."""

    def __init__(self, block_size: int, max_entries: int = 0):
        if block_size <= 0:
            raise ValueError("block_size must be positive")
        self.block_size = block_size
        self.max_entries = max_entries
        self.clear()

    def clear(self) -> None:
        self._index: dict[tuple[int, tuple[int, ...]], int] = {}
        # Per entry id (slots of forgotten entries are reused through _free_ids).
        self._block: list[int] = []
        self._parent: list[int] = []
        self._key: list[tuple[int, tuple[int, ...]] | None] = []
        self._children: list[set[int]] = []
        self._free_ids: list[int] = []
        self._by_block: dict[int, set[int]] = {}
        self._order: dict[int, None] = {}  # live entries, oldest recorded first

    @property
    def num_entries(self) -> int:
        return len(self._order)

    # -- lookup ------------------------------------------------------------------------------------

    def find_longest_prefix(self, token_ids: _Seq[int]) -> tuple[list[int], int]:
        """Return ``(block_ids, num_matched_tokens)`` of the longest recorded whole-block prefix."""
        bs = self.block_size
        chain: list[int] = []
        parent = -1
        for start in range(0, len(token_ids) - bs + 1, bs):
            e = self._index.get((parent, tuple(token_ids[start:start + bs])))
            if e is None:
                break
            chain.append(self._block[e])
            parent = e
        return chain, len(chain) * bs

    # -- recording ---------------------------------------------------------------------------------

    def _new_entry(self, key: tuple[int, tuple[int, ...]], parent: int, block: int) -> int:
        if self._free_ids:
            e = self._free_ids.pop()
            self._block[e], self._parent[e], self._key[e] = block, parent, key
            self._children[e] = set()
        else:
            e = len(self._block)
            self._block.append(block)
            self._parent.append(parent)
            self._key.append(key)
            self._children.append(set())
        self._index[key] = e
        if parent >= 0:
            self._children[parent].add(e)
        self._by_block.setdefault(block, set()).add(e)
        self._order[e] = None
        return e

    def add(self, token_ids: _Seq[int], block_ids: _Seq[int]) -> None:
        """Record every whole-block boundary of ``token_ids`` whose K/V sits in ``block_ids``
        (block ``k`` holds tokens ``[k·bs, (k+1)·bs)``). Boundaries already recorded are kept."""
        bs = self.block_size
        parent = -1
        for k in range(min(len(token_ids) // bs, len(block_ids))):
            key = (parent, tuple(token_ids[k * bs:(k + 1) * bs]))
            e = self._index.get(key)
            if e is None:
                e = self._new_entry(key, parent, int(block_ids[k]))
            parent = e
        self._trim()

    # -- forgetting --------------------------------------------------------------------------------

    def _forget(self, root: int) -> None:
        """Remove entry ``root`` and all its descendants."""
        p = self._parent[root]
        if p >= 0:
            self._children[p].discard(root)
        todo = [root]
        while todo:
            e = todo.pop()
            todo.extend(self._children[e])
            del self._index[self._key[e]]
            holders = self._by_block[self._block[e]]
            holders.discard(e)
            if not holders:
                del self._by_block[self._block[e]]
            del self._order[e]
            self._key[e] = None
            self._children[e] = set()
            self._free_ids.append(e)

    def evict_block(self, block_id: int) -> None:
        """Forget every recorded prefix whose chain contains ``block_id``."""
        for e in list(self._by_block.get(block_id, ())):
            if self._key[e] is not None:  # not already forgotten under an earlier one
                self._forget(e)

    def _trim(self) -> None:
        if self.max_entries <= 0:
            return
        while len(self._order) > self.max_entries:
            victim = next(e for e in self._order if not self._children[e])
            self._forget(victim)
