"""Block-level prefix cache: the matching and eviction rules of tileInfer's ``engine/prefix_cache.py``.

A trie keyed by full ``block_size``-token chunks of the token prefix (engine/prefix_cache.py:1-20):
because the key is the whole prefix up to a block boundary, a block is only reused at the position
where its K/V (with its rotary positions) was computed. Every node reached by ``add`` records the
physical block chain up to that boundary; ``find_longest_prefix`` returns the deepest recorded
chain (always whole blocks); ``evict_block`` invalidates every boundary whose chain ends in a block
the pool just freed, and everything below it (engine/prefix_cache.py:102-118). An optional cap
drops entries in the reference's traversal order when exceeded (engine/prefix_cache.py:120-145);
the reference's scheduler runs with no cap.
"""
from __future__ import annotations

from typing import Sequence as _Seq


class _Node:
    __slots__ = ("children", "block_ids", "num_tokens")

    def __init__(self):
        self.children: dict[tuple[int, ...], _Node] = {}
        self.block_ids: list[int] | None = None  # block chain up to this boundary, None = invalid
        self.num_tokens = 0


class PrefixCache:
    """Maps token prefixes (whole blocks) to the physical blocks that hold their K/V."""

    def __init__(self, block_size: int, max_entries: int = 0):
        if block_size <= 0:
            raise ValueError("block_size must be positive")
        self.block_size = block_size
        self.max_entries = max_entries
        self._root = _Node()
        self._num_entries = 0
        self._block_to_nodes: dict[int, list[_Node]] = {}  # last block of a chain -> its nodes

    @property
    def num_entries(self) -> int:
        return self._num_entries

    def find_longest_prefix(self, token_ids: _Seq[int]) -> tuple[list[int], int]:
        """Return ``(block_ids, num_matched_tokens)`` of the deepest valid whole-block match."""
        bs = self.block_size
        node, pos = self._root, 0
        matched: list[int] = []
        matched_tokens = 0
        while pos + bs <= len(token_ids):
            child = node.children.get(tuple(token_ids[pos:pos + bs]))
            if child is None:
                break
            node = child
            pos += bs
            if node.block_ids is not None:
                matched = list(node.block_ids)
                matched_tokens = pos
        return matched, matched_tokens

    def add(self, token_ids: _Seq[int], block_ids: _Seq[int]) -> None:
        """Record every whole-block boundary of ``token_ids`` held by ``block_ids`` (idempotent)."""
        bs = self.block_size
        n = min(len(token_ids) // bs, len(block_ids))
        node = self._root
        for k in range(1, n + 1):
            key = tuple(token_ids[(k - 1) * bs:k * bs])
            child = node.children.get(key)
            if child is None:
                child = node.children[key] = _Node()
            node = child
            if node.block_ids is None:
                self._block_to_nodes.setdefault(block_ids[k - 1], []).append(node)
                self._num_entries += 1
            node.block_ids = list(block_ids[:k])
            node.num_tokens = k * bs
        self._maybe_trim()

    def evict_block(self, block_id: int) -> None:
        """Invalidate every recorded prefix whose chain ends in ``block_id`` (and its subtree)."""
        for node in self._block_to_nodes.pop(block_id, []):
            self._invalidate_subtree(node)

    def _invalidate_subtree(self, node: _Node) -> None:
        stack = [node]
        while stack:
            cur = stack.pop()
            if cur.block_ids is not None:
                cur.block_ids = None
                cur.num_tokens = 0
                self._num_entries -= 1
            stack.extend(cur.children.values())

    def _maybe_trim(self) -> None:
        if self.max_entries <= 0 or self._num_entries <= self.max_entries:
            return
        # Same victim order as the reference: a stack walk from the root collecting valid nodes.
        live: list[_Node] = []
        stack = [self._root]
        while stack:
            cur = stack.pop()
            for child in cur.children.values():
                if child.block_ids is not None:
                    live.append(child)
                stack.append(child)
        for node in live[:self._num_entries - self.max_entries]:
            if node.block_ids is not None:
                node.block_ids = None
                node.num_tokens = 0
                self._num_entries -= 1

    def clear(self) -> None:
        self._root = _Node()
        self._block_to_nodes = {}
        self._num_entries = 0
