"""Per-request token and block-table state: the layout fields of tileInfer's ``engine/sequence.py``.

Only what the paged KV path reads is kept (engine/sequence.py:17-91): token ids, the prefill
progress counters and the block table. Sampling options are carried as an opaque object; token
selection, constraints and stop strings are outside this package.
"""
from __future__ import annotations

from enum import Enum, auto
from itertools import count
from typing import Any, Sequence as _Seq


class SequenceStatus(Enum):
    WAITING = auto()
    RUNNING = auto()
    FINISHED = auto()


class Sequence:
    """A request's tokens and the physical KV blocks that hold them.

    ``block_size`` is a class attribute (16 by default, engine/sequence.py:18) that the runner
    overwrites from its configuration, as the reference does (engine/model_runner.py:53).
    """

    block_size: int = 16
    _ids = count()

    __slots__ = ("seq_id", "status", "token_ids", "last_token", "num_tokens", "num_prompt_tokens",
                 "num_cached_tokens", "num_scheduled_tokens", "is_prefill", "block_table",
                 "table_generation", "sampling_params")

    def __init__(self, token_ids: _Seq[int], sampling_params: Any = None):
        if len(token_ids) == 0:
            raise ValueError("Prompt must contain at least one token")
        self.seq_id = next(Sequence._ids)
        self.status = SequenceStatus.WAITING
        self.token_ids = list(token_ids)
        self.last_token = self.token_ids[-1]
        self.num_tokens = len(self.token_ids)
        self.num_prompt_tokens = self.num_tokens
        self.num_cached_tokens = 0       # tokens whose K/V already sit in the cache
        self.num_scheduled_tokens = 0    # tokens computed in the current step
        self.is_prefill = True
        self.block_table: list[int] = []
        # Bumped whenever block_table is replaced or changed other than by appending (free,
        # re-admission, swap), so a device-side copy of the table knows to re-send it whole.
        self.table_generation = 0
        self.sampling_params = sampling_params

    def __len__(self) -> int:
        return self.num_tokens

    def __getitem__(self, key):
        return self.token_ids[key]

    @property
    def is_finished(self) -> bool:
        return self.status == SequenceStatus.FINISHED

    @property
    def num_blocks(self) -> int:
        """Blocks needed to hold every token: ceil(num_tokens / block_size)."""
        return (self.num_tokens + self.block_size - 1) // self.block_size

    @property
    def last_block_num_tokens(self) -> int:
        return self.num_tokens - (self.num_blocks - 1) * self.block_size

    def block(self, i: int) -> list[int]:
        """Token ids held by logical block ``i``."""
        if not 0 <= i < self.num_blocks:
            raise IndexError(f"block {i} out of range [0, {self.num_blocks})")
        return self.token_ids[i * self.block_size:(i + 1) * self.block_size]

    def table_changed(self) -> None:
        """Announce that ``block_table`` was replaced or edited in place (not just appended to)."""
        self.table_generation += 1

    def append_token(self, token_id: int) -> None:
        self.token_ids.append(token_id)
        self.last_token = token_id
        self.num_tokens += 1
