"""Device-resident block tables: the runner's per-step metadata without rebuilding it on the host.

tileInfer's model runner rebuilds, every step, each sequence's whole block table as a Python
list, converts it to a tensor and uploads all of it, plus the slot mapping and context lengths
(engine/model_runner.py:538-584 for captured decode graphs, 586-593 and 595-637 otherwise). At
config 3 that is 131,072 table entries per step, host work that grows with the context.

``DeviceBlockTables`` keeps one persistent device row per live sequence. A step uploads only what
changed -- each entry's row, new context length, new-token count and the block ids appended to
its table since the previous step (for a decode step usually none, one every 16 tokens) -- in one
pinned host-to-device copy, and one kernel (``ti_paged_metadata``) updates the rows and produces
``slot_mapping``, ``context_lens`` and the -1-padded ``block_tables`` of the batch, with the
reference's graph-padding rows (slot -1, context length 1, block -1; engine/model_runner.py:
524-527). The outputs are views of static device buffers, so a captured decode graph can read
them in place.

A table changed other than by appending (swap-in assigns new ids to old positions) must be
announced with ``invalidate(seq)``; ``release(seq)`` frees the row of a finished sequence.
"""
from __future__ import annotations

import numpy as np
import torch

from .sequence import Sequence


class DeviceBlockTables:
    def __init__(self, max_seqs: int, max_blocks_per_seq: int, block_size: int,
                 device: torch.device | str = "cuda", max_batch: int | None = None,
                 max_tokens: int | None = None):
        if max_seqs <= 0 or max_blocks_per_seq <= 0 or block_size <= 0:
            raise ValueError("max_seqs, max_blocks_per_seq and block_size must be positive")
        self.device = torch.device(device)
        self.block_size = block_size
        self.max_blocks = max_blocks_per_seq
        self.max_batch = max_batch or max_seqs
        self.max_tokens = max_tokens or self.max_batch
        self.tables = torch.full((max_seqs, max_blocks_per_seq), -1, dtype=torch.int32,
                                 device=self.device)
        self._free_rows = list(range(max_seqs - 1, -1, -1))
        self._row: dict[int, int] = {}    # seq_id -> persistent row
        self._sent: dict[int, int] = {}   # seq_id -> table entries already on the device
        # Static outputs (a captured graph reads these in place).
        self.slot_mapping = torch.full((self.max_tokens + self.max_batch,), -1, dtype=torch.int32,
                                       device=self.device)
        self.context_lens = torch.ones(self.max_batch, dtype=torch.int32, device=self.device)
        self.block_tables = torch.full((self.max_batch, max_blocks_per_seq), -1,
                                       dtype=torch.int32, device=self.device)
        # Packed per-step input: host staging (pinned, two alternating buffers) and device copy.
        self._cap = 0
        self._host: list[torch.Tensor] = []
        self._events: list[torch.cuda.Event | None] = []
        self._dev: torch.Tensor | None = None
        self._flip = 0
        self.last_upload_words = 0  # int32 words the last step sent to the device

    # -- rows --------------------------------------------------------------------------------------

    def row_of(self, seq: Sequence) -> int:
        return self._row[seq.seq_id]

    def release(self, seq: Sequence) -> None:
        """Free the sequence's row (its device contents are overwritten by the next owner)."""
        row = self._row.pop(seq.seq_id, None)
        self._sent.pop(seq.seq_id, None)
        if row is not None:
            self._free_rows.append(row)

    def invalidate(self, seq: Sequence) -> None:
        """Re-upload the sequence's whole table at the next step (after an in-place change)."""
        if seq.seq_id in self._sent:
            self._sent[seq.seq_id] = 0

    def _ensure_row(self, seq: Sequence) -> int:
        row = self._row.get(seq.seq_id)
        if row is None:
            if not self._free_rows:
                raise RuntimeError("DeviceBlockTables: no free row (raise max_seqs)")
            row = self._free_rows.pop()
            self._row[seq.seq_id] = row
            self._sent[seq.seq_id] = 0
        return row

    # -- one step ----------------------------------------------------------------------------------

    def _staging(self, words: int) -> tuple[torch.Tensor, torch.Tensor]:
        if words > self._cap:
            self._cap = max(words, 2 * self._cap, 1024)
            pin = self.device.type == "cuda"
            self._host = [torch.empty(self._cap, dtype=torch.int32, pin_memory=pin)
                          for _ in range(2)]
            self._events = [None, None]
            self._dev = torch.empty(self._cap, dtype=torch.int32, device=self.device)
        self._flip ^= 1
        ev = self._events[self._flip]
        if ev is not None:
            ev.synchronize()  # the copy that last read this staging buffer has finished
        return self._host[self._flip], self._dev

    def step(self, seqs: list[Sequence], new_tokens: list[int] | None = None,
             pad_to: int | None = None, width: int | None = None):
        """(slot_mapping, block_tables, context_lens) of one step, computed on the device.

        Decode: sequence i adds ``new_tokens[i]`` tokens (default 1, the newest token) ending at
        position ``num_tokens - 1``, and its context length is ``num_tokens``
        (engine/model_runner.py:628-637, 699). For a prefill chunk use ``prefill_step``.
        ``pad_to`` pads the batch like a captured decode graph; ``width`` is the block-table width
        (default: the longest table of the batch, as the runner's ``_build_block_tables``).
        """
        ctx = [s.num_tokens for s in seqs]
        return self._run(seqs, ctx, new_tokens if new_tokens is not None else [1] * len(seqs),
                         pad_to, width)

    def prefill_step(self, seqs: list[Sequence], pad_to: int | None = None,
                     width: int | None = None):
        """Metadata of a prefill chunk per sequence: tokens ``[num_cached_tokens,
        num_cached_tokens + num_scheduled_tokens)`` (engine/model_runner.py:595-626)."""
        ctx = [s.num_cached_tokens + s.num_scheduled_tokens for s in seqs]
        return self._run(seqs, ctx, [s.num_scheduled_tokens for s in seqs], pad_to, width)

    def _run(self, seqs, ctx, ntok, pad_to, width):
        from .. import _lib  # the library is needed only when a step runs

        n = len(seqs)
        pad = n if pad_to is None else int(pad_to)
        if pad < n or pad > self.max_batch:
            raise ValueError(f"pad_to {pad_to} outside [{n}, {self.max_batch}]")
        if len(ntok) != n:
            raise ValueError("new_tokens must have one entry per sequence")
        bs = self.block_size
        rows = np.empty(n, dtype=np.int32)
        upd_cols: list[int] = []
        upd_ids: list[int] = []
        upd_off = np.zeros(n + 1, dtype=np.int32)
        tlen = np.empty(n, dtype=np.int32)
        need_w = 0
        for i, s in enumerate(seqs):
            rows[i] = self._ensure_row(s)
            table = s.block_table
            sent = self._sent[s.seq_id]
            if len(table) > self.max_blocks:
                raise ValueError(f"sequence {s.seq_id}: {len(table)} blocks > {self.max_blocks}")
            if len(table) > sent:
                upd_cols.extend(range(sent, len(table)))
                upd_ids.extend(table[sent:])
                self._sent[s.seq_id] = len(table)
            upd_off[i + 1] = len(upd_cols)
            tlen[i] = len(table)
            need_w = max(need_w, len(table))
        tok_off = np.zeros(n + 1, dtype=np.int32)
        if n:
            tok_off[1:] = np.cumsum(np.asarray(ntok, dtype=np.int64))
        total_tok = int(tok_off[-1])
        if total_tok + (pad - n) > self.slot_mapping.numel():
            raise ValueError(f"{total_tok} tokens exceed max_tokens={self.max_tokens}")
        w = need_w if width is None else int(width)
        if w > self.max_blocks or w < 0:
            raise ValueError(f"width {w} outside [0, {self.max_blocks}]")
        u = len(upd_cols)
        # Packed words: rows | ctx | table_len | tok_off | upd_off | upd_col | upd_id.
        o_ctx, o_len, o_tok = n, 2 * n, 3 * n
        o_upd = 4 * n + 1
        o_col = 5 * n + 2
        o_id = o_col + u
        words = o_id + u
        self.last_upload_words = words
        host, dev = self._staging(words)
        h = host.numpy()
        h[0:n] = rows
        h[o_ctx:o_len] = ctx
        h[o_len:o_tok] = tlen
        h[o_tok:o_upd] = tok_off
        h[o_upd:o_col] = upd_off
        if u:
            h[o_col:o_id] = upd_cols
            h[o_id:words] = upd_ids
        stream = torch.cuda.current_stream(self.device)
        dev[:words].copy_(host[:words], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(stream)
        self._events[self._flip] = ev
        base = dev.data_ptr()
        at = lambda k: base + 4 * k  # noqa: E731
        lib = _lib.load()
        _lib.check(lib.ti_paged_metadata(
            self.tables.data_ptr(), self.tables.stride(0), self.tables.shape[0], self.max_blocks,
            at(0), at(o_ctx), at(o_len), at(o_tok), at(o_upd), at(o_col), at(o_id),
            n, pad, self.slot_mapping.data_ptr(), self.context_lens.data_ptr(),
            self.block_tables.data_ptr(), self.block_tables.stride(0), w, bs,
            stream.cuda_stream))
        return (self.slot_mapping[:total_tok + pad - n], self.block_tables[:pad, :w],
                self.context_lens[:pad])
