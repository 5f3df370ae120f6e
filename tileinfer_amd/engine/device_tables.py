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

A table replaced or changed other than by appending (freed and re-admitted, swapped out or in) is
re-sent whole: the block manager and ``PagedKVManager`` bump ``Sequence.table_generation`` when
they do that, and a step compares it with the generation it last sent. Code that edits a table
by hand calls ``seq.table_changed()`` (or ``invalidate(seq)``); ``release(seq)`` frees the row of
a finished sequence.
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
        # seq_id -> [persistent row, table entries already on the device, table generation they
        # belong to]; a new generation (the table was replaced or edited) re-sends the table.
        self._state: dict[int, list] = {}
        # Static outputs (a captured graph reads these in place).
        self.slot_mapping = torch.full((self.max_tokens + self.max_batch,), -1, dtype=torch.int32,
                                       device=self.device)
        self.context_lens = torch.ones(self.max_batch, dtype=torch.int32, device=self.device)
        self.block_tables = torch.full((self.max_batch, max_blocks_per_seq), -1,
                                       dtype=torch.int32, device=self.device)
        # Packed per-step input: host staging (pinned, two alternating buffers) and device copy.
        self._cap = 0
        self._host: list[torch.Tensor] = []
        self._host_np: list[np.ndarray] = []
        self._events: list[torch.cuda.Event] = []
        self._recorded: list[bool] = []
        self._dev: torch.Tensor | None = None
        self._flip = 0
        self.last_upload_words = 0  # int32 words the last step sent to the device

    # -- rows --------------------------------------------------------------------------------------

    def row_of(self, seq: Sequence) -> int:
        return self._state[seq.seq_id][0]

    def release(self, seq: Sequence) -> None:
        """Free the sequence's row (its device contents are overwritten by the next owner)."""
        st = self._state.pop(seq.seq_id, None)
        if st is not None:
            self._free_rows.append(st[0])

    def invalidate(self, seq: Sequence) -> None:
        """Re-upload the sequence's whole table at the next step (after an in-place change that
        did not go through ``Sequence.table_changed``)."""
        st = self._state.get(seq.seq_id)
        if st is not None:
            st[1] = 0

    def _new_row(self, seq: Sequence) -> list:
        if not self._free_rows:
            raise RuntimeError("DeviceBlockTables: no free row (raise max_seqs)")
        st = [self._free_rows.pop(), 0, seq.table_generation]
        self._state[seq.seq_id] = st
        return st

    # -- one step ----------------------------------------------------------------------------------

    def _staging(self, words: int) -> tuple[torch.Tensor, torch.Tensor]:
        if words > self._cap:
            self._cap = max(words, 2 * self._cap, 1024)
            pin = self.device.type == "cuda"
            self._host = [torch.empty(self._cap, dtype=torch.int32, pin_memory=pin)
                          for _ in range(2)]
            self._host_np = [h.numpy() for h in self._host]
            self._events = [torch.cuda.Event(), torch.cuda.Event()]
            self._recorded = [False, False]
            self._dev = torch.empty(self._cap, dtype=torch.int32, device=self.device)
        self._flip ^= 1
        if self._recorded[self._flip]:
            self._events[self._flip].synchronize()  # the copy that last read this buffer is done
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
        state = self._state
        rows: list[int] = []
        tlen: list[int] = []
        upd_off = [0]
        upd_cols: list[int] = []
        upd_ids: list[int] = []
        sent_now: list[tuple[list, int, int]] = []  # committed once the upload is enqueued
        for s in seqs:
            table = s.block_table
            k = len(table)
            st = state.get(s.seq_id)
            if st is None:
                st = self._new_row(s)
            gen = s.table_generation
            sent = st[1] if st[2] == gen else 0
            if k > sent:  # ids appended since the last step (all of them for a new generation)
                if k > self.max_blocks:
                    raise ValueError(f"sequence {s.seq_id}: {k} blocks > {self.max_blocks}")
                upd_cols.extend(range(sent, k))
                upd_ids.extend(table[sent:])
                sent_now.append((st, k, gen))
            elif k < sent:  # shrunk without a new generation: re-send what is left
                upd_cols.extend(range(k))
                upd_ids.extend(table)
                sent_now.append((st, k, gen))
            rows.append(st[0])
            tlen.append(k)
            upd_off.append(len(upd_cols))
        tok_off = [0]
        for t in ntok:
            tok_off.append(tok_off[-1] + int(t))
        total_tok = tok_off[-1]
        if total_tok + (pad - n) > self.slot_mapping.numel():
            raise ValueError(f"{total_tok} tokens exceed max_tokens={self.max_tokens}")
        w = max(tlen, default=0) if width is None else int(width)
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
        h = self._host_np[self._flip]
        h[:words] = np.fromiter(
            (x for part in (rows, ctx, tlen, tok_off, upd_off, upd_cols, upd_ids) for x in part),
            dtype=np.int32, count=words)
        stream = torch.cuda.current_stream(self.device)
        dev[:words].copy_(host[:words], non_blocking=True)
        self._events[self._flip].record(stream)
        self._recorded[self._flip] = True
        base = dev.data_ptr()
        _lib.check(_lib.load().ti_paged_metadata(
            self.tables.data_ptr(), self.tables.stride(0), self.tables.shape[0], self.max_blocks,
            base, base + 4 * o_ctx, base + 4 * o_len, base + 4 * o_tok, base + 4 * o_upd,
            base + 4 * o_col, base + 4 * o_id, n, pad, self.slot_mapping.data_ptr(),
            self.context_lens.data_ptr(), self.block_tables.data_ptr(),
            self.block_tables.stride(0), w, self.block_size, stream.cuda_stream))
        for st, k, gen in sent_now:
            st[1], st[2] = k, gen
        return (self.slot_mapping[:total_tok + pad - n], self.block_tables[:pad, :w],
                self.context_lens[:pad])
