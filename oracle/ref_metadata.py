"""Restatement of the reference runner's per-step decode metadata builder. TEST ONLY.

``ref_prepare_decode`` follows engine/model_runner.py:538-584 (``_prepare_decode_into_graph``)
step by step: for every sequence it writes the position, context length and slot of the newest
token into pinned host buffers and converts the sequence's whole block table to a tensor
(``torch.tensor(seq.block_table)``) into the pinned table buffer, -1 past its length; padding rows
get slot -1, context length 1 and an all -1 table; then every buffer is copied to the device
buffers. It is the checker of ``DeviceBlockTables`` and the timed host baseline of the bench
(the work the device-resident tables remove from every step).
"""
from __future__ import annotations

import torch


class RefDecodePrep:
    """Pinned host buffers and static device buffers sized like the runner's graph buffers."""

    def __init__(self, max_batch: int, max_blocks: int, device="cpu"):
        pin = torch.device(device).type == "cuda"
        self.pslots = torch.empty(max_batch, dtype=torch.int32, pin_memory=pin)
        self.pctx = torch.empty(max_batch, dtype=torch.int32, pin_memory=pin)
        self.ppos = torch.empty(max_batch, dtype=torch.int64, pin_memory=pin)
        self.pbt = torch.empty(max_batch, max_blocks, dtype=torch.int32, pin_memory=pin)
        self.slots = torch.empty(max_batch, dtype=torch.int32, device=device)
        self.ctx = torch.empty(max_batch, dtype=torch.int32, device=device)
        self.bt = torch.empty(max_batch, max_blocks, dtype=torch.int32, device=device)

    def __call__(self, seqs, block_size: int, bsz: int | None = None):
        """(slot_mapping [bsz], block_tables [bsz, max_blocks], context_lens [bsz])."""
        n = len(seqs)
        bsz = n if bsz is None else bsz
        for i, seq in enumerate(seqs):
            pos = seq.num_tokens - 1
            self.ppos[i] = pos
            self.pctx[i] = seq.num_tokens
            self.pslots[i] = seq.block_table[pos // block_size] * block_size + pos % block_size
            bt_len = len(seq.block_table)
            self.pbt[i, :bt_len] = torch.tensor(seq.block_table, dtype=torch.int32)
            self.pbt[i, bt_len:].fill_(-1)
        if n < bsz:
            self.pbt[n:bsz].fill_(-1)
        self.slots[:n].copy_(self.pslots[:n], non_blocking=True)
        self.ctx[:n].copy_(self.pctx[:n], non_blocking=True)
        self.bt[:bsz].copy_(self.pbt[:bsz], non_blocking=True)
        if n < bsz:
            self.slots[n:bsz].fill_(-1)
            self.ctx[n:bsz].fill_(1)
            self.bt[n:bsz].fill_(-1)
        return self.slots[:bsz], self.bt[:bsz], self.ctx[:bsz]
