"""DeviceBlockTables' host side on the CPU: what a step packs and sends, checked by running the
packed words through a numpy model of ``ti_paged_metadata`` (its contract: apply the appended ids
to the persistent rows, then emit slots, context lengths and -1-padded tables, padding rows
slot -1 / context 1 / table -1) and comparing with the host builders of engine/kv_layout.py.

The GPU suite checks the kernel itself against the same builders (tests/test_gpu_metadata.py);
this file pins the host logic -- incremental uploads, table generations after free / re-admission
and swap, deferred commits -- without a device."""
import ctypes
import random

import numpy as np
import pytest
import torch

from tileinfer_amd.engine import DeviceBlockTables, PagedKVManager, Sequence
from tileinfer_amd.engine import device_tables as dtm
from tileinfer_amd.engine import kv_layout as kl

BS = 16


def _i32(addr: int, n: int) -> np.ndarray:
    """A numpy view of n int32 words at a host address (CPU tensors stand in for device ones)."""
    if n <= 0:
        return np.zeros(0, dtype=np.int32)
    return np.ctypeslib.as_array((ctypes.c_int32 * n).from_address(addr))


class _FakeLib:
    """ti_paged_metadata's contract in numpy, on the CPU tensors' memory."""

    calls = 0

    def ti_paged_metadata(self, tables, table_stride, num_rows, max_blocks, rows, ctx_new,
                          table_len, tok_off, upd_off, upd_col, upd_id, n, pad_to, slot_out,
                          ctx_out, bt_out, bt_stride, width, page_size, stream):
        _FakeLib.calls += 1
        tab = _i32(tables, num_rows * table_stride).reshape(num_rows, table_stride)
        rows_, ctx_, tlen_ = _i32(rows, n), _i32(ctx_new, n), _i32(table_len, n)
        toff, uoff = _i32(tok_off, n + 1), _i32(upd_off, n + 1)
        u = int(uoff[n]) if n else 0
        cols, ids = _i32(upd_col, u), _i32(upd_id, u)
        total = int(toff[n]) + (pad_to - n)
        slots = _i32(slot_out, total)
        ctx_o = _i32(ctx_out, pad_to)
        bt = _i32(bt_out, pad_to * bt_stride).reshape(pad_to, bt_stride)
        for i in range(n):
            r = int(rows_[i])
            for k in range(int(uoff[i]), int(uoff[i + 1])):
                tab[r, cols[k]] = ids[k]
            nblk = min(int(tlen_[i]), max_blocks)
            ctx_o[i] = max(int(ctx_[i]), 0)
            bt[i, :width] = -1
            bt[i, :min(nblk, width)] = tab[r, :min(nblk, width)]
            nt = int(toff[i + 1] - toff[i])
            for j in range(nt):
                p = int(ctx_o[i]) - nt + j
                blk = p // page_size if p >= 0 else -1
                ok = 0 <= blk < nblk and tab[r, blk] >= 0
                slots[toff[i] + j] = tab[r, blk] * page_size + p % page_size if ok else -1
        for i in range(n, pad_to):
            slots[int(toff[n]) + i - n] = -1
            ctx_o[i] = 1
            bt[i, :width] = -1
        return 0


class _FakeEvent:
    def record(self, stream=None):
        pass

    def synchronize(self):
        pass


class _FakeStream:
    cuda_stream = 0


@pytest.fixture
def cpu_tables(monkeypatch):
    from tileinfer_amd import _lib
    monkeypatch.setattr(_lib, "load", lambda: _FakeLib())
    monkeypatch.setattr(_lib, "check", lambda rc: None)
    monkeypatch.setattr(dtm.torch.cuda, "Event", _FakeEvent)
    monkeypatch.setattr(dtm.torch.cuda, "current_stream", lambda device=None: _FakeStream())
    Sequence.block_size = BS
    yield lambda **kw: DeviceBlockTables(block_size=BS, device="cpu", **kw)


def check_decode(dt, seqs, pad_to=None, width=None):
    slots, tables, ctx = dt.step(seqs, pad_to=pad_to, width=width)
    hs, ht, hc = kl.decode_metadata(seqs, BS, device="cpu", pad_to=pad_to, width=width)
    assert torch.equal(slots, hs), "slot_mapping"
    assert torch.equal(tables, ht), "block_tables"
    assert torch.equal(ctx, hc), "context_lens"


def test_serving_run_host_side(cpu_tables):
    rng = random.Random(1)
    m = PagedKVManager(3000, BS, num_host_blocks=400)
    dt = cpu_tables(max_seqs=24, max_blocks_per_seq=64, max_batch=24, max_tokens=2048)
    prefix = [rng.randrange(1000) for _ in range(64)]
    live, parked = [], []
    steps = 0
    for _ in range(200):
        if len(live) + len(parked) < 14 and rng.random() < 0.35:
            s = Sequence((prefix if rng.random() < 0.5 else [])
                         + [rng.randrange(1000) for _ in range(rng.randrange(1, 300))])
            if m.admit(s):
                s.num_scheduled_tokens = s.num_tokens - s.num_cached_tokens
                slots, tables, ctx = dt.prefill_step([s])
                assert np.array_equal(slots.numpy(), kl.slot_mapping_prefill([s], BS))
                assert np.array_equal(tables.numpy(), kl.block_tables([s]))
                m.finish_chunk(s, s.num_scheduled_tokens)
                s.is_prefill = False
                live.append(s)
        for s in list(live):
            s.append_token(rng.randrange(1000))
            if m.can_append(s):
                m.append_slot(s)
            else:
                m.free(s)
                dt.release(s)
                live.remove(s)
        if live:
            check_decode(dt, live, pad_to=rng.choice([None, min(24, len(live) + 2)]),
                         width=rng.choice([None, 64]))
            steps += 1
        r = rng.random()
        if live and r < 0.05:                    # recompute preemption: freed, row kept
            s = live.pop(rng.randrange(len(live)))
            m.free(s)
            s.num_cached_tokens = 0
            parked.append(s)
        elif live and r < 0.09:                  # swapped out, sits out some steps
            s = live.pop(rng.randrange(len(live)))
            m.swap_out(s)
            parked.append(s)
        if parked and rng.random() < 0.25:
            s = parked.pop(0)
            if s.block_table:                     # swapped: new ids at old positions
                ok = m.can_swap_in(s) and bool(m.swap_in(s) or True)
            else:                                 # preempted: admitted again from scratch
                ok = m.admit(s)
                if ok:
                    m.finish_chunk(s, s.num_tokens - s.num_cached_tokens)
            (live if ok else parked).append(s)
    assert steps > 120


def test_readmission_resends_whole_table(cpu_tables):
    m = PagedKVManager(64, BS, enable_prefix_caching=False)
    dt = cpu_tables(max_seqs=4, max_blocks_per_seq=16)
    a = Sequence(list(range(41)))
    assert m.admit(a) and a.block_table == [0, 1, 2]
    check_decode(dt, [a])
    m.free(a)
    b = Sequence(list(range(20)))
    assert m.admit(b) and b.block_table == [0, 1]
    assert m.admit(a) and a.block_table == [2, 3, 4]
    check_decode(dt, [a, b])
    assert dt.last_upload_words == 5 * 2 + 2 + 2 * 5   # both tables whole: 3 + 2 ids


def test_failed_step_sends_the_ids_again(cpu_tables):
    """A step that raises before its upload (here: width too small) must not mark the appended
    ids as sent."""
    m = PagedKVManager(64, BS)
    dt = cpu_tables(max_seqs=2, max_blocks_per_seq=4)
    a = Sequence(list(range(50)))
    assert m.admit(a)
    with pytest.raises(ValueError):
        dt.step([a], width=5)
    check_decode(dt, [a])
