"""DeviceBlockTables (ti_paged_metadata) against the host builders over a simulated serving run:
admissions with prefix hits, prefill chunks, decode steps that cross block boundaries, finished
sequences whose rows are reused, swap-out / swap-in and re-admission (new table generations),
graph padding."""
import random

import numpy as np
import pytest
import torch

from helpers import say
from oracle.ref_metadata import RefDecodePrep
from tileinfer_amd.engine import DeviceBlockTables, PagedKVManager, Sequence
from tileinfer_amd.engine import kv_layout as kl

pytestmark = pytest.mark.gpu
BS = 16


def check_decode(dt, seqs, pad_to=None, width=None):
    slots, tables, ctx = dt.step(seqs, pad_to=pad_to, width=width)
    hs, ht, hc = kl.decode_metadata(seqs, BS, device="cpu", pad_to=pad_to, width=width)
    assert torch.equal(slots.cpu(), hs), "slot_mapping"
    assert torch.equal(tables.cpu(), ht), "block_tables"
    assert torch.equal(ctx.cpu(), hc), "context_lens"


def test_serving_run_matches_host_builders(dev):
    say("device metadata: simulated serving run")
    rng = random.Random(0)
    m = PagedKVManager(3000, BS, num_host_blocks=400)
    dt = DeviceBlockTables(max_seqs=24, max_blocks_per_seq=64, block_size=BS, device=dev,
                           max_batch=24, max_tokens=2048)
    prefix = [rng.randrange(1000) for _ in range(64)]
    live: list[Sequence] = []
    parked: list[Sequence] = []
    steps = 0
    for step in range(250):
        if len(live) + len(parked) < 14 and rng.random() < 0.35:
            tail = [rng.randrange(1000) for _ in range(rng.randrange(1, 300))]
            s = Sequence((prefix if rng.random() < 0.5 else []) + tail)
            if m.admit(s):
                s.num_scheduled_tokens = s.num_tokens - s.num_cached_tokens
                slots, tables, ctx = dt.prefill_step([s])
                assert np.array_equal(slots.cpu().numpy(), kl.slot_mapping_prefill([s], BS))
                assert np.array_equal(tables.cpu().numpy(), kl.block_tables([s]))
                assert int(ctx[0]) == s.num_tokens
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
            pad = rng.choice([None, min(24, len(live) + rng.randrange(4))])
            check_decode(dt, live, pad_to=pad, width=rng.choice([None, 64]))
            steps += 1
        if live and rng.random() < 0.05:
            s = live.pop(rng.randrange(len(live)))
            m.free(s)
            dt.release(s)
        if live and rng.random() < 0.04:        # swap a sequence out; it sits out some steps
            s = live.pop(rng.randrange(len(live)))
            m.swap_out(s)
            parked.append(s)
        if parked and rng.random() < 0.2:
            s = parked.pop(0)
            if m.can_swap_in(s):
                m.swap_in(s)                    # new ids at old positions: a new generation
                live.append(s)
            else:
                parked.append(s)
    assert steps > 150


def test_decode_uploads_only_changes(dev):
    """Steady decode uploads O(batch) words, not the tables."""
    say("device metadata: upload size")
    m = PagedKVManager(5000, BS)
    dt = DeviceBlockTables(max_seqs=8, max_blocks_per_seq=512, block_size=BS, device=dev)
    seqs = [Sequence(list(range(4000))) for _ in range(8)]
    for s in seqs:
        assert m.admit(s)
        m.finish_chunk(s, s.num_tokens)
    check_decode(dt, seqs)
    first = dt.last_upload_words
    assert first > 8 * 250                       # the whole tables went up once
    for _ in range(20):
        for s in seqs:
            s.append_token(1)
            m.append_slot(s)
        check_decode(dt, seqs)
        assert dt.last_upload_words <= 5 * 8 + 2 + 2 * 8   # rows, ctx, lengths, offsets, <=1 id each


def test_reference_builder_restatement_agrees(dev):
    """The restated reference builder (the bench's host baseline) gives the same tensors."""
    say("device metadata: reference builder restatement")
    m = PagedKVManager(2000, BS)
    seqs = [Sequence(list(range(n))) for n in (1, 16, 17, 300, 1000)]
    for s in seqs:
        assert m.admit(s)
        m.finish_chunk(s, s.num_tokens)
        s.append_token(5)
        m.append_slot(s)
    ref = RefDecodePrep(8, 80, device=dev)
    rs, rt, rc = ref(seqs, BS, bsz=8)
    dt = DeviceBlockTables(max_seqs=8, max_blocks_per_seq=80, block_size=BS, device=dev)
    ds, dtb, dc = dt.step(seqs, pad_to=8, width=80)
    assert torch.equal(rs.cpu(), ds.cpu())
    assert torch.equal(rt.cpu(), dtb.cpu())
    assert torch.equal(rc.cpu(), dc.cpu())


def test_metadata_feeds_the_kernels(dev):
    """Append + decode driven entirely by device metadata equals the host-metadata run."""
    say("device metadata: append + decode")
    from tileinfer_amd.kernels import gqa_decode_paged_fn, store_kvcache
    m = PagedKVManager(400, BS)
    seqs = [Sequence(list(range(n))) for n in (50, 700, 1300)]
    for s in seqs:
        assert m.admit(s)
        m.finish_chunk(s, s.num_tokens)
        s.append_token(1)
        m.append_slot(s)
    g = torch.Generator(device=dev).manual_seed(3)
    kc = torch.randn(400, BS, 4, 256, generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn(400, BS, 4, 256, generator=g, device=dev).to(torch.bfloat16)
    q = torch.randn(3, 24, 256, generator=g, device=dev).to(torch.bfloat16)
    kn = torch.randn(3, 4, 256, generator=g, device=dev).to(torch.bfloat16)
    dt = DeviceBlockTables(max_seqs=4, max_blocks_per_seq=100, block_size=BS, device=dev)
    outs = []
    for meta in (dt.step(seqs), kl.decode_metadata(seqs, BS, device=dev)):
        slots, tables, ctx = meta
        k2, v2 = kc.clone(), vc.clone()
        store_kvcache(kn, kn, k2.view(-1, 1024), v2.view(-1, 1024), slots)
        outs.append(gqa_decode_paged_fn(q, k2, v2, tables, ctx))
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


def test_readmitted_sequence_resends_its_table(dev):
    """Recompute preemption: a sequence is freed (its row kept: no ``release``), its blocks go to
    another sequence, and it is admitted again into other blocks. The next step must send the new
    table whole, not only the entries past the old count."""
    say("device metadata: free and re-admit without release")
    m = PagedKVManager(64, BS, enable_prefix_caching=False)
    dt = DeviceBlockTables(max_seqs=4, max_blocks_per_seq=16, block_size=BS, device=dev)
    a = Sequence(list(range(40)))                 # blocks 0, 1, 2
    assert m.admit(a)
    m.finish_chunk(a, a.num_tokens)
    a.is_prefill = False
    a.append_token(1)
    m.append_slot(a)
    check_decode(dt, [a])
    m.free(a)                                     # 2, 1, 0 back on the free stack
    b = Sequence(list(range(100, 120)))          # takes 0, 1
    assert m.admit(b)
    a.num_cached_tokens = 0
    assert m.admit(a) and a.block_table == [2, 3, 4]
    m.finish_chunk(a, a.num_tokens)
    a.append_token(2)
    m.append_slot(a)                              # 42 tokens: 3 blocks, as before the free
    check_decode(dt, [a, b])
    assert dt.block_tables[0, :3].tolist() == [2, 3, 4]
