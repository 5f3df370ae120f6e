"""Block copies (ti_copy_blocks): device<->device and device<->pinned-host, bit-exact, and an
end-to-end swap of a shared-prefix batch through PagedKVManager."""
import ctypes

import pytest
import torch

from helpers import bits, say
from tileinfer_amd import _lib
from tileinfer_amd.engine import PagedKVManager, Sequence
from tileinfer_amd.engine.kv_layout import allocate_kv_cache, layer_views
from tileinfer_amd.kernels.block_copy import copy_blocks, swap_blocks
from tileinfer_amd.kernels.gqa_decode_paged import gqa_decode_paged_fn
from tileinfer_amd.kernels.kvcache_store import store_kvcache

pytestmark = pytest.mark.gpu


def _slab(layers, nb, dev, seed, pinned=False):
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(2, layers, nb, 16, 4, 256, generator=g).to(torch.bfloat16)
    if dev == "host":
        return t.pin_memory() if pinned else t
    return t.to(dev)


def test_copy_blocks_device_to_device(dev):
    say("copy_blocks d2d")
    src = _slab(3, 40, dev, 1)
    dst = _slab(3, 25, dev, 2)
    before = dst.clone()
    pairs = torch.tensor([[5, 0], [39, 24], [0, 7], [17, 3]], dtype=torch.int64)
    copy_blocks(src, dst, pairs)
    torch.cuda.synchronize()
    for s, d in pairs.tolist():
        assert torch.equal(bits(dst[:, :, d]), bits(src[:, :, s]))
    keep = [i for i in range(25) if i not in pairs[:, 1].tolist()]
    assert torch.equal(bits(dst[:, :, keep]), bits(before[:, :, keep]))


def test_swap_roundtrip_through_pinned_host(dev):
    say("swap d2h + h2d")
    dev_cache = _slab(2, 30, dev, 3)
    host = torch.zeros(2, 2, 8, 16, 4, 256, dtype=torch.bfloat16).pin_memory()
    out_pairs = torch.tensor([[i * 3, i] for i in range(8)], dtype=torch.int64)
    swap_blocks(dev_cache, host, out_pairs)
    torch.cuda.synchronize()
    for s, d in out_pairs.tolist():
        assert torch.equal(bits(host[:, :, d]), bits(dev_cache[:, :, s].cpu()))
    back = torch.empty_like(dev_cache).fill_(0)
    swap_blocks(host, back, out_pairs[:, [1, 0]].contiguous().to(dev))
    torch.cuda.synchronize()
    for s, _ in out_pairs.tolist():
        assert torch.equal(bits(back[:, :, s]), bits(dev_cache[:, :, s]))


def test_copy_blocks_skips_invalid_ids_and_rejects_unpinned(dev):
    say("copy_blocks invalid ids / unpinned host")
    src = _slab(1, 6, dev, 4)
    dst = torch.zeros_like(src)
    copy_blocks(src, dst, torch.tensor([[2, 1], [9, 0], [-1, 2], [3, 99]], dtype=torch.int64))
    torch.cuda.synchronize()
    assert torch.equal(bits(dst[:, :, 1]), bits(src[:, :, 2]))
    assert not bool(dst[:, :, [0, 2, 3, 4, 5]].view(torch.int16).any())
    with pytest.raises(ValueError, match="not pinned"):
        copy_blocks(src, torch.zeros(2, 1, 6, 16, 4, 256, dtype=torch.bfloat16),
                    torch.tensor([[0, 0]]))
    # The library itself refuses a pointer the device cannot reach, before any launch.
    plain = torch.zeros(1024, dtype=torch.uint8)
    pairs = torch.tensor([[0, 0]], dtype=torch.int64, device=dev)
    lib = _lib.load()
    rc = lib.ti_copy_blocks(src.data_ptr(), plain.data_ptr(), pairs.data_ptr(), 1, 1, 512, 512,
                            512, 1, 1, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == _lib.TI_EINVAL and b"pinned" in lib.ti_last_error()


def test_swap_out_in_keeps_decode_bitwise(dev):
    """Shared-prefix batch (config 5 layout, small): swap 2 of 8 sequences out, let another
    sequence take and overwrite the freed blocks, swap back in: decode is bitwise unchanged."""
    say("end-to-end swap with shared prefix")
    bs, layers = 16, 2
    m = PagedKVManager(200, bs, num_host_blocks=40)
    kv = allocate_kv_cache(layers, 200, bs, 4, 256, dev)
    host = torch.zeros(2, layers, 40, bs, 4, 256, dtype=torch.bfloat16).pin_memory()
    gen = torch.Generator(device=dev).manual_seed(7)
    prefix = list(range(64))                     # 4 shared blocks
    seqs = []
    first = Sequence(prefix + [1000] * 30)
    m.admit(first)
    m.finish_chunk(first, 64)                    # the prefix is recorded at a block boundary
    m.finish_chunk(first, 30)
    seqs.append(first)
    for i in range(7):
        s = Sequence(prefix + [2000 + i] * (20 + 3 * i))
        m.admit(s)
        m.finish_chunk(s, s.num_tokens - s.num_cached_tokens)
        seqs.append(s)
    # Fill every allocated block's K/V with random values (stands in for the prefill).
    kv.normal_(generator=gen)
    width = max(len(s.block_table) for s in seqs)
    def decode():
        tbl = torch.full((8, width), -1, dtype=torch.int32)
        for i, s in enumerate(seqs):
            tbl[i, :len(s.block_table)] = torch.tensor(s.block_table, dtype=torch.int32)
        seq = torch.tensor([s.num_tokens for s in seqs], dtype=torch.int32)
        q = torch.randn(8, 24, 256, generator=torch.Generator(device=dev).manual_seed(1), device=dev).to(torch.bfloat16)
        outs = []
        for l in range(layers):
            _, _, kp, vp = layer_views(kv, l)
            outs.append(gqa_decode_paged_fn(q, kp, vp, tbl.to(dev), seq.to(dev), kv_reuse=True))
        return torch.stack(outs)
    ref = decode()
    assert m.shares_blocks(seqs) and seqs[3].block_table[:4] == first.block_table[:4]
    pairs = m.swap_out(seqs[2]) + m.swap_out(seqs[5])
    assert pairs and all(m.block_manager.blocks[b].ref_count == 0 for b, _ in pairs)
    swap_blocks(kv, host, torch.tensor(pairs, dtype=torch.int64))
    # Another sequence reuses the freed blocks and overwrites them through the append.
    intruder = Sequence([7] * (16 * len(pairs)))
    m.admit(intruder)
    assert set(intruder.block_table) & {b for b, _ in pairs}
    rows = torch.tensor([b * bs + o for b in intruder.block_table for o in range(bs)],
                        dtype=torch.int32, device=dev)
    junk = torch.randn(rows.numel(), 4, 256, generator=gen, device=dev).to(torch.bfloat16)
    for l in range(layers):
        kr, vr, _, _ = layer_views(kv, l)
        store_kvcache(junk, junk, kr, vr, rows)
    m.free(intruder)
    back = m.swap_in(seqs[2]) + m.swap_in(seqs[5])
    swap_blocks(host, kv, torch.tensor(back, dtype=torch.int64))
    torch.cuda.synchronize()
    assert torch.equal(bits(decode()), bits(ref))


def test_config5_swap_full_size(dev):
    """Config 5's swap at its stated size: 32 of the 128 sequences (a quarter) swap out their 32
    unique blocks each -- 1,024 blocks x 16 layers x K and V, 1 GiB -- through
    PagedKVManager.swap_out and one swap_blocks launch, the freed blocks are overwritten (another
    sequence's data), and the sequences swap back in through swap_in and one launch into the
    blocks the pool hands out. The round trip is bit-exact and every layer's decode of the whole
    batch (shared prefix included) is bitwise what it was before the swap."""
    from tileinfer_amd.workloads import config5_managed

    layers = 16
    say("config 5 swap, full size: 128 sequences, 16 layers, 1,024 blocks each way")
    mb = config5_managed(dev, layers=layers)
    m, kv = mb.manager, mb.kv
    assert kv.shape == (2, layers, 4608, 16, 4, 256)
    table, seqlen = mb.tables()

    def decode_all(tbl, sl):
        outs = []
        for l in range(layers):
            _, _, kp, vp = layer_views(kv, l)
            outs.append(gqa_decode_paged_fn(mb.q[l], kp, vp, tbl, sl, 16))
        return torch.stack(outs)

    ref = decode_all(table, seqlen)
    victims = mb.seqs[::4]
    pairs_out = [p for s in victims for p in m.swap_out(s)]
    assert len(pairs_out) == 1024 and len(victims) == 32
    assert all(s.block_table[:512] == mb.seqs[0].block_table[:512] for s in victims)
    old_ids = torch.tensor([b for b, _ in pairs_out], dtype=torch.int64, device=dev)
    before = kv[:, :, old_ids].clone()
    host = torch.empty((2, layers, 1024, 16, 4, 256), dtype=torch.bfloat16, pin_memory=True)
    swap_blocks(kv, host, torch.tensor(pairs_out, dtype=torch.int64))
    torch.cuda.synchronize()
    slots = torch.tensor([h for _, h in pairs_out], dtype=torch.int64)
    assert torch.equal(bits(host[:, :, slots]), bits(before.cpu()))
    # The freed blocks now belong to someone else: overwrite them.
    assert m.block_manager.num_free_blocks == 1024
    kv[:, :, old_ids] = torch.randn(before.shape, generator=torch.Generator(device=dev)
                                    .manual_seed(99), device=dev).to(torch.bfloat16)
    pairs_in = [p for s in victims for p in m.swap_in(s)]
    assert len(pairs_in) == 1024 and m.block_manager.num_free_blocks == 0
    swap_blocks(host, kv, torch.tensor(pairs_in, dtype=torch.int64))
    torch.cuda.synchronize()
    # Host slot h went out from device block b and came back into block n: bit-exact.
    out_of = {h: i for i, (_, h) in enumerate(pairs_out)}
    order = torch.tensor([out_of[h] for h, _ in pairs_in], dtype=torch.int64, device=dev)
    new_ids = torch.tensor([n for _, n in pairs_in], dtype=torch.int64, device=dev)
    assert torch.equal(bits(kv[:, :, new_ids]), bits(before[:, :, order]))
    table2, seqlen2 = mb.tables()
    assert not bool((table2 < 0).any())
    assert torch.equal(bits(decode_all(table2, seqlen2)), bits(ref))
