"""Every BASELINE configuration at its stated size on the GPU, against the CPU oracle, plus the
runner's graph-padding rows.

* config 3: one layer at batch 64 x 32,768 through the default balanced plan and through the
  configured 2,048-token partitions; appended rows bit-exact, sampled sequences vs the oracle;
* config 4: the whole mixed step -- one 2,080-token append (chunk + 32 decode tokens) and the
  batch-32 decode -- every sequence against the oracle, the cache bit-exact;
* config 5: all 128 sequences, shared vs private prefix bitwise for the plain and the
  shared-prefix calls, sampled rows against the oracle;
* a decode step padded the way the runner pads a captured graph (engine/model_runner.py:449-452,
  524-527, 580-584): slot -1, context 1, an all -1 table; through DeviceBlockTables, the append
  and the decode as model/qwen_36.py:1016-1018, 1071-1079 call them.
"""
import pytest
import torch

from helpers import ATOL, RTOL, assert_decode_close, bits, flat, say
from oracle.ref_torch import ref_gqa_decode_paged, ref_store_kvcache
from tileinfer_amd.engine import DeviceBlockTables, PagedKVManager, Sequence
from tileinfer_amd.engine.kv_layout import allocate_kv_cache, layer_views
from tileinfer_amd.kernels.gqa_decode_paged import decode_plan, gqa_decode_paged_fn
from tileinfer_amd.kernels.kvcache_store import store_kvcache
from tileinfer_amd.workloads import BLOCK, HEAD_DIM, HKV, HQ, config4, config5

pytestmark = pytest.mark.gpu


def _oracle_rows(q, k_cache, v_cache, table, seqlen, rows):
    """Oracle decode of the listed rows only: their pages copied to the host, renumbered."""
    out = []
    for b in rows:
        n = (int(seqlen[b]) + BLOCK - 1) // BLOCK
        pages = table[b, :n].long()
        kc, vc = k_cache[pages].cpu(), v_cache[pages].cpu()
        local = torch.arange(n, dtype=torch.int32).view(1, -1)
        out.append(ref_gqa_decode_paged(q[b:b + 1].cpu(), kc, vc, local,
                                        seqlen[b:b + 1].cpu(), BLOCK))
    return torch.cat(out)


def test_config3_layer_full_size(dev):
    """Batch 64 x 32,768 tokens over a randomly permuted 131,072-block pool (one layer: 4 GiB
    of K and 4 GiB of V): default balanced plan (256 workgroups of 8,192 tokens) and the
    configured 2,048-token partitions, 4 sampled sequences against the oracle."""
    b, ctx = 64, 32768
    nb = b * ctx // BLOCK
    say(f"config3 layer: batch {b} x ctx {ctx}, {nb} blocks")
    gen = torch.Generator(device=dev).manual_seed(1003)
    kc = torch.empty((nb, BLOCK, HKV, HEAD_DIM), dtype=torch.bfloat16, device=dev)
    vc = torch.empty_like(kc)
    kc.normal_(generator=gen)
    vc.normal_(generator=gen)
    table = torch.randperm(nb, generator=gen, device=dev).to(torch.int32).view(b, ctx // BLOCK)
    seqlen = torch.full((b,), ctx, dtype=torch.int32, device=dev)
    q = torch.randn((b, HQ, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    kn = torch.randn((b, HKV, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    vn = torch.randn((b, HKV, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    pos = ctx - 1
    slots = (table[:, pos // BLOCK].long() * BLOCK + pos % BLOCK).to(torch.int32)
    store_kvcache(kn, vn, flat(kc), flat(vc), slots)
    s = slots.long()
    assert torch.equal(bits(flat(kc)[s]), bits(kn.reshape(b, -1)))
    assert torch.equal(bits(flat(vc)[s]), bits(vn.reshape(b, -1)))
    assert decode_plan(b, HQ, HKV, HEAD_DIM, BLOCK, ctx // BLOCK)[:2] == (0, 256)
    balanced = gqa_decode_paged_fn(q, kc, vc, table, seqlen, BLOCK)
    split = gqa_decode_paged_fn(q, kc, vc, table, seqlen, BLOCK, split_tokens=2048)
    rows = [0, 21, 42, 63]
    ref = _oracle_rows(q, kc, vc, table, seqlen, rows)
    assert_decode_close(balanced[rows], ref)
    assert_decode_close(split[rows], ref)
    assert_decode_close(balanced, split)


def test_config4_mixed_step_full(dev):
    """Config 4 as one step: the 2,048-token chunk and the 32 decode tokens appended in one call,
    then the batch-32 decode (ctx U[1024, 16384]); the whole cache equals the oracle's, every
    decode row within tolerance of the oracle."""
    st, chunk_slots = config4()
    say(f"config4 step: append {chunk_slots.numel() + st.slot_mapping.numel()} tokens, decode "
        f"batch {st.seqlen.numel()} ctx {min(st.meta['ctx'])}..{max(st.meta['ctx'])}")
    key = torch.cat([st.meta["chunk_k"], st.k_new])
    val = torch.cat([st.meta["chunk_v"], st.v_new])
    slots = torch.cat([chunk_slots, st.slot_mapping])
    kc, vc = st.k_cache.to(dev), st.v_cache.to(dev)
    store_kvcache(key.to(dev), val.to(dev), flat(kc), flat(vc), slots.to(dev))
    out = gqa_decode_paged_fn(st.q.to(dev), kc, vc, st.block_table.to(dev), st.seqlen.to(dev))
    k_ref, v_ref = st.k_cache.clone(), st.v_cache.clone()
    ref_store_kvcache(key, val, flat(k_ref), flat(v_ref), slots)
    assert torch.equal(bits(kc.cpu()), bits(k_ref))
    assert torch.equal(bits(vc.cpu()), bits(v_ref))
    ref = ref_gqa_decode_paged(st.q, k_ref, v_ref, st.block_table, st.seqlen, BLOCK)
    assert_decode_close(out, ref)


def test_config5_full_batch(dev):
    """All 128 sequences over the shared 8,192-token prefix: the shared and the private layout
    (every sequence its own copy of the prefix blocks) give bitwise the same output for the plain
    call (both cache policies) and for the shared-prefix call; sampled rows against the oracle."""
    say("config5: 128 sequences, shared vs private prefix")
    shared = config5(device=dev, shared=True)
    private = config5(device=dev, shared=False)
    for stp in (shared, private):
        store_kvcache(stp.k_new, stp.v_new, flat(stp.k_cache), flat(stp.v_cache),
                      stp.slot_mapping)

    def call(stp, **kw):
        return gqa_decode_paged_fn(stp.q, stp.k_cache, stp.v_cache, stp.block_table, stp.seqlen,
                                   BLOCK, **kw)

    plain = call(shared, kv_reuse=True)
    assert torch.equal(bits(plain), bits(call(private, kv_reuse=True)))
    for reuse in (None, False):  # chosen on the device (keep here), and forced streaming
        assert torch.equal(bits(plain), bits(call(shared, kv_reuse=reuse)))
        assert torch.equal(bits(plain), bits(call(private, kv_reuse=reuse)))
    pre = call(shared, shared_prefix_tokens=8192)
    assert torch.equal(bits(pre), bits(call(private, shared_prefix_tokens=8192)))
    rows = [0, 1, 63, 64, 127]
    ref = _oracle_rows(shared.q, shared.k_cache, shared.v_cache, shared.block_table,
                       shared.seqlen, rows)
    assert_decode_close(plain[rows], ref)
    assert_decode_close(pre[rows], ref)
    assert_decode_close(pre, plain)


@pytest.mark.parametrize("prefixed", [False, True])
def test_runner_padding_rows(prefixed, dev):
    """A decode batch of 5 sequences padded to a graph bucket of 8 with the runner's padding rows
    (slot -1, context 1, all -1 table) at the runner's full table width: padding rows append
    nothing and decode to zeros, real rows are unchanged. With shared_prefix_tokens (every real
    sequence shares a 1,024-token prefix through the prefix cache) the padding rows, shorter than
    the prefix, still come back as zeros."""
    say(f"runner padding rows, prefixed={prefixed}")
    Sequence.block_size = BLOCK
    max_blocks, bucket, layers = 200, 8, 2
    m = PagedKVManager(1200, BLOCK)
    prefix = list(range(1024)) if prefixed else []
    g = torch.Generator().manual_seed(77)
    seqs = []
    for i, n in enumerate([1500, 1100, 2000, 1030, 1900]):
        toks = prefix + [int(x) for x in torch.randint(2000, 3000, (n - len(prefix),),
                                                       generator=g)]
        s = Sequence(toks)
        assert m.admit(s)
        whole = s.num_tokens // BLOCK * BLOCK - s.num_cached_tokens
        m.finish_chunk(s, whole)                # whole blocks: recorded in the prefix cache
        m.finish_chunk(s, s.num_tokens - s.num_cached_tokens)
        s.is_prefill = False
        s.append_token(7)
        m.append_slot(s)
        seqs.append(s)
    p = m.common_prefix_tokens(seqs)
    assert p == (1024 if prefixed else 0)
    n = len(seqs)
    kv = allocate_kv_cache(layers, 1200, BLOCK, HKV, HEAD_DIM, dev, torch.bfloat16, zero=False)
    kv.normal_(generator=torch.Generator(device=dev).manual_seed(5))
    dt = DeviceBlockTables(max_seqs=16, max_blocks_per_seq=max_blocks, block_size=BLOCK,
                           device=dev, max_batch=bucket)
    slots, tables, ctx = dt.step(seqs, pad_to=bucket, width=max_blocks)
    assert slots[n:].tolist() == [-1] * (bucket - n) and ctx[n:].tolist() == [1] * (bucket - n)
    assert bool((tables[n:] == -1).all())
    gd = torch.Generator(device=dev).manual_seed(6)
    q = torch.randn((bucket, HQ, HEAD_DIM), generator=gd, device=dev).to(torch.bfloat16)
    kn = torch.randn((bucket, HKV, HEAD_DIM), generator=gd, device=dev).to(torch.bfloat16)
    vn = torch.randn((bucket, HKV, HEAD_DIM), generator=gd, device=dev).to(torch.bfloat16)
    k_rows, v_rows, k_paged, v_paged = layer_views(kv, 1)
    before = kv.clone()
    store_kvcache(kn, vn, k_rows, v_rows, slots)
    expect = before.clone()
    _, _, ek, ev = layer_views(expect, 1)
    live = slots[:n].long()
    flat(ek)[live] = kn[:n].reshape(n, -1)
    flat(ev)[live] = vn[:n].reshape(n, -1)
    assert torch.equal(bits(kv), bits(expect)), "a padding row wrote into the cache"
    kw = {"shared_prefix_tokens": p, "prefix_pass": "always", "kv_reuse": True} if prefixed else {}
    out = gqa_decode_paged_fn(q, k_paged, v_paged, tables, ctx, BLOCK, **kw)
    assert bool((out[n:] == 0).all()), "padding rows must decode to zeros"
    unpadded = gqa_decode_paged_fn(q[:n].contiguous(), k_paged, v_paged, tables[:n], ctx[:n],
                                   BLOCK, **kw)
    assert_decode_close(out[:n], unpadded, atol=ATOL / 4, rtol=RTOL / 4)
    ref = _oracle_rows(q, k_paged, v_paged, tables, ctx, range(n))
    assert_decode_close(out[:n], ref)
    if not prefixed:
        # With fixed partitions a row's result does not depend on the rest of the batch.
        fixed = gqa_decode_paged_fn(q, k_paged, v_paged, tables, ctx, BLOCK, split_tokens=512)
        fixed_unpadded = gqa_decode_paged_fn(q[:n].contiguous(), k_paged, v_paged, tables[:n],
                                             ctx[:n], BLOCK, split_tokens=512)
        assert bool((fixed[n:] == 0).all())
        assert torch.equal(bits(fixed[:n]), bits(fixed_unpadded))
