"""The decode plans for short context bounds: fixed 32-token partitions up to 1,024 tokens, and one
4-wave workgroup per (KV head, sequence) whose waves split the sequence's tiles and combine their
parts in LDS, up to 128 tokens and, when the pairs fill three quarters to all of one round, up to
512. Both are checked against the CPU oracle and against explicit fixed partitions of the same
data, with every wave count, empty sequences, head_dim 128, fp16, pages of 8 tokens, the gate
epilogue, the fused append and graph replays."""
import pytest
import torch

from helpers import assert_decode_close, bits, flat, say
from oracle.ref_torch import ref_gqa_decode_paged, ref_store_kvcache
from tileinfer_amd.kernels import fused_sigmoid_mul
from tileinfer_amd.kernels.gqa_decode_paged import decode_plan, gqa_decode_paged_fn
from tileinfer_amd.kernels.kvcache_store import store_kvcache
from tileinfer_amd.workloads import make_step

pytestmark = pytest.mark.gpu


def _pool(ctx, page=16):
    return sum((c + page - 1) // page for c in ctx) + 8


def _call(step, dev, **kw):
    return gqa_decode_paged_fn(step.q.to(dev), step.k_cache.to(dev), step.v_cache.to(dev),
                               step.block_table.to(dev), step.seqlen.to(dev), step.page_size, **kw)


def _ref(step):
    return ref_gqa_decode_paged(step.q, step.k_cache, step.v_cache, step.block_table, step.seqlen,
                                step.page_size)


@pytest.mark.parametrize("ctx", [
    [128],                        # the longest bound of the plan: 2 tiles per wave
    [17],                         # two tiles: waves 2 and 3 have none
    [0],                          # an empty sequence: zeros
    [1, 15, 16, 33],              # tiles per wave 0..1
    [100, 0, 127, 64],            # ragged, one empty
    [64] * 64,                    # 256 (sequence, KV head) pairs: one round
])
def test_wave_split_vs_oracle(ctx, dev):
    width = max(1, (max(ctx) + 15) // 16)
    step = make_step(ctx, pool=_pool(ctx), seed=41 + len(ctx), width=width)
    plan = decode_plan(len(ctx), 24, 4, 256, 16, step.block_table.shape[1])
    say(f"decode wave split ctx={ctx} plan={plan[:2]}")
    assert plan[:2] == (0, 0), "expected the one-workgroup-per-pair plan"
    out = _call(step, dev)
    assert_decode_close(out, _ref(step))
    fixed = _call(step, dev, split_tokens=32)
    assert_decode_close(out, fixed)
    for b, c in enumerate(ctx):
        if c == 0:
            assert bool((out[b] == 0).all())


def test_wave_split_head_dim_128_fp16_and_small_pages(dev):
    """8 KV heads at head_dim 128 (fp16), and pages of 8, 4, 2 and 1 tokens bitwise against
    page 16 on the same memory (the waves split 16-token tiles whatever the page size)."""
    ctx = [120, 33]
    step = make_step(ctx, pool=_pool(ctx), seed=47, dtype=torch.float16, hq=32, hkv=8, d=128)
    say(f"decode wave split d128 fp16 ctx={ctx}")
    assert decode_plan(2, 32, 8, 128, 16, step.block_table.shape[1])[:2] == (0, 0)
    out = _call(step, dev)
    assert_decode_close(out, _ref(step))
    ctx = [100, 60, 0, 77]
    step = make_step(ctx, pool=_pool(ctx), seed=48)
    base = _call(step, dev)
    t = step.block_table
    for page in (8, 4, 2, 1):
        say(f"decode wave split page {page} ctx={ctx}")
        r = 16 // page
        cols = torch.arange(t.shape[1] * r)
        tp = torch.where(t[:, cols // r] >= 0, t[:, cols // r] * r + cols % r, -1).to(torch.int32)
        kp, vp = step.k_cache.view(-1, page, 4, 256), step.v_cache.view(-1, page, 4, 256)
        assert decode_plan(4, 24, 4, 256, page, tp.shape[1])[:2] == (0, 0)
        outp = gqa_decode_paged_fn(step.q.to(dev), kp.to(dev), vp.to(dev), tp.to(dev),
                                   step.seqlen.to(dev), page)
        assert torch.equal(bits(base), bits(outp)), page


@pytest.mark.parametrize("ctx", [
    [512],                        # config 1's shape
    [1024],                       # the longest short bound
    [512, 1, 0, 300, 17, 999, 64, 128],
])
def test_short_fixed_partitions_vs_oracle(ctx, dev):
    """Bounds of 129 to 1,024 tokens take fixed 32-token partitions: bitwise the explicit split,
    and within tolerance of the oracle."""
    step = make_step(ctx, pool=_pool(ctx), seed=51)
    plan = decode_plan(len(ctx), 24, 4, 256, 16, step.block_table.shape[1])
    say(f"decode short fixed ctx={ctx} plan={plan[:2]}")
    assert plan[0] == 32
    out = _call(step, dev)
    assert torch.equal(bits(out), bits(_call(step, dev, split_tokens=32)))
    assert_decode_close(out, _ref(step))


@pytest.mark.parametrize("ctx", [[100], [60, 0, 17, 128], [512, 0, 300]])
def test_wave_split_gate_and_fused_append(ctx, dev):
    """The gate epilogue is bitwise decode-then-gate, and the fused append bitwise
    store-then-decode (the wave holding the last token writes its row before loading it), for
    the per-pair plan and the fixed short one."""
    step = make_step(ctx, pool=_pool(ctx), seed=53)
    say(f"decode wave split gate/append ctx={ctx}")
    g = torch.Generator().manual_seed(7)
    gate = (3 * torch.randn(len(ctx), 1, 24 * 256, generator=g)).to(torch.bfloat16).to(dev)
    plain = _call(step, dev)
    gated = _call(step, dev, gate=gate)
    assert torch.equal(bits(gated), bits(fused_sigmoid_mul(plain, gate.view(len(ctx), 24, 256))))
    q, kn, vn = step.q.to(dev), step.k_new.to(dev), step.v_new.to(dev)
    table, seqlen, slot = step.block_table.to(dev), step.seqlen.to(dev), step.slot_mapping.to(dev)
    kc1, vc1 = step.k_cache.to(dev), step.v_cache.to(dev)
    store_kvcache(kn, vn, flat(kc1), flat(vc1), slot)
    two = gqa_decode_paged_fn(q, kc1, vc1, table, seqlen)
    kc2, vc2 = step.k_cache.to(dev), step.v_cache.to(dev)
    one = gqa_decode_paged_fn(q, kc2, vc2, table, seqlen, append=(kn, vn, slot))
    torch.cuda.synchronize()
    assert torch.equal(bits(one), bits(two))
    assert torch.equal(bits(kc1), bits(kc2)) and torch.equal(bits(vc1), bits(vc2))
    k_ref, v_ref = step.k_cache.clone(), step.v_cache.clone()
    ref_store_kvcache(step.k_new, step.v_new, flat(k_ref), flat(v_ref), step.slot_mapping)
    ref = ref_gqa_decode_paged(step.q, k_ref, v_ref, step.block_table, step.seqlen, 16)
    assert_decode_close(one, ref)


def _ragged(b, lo, hi, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (b,), generator=g).tolist()


@pytest.mark.parametrize("ctx,hq,hkv,d,page,dtype", [
    ([512] * 64, 24, 4, 256, 16, torch.bfloat16),             # 256 pairs: one full round
    (_ragged(48, 0, 512, 61), 24, 4, 256, 16, torch.bfloat16),  # 192 pairs, ragged, empty rows
    ([512] + [16] * 63, 24, 4, 256, 16, torch.bfloat16),       # one long sequence among short
    (_ragged(32, 100, 400, 62), 32, 8, 128, 8, torch.float16),  # 256 pairs, head_dim 128, pages of 8
])
def test_pair_round_vs_oracle(ctx, hq, hkv, d, page, dtype, dev):
    """Bounds of 129 to 512 tokens take one workgroup per (KV head, sequence) when those pairs
    fill three quarters to all of one round: against the oracle and the explicit 32-token split."""
    width = (max(ctx) + page - 1) // page
    step = make_step(ctx, pool=_pool(ctx, page), seed=60 + len(ctx), width=width, hq=hq, hkv=hkv,
                     d=d, dtype=dtype, page=page)
    plan = decode_plan(len(ctx), hq, hkv, d, page, width)
    say(f"decode pair round B={len(ctx)} hkv={hkv} d={d} page={page} bound={width * page} "
        f"plan={plan[:2]}")
    assert plan[:2] == (0, 0), "expected the one-workgroup-per-pair plan"
    out = _call(step, dev)
    assert_decode_close(out, _ref(step))
    assert_decode_close(out, _call(step, dev, split_tokens=32))
    for b, c in enumerate(ctx):
        if c == 0:
            assert bool((out[b] == 0).all())


def test_pair_round_gate_and_fused_append(dev):
    """At a 512-token bound with 256 pairs: the gate epilogue bitwise decode-then-gate, the fused
    append bitwise store-then-decode."""
    ctx = _ragged(64, 1, 512, 63)
    step = make_step(ctx, pool=_pool(ctx), seed=64, width=32)
    assert decode_plan(64, 24, 4, 256, 16, 32)[:2] == (0, 0)
    say("decode pair round gate/append, B=64, bound 512")
    g = torch.Generator().manual_seed(9)
    gate = (3 * torch.randn(64, 1, 24 * 256, generator=g)).to(torch.bfloat16).to(dev)
    plain = _call(step, dev)
    gated = _call(step, dev, gate=gate)
    assert torch.equal(bits(gated), bits(fused_sigmoid_mul(plain, gate.view(64, 24, 256))))
    q, kn, vn = step.q.to(dev), step.k_new.to(dev), step.v_new.to(dev)
    table, seqlen, slot = step.block_table.to(dev), step.seqlen.to(dev), step.slot_mapping.to(dev)
    kc1, vc1 = step.k_cache.to(dev), step.v_cache.to(dev)
    store_kvcache(kn, vn, flat(kc1), flat(vc1), slot)
    two = gqa_decode_paged_fn(q, kc1, vc1, table, seqlen)
    kc2, vc2 = step.k_cache.to(dev), step.v_cache.to(dev)
    one = gqa_decode_paged_fn(q, kc2, vc2, table, seqlen, append=(kn, vn, slot))
    torch.cuda.synchronize()
    assert torch.equal(bits(one), bits(two))
    assert torch.equal(bits(kc1), bits(kc2)) and torch.equal(bits(vc1), bits(vc2))


def test_wave_split_graph_replays(dev):
    """A captured graph of the per-pair plan, replayed three times with new queries and eager
    work between the replays, equals the eager call every time."""
    ctx = [128, 90]
    step = make_step(ctx, pool=_pool(ctx), seed=57)
    say("decode wave split graph replays")
    q = step.q.to(dev)
    kc, vc = step.k_cache.to(dev), step.v_cache.to(dev)
    table, seqlen = step.block_table.to(dev), step.seqlen.to(dev)
    out = torch.empty_like(q)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        gqa_decode_paged_fn(q, kc, vc, table, seqlen, out=out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gqa_decode_paged_fn(q, kc, vc, table, seqlen, out=out)
    for i in range(3):
        q.copy_(torch.randn(q.shape, generator=torch.Generator().manual_seed(100 + i)).to(q.dtype))
        eager = gqa_decode_paged_fn(q, kc, vc, table, seqlen)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(bits(out), bits(eager))
