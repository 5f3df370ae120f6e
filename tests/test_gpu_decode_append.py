"""The decode step's append fused into the decode call (gqa_decode_paged_fn(..., append=),
ti_gqa_decode_paged_append): bitwise what store_kvcache followed by the decode gives — the output
and every row of both caches — under the balanced plan and fixed partitions, with the runner's
graph-padding rows, sequences no workgroup covers, fp16 and head_dim 128; the unfused pair itself
is checked against the oracle elsewhere (test_gpu_decode.py)."""
import pytest
import torch

from helpers import bits, flat, say
from tileinfer_amd.kernels.gqa_decode_paged import gqa_decode_paged_fn
from tileinfer_amd.kernels.kvcache_store import store_kvcache
from tileinfer_amd.workloads import config2, make_step

pytestmark = pytest.mark.gpu


def _both(step, dev, split_tokens=None, pad_rows=0, slots=None):
    """(out, k_cache, v_cache) of store_kvcache + decode and of the fused call on copies of the
    same step; pad_rows runner-style rows (slot -1, context 1, all -1 table) are appended."""
    q, kn, vn = step.q.to(dev), step.k_new.to(dev), step.v_new.to(dev)
    table, seqlen = step.block_table.to(dev), step.seqlen.to(dev)
    slot = (step.slot_mapping if slots is None else slots).to(dev)
    if pad_rows:
        q = torch.cat([q, torch.randn((pad_rows,) + q.shape[1:], device=dev).to(q.dtype)])
        kn = torch.cat([kn, torch.randn((pad_rows,) + kn.shape[1:], device=dev).to(kn.dtype)])
        vn = torch.cat([vn, torch.randn((pad_rows,) + vn.shape[1:], device=dev).to(vn.dtype)])
        table = torch.cat([table, torch.full((pad_rows, table.shape[1]), -1, dtype=torch.int32,
                                             device=dev)])
        seqlen = torch.cat([seqlen, torch.ones(pad_rows, dtype=torch.int32, device=dev)])
        slot = torch.cat([slot, torch.full((pad_rows,), -1, dtype=torch.int32, device=dev)])
    res = []
    for fused in (False, True):
        kc, vc = step.k_cache.to(dev), step.v_cache.to(dev)
        if fused:
            out = gqa_decode_paged_fn(q, kc, vc, table, seqlen, step.page_size,
                                      split_tokens=split_tokens, append=(kn, vn, slot))
        else:
            store_kvcache(kn, vn, flat(kc), flat(vc), slot)
            out = gqa_decode_paged_fn(q, kc, vc, table, seqlen, step.page_size,
                                      split_tokens=split_tokens)
        torch.cuda.synchronize()
        res.append((out, kc, vc))
    return res


def _assert_same(res):
    (o0, k0, v0), (o1, k1, v1) = res
    assert torch.equal(bits(o0), bits(o1))
    assert torch.equal(bits(k0), bits(k1))
    assert torch.equal(bits(v0), bits(v1))


@pytest.mark.parametrize("split", [None, 256, 2048])
def test_fused_append_equals_store_then_decode(split, dev):
    step = config2()
    say(f"decode append fused config2 split={split}")
    _assert_same(_both(step, dev, split_tokens=split))


@pytest.mark.parametrize("split", [None, 512])
def test_fused_append_with_graph_padding_rows(split, dev):
    """Padding rows (slot -1) write nothing and decode to zeros, as the unfused pair."""
    step = make_step([1, 15, 16, 17, 300, 4096], pool=400, seed=31)
    say(f"decode append fused padding split={split}")
    res = _both(step, dev, split_tokens=split, pad_rows=3)
    _assert_same(res)
    assert not bool(res[1][0][-3:].float().abs().sum())


@pytest.mark.parametrize("split", [None, 512])
def test_fused_append_row_without_tokens(split, dev):
    """A slot given for a sequence with context 0 (outside the contract, no workgroup reads it)
    is still written, as store_kvcache writes it; its output is zeros."""
    step = make_step([0, 40, 0, 900], pool=80, seed=32)
    used = set(step.block_table[step.block_table >= 0].tolist())
    free = [p for p in range(80) if p not in used]
    slots = step.slot_mapping.clone()
    slots[0], slots[2] = free[0] * 16 + 3, free[1] * 16  # rows no sequence of the call reads
    say(f"decode append fused ctx0 split={split}")
    res = _both(step, dev, split_tokens=split, slots=slots)
    _assert_same(res)
    assert not bool(res[1][0][0].float().abs().sum())


def test_fused_append_fp16_and_head_dim_128(dev):
    for kwargs in ({"dtype": torch.float16}, {"hq": 16, "hkv": 2, "d": 128}):
        step = make_step([33, 1000, 2047, 5000], pool=600, seed=33, **kwargs)
        say(f"decode append fused {kwargs}")
        _assert_same(_both(step, dev))


def test_fused_append_many_sequences_balanced(dev):
    """Batch 64 of mixed lengths: runs of the balanced plan end at many sequences' last tiles."""
    gen = torch.Generator().manual_seed(34)
    ctx = torch.randint(1, 3000, (64,), generator=gen).tolist()
    step = make_step(ctx, pool=sum((c + 15) // 16 for c in ctx) + 64, seed=34)
    say("decode append fused batch 64")
    _assert_same(_both(step, dev))


def test_fused_append_rejects(dev):
    step = make_step([100, 200], pool=40, seed=35)
    q, kc, vc = step.q.to(dev), step.k_cache.to(dev), step.v_cache.to(dev)
    table, seqlen = step.block_table.to(dev), step.seqlen.to(dev)
    app = (step.k_new.to(dev), step.v_new.to(dev), step.slot_mapping.to(dev))
    say("decode append fused rejects")
    with pytest.raises(ValueError):
        gqa_decode_paged_fn(q, kc, vc, table, seqlen, append=app, gate=torch.zeros_like(q))
    with pytest.raises(ValueError):
        gqa_decode_paged_fn(q, kc, vc, table, seqlen, append=app, variant="scalar")
    with pytest.raises(ValueError):
        gqa_decode_paged_fn(q, kc, vc, table, seqlen, append=app, shared_prefix_tokens=16)
    with pytest.raises(ValueError):
        gqa_decode_paged_fn(q, kc, vc, table, seqlen, append=(app[0][:1], app[1], app[2]))
    with pytest.raises(ValueError):
        gqa_decode_paged_fn(q, kc, vc, table, seqlen, append=(app[0], app[1], app[2].long()))


def test_fused_append_graph_capture_replay(dev):
    """The fused call captured in a HIP graph: three replays, each after new q / key / value
    contents and an eager call between, equal the eager store_kvcache + decode of that data."""
    step = config2()
    say("decode append fused graph replay")
    q, kn, vn = step.q.to(dev), step.k_new.to(dev), step.v_new.to(dev)
    table, seqlen, slot = step.block_table.to(dev), step.seqlen.to(dev), step.slot_mapping.to(dev)
    kc, vc = step.k_cache.to(dev), step.v_cache.to(dev)
    out = torch.empty_like(q)
    call = lambda: gqa_decode_paged_fn(q, kc, vc, table, seqlen, step.page_size,  # noqa: E731
                                       out=out, append=(kn, vn, slot))
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    gen = torch.Generator(device=dev).manual_seed(36)
    for rep in range(3):
        for t in (q, kn, vn):
            t.copy_(torch.randn(t.shape, generator=gen, device=dev).to(t.dtype))
        kr, vr = kc.clone(), vc.clone()
        store_kvcache(kn, vn, flat(kr), flat(vr), slot)
        ref = gqa_decode_paged_fn(q, kr, vr, table, seqlen, step.page_size)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(bits(out), bits(ref)), f"replay {rep}"
        assert torch.equal(bits(kc), bits(kr)) and torch.equal(bits(vc), bits(vr)), f"replay {rep}"
