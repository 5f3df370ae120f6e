"""ti_gqa_decode_paged_noalloc (the decode entry point that allocates nothing) through the C ABI,
against ti_gqa_decode_paged with a caller workspace: bitwise equal on two calls in a row, the
second with a smaller batch and shorter contexts, for the balanced plan, a fixed split and the
plans of short context bounds."""
import pytest
import torch

from helpers import bits, say
from tileinfer_amd import _lib
from tileinfer_amd.kernels.gqa_decode_paged import decode_plan, gqa_decode_paged_fn
from tileinfer_amd.workloads import make_step

pytestmark = pytest.mark.gpu


def _noalloc_abi(step, out, split_tokens, dev):
    """One call of the new entry point with raw pointers (no workspace argument exists)."""
    q, kc, vc = step.q, step.k_cache, step.v_cache
    table, seqlen = step.block_table, step.seqlen
    nb, bs, hkv, d = kc.shape
    lib = _lib.load()
    return lib.ti_gqa_decode_paged_noalloc(
        q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), table.data_ptr(),
        table.stride(0), seqlen.data_ptr(), out.data_ptr(), q.shape[0], q.shape[1], hkv, d, bs,
        nb, table.shape[1], int(split_tokens or 0), _lib.TI_DECODE_AUTO, _lib.TI_DTYPE_BF16,
        _lib.stream_handle(dev))


def _on(step, dev):
    for name in ("q", "k_cache", "v_cache", "block_table", "seqlen"):
        setattr(step, name, getattr(step, name).to(dev))
    return step


@pytest.mark.parametrize("split", [None, 1024])
def test_noalloc_matches_workspace_entry_two_calls(split, dev):
    lib = _lib.load()
    scratch = lib.ti_gqa_decode_scratch_bytes()
    assert scratch == 32 << 20
    big = _on(make_step([4000, 7000, 33, 0, 12000, 5000, 9000, 1] * 4, pool=9400, seed=41), dev)
    small = _on(make_step([300, 17, 2000], pool=200, seed=42), dev)
    for name, step in (("first (batch 32)", big), ("second (batch 3)", small)):
        b = step.q.shape[0]
        need = decode_plan(b, 24, 4, 256, 16, step.block_table.shape[1], split)[2]
        say(f"no-alloc decode {name}: split={split}, plan workspace {need} B of {scratch}")
        assert 0 < need <= scratch
        ref = gqa_decode_paged_fn(step.q, step.k_cache, step.v_cache, step.block_table,
                                  step.seqlen, 16, split_tokens=split)
        out = torch.full_like(step.q, float("nan"))
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated(dev)
        _lib.check(_noalloc_abi(step, out, split, dev))
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated(dev) == before
        assert torch.equal(bits(out), bits(ref)), name


@pytest.mark.parametrize("variant,kv_reuse,split", [("auto", False, None), ("auto", True, None),
                                                   ("scalar", False, 2048)])
def test_noalloc_python_wrapper_matches_decode_fn(variant, kv_reuse, split, dev):
    """gqa_decode_paged_noalloc (the Python side of the entry point) marshals the same call as
    gqa_decode_paged_fn: bitwise equal output, into the caller's `out`, for the variant, cache
    policy and split flags, and with a table one column wide (stride passed as is)."""
    from tileinfer_amd.kernels.gqa_decode_paged import gqa_decode_paged_noalloc

    big = _on(make_step([4000, 7000, 33, 0, 12000, 5000, 9000, 1] * 2, pool=4800, seed=43), dev)
    narrow = _on(make_step([16, 9, 1], pool=8, seed=44), dev)
    assert narrow.block_table.shape[1] == 1
    for name, step in (("batch 16", big), ("one-column table", narrow)):
        say(f"no-alloc wrapper {name}: variant={variant} kv_reuse={kv_reuse} split={split}")
        args = (step.q, step.k_cache, step.v_cache, step.block_table, step.seqlen, 16)
        ref = gqa_decode_paged_fn(*args, split_tokens=split, variant=variant, kv_reuse=kv_reuse)
        out = torch.full_like(step.q, float("nan"))
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated(dev)
        got = gqa_decode_paged_noalloc(*args, out=out, split_tokens=split, variant=variant,
                                       kv_reuse=kv_reuse)
        torch.cuda.synchronize()
        assert got is out and torch.cuda.memory_allocated(dev) == before
        assert torch.equal(bits(out), bits(ref)), name
        del got, out, ref  # the next case's count starts without them


def test_noalloc_python_wrapper_refusals(dev):
    """The wrapper refuses, rather than copies, what the entry point cannot take: unaligned q
    rows, a strided table or lengths, and an `out` of the wrong shape, dtype, device or layout.
    Nothing is launched for a refused call (`out` keeps its contents)."""
    from tileinfer_amd.kernels.gqa_decode_paged import gqa_decode_paged_noalloc

    step = _on(make_step([100, 40], pool=16, seed=45), dev)
    q, kc, vc, table, seqlen = step.q, step.k_cache, step.v_cache, step.block_table, step.seqlen
    out = torch.zeros_like(q)
    flat = torch.empty(q.numel() + 1, dtype=q.dtype, device=dev)
    q_unaligned = flat[1:].view_as(q).copy_(q)
    table_wide = torch.zeros((table.shape[0], 2 * table.shape[1]), dtype=torch.int32, device=dev)
    table_strided = table_wide[:, ::2]
    table_strided.copy_(table)
    seqlen_strided = torch.zeros(2 * seqlen.numel(), dtype=torch.int32, device=dev)[::2]
    seqlen_strided.copy_(seqlen)
    cases = [
        ("unaligned q", (q_unaligned, kc, vc, table, seqlen), out, "16-byte aligned"),
        ("strided table", (q, kc, vc, table_strided, seqlen), out, "unit-stride"),
        ("strided lengths", (q, kc, vc, table, seqlen_strided), out, "unit-stride"),
        ("out shape", (q, kc, vc, table, seqlen), torch.zeros_like(q[:1]), "out must be"),
        ("out dtype", (q, kc, vc, table, seqlen), torch.zeros_like(q, dtype=torch.float16),
         "out must be"),
        ("out on the host", (q, kc, vc, table, seqlen), torch.zeros_like(q, device="cpu"),
         "out must be"),
        ("out strided", (q, kc, vc, table, seqlen),
         torch.zeros((q.shape[1], q.shape[0], q.shape[2]), dtype=q.dtype,
                     device=dev).transpose(0, 1), "out must be"),
    ]
    for name, args, o, msg in cases:
        say(f"no-alloc wrapper refusal: {name}")
        sentinel = o.clone()
        with pytest.raises(ValueError, match=msg):
            gqa_decode_paged_noalloc(*args, 16, out=o)
        torch.cuda.synchronize()
        assert torch.equal(bits(o), bits(sentinel)), name
    # The same operands, made valid, run.
    ref = gqa_decode_paged_fn(q, kc, vc, table, seqlen, 16)
    gqa_decode_paged_noalloc(q, kc, vc, table, seqlen, 16, out=out)
    assert torch.equal(bits(out), bits(ref))


def _pool(ctx):
    return sum((c + 15) // 16 for c in ctx) + 8


def test_noalloc_short_bounds_two_calls(dev):
    """Short context bounds take the same plans through the entry point that allocates nothing:
    one workgroup per (KV head, sequence) for 64 sequences at a 512-token bound (no scratch), fixed
    32-token partitions (split-K scratch), then per pair again at a 128-token bound, bitwise equal
    to ti_gqa_decode_paged on calls in a row, each smaller than the one before. At
    128 query heads over 8 KV heads the balanced plan of the same shape would need more than the
    scratch; the short call is taken, not refused."""
    lib = _lib.load()
    scratch = lib.ti_gqa_decode_scratch_bytes()
    cases = []
    for name, ctx, seed, kw, split in (("per pair, one round at a 512 bound (batch 64)",
                                        [512] * 63 + [7], 49, {}, 0),
                                       ("short fixed (batch 6)", [512, 1, 0, 300, 999, 64], 46, {}, 32),
                                       ("per pair (batch 3)", [100, 0, 127], 47, {}, 0),
                                       ("per pair, 128/8 heads", [100, 60], 48,
                                        {"hq": 128, "hkv": 8}, 0)):
        cases.append((name, _on(make_step(ctx, pool=_pool(ctx), seed=seed, **kw), dev), split))
    for name, step, split in cases:
        b, hq = step.q.shape[:2]
        hkv = step.k_cache.shape[2]
        plan = decode_plan(b, hq, hkv, 256, 16, step.block_table.shape[1])
        say(f"no-alloc decode short bound, {name}: plan {plan[:2]}")
        assert plan[0] == split
        if hq == 128:
            assert plan[2] > scratch  # the plans' largest workspace: the balanced one
        ref = gqa_decode_paged_fn(step.q, step.k_cache, step.v_cache, step.block_table,
                                  step.seqlen, 16)
        out = torch.full_like(step.q, float("nan"))
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated(dev)
        _lib.check(_noalloc_abi(step, out, None, dev))
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated(dev) == before
        assert torch.equal(bits(out), bits(ref)), name
