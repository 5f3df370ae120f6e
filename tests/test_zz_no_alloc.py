"""ti_gqa_decode_paged_noalloc (the decode entry point that allocates nothing) through the C ABI,
against ti_gqa_decode_paged with a caller workspace: bitwise equal on two calls in a row, the
second with a smaller batch and shorter contexts, for the balanced plan and a fixed split."""
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
