"""Pages smaller than the 16-token tile (the reference's Config.kvcache_block_size is configurable,
engine/config.py:20, and its decode takes pages that divide its 64-token tile,
kernels/gqa_decode_paged.py:57-62, 408): decode through the C ABI at pages of 8, 4, 2 and 1
tokens against the CPU oracle, and bitwise against page 16 on the same memory."""
import pytest
import torch

from helpers import assert_decode_close, bits, flat, say
from oracle.ref_torch import ref_gqa_decode_paged
from tileinfer_amd.kernels.gqa_decode_paged import gqa_decode_paged_fn
from tileinfer_amd.kernels.kvcache_store import store_kvcache
from tileinfer_amd.workloads import make_step

pytestmark = pytest.mark.gpu


def _config2_ctx(seed=1002, batch=16, lo=512, hi=8192):
    gen = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randint(lo, hi + 1, (batch,), generator=gen).tolist()


def _on(step, dev):
    for name in ("q", "k_new", "v_new", "slot_mapping", "block_table", "seqlen", "k_cache",
                 "v_cache"):
        setattr(step, name, getattr(step, name).to(dev))
    return step


@pytest.mark.parametrize("split", [None, 1024])
@pytest.mark.parametrize("variant", ["mfma", "scalar"])
@pytest.mark.parametrize("page", [8, 4])
def test_config2_shapes_vs_oracle(page, variant, split, dev):
    """Config 2's batch (16 sequences, contexts U[512, 8192]) over pages of 8 and 4 tokens, random
    tables, against the oracle at the same page size."""
    ctx = _config2_ctx()
    need = sum((c + page - 1) // page for c in ctx)
    step = make_step(ctx, pool=need * 5 // 4, seed=1002, page=page)
    say(f"small pages: page={page} variant={variant} split={split} batch 16, ctx_sum {sum(ctx)}")
    if variant == "scalar" and split is None:
        split = 2048
    out = gqa_decode_paged_fn(step.q.to(dev), step.k_cache.to(dev), step.v_cache.to(dev),
                              step.block_table.to(dev), step.seqlen.to(dev), page,
                              split_tokens=split, variant=variant)
    ref = ref_gqa_decode_paged(step.q, step.k_cache, step.v_cache, step.block_table,
                               step.seqlen, page)
    assert_decode_close(out, ref)


@pytest.mark.parametrize("page", [2, 1])
@pytest.mark.parametrize("variant", ["mfma", "scalar"])
def test_tiny_pages_vs_oracle(page, variant, dev):
    ctx = [1, 2, 3, 15, 16, 17, 100, 257, 1000]
    need = sum((c + page - 1) // page for c in ctx)
    step = make_step(ctx, pool=need + 7, seed=40 + page, page=page)
    say(f"tiny pages: page={page} variant={variant}")
    out = gqa_decode_paged_fn(step.q.to(dev), step.k_cache.to(dev), step.v_cache.to(dev),
                              step.block_table.to(dev), step.seqlen.to(dev), page,
                              variant=variant, split_tokens=512 if variant == "scalar" else None)
    ref = ref_gqa_decode_paged(step.q, step.k_cache, step.v_cache, step.block_table,
                               step.seqlen, page)
    assert_decode_close(out, ref)


@pytest.mark.parametrize("page", [8, 4, 2])
def test_same_memory_as_page16_bitwise(page, dev):
    """A page-16 cache viewed as pages of `page` tokens (block i -> blocks 16/page * i + j) is the
    same tokens in the same 16-token tiles: the decode is bitwise the page-16 decode, under the
    balanced plan, a fixed split, and the forced cache policies; the fused append too."""
    ctx = [700, 4096, 33, 1, 2500, 9000, 16, 17]
    st = _on(make_step(ctx, pool=1200, seed=51, width=600), dev)
    r = 16 // page
    nb = st.k_cache.shape[0]
    kv_small = [c.view(nb * r, page, *c.shape[2:]) for c in (st.k_cache, st.v_cache)]
    cols = torch.arange(st.block_table.shape[1] * r, device=dev)
    base = st.block_table[:, cols // r]
    table_small = torch.where(base >= 0, base * r + (cols % r), base).to(torch.int32)
    for split in (None, 512):
        for reuse in (None, False, True):
            say(f"page {page} view vs page 16: split={split} kv_reuse={reuse}")
            a = gqa_decode_paged_fn(st.q, st.k_cache, st.v_cache, st.block_table, st.seqlen, 16,
                                    split_tokens=split, kv_reuse=reuse)
            b = gqa_decode_paged_fn(st.q, *kv_small, table_small, st.seqlen, page,
                                    split_tokens=split, kv_reuse=reuse)
            assert torch.equal(bits(a), bits(b)), (split, reuse)
    # The fused append writes the same cache rows (slots do not depend on the page size).
    k16, v16 = st.k_cache.clone(), st.v_cache.clone()
    a = gqa_decode_paged_fn(st.q, k16, v16, st.block_table, st.seqlen, 16,
                            append=(st.k_new, st.v_new, st.slot_mapping))
    ks, vs = [c.view(nb * r, page, *c.shape[2:]) for c in (st.k_cache, st.v_cache)]
    b = gqa_decode_paged_fn(st.q, ks, vs, table_small, st.seqlen, page,
                            append=(st.k_new, st.v_new, st.slot_mapping))
    assert torch.equal(bits(a), bits(b))
    assert torch.equal(bits(k16), bits(st.k_cache)) and torch.equal(bits(v16), bits(st.v_cache))


@pytest.mark.parametrize("page", [8, 4])
def test_absent_pages_and_padding_rows(page, dev):
    """An id outside the cache at a used position is an absent page (its tokens masked, never
    read), also when it shares a 16-token tile with a present page; the runner's graph-padding
    rows (context 1, all -1) decode to zeros."""
    ctx = [100, 100, 40, 1]
    st = make_step(ctx, pool=80, seed=52, page=page)
    tbl = st.block_table.clone()
    tbl[0, 3] = 10**6               # one page of sequence 0
    tbl[1, 0] = -5                  # sequence 1's first page
    tbl[2, 1] = -1                  # sequence 2's second page
    tbl[3, :] = -1                  # padding row
    say(f"small pages: absent pages, page={page}")
    out = gqa_decode_paged_fn(st.q.to(dev), st.k_cache.to(dev), st.v_cache.to(dev),
                              tbl.to(dev), st.seqlen.to(dev), page).cpu()
    kf = st.k_cache.float().reshape(-1, 4, 256).double()
    vf = st.v_cache.float().reshape(-1, 4, 256).double()
    for b in range(3):
        pos = [p for p in range(ctx[b]) if 0 <= int(tbl[b, p // page]) < st.k_cache.shape[0]]
        assert len(pos) < ctx[b]
        rows = torch.tensor([int(tbl[b, p // page]) * page + p % page for p in pos])
        k, v = kf[rows], vf[rows]
        for h in range(24):
            w = torch.softmax(k[:, h // 6] @ st.q[b, h].double() / 16.0, 0)
            torch.testing.assert_close(out[b, h].double(), w @ v[:, h // 6], atol=1e-2, rtol=1e-2)
    assert not bool(out[3].view(torch.int16).any())


def test_store_then_decode_page8(dev):
    """The step's two calls at page 8 (store_kvcache through the flat row view, then decode)
    against the oracle's append + decode."""
    ctx = [1000, 333, 4097]
    st = make_step(ctx, pool=800, seed=53, page=8)
    kc, vc = st.k_cache.to(dev), st.v_cache.to(dev)
    store_kvcache(st.k_new.to(dev), st.v_new.to(dev), flat(kc), flat(vc), st.slot_mapping.to(dev))
    out = gqa_decode_paged_fn(st.q.to(dev), kc, vc, st.block_table.to(dev), st.seqlen.to(dev), 8)
    kr, vr = st.k_cache.clone(), st.v_cache.clone()
    live = st.slot_mapping.long()
    flat(kr)[live] = st.k_new.reshape(len(ctx), -1)
    flat(vr)[live] = st.v_new.reshape(len(ctx), -1)
    assert torch.equal(bits(kc.cpu()), bits(kr)) and torch.equal(bits(vc.cpu()), bits(vr))
    assert_decode_close(out, ref_gqa_decode_paged(st.q, kr, vr, st.block_table, st.seqlen, 8))


# ---------------------------------------------------------------------------- prefill


@pytest.mark.parametrize("schedule", ["balanced", "per_unit"])
@pytest.mark.parametrize("page", [8, 4])
def test_prefill_small_pages_vs_oracle(page, schedule, dev):
    """The paged prefill over pages of 8 and 4 tokens: first chunks, continuations, a ragged batch
    with an empty chunk, against the oracle and float64 at the same page size."""
    from oracle.brute import prefill_fp64
    from oracle.ref_torch import ref_gqa_prefill_paged
    from tileinfer_amd.kernels.gqa_prefill_paged import gqa_prefill_paged_fn
    from tileinfer_amd.workloads import prefill_step

    for q_lens, kv_lens in (([100], [100]), ([37], [300]), ([16, 1, 0, 50, 129], [16, 200, 5, 51, 1000]),
                            ([3], [2000])):
        say(f"prefill page={page} schedule={schedule} q_lens={q_lens} kv_lens={kv_lens}")
        st = prefill_step(q_lens, kv_lens, seed=61, page=page)
        out = gqa_prefill_paged_fn(st.q.to(dev), st.k_cache.to(dev), st.v_cache.to(dev),
                                   st.block_table.to(dev), st.cu_seqlens_q.to(dev),
                                   st.seqlen_k.to(dev), st.max_seqlen_q, page, schedule=schedule)
        ref = ref_gqa_prefill_paged(st.q, st.k_cache, st.v_cache, st.block_table, st.cu_seqlens_q,
                                    st.seqlen_k, page)
        torch.testing.assert_close(out.float().cpu(), ref.float(), atol=2e-2, rtol=1e-2)
        exact = torch.from_numpy(prefill_fp64(
            st.q.double().numpy(), st.k_cache.double().numpy(), st.v_cache.double().numpy(),
            st.block_table.numpy(), st.cu_seqlens_q.numpy(), st.seqlen_k.numpy(), page))
        torch.testing.assert_close(out.float().cpu(), exact.float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("d,hq,hkv", [(256, 24, 4), (128, 32, 8)])
@pytest.mark.parametrize("page", [8, 4])
def test_prefill_same_memory_as_page16_bitwise(page, d, hq, hkv, dev):
    """Config 4's continuation shape (2,048 queries over 8,192 keys) on a page-16 cache viewed as
    pages of 8 and 4 tokens: bitwise the page-16 prefill under each schedule (the same keys land
    in the same LDS tiles), and the shared-prefix decode over those pages likewise."""
    from tileinfer_amd.kernels.gqa_prefill_paged import gqa_prefill_paged_fn
    from tileinfer_amd.workloads import prefill_step

    st = prefill_step([2048], [8192], seed=62, device=dev, hq=hq, hkv=hkv, d=d)
    r = 16 // page
    nb = st.k_cache.shape[0]
    ks, vs = [c.view(nb * r, page, *c.shape[2:]) for c in (st.k_cache, st.v_cache)]
    cols = torch.arange(st.block_table.shape[1] * r, device=dev)
    base = st.block_table[:, cols // r]
    tsmall = torch.where(base >= 0, base * r + (cols % r), base).to(torch.int32)
    for sched in ("balanced", "per_unit"):
        say(f"prefill page {page} view vs page 16 (d={d}): {sched}")
        a = gqa_prefill_paged_fn(st.q, st.k_cache, st.v_cache, st.block_table, st.cu_seqlens_q,
                                 st.seqlen_k, 2048, 16, schedule=sched, max_seqlen_k=8192)
        b = gqa_prefill_paged_fn(st.q, ks, vs, tsmall, st.cu_seqlens_q, st.seqlen_k, 2048, page,
                                 schedule=sched, max_seqlen_k=8192)
        assert torch.equal(bits(a), bits(b)), sched
    # Absent pages inside the context are masked per page, also where a present page shares the
    # 16-key sub-tile (expected: float64 attention of each row over its visible keys minus the
    # absent page's).
    small = prefill_step([20], [40], seed=63, page=page, width=48 // page)
    t2 = small.block_table.clone()
    t2[0, 3] = 10 ** 8                       # keys 3 page .. 4 page - 1
    gone = range(3 * page, 4 * page)
    out = gqa_prefill_paged_fn(small.q.to(dev), small.k_cache.to(dev), small.v_cache.to(dev),
                               t2.to(dev), small.cu_seqlens_q.to(dev), small.seqlen_k.to(dev), 20,
                               page).float().cpu()
    kf = small.k_cache.double().reshape(-1, 4, 256)
    vf = small.v_cache.double().reshape(-1, 4, 256)
    rows = [int(small.block_table[0, j // page]) * page + j % page for j in range(40)]
    k, v = kf[rows], vf[rows]
    for i in range(20):
        keys = [j for j in range(20 + i + 1) if j not in gone]
        for h in range(24):
            w = torch.softmax(k[keys, h // 6] @ small.q[i, h].double() / 16.0, 0)
            torch.testing.assert_close(out[i, h].double(), w @ v[keys, h // 6], atol=2e-2,
                                       rtol=1e-2)


@pytest.mark.parametrize("page", [8, 4])
def test_shared_prefix_decode_small_pages(page, dev):
    """The shared-prefix decode (prefix attended once through the prefill kernel) at pages of 8
    and 4: against the plain call, and shared pages against private copies bitwise."""
    from tileinfer_amd.workloads import config5

    shared = config5(batch=16, prefix=2048, suffix=256, device=dev, shared=True)
    private = config5(batch=16, prefix=2048, suffix=256, device=dev, shared=False)
    r = 16 // page
    outs = []
    for st in (shared, private):
        nb = st.k_cache.shape[0]
        ks, vs = [c.view(nb * r, page, *c.shape[2:]) for c in (st.k_cache, st.v_cache)]
        cols = torch.arange(st.block_table.shape[1] * r, device=dev)
        base = st.block_table[:, cols // r]
        tb = (base * r + (cols % r)).to(torch.int32)
        say(f"shared-prefix decode page {page}: shared={st.meta['shared']}")
        pre = gqa_decode_paged_fn(st.q, ks, vs, tb, st.seqlen, page, shared_prefix_tokens=2048,
                                  prefix_pass="always")
        plain = gqa_decode_paged_fn(st.q, ks, vs, tb, st.seqlen, page)
        assert_decode_close(pre, plain.float(), atol=2e-3, rtol=1e-2)
        p16 = gqa_decode_paged_fn(st.q, st.k_cache, st.v_cache, st.block_table, st.seqlen, 16,
                                  shared_prefix_tokens=2048, prefix_pass="always")
        assert torch.equal(bits(pre), bits(p16))
        outs.append(pre)
    assert torch.equal(bits(outs[0]), bits(outs[1]))
