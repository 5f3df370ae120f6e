"""A block pool larger than 4 GiB per K view and per V view (262,208 blocks of 32 KiB): pages just
below and above 2^31 elements (block 131,072) and at the top of the pool (byte offsets past 2^33)
go through every kernel of the path — append, decode (plain and with a shared prefix), paged
prefill in both schedules, block copy — and match the oracle run on a compact CPU copy of the
pages used. Config 3's pool is 131,072 blocks per layer; a pool sized from the free HBM of a
smaller model is larger, so page addressing must not wrap at 32 bits anywhere."""
import pytest
import torch

from helpers import ATOL, RTOL, assert_decode_close, bits, flat, say
from oracle.ref_torch import ref_gqa_decode_paged, ref_gqa_prefill_paged
from tileinfer_amd.kernels import copy_blocks, gqa_decode_paged_fn, store_kvcache
from tileinfer_amd.kernels.gqa_prefill_paged import gqa_prefill_paged_fn

pytestmark = pytest.mark.gpu

NB, BS, HQ, HKV, D = 262144 + 64, 16, 24, 4, 256
MID = 131072  # first block whose element offset reaches 2^31


@pytest.fixture(scope="module")
def pool(dev):
    say(f"large pool: 2 x {NB} blocks x {BS * HKV * D * 2} B")
    kv = torch.empty(2, NB, BS, HKV, D, dtype=torch.bfloat16, device=dev)
    yield kv
    del kv
    torch.cuda.empty_cache()


def pick_blocks(n, seed):
    """n distinct block ids: half from the top 4,096 blocks of the pool, half from the 4,096
    around block 131,072, shuffled."""
    g = torch.Generator().manual_seed(seed)
    hi = NB - 1 - torch.randperm(4096, generator=g)[: n // 2]
    mid = MID - 2048 + torch.randperm(4096, generator=g)[: n - n // 2]
    ids = torch.cat([hi, mid])
    return ids[torch.randperm(n, generator=g)]


def fill(pool, ids, seed):
    """Random pages at `ids` in the pool; returns their CPU copies [n, BS, HKV, D] for K and V."""
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(len(ids), BS, HKV, D, generator=g).to(torch.bfloat16)
    v = torch.randn(len(ids), BS, HKV, D, generator=g).to(torch.bfloat16)
    dev_ids = ids.to(pool.device)
    pool[0, dev_ids] = k.to(pool.device)
    pool[1, dev_ids] = v.to(pool.device)
    return k, v


def tables(lens, ids):
    """Pool tables (-1 padded) over consecutive runs of `ids`, and the same tables over the
    compact copy (page i of the copy = ids[i])."""
    width = max(1, max((n + BS - 1) // BS for n in lens))
    pool_t = torch.full((len(lens), width), -1, dtype=torch.int32)
    compact_t = torch.full((len(lens), width), -1, dtype=torch.int32)
    at = 0
    for b, n in enumerate(lens):
        pages = (n + BS - 1) // BS
        pool_t[b, :pages] = ids[at:at + pages].to(torch.int32)
        compact_t[b, :pages] = torch.arange(at, at + pages, dtype=torch.int32)
        at += pages
    return pool_t, compact_t


def test_decode_high_pages(pool, dev):
    ctx = [32768, 9001, 1, 300]
    say(f"large pool decode ctx={ctx}")
    need = sum((n + BS - 1) // BS for n in ctx)
    ids = pick_blocks(need, seed=41)
    kc, vc = fill(pool, ids, seed=42)
    pool_t, compact_t = tables(ctx, ids)
    g = torch.Generator().manual_seed(43)
    q = torch.randn(len(ctx), HQ, D, generator=g).to(torch.bfloat16)
    seqlen = torch.tensor(ctx, dtype=torch.int32)
    out = gqa_decode_paged_fn(q.to(dev), pool[0], pool[1], pool_t.to(dev), seqlen.to(dev), BS)
    ref = ref_gqa_decode_paged(q, kc, vc, compact_t, seqlen, BS)
    assert_decode_close(out, ref)


def test_shared_prefix_decode_high_pages(pool, dev):
    """Three sequences whose first 4,096 tokens are the same 256 high pages, each with pages of
    its own after them: the shared-prefix call against the oracle and the plain call."""
    prefix, own = 4096, [700, 33, 1200]
    say(f"large pool shared-prefix decode prefix={prefix} own={own}")
    pp = prefix // BS
    own_pages = [(n + BS - 1) // BS for n in own]
    ids = pick_blocks(pp + sum(own_pages), seed=44)
    kc, vc = fill(pool, ids, seed=45)
    width = pp + max(own_pages)
    pool_t = torch.full((len(own), width), -1, dtype=torch.int32)
    compact_t = torch.full((len(own), width), -1, dtype=torch.int32)
    at = pp
    for b, n in enumerate(own_pages):
        pool_t[b, :pp] = ids[:pp].to(torch.int32)
        compact_t[b, :pp] = torch.arange(pp, dtype=torch.int32)
        pool_t[b, pp:pp + n] = ids[at:at + n].to(torch.int32)
        compact_t[b, pp:pp + n] = torch.arange(at, at + n, dtype=torch.int32)
        at += n
    g = torch.Generator().manual_seed(46)
    q = torch.randn(len(own), HQ, D, generator=g).to(torch.bfloat16)
    seqlen = torch.tensor([prefix + n for n in own], dtype=torch.int32)
    args = (q.to(dev), pool[0], pool[1], pool_t.to(dev), seqlen.to(dev), BS)
    shared = gqa_decode_paged_fn(*args, shared_prefix_tokens=prefix, prefix_pass="always")
    plain = gqa_decode_paged_fn(*args)
    ref = ref_gqa_decode_paged(q, kc, vc, compact_t, seqlen, BS)
    assert_decode_close(shared, ref)
    assert_decode_close(shared, plain)


@pytest.mark.parametrize("schedule", ["balanced", "per_unit"])
def test_prefill_high_pages(pool, schedule, dev):
    q_lens, kv_lens = [300, 5, 64], [4000, 5, 2100]
    say(f"large pool prefill q_lens={q_lens} kv_lens={kv_lens} schedule={schedule}")
    need = sum((n + BS - 1) // BS for n in kv_lens)
    ids = pick_blocks(need, seed=47)
    kc, vc = fill(pool, ids, seed=48)
    pool_t, compact_t = tables(kv_lens, ids)
    g = torch.Generator().manual_seed(49)
    q = torch.randn(sum(q_lens), HQ, D, generator=g).to(torch.bfloat16)
    cu = torch.tensor([0] + list(torch.tensor(q_lens).cumsum(0)), dtype=torch.int32)
    seqlen_k = torch.tensor(kv_lens, dtype=torch.int32)
    out = gqa_prefill_paged_fn(q.to(dev), pool[0], pool[1], pool_t.to(dev), cu.to(dev),
                               seqlen_k.to(dev), max(q_lens), BS, schedule=schedule)
    ref = ref_gqa_prefill_paged(q, kc, vc, compact_t, cu, seqlen_k, BS)
    torch.testing.assert_close(out.float().cpu(), ref.float(), atol=ATOL, rtol=RTOL)


def test_append_high_slots(pool, dev):
    """Rows written at slots in high pages (and -1 skips) equal the new rows; every other row of
    the 16 GiB pool keeps its bits."""
    n = 96
    say(f"large pool append n={n}")
    ids = pick_blocks(n, seed=50)
    g = torch.Generator().manual_seed(51)
    slots = ids * BS + torch.randint(0, BS, (n,), generator=g)
    slots[::9] = -1
    key = torch.randn(n, HKV, D, generator=g).to(torch.bfloat16).to(dev)
    value = torch.randn(n, HKV, D, generator=g).to(torch.bfloat16).to(dev)
    expect = pool.clone()
    store_kvcache(key, value, flat(pool[0]), flat(pool[1]), slots.to(torch.int32).to(dev))
    live = slots >= 0
    rows, live = slots[live].to(dev), live.to(dev)
    flat(expect[0])[rows] = key[live].reshape(-1, HKV * D)
    flat(expect[1])[rows] = value[live].reshape(-1, HKV * D)
    assert torch.equal(bits(pool), bits(expect))


def test_copy_blocks_high_ids(pool, dev):
    """Copies from the top of the pool to pages near block 131,072 and back are bit-exact and
    touch nothing else."""
    n = 64
    say(f"large pool copy_blocks n={n}")
    ids = pick_blocks(2 * n, seed=52)
    src = torch.tensor([int(i) for i in ids if i >= MID + 4096][:n // 2] +
                       [int(i) for i in ids if i < MID + 4096][:n // 2])
    dst = torch.tensor([int(i) for i in ids if i < MID + 4096][n // 2:n] +
                       [int(i) for i in ids if i >= MID + 4096][n // 2:n])
    assert len(src) == len(dst) == n
    fill(pool, ids, seed=53)
    mapping = torch.stack([src, dst], dim=1).to(dev)
    expect = pool.clone()
    expect[:, dst.to(dev)] = pool[:, src.to(dev)]
    copy_blocks(pool, pool, mapping)  # [2, blocks, ...]: K and V pages together
    assert torch.equal(bits(pool), bits(expect))
