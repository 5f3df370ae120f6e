"""A seeded sweep of random decode shapes against the CPU oracle. Batch, KV heads and query group,
head_dim, page size, dtype, context lengths (empty, one token, page and tile edges, the bound
itself, ragged) and the partition plan (the default for the shape, or an explicit split) are drawn
together, so that their combinations are checked and not only each one alone. Every case appends
the step's token first (store_kvcache, then decode; the oracle does the same on CPU copies), and
every other case also runs the decode with the append fused in (`append=`), which must give the
same output and cache bit for bit. A second test runs one long sequence among short ones, whose
rows the merge sums with 8, 4 or 2 waves, over head dims, dtypes and page sizes."""
import random

import pytest
import torch

from helpers import assert_decode_close, bits, cpu_step, flat, gpu_step, say
from tileinfer_amd.kernels.gqa_decode_paged import decode_plan, gqa_decode_paged_fn
from tileinfer_amd.workloads import make_step

pytestmark = pytest.mark.gpu

N_CASES = 96
MAX_CACHE_ELEMS = 1 << 25  # pool tokens x KV heads x head_dim per cache: keeps the CPU side quick


def _draw(seed):
    """One case: (ctx, page, hq, hkv, d, dtype, width, split). Redrawn from the same stream until
    the pool is small enough for the CPU oracle."""
    r = random.Random(seed)
    while True:
        hkv = r.choice([1, 2, 4, 8])
        group = r.choice([1, 2, 3, 4, 6, 8, 16])
        d = r.choice([128, 256])
        page = r.choice([1, 2, 4, 8, 16, 32])
        dtype = r.choice([torch.bfloat16, torch.float16])
        batch = r.choice([1, 2, 3, 5, 8, 17, 40])
        bound = r.choice([16, 100, 128, 600, 1024, 3000])
        edges = [0, 1, page, 15, 16, 17, 31, 32, 33, bound]
        ctx = [min(bound, r.choice(edges) if r.random() < 0.3 else r.randint(0, bound))
               for _ in range(batch)]
        width = -(-bound // page) + r.choice([0, 0, 1])
        unit = 32 if page <= 32 else page
        split = r.choice([None, None, None, unit, 4 * unit, 256])
        pool = sum(-(-c // page) for c in ctx) + 4
        if pool * page * hkv * d <= MAX_CACHE_ELEMS:
            return ctx, page, hkv * group, hkv, d, dtype, width, split


@pytest.mark.parametrize("seed", range(N_CASES))
def test_decode_random_shape_vs_oracle(seed, dev):
    ctx, page, hq, hkv, d, dtype, width, split = _draw(1000 + seed)
    pool = sum(-(-c // page) for c in ctx) + 4
    step = make_step(ctx, pool=pool, seed=seed, dtype=dtype, width=width, hq=hq, hkv=hkv, d=d,
                     page=page)
    plan = decode_plan(len(ctx), hq, hkv, d, page, width, split)
    say(f"decode sweep seed={seed}: B={len(ctx)} hq={hq} hkv={hkv} d={d} page={page} "
        f"{str(dtype)[6:]} width={width} split={split} plan={plan[:2]} ctx={ctx}")
    out, kc, vc = gpu_step(step, dev, split_tokens=split)
    ref, kr, vr = cpu_step(step)
    assert torch.equal(bits(kc.cpu()), bits(kr)) and torch.equal(bits(vc.cpu()), bits(vr))
    assert_decode_close(out, ref)
    for b, c in enumerate(ctx):
        if c == 0:
            assert bool((out[b] == 0).all()), b
    if seed % 2 == 0:
        kf, vf = step.k_cache.to(dev), step.v_cache.to(dev)
        fused = gqa_decode_paged_fn(step.q.to(dev), kf, vf, step.block_table.to(dev),
                                    step.seqlen.to(dev), page, split_tokens=split,
                                    append=(step.k_new.to(dev), step.v_new.to(dev),
                                            step.slot_mapping.to(dev)))
        torch.cuda.synchronize()
        assert torch.equal(bits(fused), bits(out))
        assert torch.equal(bits(flat(kf)), bits(flat(kc))) and torch.equal(bits(flat(vf)),
                                                                           bits(flat(vc)))


@pytest.mark.parametrize("batch", [3, 10, 40])
@pytest.mark.parametrize("page", [8, 16])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [128, 256])
def test_long_row_merge_widths(d, dtype, page, batch, dev):
    """One 6,000-token sequence among short ones: its rows are cut into ~94 parts, which the merge
    sums with 8, 4 or 2 waves per row by the batch's row count (q-heads x sequences: 72-96, 240-
    320, 960-1,280 here), for both head dims, both dtypes and pages of 8 and 16. The fused append
    runs first. Against the oracle."""
    hq, hkv = (24, 4) if d == 256 else (32, 8)
    r = random.Random(batch * 1000 + page * 10 + d)
    ctx = [6000] + [r.randint(0, 300) for _ in range(batch - 1)]
    pool = sum(-(-c // page) for c in ctx) + 4
    step = make_step(ctx, pool=pool, seed=batch + page + d, dtype=dtype, hq=hq, hkv=hkv, d=d,
                     page=page)
    plan = decode_plan(batch, hq, hkv, d, page, step.block_table.shape[1])
    say(f"decode long-row merge: B={batch} hq={hq} d={d} page={page} {str(dtype)[6:]} "
        f"plan={plan[:2]}")
    assert plan[0] == 0 and plan[1] > 0  # balanced
    out, kc, vc = gpu_step(step, dev)
    ref, kr, vr = cpu_step(step)
    assert torch.equal(bits(kc.cpu()), bits(kr))
    assert_decode_close(out, ref)
