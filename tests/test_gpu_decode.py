"""Parity of the HIP paged decode (ti_gqa_decode_paged) with the CPU oracle, plus the bitwise
invariants the layout promises (shared vs private prefix, block permutation, padding)."""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import (assert_decode_close, bits, cpu_step, flat, fp64_decode, gpu_step, say)
from oracle.ref_torch import ref_gqa_decode_paged
from tileinfer_amd.kernels.gqa_decode_paged import decode_plan, gqa_decode_paged_fn
from tileinfer_amd.kernels.kvcache_store import store_kvcache
from tileinfer_amd.workloads import PagedStep, config1, config2, config5, make_step

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
VARIANTS = ["mfma", "scalar"]


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("ctx", [512, 513])
def test_config1_vs_oracle_and_golden(ctx, variant, dev):
    say(f"decode config1 ctx={ctx} variant={variant}")
    step = config1(ctx=ctx)
    out, kc, vc = gpu_step(step, dev, variant=variant)
    ref, k_ref, _ = cpu_step(step)
    assert torch.equal(bits(kc.cpu()), bits(k_ref))
    assert_decode_close(out, ref)
    # Tighter against the exact value: the kernel keeps scores in fp32.
    assert_decode_close(out, fp64_decode(step, k_ref, vc.cpu()), atol=4e-3, rtol=1e-2)
    meta = json.loads((GOLDEN / f"config1_ctx{ctx}.json").read_text())
    gold = torch.from_numpy(np.load(GOLDEN / f"config1_ctx{ctx}_out.npy")).view(torch.bfloat16)
    assert_decode_close(out, gold.view(1, 24, 256))
    assert meta["ctx"] == ctx


@pytest.mark.parametrize("variant", VARIANTS)
def test_config2_vs_oracle(variant, dev):
    step = config2()
    say(f"decode config2 ctx={step.meta['ctx']} variant={variant}")
    out, _, _ = gpu_step(step, dev, variant=variant)
    ref, _, _ = cpu_step(step)
    assert_decode_close(out, ref)


@pytest.mark.parametrize("variant", VARIANTS)
def test_reference_selftest_shape(variant, dev):
    """kernels/gqa_decode_paged.py:472-512 at its default batch: B 32, Hq 32, Hkv 8, D 128,
    seqlen 8192, a fifth of the batch shortened to U[2048, 8192), every sequence on the same
    sequential table."""
    say(f"decode reference selftest shape variant={variant}")
    g = torch.Generator().manual_seed(0)
    b, hq, hkv, d, seqlen, ps = 32, 32, 8, 128, 8192, 16
    max_pages = int(seqlen * 1.1) // ps
    seq = torch.full((b,), seqlen, dtype=torch.int32)
    seq[: b // 5] = torch.randint(seqlen // 4, seqlen, (b // 5,), generator=g, dtype=torch.int32)
    q = torch.randn(b, hq, d, generator=g).to(torch.bfloat16)
    kc = torch.randn(max_pages, ps, hkv, d, generator=g).to(torch.bfloat16)
    vc = torch.randn(max_pages, ps, hkv, d, generator=g).to(torch.bfloat16)
    table = torch.arange(max_pages, dtype=torch.int32).unsqueeze(0).expand(b, -1).contiguous()
    out = gqa_decode_paged_fn(q.to(dev), kc.to(dev), vc.to(dev), table.to(dev), seq.to(dev), ps,
                              variant=variant)
    ref = ref_gqa_decode_paged(q, kc, vc, table, seq, ps)
    assert_decode_close(out, ref)


@pytest.mark.parametrize("variant", VARIANTS)
def test_edge_lengths_and_splits(variant, dev):
    """Context lengths around tile, page and partition boundaries, with a small partition so the
    merge runs; ctx 0 must give zeros."""
    ctx = [0, 1, 2, 15, 16, 17, 31, 32, 33, 255, 256, 257, 511, 512, 513, 1000]
    say(f"decode edge lengths variant={variant} ctx={ctx}")
    step = make_step(ctx, pool=300, seed=21)
    for split in (256, None):
        out, kc, vc = gpu_step(step, dev, variant=variant, split_tokens=split, append=False)
        ref, _, _ = cpu_step(step, append=False)
        assert_decode_close(out, ref)
        assert not bool(out[0].float().abs().sum() != 0), "ctx 0 must give a zero row"
        assert_decode_close(out, fp64_decode(step, step.k_cache, step.v_cache), atol=1e-2)


def test_ctx1_and_constant_v(dev):
    """Closed forms: ctx 1 returns V[0] of the mapped KV head; constant V returns that constant."""
    say("decode closed forms")
    step = make_step([1, 40, 300], pool=40, seed=3)
    out, _, _ = gpu_step(step, dev, append=False)
    g = 6
    blk = int(step.block_table[0, 0])
    v0 = step.v_cache[blk, 0]  # [Hkv, D]
    expect = v0.repeat_interleave(g, dim=0)
    assert torch.equal(bits(out[0].cpu()), bits(expect))
    vc = torch.full_like(step.v_cache, 0.375)
    out2 = gqa_decode_paged_fn(step.q.to(dev), step.k_cache.to(dev), vc.to(dev),
                               step.block_table.to(dev), step.seqlen.to(dev))
    assert bool((out2.float() == 0.375).all())


def test_shared_vs_private_prefix_bitwise(dev):
    """Sequences whose tables alias one prefix give bitwise the same output as private copies."""
    say("decode shared vs private (config5 at batch 8)")
    shared = config5(batch=8, device=dev, shared=True)
    private = config5(batch=8, device=dev, shared=False)
    o1 = None
    for variant in VARIANTS:
        for reuse in (None, False, True):
            a = gqa_decode_paged_fn(shared.q, shared.k_cache, shared.v_cache, shared.block_table,
                                    shared.seqlen, variant=variant, kv_reuse=reuse)
            b = gqa_decode_paged_fn(private.q, private.k_cache, private.v_cache,
                                    private.block_table, private.seqlen, variant=variant,
                                    kv_reuse=reuse)
            assert torch.equal(bits(a), bits(b)), (variant, reuse)
            if variant == "mfma":
                o1 = a if o1 is None else o1
                assert torch.equal(bits(a), bits(o1)), "the cache policy changed the result"
    # And against the oracle for two sampled sequences (CPU copies of their blocks only).
    for i in (0, 5):
        pages = shared.block_table[i].long()
        sub = PagedStep(q=shared.q[i:i + 1].cpu(), k_new=shared.k_new[i:i + 1].cpu(),
                        v_new=shared.v_new[i:i + 1].cpu(), slot_mapping=shared.slot_mapping[i:i + 1].cpu(),
                        block_table=torch.arange(len(pages), dtype=torch.int32).view(1, -1),
                        seqlen=shared.seqlen[i:i + 1].cpu(), k_cache=shared.k_cache[pages].cpu(),
                        v_cache=shared.v_cache[pages].cpu())
        ref, _, _ = cpu_step(sub, append=False)
        assert_decode_close(o1[i:i + 1], ref)


def test_cache_policy_chosen_on_device_bitwise(dev):
    """The default call picks each sequence's cache policy on the device (a first block another
    sequence also starts with -> keep, else stream). Whatever it picks, the output is bitwise the
    forced-keep and forced-stream output: two groups sharing different prefixes, private rows,
    the runner's graph-padding rows (context 1, all -1), both plans; and at the batch sizes on
    either side of the device set's limit (2,048 sequences: every first block shared; 2,049: no
    set, every sequence streams)."""
    say("decode cache policy: device choice vs forced, two prefix groups + padding rows")
    step = make_step([700, 900, 260, 1100, 640, 850, 480, 2000, 33, 1, 1, 1], pool=640, seed=17)
    table = step.block_table.clone()
    table[1:4, :16] = table[0, :16]          # group A: 256 tokens of shared pages
    table[5:7, :8] = table[4, :8]            # group B: 128 tokens
    table[9:] = -1                           # graph-padding rows
    q, kc, vc = step.q.to(dev), step.k_cache.to(dev), step.v_cache.to(dev)
    tb, sl = table.to(dev), step.seqlen.to(dev)
    for split in (None, 512):
        outs = [gqa_decode_paged_fn(q, kc, vc, tb, sl, split_tokens=split, kv_reuse=r)
                for r in (None, True, False)]
        assert torch.equal(bits(outs[0]), bits(outs[1])), split
        assert torch.equal(bits(outs[0]), bits(outs[2])), split
        assert not bool(outs[0][9:].view(torch.int16).any())
    ref = ref_gqa_decode_paged(step.q[:9], step.k_cache, step.v_cache, table[:9],
                               step.seqlen[:9], 16)
    assert_decode_close(outs[0][:9], ref)
    for b, share in ((2048, True), (2049, False)):
        say(f"decode cache policy at batch {b}")
        big = make_step([17] * b, pool=2 * b, seed=18, device=dev)
        t = big.block_table.clone()
        if share:
            t[:, 0] = t[0, 0]
        res = [gqa_decode_paged_fn(big.q, big.k_cache, big.v_cache, t, big.seqlen, kv_reuse=r)
               for r in (None, True, False)]
        assert torch.equal(bits(res[0]), bits(res[1])) and torch.equal(bits(res[0]), bits(res[2]))


def test_block_permutation_and_padding_bitwise(dev):
    """Renaming physical blocks, or widening the table with -1 columns, changes no output bit."""
    say("decode block permutation / padding invariance")
    step = make_step([700, 1234, 65, 2048], pool=400, seed=8)
    base, _, _ = gpu_step(step, dev, append=False)
    g = torch.Generator().manual_seed(9)
    perm = torch.randperm(400, generator=g)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(400)
    kc2 = step.k_cache[inv]  # block j moves to perm[j]
    vc2 = step.v_cache[inv]
    tbl = step.block_table.clone()
    live = tbl >= 0
    tbl[live] = perm[tbl[live].long()].to(torch.int32)
    out2 = gqa_decode_paged_fn(step.q.to(dev), kc2.to(dev), vc2.to(dev), tbl.to(dev),
                               step.seqlen.to(dev))
    assert torch.equal(bits(base), bits(out2))
    wide = torch.full((4, tbl.shape[1] + 37), -1, dtype=torch.int32)
    wide[:, :tbl.shape[1]] = tbl
    out3 = gqa_decode_paged_fn(step.q.to(dev), kc2.to(dev), vc2.to(dev), wide.to(dev),
                               step.seqlen.to(dev), split_tokens=decode_plan(4, 24, 4, 256, 16, tbl.shape[1])[0])
    assert torch.equal(bits(base), bits(out3))


def test_invalid_block_ids_are_masked(dev):
    """A block id outside the cache at a used position is treated as absent (never read)."""
    say("decode invalid block ids")
    step = make_step([100, 100], pool=20, seed=4)
    tbl = step.block_table.clone()
    tbl[0, 2] = 10**6      # page 2 (tokens 32..47) of sequence 0 -> absent
    tbl[1, 0] = -5         # page 0 (tokens 0..15) of sequence 1 -> absent
    out = gqa_decode_paged_fn(step.q.to(dev), step.k_cache.to(dev), step.v_cache.to(dev),
                              tbl.to(dev), step.seqlen.to(dev))
    # Expected: attention over the remaining positions only (fp64, built by hand).
    kf = step.k_cache.float().reshape(-1, 4, 256)
    vf = step.v_cache.float().reshape(-1, 4, 256)
    for b, gone in ((0, range(32, 48)), (1, range(0, 16))):
        pos = [p for p in range(100) if p not in gone]
        rows = torch.tensor([int(step.block_table[b, p // 16]) * 16 + p % 16 for p in pos])
        k, v = kf[rows].double(), vf[rows].double()
        for h in range(24):
            s = k[:, h // 6] @ step.q[b, h].double() / 16.0
            w = torch.softmax(s, 0)
            torch.testing.assert_close(out[b, h].double().cpu(), w @ v[:, h // 6],
                                       atol=1e-2, rtol=1e-2)


def test_determinism_and_split_invariance(dev):
    say("decode determinism / split sizes")
    step = make_step([3000, 5000, 1, 4097], pool=900, seed=12)
    a, _, _ = gpu_step(step, dev, append=False)
    b, _, _ = gpu_step(step, dev, append=False)
    assert torch.equal(bits(a), bits(b))
    ref, _, _ = cpu_step(step, append=False)
    for split in (32, 64, 256, 1024, 2048, 8192):
        o, _, _ = gpu_step(step, dev, append=False, split_tokens=split)
        assert_decode_close(o, ref)


def test_fp16(dev):
    say("decode fp16")
    step = make_step([333, 1500], pool=150, seed=14, dtype=torch.float16)
    for variant in VARIANTS:
        out, _, _ = gpu_step(step, dev, variant=variant)
        ref, _, _ = cpu_step(step)
        assert out.dtype == torch.float16
        assert_decode_close(out, ref)


def test_long_context_32k(dev):
    """Two sequences of config 3's shape (32,768 tokens, randomly permuted blocks)."""
    say("decode 2 x 32768")
    step = make_step([32768, 32768], pool=4096, seed=1003)
    out, _, _ = gpu_step(step, dev)
    ref, _, _ = cpu_step(step)
    assert_decode_close(out, ref)


def test_one_long_sequence_many_parts(dev):
    """One 100,003-token sequence: the balanced plan cuts it into one part per workgroup (far more
    than 64), which the merge sums as ordered ranges, one per wave, the ragged tail tile included."""
    say("decode 1 x 100003")
    step = make_step([100003], pool=6300, seed=1010)
    out, _, _ = gpu_step(step, dev)
    ref, _, _ = cpu_step(step)
    assert_decode_close(out, ref)


def test_many_short_sequences(dev):
    """1,500 sequences of 0 to 300 tokens: each workgroup's run crosses many sequences; the merge
    finds each cut sequence's parts from the first-tile entries the partial kernel records, and
    writes the zero rows of the empty ones."""
    g = torch.Generator().manual_seed(1011)
    ctx = torch.randint(0, 301, (1500,), generator=g)
    ctx[::97] = 0
    ctx = ctx.tolist()
    say(f"decode 1500 short sequences, {sum(ctx)} tokens")
    step = make_step(ctx, pool=sum((c + 15) // 16 for c in ctx) + 16, seed=1011)
    out, _, _ = gpu_step(step, dev)
    ref, _, _ = cpu_step(step)
    assert_decode_close(out, ref)
    assert not bool(out[::97].float().abs().sum())


def test_graph_capture_replay(dev):
    """Append + decode captured in a HIP graph; every replay matches the eager result."""
    say("graph capture")
    step = make_step([900, 77, 2500], pool=300, seed=31)
    kc = step.k_cache.to(dev)
    vc = step.v_cache.to(dev)
    q = step.q.to(dev)
    kn, vn = step.k_new.to(dev), step.v_new.to(dev)
    slots = step.slot_mapping.to(dev)
    tbl = step.block_table.to(dev)
    seq = step.seqlen.to(dev)

    def fn():
        store_kvcache(kn, vn, flat(kc), flat(vc), slots)
        return gqa_decode_paged_fn(q, kc, vc, tbl, seq)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = fn()
    gen = torch.Generator(device=dev).manual_seed(2)
    for r in range(3):
        q.copy_(torch.randn(q.shape, generator=gen, device=dev).to(q.dtype))
        kn.copy_(torch.randn(kn.shape, generator=gen, device=dev).to(kn.dtype))
        graph.replay()
        torch.cuda.synchronize()
        eager = fn()
        torch.cuda.synchronize()
        assert torch.equal(bits(static_out), bits(eager)), f"replay {r}"


@pytest.mark.parametrize("page", [32, 48, 64])
def test_larger_pages_vs_oracle(page, dev):
    """Pages of 32, 48 and 64 rows: the same cache rows addressed through coarser page ids."""
    say(f"decode page_size={page}")
    g = torch.Generator().manual_seed(page)
    ctx = [5, page, page + 1, 3000]
    need = sum((n + page - 1) // page for n in ctx)
    perm = torch.randperm(need + 3, generator=g).to(torch.int32)
    width = max((n + page - 1) // page for n in ctx)
    table = torch.full((len(ctx), width), -1, dtype=torch.int32)
    at = 0
    for b, n in enumerate(ctx):
        k = (n + page - 1) // page
        table[b, :k] = perm[at:at + k]
        at += k
    kc = torch.randn(need + 3, page, 4, 256, generator=g).to(torch.bfloat16)
    vc = torch.randn(need + 3, page, 4, 256, generator=g).to(torch.bfloat16)
    q = torch.randn(len(ctx), 24, 256, generator=g).to(torch.bfloat16)
    seq = torch.tensor(ctx, dtype=torch.int32)
    out = gqa_decode_paged_fn(q.to(dev), kc.to(dev), vc.to(dev), table.to(dev), seq.to(dev), page)
    assert_decode_close(out, ref_gqa_decode_paged(q, kc, vc, table, seq, page))


@pytest.mark.parametrize("seed", range(200, 216))
def test_random_calls_vs_oracle(seed, dev):
    """Seeded random calls against the oracle: batch 1-6 with contexts 0-3,000, GQA groups 1-16,
    1-8 KV heads, head_dim 128/256, bf16/fp16, pages of 16/32/48 rows, the balanced plan and fixed
    splits, the MFMA and (groups 4, 6, 8) the scalar variants."""
    g = torch.Generator().manual_seed(seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=g))]  # noqa: E731
    hkv, group, d = pick([1, 2, 4, 8]), pick([1, 2, 3, 5, 6, 8, 11, 16]), pick([128, 256])
    dtype, page = pick([torch.bfloat16, torch.float16]), pick([16, 32, 48])
    unit = 32 * page // math.gcd(32, page)             # fixed splits are multiples of lcm(32, page)
    split = pick([None, None, unit, 8 * unit])
    batch = int(torch.randint(1, 7, (1,), generator=g))
    ctx = [int(torch.randint(0, 3001, (1,), generator=g)) for _ in range(batch)]
    say(f"decode random seed={seed} ctx={ctx} hkv={hkv} group={group} d={d} page={page} split={split}")
    need = sum((n + page - 1) // page for n in ctx)
    perm = torch.randperm(need + 3, generator=g).to(torch.int32)
    width = max(1, max((n + page - 1) // page for n in ctx))
    table = torch.full((len(ctx), width), -1, dtype=torch.int32)
    at = 0
    for b, n in enumerate(ctx):
        k = (n + page - 1) // page
        table[b, :k] = perm[at:at + k]
        at += k
    kc = torch.randn(need + 3, page, hkv, d, generator=g).to(dtype)
    vc = torch.randn(need + 3, page, hkv, d, generator=g).to(dtype)
    q = torch.randn(len(ctx), hkv * group, d, generator=g).to(dtype)
    seqlen = torch.tensor(ctx, dtype=torch.int32)
    ref = ref_gqa_decode_paged(q, kc, vc, table, seqlen, page)
    # The scalar variant is built for groups of 4, 6 and 8 only.
    for variant in VARIANTS if group in (4, 6, 8) else ["mfma"]:
        out = gqa_decode_paged_fn(q.to(dev), kc.to(dev), vc.to(dev), table.to(dev), seqlen.to(dev),
                                  page, split_tokens=split, variant=variant)
        assert_decode_close(out, ref)


def _shared_prefix_step(suffix, prefix, seed, hq=24, hkv=4, d=256, page=16):
    """A batch whose sequences share their first `prefix` tokens: the shared layout (every table
    aliases sequence 0's prefix pages) and a private one (each sequence has its own copy of the
    same values)."""
    g = torch.Generator().manual_seed(seed)
    ctx = [prefix + s for s in suffix]
    pp = prefix // page
    own = [(c + page - 1) // page - pp for c in ctx]
    pool = pp * (len(ctx) + 1) + sum(own) + 3
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    width = max(1, max((c + page - 1) // page for c in ctx))
    shared = torch.full((len(ctx), width), -1, dtype=torch.int32)
    private = shared.clone()
    kc = torch.randn(pool, page, hkv, d, generator=g).to(torch.bfloat16)
    vc = torch.randn(pool, page, hkv, d, generator=g).to(torch.bfloat16)
    at = pp
    prefix_ids = perm[:pp]
    for b in range(len(ctx)):
        shared[b, :pp] = prefix_ids
        private[b, :pp] = perm[at:at + pp]
        kc[perm[at:at + pp].long()] = kc[prefix_ids.long()]
        vc[perm[at:at + pp].long()] = vc[prefix_ids.long()]
        at += pp
        shared[b, pp:pp + own[b]] = perm[at:at + own[b]]
        private[b, pp:pp + own[b]] = perm[at:at + own[b]]
        at += own[b]
    q = torch.randn(len(ctx), hq, d, generator=g).to(torch.bfloat16)
    return q, kc, vc, shared, private, torch.tensor(ctx, dtype=torch.int32)


@pytest.mark.parametrize("suffix,prefix,split", [
    ([512] * 6, 2048, None),                     # config 5's shape, scaled down
    ([0, 1, 700, 33, 4000, 16], 1024, None),     # empty and short suffixes, one cut over many runs
    ([300, 300, 5], 512, 256),                   # a fixed split
    ([90] * 40, 4096, None),                     # many sequences, long prefix
    ([32] * 64, 1024, None),                     # every run covers two whole sequences
    ([20000, 3], 1024, None),                    # B = 2: a row of ~250 parts, the 8-wave merge
])
def test_shared_prefix_decode(suffix, prefix, split, dev):
    """shared_prefix_tokens: the prefix attended once for the batch and merged into each row —
    against the oracle and the plain call (tolerance), bitwise the same for the shared and the
    private layout, and (gated) bitwise the unfused gate."""
    say(f"decode shared prefix={prefix} suffix={suffix} split={split}")
    q, kc, vc, shared, private, seq = _shared_prefix_step(suffix, prefix, seed=prefix + len(suffix))
    ref = ref_gqa_decode_paged(q, kc, vc, shared, seq)
    d_q, d_kc, d_vc, d_seq = q.to(dev), kc.to(dev), vc.to(dev), seq.to(dev)
    run = lambda tbl, **kw: gqa_decode_paged_fn(d_q, d_kc, d_vc, tbl.to(dev), d_seq,  # noqa: E731
                                                split_tokens=split, **kw)
    out_shared = run(shared, shared_prefix_tokens=prefix, prefix_pass="always", kv_reuse=True)
    out_private = run(private, shared_prefix_tokens=prefix, prefix_pass="always")
    assert_decode_close(out_shared, ref)
    assert_decode_close(out_shared, run(shared))
    assert torch.equal(bits(out_shared), bits(out_private))
    gate = (2 * torch.randn(len(suffix), 1, 24 * 256, generator=torch.Generator().manual_seed(9))
            ).to(torch.bfloat16).to(dev)
    gated = run(shared, shared_prefix_tokens=prefix, prefix_pass="always", gate=gate)
    from tileinfer_amd.kernels import fused_sigmoid_mul
    assert torch.equal(bits(gated), bits(fused_sigmoid_mul(out_shared, gate.view_as(out_shared))))


def test_shared_prefix_zero_and_whole_context(dev):
    """shared_prefix_tokens=0 is the plain call (bitwise); a prefix that is some sequences' whole
    context leaves the decode kernel nothing for them (the prefix part alone)."""
    say("decode shared prefix edge cases")
    q, kc, vc, shared, _, seq = _shared_prefix_step([0, 0, 200], 640, seed=5)
    args = (q.to(dev), kc.to(dev), vc.to(dev), shared.to(dev), seq.to(dev))
    plain = gqa_decode_paged_fn(*args)
    assert torch.equal(bits(gqa_decode_paged_fn(*args, shared_prefix_tokens=0)), bits(plain))
    # Three sequences are below the prefix pass's break-even: "auto" is the plain call, bitwise.
    assert torch.equal(bits(gqa_decode_paged_fn(*args, shared_prefix_tokens=640)), bits(plain))
    assert_decode_close(gqa_decode_paged_fn(*args, shared_prefix_tokens=640, prefix_pass="always"),
                        ref_gqa_decode_paged(q, kc, vc, shared, seq))
    with pytest.raises(ValueError):
        gqa_decode_paged_fn(*args, shared_prefix_tokens=640, prefix_pass="never")
    with pytest.raises(ValueError):
        gqa_decode_paged_fn(*args, shared_prefix_tokens=100)        # not a page multiple
    with pytest.raises(ValueError):
        gqa_decode_paged_fn(*args, shared_prefix_tokens=640, variant="scalar")


def test_shared_prefix_graph_capture_replay(dev):
    """The shared-prefix decode (prefix pass + suffix decode + merge) captured in a HIP graph after
    a warm-up call: every replay matches the eager call bitwise."""
    say("decode shared prefix graph capture")
    q, kc, vc, shared, _, seq = _shared_prefix_step([300, 17, 900], 1024, seed=12)
    q = q.to(dev)
    args = (kc.to(dev), vc.to(dev), shared.to(dev), seq.to(dev))

    def fn():
        return gqa_decode_paged_fn(q, *args, kv_reuse=True, shared_prefix_tokens=1024,
                                   prefix_pass="always")

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = fn()
    gen = torch.Generator(device=dev).manual_seed(4)
    for r in range(3):
        q.copy_(torch.randn(q.shape, generator=gen, device=dev).to(q.dtype))
        graph.replay()
        torch.cuda.synchronize()
        eager = fn()
        torch.cuda.synchronize()
        assert torch.equal(bits(static_out), bits(eager)), f"replay {r}"


@pytest.mark.parametrize("ctx,waves", [
    ([40000] + [300] * 7, 4),       # B = 8: the long rows cut into ~230 parts, 4-wave merge
    ([20000] + [200] * 31, 4),      # B = 32 (768 rows): the 4-wave merge's largest batch
    ([24000] + [200] * 39, 2),      # B = 40: 2 waves per row, ~190 parts
    ([24000] + [200] * 79, 1),      # B = 80 (1,920 rows): one wave, ~150 parts in bursts of 16
])
def test_one_long_sequence_among_short_ones(ctx, waves, dev):
    """A batch whose first sequence holds most of the tiles: the balanced plan cuts its rows into
    more than 64 parts whatever the batch size, and the merge sums them with 4 waves per row up
    to 768 rows (q-heads x sequences), 2 up to 1,536 and one above (8 up to 96 rows, tested
    elsewhere). Against the oracle."""
    step = make_step(ctx, pool=sum((c + 15) // 16 for c in ctx) + 8, seed=73 + len(ctx))
    tiles = [(c + 15) // 16 for c in ctx]
    split, wgs, _ = decode_plan(len(ctx), 24, 4, 256, 16, step.block_table.shape[1])
    chunk = max(-(-sum(tiles) // wgs), 4)
    parts = -(-tiles[0] // chunk)
    say(f"decode one long sequence: B={len(ctx)}, long row {ctx[0]} tokens in ~{parts} parts, "
        f"{waves}-wave merge")
    assert split == 0 and parts > 64
    out, _, _ = gpu_step(step, dev)
    ref, _, _ = cpu_step(step)
    assert_decode_close(out, ref)
