"""Seeded synthetic inputs of the paged KV-cache benchmark configurations.

Shapes follow the model the reference serves (24 query heads, 4 KV heads, head_dim 256, block
size 16, bf16). Every builder takes a ``torch.Generator`` seed and a device; values are drawn on
that device, so CPU-generated inputs copied to the GPU are identical to what a CPU checker sees.

A decode step of one attention layer is: append the new token of each sequence through
``slot_mapping`` (its position is ``ctx - 1``), then decode with ``seqlen = ctx``
(model/qwen_36.py:1018 then 1074).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

HQ, HKV, HEAD_DIM, BLOCK = 24, 4, 256, 16


@dataclass
class PagedStep:
    """One attention layer's inputs for append + decode."""
    q: torch.Tensor             # [B, HQ, D]
    k_new: torch.Tensor         # [N, HKV, D]
    v_new: torch.Tensor         # [N, HKV, D]
    slot_mapping: torch.Tensor  # [N] int32
    block_table: torch.Tensor   # [B, W] int32, -1 padded
    seqlen: torch.Tensor        # [B] int32 (after the append)
    k_cache: torch.Tensor       # [num_blocks, BLOCK, HKV, D]
    v_cache: torch.Tensor
    page_size: int = BLOCK
    meta: dict = field(default_factory=dict)

    def append_bytes(self) -> int:
        return append_bytes(self.slot_mapping, self.k_new.shape[1] * self.k_new.shape[2],
                            self.k_new.element_size())

    def decode_bytes(self) -> int:
        return decode_bytes(self.seqlen.tolist(), self.q.shape[1], self.k_cache.shape[2],
                            self.q.shape[2], self.page_size, self.q.element_size())


def append_bytes(slot_mapping: torch.Tensor, row_elems: int, elem: int = 2) -> int:
    """Algorithmic bytes of an append: read + write K and V rows of valid slots, read the slots."""
    n_valid = int((slot_mapping >= 0).sum())
    return 4 * row_elems * elem * n_valid + 4 * slot_mapping.numel()


def decode_bytes(ctx: list[int], hq: int = HQ, hkv: int = HKV, d: int = HEAD_DIM,
                 page_size: int = BLOCK, elem: int = 2) -> int:
    """Algorithmic bytes of a decode: K+V rows, q in and out, block-table entries, seqlens."""
    tot = sum(ctx)
    pages = sum((c + page_size - 1) // page_size for c in ctx)
    return 2 * hkv * d * elem * tot + 2 * hq * d * elem * len(ctx) + 4 * pages + 4 * len(ctx)


def decode_flops(ctx: list[int], hq: int = HQ, d: int = HEAD_DIM) -> int:
    return 4 * hq * d * sum(ctx)


def _randn(shape, gen, device, dtype, scale=1.0):
    x = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    if scale != 1.0:
        x.mul_(scale)
    return x.to(dtype)


def tables_from_pool(ctx: list[int], pool: int, gen: torch.Generator, device,
                     width: int | None = None, page: int = BLOCK) -> torch.Tensor:
    """Disjoint random physical blocks per sequence, drawn from randperm(pool); -1 padded."""
    need = [(c + page - 1) // page for c in ctx]
    if sum(need) > pool:
        raise ValueError(f"pool {pool} < {sum(need)} blocks needed")
    perm = torch.randperm(pool, generator=gen, device=device).to(torch.int32)
    w = max(need) if width is None else width
    table = torch.full((len(ctx), w), -1, dtype=torch.int32, device=device)
    off = 0
    for i, n in enumerate(need):
        table[i, :n] = perm[off:off + n]
        off += n
    return table


def decode_slots(table: torch.Tensor, ctx: list[int], page: int = BLOCK) -> torch.Tensor:
    """Slot of the token at position ctx-1 of every sequence (-1 for an empty sequence)."""
    pos = torch.tensor([max(c - 1, 0) for c in ctx], dtype=torch.int64)
    rows = table.cpu()[torch.arange(len(ctx)), pos // page].long()
    slots = rows * page + pos % page
    slots[torch.tensor([c <= 0 for c in ctx], dtype=torch.bool)] = -1
    return slots.to(torch.int32).to(table.device)


def make_step(ctx: list[int], pool: int, seed: int, device="cpu", dtype=torch.bfloat16,
              value_scale: float = 1.0, width: int | None = None, hq: int = HQ, hkv: int = HKV,
              d: int = HEAD_DIM, page: int = BLOCK) -> PagedStep:
    """Random tables over a pool of `pool` pages of `page` tokens ([pool, page, hkv, d] caches)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    table = tables_from_pool(ctx, pool, gen, device, width, page)
    k_cache = _randn((pool, page, hkv, d), gen, device, dtype, value_scale)
    v_cache = _randn((pool, page, hkv, d), gen, device, dtype, value_scale)
    b = len(ctx)
    q = _randn((b, hq, d), gen, device, dtype, value_scale)
    k_new = _randn((b, hkv, d), gen, device, dtype, value_scale)
    v_new = _randn((b, hkv, d), gen, device, dtype, value_scale)
    return PagedStep(q=q, k_new=k_new, v_new=v_new, slot_mapping=decode_slots(table, ctx, page),
                     block_table=table, seqlen=torch.tensor(ctx, dtype=torch.int32, device=device),
                     k_cache=k_cache, v_cache=v_cache, page_size=page,
                     meta={"seed": seed, "ctx": list(ctx)})


def config1(seed: int = 1001, device="cpu", ctx: int = 512) -> PagedStep:
    """One sequence, 64-block pool, table = randperm(64), values N(0,1)/sqrt(256)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    perm = torch.randperm(64, generator=gen, device=device).to(torch.int32)
    s = 1.0 / math.sqrt(HEAD_DIM)
    k_cache = _randn((64, BLOCK, HKV, HEAD_DIM), gen, device, torch.bfloat16, s)
    v_cache = _randn((64, BLOCK, HKV, HEAD_DIM), gen, device, torch.bfloat16, s)
    q = _randn((1, HQ, HEAD_DIM), gen, device, torch.bfloat16, s)
    k_new = _randn((1, HKV, HEAD_DIM), gen, device, torch.bfloat16, s)
    v_new = _randn((1, HKV, HEAD_DIM), gen, device, torch.bfloat16, s)
    table = perm.view(1, 64)
    return PagedStep(q=q, k_new=k_new, v_new=v_new, slot_mapping=decode_slots(table, [ctx]),
                     block_table=table, seqlen=torch.tensor([ctx], dtype=torch.int32, device=device),
                     k_cache=k_cache, v_cache=v_cache, meta={"seed": seed, "ctx": [ctx]})


def config2(seed: int = 1002, device="cpu", batch: int = 16, lo: int = 512,
            hi: int = 8192) -> PagedStep:
    """Batch 16, ctx ~ U[512, 8192], pool 1.25x the blocks needed, values N(0,1)."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    ctx = torch.randint(lo, hi + 1, (batch,), generator=gen).tolist()
    need = sum((c + BLOCK - 1) // BLOCK for c in ctx)
    return make_step(ctx, math.ceil(1.25 * need), seed, device)


def config3(seed: int = 1003, device="cpu", batch: int = 64, ctx: int = 32768) -> PagedStep:
    """One layer of batch 64 x 32k context; tables are one randperm of the pool split per sequence."""
    need = batch * ((ctx + BLOCK - 1) // BLOCK)
    return make_step([ctx] * batch, need, seed, device)


def config4(seed: int = 1004, device="cpu", chunk: int = 2048, batch: int = 32, lo: int = 1024,
            hi: int = 16384):
    """Mixed step: a 2048-token prefill chunk over 128 non-contiguous blocks + 32 decode tokens.

    Returns (step, chunk_slots): ``step`` is the decode batch with its 32 appended tokens;
    ``chunk_slots``/``step.meta['chunk_k']``/``['chunk_v']`` are the prefill chunk's append.
    """
    gen = torch.Generator(device="cpu").manual_seed(seed)
    ctx = torch.randint(lo, hi + 1, (batch,), generator=gen).tolist()
    need = sum((c + BLOCK - 1) // BLOCK for c in ctx)
    chunk_blocks = chunk // BLOCK
    pool = math.ceil(1.25 * (need + chunk_blocks))
    step = make_step(ctx, pool, seed, device)
    used = set(step.block_table[step.block_table >= 0].cpu().tolist())
    free = [i for i in range(pool) if i not in used]
    g2 = torch.Generator(device="cpu").manual_seed(seed + 1)
    pick = torch.randperm(len(free), generator=g2)[:chunk_blocks].tolist()
    blocks = torch.tensor([free[i] for i in pick], dtype=torch.int64)
    pos = torch.arange(chunk)
    chunk_slots = (blocks[pos // BLOCK] * BLOCK + pos % BLOCK).to(torch.int32).to(device)
    gd = torch.Generator(device=device).manual_seed(seed + 2)
    step.meta["chunk_k"] = _randn((chunk, HKV, HEAD_DIM), gd, device, torch.bfloat16)
    step.meta["chunk_v"] = _randn((chunk, HKV, HEAD_DIM), gd, device, torch.bfloat16)
    step.meta["chunk_blocks"] = blocks.tolist()
    return step, chunk_slots


def config5(seed: int = 1005, device="cpu", batch: int = 128, prefix: int = 8192,
            suffix: int = 512, shared: bool = True) -> PagedStep:
    """128 sequences whose tables alias one 8192-token prefix (512 blocks) + 512 own tokens.

    ``shared=False`` builds the same logical contents with every sequence holding a private copy
    of the prefix blocks (same values, different physical ids), for the shared-vs-private check.
    """
    pb, sb = prefix // BLOCK, suffix // BLOCK
    gen = torch.Generator(device=device).manual_seed(seed)
    pool_shared = pb + batch * sb
    pool = pool_shared if shared else batch * (pb + sb)
    kp = _randn((pb, BLOCK, HKV, HEAD_DIM), gen, device, torch.bfloat16)
    vp = _randn((pb, BLOCK, HKV, HEAD_DIM), gen, device, torch.bfloat16)
    ks = _randn((batch * sb, BLOCK, HKV, HEAD_DIM), gen, device, torch.bfloat16)
    vs = _randn((batch * sb, BLOCK, HKV, HEAD_DIM), gen, device, torch.bfloat16)
    q = _randn((batch, HQ, HEAD_DIM), gen, device, torch.bfloat16)
    k_new = _randn((batch, HKV, HEAD_DIM), gen, device, torch.bfloat16)
    v_new = _randn((batch, HKV, HEAD_DIM), gen, device, torch.bfloat16)
    k_cache = torch.empty((pool, BLOCK, HKV, HEAD_DIM), dtype=torch.bfloat16, device=device)
    v_cache = torch.empty_like(k_cache)
    table = torch.empty((batch, pb + sb), dtype=torch.int32, device=device)
    if shared:
        k_cache[:pb], v_cache[:pb] = kp, vp
        k_cache[pb:], v_cache[pb:] = ks, vs
        table[:, :pb] = torch.arange(pb, dtype=torch.int32, device=device)
        table[:, pb:] = (pb + torch.arange(batch * sb, dtype=torch.int32, device=device)).view(batch, sb)
    else:
        for i in range(batch):
            base = i * (pb + sb)
            k_cache[base:base + pb], v_cache[base:base + pb] = kp, vp
            k_cache[base + pb:base + pb + sb] = ks[i * sb:(i + 1) * sb]
            v_cache[base + pb:base + pb + sb] = vs[i * sb:(i + 1) * sb]
            table[i] = base + torch.arange(pb + sb, dtype=torch.int32, device=device)
    ctx = [prefix + suffix] * batch
    return PagedStep(q=q, k_new=k_new, v_new=v_new, slot_mapping=decode_slots(table, ctx),
                     block_table=table, seqlen=torch.tensor(ctx, dtype=torch.int32, device=device),
                     k_cache=k_cache, v_cache=v_cache,
                     meta={"seed": seed, "ctx": ctx, "shared": shared, "prefix_tokens": prefix})


@dataclass
class ManagedBatch:
    """A batch whose blocks a ``PagedKVManager`` owns, over an all-layer cache slab."""
    manager: "object"           # tileinfer_amd.engine.PagedKVManager
    seqs: list                  # [Sequence]
    kv: torch.Tensor            # [2, L, pool, BLOCK, HKV, D]
    q: torch.Tensor             # [L, B, HQ, D]

    def tables(self) -> tuple[torch.Tensor, torch.Tensor]:
        """(block_table [B, W] int32 with -1 padding, seqlen [B] int32) on the cache's device,
        built from the sequences' current tables (W = the longest)."""
        w = max(len(s.block_table) for s in self.seqs)
        table = torch.full((len(self.seqs), w), -1, dtype=torch.int32)
        for i, s in enumerate(self.seqs):
            table[i, :len(s.block_table)] = torch.tensor(s.block_table, dtype=torch.int32)
        seqlen = torch.tensor([s.num_tokens for s in self.seqs], dtype=torch.int32)
        return table.to(self.kv.device), seqlen.to(self.kv.device)


def config5_managed(device="cuda", layers: int = 16, batch: int = 128, prefix: int = 8192,
                    suffix: int = 512, seed: int = 1005, swap_fraction: float = 0.25,
                    dtype=torch.bfloat16) -> ManagedBatch:
    """Config 5 set up the way a serving engine gets there: sequence 0's prompt is computed and
    its whole-block prefix recorded in the prefix cache; the other sequences share those
    ``prefix / 16`` blocks through the cache hit (``share_blocks``, refcounted) and own ``suffix
    / 16`` blocks each. The pool holds exactly the physical blocks (512 + 128 x 32 = 4,608) and a
    pinned host pool the blocks of ``swap_fraction`` of the sequences (1,024). All ``layers``
    layers' K/V are N(0,1) values (the stand-in for the prefill), q one [B, 24, 256] per layer."""
    from .engine import PagedKVManager, Sequence
    from .engine.kv_layout import allocate_kv_cache

    pb, sb = prefix // BLOCK, suffix // BLOCK
    pool = pb + batch * sb
    host_blocks = int(batch * swap_fraction) * sb
    m = PagedKVManager(pool, BLOCK, enable_prefix_caching=True, num_host_blocks=host_blocks)
    shared = list(range(prefix))
    seqs = []
    for i in range(batch):
        own = [prefix + 1 + i * suffix + j for j in range(suffix)]
        s = Sequence(shared + own)
        if not m.admit(s):
            raise RuntimeError("config5_managed: pool too small")
        if i == 0:
            m.finish_chunk(s, prefix)            # whole-block prefix recorded here
        m.finish_chunk(s, s.num_tokens - s.num_cached_tokens)
        seqs.append(s)
    if any(s.block_table[:pb] != seqs[0].block_table[:pb] for s in seqs[1:]):
        raise AssertionError("config5_managed: the prefix was not shared")
    kv = allocate_kv_cache(layers, pool, BLOCK, HKV, HEAD_DIM, device, dtype, zero=False)
    gen = torch.Generator(device=device).manual_seed(seed)
    kv.normal_(generator=gen)
    q = _randn((layers, batch, HQ, HEAD_DIM), gen, device, dtype)
    return ManagedBatch(manager=m, seqs=seqs, kv=kv, q=q)


@dataclass
class PrefillStep:
    """One attention layer's chunked-prefill inputs: packed query rows over paged K/V.

    Sequence b owns query rows ``cu_seqlens_q[b]:cu_seqlens_q[b+1]`` (its chunk) and has
    ``seqlen_k[b]`` tokens in the cache, the chunk's own K/V included (already appended).
    """
    q: torch.Tensor             # [total_q, HQ, D]
    block_table: torch.Tensor   # [B, W] int32, -1 padded
    cu_seqlens_q: torch.Tensor  # [B + 1] int32
    seqlen_k: torch.Tensor      # [B] int32
    k_cache: torch.Tensor       # [num_blocks, BLOCK, HKV, D]
    v_cache: torch.Tensor
    max_seqlen_q: int = 0
    page_size: int = BLOCK
    meta: dict = field(default_factory=dict)

    def flops(self) -> int:
        return prefill_flops(self.q_lens(), self.seqlen_k.tolist(), self.q.shape[1],
                             self.q.shape[2])

    def q_lens(self) -> list[int]:
        cu = self.cu_seqlens_q.tolist()
        return [cu[i + 1] - cu[i] for i in range(len(cu) - 1)]


def prefill_visible(q_len: int, kv_len: int, causal: bool = True) -> int:
    """Number of (query, key) pairs a chunk attends over: query i sees keys
    ``0..kv_len - q_len + i`` under the bottom-right causal mask."""
    if not causal:
        return q_len * kv_len
    off = kv_len - q_len
    return sum(max(0, min(kv_len, off + i + 1)) for i in range(q_len))


def prefill_flops(q_lens: list[int], kv_lens: list[int], hq: int = HQ, d: int = HEAD_DIM,
                  causal: bool = True) -> int:
    """Algorithmic flops of the chunks' attention: 2·D for Q·K and 2·D for P·V per visible pair."""
    return 4 * hq * d * sum(prefill_visible(a, b, causal) for a, b in zip(q_lens, kv_lens))


def prefill_step(q_lens: list[int], kv_lens: list[int], seed: int, device="cpu",
                 pool: int | None = None, dtype=torch.bfloat16, value_scale: float = 1.0,
                 hq: int = HQ, hkv: int = HKV, d: int = HEAD_DIM,
                 width: int | None = None, page: int = BLOCK) -> PrefillStep:
    """Random non-contiguous tables from a pool (1.25x the need by default), N(0,1)·scale values;
    pages of `page` tokens."""
    if len(q_lens) != len(kv_lens):
        raise ValueError("q_lens and kv_lens differ in length")
    need = sum((c + page - 1) // page for c in kv_lens)
    pool = max(1, math.ceil(1.25 * need)) if pool is None else pool
    gen = torch.Generator(device=device).manual_seed(seed)
    table = tables_from_pool(kv_lens, pool, gen, device, width, page)
    k_cache = _randn((pool, page, hkv, d), gen, device, dtype, value_scale)
    v_cache = _randn((pool, page, hkv, d), gen, device, dtype, value_scale)
    cu = [0]
    for n in q_lens:
        cu.append(cu[-1] + n)
    q = _randn((cu[-1], hq, d), gen, device, dtype, value_scale)
    return PrefillStep(q=q, block_table=table,
                       cu_seqlens_q=torch.tensor(cu, dtype=torch.int32, device=device),
                       seqlen_k=torch.tensor(kv_lens, dtype=torch.int32, device=device),
                       k_cache=k_cache, v_cache=v_cache, max_seqlen_q=max(q_lens, default=0),
                       page_size=page,
                       meta={"seed": seed, "q_lens": list(q_lens), "kv_lens": list(kv_lens)})


def config4_prefill(seed: int = 1004, device="cpu", chunk: int = 2048,
                    cached: int = 0) -> PrefillStep:
    """Config 4's prefill chunk as attention input: ``chunk`` query tokens over ``cached + chunk``
    tokens held in random non-contiguous blocks (``cached = 0``: the first chunk, 128 blocks)."""
    return prefill_step([chunk], [cached + chunk], seed, device)
