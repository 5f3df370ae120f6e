"""Block manager, prefix cache, sharing flow and metadata builders (CPU, pure Python).

Expected block ids are derived by hand from the reference's rules: a fresh pool hands out 0, 1,
2, ... (free list [n-1..0] popped from the end, engine/block_manager.py:33, 45), freed blocks are
reused last-in first-out, and deallocation walks a table in reverse (engine/block_manager.py:95).
"""
import numpy as np
import pytest
import torch
from hypothesis import example, given, settings
from hypothesis import strategies as st

from tileinfer_amd.engine import (AttentionContext, BlockManager, PagedKVManager, PrefixCache,
                                  Sequence, get_context, reset_context, set_context)
from tileinfer_amd.engine import kv_layout as kl


@pytest.fixture(autouse=True)
def _bs16():
    Sequence.block_size = 16
    yield
    Sequence.block_size = 16


def seq(n, start=0):
    return Sequence(list(range(start, start + n)))


# ----------------------------------------------------------------------------- sequence


def test_sequence_layout_fields():
    s = seq(33)
    assert len(s) == 33 and s.num_blocks == 3 and s.last_block_num_tokens == 1
    assert s.block(2) == [32]
    s.append_token(99)
    assert s.num_tokens == 34 and s.last_token == 99 and s.num_prompt_tokens == 33
    with pytest.raises(ValueError):
        Sequence([])
    with pytest.raises(IndexError):
        s.block(3)


# ----------------------------------------------------------------------------- block manager


def test_allocation_order_and_lifo_reuse():
    bm = BlockManager(8, 16)
    a, b = seq(40), seq(17)
    bm.allocate(a)
    bm.allocate(b)
    assert a.block_table == [0, 1, 2] and b.block_table == [3, 4]
    assert bm.num_free_blocks == 3
    freed = bm.deallocate(a)
    assert freed == [2, 1, 0] and a.block_table == []
    c = seq(48)
    bm.allocate(c)
    assert c.block_table == [0, 1, 2]  # last freed (0) comes back first


def test_share_blocks_refcounts_and_release():
    bm = BlockManager(6, 16)
    events = []
    bm.on_block_freed = events.append
    a = seq(32)
    bm.allocate(a)
    b = seq(40)
    bm.share_blocks(b, a.block_table[:2])
    bm.allocate_extra(b)
    assert b.block_table == [0, 1, 2]
    assert [bm.blocks[i].ref_count for i in range(3)] == [2, 2, 1]
    assert bm.deallocate(a) == [] and events == []
    assert bm.deallocate(b) == [2, 1, 0] and events == [2, 1, 0]
    assert bm.num_free_blocks == 6
    with pytest.raises(ValueError):
        bm.share_blocks(seq(1), [5])  # a free block cannot be shared


def test_may_append_reference_trigger_and_capacity_fix():
    bm = BlockManager(10, 16)
    a = seq(20)                     # 2 blocks: 0, 1
    bm.allocate(a)
    while len(a) < 31:
        a.append_token(0)
        bm.may_append(a)
    assert a.block_table == [0, 1]
    a.append_token(0)               # len 32: the reference allocates one block ahead
    assert bm.can_append(a)
    bm.may_append(a)
    assert a.block_table == [0, 1, 2]
    b = seq(16)                     # prompt a multiple of 16: block 3
    bm.allocate(b)
    b.append_token(0)               # len 17: position 16 needs a second block (reference misses it)
    bm.may_append(b)
    assert b.block_table == [3, 4]
    assert len(b.block_table) * 16 >= len(b)


def test_can_append_on_exhausted_pool():
    bm = BlockManager(1, 16)
    a = seq(16)
    bm.allocate(a)
    a.append_token(0)
    assert not bm.can_append(a)
    with pytest.raises(RuntimeError):
        bm.may_append(a)


# ----------------------------------------------------------------------------- prefix cache


def test_prefix_cache_whole_blocks_only():
    pc = PrefixCache(4)
    toks = list(range(10))
    pc.add(toks, [7, 8, 9])
    assert pc.num_entries == 2                              # boundaries at 4 and 8 tokens
    assert pc.find_longest_prefix(toks) == ([7, 8], 8)
    assert pc.find_longest_prefix(toks[:7]) == ([7], 4)
    assert pc.find_longest_prefix([0, 1, 2, 99, 4]) == ([], 0)
    pc.add(toks, [7, 8, 9])                                 # idempotent
    assert pc.num_entries == 2


def test_prefix_cache_position_sensitive():
    pc = PrefixCache(2)
    pc.add([1, 2, 3, 4], [10, 11])
    assert pc.find_longest_prefix([3, 4, 1, 2]) == ([], 0)  # same tokens, other position


def test_prefix_cache_eviction_invalidates_subtree():
    pc = PrefixCache(2)
    pc.add([1, 2, 3, 4, 5, 6], [10, 11, 12])
    pc.add([1, 2, 7, 8], [10, 13])
    assert pc.num_entries == 4
    pc.evict_block(11)                 # chain [10, 11] and its child [10, 11, 12] go
    assert pc.find_longest_prefix([1, 2, 3, 4, 5, 6]) == ([10], 2)
    assert pc.find_longest_prefix([1, 2, 7, 8]) == ([10, 13], 4)
    assert pc.num_entries == 2
    pc.evict_block(10)
    assert pc.find_longest_prefix([1, 2, 7, 8]) == ([], 0)
    assert pc.num_entries == 0


def test_prefix_cache_trim():
    pc = PrefixCache(1, max_entries=2)
    pc.add([1, 2, 3], [5, 6, 7])
    assert pc.num_entries == 2


# ----------------------------------------------------------------------------- sharing flow


def test_manager_prefix_hit_shares_and_allocates_rest():
    m = PagedKVManager(20, 16)
    a = Sequence(list(range(40)))
    assert m.admit(a) and a.block_table == [0, 1, 2]
    m.finish_chunk(a, 32)                      # 32 tokens computed: 2 whole blocks recorded
    b = Sequence(list(range(32)) + [100] * 10)
    assert m.admit(b)
    assert b.block_table[:2] == [0, 1] and b.num_cached_tokens == 32 and b.block_table[2] == 3
    assert m.block_manager.blocks[0].ref_count == 2
    m.free(a)
    m.free(b)
    assert m.prefix_cache.num_entries == 0     # blocks 0, 1 freed -> entries evicted
    assert m.block_manager.num_free_blocks == 20


def test_manager_shares_blocks_hint():
    m = PagedKVManager(20, 16)
    a = Sequence(list(range(40)))
    m.admit(a)
    assert not m.shares_blocks([a])
    m.finish_chunk(a, 32)
    b = Sequence(list(range(32)) + [7] * 9)
    m.admit(b)
    c = Sequence([5] * 20)
    m.admit(c)
    assert m.shares_blocks([a, b]) and m.shares_blocks([b]) and not m.shares_blocks([c])


def test_manager_common_prefix_tokens():
    """The whole blocks every sequence of a batch holds in common (the shared_prefix_tokens of a
    decode over it): 2 blocks for a and b, none once c joins, none for a single sequence."""
    m = PagedKVManager(20, 16)
    a = Sequence(list(range(40)))
    m.admit(a)
    m.finish_chunk(a, 32)
    b = Sequence(list(range(32)) + [7] * 9)
    m.admit(b)
    c = Sequence([5] * 20)
    m.admit(c)
    assert m.common_prefix_tokens([a, b]) == 32
    assert m.common_prefix_tokens([a, b, c]) == 0
    assert m.common_prefix_tokens([a]) == 0


def test_manager_full_prefix_match_leaves_a_token_to_prefill():
    m = PagedKVManager(10, 16)
    a = Sequence(list(range(32)))
    m.admit(a)
    m.finish_chunk(a, 32)
    b = Sequence(list(range(32)))
    assert m.admit(b)
    assert b.num_cached_tokens == 16 and b.block_table[0] == 0 and b.block_table[1] != 1


def test_manager_admission_fails_without_room():
    m = PagedKVManager(2, 16)
    assert not m.admit(Sequence(list(range(40))))
    assert m.block_manager.num_free_blocks == 2


@settings(max_examples=60, deadline=None)
@given(st.lists(st.tuples(st.sampled_from(["admit", "decode", "free"]),
                          st.integers(0, 5), st.integers(1, 70)), max_size=40))
def test_manager_invariants(ops):
    """Refcounts equal table membership, the free list is the complement of used blocks, and no
    two live sequences write the same slot."""
    m = PagedKVManager(24, 16)
    live: dict[int, Sequence] = {}
    prompts = [list(range(40)), list(range(40)) + [1, 2], list(range(17)), [9] * 50]
    for op, k, n in ops:
        if op == "admit" and k not in live:
            s = Sequence((prompts[k % 4] * 3)[:n])
            if m.admit(s):
                m.finish_chunk(s, s.num_tokens - s.num_cached_tokens)
                s.is_prefill = False
                live[k] = s
        elif op == "decode" and k in live:
            s = live[k]
            s.append_token(n)
            if m.can_append(s):
                m.append_slot(s)
            else:
                m.free(s)
                del live[k]
        elif op == "free" and k in live:
            m.free(live.pop(k))
        bm = m.block_manager
        counts = {}
        for s in live.values():
            assert len(s.block_table) * 16 >= len(s)
            for bid in s.block_table:
                counts[bid] = counts.get(bid, 0) + 1
        for bid in range(24):
            assert bm.blocks[bid].ref_count == counts.get(bid, 0)
        assert set(bm.free_block_ids) == set(range(24)) - set(counts)
        slots = [s.block_table[(len(s) - 1) // 16] * 16 + (len(s) - 1) % 16 for s in live.values()]
        assert len(slots) == len(set(slots))


# ----------------------------------------------------------------------------- builders


def test_slot_mappings_match_definition():
    a, b = seq(37), seq(5)
    a.block_table = [9, 4, 7]
    b.block_table = [2]
    got = kl.slot_mapping_decode([a, b], 16)
    assert got.tolist() == [7 * 16 + 4, 2 * 16 + 4]
    a.num_cached_tokens, a.num_scheduled_tokens = 14, 20
    b.num_cached_tokens, b.num_scheduled_tokens = 0, 5
    got = kl.slot_mapping_prefill([a, b], 16)
    want = [a.block_table[p // 16] * 16 + p % 16 for p in range(14, 34)] + [32, 33, 34, 35, 36]
    assert got.tolist() == want and got.dtype == np.int32
    a.num_scheduled_tokens = 40
    with pytest.raises(IndexError):
        kl.slot_mapping_prefill([a], 16)


def test_block_tables_and_graph_padding():
    a, b = seq(37), seq(5)
    a.block_table, b.block_table = [9, 4, 7], [2]
    t = kl.block_tables([a, b])
    assert t.tolist() == [[9, 4, 7], [2, -1, -1]]
    slots, tables, ctx = kl.decode_metadata([a, b], 16, device="cpu", pad_to=4, width=5)
    assert slots.tolist() == [7 * 16 + 4, 36, -1, -1]
    assert ctx.tolist() == [37, 5, 1, 1]
    assert tables.tolist() == [[9, 4, 7, -1, -1], [2, -1, -1, -1, -1], [-1] * 5, [-1] * 5]
    assert tables.dtype == torch.int32 and slots.dtype == torch.int32


def test_kv_cache_layout_views():
    kv = kl.allocate_kv_cache(3, 5, 16, 4, 8, device="cpu")
    assert tuple(kv.shape) == (2, 3, 5, 16, 4, 8)
    k_rows, v_rows, k_paged, v_paged = kl.layer_views(kv, 1)
    assert tuple(k_rows.shape) == (80, 32) and tuple(k_paged.shape) == (5, 16, 4, 8)
    k_rows[17, 9] = 1.0                                    # the views alias the slab
    assert float(kv[0, 1, 1, 1, 1, 1]) == 1.0
    v_paged[0, 0, 0, 0] = 2.0
    assert float(v_rows[0, 0]) == 2.0
    assert kl.num_blocks_for_budget(2 * 16 * 4 * 8 * 2 * 3 * 10 + 5, 16, 4, 8, 3) == 10


def test_pool_sizing_from_free_memory():
    """The runner's sizing (engine/model_runner.py:218-256): budget = total·util − used − other
    pools; blocks = budget // bytes per block id over K, V and every attention layer (at least 1);
    the table width is max_model_len // 16 + 2, clamped to the pool."""
    gib = 2**30
    # 288 GiB card, 20 GiB in use (weights), 90 % target, 4 GiB of other pools.
    budget = kl.kv_budget(288 * gib, 268 * gib, 0.9, reserved_bytes=4 * gib)
    assert budget == int(288 * gib * 0.9) - 20 * gib - 4 * gib
    per_block = 2 * 16 * 4 * 256 * 2 * 16                  # K+V x 16 rows x 4 heads x 256 x bf16 x 16 layers
    assert kl.block_bytes(16, 4, 256, 16) == per_block == 1 << 20
    nb = kl.num_blocks_for_budget(budget, 16, 4, 256, 16)
    assert nb == budget // per_block and nb == 240_844    # 235.2 GiB of 1 MiB blocks
    assert kl.num_blocks_for_budget(-5, 16, 4, 256, 16) == 1
    assert kl.max_blocks_per_seq(262_144, 16, nb) == 16_386
    assert kl.max_blocks_per_seq(262_144, 16, 1000) == 1000


def test_attention_context_is_thread_local():
    import threading
    ctx = AttentionContext()
    ctx.is_prefill = True
    set_context(ctx)
    seen = []
    t = threading.Thread(target=lambda: seen.append(get_context()))
    t.start()
    t.join()
    assert seen == [None] and get_context() is ctx
    reset_context()
    assert get_context() is None


# ----------------------------------------------------------------------------- swapping


def test_swap_out_moves_only_unshared_blocks():
    m = PagedKVManager(12, 16, num_host_blocks=4)
    a = Sequence(list(range(40)))
    m.admit(a)                                   # blocks 0, 1, 2
    m.finish_chunk(a, 32)
    b = Sequence(list(range(32)) + [9] * 30)
    m.admit(b)                                   # shares 0, 1; owns 3, 4
    assert b.block_table == [0, 1, 3, 4]
    pairs = m.swap_out(b)
    assert pairs == [(3, 0), (4, 1)]             # host slots handed out 0, 1 (LIFO pool)
    assert b.block_table == [0, 1, -1, -1]
    assert m.block_manager.blocks[3].ref_count == 0 and 3 in m.block_manager.free_block_ids
    assert m.block_manager.blocks[0].ref_count == 2
    assert m.can_swap_in(b)
    back = m.swap_in(b)
    assert [slot for slot, _ in back] == [0, 1]
    assert b.block_table[:2] == [0, 1] and -1 not in b.block_table
    assert sorted(m.host_free) == [0, 1, 2, 3]
    assert [bid for _, bid in back] == b.block_table[2:]


def test_swap_pool_exhaustion_and_free_while_swapped():
    m = PagedKVManager(10, 16, num_host_blocks=1)
    a = Sequence(list(range(40)))
    m.admit(a)
    with pytest.raises(RuntimeError):
        m.swap_out(a)                            # 3 unshared blocks, 1 host slot
    assert a.block_table == [0, 1, 2]            # nothing changed
    assert m.swap_out(a, max_blocks=1) == [(0, 0)]
    m.free(a)                                    # freeing a swapped sequence returns its host slot
    assert m.host_free == [0] and m.block_manager.num_free_blocks == 10


def test_deallocate_swapped_sequence_directly_leaves_other_blocks_alone():
    """The reference scheduler calls block_manager.deallocate itself (engine/scheduler.py:66,
    228, 291). A swapped-out table holds -1 at swapped positions; those hold no device block and
    must not wrap to the pool's last block."""
    m = PagedKVManager(4, 16, num_host_blocks=2)
    a = Sequence(list(range(32)))
    m.admit(a)                                   # blocks 0, 1
    other = Sequence([7] * 32)
    m.admit(other)                               # blocks 2, 3 (3 is the pool's last id)
    assert other.block_table == [2, 3]
    bm = m.block_manager
    assert m.swap_out(a, max_blocks=1) == [(0, 0)]
    assert a.block_table == [-1, 1]
    counts = bm.ref_counts.copy()
    freed = bm.deallocate(a)
    assert freed == [1]
    assert bm.ref_counts[3] == counts[3] == 1 and bm.ref_counts[2] == 1
    assert -1 not in bm.free_block_ids and sorted(bm.free_block_ids) == [0, 1]
    assert bm.allocate_block() == 1              # LIFO: the last freed block comes back first
    assert bm.allocate_block() == 0


def test_block_ids_outside_the_pool_are_refused():
    bm = BlockManager(4, 16)
    s = seq(16)
    bm.allocate(s)
    for bad in ([-1], [4], [0, 9]):
        with pytest.raises(ValueError, match="outside the pool"):
            bm._drop(bad)
        t = seq(16)
        with pytest.raises(ValueError, match="outside the pool"):
            bm.share_blocks(t, bad)
        assert t.block_table == []
    with pytest.raises(ValueError, match="outside the pool"):
        bm.release(-1)
    assert bm.ref_counts.tolist() == [1, 0, 0, 0] and bm.num_free_blocks == 3


def test_config5_managed_builder_shares_the_prefix_and_swaps_private_blocks():
    """The managed config-5 set-up at a small size on the CPU: every sequence's table starts with
    the same physical prefix blocks (refcount = batch), the pool holds exactly the physical blocks,
    the shared-prefix length is the whole prefix, and swapping out a quarter of the sequences moves
    only their private blocks into the host pool, which then holds exactly those."""
    from tileinfer_amd.workloads import config5_managed
    batch, prefix, suffix = 8, 256, 64
    mb = config5_managed(device="cpu", layers=2, batch=batch, prefix=prefix, suffix=suffix)
    m, pb, sb = mb.manager, prefix // 16, suffix // 16
    table, seqlen = mb.tables()
    assert table.shape == (batch, pb + sb) and seqlen.tolist() == [prefix + suffix] * batch
    assert bool((table[:, :pb] == table[0, :pb]).all())
    private = table[:, pb:].flatten().tolist()
    assert len(set(private)) == batch * sb and not set(private) & set(table[0, :pb].tolist())
    bm = m.block_manager
    assert bm.num_free_blocks == 0 and mb.kv.shape[2] == pb + batch * sb
    assert all(int(bm.ref_counts[b]) == batch for b in table[0, :pb].tolist())
    assert m.common_prefix_tokens(mb.seqs) == prefix
    assert mb.q.shape == (2, batch, 24, 256)
    victims = mb.seqs[:batch // 4]
    pairs = [p for s in victims for p in m.swap_out(s)]
    assert sorted(d for d, _ in pairs) == sorted(table[:batch // 4, pb:].flatten().tolist())
    assert m.host_free == [] and bm.num_free_blocks == len(pairs)
    for s in victims:
        assert s.block_table[:pb] == table[0, :pb].tolist() and s.block_table[pb:] == [-1] * sb
        assert m.can_swap_in(s) and len(m.swap_in(s)) == sb


# ----------------------------------------------------------------------------- prefix index: races


def test_identical_prompts_recorded_twice_never_share_foreign_blocks():
    """Two identical prompts admitted before either is recorded compute the same prefix into
    different blocks. After both are recorded and the second is freed, a third copy may share only
    blocks that still hold that prefix -- never blocks that now belong to another sequence."""
    m = PagedKVManager(12, 16)
    prompt = list(range(40))
    a, b = Sequence(prompt), Sequence(prompt)
    assert m.admit(a) and m.admit(b)
    assert a.block_table == [0, 1, 2] and b.block_table == [3, 4, 5]
    m.finish_chunk(a, 32)                       # two whole blocks of each are recorded
    m.finish_chunk(b, 32)
    m.free(b)                                   # frees 5, 4, 3 (3 on top of the stack)
    d = Sequence([7] * 40)
    assert m.admit(d)
    assert d.block_table == [3, 4, 5]           # the unrelated sequence now owns b's old blocks
    c = Sequence(prompt + [99])
    assert m.admit(c)
    shared = c.block_table[:c.num_cached_tokens // 16]
    assert c.num_cached_tokens == 32 and shared == [0, 1]
    assert not set(shared) & set(d.block_table)
    refs = m.block_manager.ref_counts
    assert refs[0] == 2 and refs[1] == 2 and refs[3] == 1


def test_prefix_index_evicts_exactly_the_freed_chains():
    """A boundary recorded under the first block that computed it keeps that block; freeing the
    sequence that holds it forgets it (and everything below), freeing the duplicate does not."""
    pc = PrefixCache(2)
    pc.add([1, 2, 3, 4], [10, 11])
    pc.add([1, 2, 3, 4, 5, 6], [20, 21, 22])   # same first two boundaries: kept as 10, 11
    assert pc.find_longest_prefix([1, 2, 3, 4, 5, 6]) == ([10, 11, 22], 6)
    pc.evict_block(21)                          # names no entry: nothing forgotten
    assert pc.num_entries == 3
    pc.evict_block(11)                          # [10, 11] and [10, 11, 22] go
    assert pc.find_longest_prefix([1, 2, 3, 4, 5, 6]) == ([10], 2)
    assert pc.num_entries == 1
    pc.add([1, 2, 3, 4], [10, 30])
    assert pc.find_longest_prefix([1, 2, 3, 4]) == ([10, 30], 4)


@settings(max_examples=300, deadline=None)
@given(st.lists(st.tuples(st.sampled_from(["admit", "finish", "decode", "free"]),
                          st.integers(0, 3), st.integers(5, 14)), max_size=50))
# The race that needs a careful index: two copies of one prompt computed into different blocks,
# both recorded, the second freed and its blocks taken by another prompt, then a third copy.
@example([("admit", 0, 14), ("admit", 2, 14), ("finish", 0, 5), ("finish", 2, 5),
          ("free", 2, 5), ("admit", 1, 14), ("admit", 2, 14)])
def test_shared_blocks_always_hold_the_shared_tokens(ops):
    """Whatever the interleaving of admissions, recordings and frees, a prefix hit shares only
    blocks whose recorded tokens are the new sequence's tokens at the same positions: every block
    of a live table is tagged with the (position, tokens) it holds, and a shared block's tag must
    match."""
    Sequence.block_size = 4                 # the fixture restores 16
    m = PagedKVManager(24, 4)
    prompts = [[1] * 14, [3] * 14, [1] * 8 + [2] * 6]
    live: dict[int, Sequence] = {}
    tag: dict[int, tuple] = {}              # block -> (logical index, tokens) it holds
    for op, k, n in ops:
        if op == "admit" and k not in live:
            s = Sequence(prompts[k % 2 if k < 3 else 2][:n])
            if m.admit(s):
                for i, bid in enumerate(s.block_table[:s.num_cached_tokens // 4]):
                    assert tag[bid] == (i, tuple(s.token_ids[4 * i:4 * i + 4])), (bid, tag[bid])
                for i in range(s.num_cached_tokens // 4, len(s.block_table)):
                    tag[s.block_table[i]] = (i, tuple(s.token_ids[4 * i:4 * i + 4]))
                live[k] = s
        elif op == "finish" and k in live and live[k].is_prefill:
            s = live[k]
            whole = s.num_tokens // 4 * 4 - s.num_cached_tokens    # whole blocks first: recorded
            if whole > 0:
                m.finish_chunk(s, whole)
            if s.num_tokens > s.num_cached_tokens:
                m.finish_chunk(s, s.num_tokens - s.num_cached_tokens)
            s.is_prefill = False
        elif op == "decode" and k in live and not live[k].is_prefill:
            s = live[k]
            s.append_token(n % 3)
            if not m.can_append(s):
                m.free(live.pop(k))
                continue
            m.append_slot(s)
            i = (len(s) - 1) // 4
            tag[s.block_table[i]] = (i, tuple(s.token_ids[4 * i:4 * i + 4]))
        elif op == "free" and k in live:
            m.free(live.pop(k))
