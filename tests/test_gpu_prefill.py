"""Parity of the HIP paged prefill attention (ti_gqa_prefill_paged) with the CPU oracle, in both
schedules (balanced: key tiles shared evenly over the CUs, units cut between workgroups and merged;
batch_invariant: one workgroup per unit), and the bitwise properties at full size: a chunked
prefill equals the one-shot prefill of the same tokens (batch-invariant schedule), shared prefix
pages equal private copies, physical placement does not matter."""
import pytest
import torch

from helpers import ATOL, RTOL, bits, say
from oracle.brute import prefill_fp64
from oracle.ref_torch import ref_gqa_prefill_paged
from tileinfer_amd.kernels.gqa_decode_paged import gqa_decode_paged_fn
from tileinfer_amd.kernels.gqa_prefill_paged import gqa_prefill_paged_fn
from tileinfer_amd.workloads import config4_prefill, prefill_step

pytestmark = pytest.mark.gpu


def run_gpu(step, dev, causal=True, **kw):
    return gqa_prefill_paged_fn(step.q.to(dev), step.k_cache.to(dev), step.v_cache.to(dev),
                                step.block_table.to(dev), step.cu_seqlens_q.to(dev),
                                step.seqlen_k.to(dev), step.max_seqlen_q, step.page_size,
                                causal=causal, **kw)


def run_ref(step, causal=True):
    return ref_gqa_prefill_paged(step.q, step.k_cache, step.v_cache, step.block_table,
                                 step.cu_seqlens_q, step.seqlen_k, step.page_size, causal)


def close(out, ref, atol=ATOL, rtol=RTOL):
    torch.testing.assert_close(out.float().cpu(), ref.float().cpu(), atol=atol, rtol=rtol)


MODES = [pytest.param(False, id="balanced"), pytest.param(True, id="per_unit")]
SCHED = {False: "balanced", True: "per_unit"}


@pytest.mark.parametrize("invariant", MODES)
@pytest.mark.parametrize("q_lens,kv_lens", [
    ([64], [64]),                        # one full workgroup, first chunk
    ([100], [100]),                      # ragged last workgroup
    ([37], [300]),                       # continuation: 263 cached tokens before the chunk
    ([16, 1, 0, 50, 129], [16, 200, 5, 51, 1000]),   # ragged batch, an empty chunk
    ([1], [1]),
    ([3], [2000]),                       # balanced: each unit cut over 8 workgroups
    ([5, 2], [9000, 40]),                # balanced: one unit over many workgroups, one whole
])
def test_vs_oracle(q_lens, kv_lens, invariant, dev):
    say(f"prefill q_lens={q_lens} kv_lens={kv_lens} invariant={invariant}")
    step = prefill_step(q_lens, kv_lens, seed=21)
    out = run_gpu(step, dev, schedule=SCHED[invariant])
    close(out, run_ref(step))
    exact = torch.from_numpy(prefill_fp64(
        step.q.double().numpy(), step.k_cache.double().numpy(), step.v_cache.double().numpy(),
        step.block_table.numpy(), step.cu_seqlens_q.numpy(), step.seqlen_k.numpy()))
    close(out, exact)


@pytest.mark.parametrize("invariant", MODES)
def test_noncausal_vs_oracle(invariant, dev):
    say(f"prefill non-causal invariant={invariant}")
    step = prefill_step([40, 70], [90, 70], seed=22)
    close(run_gpu(step, dev, causal=False, schedule=SCHED[invariant]),
          run_ref(step, causal=False))


@pytest.mark.parametrize("hq,hkv,d,dtype", [
    (24, 4, 256, torch.float16), (32, 4, 128, torch.bfloat16), (8, 8, 128, torch.float16),
    (16, 1, 256, torch.bfloat16)])
def test_shapes_and_dtypes(hq, hkv, d, dtype, dev):
    say(f"prefill hq={hq} hkv={hkv} d={d} dtype={dtype}")
    step = prefill_step([70, 19], [1300, 19], seed=23, hq=hq, hkv=hkv, d=d, dtype=dtype)
    ref = run_ref(step)
    close(run_gpu(step, dev, schedule="balanced"), ref)
    close(run_gpu(step, dev, batch_invariant=True), ref)


def test_config4_first_chunk_vs_oracle(dev):
    """Config 4's 2048-token chunk over its 128 non-contiguous blocks, against the oracle."""
    step = config4_prefill()
    say("prefill config4 chunk 2048 (first chunk)")
    ref = run_ref(step)
    per_unit = run_gpu(step, dev, batch_invariant=True)
    close(run_gpu(step, dev, schedule="balanced"), ref)
    close(per_unit, ref)
    # No cached context: the automatic choice is one workgroup per unit.
    assert torch.equal(bits(run_gpu(step, dev, max_seqlen_k=2048)), bits(per_unit))


def test_config4_continuation_schedules_agree(dev):
    """Config 4's continuation chunk (2048 queries over 8192 keys): the balanced schedule (192-row
    units, 32-key tiles, cut units merged in fp32) against the one-unit-per-workgroup one (128-row
    units, 64-key tiles): equal within rounding; the balanced run is deterministic."""
    say("prefill config4 continuation: balanced vs invariant")
    st = config4_prefill(device=dev, cached=6144)
    args = (st.q, st.k_cache, st.v_cache, st.block_table, st.cu_seqlens_q, st.seqlen_k, 2048)
    bal = gqa_prefill_paged_fn(*args, schedule="balanced")
    inv = gqa_prefill_paged_fn(*args, batch_invariant=True)
    close(bal, inv, atol=1e-2, rtol=1e-2)
    assert torch.equal(bits(bal), bits(gqa_prefill_paged_fn(*args, schedule="balanced")))
    # The automatic choice with the host bound the reference's context carries (max_seqlen_k):
    # balanced here (cached context, 256 units of 192 rows, one per CU but cut in merged runs).
    assert torch.equal(bits(bal), bits(gqa_prefill_paged_fn(*args, max_seqlen_k=8192)))
    # Spot rows against the oracle: query i alone over its visible keys 0..6144+i.
    rows = torch.arange(0, 2048, 97)
    ref = ref_gqa_prefill_paged(st.q[rows.to(dev)].cpu(), st.k_cache.cpu(), st.v_cache.cpu(),
                                st.block_table.cpu().expand(len(rows), -1),
                                torch.arange(len(rows) + 1, dtype=torch.int32),
                                (rows + 6145).to(torch.int32))
    close(bal[rows.to(dev)], ref)


def test_chunked_equals_one_shot_bitwise(dev):
    """A 4096-token prompt prefilled in chunks of 1000/1000/2000/96 tokens gives bitwise the
    rows of the one-shot prefill: key tiles sit at absolute positions and masked keys add
    exact zeros, so no result depends on how the prompt was chunked."""
    say("prefill chunked vs one-shot, 4096 tokens")
    full = prefill_step([4096], [4096], seed=24)
    q = full.q.to(dev)
    kc, vc = full.k_cache.to(dev), full.v_cache.to(dev)
    bt = full.block_table.to(dev)
    one = gqa_prefill_paged_fn(q, kc, vc, bt, full.cu_seqlens_q.to(dev), full.seqlen_k.to(dev),
                               4096, batch_invariant=True)
    start = 0
    for n in (1000, 1000, 2000, 96):
        cu = torch.tensor([0, n], dtype=torch.int32, device=dev)
        sk = torch.tensor([start + n], dtype=torch.int32, device=dev)
        part = gqa_prefill_paged_fn(q[start:start + n], kc, vc, bt, cu, sk, n,
                                    batch_invariant=True)
        assert torch.equal(bits(part), bits(one[start:start + n])), f"chunk at {start}"
        start += n


def test_batched_equals_separate_bitwise(dev):
    """Several sequences in one launch give bitwise what each gives alone."""
    say("prefill batched vs separate")
    step = prefill_step([300, 64, 5], [900, 64, 700], seed=25)
    dq = step.q.to(dev)
    kc, vc = step.k_cache.to(dev), step.v_cache.to(dev)
    bt = step.block_table.to(dev)
    together = run_gpu(step, dev, batch_invariant=True)
    cu = step.cu_seqlens_q.tolist()
    for b in range(3):
        alone = gqa_prefill_paged_fn(
            dq[cu[b]:cu[b + 1]], kc, vc, bt[b:b + 1],
            torch.tensor([0, cu[b + 1] - cu[b]], dtype=torch.int32, device=dev),
            step.seqlen_k[b:b + 1].to(dev), batch_invariant=True)
        assert torch.equal(bits(alone), bits(together[cu[b]:cu[b + 1]]))


@pytest.mark.parametrize("invariant", MODES)
def test_shared_prefix_equals_private_bitwise(invariant, dev):
    """Two sequences whose tables alias one cached prefix, against private copies of it (the
    balanced schedule depends on lengths only, so it is the same for both)."""
    say(f"prefill shared vs private prefix invariant={invariant}")
    pre, chunk, bs = 512, 200, 16
    base = prefill_step([chunk, chunk], [pre + chunk, pre + chunk], seed=26)
    pb = pre // bs
    shared_bt = base.block_table.clone()
    shared_bt[1, :pb] = shared_bt[0, :pb]            # sequence 1 aliases sequence 0's prefix
    kc, vc = base.k_cache.clone(), base.v_cache.clone()
    private = base.block_table
    for j in range(pb):                               # make the private copies equal in value
        kc[private[1, j]] = kc[private[0, j]]
        vc[private[1, j]] = vc[private[0, j]]
    args = (base.q.to(dev), kc.to(dev), vc.to(dev))
    tail = (base.cu_seqlens_q.to(dev), base.seqlen_k.to(dev), chunk)
    a = gqa_prefill_paged_fn(*args, shared_bt.to(dev), *tail, schedule=SCHED[invariant])
    b = gqa_prefill_paged_fn(*args, private.to(dev), *tail, schedule=SCHED[invariant])
    assert torch.equal(bits(a), bits(b))


def test_last_row_matches_decode(dev):
    """The chunk's last query sees the whole context: the same value as a decode of that query
    (two different kernels; within the decode tolerance)."""
    say("prefill last row vs decode kernel")
    step = prefill_step([128], [3000], seed=27)
    out = run_gpu(step, dev)
    dec = gqa_decode_paged_fn(step.q[-1:].to(dev), step.k_cache.to(dev), step.v_cache.to(dev),
                              step.block_table.to(dev), step.seqlen_k.to(dev))
    close(out[-1:], dec)


@pytest.mark.parametrize("invariant", MODES)
def test_empty_contexts_give_zeros_and_rows_outside_untouched(invariant, dev):
    """kv_len 0 gives zeros; rows with no visible key (kv_len < q_len) give zeros; rows outside
    every chunk (past cu_seqlens_q[-1]) keep what the caller's buffer held."""
    say(f"prefill zero rows and untouched rows invariant={invariant}")
    step = prefill_step([4, 6], [0, 3], seed=28)
    q = torch.cat([step.q, torch.randn(5, 24, 256).to(torch.bfloat16)]).to(dev)
    out = torch.full((q.shape[0], 24, 256), 7.0, dtype=torch.bfloat16, device=dev)
    gqa_prefill_paged_fn(q, step.k_cache.to(dev), step.v_cache.to(dev), step.block_table.to(dev),
                         step.cu_seqlens_q.to(dev), step.seqlen_k.to(dev), 6, out=out,
                         schedule=SCHED[invariant])
    o = out.float().cpu()
    assert (o[:4] == 0).all()                 # kv_len 0
    assert (o[4:7] == 0).all()                # offset -3: rows 0..2 see nothing
    assert (o[7:10] != 0).any()
    close(o[4:10], run_ref(step)[4:10])
    assert (o[10:] == 7.0).all()


def test_out_of_range_block_ids_are_masked(dev):
    """A block id outside the cache inside the context is an absent page: its 16 keys are masked
    (never read); -1 padding past the context is ignored."""
    say("prefill bad block ids")
    step = prefill_step([20], [40], seed=29, width=6)
    bt = step.block_table.clone()
    bt[0, 1] = 10 ** 8                        # keys 16..31 live in a block that does not exist
    out = gqa_prefill_paged_fn(step.q.to(dev), step.k_cache.to(dev), step.v_cache.to(dev),
                               bt.to(dev), step.cu_seqlens_q.to(dev), step.seqlen_k.to(dev))
    # Expected: float64 attention of each row over its visible keys minus 16..31.
    kf = step.k_cache.double().reshape(-1, 4, 256)
    vf = step.v_cache.double().reshape(-1, 4, 256)
    rows = [int(step.block_table[0, j // 16]) * 16 + j % 16 for j in range(40)]
    k, v = kf[rows], vf[rows]
    want = torch.zeros(20, 24, 256, dtype=torch.float64)
    for i in range(20):
        keys = [j for j in range(20 + i + 1) if not 16 <= j < 32]
        for h in range(24):
            s = k[keys, h // 6] @ step.q[i, h].double() / 16.0
            want[i, h] = torch.softmax(s, 0) @ v[keys, h // 6]
    close(out, want)


def test_rejects_bad_arguments(dev):
    step = prefill_step([8], [8], seed=30)
    q, kc, vc = step.q.to(dev), step.k_cache.to(dev), step.v_cache.to(dev)
    bt, cu, sk = step.block_table.to(dev), step.cu_seqlens_q.to(dev), step.seqlen_k.to(dev)
    with pytest.raises(TypeError):
        gqa_prefill_paged_fn(q, kc, vc, bt.long(), cu, sk)
    with pytest.raises(ValueError):
        gqa_prefill_paged_fn(q, kc, vc, bt, cu[:1], sk)
    with pytest.raises(ValueError):
        gqa_prefill_paged_fn(q, kc, vc, bt, cu, sk, page_size=24)
    from tileinfer_amd._lib import TileInferError
    q96 = torch.zeros(8, 24, 96, dtype=torch.bfloat16, device=dev)
    k96 = torch.zeros(kc.shape[0], 16, 4, 96, dtype=torch.bfloat16, device=dev)
    with pytest.raises(TileInferError):
        gqa_prefill_paged_fn(q96, k96, k96, bt, cu, sk)


@pytest.mark.parametrize("invariant", MODES)
def test_many_sequences_vs_oracle(invariant, dev):
    """A ragged batch of 40 chunks (1 to 300 queries over up to 2,000 cached tokens, some empty):
    hundreds of units, many of them cut between workgroups in the balanced schedule."""
    say(f"prefill 40 ragged sequences invariant={invariant}")
    g = torch.Generator().manual_seed(40)
    q_lens = torch.randint(1, 301, (40,), generator=g).tolist()
    q_lens[7] = 0
    kv_lens = [q + int(torch.randint(0, 2001, (1,), generator=g)) for q in q_lens]
    kv_lens[11] = 0                                  # no context at all: zero rows
    step = prefill_step(q_lens, kv_lens, seed=41)
    close(run_gpu(step, dev, schedule=SCHED[invariant]), run_ref(step))


def paged_step(q_lens, kv_lens, page, seed, hq=24, hkv=4, d=256, dtype=torch.bfloat16):
    """A prefill step whose cache pages hold `page` rows (the flattened layout is the same)."""
    g = torch.Generator().manual_seed(seed)
    need = sum((n + page - 1) // page for n in kv_lens)
    pool = need + 5
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    width = max(1, max((n + page - 1) // page for n in kv_lens))
    table = torch.full((len(kv_lens), width), -1, dtype=torch.int32)
    at = 0
    for b, n in enumerate(kv_lens):
        k = (n + page - 1) // page
        table[b, :k] = perm[at:at + k]
        at += k
    kc = torch.randn(pool, page, hkv, d, generator=g).to(dtype)
    vc = torch.randn(pool, page, hkv, d, generator=g).to(dtype)
    cu = torch.tensor([0] + list(torch.tensor(q_lens).cumsum(0)), dtype=torch.int32)
    q = torch.randn(int(cu[-1]), hq, d, generator=g).to(dtype)
    return q, kc, vc, table, cu, torch.tensor(kv_lens, dtype=torch.int32)


@pytest.mark.parametrize("page", [32, 48, 64])
@pytest.mark.parametrize("invariant", MODES)
def test_larger_pages_vs_oracle(page, invariant, dev):
    """Pages of 32, 48 (not a power of two: the division path) and 64 rows; sub-tiles of 16 keys
    always lie inside one page."""
    say(f"prefill page_size={page} invariant={invariant}")
    q, kc, vc, table, cu, sk = paged_step([50, 130], [700, 130], page, seed=page)
    out = gqa_prefill_paged_fn(q.to(dev), kc.to(dev), vc.to(dev), table.to(dev), cu.to(dev),
                               sk.to(dev), 130, page, schedule=SCHED[invariant])
    close(out, ref_gqa_prefill_paged(q, kc, vc, table, cu, sk, page))


@pytest.mark.parametrize("invariant", MODES)
def test_repeated_calls_bitwise_identical(invariant, dev):
    """Every K/V stage is loaded into LDS by all waves together; each must wait for its own loads
    before the barrier that publishes the stage. Without that wait a wave could read another
    wave's part before it landed and a few calls in a hundred came out different: 24 repeats of
    the ragged 40-sequence batch must agree bitwise."""
    say(f"prefill repeated calls invariant={invariant}")
    g = torch.Generator().manual_seed(40)
    q_lens = torch.randint(1, 301, (40,), generator=g).tolist()
    kv_lens = [q + int(torch.randint(0, 2001, (1,), generator=g)) for q in q_lens]
    step = prefill_step(q_lens, kv_lens, seed=41)
    args = (step.q.to(dev), step.k_cache.to(dev), step.v_cache.to(dev), step.block_table.to(dev),
            step.cu_seqlens_q.to(dev), step.seqlen_k.to(dev), step.max_seqlen_q)
    first = bits(gqa_prefill_paged_fn(*args, schedule=SCHED[invariant]))
    for _ in range(23):
        assert torch.equal(bits(gqa_prefill_paged_fn(*args, schedule=SCHED[invariant])), first)


def _random_case(seed):
    """A seeded random call: batch 1-4, chunk and context lengths, GQA group (including groups
    that do not divide the workgroup's rows), head_dim, dtype, page size, causal or not."""
    g = torch.Generator().manual_seed(seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=g))]  # noqa: E731
    hkv = pick([1, 2, 4])
    group = pick([1, 3, 5, 6, 7, 8, 12])
    d = pick([128, 256])
    batch = int(torch.randint(1, 5, (1,), generator=g))
    q_lens = [int(torch.randint(0, 160, (1,), generator=g)) for _ in range(batch)]
    kv_lens = [q + int(torch.randint(0, 900, (1,), generator=g)) for q in q_lens]
    return dict(q_lens=q_lens, kv_lens=kv_lens, hq=hkv * group, hkv=hkv, d=d,
                dtype=pick([torch.bfloat16, torch.float16]), page=pick([4, 8, 16, 32]),
                causal=bool(torch.randint(2, (1,), generator=g)))


@pytest.mark.parametrize("seed", range(100, 148))
def test_random_calls_vs_oracle(seed, dev):
    """Seeded random calls through both schedules against the oracle."""
    c = _random_case(seed)
    say(f"prefill random seed={seed} {c}")
    q, kc, vc, table, cu, sk = paged_step(c["q_lens"], c["kv_lens"], c["page"], seed, hq=c["hq"],
                                          hkv=c["hkv"], d=c["d"], dtype=c["dtype"])
    ref = ref_gqa_prefill_paged(q, kc, vc, table, cu, sk, c["page"], c["causal"])
    args = (q.to(dev), kc.to(dev), vc.to(dev), table.to(dev), cu.to(dev), sk.to(dev),
            max(c["q_lens"]), c["page"])
    for schedule in ("balanced", "per_unit"):
        close(gqa_prefill_paged_fn(*args, causal=c["causal"], schedule=schedule), ref)


@pytest.mark.parametrize("invariant", MODES)
def test_graph_capture_replay(invariant, dev):
    """The prefill (with its schedule and merge launches and the workspace from torch's graph
    pool) captured in a HIP graph: every replay, with new queries and eager work between, matches
    the eager result bitwise."""
    say(f"prefill graph capture invariant={invariant}")
    step = prefill_step([300, 77, 5], [1200, 77, 600], seed=33)
    q = step.q.to(dev)
    args = (step.k_cache.to(dev), step.v_cache.to(dev), step.block_table.to(dev),
            step.cu_seqlens_q.to(dev), step.seqlen_k.to(dev), step.max_seqlen_q)

    def fn():
        return gqa_prefill_paged_fn(q, *args, schedule=SCHED[invariant])

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = fn()
    gen = torch.Generator(device=dev).manual_seed(3)
    for r in range(3):
        q.copy_(torch.randn(q.shape, generator=gen, device=dev).to(q.dtype))
        graph.replay()
        torch.cuda.synchronize()
        eager = fn()
        torch.cuda.synchronize()
        assert torch.equal(bits(static_out), bits(eager)), f"replay {r}"
