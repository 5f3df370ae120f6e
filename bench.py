"""Benchmark of the paged KV-cache hot path on one MI355X.

Default workload: one decode step of the 16 full-attention layers of
Qwen3.6-27B at batch 64 x 32,768 tokens of context (24 query heads, 4 KV heads, head_dim 256,
block size 16, bf16 cache of [2, 16, 131072, 16, 4, 256] = 128 GiB, block tables = an independent
random permutation of the 131,072 blocks per layer). A step = for every layer: append the batch's
new tokens through slot_mapping, then paged decode over 32,768 tokens (split-K).

Prints ONE JSON line. ``value`` is the algorithmic byte rate of the whole step (append + decode
bytes of every layer / step time); ``roofline`` is the decode launch's algorithmic rate against
8 TB/s, timed with HIP events on the launch stream; ``cpu_baseline`` is the CPU oracle (a
restatement of the reference's torch path) timed on a sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3] [--variant auto]
"""
from __future__ import annotations

import argparse
import functools
import json
import os
import re
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from tileinfer_amd.engine.kv_layout import allocate_kv_cache, layer_views  # noqa: E402
from tileinfer_amd.kernels.gqa_decode_paged import decode_plan, gqa_decode_paged_fn  # noqa: E402
from tileinfer_amd.kernels.kvcache_store import store_kvcache  # noqa: E402
from tileinfer_amd.workloads import (BLOCK, HEAD_DIM, HKV, HQ, append_bytes,  # noqa: E402
                                     decode_bytes, decode_flops)

METRIC = "paged GQA decode achieved HBM GB/s (% of peak) + µs/layer-step; append GB/s"
PEAK_HBM_GBPS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "decode_config3_traffic.txt"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_state(batch: int, ctx: int, layers: int, dev, seed: int, sequential: bool = False):
    """Cache slab, per-layer tables and inputs of the config-3 style decode step.

    Tables are an independent random permutation of the pool per layer (config 3);
    ``sequential`` lays every sequence's blocks out contiguously instead (a diagnostic only).
    """
    blocks_per_seq = (ctx + BLOCK - 1) // BLOCK
    nb = batch * blocks_per_seq
    kv = allocate_kv_cache(layers, nb, BLOCK, HKV, HEAD_DIM, dev, torch.bfloat16, zero=False)
    gen = torch.Generator(device=dev).manual_seed(seed)
    for kvi in range(2):
        for l in range(layers):
            kv[kvi, l].normal_(generator=gen)
    tables, slots = [], []
    pos = ctx - 1
    for l in range(layers):
        order = (torch.arange(nb, device=dev) if sequential
                 else torch.randperm(nb, generator=gen, device=dev))
        t = order.to(torch.int32).view(batch, blocks_per_seq)
        tables.append(t)
        slots.append((t[:, pos // BLOCK].long() * BLOCK + pos % BLOCK).to(torch.int32))
    seqlen = torch.full((batch,), ctx, dtype=torch.int32, device=dev)
    q = torch.randn((layers, batch, HQ, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    k_new = torch.randn((layers, batch, HKV, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    v_new = torch.randn((layers, batch, HKV, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    return kv, tables, slots, seqlen, q, k_new, v_new


def read_traffic():
    """Per-launch HBM bytes of the decode kernels from the committed rocprofv3 --pmc summary."""
    if not TRAFFIC_FILE.exists():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", TRAFFIC_FILE.read_text(), re.M)
    return float(m.group(1)) if m else None


def cpu_baseline(kv, tables, seqlen, q, k_new, v_new, budget_s: float = 12.0):
    """Time the CPU oracle (append + decode of the reference recipe) on a sample of layer 0."""
    from oracle.ref_torch import ref_gqa_decode_paged, ref_store_kvcache

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    batch = seqlen.shape[0]
    ctx = int(seqlen[0])

    def sample(n):
        t = tables[0][:n].cpu()
        pages = t.reshape(-1).long()
        kc = kv[0, 0][pages.to(kv.device)].cpu()
        vc = kv[1, 0][pages.to(kv.device)].cpu()
        local = torch.arange(pages.numel(), dtype=torch.int32).view(n, -1)
        pos = ctx - 1
        sl = (local[:, pos // BLOCK].long() * BLOCK + pos % BLOCK).to(torch.int32)
        return (q[0, :n].cpu(), k_new[0, :n].cpu(), v_new[0, :n].cpu(), sl, local,
                seqlen[:n].cpu(), kc, vc)

    def run(args):
        qq, kn, vn, sl, tb, sq, kc, vc = args
        t0 = time.perf_counter()
        ref_store_kvcache(kn, vn, kc.view(-1, HKV * HEAD_DIM), vc.view(-1, HKV * HEAD_DIM), sl)
        ref_gqa_decode_paged(qq, kc, vc, tb, sq, BLOCK)
        return time.perf_counter() - t0

    one = sample(1)
    run(one)  # warm-up
    per_seq = run(one)
    n = max(1, min(batch, int(budget_s / 4 / max(per_seq, 1e-6))))
    args = sample(n)
    run(args)
    times = [run(args) for _ in range(3)]
    t = statistics.median(times)
    nbytes = decode_bytes([ctx] * n) + append_bytes(args[3], HKV * HEAD_DIM)
    return {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": (f"layer 0 of the same step, {n} of {batch} sequences x {ctx} tokens: append "
                       f"+ decode by the CPU oracle (oracle/ref_torch.py), median of 3 after 1 "
                       f"warm-up, {t * 1e3:.1f} ms per run"),
            "us_per_layer_step_extrapolated": round(t / n * batch * 1e6, 1)}


def parity_sample(kv, tables, seqlen, q, k_new, v_new, out_last, layer: int, idx=(0, 37)):
    """Full-size checks on the run itself: appended rows bit-exact; decode of sampled sequences
    within atol 2e-2 / rtol 1e-2 of the CPU oracle."""
    from oracle.ref_torch import ref_gqa_decode_paged

    k_rows, v_rows, _, _ = layer_views(kv, layer)
    ctx = int(seqlen[0])
    pos = ctx - 1
    sl = (tables[layer][:, pos // BLOCK].long() * BLOCK + pos % BLOCK)
    append_ok = bool(torch.equal(k_rows[sl].view(torch.int16), k_new[layer].reshape(len(sl), -1).view(torch.int16))
                     and torch.equal(v_rows[sl].view(torch.int16), v_new[layer].reshape(len(sl), -1).view(torch.int16)))
    worst = 0.0
    ok = True
    for b in idx:
        b = b % seqlen.shape[0]
        pages = tables[layer][b].long()
        kc = kv[0, layer][pages].cpu()
        vc = kv[1, layer][pages].cpu()
        tb = torch.arange(pages.numel(), dtype=torch.int32).view(1, -1)
        ref = ref_gqa_decode_paged(q[layer, b:b + 1].cpu(), kc, vc, tb, seqlen[b:b + 1].cpu(), BLOCK)
        got = out_last[b:b + 1].float().cpu()
        err = (got - ref.float()).abs()
        worst = max(worst, err.max().item())
        ok = ok and bool((err <= 2e-2 + 1e-2 * ref.float().abs()).all())
    return {"append_bit_exact": append_ok, "decode_within_tol": ok,
            "decode_max_abs_err": round(worst, 6), "sampled_sequences": list(idx), "layer": layer}


def calibrate(dev, gib: float = 4.0, reps: int = 5):
    """Plain device copy and read of known size: the scale for rocprofv3 FETCH_SIZE/WRITE_SIZE
    (bytes the counters report per byte moved) and the streaming bandwidth torch reaches."""
    n = int(gib * 2**30) // 2
    src = torch.empty(n, dtype=torch.bfloat16, device=dev).normal_()
    dst = torch.empty_like(src)
    res = {}
    for name, fn, nbytes in (("copy", lambda: dst.copy_(src), 4 * n),
                             ("read_sum", lambda: src.sum(dtype=torch.float32), 2 * n)):
        us = _time(fn, reps, 1)
        res[name] = {"bytes_per_launch": nbytes, "us": round(us, 1),
                     "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}
    del src, dst
    print(json.dumps({"calibration": res, "copy_read_bytes": 2 * n, "copy_write_bytes": 2 * n}),
          flush=True)


def _time(fn, steps: int, warmup: int) -> float:
    """Mean µs of fn() over `steps` calls after `warmup`, HIP events on the current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / steps


def _time_interleaved(fns, steps: int, warmup: int, rounds: int = 5) -> list:
    """Median over `rounds` of the mean µs of each fn over `steps` calls, the functions taking
    turns in every round (so clock ramps and a neighbour's state weigh on all of them alike)."""
    for fn in fns:
        for _ in range(warmup):
            fn()
    torch.cuda.synchronize()
    per_fn = [[] for _ in fns]
    for _ in range(rounds):
        for i, fn in enumerate(fns):
            per_fn[i].append(_time(fn, steps, 0))
    return [statistics.median(v) for v in per_fn]


def swap_config5(dev, args, layers: int = 16, fraction: float = 0.25) -> dict:
    """Config 5's swap at its stated size, the way a serving engine does it: the 128-sequence
    shared-prefix batch set up through PagedKVManager (workloads.config5_managed), a quarter of
    the sequences swapped out with PagedKVManager.swap_out (their 32 unique blocks each: 1,024
    blocks, K and V of all 16 layers, 1 GiB) through one swap_blocks launch to pinned host
    memory, the freed blocks overwritten, then swap_in into the blocks the pool hands out and one
    launch back. Copies timed with HIP events (each launch repeated, same pairs); the round trip
    is checked bit-exact and every layer's decode of the batch bitwise unchanged."""
    from tileinfer_amd.kernels.block_copy import swap_blocks
    from tileinfer_amd.workloads import config5_managed

    mb = config5_managed(dev, layers=layers, swap_fraction=fraction)
    m, kv = mb.manager, mb.kv

    def decode_all(tbl, sl):
        return torch.stack([gqa_decode_paged_fn(mb.q[l], kv[0, l], kv[1, l], tbl, sl, BLOCK)
                            for l in range(layers)])

    ref = decode_all(*mb.tables())
    victims = mb.seqs[::round(1 / fraction)]
    pairs_out = [p for s_ in victims for p in m.swap_out(s_)]
    n = len(pairs_out)
    old_ids = torch.tensor([b_ for b_, _ in pairs_out], dtype=torch.int64, device=dev)
    before = kv[:, :, old_ids].clone()
    host = torch.empty((2, layers, n, BLOCK, HKV, HEAD_DIM), dtype=torch.bfloat16, pin_memory=True)
    out_map = torch.tensor(pairs_out, dtype=torch.int64, device=dev)
    reps = max(2, args.steps // 4)
    out_us = _time(lambda: swap_blocks(kv, host, out_map), reps, 1)
    kv[:, :, old_ids] = 0                                  # the freed blocks are reused
    pairs_in = [p for s_ in victims for p in m.swap_in(s_)]
    in_map = torch.tensor(pairs_in, dtype=torch.int64, device=dev)
    in_us = _time(lambda: swap_blocks(host, kv, in_map), reps, 1)
    torch.cuda.synchronize()
    out_of = {h: i for i, (_, h) in enumerate(pairs_out)}
    order = torch.tensor([out_of[h] for h, _ in pairs_in], dtype=torch.int64, device=dev)
    new_ids = in_map[:, 1]
    ok = bool(torch.equal(kv[:, :, new_ids].view(torch.int16),
                          before[:, :, order].view(torch.int16)))
    same = bool(torch.equal(decode_all(*mb.tables()).view(torch.int16), ref.view(torch.int16)))
    moved = 2 * layers * n * BLOCK * HKV * HEAD_DIM * 2
    del mb, kv, before, host, ref
    return {"sequences_swapped": len(victims), "blocks": n, "layers": layers,
            "bytes_each_way": moved,
            "swap_out_us": round(out_us, 1), "swap_out_GBps": round(moved / (out_us * 1e-6) / 1e9, 1),
            "swap_in_us": round(in_us, 1), "swap_in_GBps": round(moved / (in_us * 1e-6) / 1e9, 1),
            "roundtrip_bit_exact": ok, "decode_bitwise_unchanged": same,
            "bound": "host link (pinned host memory over the fabric)"}


def metadata_compare(b: int, ctx: int, dev, steps: int = 16, warmup: int = 2) -> dict:
    """Per-step decode metadata at the bench's batch and context. The reference runner's host
    builder (restated in oracle/ref_metadata.py: every sequence's whole block table through
    torch.tensor into pinned buffers, then the uploads; engine/model_runner.py:538-584) against
    DeviceBlockTables (the appended ids go up, the GPU derives tables, slots and lengths). Both
    are timed wall-clock per step including the device work (synchronised)."""
    from oracle.ref_metadata import RefDecodePrep
    from tileinfer_amd.engine import DeviceBlockTables, PagedKVManager, Sequence

    width = ctx // BLOCK + 2
    m = PagedKVManager(b * width, BLOCK, enable_prefix_caching=False)
    seqs = []
    for _ in range(b):
        s = Sequence(range(ctx - 1))
        if not m.admit(s):
            raise RuntimeError("metadata_compare: pool too small")
        m.finish_chunk(s, s.num_tokens)
        seqs.append(s)
    ref = RefDecodePrep(b, width, device=dev)
    dt = DeviceBlockTables(max_seqs=b, max_blocks_per_seq=width, block_size=BLOCK, device=dev)
    ref_t, dev_t, words = [], [], []
    for it in range(warmup + steps):
        for s in seqs:
            s.append_token(0)
            m.append_slot(s)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ref(seqs, BLOCK, bsz=b)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        dt.step(seqs, width=width)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        if it >= warmup:
            ref_t.append((t1 - t0) * 1e6)
            dev_t.append((t2 - t1) * 1e6)
            words.append(dt.last_upload_words)
    rs, rt, rc = ref(seqs, BLOCK, bsz=b)
    ds, dtb, dc = dt.step(seqs, width=width)
    same = bool(torch.equal(rs, ds) and torch.equal(rt, dtb) and torch.equal(rc, dc))
    return {"batch": b, "blocks_per_seq": ctx // BLOCK, "steps": steps,
            "reference_host_builder_us_per_step": round(statistics.median(ref_t), 1),
            "device_tables_us_per_step": round(statistics.median(dev_t), 1),
            "reference_upload_bytes_per_step": 4 * b * (width + 3),
            "device_upload_bytes_per_step": 4 * int(statistics.median(words)),
            "outputs_identical": same,
            "note": "wall clock per step incl. device work; the reference builder is restated "
                    "in oracle/ref_metadata.py"}


def _graph_us(fn, reps: int = 20, replays: int = 5) -> float:
    """Mean GPU µs of fn(): `reps` calls captured in one HIP graph, replayed `replays` times and
    timed with events (no Python launch overhead in the figure)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * replays)


def fusions_compare(kv, tables, slots, seqlen, q, dev) -> dict:
    """One layer of the decode step with the element-wise work around attention (model/qwen_36.py:
    977-1018 before, 1083 after), unfused against fused, GPU time from captured graphs."""
    from tileinfer_amd.kernels import (fused_sigmoid_mul, qknorm_rope, qknorm_rope_append,
                                       store_kvcache as store)

    b = q.shape[1]
    gen = torch.Generator(device=dev).manual_seed(21)
    rnd = lambda *sh: torch.randn(sh, generator=gen, device=dev).to(torch.bfloat16)  # noqa: E731
    q0, k0, v0 = rnd(b, HQ, HEAD_DIM), rnd(b, HKV, HEAD_DIM), rnd(b, HKV, HEAD_DIM)
    qw, kw = 0.1 * rnd(HEAD_DIM), 0.1 * rnd(HEAD_DIM)
    pos = torch.arange(b, device=dev, dtype=torch.float32) * 1000.0
    inv = 1.0 / 1e7 ** (torch.arange(0, 64, 2, device=dev).float() / 64)
    emb = torch.cat([pos[:, None] * inv, pos[:, None] * inv], dim=-1)
    cos, sin = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
    k_rows, v_rows, k_paged, v_paged = layer_views(kv, 0)
    gate = rnd(b, 1, HQ * HEAD_DIM)

    def unfused_in():
        qn = qknorm_rope(q0, qw, cos, sin)
        kn = qknorm_rope(k0, kw, cos, sin)
        store(kn, v0, k_rows, v_rows, slots[0])
        return qn

    def fused_in():
        return qknorm_rope_append(q0, k0, v0, qw, kw, cos, sin, k_rows, v_rows, slots[0])

    def unfused_out():
        o = gqa_decode_paged_fn(q[0], k_paged, v_paged, tables[0], seqlen, BLOCK)
        return fused_sigmoid_mul(o, gate)

    def fused_out():
        return gqa_decode_paged_fn(q[0], k_paged, v_paged, tables[0], seqlen, BLOCK, gate=gate)

    res = {"batch": b,
           "input_side_unfused_us": round(_graph_us(unfused_in), 2),
           "input_side_fused_us": round(_graph_us(fused_in), 2),
           "decode_then_gate_us": round(_graph_us(unfused_out, reps=3, replays=3), 2),
           "decode_gated_us": round(_graph_us(fused_out, reps=3, replays=3), 2)}
    same_in = bool(torch.equal(unfused_in().view(torch.int16), fused_in().view(torch.int16)))
    same_out = bool(torch.equal(unfused_out().view(torch.int16), fused_out().view(torch.int16)))
    res["bitwise_equal"] = same_in and same_out
    res["note"] = ("input side: qknorm_rope(q), qknorm_rope(k), store_kvcache vs one "
                   "qknorm_rope_append; output side: decode + fused_sigmoid_mul vs decode with "
                   "the gate in its epilogue; per layer, GPU time of captured graphs")
    return res


def prefill_config4(st, chunk_slots, kc, vc, dev, args) -> dict:
    """Config 4's 2048-token chunk through the paged prefill attention, straight from the cache
    pages the append just wrote (first chunk: the chunk attends over itself), and a continuation
    chunk of 2048 after 6144 cached tokens. Also timed: the reference recipe's torch gather of the
    continuation's 8192 positions into contiguous K/V (model/qwen_36.py:1034-1044), which the
    paged kernel does not need."""
    from tileinfer_amd import workloads as wl
    from tileinfer_amd.kernels.gqa_prefill_paged import gqa_prefill_paged_fn

    chunk = chunk_slots.numel()
    table = torch.tensor(st.meta["chunk_blocks"], dtype=torch.int32, device=dev).view(1, -1)
    gen = torch.Generator(device=dev).manual_seed(6)
    q = torch.randn((chunk, HQ, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
    cu = torch.tensor([0, chunk], dtype=torch.int32, device=dev)
    sk = torch.tensor([chunk], dtype=torch.int32, device=dev)
    # The default ("auto") schedule chooses from host sizes, here with the max_seqlen_k the
    # reference's context carries; both schedules are also timed on their own.
    scheds = ("auto", "balanced", "per_unit")
    first_us, first_bal_us, first_pu_us = _time_interleaved(
        [functools.partial(gqa_prefill_paged_fn, q, kc, vc, table, cu, sk, chunk, schedule=sc,
                           max_seqlen_k=chunk) for sc in scheds], args.steps, args.warmup)
    first_flops = wl.prefill_flops([chunk], [chunk])
    cont = wl.config4_prefill(device=dev, cached=6144, chunk=chunk)
    kv_len = int(cont.seqlen_k[0])
    cont_us, cont_bal_us, cont_pu_us = _time_interleaved(
        [functools.partial(gqa_prefill_paged_fn, cont.q, cont.k_cache, cont.v_cache,
                           cont.block_table, cont.cu_seqlens_q, cont.seqlen_k, chunk, schedule=sc,
                           max_seqlen_k=kv_len) for sc in scheds], args.steps, args.warmup)
    cont_flops = cont.flops()
    pos = torch.arange(kv_len, device=dev)
    blocks = cont.block_table[0, pos // BLOCK].long()
    offs = pos % BLOCK
    gather_us = _time(lambda: (cont.k_cache[blocks, offs].contiguous(),
                               cont.v_cache[blocks, offs].contiguous()), args.steps, args.warmup)
    tf = lambda f, us: round(f / (us * 1e-6) / 1e12, 1)  # noqa: E731
    # "us": the default (automatic) schedule; then each schedule forced.
    return {"first_chunk": {"q_len": chunk, "kv_len": chunk, "us": round(first_us, 2),
                            "flops": first_flops, "TFLOPs": tf(first_flops, first_us),
                            "balanced_us": round(first_bal_us, 2),
                            "per_unit_us": round(first_pu_us, 2)},
            "continuation": {"q_len": chunk, "kv_len": kv_len, "us": round(cont_us, 2),
                             "flops": cont_flops, "TFLOPs": tf(cont_flops, cont_us),
                             "balanced_us": round(cont_bal_us, 2),
                             "per_unit_us": round(cont_pu_us, 2)},
            "reference_gather_of_continuation_us": round(gather_us, 2),
            "peak_TFLOPs_bf16_dense": 2500.0}


def metric_extras(kv, tables, seqlen, q, dev, args) -> dict:
    """The rest of the metric on the same cache (layer 0's pool, after the timed steps):
    * append GB/s at config 4's N = 2,080 (a 2,048-token chunk over 128 random blocks + 32 decode
      tokens) and at a bulk N = 65,536 (random distinct slots), as the reference benches a bulk
      store (kernels/kvcache_store.py:117-123); GPU time from a captured graph, since back-to-back
      eager calls of a few-µs kernel measure the Python wrapper;
    * the decode at the configured 2,048-token partitions (config 3) beside the balanced default;
    * a batch-64 decode sweep over context 256..32k (each sequence's first ctx/16 blocks of its
      permuted table), % of peak per point, as the reference's seqlen sweep
      (kernels/gqa_decode_paged.py:614-656); up to 2k also the GPU time per call from a captured
      graph, since an eager call of a few tens of µs partly measures the Python wrapper (at 256
      and 512 tokens the 256 (sequence, KV head) pairs take one workgroup each).
    All timed with HIP events on the launch stream (mean over --steps calls after --warmup)."""
    k_rows, v_rows, k_paged, v_paged = layer_views(kv, 0)
    nb = k_paged.shape[0]
    b, full_ctx = seqlen.shape[0], int(seqlen[0])
    gen = torch.Generator(device=dev).manual_seed(7)
    rnd = lambda *sh: torch.randn(sh, generator=gen, device=dev).to(torch.bfloat16)  # noqa: E731
    gbps = lambda nbytes, us: round(nbytes / (us * 1e-6) / 1e9, 1)  # noqa: E731
    res = {}
    blocks = torch.randperm(nb, generator=gen, device=dev)[:160].long()
    chunk = (blocks[:128, None] * BLOCK + torch.arange(BLOCK, device=dev)).reshape(-1)
    dec = blocks[128:] * BLOCK + torch.randint(0, BLOCK, (32,), generator=gen, device=dev)
    for name, slots in (("append_2080", torch.cat([chunk, dec]).to(torch.int32)),
                        ("append_65536", torch.randperm(nb * BLOCK, generator=gen,
                                                        device=dev)[:65536].to(torch.int32))):
        n = slots.numel()
        key, val = rnd(n, HKV, HEAD_DIM), rnd(n, HKV, HEAD_DIM)
        fn = lambda: store_kvcache(key, val, k_rows, v_rows, slots)  # noqa: E731
        eager = _time(fn, args.steps, args.warmup)
        us = _graph_us(fn)
        nbytes = append_bytes(slots, HKV * HEAD_DIM)
        res[name] = {"tokens": n, "us": round(us, 2), "GBps_algorithmic": gbps(nbytes, us),
                     "pct_of_peak_hbm": round(100 * nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 1),
                     "us_eager_call": round(eager, 2),
                     "timing": "us: GPU time per call from a captured graph of 20 calls; "
                               "us_eager_call: back-to-back Python calls (host-bound when small)"}
    d_bytes = decode_bytes([full_ctx] * b)
    for name, split in (("decode_balanced", None), ("decode_split_2048", 2048)):
        us = _time(lambda: gqa_decode_paged_fn(q[0], k_paged, v_paged, tables[0], seqlen, BLOCK,
                                               split_tokens=split), args.steps, args.warmup)
        res[name] = {"ctx": full_ctx, "us": round(us, 2), "GBps_algorithmic": gbps(d_bytes, us),
                     "pct_of_peak_hbm": round(100 * d_bytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 2)}
    sweep = []
    ctx = 256
    while ctx <= full_ctx:
        tb = tables[0][:, :ctx // BLOCK]
        sl = torch.full((b,), ctx, dtype=torch.int32, device=dev)
        fn = lambda: gqa_decode_paged_fn(q[0], k_paged, v_paged, tb, sl, BLOCK)  # noqa: E731
        us = _time(fn, args.steps, args.warmup)
        nbytes = decode_bytes([ctx] * b)
        point = {"ctx": ctx, "us": round(us, 2), "GBps_algorithmic": gbps(nbytes, us),
                 "pct_of_peak_hbm": round(100 * nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 2)}
        if ctx <= 2048:
            ug = _graph_us(fn)
            point["us_graph"] = round(ug, 2)
            point["pct_of_peak_hbm_graph"] = round(
                100 * nbytes / (ug * 1e-6) / 1e9 / PEAK_HBM_GBPS, 2)
        sweep.append(point)
        ctx *= 2
    res["decode_ctx_sweep_batch64"] = sweep
    res["other_configs"] = other_configs_decode(dev, args)
    res["decode_other_shapes"] = decode_shapes_extras(dev, args)
    res["prefill_config4"] = prefill_extras(dev, args)
    return res


def prefill_extras(dev, args) -> dict:
    """Config 4's paged prefill attention on its own seeded pages (the `--config 4` run times the
    same calls on the pages its append wrote): the 2,048-token first chunk (causal over itself)
    and a 2,048-token continuation over 6,144 cached tokens, with the default schedule and each
    schedule forced; HIP events on the launch stream."""
    from tileinfer_amd import workloads as wl
    from tileinfer_amd.kernels.gqa_prefill_paged import gqa_prefill_paged_fn

    res = {}
    for name, cached in (("first_chunk", 0), ("continuation", 6144)):
        w = wl.config4_prefill(device=dev, cached=cached)
        q_len, kv_len = int(w.q.shape[0]), int(w.seqlen_k[0])
        times = _time_interleaved(
            [functools.partial(gqa_prefill_paged_fn, w.q, w.k_cache, w.v_cache, w.block_table,
                               w.cu_seqlens_q, w.seqlen_k, q_len, schedule=sc,
                               max_seqlen_k=kv_len) for sc in ("auto", "balanced", "per_unit")],
            args.steps, args.warmup)
        flops = w.flops()
        res[name] = {"q_len": q_len, "kv_len": kv_len, "flops": flops,
                     "us": round(times[0], 2),
                     "TFLOPs": round(flops / (times[0] * 1e-6) / 1e12, 1),
                     "pct_of_peak_bf16_dense": round(100 * flops / (times[0] * 1e-6) / 2.5e15, 1),
                     "balanced_us": round(times[1], 2), "per_unit_us": round(times[2], 2)}
        if cached == 0:
            res["torch_sdpa_flash"] = {"first_chunk_causal": _sdpa_flash_us(w, True, args)}
        else:
            ours = _time(functools.partial(gqa_prefill_paged_fn, w.q, w.k_cache, w.v_cache,
                                           w.block_table, w.cu_seqlens_q, w.seqlen_k, q_len,
                                           causal=False, max_seqlen_k=kv_len),
                         args.steps, args.warmup)
            nc = wl.prefill_flops([q_len], [kv_len], causal=False)
            res["torch_sdpa_flash"]["noncausal_2048x8192"] = _sdpa_flash_us(w, False, args)
            res["noncausal_2048x8192"] = {"us": round(ours, 2), "flops": nc,
                                          "TFLOPs": round(nc / (ours * 1e-6) / 1e12, 1)}
        del w
    return res


def _sdpa_flash_us(w, causal: bool, args) -> dict:
    """The vendor reference point: torch.nn.functional.scaled_dot_product_attention with the
    flash backend forced (PyTorch-ROCm's prebuilt kernels) on the same queries over the step's K/V
    gathered into dense [1, H_q, S, D] tensors (K/V heads expanded to the 24 query heads), top-left
    causal mask (equal to the bottom-right one when S_q = S_k)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    from tileinfer_amd import workloads as wl

    q_len, kv_len = int(w.q.shape[0]), int(w.seqlen_k[0])
    if causal and q_len != kv_len:
        return {"us": None, "note": "top-left mask differs from the call's"}
    pos = torch.arange(kv_len, device=w.q.device)
    blocks = w.block_table[0, pos // BLOCK].long()
    dense = lambda c: c[blocks, pos % BLOCK].permute(1, 0, 2).repeat_interleave(  # noqa: E731
        HQ // HKV, dim=0).unsqueeze(0).contiguous()
    k, v = dense(w.k_cache), dense(w.v_cache)
    q = w.q.permute(1, 0, 2).unsqueeze(0).contiguous()
    flops = wl.prefill_flops([q_len], [kv_len], causal=causal)
    try:
        with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
            us = _time(lambda: torch.nn.functional.scaled_dot_product_attention(
                q, k, v, is_causal=causal), args.steps, args.warmup)
    except RuntimeError as e:
        return {"us": None, "note": f"flash backend unavailable: {str(e)[:100]}"}
    return {"us": round(us, 2), "TFLOPs": round(flops / (us * 1e-6) / 1e12, 1)}


def other_configs_decode(dev, args) -> dict:
    """One decode launch of BASELINE configs 1, 2, 4 and 5 at their stated sizes (their own seeded
    caches, separate from the config-3 slab), timed with HIP events; config 1 (a few microseconds
    of GPU work, below the wrapper's host time) also as GPU time per call in a captured graph;
    configs 1 and 2 are also checked against the CPU oracle, config 5 is timed both plain
    (cache-keeping policy) and with shared_prefix_tokens=8192."""
    from oracle.ref_torch import ref_gqa_decode_paged
    from tileinfer_amd import workloads as wl

    res = {}
    st = wl.config1(device=dev)
    ctx = st.seqlen.tolist()
    call = functools.partial(gqa_decode_paged_fn, st.q, st.k_cache, st.v_cache, st.block_table,
                             st.seqlen, BLOCK)
    split, max_splits, _ = decode_plan(1, HQ, HKV, HEAD_DIM, BLOCK, st.block_table.shape[1])
    g_us = _graph_us(call)
    res["config1"] = {"batch": 1, "ctx_sum": sum(ctx), "decode_us": round(_time(call, args.steps,
                                                                                 args.warmup), 2),
                      "decode_us_graph": round(g_us, 2),
                      "decode_GBps_algorithmic_graph": round(
                          decode_bytes(ctx) / (g_us * 1e-6) / 1e9, 1),
                      "partition": f"fixed {split} tokens, up to {max_splits} per sequence"
                      if split else "balanced" if max_splits else "one workgroup per (KV head, "
                      "sequence)"}
    out = call()
    ref = ref_gqa_decode_paged(st.q.cpu(), st.k_cache.cpu(), st.v_cache.cpu(),
                               st.block_table.cpu(), st.seqlen.cpu(), BLOCK).float()
    err = (out.float().cpu() - ref).abs()
    res["config1"]["decode_within_tol"] = bool((err <= 2e-2 + 1e-2 * ref.abs()).all())
    del st
    for cfg in (2, 4, 5):
        st = {2: wl.config2, 4: lambda device: wl.config4(device=device)[0],
              5: wl.config5}[cfg](device=dev)
        ctx = st.seqlen.tolist()
        nbytes = decode_bytes(ctx)
        # The unchanged call site's call (model/qwen_36.py:1071-1079 passes no hint): the cache
        # policy is chosen on the device.
        call = functools.partial(gqa_decode_paged_fn, st.q, st.k_cache, st.v_cache,
                                 st.block_table, st.seqlen, BLOCK)
        us = _time(call, args.steps, args.warmup)
        entry = {"batch": len(ctx), "ctx_sum": sum(ctx), "decode_us": round(us, 2),
                 "decode_GBps_algorithmic": round(nbytes / (us * 1e-6) / 1e9, 1),
                 "decode_pct_of_peak_hbm": round(100 * nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 2)}
        if cfg == 2:
            out = call()
            ref = ref_gqa_decode_paged(st.q.cpu(), st.k_cache.cpu(), st.v_cache.cpu(),
                                       st.block_table.cpu(), st.seqlen.cpu(), BLOCK).float()
            err = (out.float().cpu() - ref).abs()
            entry["decode_within_tol"] = bool((err <= 2e-2 + 1e-2 * ref.abs()).all())
            entry["decode_max_abs_err"] = round(float(err.max()), 6)
        if cfg == 5:
            pre = functools.partial(gqa_decode_paged_fn, st.q, st.k_cache, st.v_cache,
                                    st.block_table, st.seqlen, BLOCK,
                                    shared_prefix_tokens=st.meta["prefix_tokens"])
            entry["decode_us_shared_prefix"] = round(_time(pre, args.steps, args.warmup), 2)
            for name, reuse in (("decode_us_forced_keep", True), ("decode_us_forced_stream", False)):
                entry[name] = round(_time(functools.partial(call, kv_reuse=reuse), args.steps,
                                          args.warmup), 2)
            out = call()
            entry["policies_bitwise_equal"] = all(
                torch.equal(out.view(torch.int16), call(kv_reuse=r).view(torch.int16))
                for r in (True, False))
            entry["note"] = ("decode_us: the call with no keywords (cache policy chosen per "
                             "sequence on the device: the shared prefix pages are kept in "
                             "L2/MALL, so the logical % can exceed 100); forced_keep / "
                             "forced_stream: kv_reuse=True / False; shared_prefix: the "
                             "8,192-token prefix attended once for the batch")
        res[f"config{cfg}"] = entry
        del st
        if cfg == 5:
            entry["swap"] = swap_config5(dev, args)
    return res


def decode_shapes_extras(dev, args) -> dict:
    """The decode at head shapes and batch layouts besides the BASELINE configs (random tables,
    N(0,1) values, HIP events): the reference's own self-test shape at its default batch
    (kernels/gqa_decode_paged.py:472-512: B 32, 32 query / 8 KV heads, head_dim 128, 8k), head_dim
    128 at 64 x 32k, one 128k-token sequence, and 1,024 sequences of 512 tokens."""
    from tileinfer_amd import workloads as wl

    res = {}
    for name, b, ctx, hq, hkv, d in (("ref_selftest_b32_hq32_hkv8_d128_8k", 32, 8192, 32, 8, 128),
                                     ("b64_hq32_hkv8_d128_32k", 64, 32768, 32, 8, 128),
                                     ("b1_128k", 1, 131072, HQ, HKV, HEAD_DIM),
                                     ("b1024_512", 1024, 512, HQ, HKV, HEAD_DIM)):
        st = wl.make_step([ctx] * b, pool=b * ctx // BLOCK, seed=31, device=dev, hq=hq, hkv=hkv,
                          d=d)
        nbytes = decode_bytes([ctx] * b, hq=hq, hkv=hkv, d=d)
        us = _time(lambda: gqa_decode_paged_fn(st.q, st.k_cache, st.v_cache, st.block_table,
                                               st.seqlen, BLOCK), args.steps, args.warmup)
        res[name] = {"us": round(us, 2), "GBps_algorithmic": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "pct_of_peak_hbm": round(100 * nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 2)}
        del st
    return res


def config_parity(cfg: int, st, key, val, slots, out, dev) -> dict:
    """Parity on the run itself: appended rows bit-exact; the decode output of every sequence
    against the CPU oracle (max abs error; max relative error over outputs with |ref| >= 0.05;
    the largest fraction of atol 2e-2 + rtol 1e-2 · |ref| used); for config 5 the shared and
    the private prefix layout bitwise equal (plain call and shared-prefix call)."""
    from oracle.ref_torch import ref_gqa_decode_paged
    from tileinfer_amd import workloads as wl

    rows = lambda c: c.view(-1, HKV * HEAD_DIM)  # noqa: E731
    live = slots >= 0
    sl = slots[live].long()
    append_ok = all(torch.equal(rows(c)[sl].view(torch.int16),
                                x.reshape(-1, HKV * HEAD_DIM)[live].view(torch.int16))
                    for c, x in ((st.k_cache, key), (st.v_cache, val)))
    ref = ref_gqa_decode_paged(st.q.cpu(), st.k_cache.cpu(), st.v_cache.cpu(),
                               st.block_table.cpu(), st.seqlen.cpu(), BLOCK).float()
    err = (out.float().cpu() - ref).abs()
    big = ref.abs() >= 0.05
    res = {"append_bit_exact": append_ok,
           "decode_max_abs_err": round(float(err.max()), 6),
           "decode_max_rel_err": round(float((err[big] / ref[big].abs()).max()), 6)
           if bool(big.any()) else None,
           "decode_tol_used": round(float((err / (2e-2 + 1e-2 * ref.abs())).max()), 4),
           "decode_within_tol": bool((err <= 2e-2 + 1e-2 * ref.abs()).all()),
           "sequences_checked": int(st.seqlen.numel())}
    if cfg == 5:
        pv = wl.config5(device=dev, shared=False)  # same values, every prefix block a private copy
        store_kvcache(pv.k_new, pv.v_new, rows(pv.k_cache), rows(pv.v_cache), pv.slot_mapping)
        bits = lambda t: t.view(torch.int16)  # noqa: E731
        priv = gqa_decode_paged_fn(pv.q, pv.k_cache, pv.v_cache, pv.block_table, pv.seqlen,
                                   kv_reuse=True)
        res["shared_vs_private_bitwise"] = bool(torch.equal(bits(out), bits(priv)))
        prefix = st.meta["prefix_tokens"]
        a = gqa_decode_paged_fn(st.q, st.k_cache, st.v_cache, st.block_table, st.seqlen,
                                shared_prefix_tokens=prefix)
        b = gqa_decode_paged_fn(pv.q, pv.k_cache, pv.v_cache, pv.block_table, pv.seqlen,
                                shared_prefix_tokens=prefix)
        res["shared_vs_private_bitwise_shared_prefix_call"] = bool(torch.equal(bits(a), bits(b)))
        del pv, priv, a, b
    return res


def config_cpu_reference(st, key, val, slots) -> dict:
    """The CPU oracle (append + decode of the reference recipe) over the whole layer on the host
    cores: 1 warm-up, then the median of 3 runs."""
    from oracle.ref_torch import ref_gqa_decode_paged, ref_store_kvcache

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    kc, vc = st.k_cache.cpu(), st.v_cache.cpu()
    k, v, sl = key.cpu(), val.cpu(), slots.cpu()
    q, tb, sq = st.q.cpu(), st.block_table.cpu(), st.seqlen.cpu()

    def run():
        t0 = time.perf_counter()
        ref_store_kvcache(k, v, kc.view(-1, HKV * HEAD_DIM), vc.view(-1, HKV * HEAD_DIM), sl)
        ref_gqa_decode_paged(q, kc, vc, tb, sq, BLOCK)
        return time.perf_counter() - t0

    run()
    t = statistics.median([run() for _ in range(3)])
    return {"us_per_layer_step": round(t * 1e6, 1), "cores": cores, "kind": "port",
            "sample": f"the whole layer ({sq.numel()} sequences), append + decode by the CPU "
                      f"oracle (oracle/ref_torch.py), median of 3 after 1 warm-up"}


def run_config(cfg: int, args, dev) -> dict:
    """One attention layer of BASELINE config 1, 2, 4 or 5 (append, then decode), on the GPU."""
    from tileinfer_amd import workloads as wl

    extra = {}
    if cfg == 1:
        st = wl.config1(device=dev)
    elif cfg == 2:
        st = wl.config2(device=dev)
    elif cfg == 4:
        st, chunk_slots = wl.config4(device=dev)
    elif cfg == 5:
        st = wl.config5(device=dev)
    else:
        raise SystemExit(f"--config {cfg}: choose 1, 2, 3 (default), 4 or 5")
    kc, vc = st.k_cache, st.v_cache
    rows = lambda c: c.view(-1, HKV * HEAD_DIM)  # noqa: E731
    if cfg == 4:
        key = torch.cat([st.meta["chunk_k"], st.k_new])
        val = torch.cat([st.meta["chunk_v"], st.v_new])
        slots = torch.cat([chunk_slots, st.slot_mapping])
    else:
        key, val, slots = st.k_new, st.v_new, st.slot_mapping
    ctx = st.seqlen.tolist()
    a_us = _time(lambda: store_kvcache(key, val, rows(kc), rows(vc), slots), args.steps, args.warmup)
    # No cache-policy hint, as the unchanged call site passes none: chosen on the device.
    decode = functools.partial(gqa_decode_paged_fn, st.q, kc, vc, st.block_table, st.seqlen,
                               split_tokens=args.split_tokens, variant=args.variant)
    d_us = _time(decode, args.steps, args.warmup)
    # Back to back in a captured graph, as a serving loop replays its decode step: GPU time per
    # call with no host time between calls (a launch after the GPU idled starts its XCDs up to
    # ~4 us apart, which the event-timed figure of a small call includes).
    g_us = _graph_us(decode)
    a_bytes = append_bytes(slots, HKV * HEAD_DIM)
    d_bytes = decode_bytes(ctx)
    # Parity and the CPU reference on this state (the timed append, then decode), before the
    # extra measurements below write elsewhere in the pool.
    out = gqa_decode_paged_fn(st.q, kc, vc, st.block_table, st.seqlen,
                              split_tokens=args.split_tokens, variant=args.variant)
    checks = {"parity": config_parity(cfg, st, key, val, slots, out, dev)}
    if not args.no_cpu_baseline:
        checks["cpu_reference"] = config_cpu_reference(st, key, val, slots)
    if cfg == 4:
        # Also as two calls (chunk, then the 32 decode tokens), and a bulk append rate.
        two = _time(lambda: (store_kvcache(st.meta["chunk_k"], st.meta["chunk_v"], rows(kc),
                                           rows(vc), chunk_slots),
                             store_kvcache(st.k_new, st.v_new, rows(kc), rows(vc),
                                           st.slot_mapping)), args.steps, args.warmup)
        n = 65536
        gen = torch.Generator(device=dev).manual_seed(5)
        bk = torch.randn((n, HKV, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
        bv = torch.randn((n, HKV, HEAD_DIM), generator=gen, device=dev).to(torch.bfloat16)
        bs = torch.randperm(kc.shape[0] * BLOCK, generator=gen, device=dev)[:n].to(torch.int32)
        b_us = _time(lambda: store_kvcache(bk, bv, rows(kc), rows(vc), bs), args.steps, args.warmup)
        extra = {"append_two_calls_us": round(two, 2),
                 "append_bulk_65536_us": round(b_us, 2),
                 "append_bulk_GBps_algorithmic": round(append_bytes(bs, HKV * HEAD_DIM) / (b_us * 1e-6) / 1e9, 1),
                 "prefill": prefill_config4(st, chunk_slots, kc, vc, dev, args)}
    if cfg == 5:
        unique = int(torch.unique(st.block_table).numel())
        stream_us = _time(lambda: gqa_decode_paged_fn(st.q, kc, vc, st.block_table, st.seqlen,
                                                      split_tokens=args.split_tokens,
                                                      variant=args.variant, kv_reuse=False),
                          args.steps, args.warmup)
        keep_us = _time(lambda: gqa_decode_paged_fn(st.q, kc, vc, st.block_table, st.seqlen,
                                                    split_tokens=args.split_tokens,
                                                    variant=args.variant, kv_reuse=True),
                        args.steps, args.warmup)
        # The prefix attended once for the batch (the caller's statement that every sequence
        # shares its first 8192 tokens), against the plain call's output.
        prefix = st.meta["prefix_tokens"]
        # (The suffixes are each sequence's own pages, read once: the streaming cache policy.)
        shared_fn = lambda: gqa_decode_paged_fn(st.q, kc, vc, st.block_table, st.seqlen,  # noqa: E731
                                                 shared_prefix_tokens=prefix)
        shared_us = _time(shared_fn, args.steps, args.warmup)
        plain = gqa_decode_paged_fn(st.q, kc, vc, st.block_table, st.seqlen, kv_reuse=True)
        shared_err = float((shared_fn().float() - plain.float()).abs().max())
        extra = {"decode_us_streaming_policy": round(stream_us, 2),
                 "decode_us_keep_policy": round(keep_us, 2),
                 "decode_us_shared_prefix": round(shared_us, 2),
                 "decode_GBps_logical_shared_prefix": round(d_bytes / (shared_us * 1e-6) / 1e9, 1),
                 "shared_prefix_tokens": prefix,
                 "shared_prefix_max_abs_diff_vs_plain": shared_err,
                 "swap": swap_config5(dev, args),
                 "decode_logical_bytes": d_bytes,
                 "decode_physical_unique_kv_bytes": unique * 2 * BLOCK * HKV * HEAD_DIM * 2,
                 "note": "shared prefix blocks are re-read from L2/MALL, so the logical rate can "
                         "exceed HBM peak; rocprof FETCH_SIZE gives the HBM share"}
    split, max_splits, _ = decode_plan(len(ctx), HQ, HKV, HEAD_DIM, BLOCK,
                                       st.block_table.shape[1], args.split_tokens)
    return {
        "metric": METRIC, "config": {"workload": f"config{cfg}", "batch": len(ctx),
                                     "ctx_min": min(ctx), "ctx_max": max(ctx), "ctx_sum": sum(ctx),
                                     "append_tokens": slots.numel(),
                                     "partition": (f"fixed {split} tokens, up to {max_splits} per sequence"
                                                   if split else
                                                   f"balanced over {max_splits} workgroups"
                                                   if max_splits else
                                                   "one 4-wave workgroup per (KV head, sequence)"),
                                     "variant": args.variant},
        "decode_us": round(d_us, 2), "decode_GBps_algorithmic": round(d_bytes / (d_us * 1e-6) / 1e9, 1),
        "decode_pct_of_peak_hbm": round(100 * d_bytes / (d_us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 2),
        "decode_us_graph": round(g_us, 2),
        "decode_pct_of_peak_hbm_graph": round(100 * d_bytes / (g_us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 2),
        "append_us": round(a_us, 2), "append_GBps_algorithmic": round(a_bytes / (a_us * 1e-6) / 1e9, 1),
        "us_per_layer_step": round(a_us + d_us, 2), **extra, **checks,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--calibrate", action="store_true",
                    help="run only the copy/read calibration of known size and exit")
    ap.add_argument("--config", type=int, default=3,
                    help="BASELINE config: 3 (default, the headline line) or 1, 2, 4, 5 (one layer)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--layers", type=int, default=16)
    ap.add_argument("--variant", default="auto", choices=["auto", "mfma", "scalar"])
    ap.add_argument("--split-tokens", type=int, default=None)
    ap.add_argument("--seed", type=int, default=1003)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-parity", action="store_true")
    ap.add_argument("--no-fusions", action="store_true",
                    help="skip the unfused-vs-fused timing of the element-wise work around attention")
    ap.add_argument("--no-metadata", action="store_true",
                    help="skip the per-step metadata comparison (host builder vs device tables)")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the append sizes, 2,048-token partitions and context sweep")
    ap.add_argument("--sequential-tables", action="store_true",
                    help="diagnostic: contiguous blocks per sequence instead of random permutations")
    ap.add_argument("--page-size", type=int, default=BLOCK,
                    help="config 3's decode through pages of 1, 2, 4 or 8 tokens viewing the same "
                         "memory (the same tokens in the same 16-token tiles), default 16")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}): "
              "this build has no multi-GPU path (the path would shard by KV head or by sequence, "
              "neither of which exchanges K/V between GPUs).",
              file=sys.stderr)
        sys.exit(2)

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibrate:
        calibrate(dev)
        return
    if args.config != 3:
        print(json.dumps(run_config(args.config, args, dev)), flush=True)
        return
    b, ctx, layers = args.batch, args.ctx, args.layers
    log(f"allocating cache: batch {b} x ctx {ctx} x {layers} layers")
    kv, tables, slots, seqlen, q, k_new, v_new = build_state(b, ctx, layers, dev, args.seed,
                                                             args.sequential_tables)
    torch.cuda.synchronize()
    log(f"cache {kv.numel() * 2 / 2**30:.1f} GiB ready")
    page = args.page_size
    if page <= 0 or BLOCK % page:
        raise SystemExit(f"--page-size {page}: choose 1, 2, 4, 8 or 16")
    views = [layer_views(kv, l) for l in range(layers)]
    dec_tables = tables
    if page != BLOCK:
        # The same slab viewed as pages of `page` tokens: block i of a table becomes blocks
        # r i .. r i + r - 1 (r = 16 / page), the same rows in the same order.
        r = BLOCK // page
        cols = torch.arange(tables[0].shape[1] * r, device=dev)
        dec_tables = [(t[:, cols // r] * r + cols % r).to(torch.int32) for t in tables]
        views = [(kr, vr, kp.view(-1, page, HKV, HEAD_DIM), vp.view(-1, page, HKV, HEAD_DIM))
                 for kr, vr, kp, vp in views]
    split, max_splits, ws = decode_plan(b, HQ, HKV, HEAD_DIM, page, dec_tables[0].shape[1],
                                        args.split_tokens)

    def step(ev=None):
        out = None
        for l in range(layers):
            k_rows, v_rows, k_paged, v_paged = views[l]
            if ev is not None:
                ev[l][0].record()
            store_kvcache(k_new[l], v_new[l], k_rows, v_rows, slots[l])
            if ev is not None:
                ev[l][1].record()
            out = gqa_decode_paged_fn(q[l], k_paged, v_paged, dec_tables[l], seqlen, page,
                                      split_tokens=args.split_tokens, variant=args.variant)
            if ev is not None:
                ev[l][2].record()
        return out

    for i in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"warm-up done ({args.warmup} steps); timing {args.steps} steps")
    # The timed steps carry no per-call events (three events per layer cost ~1 % of a step); the
    # per-call append and decode times come from a second, instrumented run of as many steps.
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    out = None
    for s in range(args.steps):
        out = step()
    stop.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(stop)
    log(f"timed: {total_ms:.2f} ms total")
    evs = [[[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(layers)]
           for _ in range(args.steps)]
    for s in range(args.steps):
        step(evs[s])
    torch.cuda.synchronize()
    app_ms = [e[l][0].elapsed_time(e[l][1]) for e in evs for l in range(layers)]
    dec_ms = [e[l][1].elapsed_time(e[l][2]) for e in evs for l in range(layers)]

    # The append's own time: a 4 µs kernel between two events mostly measures the markers, so the
    # headline append figure is the GPU time of the same 64-token call captured in a HIP graph
    # (one layer's call, replayed; the events' figure is kept beside it under its own name).
    k_rows0, v_rows0, _, _ = views[0]
    app_graph_us = _graph_us(lambda: store_kvcache(k_new[0], v_new[0], k_rows0, v_rows0, slots[0]))

    ms_step = total_ms / args.steps
    a_bytes = append_bytes(slots[0], HKV * HEAD_DIM)
    d_bytes = decode_bytes([ctx] * b, page_size=page)
    step_bytes = layers * (a_bytes + d_bytes)
    dec_avg_us = statistics.mean(dec_ms) * 1e3
    app_avg_us = statistics.mean(app_ms) * 1e3
    dec_gbps = d_bytes / (dec_avg_us * 1e-6) / 1e9
    traffic = read_traffic()

    result = {
        "metric": METRIC,
        "value": round(step_bytes / (ms_step * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) K/V/q, random block permutations; resident in HBM",
        "config": {
            "workload": (f"config3: decode step of {layers} full-attention layers, batch {b} x "
                         f"context {ctx}, 24Q/4KV heads, head_dim 256, block 16, bf16; per layer "
                         f"append {b} tokens then split-K paged decode"),
            "batch": b, "ctx": ctx, "layers": layers,
            "partition": (f"balanced over {max_splits} workgroups" if split == 0
                          else f"fixed {split} tokens, up to {max_splits} per sequence"),
            "variant": args.variant,
            "tables": "sequential" if args.sequential_tables else "random permutation per layer",
            "page_size": page,
        },
        "us_per_layer_step": round(ms_step * 1e3 / layers, 2),
        "decode_us_per_layer": round(dec_avg_us, 2),
        "append_us_per_layer": round(app_graph_us, 2),
        "append_us_per_layer_events": round(app_avg_us, 2),
        "decode_GBps_algorithmic": round(dec_gbps, 1),
        "decode_pct_of_peak_hbm": round(100 * dec_gbps / PEAK_HBM_GBPS, 2),
        "decode_TFLOPs": round(decode_flops([ctx] * b) / (dec_avg_us * 1e-6) / 1e12, 2),
        "append_GBps_algorithmic": round(a_bytes / (app_graph_us * 1e-6) / 1e9, 2),
        "append_note": ("append_us_per_layer: GPU time of the 64-token store_kvcache call "
                        "captured in a HIP graph and replayed; append_us_per_layer_events: HIP "
                        "events around each call in the instrumented steps (marker overhead "
                        "included)"),
        "roofline": {
            "bound": "hbm",
            "achieved": round(dec_gbps, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(dec_gbps / PEAK_HBM_GBPS, 4),
            "traffic": traffic,
            "kernel": "decode launch (split-K partial + merge), one layer",
            "algorithmic_bytes_per_launch": d_bytes,
        },
    }
    if not args.no_extras:
        # The same step with each layer's append fused into its decode call (append=, bitwise the
        # same cache and output), timed against the two-call step; neither with per-layer events.
        def fused_step():
            for l in range(layers):
                _, _, k_paged, v_paged = views[l]
                gqa_decode_paged_fn(q[l], k_paged, v_paged, dec_tables[l], seqlen, page,
                                    split_tokens=args.split_tokens, variant=args.variant,
                                    append=(k_new[l], v_new[l], slots[l]))
        two_ms, fused_ms = (t / 1e3 for t in _time_interleaved([step, fused_step], args.steps,
                                                               args.warmup))
        result["fused_append_step"] = {
            "us_per_layer_step_two_calls": round(two_ms * 1e3 / layers, 2),
            "us_per_layer_step_fused": round(fused_ms * 1e3 / layers, 2),
            "GBps_step_fused": round(step_bytes / (fused_ms * 1e-3) / 1e9, 2),
            "note": "store_kvcache then gqa_decode_paged_fn per layer (the headline step), "
                    "against one gqa_decode_paged_fn(..., append=) call per layer; interleaved "
                    "rounds, no per-layer events in either"}
    if not args.no_fusions:
        log("fusions around attention: unfused vs fused (captured graphs)")
        result["fusions"] = fusions_compare(kv, tables, slots, seqlen, q, dev)
    if not args.no_metadata:
        log("per-step metadata: reference host builder vs device-resident tables")
        result["metadata"] = metadata_compare(b, ctx, dev)
    if not args.no_parity:
        log("full-size parity sample")
        result["parity"] = parity_sample(kv, tables, seqlen, q, k_new, v_new, out, layers - 1)
    if not args.no_extras:
        log("append at N=2,080 / 65,536, decode at 2,048-token partitions, context sweep")
        result["extras"] = metric_extras(kv, tables, seqlen, q, dev, args)
    if not args.no_cpu_baseline:
        log("CPU baseline (oracle) on a sample")
        result["cpu_baseline"] = cpu_baseline(kv, tables, seqlen, q, k_new, v_new)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
