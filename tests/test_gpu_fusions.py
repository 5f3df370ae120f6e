"""The fusions on either side of the path, through the C ABI: QK-norm + RoPE (+ append) against
the oracle, the fused append bitwise against the unfused kernels, the sigmoid gate, and decode
with the gate in its epilogue bitwise against decode followed by the gate, and the same for the
paged prefill."""
import pytest
import torch

from helpers import bits, flat, say
from oracle.ref_torch import ref_qknorm_rope, ref_qknorm_rope_fp32, ref_sigmoid_mul
from tileinfer_amd.kernels import (fused_qknorm_rope, fused_sigmoid_mul, gqa_decode_paged_fn,
                                   qknorm_rope, qknorm_rope_append, store_kvcache)
from tileinfer_amd.kernels.gqa_prefill_paged import gqa_prefill_paged_fn
from tileinfer_amd.workloads import make_step, prefill_step

pytestmark = pytest.mark.gpu


def angles(n, rd, base=1e7, dtype=torch.bfloat16):
    inv = 1.0 / base ** (torch.arange(0, rd, 2).float() / rd)
    f = (torch.arange(n).float() * 97.0)[:, None] * inv[None, :]
    emb = torch.cat([f, f], dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def inputs(t, h, d, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = (3 * torch.randn(t, h, d, generator=g)).to(dtype)
    w = (0.2 * torch.randn(d, generator=g)).to(dtype)
    return x, w


def near_exact(out, ref):
    """Within the reference test's tolerance, and identical for nearly every element (the only
    differences are fp32 reduction order flipping a final rounding)."""
    out, ref = out.cpu(), ref.cpu()
    torch.testing.assert_close(out, ref, rtol=1e-2, atol=1e-2)
    same = (bits(out) == bits(ref)).float().mean().item()
    assert same > 0.99, same


@pytest.mark.parametrize("t,h,d,rd,dtype", [(7, 24, 256, 64, torch.bfloat16),
                                            (33, 4, 256, 64, torch.bfloat16),
                                            (5, 8, 128, 128, torch.float16),
                                            (3, 2, 128, 0, torch.bfloat16)])
def test_qknorm_rope_vs_oracle(t, h, d, rd, dtype, dev):
    say(f"qknorm_rope t={t} h={h} d={d} rd={rd} {dtype}")
    x, w = inputs(t, h, d, seed=t + h, dtype=dtype)
    cos, sin = angles(t, rd, dtype=dtype)
    out = qknorm_rope(x.to(dev), w.to(dev), cos.to(dev), sin.to(dev))
    near_exact(out, ref_qknorm_rope(x, w, cos, sin))


def test_fused_qknorm_rope_dropin_reference_test(dev):
    """The reference's own test (kernels/qknorm_rope.py:86-110): [4, 8, 1, 128], rotary 64, one
    cos/sin vector, against its fp32 reference at its tolerance."""
    say("fused_qknorm_rope reference test shape")
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4, 8, 1, 128, generator=g).to(torch.bfloat16)
    w = torch.randn(128, generator=g).to(torch.bfloat16)
    cos, sin = angles(1, 64)
    y = fused_qknorm_rope(x.to(dev), w.to(dev), cos[0].to(dev), sin[0].to(dev))
    assert y.shape == (4, 8, 1, 128)
    ref = ref_qknorm_rope_fp32(x, w, cos.expand(4, 1, 64), sin.expand(4, 1, 64))
    torch.testing.assert_close(y.cpu(), ref, rtol=1e-2, atol=1e-2)
    near_exact(y.view(4, 8, 128), ref_qknorm_rope(x.view(4, 8, 128), w, cos[0], sin[0]))


@pytest.mark.parametrize("t,d", [(64, 256), (300, 256), (9, 128)])
def test_fused_append_equals_unfused(t, d, dev):
    """One launch = qknorm_rope(q), qknorm_rope(k), store_kvcache(k', v): bitwise, including
    skipped (-1) slots; untouched rows stay as they were."""
    say(f"qknorm_rope_append t={t} d={d}")
    hq, hkv, slots_n = 24, 4, 2048
    q, qw = inputs(t, hq, d, seed=1)
    k, kw = inputs(t, hkv, d, seed=2)
    v, _ = inputs(t, hkv, d, seed=3)
    cos, sin = angles(t, 64)
    g = torch.Generator().manual_seed(4)
    slots = torch.randperm(slots_n, generator=g)[:t].to(torch.int32)
    slots[::7] = -1
    kc0 = torch.randn(slots_n, hkv * d, generator=g).to(torch.bfloat16)
    vc0 = torch.randn(slots_n, hkv * d, generator=g).to(torch.bfloat16)
    to = lambda x: x.to(dev)  # noqa: E731
    kc, vc = to(kc0), to(vc0)
    q_out = qknorm_rope_append(to(q), to(k), to(v), to(qw), to(kw), to(cos), to(sin), kc, vc,
                               to(slots))
    q_ref = qknorm_rope(to(q), to(qw), to(cos), to(sin))
    k_ref = qknorm_rope(to(k), to(kw), to(cos), to(sin))
    kc2, vc2 = to(kc0), to(vc0)
    store_kvcache(k_ref, to(v), kc2, vc2, to(slots))
    assert torch.equal(bits(q_out), bits(q_ref))
    assert torch.equal(bits(kc), bits(kc2))
    assert torch.equal(bits(vc), bits(vc2))
    near_exact(q_out, ref_qknorm_rope(q, qw, cos, sin))


@pytest.mark.parametrize("n", [2, 4096, 24 * 256 * 3 + 1])
def test_sigmoid_mul_vs_oracle(n, dev):
    say(f"sigmoid_mul n={n}")
    g = torch.Generator().manual_seed(n)
    a = (4 * torch.randn(n, generator=g)).to(torch.bfloat16)
    b = (4 * torch.randn(n, generator=g)).to(torch.bfloat16)
    out = fused_sigmoid_mul(a.to(dev), b.to(dev))
    near_exact(out, ref_sigmoid_mul(a, b))


@pytest.mark.parametrize("ctx,split", [([300, 5000, 0, 17], None), ([3000, 1, 4097], 1024),
                                       ([64] * 3, None)])
def test_gated_decode_equals_decode_then_gate(ctx, split, dev):
    """Decode with the gate in its epilogue = decode, then fused_sigmoid_mul: bitwise, for whole
    sequences, sequences cut between workgroups, empty sequences and a fixed split."""
    say(f"gated decode ctx={ctx} split={split}")
    step = make_step(ctx, pool=sum((c + 15) // 16 for c in ctx) + 8, seed=31)
    g = torch.Generator().manual_seed(5)
    gate = (3 * torch.randn(len(ctx), 1, 24 * 256, generator=g)).to(torch.bfloat16).to(dev)
    args = (step.q.to(dev), step.k_cache.to(dev), step.v_cache.to(dev), step.block_table.to(dev),
            step.seqlen.to(dev))
    plain = gqa_decode_paged_fn(*args, split_tokens=split)
    gated = gqa_decode_paged_fn(*args, split_tokens=split, gate=gate)
    ref = fused_sigmoid_mul(plain, gate.view(len(ctx), 24, 256))
    assert torch.equal(bits(gated), bits(ref))


@pytest.mark.parametrize("schedule", ["balanced", "per_unit"])
@pytest.mark.parametrize("q_lens,kv_lens,d,hq,hkv", [
    ([300, 7, 0, 129], [900, 7, 5, 2000], 256, 24, 4),   # cut units, a whole one, an empty chunk
    ([2048], [8192], 256, 24, 4),                        # config 4's continuation chunk
    ([100, 33], [600, 33], 128, 16, 2),
])
def test_gated_prefill_equals_prefill_then_gate(q_lens, kv_lens, d, hq, hkv, schedule, dev):
    """Prefill with the gate in its epilogue = prefill, then fused_sigmoid_mul: bitwise, for rows
    the attention kernel stores and rows the merge kernel stores (balanced schedule), with the
    gate as the model holds it (q_gate [1, total_q, H_q * D])."""
    say(f"gated prefill q_lens={q_lens} kv_lens={kv_lens} d={d} schedule={schedule}")
    step = prefill_step(q_lens, kv_lens, seed=32, hq=hq, hkv=hkv, d=d)
    total_q = step.q.shape[0]
    g = torch.Generator().manual_seed(6)
    gate = (3 * torch.randn(1, total_q, hq * d, generator=g)).to(torch.bfloat16).to(dev)
    args = (step.q.to(dev), step.k_cache.to(dev), step.v_cache.to(dev), step.block_table.to(dev),
            step.cu_seqlens_q.to(dev), step.seqlen_k.to(dev), step.max_seqlen_q, step.page_size)
    plain = gqa_prefill_paged_fn(*args, schedule=schedule)
    gated = gqa_prefill_paged_fn(*args, schedule=schedule, gate=gate)
    ref = fused_sigmoid_mul(plain, gate.view(total_q, hq, d))
    assert torch.equal(bits(gated), bits(ref))


def test_fused_decode_step_graph_capture_replay(dev):
    """A whole fused decode step — QK-norm + RoPE + append in one launch, then decode with the gate
    in its epilogue — captured in a HIP graph: every replay, with new inputs and eager work
    between, matches the eager step bitwise (outputs and cache)."""
    say("fused decode step graph capture")
    step = make_step([700, 33, 1500], pool=200, seed=34)
    b = step.q.shape[0]
    kc, vc = step.k_cache.to(dev), step.v_cache.to(dev)
    q, k, v = step.q.to(dev), step.k_new.to(dev), step.v_new.to(dev)
    _, qw = inputs(1, 1, 256, seed=5)
    _, kw = inputs(1, 1, 256, seed=6)
    qw, kw = qw.to(dev), kw.to(dev)
    cos, sin = (x.to(dev) for x in angles(b, 64))
    slots, tbl, seq = step.slot_mapping.to(dev), step.block_table.to(dev), step.seqlen.to(dev)
    gate = torch.zeros(b, 1, 24 * 256, dtype=torch.bfloat16, device=dev)

    def fn():
        qo = qknorm_rope_append(q, k, v, qw, kw, cos, sin, flat(kc), flat(vc), slots)
        return gqa_decode_paged_fn(qo, kc, vc, tbl, seq, gate=gate)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = fn()
    gen = torch.Generator(device=dev).manual_seed(7)
    for r in range(3):
        for x in (q, k, v, gate):
            x.copy_((2 * torch.randn(x.shape, generator=gen, device=dev)).to(x.dtype))
        graph.replay()
        torch.cuda.synchronize()
        kc_g, vc_g, out_g = kc.clone(), vc.clone(), static_out.clone()
        eager = fn()
        torch.cuda.synchronize()
        assert torch.equal(bits(out_g), bits(eager)), f"replay {r}"
        assert torch.equal(bits(kc_g), bits(kc)) and torch.equal(bits(vc_g), bits(vc)), f"cache {r}"
