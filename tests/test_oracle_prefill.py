"""Pins the prefill oracle (CPU only).

``prefill_fp64`` is checked against two things it does not share code with: the pinned decode
closed form (row i of a chunk is a single-query decode over the first ``kv_len - q_len + i + 1``
tokens, which pins the bottom-right mask alignment) and torch's own scaled_dot_product_attention
in float64 (causal square chunks and unmasked chunks). ``ref_gqa_prefill_paged`` (the reference
recipe with bf16 P) is then held to the decode tolerance of ``prefill_fp64``, with planted
mistakes (top-left mask, wrong KV head, dropped scale, one key short) that the check must catch.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.brute import decode_fp64, prefill_fp64
from oracle.ref_torch import ref_gqa_prefill_paged
from tileinfer_amd.workloads import prefill_step

ATOL, RTOL = 2e-2, 1e-2


def _np(step):
    return (step.q.double().numpy(), step.k_cache.double().numpy(), step.v_cache.double().numpy(),
            step.block_table.numpy(), step.cu_seqlens_q.numpy(), step.seqlen_k.numpy())


def _fp64(step, causal=True):
    return prefill_fp64(*_np(step), 16, causal)


def _ref(step, causal=True):
    return ref_gqa_prefill_paged(step.q, step.k_cache, step.v_cache, step.block_table,
                                 step.cu_seqlens_q, step.seqlen_k, 16, causal)


def _gathered(step, b):
    """[kv_len, H_kv, D] float64 K and V of sequence b, gathered with plain indexing."""
    kv = int(step.seqlen_k[b])
    rows = [int(step.block_table[b, j // 16]) * 16 + j % 16 for j in range(kv)]
    kf = step.k_cache.double().reshape(-1, *step.k_cache.shape[2:])
    vf = step.v_cache.double().reshape(-1, *step.v_cache.shape[2:])
    return kf[rows], vf[rows]


@pytest.mark.parametrize("q_lens,kv_lens", [([7], [7]), ([5], [40]), ([16, 3, 0], [48, 3, 9]),
                                            ([33], [70])])
def test_fp64_rows_equal_single_query_decode(q_lens, kv_lens):
    """Row i of a chunk = decode of that query over the first kv_len - q_len + i + 1 tokens."""
    step = prefill_step(q_lens, kv_lens, seed=11, hq=6, hkv=2, d=32)
    want = _fp64(step)
    q, kc, vc, bt, cu, sk = _np(step)
    for b, (ql, kvl) in enumerate(zip(q_lens, kv_lens)):
        for i in range(ql):
            row = cu[b] + i
            ctx = np.array([kvl - ql + i + 1], dtype=np.int32)
            dec = decode_fp64(q[row:row + 1], kc, vc, bt[b:b + 1], ctx, 16)
            np.testing.assert_allclose(want[row], dec[0], rtol=1e-12, atol=1e-12)


def _sdpa(step, b, causal):
    """torch's float64 attention for sequence b (KV heads repeated over their query group)."""
    k, v = _gathered(step, b)
    cu = step.cu_seqlens_q.tolist()
    q = step.q.double()[cu[b]:cu[b + 1]].transpose(0, 1)          # [Hq, q_len, D]
    g = step.q.shape[1] // k.shape[1]
    k = k.transpose(0, 1).repeat_interleave(g, dim=0)             # [Hq, kv_len, D]
    v = v.transpose(0, 1).repeat_interleave(g, dim=0)
    return F.scaled_dot_product_attention(q, k, v, is_causal=causal).transpose(0, 1)


@pytest.mark.parametrize("causal", [True, False])
def test_fp64_equals_torch_sdpa(causal):
    """First chunks (kv_len == q_len: both mask alignments coincide) and unmasked chunks."""
    q_lens = [9, 31, 64]
    kv_lens = q_lens if causal else [20, 31, 100]
    step = prefill_step(q_lens, kv_lens, seed=12, hq=6, hkv=2, d=32)
    want = _fp64(step, causal)
    cu = step.cu_seqlens_q.tolist()
    for b in range(len(q_lens)):
        np.testing.assert_allclose(want[cu[b]:cu[b + 1]], _sdpa(step, b, causal).numpy(),
                                   rtol=1e-10, atol=1e-12)


def test_fp64_zero_rows():
    """A sequence with no cached token, and rows whose visible range is empty, give zeros."""
    step = prefill_step([4, 3], [0, 2], seed=13, hq=4, hkv=2, d=16)
    out = _fp64(step)
    assert not out[:4].any()          # kv_len 0
    assert not out[4].any()           # offset -1: row 0 sees nothing
    assert out[5].any() and out[6].any()


@pytest.mark.parametrize("q_lens,kv_lens,causal", [
    ([64], [64], True), ([37], [300], True), ([16, 1, 0, 50], [16, 200, 5, 51], True),
    ([40], [90], False)])
def test_ref_recipe_within_tolerance_of_fp64(q_lens, kv_lens, causal):
    step = prefill_step(q_lens, kv_lens, seed=14)
    np.testing.assert_allclose(_ref(step, causal).float().numpy(), _fp64(step, causal),
                               atol=ATOL, rtol=RTOL)


def test_ref_recipe_physical_layout_invariance():
    """Permuting which physical block holds which page leaves the output bitwise unchanged."""
    step = prefill_step([20, 7], [70, 33], seed=15)
    perm = torch.randperm(step.k_cache.shape[0], generator=torch.Generator().manual_seed(3))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    k2, v2 = step.k_cache[perm], step.v_cache[perm]
    bt2 = torch.where(step.block_table >= 0, inv[step.block_table.clamp(min=0).long()].int(),
                      step.block_table)
    base = _ref(step)
    moved = ref_gqa_prefill_paged(step.q, k2, v2, bt2, step.cu_seqlens_q, step.seqlen_k, 16)
    assert torch.equal(base.view(torch.int16), moved.view(torch.int16))


def _mutant_top_left(step):
    """Planted mistake: the causal mask aligned top-left (query i sees keys 0..i)."""
    out = torch.zeros_like(step.q)
    cu = step.cu_seqlens_q.tolist()
    for b in range(len(cu) - 1):
        ql = cu[b + 1] - cu[b]
        kv = int(step.seqlen_k[b])
        k, v = _gathered(step, b)
        for i in range(ql):
            for h in range(step.q.shape[1]):
                kh = h // (step.q.shape[1] // k.shape[1])
                n = min(i + 1, kv)
                s = k[:n, kh] @ step.q[cu[b] + i, h].double() / k.shape[-1] ** 0.5
                out[cu[b] + i, h] = (torch.softmax(s, 0) @ v[:n, kh]).to(out.dtype)
    return out


def _mutant_head_mod(step):
    """Planted mistake: query head h reads KV head h % H_kv instead of h // G."""
    out = torch.zeros_like(step.q)
    cu = step.cu_seqlens_q.tolist()
    hq = step.q.shape[1]
    for b in range(len(cu) - 1):
        ql = cu[b + 1] - cu[b]
        kv = int(step.seqlen_k[b])
        k, v = _gathered(step, b)
        for i in range(ql):
            vis = kv - ql + i + 1
            for h in range(hq):
                kh = h % k.shape[1]
                s = k[:vis, kh] @ step.q[cu[b] + i, h].double() / k.shape[-1] ** 0.5
                out[cu[b] + i, h] = (torch.softmax(s, 0) @ v[:vis, kh]).to(out.dtype)
    return out


def _mutant_no_scale(step):
    """Planted mistake: the D^-1/2 score scale dropped."""
    return ref_gqa_prefill_paged(step.q * 16.0, step.k_cache, step.v_cache, step.block_table,
                                 step.cu_seqlens_q, step.seqlen_k, 16)


def _mutant_one_key_short(step):
    """Planted mistake: each query misses its own position (sees keys < kv_len - q_len + i)."""
    return ref_gqa_prefill_paged(step.q, step.k_cache, step.v_cache, step.block_table,
                                 step.cu_seqlens_q, (step.seqlen_k - 1).clamp(min=0), 16)


@pytest.mark.parametrize("mutant", [_mutant_top_left, _mutant_head_mod, _mutant_no_scale,
                                    _mutant_one_key_short])
def test_checks_catch_planted_mistakes(mutant):
    step = prefill_step([24, 9], [60, 9], seed=16)
    exact = _fp64(step)
    np.testing.assert_allclose(_ref(step).float().numpy(), exact, atol=ATOL, rtol=RTOL)
    with pytest.raises(AssertionError):
        np.testing.assert_allclose(mutant(step).float().numpy(), exact, atol=ATOL, rtol=RTOL)
