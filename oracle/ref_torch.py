"""Restatement of the reference's PyTorch implementations of the two kernels (CPU). TEST ONLY.

These follow tileInfer's own torch references operation by operation, so their rounding matches:
  * ``ref_store_kvcache``    — kernels/kvcache_store.py:74-84 (a per-token loop with ``.item()``);
  * ``ref_gqa_decode_paged`` — kernels/gqa_decode_paged.py:444-461: per sequence, gather the used
    pages through the block table, then per KV head ``scores = (q_h @ K^T) * D^-1/2`` in the input
    dtype, ``softmax(scores.float())`` cast back to the input dtype, ``weights @ V`` in the input
    dtype, into a zero-initialised output.
A negative block id inside the used pages wraps to the last block (Python indexing), exactly as
the reference's gather does; the GPU path treats it as absent instead, so tests never pass one.
"""
from __future__ import annotations

import torch


def ref_store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                      v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """In-place: rows ``slot_mapping[i] >= 0`` of the flat caches receive key/value row i."""
    n, num_heads, head_dim = key.shape
    d = num_heads * head_dim
    key_flat = key.reshape(n, d)
    value_flat = value.reshape(n, d)
    for i in range(n):
        slot = slot_mapping[i].item()
        if slot >= 0:
            k_cache[slot] = key_flat[i]
            v_cache[slot] = value_flat[i]


def ref_gqa_decode_paged(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                         block_table: torch.Tensor, seqlen_kv: torch.Tensor,
                         page_size: int = 16) -> torch.Tensor:
    """[B, H_q, D] decode output of the reference recipe, computed on whatever device q is on."""
    b_sz, h_q, d = q.shape
    h_kv = k_cache.shape[2]
    groups = h_q // h_kv
    output = torch.zeros(b_sz, h_q, d, dtype=q.dtype, device=q.device)
    scale = d ** -0.5
    for b in range(b_sz):
        seq_len = int(seqlen_kv[b].item())
        num_used_pages = (seq_len + page_size - 1) // page_size
        pages = block_table[b, :num_used_pages].long()
        k_full = k_cache[pages].reshape(-1, h_kv, d)[:seq_len]
        v_full = v_cache[pages].reshape(-1, h_kv, d)[:seq_len]
        for kv_h in range(h_kv):
            q_h = q[b, kv_h * groups:(kv_h + 1) * groups, :]
            scores = torch.matmul(q_h, k_full[:, kv_h, :].T) * scale
            weights = torch.softmax(scores.float(), dim=-1).to(q.dtype)
            output[b, kv_h * groups:(kv_h + 1) * groups, :] = torch.matmul(weights,
                                                                            v_full[:, kv_h, :])
    return output


def ref_gqa_prefill_paged(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                          block_table: torch.Tensor, cu_seqlens_q: torch.Tensor,
                          seqlen_k: torch.Tensor, page_size: int = 16,
                          causal: bool = True) -> torch.Tensor:
    """[total_q, H_q, D] chunked-prefill attention of the reference recipe.

    Gather: model/qwen_36.py:1034-1044 — positions ``0..kv_len-1`` of sequence b through
    ``block_table[b]`` (``positions // page_size`` into the table, ``positions % page_size`` in
    the page). Math: kernels/gqa_varlen.py:88-175 with one key tile covering the whole context —
    ``S = Q K^T`` in fp32 from the input dtype, keys ``j > kv_len - q_len + i`` masked to -inf
    under ``causal`` (120-131), ``P = exp2(S·scale - max·scale)`` with ``scale = D^-1/2 log2 e``
    (44, 150-154), ``l = sum(P)`` in fp32 (155-157), ``P`` rounded to the input dtype before
    ``P @ V`` (160-162), ``O = acc / l`` rounded to the input dtype, 0 where ``l == 0``
    (166-175). The kernel's online softmax over 16/64-key tiles rounds P relative to the running
    maximum instead, a difference well inside the bf16 tolerance.
    """
    total_q, h_q, d = q.shape
    h_kv = k_cache.shape[2]
    groups = h_q // h_kv
    scale = (1.0 / d) ** 0.5 * 1.44269504
    out = torch.zeros(total_q, h_q, d, dtype=q.dtype, device=q.device)
    k_flat = k_cache.reshape(-1, h_kv, d)
    v_flat = v_cache.reshape(-1, h_kv, d)
    cu = cu_seqlens_q.tolist()
    for b in range(block_table.shape[0]):
        q0, q1 = cu[b], cu[b + 1]
        q_len = q1 - q0
        kv_len = int(seqlen_k[b].item())
        if q_len <= 0:
            continue
        positions = torch.arange(kv_len)
        rows = block_table[b, positions // page_size].long() * page_size + positions % page_size
        k_full = k_flat[rows]
        v_full = v_flat[rows]
        offset = kv_len - q_len
        qi = torch.arange(q_len).unsqueeze(1)
        kj = torch.arange(kv_len).unsqueeze(0)
        masked = (qi + offset < kj) if causal else torch.zeros(q_len, kv_len, dtype=torch.bool)
        for h in range(h_q):
            kvh = h // groups
            s = q[q0:q1, h, :].float() @ k_full[:, kvh, :].float().T
            s = s.masked_fill(masked, float("-inf"))
            m = s.max(dim=1, keepdim=True).values if kv_len else torch.full((q_len, 1), -torch.inf)
            m_use = torch.where(torch.isinf(m), torch.zeros_like(m), m)
            p = torch.exp2(s * scale - m_use * scale)
            l = p.sum(dim=1, keepdim=True)
            acc = p.to(q.dtype).float() @ v_full[:, kvh, :].float()
            o = torch.where(l > 0, acc / torch.where(l > 0, l, torch.ones_like(l)),
                            torch.zeros_like(acc))
            out[q0:q1, h, :] = o.to(q.dtype)
    return out


def ref_qknorm_rope(x: torch.Tensor, weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                    eps: float = 1e-5) -> torch.Tensor:
    """QK-norm + partial RoPE as the reference's fused kernel computes it, rows ``[..., D]``.

    kernels/qknorm_rope.py:29-49: sum of squares in fp32, ``rsqrt(sum / D + eps)``, scale by
    ``(1 + w)`` and round the normalised row to the input dtype (33-39); then for i < h =
    rotary_dim/2, in fp32 from those rounded values, ``out[i] = y[i] c[i] - y[i+h] s[i]`` and
    ``out[i+h] = y[i+h] c[i] + y[i] s[i]`` with ``c, s = cos/sin[:h]`` (41-48), rounded once; the
    rest passes through. ``cos``/``sin`` are ``[rotary_dim]`` or ``[..tokens.., rotary_dim]``
    broadcasting against ``x`` without its head axis (``x`` is ``[T, H, D]``).
    """
    d = x.shape[-1]
    xf = x.float()
    r = torch.rsqrt((xf * xf).sum(-1, keepdim=True) / d + eps)
    y = (xf * r * (1.0 + weight.float())).to(x.dtype).float()
    rd = cos.shape[-1]
    half = rd // 2
    if rd == 0:
        return y.to(x.dtype)
    c = cos[..., :half].float()
    s = sin[..., :half].float()
    if c.dim() == 2:          # per token: [T, half] -> [T, 1, half]
        c, s = c.unsqueeze(1), s.unsqueeze(1)
    y1, y2 = y[..., :half], y[..., half:rd]
    out = torch.cat([y1 * c - y2 * s, y2 * c + y1 * s, y[..., rd:]], dim=-1)
    return out.to(x.dtype)


def ref_qknorm_rope_fp32(x: torch.Tensor, weight: torch.Tensor, cos: torch.Tensor,
                         sin: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """The reference's own fp32 check of that kernel (kernels/qknorm_rope.py:58-84): everything in
    fp32, ``mean(x^2)``, one rounding at the end. ``x`` ``[B, H, 1, D]``, cos/sin ``[B, 1, rd]``."""
    xf = x.float()
    xn = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    xn = (1.0 + weight.float()) * xn
    rd = cos.shape[-1]
    half = rd // 2
    rot1, rot2 = xn[..., :half], xn[..., half:rd]
    c = cos[..., :half].unsqueeze(2).float()
    s = sin[..., :half].unsqueeze(2).float()
    out = torch.cat([rot1 * c - rot2 * s, rot2 * c + rot1 * s, xn[..., rd:]], dim=-1)
    return out.to(x.dtype)


def ref_sigmoid_mul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``a * sigmoid(b)`` in fp32, rounded once (kernels/act_mul.py:81-114)."""
    return (a.float() * torch.sigmoid(b.float())).to(a.dtype)
