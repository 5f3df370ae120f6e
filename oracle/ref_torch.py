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
