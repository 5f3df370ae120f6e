"""Closed forms of the two operations on numpy arrays (float64 for attention). TEST ONLY.

``store_np`` is the append's definition: a copy of the cache with rows ``slot >= 0`` replaced.
``decode_fp64`` is textbook single-query softmax attention per (sequence, query head) over the
logical context gathered through the block table, in float64 — the mathematical value the
reference's recipe (kernels/gqa_decode_paged.py:444-461) approximates in bf16/fp32.
``decode_loop_fp64`` is the same thing written as explicit scalar loops, for tiny inputs only, so
the vectorised form is checked against an independent spelling.
"""
from __future__ import annotations

import math

import numpy as np


def store_np(key: np.ndarray, value: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
             slot_mapping: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Return (k_cache', v_cache') after the append; inputs are not modified.

    Works on any dtype (use uint16 views of bf16 for bit-exact comparisons).
    """
    n = key.shape[0]
    kf = key.reshape(n, -1)
    vf = value.reshape(n, -1)
    k_out = k_cache.copy()
    v_out = v_cache.copy()
    for i in range(n):
        s = int(slot_mapping[i])
        if s >= 0:
            k_out[s] = kf[i]
            v_out[s] = vf[i]
    return k_out, v_out


def gather_context(cache: np.ndarray, table: np.ndarray, ctx: int, page_size: int) -> np.ndarray:
    """[ctx, H_kv, D] rows of one sequence from a [num_pages*page_size, H_kv, D] flat cache."""
    pos = np.arange(ctx)
    rows = table[pos // page_size].astype(np.int64) * page_size + pos % page_size
    return cache[rows]


def decode_fp64(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, block_table: np.ndarray,
                seqlen: np.ndarray, page_size: int = 16) -> np.ndarray:
    """float64 [B, H_q, D]; caches are [num_blocks, block_size, H_kv, D] (any float dtype)."""
    b_sz, h_q, d = q.shape
    h_kv = k_cache.shape[2]
    g = h_q // h_kv
    kf = np.asarray(k_cache, dtype=np.float64).reshape(-1, h_kv, d)
    vf = np.asarray(v_cache, dtype=np.float64).reshape(-1, h_kv, d)
    qf = np.asarray(q, dtype=np.float64)
    out = np.zeros((b_sz, h_q, d), dtype=np.float64)
    for b in range(b_sz):
        ctx = int(seqlen[b])
        if ctx <= 0:
            continue
        k = gather_context(kf, block_table[b], ctx, page_size)
        v = gather_context(vf, block_table[b], ctx, page_size)
        for h in range(h_q):
            s = k[:, h // g, :] @ qf[b, h] / math.sqrt(d)
            w = np.exp(s - s.max())
            out[b, h] = (w / w.sum()) @ v[:, h // g, :]
    return out


def decode_loop_fp64(q, k_cache, v_cache, block_table, seqlen, page_size=16):
    """Scalar-loop spelling of decode_fp64 (tiny inputs only)."""
    b_sz, h_q, d = len(q), len(q[0]), len(q[0][0])
    h_kv = len(k_cache[0][0])
    g = h_q // h_kv
    out = [[[0.0] * d for _ in range(h_q)] for _ in range(b_sz)]
    for b in range(b_sz):
        ctx = int(seqlen[b])
        for h in range(h_q):
            kvh = h // g
            scores = []
            for j in range(ctx):
                blk = int(block_table[b][j // page_size])
                off = j % page_size
                acc = 0.0
                for e in range(d):
                    acc += float(q[b][h][e]) * float(k_cache[blk][off][kvh][e])
                scores.append(acc / math.sqrt(d))
            if not scores:
                continue
            m = max(scores)
            ws = [math.exp(s - m) for s in scores]
            tot = sum(ws)
            for j in range(ctx):
                blk = int(block_table[b][j // page_size])
                off = j % page_size
                for e in range(d):
                    out[b][h][e] += ws[j] / tot * float(v_cache[blk][off][kvh][e])
    return out


def prefill_fp64(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                 block_table: np.ndarray, cu_seqlens_q: np.ndarray, seqlen_k: np.ndarray,
                 page_size: int = 16, causal: bool = True) -> np.ndarray:
    """float64 [total_q, H_q, D]: textbook softmax attention of every chunk query row.

    Query i of sequence b (q_len rows, kv_len cached tokens) sits at absolute position
    ``kv_len - q_len + i`` and, under ``causal``, sees keys ``0..kv_len - q_len + i``; a row that
    sees no key is zero.
    """
    total_q, h_q, d = q.shape
    h_kv = k_cache.shape[2]
    g = h_q // h_kv
    kf = np.asarray(k_cache, dtype=np.float64).reshape(-1, h_kv, d)
    vf = np.asarray(v_cache, dtype=np.float64).reshape(-1, h_kv, d)
    qf = np.asarray(q, dtype=np.float64)
    out = np.zeros((total_q, h_q, d), dtype=np.float64)
    for b in range(len(seqlen_k)):
        q0, q1 = int(cu_seqlens_q[b]), int(cu_seqlens_q[b + 1])
        kv_len = int(seqlen_k[b])
        k = gather_context(kf, block_table[b], kv_len, page_size)
        v = gather_context(vf, block_table[b], kv_len, page_size)
        for i in range(q1 - q0):
            visible = min(kv_len, kv_len - (q1 - q0) + i + 1) if causal else kv_len
            if visible <= 0:
                continue
            for h in range(h_q):
                s = k[:visible, h // g, :] @ qf[q0 + i, h] / math.sqrt(d)
                w = np.exp(s - s.max())
                out[q0 + i, h] = (w / w.sum()) @ v[:visible, h // g, :]
    return out
