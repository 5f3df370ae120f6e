"""Paged KV-cache layout and the per-step metadata builders.

Restates the parts of tileInfer's ``engine/model_runner.py`` that define where every token's K/V
lives and what the two kernels are handed:

* the cache slab ``[2, num_attn_layers, num_blocks, block_size, H_kv, D]`` (K = index 0, V = 1) and
  its block count from a memory budget (engine/model_runner.py:216-263);
* the per-layer views the attention call sites pass to the kernels (model/qwen_36.py:1016-1017,
  1071-1072);
* ``slot = block_table[pos // bs] * bs + pos % bs`` for decode (the newest token, at
  ``num_tokens - 1``, engine/model_runner.py:628-637) and for a prefill chunk
  (``[num_cached_tokens, num_cached_tokens + num_scheduled_tokens)``, 595-626);
* ``-1``-padded block tables (586-593), ``context_lens = num_tokens`` (699), and the padding rows of
  a captured decode batch: slot -1, context length 1, block -1 (524-527, 580-584).

Builders work on host numpy arrays and return int32 tensors on the requested device (one copy
each). Unlike the reference, a prefill position without a block raises instead of emitting -1.
"""
from __future__ import annotations

from typing import Iterable

import numpy as np
import torch

from .sequence import Sequence

KV_DTYPE_BYTES = {torch.bfloat16: 2, torch.float16: 2}


def kv_cache_shape(num_layers: int, num_blocks: int, block_size: int, num_kv_heads: int,
                   head_dim: int) -> tuple[int, ...]:
    return (2, num_layers, num_blocks, block_size, num_kv_heads, head_dim)


def block_bytes(block_size: int, num_kv_heads: int, head_dim: int, num_layers: int,
                dtype: torch.dtype = torch.bfloat16) -> int:
    """Bytes one block id costs across K, V and every attention layer."""
    return 2 * block_size * num_kv_heads * head_dim * KV_DTYPE_BYTES[dtype] * num_layers


def num_blocks_for_budget(budget_bytes: int, block_size: int, num_kv_heads: int, head_dim: int,
                          num_layers: int, dtype: torch.dtype = torch.bfloat16) -> int:
    """Blocks that fit ``budget_bytes`` (at least 1), as engine/model_runner.py:232-256 sizes it."""
    return max(1, int(budget_bytes) // block_bytes(block_size, num_kv_heads, head_dim,
                                                    num_layers, dtype))


def kv_budget(total_bytes: int, free_bytes: int, gpu_memory_utilization: float,
              reserved_bytes: int = 0) -> int:
    """Bytes the cache slab may take: ``total · utilization − used − reserved``, with
    ``used = total − free`` measured before the slab exists and ``reserved`` the other pools the
    runner sizes from the same budget (its recurrent-state pools; engine/model_runner.py:218-221,
    249-250). May be negative when memory is already over the utilisation target."""
    used = int(total_bytes) - int(free_bytes)
    return int(int(total_bytes) * gpu_memory_utilization) - used - int(reserved_bytes)


def kv_budget_from_device(gpu_memory_utilization: float, reserved_bytes: int = 0,
                          device: torch.device | str | None = None) -> int:
    """``kv_budget`` with the device's current free and total memory (``torch.cuda.mem_get_info``)."""
    free, total = torch.cuda.mem_get_info(device)
    return kv_budget(total, free, gpu_memory_utilization, reserved_bytes)


def max_blocks_per_seq(max_model_len: int, block_size: int, num_blocks: int) -> int:
    """Width of the runner's static block tables: ``max_model_len // block_size + 2``, clamped to
    the blocks the pool has (engine/model_runner.py:117, 284-288)."""
    return min(int(max_model_len) // int(block_size) + 2, int(num_blocks))


def allocate_kv_cache(num_layers: int, num_blocks: int, block_size: int, num_kv_heads: int,
                      head_dim: int, device: torch.device | str = "cuda",
                      dtype: torch.dtype = torch.bfloat16, zero: bool = True) -> torch.Tensor:
    """The single cache slab; zero-filled like the reference (engine/model_runner.py:259-263)."""
    shape = kv_cache_shape(num_layers, num_blocks, block_size, num_kv_heads, head_dim)
    alloc = torch.zeros if zero else torch.empty
    return alloc(shape, dtype=dtype, device=device)


def layer_views(kv_cache: torch.Tensor, layer: int):
    """(k_rows, v_rows, k_paged, v_paged) of one attention layer.

    ``*_rows`` are ``[num_blocks * block_size, H_kv * D]`` for ``store_kvcache``;
    ``*_paged`` are ``[num_blocks, block_size, H_kv, D]`` for ``gqa_decode_paged_fn``.
    """
    _, _, nb, bs, h, d = kv_cache.shape
    k_paged = kv_cache[0, layer]
    v_paged = kv_cache[1, layer]
    return k_paged.reshape(nb * bs, h * d), v_paged.reshape(nb * bs, h * d), k_paged, v_paged


def _slot(table: list[int], pos: int, bs: int) -> int:
    return table[pos // bs] * bs + pos % bs


def slot_mapping_decode(seqs: Iterable[Sequence], block_size: int) -> np.ndarray:
    """One slot per sequence: the cache row of its newest token."""
    return np.array([_slot(s.block_table, s.num_tokens - 1, block_size) for s in seqs],
                    dtype=np.int32)


def slot_mapping_prefill(seqs: Iterable[Sequence], block_size: int) -> np.ndarray:
    """Slots of every scheduled prefill token, sequences concatenated in order."""
    parts = []
    for s in seqs:
        start = s.num_cached_tokens
        pos = np.arange(start, start + s.num_scheduled_tokens, dtype=np.int64)
        if pos.size and (pos[-1] // block_size) >= len(s.block_table):
            raise IndexError(f"sequence {s.seq_id}: position {int(pos[-1])} has no block")
        table = np.asarray(s.block_table, dtype=np.int64)
        parts.append(table[pos // block_size] * block_size + pos % block_size)
    if not parts:
        return np.zeros(0, dtype=np.int32)
    return np.concatenate(parts).astype(np.int32)


def block_tables(seqs: list[Sequence], width: int | None = None) -> np.ndarray:
    """``[len(seqs), width]`` int32 tables, -1 padded (width defaults to the longest table)."""
    longest = max((len(s.block_table) for s in seqs), default=0)
    w = longest if width is None else width
    if w < longest:
        raise ValueError(f"width {w} < longest block table {longest}")
    out = np.full((len(seqs), w), -1, dtype=np.int32)
    for i, s in enumerate(seqs):
        out[i, :len(s.block_table)] = s.block_table
    return out


def context_lens(seqs: Iterable[Sequence]) -> np.ndarray:
    return np.array([s.num_tokens for s in seqs], dtype=np.int32)


def decode_metadata(seqs: list[Sequence], block_size: int, device: torch.device | str = "cuda",
                    pad_to: int | None = None, width: int | None = None):
    """(slot_mapping [n], block_tables [n, W], context_lens [n]) int32 tensors for a decode step.

    With ``pad_to`` the batch is padded the way a captured decode graph's static buffers are:
    extra rows get slot -1, context length 1 and an all -1 block table.
    """
    n = len(seqs)
    rows = n if pad_to is None else pad_to
    if rows < n:
        raise ValueError(f"pad_to {pad_to} < batch {n}")
    slots = np.full(rows, -1, dtype=np.int32)
    ctx = np.ones(rows, dtype=np.int32)
    tables = np.full((rows, 0), -1, dtype=np.int32)
    if n:
        slots[:n] = slot_mapping_decode(seqs, block_size)
        ctx[:n] = context_lens(seqs)
        t = block_tables(seqs, width)
        tables = np.full((rows, t.shape[1]), -1, dtype=np.int32)
        tables[:n] = t
    elif width:
        tables = np.full((rows, width), -1, dtype=np.int32)
    to = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    return to(slots), to(tables), to(ctx)
