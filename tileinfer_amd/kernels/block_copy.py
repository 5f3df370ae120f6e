"""Whole-block copies between paged KV caches: swap to/from pinned host memory, and device copies.

tileInfer advertises SWAP preemption but never moves KV blocks (engine/config.py:22,
engine/block_manager.py:29, engine/scheduler.py:28-31). ``swap_blocks`` / ``copy_blocks`` are the
data path such a policy needs: for every ``(src_block, dst_block)`` row of ``block_mapping`` the
block's K and V rows of every layer move from ``src`` to ``dst``. Either cache may live on the GPU
or in pinned host memory (``pin_memory=True``); the GPU kernel ``ti_copy_blocks`` accesses pinned
memory directly, so one call is one launch on the current stream.
"""
from __future__ import annotations

import torch

from .. import _lib

__all__ = ["copy_blocks", "swap_blocks"]


def _geometry(t: torch.Tensor, name: str):
    """(n_chunks, num_blocks, chunk_bytes, chunk_stride_bytes) of a cache [..., nb, bs, H, D]."""
    if t.dim() < 4:
        raise ValueError(f"{name} must be [..., num_blocks, block_size, H_kv, D], got {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    nb = t.shape[-4]
    chunk_bytes = t.shape[-3] * t.shape[-2] * t.shape[-1] * t.element_size()
    n_chunks = 1
    for s in t.shape[:-4]:
        n_chunks *= s
    return n_chunks, nb, chunk_bytes, nb * chunk_bytes


def copy_blocks(src: torch.Tensor, dst: torch.Tensor, block_mapping: torch.Tensor) -> None:
    """Copy block ``block_mapping[i, 0]`` of ``src`` to block ``block_mapping[i, 1]`` of ``dst``.

    Args:
        src, dst: caches with the same per-block shape and dtype, e.g. the slab
            ``[2, layers, num_blocks, block_size, H_kv, D]`` (K/V and layers are copied together)
            or one layer's ``[num_blocks, block_size, H_kv, D]``; the block counts may differ.
            Each is a GPU tensor or pinned host memory; at least one is on the GPU.
        block_mapping: ``[n, 2]`` int64 (source id, destination id); destination ids distinct.
            Ids outside a cache are skipped.
    """
    if src.dtype != dst.dtype or src.shape[-3:] != dst.shape[-3:] or src.shape[:-4] != dst.shape[:-4]:
        raise ValueError(f"caches differ: src {tuple(src.shape)} {src.dtype}, "
                         f"dst {tuple(dst.shape)} {dst.dtype}")
    gpu = src.device if src.device.type == "cuda" else dst.device
    if gpu.type != "cuda":
        raise ValueError("copy_blocks needs at least one GPU cache")
    for name, t in (("src", src), ("dst", dst)):
        if t.device.type == "cuda":
            if t.device != gpu:
                raise ValueError("src and dst are on different GPUs")
        elif not t.is_pinned():
            raise ValueError(f"{name} is host memory that is not pinned (use pin_memory=True)")
    if block_mapping.dim() != 2 or block_mapping.shape[1] != 2:
        raise ValueError(f"block_mapping must be [n, 2], got {tuple(block_mapping.shape)}")
    if block_mapping.dtype != torch.int64:
        block_mapping = block_mapping.to(torch.int64)
    n = block_mapping.shape[0]
    if n == 0:
        return
    if block_mapping.device != gpu:
        block_mapping = block_mapping.to(gpu)
    block_mapping = block_mapping.contiguous()
    sc, snb, cbytes, sstride = _geometry(src, "src")
    _, dnb, _, dstride = _geometry(dst, "dst")
    lib = _lib.load()
    with torch.cuda.device(gpu):
        _lib.check(lib.ti_copy_blocks(src.data_ptr(), dst.data_ptr(), block_mapping.data_ptr(), n,
                                      sc, cbytes, sstride, dstride, snb, dnb,
                                      _lib.stream_handle(gpu)))


# vLLM-style name for the host<->device direction; the operation is the same.
swap_blocks = copy_blocks
