"""Slot-mapped K/V append into the paged cache — drop-in for tileInfer's ``kernels/kvcache_store.py``.

``store_kvcache`` keeps the reference's positional signature and semantics
(kernels/kvcache_store.py:43-71): for every token ``i`` whose ``slot_mapping[i] >= 0`` the rows
``k_cache[slot]`` / ``v_cache[slot]`` become ``key[i]`` / ``value[i]`` flattened over heads; ``-1``
slots are skipped. The copy runs in the gfx950 kernel ``ti_kv_append`` of libtileinfer_amd.so
(one 16-byte vector per lane, no staging), enqueued on the current stream; it allocates nothing, so
it is safe under graph capture.

Differences from the reference, all on inputs the reference never produces:
  * a slot ``>= num_slots`` is skipped instead of written out of bounds;
  * duplicate non-negative slots are unsupported (the reference's torch loop is last-write-wins,
    its TileLang kernel is unordered, kernels/kvcache_store.py:98);
  * wrong dtypes/devices/shapes raise ``ValueError``/``TypeError`` instead of failing inside JIT.
"""
from __future__ import annotations

import torch

from .. import _lib

__all__ = ["store_kvcache"]


def _rows(t: torch.Tensor, n: int, d: int) -> torch.Tensor:
    """``t`` viewed as [n, d] rows with unit element stride (copied only if it must be)."""
    flat = t.reshape(n, d)
    if d > 0 and flat.stride(1) != 1:
        flat = flat.contiguous()
    return flat


def store_kvcache(
    key: torch.Tensor,
    value: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    *,
    validate: bool = False,
) -> None:
    """Store K/V into the paged KV cache (in-place scatter write).

    Args (kernels/kvcache_store.py:52-57):
        key: [N, num_heads, head_dim]
        value: [N, num_heads, head_dim]
        k_cache: [num_slots, num_heads * head_dim], rows contiguous (updated in place)
        v_cache: [num_slots, num_heads * head_dim], rows contiguous (updated in place)
        slot_mapping: [N] int32, -1 means skip
        validate: keyword-only; also check on the host (synchronising) that every slot is in
            ``[-1, num_slots)`` and that non-negative slots are unique.
    """
    if key.dim() != 3:
        raise ValueError(f"key must be [N, num_heads, head_dim], got {tuple(key.shape)}")
    n, num_heads, head_dim = key.shape
    d = num_heads * head_dim
    if value.shape != key.shape:
        raise ValueError(f"value shape {tuple(value.shape)} != key shape {tuple(key.shape)}")
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        if c.dim() != 2 or c.shape[1] != d:
            raise ValueError(f"{name} must be [num_slots, {d}], got {tuple(c.shape)}")
        if c.stride(1) != 1:
            raise ValueError(f"{name} rows must be contiguous (stride {c.stride()})")
    if v_cache.shape != k_cache.shape or v_cache.stride() != k_cache.stride():
        raise ValueError("k_cache and v_cache must have the same shape and strides")
    dt = key.dtype
    if not (value.dtype == k_cache.dtype == v_cache.dtype == dt):
        raise TypeError(f"dtype mismatch: key {dt}, value {value.dtype}, "
                        f"k_cache {k_cache.dtype}, v_cache {v_cache.dtype}")
    code = _lib.dtype_code(dt)
    if slot_mapping.dtype != torch.int32:
        raise TypeError(f"slot_mapping must be int32, got {slot_mapping.dtype}")
    if slot_mapping.dim() != 1 or slot_mapping.shape[0] != n:
        raise ValueError(f"slot_mapping must be [{n}], got {tuple(slot_mapping.shape)}")
    dev = key.device
    if dev.type != "cuda":
        raise ValueError("store_kvcache runs on the GPU; key is on " + str(dev))
    for name, t in (("value", value), ("k_cache", k_cache), ("v_cache", v_cache),
                    ("slot_mapping", slot_mapping)):
        if t.device != dev:
            raise ValueError(f"{name} is on {t.device}, key on {dev}")
    if n == 0:
        return
    if not slot_mapping.is_contiguous():
        slot_mapping = slot_mapping.contiguous()
    num_slots = k_cache.shape[0]
    if validate:
        s = slot_mapping.cpu()
        bad = (s < -1) | (s >= num_slots)
        if bool(bad.any()):
            raise ValueError(f"slot_mapping has entries outside [-1, {num_slots}): "
                             f"{s[bad][:8].tolist()}")
        live = s[s >= 0]
        if live.unique().numel() != live.numel():
            raise ValueError("slot_mapping has duplicate non-negative slots")
    kf = _rows(key, n, d)
    vf = _rows(value, n, d)
    lib = _lib.load()
    _lib.check(lib.ti_kv_append(
        kf.data_ptr(), vf.data_ptr(), kf.stride(0), vf.stride(0),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0),
        slot_mapping.data_ptr(), n, d, num_slots, code, _lib.stream_handle(dev)))
