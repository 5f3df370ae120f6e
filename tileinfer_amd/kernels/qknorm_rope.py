"""QK-norm + partial RoPE, and its fusion with the K/V append — the inputs side of the path.

``fused_qknorm_rope(x, weight, cos_flat, sin_flat, eps=1e-5)`` keeps the reference's signature
and result (kernels/qknorm_rope.py:52-56): ``x`` ``[B, H, 1, D]``, one cos/sin vector for every
row; per-head RMSNorm with ``(1 + weight)``, then rotate-half RoPE on the first
``rotary_dim = cos_flat.numel()`` dimensions using ``cos/sin[:rotary_dim // 2]``.

``qknorm_rope(x, weight, cos, sin, eps)`` is the same operation for any number of tokens
(``x`` ``[T, H, D]``) with per-token ``cos``/``sin`` ``[T, rotary_dim]`` (or one ``[rotary_dim]``
vector) — what the reference's batched-decode and prefill branches compute with separate torch ops
(model/qwen_36.py:985-1003).

``qknorm_rope_append(q, k, v, q_weight, k_weight, cos, sin, k_cache, v_cache, slot_mapping, eps)``
does the whole input side of a step in one launch: q normalised and rotated (returned), k
normalised and rotated and v as is, written into the cache rows at ``slot_mapping``
(model/qwen_36.py:977-1018) — bitwise what ``qknorm_rope`` on q and k followed by
``store_kvcache`` writes.

Numerics follow the reference's fused kernel (kernels/qknorm_rope.py:29-49): fp32 statistics,
normalised row rounded to the storage type, rotation in fp32, rounded once.
"""
from __future__ import annotations

import torch

from .. import _lib

__all__ = ["fused_qknorm_rope", "qknorm_rope", "qknorm_rope_append"]


def _rows_ok(t: torch.Tensor) -> bool:
    return t.stride(-1) == 1 and t.data_ptr() % 4 == 0 and all(s % 2 == 0 for s in t.stride()[:-1])


def _cos_sin(cos: torch.Tensor, sin: torch.Tensor, n_tokens: int, dtype, dev):
    if cos.shape != sin.shape:
        raise ValueError(f"cos {tuple(cos.shape)} and sin {tuple(sin.shape)} differ")
    if cos.dtype != dtype or sin.dtype != dtype:
        raise TypeError(f"cos/sin must be {dtype}")
    if cos.device != dev or sin.device != dev:
        raise ValueError("cos/sin must be on the same device as x")
    if cos.dim() == 1:
        rd, stride = cos.shape[0], 0
    elif cos.dim() == 2 and cos.shape[0] in (1, n_tokens):
        rd = cos.shape[1]
        stride = 0 if cos.shape[0] == 1 else cos.stride(0)
    else:
        raise ValueError(f"cos must be [rotary_dim] or [{n_tokens}, rotary_dim], got {tuple(cos.shape)}")
    if cos.stride(-1) != 1 or sin.stride(-1) != 1 or (cos.dim() == 2 and sin.stride(0) != cos.stride(0)):
        cos, sin = cos.contiguous(), sin.contiguous()
        stride = 0 if cos.dim() == 1 or cos.shape[0] == 1 else cos.stride(0)
    return cos, sin, rd, stride


def qknorm_rope(x: torch.Tensor, weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                eps: float = 1e-5, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """RMSNorm(1 + weight) then partial RoPE of ``x`` ``[T, H, D]``; returns ``[T, H, D]``."""
    if x.dim() != 3:
        raise ValueError(f"x must be [T, H, D], got {tuple(x.shape)}")
    t, h, d = x.shape
    dev, dt = x.device, x.dtype
    code = _lib.dtype_code(dt)
    if dev.type != "cuda":
        raise ValueError("qknorm_rope runs on the GPU; x is on " + str(dev))
    if weight.shape != (d,) or weight.dtype != dt or weight.device != dev:
        raise ValueError(f"weight must be [{d}] {dt} on {dev}")
    cos, sin, rd, cs_stride = _cos_sin(cos, sin, t, dt, dev)
    if rd > d or rd % 2:
        raise ValueError(f"rotary_dim {rd} must be even and <= head_dim {d}")
    if not _rows_ok(x):
        x = x.contiguous()
    weight = weight.contiguous()
    if out is None:
        out = torch.empty((t, h, d), dtype=dt, device=dev)
    elif out.shape != (t, h, d) or out.dtype != dt or out.device != dev or not _rows_ok(out):
        raise ValueError("out must be a [T, H, D] tensor of x's dtype and device")
    _lib.check(_lib.load().ti_qknorm_rope(
        x.data_ptr(), x.stride(0), x.stride(1), out.data_ptr(), out.stride(0), out.stride(1),
        weight.data_ptr(), cos.data_ptr(), sin.data_ptr(), cs_stride, t, h, d, rd, float(eps),
        code, _lib.stream_handle(dev)))
    return out


def fused_qknorm_rope(x: torch.Tensor, weight: torch.Tensor, cos_flat: torch.Tensor,
                      sin_flat: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """Drop-in for the reference's ``fused_qknorm_rope``: ``x`` ``[B, H, 1, D]``, one vector."""
    if x.dim() != 4 or x.shape[2] != 1:
        raise ValueError(f"x must be [B, H, 1, D], got {tuple(x.shape)}")
    b, h, _, d = x.shape
    y = qknorm_rope(x.reshape(b, h, d), weight, cos_flat.reshape(-1), sin_flat.reshape(-1), eps)
    return y.view(b, h, 1, d)


def qknorm_rope_append(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       q_weight: torch.Tensor, k_weight: torch.Tensor, cos: torch.Tensor,
                       sin: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                       slot_mapping: torch.Tensor, eps: float = 1e-5, *,
                       q_out: torch.Tensor | None = None) -> torch.Tensor:
    """Input side of one step in one launch; returns the normalised, rotated ``q``.

    q ``[T, H_q, D]``, k and v ``[T, H_kv, D]``; ``k_cache``/``v_cache`` are the layer's cache rows
    ``[num_slots, H_kv * D]`` (the views ``store_kvcache`` takes); ``slot_mapping`` ``[T]`` int32
    (slots < 0 are skipped). K is written normalised and rotated, V as is.
    """
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q, k, v must be [T, heads, D]")
    t, hq, d = q.shape
    if k.shape[0] != t or v.shape != k.shape or k.shape[2] != d:
        raise ValueError(f"k {tuple(k.shape)} / v {tuple(v.shape)} do not match q {tuple(q.shape)}")
    hkv = k.shape[1]
    dev, dt = q.device, q.dtype
    if q_out is not None and (q_out.shape != (t, hq, d) or q_out.dtype != dt
                              or q_out.device != dev or not _rows_ok(q_out)):
        raise ValueError("q_out must be a [T, H_q, D] tensor of q's dtype and device")
    code = _lib.dtype_code(dt)
    if dev.type != "cuda":
        raise ValueError("qknorm_rope_append runs on the GPU; q is on " + str(dev))
    for name, w in (("q_weight", q_weight), ("k_weight", k_weight)):
        if w.shape != (d,) or w.dtype != dt or w.device != dev:
            raise ValueError(f"{name} must be [{d}] {dt} on {dev}")
    for name, tns in (("k", k), ("v", v), ("k_cache", k_cache), ("v_cache", v_cache)):
        if tns.dtype != dt or tns.device != dev:
            raise ValueError(f"{name} must be {dt} on {dev}")
    if k_cache.dim() != 2 or v_cache.shape != k_cache.shape or k_cache.shape[1] != hkv * d:
        raise ValueError(f"caches must be [num_slots, {hkv * d}] rows")
    if k_cache.stride(1) != 1 or v_cache.stride() != k_cache.stride():
        raise ValueError("k_cache and v_cache must be row views with the same strides")
    if slot_mapping.dtype != torch.int32 or slot_mapping.shape != (t,) or slot_mapping.device != dev:
        raise ValueError(f"slot_mapping must be [{t}] int32 on {dev}")
    cos, sin, rd, cs_stride = _cos_sin(cos, sin, t, dt, dev)
    if rd > d or rd % 2:
        raise ValueError(f"rotary_dim {rd} must be even and <= head_dim {d}")
    q = q if _rows_ok(q) else q.contiguous()
    k = k if _rows_ok(k) else k.contiguous()
    v = v if _rows_ok(v) else v.contiguous()
    slot_mapping = slot_mapping.contiguous()
    if q_out is None:
        q_out = torch.empty((t, hq, d), dtype=dt, device=dev)
    _lib.check(_lib.load().ti_qknorm_rope_append(
        q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr(), v.stride(0), v.stride(1), q_weight.contiguous().data_ptr(),
        k_weight.contiguous().data_ptr(), cos.data_ptr(), sin.data_ptr(), cs_stride,
        q_out.data_ptr(), q_out.stride(0), q_out.stride(1), k_cache.data_ptr(),
        v_cache.data_ptr(), k_cache.stride(0), slot_mapping.data_ptr(), k_cache.shape[0], t, hq,
        hkv, d, rd, float(eps), code, _lib.stream_handle(dev)))
    return q_out
