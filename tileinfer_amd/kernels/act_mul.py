"""The attention output gate — drop-in for ``fused_sigmoid_mul`` of tileInfer's ``kernels/act_mul.py``.

``fused_sigmoid_mul(a, b)`` returns ``a * sigmoid(b)`` in a's shape and dtype
(kernels/act_mul.py:62-79; applied to the attention output at model/qwen_36.py:1083), computed in
fp32 and rounded once, by ``ti_sigmoid_mul``. For decode the same gate can run inside the attention
kernel's output epilogue instead: ``gqa_decode_paged_fn(..., gate=q_gate)``.
"""
from __future__ import annotations

import torch

from .. import _lib

__all__ = ["fused_sigmoid_mul"]


def fused_sigmoid_mul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``a * sigmoid(b)`` (same number of elements; bf16 or fp16)."""
    if a.numel() != b.numel():
        raise ValueError(f"a has {a.numel()} elements, b {b.numel()}")
    if a.dtype != b.dtype:
        raise TypeError(f"dtype mismatch: {a.dtype} vs {b.dtype}")
    code = _lib.dtype_code(a.dtype)
    if a.device.type != "cuda" or b.device != a.device:
        raise ValueError("fused_sigmoid_mul runs on the GPU with a and b on the same device")
    af = a.contiguous().view(-1)
    bf = b.contiguous().view(-1)
    if af.data_ptr() % 4:
        af = af.clone()
    if bf.data_ptr() % 4:
        bf = bf.clone()
    out = torch.empty_like(af)
    n = af.numel()
    if n % 2:
        # The kernel works on pairs; an odd tail element goes through a padded copy.
        af = torch.cat([af, af.new_zeros(1)])
        bf = torch.cat([bf, bf.new_zeros(1)])
        padded = torch.empty_like(af)
        _lib.check(_lib.load().ti_sigmoid_mul(af.data_ptr(), bf.data_ptr(), padded.data_ptr(),
                                              n + 1, code, _lib.stream_handle(a.device)))
        out.copy_(padded[:n])
    elif n:
        _lib.check(_lib.load().ti_sigmoid_mul(af.data_ptr(), bf.data_ptr(), out.data_ptr(), n,
                                              code, _lib.stream_handle(a.device)))
    return out.view(a.shape)
