"""Paged GQA decode attention — drop-in for tileInfer's ``kernels/gqa_decode_paged.py``.

``gqa_decode_paged_fn(q, k_cache, v_cache, block_table, seqlen_kv, page_size=16)`` keeps the
reference's positional signature, defaults and result (kernels/gqa_decode_paged.py:392-437): one
query token per sequence attends over ``seqlen_kv[b]`` cached tokens gathered through
``block_table[b]``, with query head ``h`` reading KV head ``h // (H_q // H_kv)``; the return value
is a new ``[B, H_q, D]`` tensor in ``q``'s dtype.

The work runs in libtileinfer_amd.so (``ti_gqa_decode_paged``): a split-K partial kernel on the
gfx950 matrix cores plus a fixed-order merge, enqueued on the current stream. The plan follows from
the table's width: balanced runs over the batch's tiles by default, fixed 32-token partitions for
context bounds up to 1,024 tokens, and one workgroup per (KV head, sequence) whose waves combine
their parts without a merge launch up to 128 tokens (up to 512 when those pairs fill three quarters
to all of one round of workgroups). The output and the split-K workspace come from torch's caching
allocator, so the call is graph-capture safe. Unlike the reference wrapper it never pads the block
table (kernels/gqa_decode_paged.py:421-430): any table width works, entries at or beyond
``ceil(seqlen/page_size)`` are never read, and block ids outside the cache at positions
``< seqlen`` are treated as absent instead of being read.

As in the reference, the caches are treated as flat ``[num_rows, H_kv, D]`` token rows grouped in
pages of ``page_size`` rows (kernels/gqa_decode_paged.py:403-406), so ``page_size`` need not equal
``k_cache.shape[1]`` as long as it tiles the rows; this build takes pages of 1, 2, 4, 8 or a
multiple of 16 tokens.
"""
from __future__ import annotations

import ctypes
import functools

import torch

from .. import _lib

__all__ = ["gqa_decode_paged_fn", "gqa_decode_paged_noalloc", "decode_plan"]

_VARIANTS = {"auto": _lib.TI_DECODE_AUTO, "mfma": _lib.TI_DECODE_MFMA,
             "scalar": _lib.TI_DECODE_SCALAR}


@functools.lru_cache(maxsize=256)
def decode_plan(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int, page_size: int,
                max_blocks_per_seq: int, split_tokens: int | None = None) -> tuple[int, int, int]:
    """(split_tokens, max_splits, workspace_bytes) the library uses for these host-known bounds."""
    lib = _lib.load()
    s, m, w = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
    _lib.check(lib.ti_gqa_decode_plan(batch, num_q_heads, num_kv_heads, head_dim, page_size,
                                      max_blocks_per_seq, int(split_tokens or 0),
                                      ctypes.byref(s), ctypes.byref(m), ctypes.byref(w)))
    return s.value, m.value, w.value


# Where attending a shared prefix once (prefill pass over the prefix, suffix decode, merge) beats
# the plain decode reading the prefix pages per sequence (cache-keeping policy: they hit in
# L2/MALL): the pass has a fixed cost of ~30-50 us, so it needs enough sequences and prefix.
_PREFIX_MIN_BATCH, _PREFIX_MIN_TOKENS = 4, 131072


@functools.lru_cache(maxsize=256)
def _prefix_splits(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                   prefix_tokens: int) -> int:
    """Key ranges the shared-prefix pass is cut into (host-known sizes only)."""
    return int(_lib.load().ti_gqa_prefill_key_splits(batch, num_q_heads, num_kv_heads, head_dim,
                                                     prefix_tokens))


def _append_rows(append, b: int, h_kv: int, d: int, dt, dev):
    """The append= operands checked as store_kvcache checks them: key/value as [B, H_kv * D] rows
    (16-byte aligned, unit element stride; copied only if they are not) and slot_mapping as a
    contiguous [B] int32 tensor."""
    if not isinstance(append, (tuple, list)) or len(append) != 3:
        raise ValueError("append must be (key, value, slot_mapping)")
    key, value, slots = append
    row = h_kv * d
    for name, t in (("key", key), ("value", value)):
        if not isinstance(t, torch.Tensor) or t.numel() != b * row or t.shape[0] != b:
            raise ValueError(f"append {name} must hold [{b}, {h_kv}, {d}] values")
        if t.dtype != dt or t.device != dev:
            raise ValueError(f"append {name} must be {dt} on {dev}")
    if (not isinstance(slots, torch.Tensor) or slots.dtype != torch.int32 or slots.dim() != 1
            or slots.shape[0] != b or slots.device != dev):
        raise ValueError(f"append slot_mapping must be [{b}] int32 on {dev}")
    flat = []
    for t in (key, value):
        f = t.reshape(b, row)
        if f.stride(1) != 1 or f.stride(0) % 8 or f.data_ptr() % 16:
            f = f.contiguous()
        flat.append(f)
    return flat[0], flat[1], slots.contiguous()


_STATIC_I32: dict = {}


def _static_i32(values: tuple, dev: torch.device) -> torch.Tensor:
    """A small int32 device tensor kept for reuse (made once per values/device, so that a call
    captured in a graph does not create or upload it). Entries are never evicted: a captured
    graph holds their addresses, and there is one per (batch size, prefix length) in use."""
    key = (values, str(dev))
    t = _STATIC_I32.get(key)
    if t is None:
        t = _STATIC_I32[key] = torch.tensor(values, dtype=torch.int32, device=dev)
    return t


def _policy_flag(kv_reuse: bool | None) -> int:
    """Variant flag of the K/V cache policy: none (chosen on the device) for None."""
    if kv_reuse is None:
        return 0
    return _lib.TI_DECODE_REUSE_KV if kv_reuse else _lib.TI_DECODE_STREAM_KV


def _aligned_rows(t: torch.Tensor) -> bool:
    return (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
            and all(s % 8 == 0 for s in t.stride()[:-1]))


def _checked(q, k_cache, v_cache, block_table, seqlen_kv, page_size, variant):
    """Validate a decode call's arguments; returns the (possibly made contiguous) q, table and
    lengths with the sizes the library needs."""
    if q.dim() != 3:
        raise ValueError(f"q must be [B, H_q, D], got {tuple(q.shape)}")
    b, h_q, d = q.shape
    if k_cache.dim() != 4:
        raise ValueError(f"k_cache must be [num_blocks, block_size, H_kv, D], got {tuple(k_cache.shape)}")
    if v_cache.shape != k_cache.shape:
        raise ValueError(f"v_cache shape {tuple(v_cache.shape)} != k_cache {tuple(k_cache.shape)}")
    nb, bs, h_kv, d2 = k_cache.shape
    if d2 != d:
        raise ValueError(f"head_dim mismatch: q {d}, cache {d2}")
    if h_kv <= 0 or h_q % h_kv != 0:
        raise ValueError(f"H_q={h_q} is not a multiple of H_kv={h_kv}")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache and v_cache must be contiguous (a copy of the cache is never made)")
    dt = q.dtype
    if not (k_cache.dtype == v_cache.dtype == dt):
        raise TypeError(f"dtype mismatch: q {dt}, k_cache {k_cache.dtype}, v_cache {v_cache.dtype}")
    code = _lib.dtype_code(dt)
    if block_table.dtype != torch.int32 or seqlen_kv.dtype != torch.int32:
        raise TypeError(f"block_table/seqlen_kv must be int32, got {block_table.dtype}/{seqlen_kv.dtype}")
    if block_table.dim() != 2 or block_table.shape[0] != b:
        raise ValueError(f"block_table must be [{b}, W], got {tuple(block_table.shape)}")
    if seqlen_kv.dim() != 1 or seqlen_kv.shape[0] != b:
        raise ValueError(f"seqlen_kv must be [{b}], got {tuple(seqlen_kv.shape)}")
    page_size = int(page_size)
    rows = nb * bs
    if page_size <= 0 or rows % page_size != 0:
        raise ValueError(f"page_size {page_size} does not tile the cache's {rows} rows")
    if variant not in _VARIANTS:
        raise ValueError(f"variant must be one of {sorted(_VARIANTS)}, got {variant!r}")
    dev = q.device
    if dev.type != "cuda":
        raise ValueError("gqa_decode_paged_fn runs on the GPU; q is on " + str(dev))
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache), ("block_table", block_table),
                    ("seqlen_kv", seqlen_kv)):
        if t.device != dev:
            raise ValueError(f"{name} is on {t.device}, q on {dev}")
    if block_table.stride(-1) != 1:
        block_table = block_table.contiguous()
    if not seqlen_kv.is_contiguous():
        seqlen_kv = seqlen_kv.contiguous()
    if not _aligned_rows(q):
        q = q.contiguous()
    return q, block_table, seqlen_kv, (b, h_q, d, h_kv, rows, page_size, dt, code, dev)


def gqa_decode_paged_fn(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    seqlen_kv: torch.Tensor,
    page_size: int = 16,
    *,
    out: torch.Tensor | None = None,
    split_tokens: int | None = None,
    variant: str = "auto",
    kv_reuse: bool | None = None,
    gate: torch.Tensor | None = None,
    shared_prefix_tokens: int = 0,
    prefix_pass: str = "auto",
    append: tuple | None = None,
) -> torch.Tensor:
    """Single-query paged GQA attention.

    Args (kernels/gqa_decode_paged.py:392-399, shapes at model/qwen_36.py:1071-1079):
        q: [B, H_q, D]
        k_cache, v_cache: [num_blocks, block_size, H_kv, D], contiguous
        block_table: [B, W] int32 physical page ids (-1 padding allowed past each sequence)
        seqlen_kv: [B] int32 context lengths (including the token appended this step)
        page_size: tokens per page of the flattened cache
        out: keyword-only preallocated [B, H_q, D] output (contiguous, q's dtype)
        split_tokens: keyword-only split-K partition length (None: the library's choice)
        variant: keyword-only "auto" | "mfma" | "scalar" kernel choice
        kv_reuse: keyword-only cache policy of the K/V loads. None (the default): chosen per
            sequence on the device -- a sequence whose first block another sequence of the batch
            also starts with (prefix caching shares block chains from the table's first column)
            keeps the default policy, so the shared pages hit in L2/MALL for the other readers;
            every other sequence streams its pages once (``nt``), which is faster when nothing is
            shared (batches above 2,048 sequences stream). True forces the default policy, False
            forces streaming. The scalar variant streams unless True. Results are bitwise
            identical under every policy.
        gate: keyword-only; the attention output gate (model/qwen_36.py:1083), any tensor of
            B * H_q * D values laid out [B, H_q, D] (``q_gate`` [B, 1, H_q * D] as the model has
            it): the output is ``decode * sigmoid(gate)``, applied in the kernel's epilogue —
            bitwise ``fused_sigmoid_mul(gqa_decode_paged_fn(...), gate)``.
        shared_prefix_tokens: keyword-only P (a multiple of page_size, at most every seqlen_kv):
            the caller's statement that the first P tokens of every sequence hold the same K/V
            (prefix caching: shared blocks, or private copies of equal values). The prefix is then
            attended once for the whole batch — all B x H_q queries against sequence 0's first P
            tokens through the MFMA prefill kernel, unnormalised — and the decode kernel covers
            tokens [P, seqlen) of each sequence and merges the two parts. Within the decode
            tolerance of the plain call; bitwise the same for shared and private prefix pages.
            MFMA variant only.
        prefix_pass: keyword-only, with ``shared_prefix_tokens``: "auto" attends the prefix once
            only where that is faster than the plain decode, i.e. for at least 4 sequences and
            B x P >= 131,072 prefix tokens (measured against the plain call with the
            cache-keeping policy: the prefix pass wins from 16 sequences at an 8k prefix, from 32
            at 2k and from 4 at 32k); below that the call is the plain decode, bitwise. "always"
            takes the prefix pass for any batch.
        append: keyword-only ``(key, value, slot_mapping)``, the decode step's new token per
            sequence (key/value [B, H_kv, D] in q's dtype, slot_mapping [B] int32 with
            slot_mapping[b] the slot of position seqlen_kv[b] - 1, or -1 to skip): written into
            the cache inside this call, bitwise what ``store_kvcache(key, value, k_cache rows,
            v_cache rows, slot_mapping)`` before the decode gives (model/qwen_36.py:1018, 1074),
            without the append's launch. Not combined with ``gate``, ``shared_prefix_tokens`` or
            the scalar variant.
    Returns:
        [B, H_q, D] tensor in q's dtype.
    """
    q, block_table, seqlen_kv, (b, h_q, d, h_kv, rows, page_size, dt, code, dev) = _checked(
        q, k_cache, v_cache, block_table, seqlen_kv, page_size, variant)
    if append is not None and (gate is not None or shared_prefix_tokens or variant == "scalar"):
        raise ValueError("append= combines with neither gate=, shared_prefix_tokens= nor the "
                         "scalar variant")
    if out is None:
        out = torch.empty((b, h_q, d), dtype=dt, device=dev)
    elif (out.shape != (b, h_q, d) or out.dtype != dt or out.device != dev
          or not out.is_contiguous()):
        raise ValueError("out must be a contiguous [B, H_q, D] tensor of q's dtype and device")
    if b == 0:
        return out
    width = block_table.shape[1]
    lib = _lib.load()
    prefix = int(shared_prefix_tokens or 0)
    if prefix:
        if prefix < 0 or prefix % page_size or prefix // page_size > width:
            raise ValueError(f"shared_prefix_tokens {prefix} must be a multiple of page_size "
                             f"{page_size} within the block table's {width} pages")
        if variant == "scalar":
            raise ValueError("shared_prefix_tokens needs the MFMA variant")
        if prefix_pass not in ("auto", "always"):
            raise ValueError(f"prefix_pass must be 'auto' or 'always', got {prefix_pass!r}")
        if prefix_pass == "auto" and (b < _PREFIX_MIN_BATCH or b * prefix < _PREFIX_MIN_TOKENS):
            prefix = 0  # the plain decode is the faster one here
    if prefix:
        # The batch's queries as the B "tokens" of one non-causal chunk over sequence 0's prefix,
        # its keys cut into `splits` ranges, each range's unnormalised part merged by the decode.
        splits = _prefix_splits(b, h_q, h_kv, d, prefix)
        pre_o = torch.empty((splits, b, h_q, d), dtype=torch.float32, device=dev)
        pre_ml = torch.empty((splits, b, h_q, 2), dtype=torch.float32, device=dev)
        _lib.check(lib.ti_gqa_prefill_paged_partial(
            q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(),
            block_table.data_ptr(), block_table.stride(0), _static_i32((0, b), dev).data_ptr(),
            _static_i32((prefix,), dev).data_ptr(), pre_o.data_ptr(), pre_ml.data_ptr(),
            None, 0, 1, b, b, h_q, h_kv, d, page_size, rows // page_size, prefix // page_size, 0,
            code, splits, _lib.stream_handle(dev)))
        width -= prefix // page_size
    _, _, ws_bytes = decode_plan(b, h_q, h_kv, d, page_size, width, split_tokens)
    if prefix:
        ws_bytes += b * h_q * (d + 2) * 4  # whole sequences' rows, folded with the prefix parts
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes > 0 else None
    table_width = block_table.shape[1]
    args = (q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(),
            block_table.data_ptr(), block_table.stride(0) if table_width > 0 else 0,
            seqlen_kv.data_ptr(), out.data_ptr(), ws.data_ptr() if ws is not None else None,
            ws_bytes, b, h_q, h_kv, d, page_size, rows // page_size,
            table_width if prefix else width, int(split_tokens or 0),
            _VARIANTS[variant] | _policy_flag(kv_reuse), code)
    g3 = None
    if gate is not None:
        if gate.numel() != b * h_q * d or gate.dtype != dt or gate.device != dev:
            raise ValueError(f"gate must hold {b}x{h_q}x{d} values of q's dtype on q's device")
        g3 = gate.reshape(b, h_q, d)
        if not _aligned_rows(g3):
            g3 = g3.contiguous()
    if prefix:
        _lib.check(lib.ti_gqa_decode_paged_prefixed(
            *args, g3.data_ptr() if g3 is not None else None, g3.stride(0) if g3 is not None else 0,
            g3.stride(1) if g3 is not None else 0, pre_o.data_ptr(), pre_ml.data_ptr(), splits,
            prefix, _lib.stream_handle(dev)))
        return out
    if append is not None:
        kf, vf, slots = _append_rows(append, b, h_kv, d, dt, dev)
        _lib.check(lib.ti_gqa_decode_paged_append(
            *args, kf.data_ptr(), vf.data_ptr(), kf.stride(0), vf.stride(0), slots.data_ptr(),
            rows, _lib.stream_handle(dev)))
        return out
    if gate is None:
        _lib.check(lib.ti_gqa_decode_paged(*args, _lib.stream_handle(dev)))
        return out
    _lib.check(lib.ti_gqa_decode_paged_gated(*args, g3.data_ptr(), g3.stride(0), g3.stride(1),
                                             _lib.stream_handle(dev)))
    return out


def gqa_decode_paged_noalloc(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    seqlen_kv: torch.Tensor,
    page_size: int = 16,
    *,
    out: torch.Tensor,
    split_tokens: int | None = None,
    variant: str = "auto",
    kv_reuse: bool | None = None,
) -> torch.Tensor:
    """``gqa_decode_paged_fn`` for callers that cannot allocate: no output, workspace or copy is
    made (``ti_gqa_decode_paged_noalloc``; the split-K partials live in the library's per-GPU
    static scratch). ``out`` is required; ``q`` must have 16-byte aligned rows and the table and
    lengths unit stride (they are refused rather than copied). Calls that overlap on one GPU share
    that scratch and must not run concurrently. Results are bitwise those of
    ``gqa_decode_paged_fn`` with the same plan."""
    if not _aligned_rows(q) or block_table.stride(-1) != 1 or not seqlen_kv.is_contiguous():
        raise ValueError("gqa_decode_paged_noalloc: q rows must be 16-byte aligned and the table "
                         "and lengths unit-stride (no copies are made)")
    _, _, _, (b, h_q, d, h_kv, rows, page_size, dt, code, dev) = _checked(
        q, k_cache, v_cache, block_table, seqlen_kv, page_size, variant)
    if (out.shape != (b, h_q, d) or out.dtype != dt or out.device != dev
            or not out.is_contiguous()):
        raise ValueError("out must be a contiguous [B, H_q, D] tensor of q's dtype and device")
    width = block_table.shape[1]
    lib = _lib.load()
    _lib.check(lib.ti_gqa_decode_paged_noalloc(
        q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(),
        block_table.data_ptr(), block_table.stride(0) if width > 0 else 0, seqlen_kv.data_ptr(),
        out.data_ptr(), b, h_q, h_kv, d, page_size, rows // page_size, width,
        int(split_tokens or 0), _VARIANTS[variant] | _policy_flag(kv_reuse),
        code, _lib.stream_handle(dev)))
    return out
