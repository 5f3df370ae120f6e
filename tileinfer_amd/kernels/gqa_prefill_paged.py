"""Paged causal GQA prefill attention — replaces tileInfer's gather + varlen flash attention.

The reference's chunked prefill (model/qwen_36.py:1030-1065) gathers all ``full_kv_len`` cached
positions of the sequence through ``ctx.block_tables[0]`` into contiguous K/V copies and calls the
varlen flash-attention kernel (kernels/gqa_varlen.py:40-185, dispatch 369-389) with
``cu_seqlens_k = [0, full_kv_len]``. ``gqa_prefill_paged_fn`` computes the same thing straight from
the cache pages, for any number of sequences in one launch:

    out = gqa_prefill_paged_fn(q_unpad, k_cache, v_cache, block_tables, cu_seqlens_q, seqlen_k,
                               max_seqlen_q, page_size)

Semantics follow kernels/gqa_varlen.py:88-175: sequence ``b`` owns query rows
``[cu_seqlens_q[b], cu_seqlens_q[b+1])`` and sees its first ``seqlen_k[b]`` cached tokens (the
chunk's own K/V must already be appended, as store_kvcache does at model/qwen_36.py:1016-1018);
the causal mask is bottom-right aligned (query ``i`` sees keys ``j <= seqlen_k - q_len + i``);
query head ``h`` reads KV head ``h // (H_q // H_kv)``; softmax in base 2 with ``D^-1/2`` scale,
P rounded to the cache dtype before P·V, fp32 accumulation; a row with no visible key is zero.
The first chunk (no cached prefix) is the case ``seqlen_k == q_len``.

Scheduling. A unit is one KV head of one block of query tokens. ``schedule="per_unit"`` runs one
workgroup per unit (one launch, heaviest blocks first): each row's result is then bitwise
independent of the other sequences in the batch and of how the prompt was chunked
(``batch_invariant=True`` asks for exactly that). ``schedule="balanced"`` gives every CU the same
work (units may be cut between workgroups and merged in fp32 afterwards, in a fixed order; three
launches), which removes the partial last round of a continuation chunk and spreads a few long
units over the whole GPU. ``schedule="auto"`` (default) picks per call from host-known sizes: the
per-unit schedule when no sequence has cached context (``max_seqlen_k <= max_seqlen_q``: causal
first chunks pack well heaviest-first), a greedy estimate of both for a single sequence, the
balanced schedule otherwise (and whenever ``max_seqlen_k`` is not given).
"""
from __future__ import annotations

import ctypes
import functools
import heapq

import torch

from .. import _lib

__all__ = ["gqa_prefill_paged_fn"]


@functools.lru_cache(maxsize=256)
def _workspace_bytes(batch: int, total_q: int, h_q: int, h_kv: int, d: int, page_size: int,
                     width: int) -> int:
    """Bytes of the balanced schedule's workspace (0: the call runs one workgroup per unit)."""
    nbytes = ctypes.c_int64(0)
    _lib.check(_lib.load().ti_gqa_prefill_workspace_bytes(batch, total_q, h_q, h_kv, d, page_size,
                                                          width, ctypes.byref(nbytes)))
    return nbytes.value


# Schedule model (in 64-key tiles): a unit costs its key tiles plus _UNIT_COST (start-up and
# epilogue); the balanced schedule adds its plan and merge launches, ~_BALANCE_OVERHEAD tiles.
_KEY_TILE, _UNIT_COST, _BALANCE_OVERHEAD = 64, 2, 9


@functools.lru_cache(maxsize=1024)
def _per_unit_wins(q_len: int, kv_len: int, causal: bool, h_kv: int, group: int, rows: int,
                   wgs: int) -> bool:
    """One sequence: greedy (heaviest-first) makespan of one workgroup per unit (``rows``
    consecutive (token, query head) rows, row = token * group + head) against the balanced
    schedule's even share plus its overhead."""
    costs = []
    for r0 in range(0, q_len * group, rows):
        last = (r0 + min(rows, q_len * group - r0) - 1) // group  # the unit's last token
        k_end = min(kv_len, kv_len - q_len + last + 1) if causal else kv_len
        nt = -(-max(k_end, 0) // _KEY_TILE)
        if nt:
            costs.extend([nt + _UNIT_COST] * h_kv)
    if not costs:
        return True
    costs.sort(reverse=True)
    loads = [0] * min(wgs, len(costs))
    heapq.heapify(loads)
    for c in costs:
        heapq.heappush(loads, heapq.heappop(loads) + c)
    return max(loads) <= sum(costs) / wgs + _BALANCE_OVERHEAD


def _choose_per_unit(batch: int, total_q: int, max_q: int, max_k: int | None, causal: bool,
                     h_q: int, h_kv: int, d: int, dev: torch.device) -> bool:
    if max_k is None:
        return False
    if causal and max_k <= max_q:
        return True  # no cached context: first chunks
    if batch != 1:
        return False
    rows = 128 if d == 256 else 256           # rows of a workgroup (the kernel's launch shape)
    wgs = torch.cuda.get_device_properties(dev).multi_processor_count
    return _per_unit_wins(int(total_q), int(max_k), bool(causal), h_kv, h_q // h_kv, rows, wgs)


def _aligned_rows(t: torch.Tensor) -> bool:
    return (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
            and all(s % 8 == 0 for s in t.stride()[:-1]))


def gqa_prefill_paged_fn(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    seqlen_k: torch.Tensor,
    max_seqlen_q: int | None = None,
    page_size: int = 16,
    *,
    causal: bool = True,
    out: torch.Tensor | None = None,
    batch_invariant: bool = False,
    max_seqlen_k: int | None = None,
    schedule: str = "auto",
    gate: torch.Tensor | None = None,
) -> torch.Tensor:
    """Varlen (causal) GQA attention of packed queries over paged K/V.

    Args:
        q: [total_q, H_q, D] packed query rows (the reference's ``q_unpad``)
        k_cache, v_cache: [num_blocks, block_size, H_kv, D] one layer's cache, contiguous
        block_table: [B, W] int32 physical page ids (-1 padding past each sequence is never read)
        cu_seqlens_q: [B + 1] int32 query row offsets
        seqlen_k: [B] int32 cached tokens per sequence, the chunk included (the reference's
            ``cu_seqlens_k[b+1] - cu_seqlens_k[b]``, i.e. ``full_kv_len``)
        max_seqlen_q: host bound on every query length (the reference's ``max_seqlen_q``); None
            reads it from ``cu_seqlens_q`` (one device-to-host copy)
        page_size: tokens per page of the flattened cache (4, 8 or a multiple of 16)
        causal: keyword-only; False drops the causal mask (the reference's ``is_causal=False``)
        out: keyword-only preallocated [total_q, H_q, D] output
        batch_invariant: keyword-only; forces the per-unit schedule (bitwise batch- and
            chunking-invariant rows)
        max_seqlen_k: keyword-only host bound on every ``seqlen_k`` (the reference's
            ``ctx.max_seqlen_k``); only used to choose the schedule
        schedule: keyword-only, "auto", "balanced" or "per_unit" (see the module docstring)
        gate: keyword-only; the attention output gate (model/qwen_36.py:1083), total_q * H_q * D
            values laid out [total_q, H_q, D] (``q_gate`` [1, q_len, H_q * D] as the model has it):
            the output is ``prefill * sigmoid(gate)``, applied in the kernels' epilogue — bitwise
            ``fused_sigmoid_mul(gqa_prefill_paged_fn(...), gate)``.
    Returns:
        [total_q, H_q, D] tensor in q's dtype.
    """
    if q.dim() != 3:
        raise ValueError(f"q must be [total_q, H_q, D], got {tuple(q.shape)}")
    total_q, h_q, d = q.shape
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
    for name, t in (("block_table", block_table), ("cu_seqlens_q", cu_seqlens_q),
                    ("seqlen_k", seqlen_k)):
        if t.dtype != torch.int32:
            raise TypeError(f"{name} must be int32, got {t.dtype}")
    if block_table.dim() != 2:
        raise ValueError(f"block_table must be [B, W], got {tuple(block_table.shape)}")
    batch = block_table.shape[0]
    if cu_seqlens_q.shape != (batch + 1,):
        raise ValueError(f"cu_seqlens_q must be [{batch + 1}], got {tuple(cu_seqlens_q.shape)}")
    if seqlen_k.shape != (batch,):
        raise ValueError(f"seqlen_k must be [{batch}], got {tuple(seqlen_k.shape)}")
    page_size = int(page_size)
    rows = nb * bs
    if page_size <= 0 or rows % page_size != 0:
        raise ValueError(f"page_size {page_size} does not tile the cache's {rows} rows")
    dev = q.device
    if dev.type != "cuda":
        raise ValueError("gqa_prefill_paged_fn runs on the GPU; q is on " + str(dev))
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache), ("block_table", block_table),
                    ("cu_seqlens_q", cu_seqlens_q), ("seqlen_k", seqlen_k)):
        if t.device != dev:
            raise ValueError(f"{name} is on {t.device}, q on {dev}")
    if block_table.stride(-1) != 1:
        block_table = block_table.contiguous()
    cu_seqlens_q = cu_seqlens_q.contiguous()
    seqlen_k = seqlen_k.contiguous()
    if max_seqlen_q is None:
        max_seqlen_q = int((cu_seqlens_q[1:] - cu_seqlens_q[:-1]).max().item()) if batch else 0
    max_seqlen_q = int(max_seqlen_q)
    if max_seqlen_q < 0:
        raise ValueError(f"max_seqlen_q must be >= 0, got {max_seqlen_q}")
    if not _aligned_rows(q):
        q = q.contiguous()
    if out is None:
        out = torch.empty((total_q, h_q, d), dtype=dt, device=dev)
    elif (out.shape != (total_q, h_q, d) or out.dtype != dt or out.device != dev
          or not _aligned_rows(out)):
        raise ValueError("out must be a [total_q, H_q, D] tensor of q's dtype and device with "
                         "16-byte aligned rows")
    g3 = None
    if gate is not None:
        if gate.numel() != total_q * h_q * d or gate.dtype != dt or gate.device != dev:
            raise ValueError(f"gate must hold {total_q}x{h_q}x{d} values of q's dtype on q's device")
        g3 = gate.reshape(total_q, h_q, d)
        if not _aligned_rows(g3):
            g3 = g3.contiguous()
    if batch == 0 or total_q == 0:
        return out
    width = block_table.shape[1]
    lib = _lib.load()
    if schedule not in ("auto", "balanced", "per_unit"):
        raise ValueError(f"schedule must be 'auto', 'balanced' or 'per_unit', got {schedule!r}")
    per_unit = batch_invariant or schedule == "per_unit" or (
        schedule == "auto" and _choose_per_unit(batch, total_q, max_seqlen_q, max_seqlen_k, causal,
                                                h_q, h_kv, d, dev))
    ws, ws_bytes = None, 0
    if not per_unit:
        ws_bytes = _workspace_bytes(batch, total_q, h_q, h_kv, d, page_size, width)
        if ws_bytes > 0:
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    args = (q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(),
            block_table.data_ptr(), block_table.stride(0) if width > 0 else 0,
            cu_seqlens_q.data_ptr(), seqlen_k.data_ptr(), out.data_ptr(), out.stride(0),
            out.stride(1), ws.data_ptr() if ws is not None else None, ws_bytes,
            batch, total_q, max_seqlen_q, h_q, h_kv, d, page_size, rows // page_size, width,
            1 if causal else 0, code)
    if g3 is None:
        _lib.check(lib.ti_gqa_prefill_paged(*args, _lib.stream_handle(dev)))
    else:
        _lib.check(lib.ti_gqa_prefill_paged_gated(*args, g3.data_ptr(), g3.stride(0), g3.stride(1),
                                                  _lib.stream_handle(dev)))
    return out
