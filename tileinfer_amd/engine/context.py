"""Per-thread carrier of the paged-attention metadata of one forward pass.

Mirrors tileInfer's ``engine/context.py:7-49``: the runner fills an ``AttentionContext`` and
publishes it with ``set_context`` before the forward pass; each attention layer reads it with
``get_context`` (``model/qwen_36.py:1005-1006``) to find ``slot_mapping`` for the append and
``block_tables`` / ``context_lens`` for decode.
"""
from __future__ import annotations

import threading

_local = threading.local()


class AttentionContext:
    __slots__ = (
        "slot_mapping",   # [total_tokens] int32 cache row of each new token, -1 = skip
        "block_tables",   # [bsz, max_blocks] int32 physical page ids, -1 padded
        "context_lens",   # [bsz] int32 tokens visible to decode (including the new one)
        "cu_seqlens_q",   # [bsz+1] prefill query offsets
        "cu_seqlens_k",   # [bsz+1] prefill key offsets
        "max_seqlen_q",
        "max_seqlen_k",
        "deltanet_slots",  # carried for signature parity with the reference; unused here
        "is_prefill",
    )

    def __init__(self):
        self.slot_mapping = None
        self.block_tables = None
        self.context_lens = None
        self.cu_seqlens_q = None
        self.cu_seqlens_k = None
        self.max_seqlen_q = 0
        self.max_seqlen_k = 0
        self.deltanet_slots = None
        self.is_prefill = False


def get_context() -> AttentionContext | None:
    return getattr(_local, "attn_ctx", None)


def set_context(ctx: AttentionContext | None) -> None:
    _local.attn_ctx = ctx


def reset_context() -> None:
    _local.attn_ctx = None
