"""Drop-in replacements for tileInfer's ``kernels.kvcache_store`` and ``kernels.gqa_decode_paged``,
the paged prefill attention that replaces its gather + ``kernels.gqa_varlen`` call, and block
copies for swapping."""
from .block_copy import copy_blocks, swap_blocks  # noqa: F401
from .gqa_decode_paged import gqa_decode_paged_fn  # noqa: F401
from .gqa_prefill_paged import gqa_prefill_paged_fn  # noqa: F401
from .kvcache_store import store_kvcache  # noqa: F401
