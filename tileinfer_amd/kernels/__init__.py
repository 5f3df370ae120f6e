"""Drop-in replacements for tileInfer's ``kernels.kvcache_store`` and ``kernels.gqa_decode_paged``."""
from .gqa_decode_paged import gqa_decode_paged_fn  # noqa: F401
from .kvcache_store import store_kvcache  # noqa: F401
