"""Drop-in replacements for tileInfer's ``kernels.kvcache_store``, ``kernels.gqa_decode_paged``,
``kernels.qknorm_rope.fused_qknorm_rope`` and ``kernels.act_mul.fused_sigmoid_mul``; the paged
prefill attention that replaces its gather + ``kernels.gqa_varlen`` call; the fused
QK-norm + RoPE + append; block copies for swapping."""
from .act_mul import fused_sigmoid_mul  # noqa: F401
from .block_copy import copy_blocks, swap_blocks  # noqa: F401
from .gqa_decode_paged import gqa_decode_paged_fn  # noqa: F401
from .gqa_prefill_paged import gqa_prefill_paged_fn  # noqa: F401
from .kvcache_store import store_kvcache  # noqa: F401
from .qknorm_rope import fused_qknorm_rope, qknorm_rope, qknorm_rope_append  # noqa: F401
