"""tileinfer_amd — tileInfer's paged KV-cache hot path on MI355X (gfx950).

* ``tileinfer_amd.kernels.kvcache_store.store_kvcache``      slot-mapped K/V append
* ``tileinfer_amd.kernels.gqa_decode_paged.gqa_decode_paged_fn``  paged GQA decode (split-K)
* ``tileinfer_amd.engine``  block manager, prefix cache, sequences and the metadata builders

The kernels live in ``libtileinfer_amd.so`` (HIP, built by ``python -m tileinfer_amd.build``) and
are reached through its C ABI (``include/tileinfer_amd.h``); importing this package does not load
the library, the first kernel call does.
"""
__version__ = "0.1.0"
