"""CPU oracle for tileInfer's paged KV-cache path. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import this
package, and only as the checker (or as the timed CPU baseline). The product path
(``tileinfer_amd``) never imports it and has no CPU fallback.

Contents
  ref_torch.ref_store_kvcache     restates kernels/kvcache_store.py:74-84  (torch, CPU)
  ref_torch.ref_gqa_decode_paged  restates kernels/gqa_decode_paged.py:444-461 (torch, CPU)
  brute.store_np                  closed form of the append on numpy arrays
  brute.decode_fp64               textbook single-query attention in float64 (numpy)
  brute.decode_loop_fp64          the same as scalar loops, for tiny inputs
  ref_torch.ref_gqa_prefill_paged restates model/qwen_36.py:1034-1044 + kernels/gqa_varlen.py:88-175
  brute.prefill_fp64              textbook chunked causal attention in float64 (numpy)
  ref_metadata.RefDecodePrep      restates engine/model_runner.py:538-584 (per-step decode metadata)

How each function is pinned (checks live in tests/test_oracle.py):
  ref_store_kvcache      equals the closed form (cache unchanged except rows slot>=0 = key rows)
                         on random and edge inputs (N=0, all -1, fp16), and the committed golden
                         fixture of config 1.
  ref_gqa_decode_paged   within bf16 rounding of decode_fp64; bitwise invariants (physical block
                         permutation, shared vs private prefix, -1 padding ignored, ctx=1 gives
                         V[0], constant V gives V, ctx=0 gives zeros, head h reads KV head h//G);
                         a hand-computed 2-token case; the committed config-1 golden fixture.
  decode_fp64            closed forms (ctx=1, constant V, equal scores -> mean of V) and a
                         brute-force loop on tiny inputs written independently of the vectorised
                         form.
  prefill_fp64           each chunk row equals decode_fp64 over the keys it sees (pins the
                         bottom-right mask), and torch's scaled_dot_product_attention in float64
                         on first and unmasked chunks (tests/test_oracle_prefill.py).
  ref_gqa_prefill_paged  within tolerance of prefill_fp64; planted mistakes (top-left mask,
                         h % Hkv, dropped scale, one key short) must fail.
  RefDecodePrep          equals kv_layout.decode_metadata (itself checked against the slot
                         definition and graph padding in tests/test_engine.py) on CPU
                         (tests/test_oracle_metadata.py).
The reference publishes no golden vectors for this path and its own self-checks are random-input
tolerance checks (kernels/kvcache_store.py:87-115, kernels/gqa_decode_paged.py:468-536); the
reference modules import tilelang, which is absent here, so nothing from /root/reference is run.
"""
