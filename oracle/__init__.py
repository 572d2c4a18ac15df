"""CPU oracle of the sparse-attention KV-retrieval path -- test infrastructure.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import anything here, and only as the checker.  The product
package ``kv_cache_amd`` never imports it.

* ``qkv_oracle``    -- numpy specification of the int4 path (pack, channel
                       subset, slab, int32 scores, block max, top-k, fp64
                       attention, prefill scoring).
* ``ref_semantics`` -- numpy restatement of the reference's four fp32 kernels
                       and its PyTorch CPU op sequence (the CPU baseline).
"""
