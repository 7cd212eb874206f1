"""Physical compressed-KV-cache decode path on MI355X (drop-in for ``dynakv.kernels``).

Modules mirror the reference package ``src/dynakv/kernels/``:

* :mod:`.router` -- ``KernelPolicy`` and ``compressed_decode_attention``
* :mod:`.compressed_cache` -- ``CustomDynamicCache`` (packed coefficient cache)
* :mod:`.fused` -- ``fused_attention_dispatch`` (short-cache route)
* :mod:`.two_stage` -- ``abx_sparse`` and ``avx`` (long-cache route)
* :mod:`.decode` -- the native multi-group split-K entry used by the benchmark
"""
