"""CPU oracle for the compressed-cache decode path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference's algorithm (LUMIA-Group/DynaKV, ``src/dynakv/kernels/`` and
the masked-dimension research path ``src/dynakv/custom_attn.py``) in numpy / CPU torch so the
gfx950 kernels can be checked against it. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker or the reported CPU
baseline: the product path (``dynakv_amd``) never imports, links or calls anything here.

Modules and the reference code each follows:

* ``router``     -- ``KernelPolicy.select`` closed form (router.py:8-17).
* ``packing``    -- packed-cache layout and growth policy (compressed_cache.py:7-34, 96-227).
* ``attention``  -- decode attention over a packed cache, both routes (fused.py:28-142,
                    two_stage.py:28-157 and 207-281).
* ``masked_dim`` -- the dense masked-dimension CPU path (custom_attn.py:140-191, 214-259),
                    used as an independent formulation to pin ``attention`` and as the CPU
                    baseline that ``bench.py`` times.

How each function is pinned (none is "parity unpinned"):

* ``router``: the reference's own known-answer tests (tests/test_kernel_router.py:7-20).
* ``packing``: hand-computed layouts and capacities from the reference's arithmetic, plus the
  invariants (offs = exclusive prefix sum of lens, ptr = sum of lens, payload = first-r prefix,
  zero tail) checked on random and edge-case inputs (tests/test_oracle_packing.py).
* ``attention``: agreement with ``masked_dim`` (a different formulation: dense masked
  coefficients, joint block-diagonal basis, HF-style rotate-half RoPE, eager softmax), closed
  forms (one token -> its V; zero query -> mean of V; identity basis at position 0 -> plain
  attention), the RoPE norm/relative-position identities, and brute-force scalar loops on tiny
  inputs (tests/test_oracle_attention.py).
"""
