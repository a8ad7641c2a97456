"""CPU oracle for the CacheIR decode-step hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy (and plain C under ``oracle/c``), the arithmetic of
CacheIR's reference CPU backend for the decode step, so the HIP backend in
``cacheir_amd`` can be checked against it on identical seeded inputs.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import or run anything here, and only as the checker or as the
reported CPU baseline.  The product path (``cacheir_amd``) never imports it.

Modules and the reference code each one restates (paths relative to the
reference repository root):

* ``ops``      -- ``cacheir/runtime/cpu.py:221-377`` (rms_norm, matmul, interleaved
                  RoPE, GQA softmax attention, SiLU-mul) and ``cpu.py:181-182``
                  (greedy argmax).
* ``quant``    -- ``cacheir/importers/gguf.py:249-310`` (Q4_0 / Q8_0 block decode) and
                  ``cacheir/quantization.py:63-139`` (per-row asymmetric int4/int8).
* ``paged``    -- ``cacheir/runtime/kv_cache.py:66-122`` (page extension) and the
                  page-table gather of ``cacheir/backends/triton_kernels.py:174-217``.
* ``runtime``  -- ``cacheir/runtime/cpu.py:82-184`` (graph walk, KV cache, greedy
                  generate) and ``cacheir/importers/tiny.py:9-65`` (tiny model draw
                  order).
* ``cbase``    -- ctypes bridge to ``oracle/c/oracle_cpu.c`` (OpenMP C restatement of
                  the same kernels, used for the timed CPU baseline).

Parity pinning (what fixes each function beyond re-typing its formula) is listed in
each module's docstring.
"""
