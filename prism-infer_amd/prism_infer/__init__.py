"""MI355X-native (gfx950) drop-in for Prism-Infer's scaled-FP8 paged KV ops.

Only the hot path lives here: ``prism_infer.ops.kv_cache_store``,
``prism_infer.ops.paged_decode`` and ``prism_infer.ops.kv_compaction`` with the
reference's call signatures, plus the format constants of
``prism_infer.engine.kv_quantization`` and the compaction slot planner of
``prism_infer.engine.kv_compaction_plan``.  The ops call hand-written HIP
kernels in ``_native/libprism_mi355x.so`` through a C ABI; there is no Triton
and no CPU fallback.
"""

__version__ = "0.1.0"
