"""PageGauge compressed-KV decode path for AMD MI355X (gfx950).

Hand-written HIP kernels behind the C ABI of ``libpagegauge_hip.so``
(``include/pagegauge_hip.h``), with Python operators that keep the reference's
call signatures:

* ``runtime.load_append_extension()`` -- fused RoPE + (centered) append +
  completed-page INT8 finalize, the fused exact-tail merge;
* ``decode`` -- paged decode over INT8 page-affine and FP16 pages
  (``BatchDecodeWithPagedKVCacheWrapper``, ``make_page_gauge_wrapper``,
  ``PageGaugeSegmentedDecode``, the heterogeneous one-table wrapper,
  ``merge_state_in_place``) and the split scheduler (``plan_work_items``);
* ``update`` -- the paged append / finalize, bulk quantizers, prefill
  population and exact centers;
* ``page_table`` -- the page-table algebra of the decoder harness;
* ``decoder`` -- the Mistral-shaped decoder over these kernels;
* ``serving`` / ``serving_bridge`` -- request slots, decode-batch tables and
  the scheduler bridge;
* ``workloads`` -- the seeded benchmark configurations.
"""

__all__ = ["runtime", "decode", "update", "page_table", "decoder", "serving", "serving_bridge",
           "workloads"]
