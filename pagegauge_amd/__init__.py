"""PageGauge compressed-KV decode path for AMD MI355X (gfx950).

Hand-written HIP kernels behind the C ABI of ``libpagegauge_hip.so``
(``include/pagegauge_hip.h``), with Python operators that keep the reference's
call signatures:

* ``runtime.load_append_extension()`` -- fused RoPE + (centered) append +
  completed-page INT8 finalize, the fused exact-tail merge;
* ``decode`` -- paged decode over INT8 page-affine and FP16 pages
  (``BatchDecodeWithPagedKVCacheWrapper``, ``make_page_gauge_wrapper``,
  ``PageGaugeSegmentedDecode``, ``merge_state_in_place``);
* ``page_table`` -- the page-table algebra of the decoder harness;
* ``scheduler`` -- split-KV selection for 256 CUs.
"""

__all__ = ["runtime", "decode", "page_table", "scheduler", "workloads"]
