/*
 * pagegauge_bench.h -- C ABI of libpagegauge_bench.so, bench.py's
 * measurement helpers.  None of these has a counterpart in the reference,
 * which never measures its GPU's peak; none is part of the decode path, and
 * the product library (pagegauge_hip.h) does not export them.
 *
 * Conventions as in pagegauge_hip.h: device pointers, a hipStream_t passed as
 * void*, PG_OK (0) or an error code, and pg_last_error() of this library for
 * the message.  start_event / stop_event (hipEvent_t, may be NULL): the
 * dispatch stamps its own begin and end.
 */
#ifndef PAGEGAUGE_BENCH_H
#define PAGEGAUGE_BENCH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message of the last failing call on this thread ("" if none). */
const char* pg_last_error(void);
/* ABI version of the library (the product's, 4). */
int32_t pg_abi_version(void);

/* ------------------------------------------------------------------------
 * HBM read probes: the read bandwidth this device reaches, beside the
 * specification's 8 TB/s.  sink: int32 [sink_len] device buffer; workgroup
 * b may write sink[b] (only under a condition on the loaded data, so its
 * contents are meaningless), and every probe refuses a grid with more
 * workgroups than sink_len.
 * ---------------------------------------------------------------------- */

/* Grid-stride read of ``bytes`` contiguous bytes (16-byte aligned multiple
 * of 16), 16 B per lane per load, ``blocks`` workgroups of 256 threads. */
int32_t pg_probe_linear_read(const void* src, int64_t bytes, int32_t* sink, int64_t sink_len,
                             int32_t blocks, void* start_event, void* stop_event, void* stream);
/* Reads pages indices[0..pages) of two page pools, each page as one
 * contiguous block of ``page_bytes`` K bytes and ``page_bytes`` V bytes,
 * ``pages_per_block`` pages per 256-thread workgroup. */
int32_t pg_probe_page_walk(const void* k_pages, const void* v_pages, const int32_t* indices,
                           int32_t pages, int32_t pages_per_block, int32_t page_bytes,
                           int32_t* sink, int64_t sink_len, void* start_event, void* stop_event,
                           void* stream);
/* Reads pages indices[0..pages) the way the INT8 decode kernel does, loads
 * only: work items of ``pages_per_item`` consecutive entries (4..64, a
 * multiple of 4, dividing ``pages``), one wave per KV head (8 KV heads of
 * 128 codes, 16 KiB pages), ``heads_per_block`` (4 or 8) waves per
 * workgroup, 4-page groups with ``depth`` (1 or 2) groups in flight per wave.
 * ``mode`` 0 = the decode kernel's lane pattern, 1 = whole 128-byte head
 * rows per lane group, 2 = whole pages as contiguous 1 KiB per instruction
 * (heads_per_block 8).  Gives the stream rate of the decode's own access
 * pattern, to set the decode kernel against. */
int32_t pg_probe_decode_walk(const void* k_pages, const void* v_pages, const int32_t* indices,
                             int32_t pages, int32_t pages_per_item, int32_t heads_per_block,
                             int32_t depth, int32_t mode, int32_t* sink, int64_t sink_len,
                             void* start_event, void* stop_event, void* stream);

/* ------------------------------------------------------------------------
 * Phase trace of the decode kernels.  Exported only by the trace builds of
 * the product library (python -m pagegauge_amd.build --variant trace), not
 * by libpagegauge_bench.so: sets the device buffer the partial kernel
 * writes one 64-word row per wave into (s_memrealtime marks of the wave's
 * start, page-id arrival, first loads issued, scale arrival, each group's K
 * and V arrival, end; XCC and HW_ID registers), followed by one row per
 * wave of the four-workgroup combine kernel (start, value center and item
 * range arrival, partial rows arrival, maximum, sums, end; lane 56 holds
 * 100).  A launch whose rows do not fit in ``bytes`` writes none; NULL
 * turns the trace off.
 * ---------------------------------------------------------------------- */
int32_t pg_trace_set_buffer(void* device_words, int64_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* PAGEGAUGE_BENCH_H */
