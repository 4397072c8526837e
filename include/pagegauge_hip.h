/*
 * pagegauge_hip.h -- C ABI of libpagegauge_hip.so, the MI355X (gfx950)
 * implementation of PageGauge's compressed-KV decode path.
 *
 * Plain pointers and sizes only.  Every pointer argument is device memory
 * unless its name starts with ``host_``; ``stream`` is a hipStream_t passed as
 * void* (NULL = the null stream).  Every function returns PG_OK (0) or an
 * error code; pg_last_error() then gives the message of the failing call on
 * the calling thread.  No entry point allocates device memory, synchronises
 * the stream or returns data to the host except pg_decode_plan (which copies
 * a work list into the caller's workspace and waits for that copy).
 *
 * Layouts (reference conventions, tests/page_gauge_append_extension.cu:1-40):
 *   query / key / value rows   fp16 [B, H, 128] with contiguous head rows,
 *                              batch stride given in elements
 *   FP16 and INT8 page caches  NHD [pages, 16, Hkv, 128]
 *   page scales                fp16 [pages, Hkv]
 *   centers                    fp16 [B, Hkv, 128] (or [Hkv, 128] when B == 1)
 *   lse                        float32 [B, Hq], base 2 (log2-sum-exp2 of
 *                              sm_scale*log2(e)*q.k)
 */
#ifndef PAGEGAUGE_HIP_H
#define PAGEGAUGE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  PG_OK = 0,
  PG_ERROR_INVALID_ARGUMENT = 1,
  PG_ERROR_LAUNCH = 2,
  PG_ERROR_UNSUPPORTED = 3,
  PG_ERROR_WORKSPACE = 4
};

/* Message of the last failing call on this thread ("" if none). */
const char* pg_last_error(void);
/* ABI version of this library (increments on incompatible changes). */
int32_t pg_abi_version(void);

/* ------------------------------------------------------------------------
 * Cache update (K2).  Replaces the pybind entry points of
 * tests/page_gauge_append_extension.cu:1030-1040.
 * ---------------------------------------------------------------------- */

/* Fused RoPE + FP16 NHD append.  Replaces rope_append_fp16
 * (tests/page_gauge_append_extension.cu:644-685) when device_position is NULL
 * (position = host_position, cosine/sine are the [128] rows of that
 * position) and rope_append_fp16_dynamic (:687-745) otherwise (position read
 * on the device from device_position[0]; cosine/sine are [rope_rows, 128]
 * tables with row stride rope_row_stride).  Writes rotated_query [B,Hq,128]
 * and row (position % 16) of physical page request*pages_per_request +
 * position/16.  A position outside the cache (or the RoPE table) is a no-op,
 * as in the reference kernel (:202-207). */
int32_t pg_rope_append_fp16(const void* query, const void* key, const void* value,
                            const void* cosine, const void* sine, void* rotated_query,
                            void* key_pages, void* value_pages,
                            int64_t query_batch_stride, int64_t key_batch_stride,
                            int64_t value_batch_stride, int32_t batch_size,
                            int32_t query_heads, int32_t kv_heads,
                            int32_t pages_per_request, int32_t host_position,
                            const int32_t* device_position, int64_t rope_row_stride,
                            int32_t rope_rows, void* stream);

/* Fused RoPE + centered K/V append into the FP16 exact ring + completed-page
 * INT8 finalize.  Replaces rope_append_page_gauge
 * (tests/page_gauge_append_extension.cu:747-836, device_position == NULL)
 * and rope_append_page_gauge_dynamic (:838-948).  Ring slot of logical page p
 * is request*exact_pages_per_request + (p < sink ? p : sink + p % (E - sink));
 * on the page's last token the page is quantised into code page
 * request*code_pages_per_request + p and scale row of that code page.
 * center_batch_stride is Hkv*128 for [B,Hkv,128] centers, 0 for [Hkv,128]. */
int32_t pg_rope_append_page_gauge(const void* query, const void* key, const void* value,
                                  const void* cosine, const void* sine,
                                  const void* key_center, const void* value_center,
                                  int64_t center_batch_stride, void* rotated_query,
                                  void* exact_key_pages, void* exact_value_pages,
                                  int8_t* key_codes, int8_t* value_codes,
                                  void* key_scales, void* value_scales,
                                  int64_t query_batch_stride, int64_t key_batch_stride,
                                  int64_t value_batch_stride, int32_t batch_size,
                                  int32_t query_heads, int32_t kv_heads,
                                  int32_t exact_pages_per_request, int32_t exact_sink_pages,
                                  int32_t code_pages_per_request, int32_t host_position,
                                  const int32_t* device_position, int64_t rope_row_stride,
                                  int32_t rope_rows, void* stream);

/* Per-request-position variant of pg_rope_append_page_gauge (no reference
 * counterpart in the CUDA extension; the per-request page semantics follow
 * the Triton append_finalize_page_gauge,
 * scripts/benchmark_page_gauge_overheads.py:112-205).  Request r uses
 * position positions[r] (device int32 [B]) and RoPE row positions[r] of the
 * [rope_rows, 128] tables; each row behaves exactly as the scalar kernel. */
int32_t pg_rope_append_page_gauge_positions(
    const void* query, const void* key, const void* value, const void* cosine,
    const void* sine, const int32_t* positions, const void* key_center,
    const void* value_center, int64_t center_batch_stride, void* rotated_query,
    void* exact_key_pages, void* exact_value_pages, int8_t* key_codes,
    int8_t* value_codes, void* key_scales, void* value_scales,
    int64_t query_batch_stride, int64_t key_batch_stride, int64_t value_batch_stride,
    int32_t batch_size, int32_t query_heads, int32_t kv_heads,
    int32_t exact_pages_per_request, int32_t exact_sink_pages,
    int32_t code_pages_per_request, int64_t rope_row_stride, int32_t rope_rows,
    void* stream);

/* Serving-table variant of pg_rope_append_page_gauge_positions (no kernel
 * of the reference: its serving prototype leaves the device scatter open,
 * experiments/mlsys2027/serving_v1/pagegauge_vllm/decode_metadata.py:1-5).
 * Row r appends the token at positions[r] into row positions[r] % 16 of
 * exact page exact_page_ids[r] (FP16 centered) and, on the page's 16th
 * token, quantises that exact page into code page code_page_ids[r]; both ids
 * come from the caller's block tables (any physical page, any exact slot).
 * Rows with a negative id or one outside [0, num_exact_pages) /
 * [0, num_code_pages) are skipped.  RoPE rows come from the [rope_rows, 128]
 * tables at positions[r]. */
int32_t pg_rope_append_page_gauge_slots(
    const void* query, const void* key, const void* value, const void* cosine,
    const void* sine, const int32_t* positions, const int32_t* exact_page_ids,
    const int32_t* code_page_ids, const void* key_center, const void* value_center,
    int64_t center_batch_stride, void* rotated_query, void* exact_key_pages,
    void* exact_value_pages, int8_t* key_codes, int8_t* value_codes, void* key_scales,
    void* value_scales, int64_t query_batch_stride, int64_t key_batch_stride,
    int64_t value_batch_stride, int32_t batch_size, int32_t query_heads, int32_t kv_heads,
    int64_t num_exact_pages, int64_t num_code_pages, int64_t rope_row_stride,
    int32_t rope_rows, void* stream);

/* Per-request FP16 append at (page_ids[r], page_offsets[r]).  Replaces the
 * Triton append_kv (scripts/benchmark_page_gauge_overheads.py:86-109,
 * :242-269).  key/value contiguous [B, H, 128]. */
int32_t pg_append_kv(const void* key, const void* value, void* key_pages, void* value_pages,
                     const int32_t* page_ids, const int32_t* page_offsets,
                     int32_t batch_size, int32_t heads, int32_t num_pages, void* stream);

/* Per-request centered append + completed-page finalize without RoPE.
 * Replaces the Triton append_finalize_page_gauge
 * (scripts/benchmark_page_gauge_overheads.py:112-205, :272-317).  Exact and
 * code caches share page indices; centers are [H,128]. */
int32_t pg_append_finalize_page_gauge(const void* key, const void* value,
                                      const void* key_center, const void* value_center,
                                      void* exact_key_pages, void* exact_value_pages,
                                      int8_t* key_codes, int8_t* value_codes,
                                      void* key_scales, void* value_scales,
                                      const int32_t* page_ids, const int32_t* page_offsets,
                                      int32_t batch_size, int32_t heads, int32_t num_pages,
                                      void* stream);

/* Bulk completed-page quantizer.  Replaces the Triton
 * quantize_completed_kv_pages (scripts/benchmark_page_gauge_overheads.py:23-83,
 * :208-239): float32-centered values, scale fp16(max(amax/127, 2^-20)),
 * sign-symmetric floor(q+0.5) codes.  key/value [pages,16,H,128] fp16,
 * centers [H,128]. */
int32_t pg_quantize_completed_kv_pages(const void* key, const void* value,
                                       const void* key_center, const void* value_center,
                                       int8_t* key_codes, int8_t* value_codes,
                                       void* key_scales, void* value_scales,
                                       int64_t num_pages, int32_t heads, void* stream);

/* The K1 driver's page quantizer quantize_page_gauge
 * (scripts/benchmark_flashinfer_page_affine_int8.py:256-278) given its
 * center: values [pages,16,H,128] fp16, center [H,128] fp16; float32-centered
 * values, scale fp16(max(amax/127, 2^-20)) per (page, head) into scales
 * [pages,H], codes round-half-even(x / scale) clamped to [-127, 127] (torch's
 * round) into codes [pages,16,H,128] int8.  One tensor per call. */
int32_t pg_quantize_page_gauge(const void* values, const void* center, int8_t* codes,
                               void* scales, int64_t num_pages, int32_t heads, void* stream);

/* Prefill cache population of one (layer, request): the bulk quantizer above
 * plus the centered FP16 exact pages, in one launch.  Replaces the body of
 * populate_backend_cache_layer (diagnostics/benchmark_backend_exclusive.py:442-506)
 * and the per-page copies of build_caches
 * (scripts/benchmark_page_gauge_transformer.py:1215-1245).
 *   key/value: token-major prefix [pages*16, H, 128] fp16 whose token rows are
 *     key_token_stride / value_token_stride elements apart (>= H*128, even;
 *     e.g. a K/V slice of a fused QKV projection);
 *   codes [pages,16,H,128] int8 and scales [pages,H] fp16 receive every page;
 *   exact_page_map: optional int32[pages]; page i is also written as
 *     fp16(f32(x) - f32(center)) to ring page exact_page_map[i] of
 *     exact_key_pages / exact_value_pages ([*,16,H,128] fp16) when >= 0. */
int32_t pg_prefill_page_gauge(const void* key, int64_t key_token_stride, const void* value,
                              int64_t value_token_stride, const void* key_center,
                              const void* value_center, int8_t* key_codes, int8_t* value_codes,
                              void* key_scales, void* value_scales,
                              const int32_t* exact_page_map, void* exact_key_pages,
                              void* exact_value_pages, int64_t num_pages, int32_t heads,
                              void* stream);

/* Per-(head, dim) channel centers of a token-major K/V prefix: replaces
 * token_major_centers (diagnostics/benchmark_backend_exclusive.py:372-395) and
 * the center lines of build_caches (scripts/benchmark_page_gauge_transformer.py:1201-1214),
 * `x.float().mean(dim=tokens).half()`.  The float32 reduction order of the
 * reference is unspecified; here the sum is exact (int64 multiples of 2^-24),
 * and the center is f16(f32(f64(sum)/tokens)), independent of order.
 * tokens <= 2^22.  Workspace: pg_token_major_centers_workspace_bytes bytes of
 * device memory, caller-owned; two launches, no allocation, no memset. */
int64_t pg_token_major_centers_workspace_bytes(int64_t tokens, int32_t heads);
int32_t pg_token_major_centers(const void* key, int64_t key_token_stride, const void* value,
                               int64_t value_token_stride, int64_t tokens, int32_t heads,
                               void* key_center, void* value_center, void* workspace,
                               int64_t workspace_bytes, void* stream);

/* pg_token_major_centers without a workspace argument, for callers that
 * cannot allocate (code under HIP graph capture, serving loops that forbid
 * allocation).  It has no counterpart in the reference.  The chunk sums live
 * in a file-scope device array of pg_token_major_centers_noalloc_max_bytes()
 * bytes (8 MiB: ceil(tokens / 64) * heads <= 4096), one copy per GPU, held
 * until the process ends; larger calls fail with PG_ERROR_WORKSPACE.  The
 * call allocates nothing (no hipMalloc, hipFree or memset); the stream must
 * belong to the current device.  Every call on a GPU shares that GPU's
 * array: calls that overlap on one GPU (other streams, other threads) race
 * and must be serialised by the caller.  Results are bit-identical to
 * pg_token_major_centers.  The first call on a device resolves that
 * device's scratch address (hipGetSymbolAddress) and caches it: make it
 * once before capturing the call in a graph, and do not reset the device
 * (hipDeviceReset) while the library is loaded. */
int64_t pg_token_major_centers_noalloc_max_bytes(void);
int32_t pg_token_major_centers_noalloc(const void* key, int64_t key_token_stride,
                                       const void* value, int64_t value_token_stride,
                                       int64_t tokens, int32_t heads, void* key_center,
                                       void* value_center, void* stream);

/* ------------------------------------------------------------------------
 * Paged decode (K1) and the split scheduler (S).
 * ---------------------------------------------------------------------- */

/* Host-side description of a planned decode; filled by pg_decode_plan and
 * passed unchanged to pg_decode_run.  Plain data, safe to copy. */
typedef struct pg_decode_plan {
  int32_t batch_size;
  int32_t num_qo_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t page_size;
  int32_t primary_kind;   /* PG_KV_INT8, PG_KV_FP16 or PG_KV_HETEROGENEOUS (segment 0) */
  int32_t has_tail;       /* 1 if an FP16 tail segment joins the softmax */
  int32_t split_pages;    /* pages per work item, segment 0 */
  int32_t tail_split_pages;
  int32_t num_items;      /* work items (one workgroup each) */
  int32_t num_items_primary;
  int32_t max_items_per_request;
  int32_t waves_per_block; /* KV heads (one wave each) per workgroup of the partial kernel */
  /* closed_form = 1 (one request): work item i is derived from the block
   * index instead of being loaded.  The FP16 tail segment's cf_tail_items
   * items come first, then the primary segment's; segment s with n pages in
   * c items gives item k the pages [begin + k*(n/c) + min(k, n%c), +
   * n/c + (k < n%c)).  The planner sets it only when this reproduces every
   * work item it wrote. */
  int32_t closed_form;
  int32_t cf_tail_items;
  int32_t cf_tail_begin;
  int32_t cf_tail_pages;
  int32_t cf_primary_begin;
  int32_t cf_primary_pages;
  int32_t reserved;
  int64_t items_offset;   /* byte offsets inside the workspace */
  int64_t item_ptr_offset;
  int64_t partial_offset;
  int64_t workspace_bytes;
} pg_decode_plan_t;

/* PG_KV_HETEROGENEOUS: one unified page table per request whose first
 * old_kv_len[r] / 16 entries index INT8 code pages and the rest FP16 exact
 * pages; old_kv_len is a device array read by every run
 * (pg_decode_run_heterogeneous), so the boundary may move without re-planning.
 * Work items are 48 bytes. */
enum { PG_KV_INT8 = 0, PG_KV_FP16 = 1, PG_KV_HETEROGENEOUS = 2 };

/* Bytes of workspace a plan with these bounds needs: total work items over
 * the batch, and the largest number of work items of one request. */
int64_t pg_decode_workspace_bytes(int32_t batch_size, int32_t num_qo_heads,
                                  int64_t total_items, int64_t max_items_per_request);

/* Split selection: the pages per work item that pg_decode_plan's balanced
 * planner (split_pages <= 0) chooses on num_cus CUs for batch_size requests
 * sharing total_pages pages evenly, with no tail segment.  bytes_per_page is
 * the per-(page, kv head) K+V traffic: 4096 plans INT8 pages, 8192 FP16
 * pages.  Returns 0 (message in pg_last_error) for invalid arguments or a
 * batch the planner cannot cut.  Replaces FlashInfer's automatic split
 * (fixed_split_size=None) and the capacity bound (2*num_SMs)//Hkv of
 * diagnostics/benchmark_sustained_dynamic_graphs.py:1497-1534. */
int32_t pg_select_split_pages(int64_t total_pages, int32_t batch_size, int32_t num_kv_heads,
                              int32_t bytes_per_page, int32_t num_cus);

/* Plan a decode.  host_indptr [B+1] / host_last_page_len [B]: segment 0
 * (INT8 codes or FP16 pages, primary_kind); host_tail_indptr/_last_len: the
 * optional FP16 tail segment (NULL if none).  split_pages > 0 cuts each
 * request's segment 0 of n pages into ceil(n / split_pages) nearly equal
 * items (the item count of FlashInfer's fixed_split_size, balanced sizes);
 * the tail likewise with tail_split_pages, default ceil(split_pages/2) for
 * INT8 (an FP16 page streams twice the bytes);
 * split_pages <= 0 balances the batch over num_cus workgroups (every item at
 * most 64 pages, FP16 pages weighted twice INT8 pages).
 * exact_tail_pages_hint (heterogeneous plans only, else 0): the number of
 * trailing pages of each request's unified table expected to be FP16 exact
 * pages at run time; they are planned like a tail segment (own items,
 * weighted as FP16 pages).  It only balances the work: the kernel reads
 * old_kv_len at run time, so any boundary is handled correctly.  (A builder
 * addition: the reference's heterogeneous plan has no such argument.)
 * Writes the work list into the device workspace (synchronous copy on
 * ``stream``).  Replaces BatchDecodeWithPagedKVCacheWrapper.plan as called by
 * scripts/benchmark_flashinfer_page_affine_int8.py:363-389. */
int32_t pg_decode_plan(const int32_t* host_indptr, const int32_t* host_last_page_len,
                       int32_t batch_size, int32_t primary_kind,
                       const int32_t* host_tail_indptr, const int32_t* host_tail_last_len,
                       int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                       int32_t page_size, int32_t split_pages, int32_t tail_split_pages,
                       int32_t exact_tail_pages_hint, int32_t num_cus, void* workspace,
                       int64_t workspace_bytes, pg_decode_plan_t* plan, void* stream);

/* The host half of pg_decode_plan (same arguments, same validation and
 * errors) without a device: fills *plan and, if items_out != NULL, the work
 * list as 12 int32 per item (items_capacity counts items, so items_out holds
 * 12 * items_capacity int32) {request, kind (PG_KV_*), segment (0 primary,
 * 1 tail), page_begin, page_end (positions in indices/tail_indices), last
 * position of the segment, item index inside its request, items of the
 * request, position of the request's first page in the segment, the
 * planner's weight per page of the item (2 for FP16 pages planned beside
 * INT8 pages: a tail, or a heterogeneous table's hinted exact pages; else
 * 1), 2 reserved}; item_ptr_out (if != NULL) receives [B+1] offsets of each
 * request's items.  Call once with items_out NULL to learn plan->num_items.  For inspection and tests of
 * the scheduler; no reference counterpart (FlashInfer's plan info is opaque). */
int32_t pg_decode_plan_host(const int32_t* host_indptr, const int32_t* host_last_page_len,
                            int32_t batch_size, int32_t primary_kind,
                            const int32_t* host_tail_indptr, const int32_t* host_tail_last_len,
                            int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
                            int32_t page_size, int32_t split_pages, int32_t tail_split_pages,
                            int32_t exact_tail_pages_hint, int32_t num_cus,
                            pg_decode_plan_t* plan, int32_t* items_out, int64_t items_capacity,
                            int32_t* item_ptr_out);

/* Run a planned decode.  Segment 0: pages ``indices`` (indptr/last_page_len
 * as planned; last_page_len is re-read on the device every call, so a
 * caller may advance it without re-planning) of k_cache/v_cache, which are
 * INT8 codes with k_scale/v_scale [N,Hkv] for PG_KV_INT8 or FP16 pages
 * (scales NULL) for PG_KV_FP16.  Tail segment (if planned): FP16 centered
 * ring pages tail_k/tail_v through tail_indices.  value_center (may be NULL)
 * is added once after normalisation, repeated over the GQA group.  Writes
 * out fp16 [B,Hq,128] and, if lse != NULL, base-2 lse [B,Hq].
 * Replaces the patched FlashInfer run (int8 patch, prefill.cuh), FlashInfer's
 * split merge, the tail decode, merge_state_in_place and add_(output_center)
 * of scripts/benchmark_flashinfer_page_affine_int8.py:566-602.  GQA group
 * size must be 4 and head_dim 128.  Unused rows of an FP16 last page may hold
 * anything (NaN included): they never reach the output. */
int32_t pg_decode_run(const pg_decode_plan_t* plan, const void* query,
                      int64_t query_batch_stride, const void* k_cache, const void* v_cache,
                      const void* k_scale, const void* v_scale, const int32_t* indices,
                      const int32_t* last_page_len, const void* tail_k, const void* tail_v,
                      const int32_t* tail_indices, const int32_t* tail_last_len,
                      const void* value_center, int64_t center_batch_stride, void* out,
                      float* lse, float sm_scale, void* workspace, void* stream);

/* Run a PG_KV_HETEROGENEOUS plan: replaces the heterogeneous one-launch run
 * (scripts/page_gauge_heterogeneous_fa2.py:336-381, kernel
 * patches/flashinfer-0.6.17-page-gauge-heterogeneous.patch).  Entry j of
 * request r's table (indices[indptr[r] + j]) indexes k_codes/v_codes (with
 * k_scale/v_scale) when j < old_kv_len[r] / 16 and exact_k/exact_v (FP16
 * centered pages) otherwise; old_kv_len (device int32 [B], page aligned) and
 * last_page_len are read at run time.  value_center [B,Hkv,128] (stride
 * center_batch_stride) is added once.  Same partial + combine launches and
 * outputs as pg_decode_run. */
int32_t pg_decode_run_heterogeneous(const pg_decode_plan_t* plan, const void* query,
                                    int64_t query_batch_stride, const void* k_codes,
                                    const void* v_codes, const void* k_scale, const void* v_scale,
                                    const void* exact_k, const void* exact_v,
                                    const int32_t* indices, const int32_t* last_page_len,
                                    const int32_t* old_kv_len, const void* value_center,
                                    int64_t center_batch_stride, void* out, float* lse,
                                    float sm_scale, void* workspace, void* stream);

/* pg_decode_run / pg_decode_run_heterogeneous plus the completed-page
 * finalize of the decode step's cache update.  No reference counterpart as
 * one call: the finalize of rope_append_page_gauge(_dynamic)
 * (tests/page_gauge_append_extension.cu:327-382), moved into the FP16 pass
 * over the exact pages for callers whose cache update ran without it
 * (pg_decoder_qkv_rope_append).  When the token at positions[r *
 * position_stride] completed its page (position % 16 == 15, and that page is
 * the last page of r's FP16 segment), the wave that attends to the page
 * writes its INT8 codes and scales into code page r * code_pages_per_request
 * + position / 16 of k_cache/v_cache and k_scale/v_scale: the same codes and
 * scales as that finalize.  Attention outputs are those of the run without
 * it. */
int32_t pg_decode_run_finalize(const pg_decode_plan_t* plan, const void* query,
                               int64_t query_batch_stride, const void* k_cache,
                               const void* v_cache, const void* k_scale, const void* v_scale,
                               const int32_t* indices, const int32_t* last_page_len,
                               const void* tail_k, const void* tail_v,
                               const int32_t* tail_indices, const int32_t* tail_last_len,
                               const void* value_center, int64_t center_batch_stride, void* out,
                               float* lse, float sm_scale, void* workspace,
                               const int32_t* positions, int32_t position_stride,
                               int32_t code_pages_per_request, void* stream);
int32_t pg_decode_run_heterogeneous_finalize(
    const pg_decode_plan_t* plan, const void* query, int64_t query_batch_stride,
    const void* k_codes, const void* v_codes, const void* k_scale, const void* v_scale,
    const void* exact_k, const void* exact_v, const int32_t* indices,
    const int32_t* last_page_len, const int32_t* old_kv_len, const void* value_center,
    int64_t center_batch_stride, void* out, float* lse, float sm_scale, void* workspace,
    const int32_t* positions, int32_t position_stride, int32_t code_pages_per_request,
    void* stream);

/* The two launches of pg_decode_run, for callers that schedule them
 * separately (e.g. to time the partial kernel, or to overlap the combine
 * with other work): pg_decode_run_partial writes one unnormalised partial
 * (o[128], m, l) per work item and query head into the workspace;
 * pg_decode_run_combine merges each request's partials (base-2 LSE merge),
 * normalises, adds value_center and writes out/lse.  Together they are
 * exactly pg_decode_run.  These replace FlashInfer's split-KV decode kernel
 * and its VariableLengthMergeStates merge (plan fields merge_indptr /
 * block_valid_mask, scripts/benchmark_page_gauge_transformer.py:1401-1416). */
int32_t pg_decode_run_partial(const pg_decode_plan_t* plan, const void* query,
                              int64_t query_batch_stride, const void* k_cache,
                              const void* v_cache, const void* k_scale, const void* v_scale,
                              const int32_t* indices, const int32_t* last_page_len,
                              const void* tail_k, const void* tail_v, const int32_t* tail_indices,
                              const int32_t* tail_last_len, float sm_scale, void* workspace,
                              void* stream);
/* pg_decode_run with kernel timing: start_event / stop_event (hipEvent_t
 * created with timing enabled) receive the begin timestamp of the partial
 * kernel's dispatch and the end timestamp of the combine kernel's
 * (hipExtLaunchKernelGGL), i.e. the GPU time of the call without the launch
 * gap before it.  For benchmarks; no reference counterpart. */
int32_t pg_decode_run_timed(const pg_decode_plan_t* plan, const void* query,
                            int64_t query_batch_stride, const void* k_cache, const void* v_cache,
                            const void* k_scale, const void* v_scale, const int32_t* indices,
                            const int32_t* last_page_len, const void* tail_k, const void* tail_v,
                            const int32_t* tail_indices, const int32_t* tail_last_len,
                            const void* value_center, int64_t center_batch_stride, void* out,
                            float* lse, float sm_scale, void* workspace, void* stream,
                            void* start_event, void* stop_event);

/* pg_decode_run_partial with kernel timing: start_event / stop_event
 * (hipEvent_t created with timing enabled, either may be NULL) receive the
 * partial kernel's own dispatch begin/end timestamps (hipExtLaunchKernelGGL),
 * so hipEventElapsedTime gives the kernel duration without the launch gap
 * that events recorded around the call include.  For benchmarks; no
 * reference counterpart. */
int32_t pg_decode_run_partial_timed(const pg_decode_plan_t* plan, const void* query,
                                    int64_t query_batch_stride, const void* k_cache,
                                    const void* v_cache, const void* k_scale, const void* v_scale,
                                    const int32_t* indices, const int32_t* last_page_len,
                                    const void* tail_k, const void* tail_v,
                                    const int32_t* tail_indices, const int32_t* tail_last_len,
                                    float sm_scale, void* workspace, void* stream,
                                    void* start_event, void* stop_event);
int32_t pg_decode_run_combine(const pg_decode_plan_t* plan, const void* value_center,
                              int64_t center_batch_stride, void* out, float* lse,
                              void* workspace, void* stream);

/* Base-2 LSE state merge in place: v, s <- merge((v, s), (v_other, s_other)).
 * Replaces flashinfer.merge_state_in_place as used by
 * scripts/benchmark_flashinfer_page_affine_int8.py:598-600.  v [rows, heads,
 * head_dim] fp16 contiguous, s [rows, heads] float32; mask (uint8 [rows] or
 * NULL): rows with mask 0 are left unchanged. */
int32_t pg_merge_state_in_place(void* v, float* s, const void* v_other, const float* s_other,
                                const uint8_t* mask, int32_t rows, int32_t heads,
                                int32_t head_dim, void* stream);

/* Fused exact-tail attention + state merge + value-center restore.  Replaces
 * exact_tail_merge_center (tests/page_gauge_append_extension.cu:950-1028).
 * query [B,Hq,128] contiguous; tail of request r = (n-1)*16 +
 * exact_last_page_len[r] tokens through exact_page_indices[r*n .. r*n+n-1]
 * (1 <= n <= 16); old_output/old_lse updated in place. */
int32_t pg_exact_tail_merge_center(const void* query, const void* exact_key_pages,
                                   const void* exact_value_pages,
                                   const int32_t* exact_page_indices,
                                   const int32_t* exact_last_page_len, void* old_output,
                                   float* old_lse, const void* value_center,
                                   int64_t center_batch_stride, int32_t batch_size,
                                   int32_t query_heads, int32_t kv_heads,
                                   int32_t pages_per_request, float sm_scale, void* stream);

/* ------------------------------------------------------------------------
 * Decoder step (the caller of the path): fused projections.
 * ------------------------------------------------------------------------ */

/* out = epilogue(W @ prologue(x)) for a decode batch of 1-4 rows.
 * Replaces the F.linear calls of the decoder layer and the element-wise work
 * around them (scripts/benchmark_page_gauge_transformer.py:2754-2805:
 * MistralRMSNorm before the QKV and gate/up projections, SiLU(gate)*up after
 * the gate/up projection, the two residual adds, the final norm + LM head).
 *   weight [n, k] fp16 row-major, k a multiple of 512;
 *   x [batch, x_stride] fp16 (x_stride a multiple of 8); with norm_weight [k]
 *     the input is fp16(w * fp16(x * rsqrt(mean(x^2) + eps)));
 *   swiglu != 0: n is even, rows [0, n/2) are the gate and [n/2, n) the up
 *     projection, and out[i] = fp16(fp16(silu(y[i])) * y[i + n/2]) for
 *     i < n/2 (out has n/2 columns);
 *   residual [batch, residual_stride] fp16 or NULL (may alias out): the
 *     projection is rounded to fp16 first, then added in fp16;
 *   out [batch, out_stride] fp16, or float32 when out_f32 != 0 (the fp16
 *     result widened, as `linear(...).float()`).
 * k = 4096 and k = 14336 run the blocked kernel (weights prefetched before
 * the input prologue); other k stage the input in LDS (batch * k <= 32768).
 * Float32 accumulation with v_dot2_f32_f16; every weight byte is read once. */
int32_t pg_decoder_gemv(const void* weight, int32_t n, int32_t k, const void* x,
                        int64_t x_stride, int32_t batch, const void* norm_weight, float eps,
                        int32_t swiglu, const void* residual, int64_t residual_stride, void* out,
                        int64_t out_stride, int32_t out_f32, void* stream);

/* The QKV projection of a decode step fused with its cache update: the
 * decoder layer's qkv F.linear (with the input RMSNorm, as pg_decoder_gemv)
 * followed by rope_append_page_gauge_dynamic / rope_append_fp16_dynamic
 * (tests/page_gauge_append_extension.cu:244-383, :686-948) without the page
 * finalize, which pg_decode_run_finalize performs.  weight [(Hq + 2 Hkv)*128,
 * 4096] (query rows, key rows, value rows); for batch row b at position p =
 * positions[b * position_stride]:
 *   rotated_query[b, h] = RoPE(q) with the cosine/sine rows p, each element
 *     rn16(rn16(x*c) + rn16(partner*s)) from the fp16-rounded projection;
 *   key_center != NULL (PageGauge): the rotated key and the value, centered
 *     as fp16(f32(x) - f32(center)), go to token p % 16 of exact page
 *     b * pages_per_request + (page < sink_pages ? page : sink_pages + page %
 *     (pages_per_request - sink_pages)), page = p / 16;
 *   key_center == NULL: rotated key and value go to token p % 16 of page
 *     b * pages_per_request + p / 16 of key_pages/value_pages;
 * a position outside [0, capacity_tokens) or the RoPE table writes nothing.
 * Bit-identical to the projection followed by the cache-update launch. */
int32_t pg_decoder_qkv_rope_append(const void* weight, int32_t k, const void* x,
                                   int64_t x_stride, int32_t batch, const void* norm_weight,
                                   float eps, int32_t query_heads, int32_t kv_heads,
                                   const void* cosine, const void* sine, int64_t rope_row_stride,
                                   int32_t rope_rows, const int32_t* positions,
                                   int32_t position_stride, void* rotated_query, void* key_pages,
                                   void* value_pages, const void* key_center,
                                   const void* value_center, int64_t center_batch_stride,
                                   int32_t pages_per_request, int32_t sink_pages,
                                   int32_t capacity_tokens, void* stream);

/* Greedy token selection of the decode loop: out[r] = argmax of row r of
 * x [rows, row_stride] float32 over its first n elements, as
 * logits.argmax(dim=-1) in the reference decoder (the step's "gpu_argmax",
 * scripts/benchmark_page_gauge_transformer.py:2602 and :2650; the top-1
 * comparison at :3880; scripts/probe_certified_hierarchical_attention.py:249):
 * the first index of the maximum, NaN counting as the largest value.  One
 * workgroup per row. */
int32_t pg_argmax_f32(const float* x, int32_t rows, int32_t n, int64_t row_stride, int64_t* out,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PAGEGAUGE_HIP_H */
