// Decode work items and the split planner: host C++ shared with the decode
// kernels (pg_decode.hip), free of HIP so that the planner also builds, and
// is fuzzed under the sanitizers, with a host compiler.
#pragma once

#include <stdint.h>

#include <vector>

#include "pg_host.h"

namespace pg {

#ifndef PG_MAX_WAVES_PER_BLOCK
#define PG_MAX_WAVES_PER_BLOCK 8
#endif
constexpr int kMaxWavesPerBlock = PG_MAX_WAVES_PER_BLOCK;   // KV heads (waves) per workgroup
constexpr int kMaxItemsPerRequest = 4096;
constexpr int kMaxChunkPages = 64;      // pages per work item (one wave lane per page)
constexpr int kMinChunkPages = 4;       // balanced plans keep at least one PV group per item
#ifndef PG_LARGE_BATCH_MIN_CHUNK
#define PG_LARGE_BATCH_MIN_CHUNK 16.0
#endif
constexpr double kLargeBatchMinChunk = PG_LARGE_BATCH_MIN_CHUNK;  // weighted pages
// Upper end of the medium regime (weighted pages per CU).  Up to 30, 7/16 of
// the CUs in items of at most 64 pages (at most 120 items, 240 half-height
// workgroups) still cover the batch in one wave of workgroups.
#ifndef PG_MEDIUM_MAX_PAGES_PER_CU
#define PG_MEDIUM_MAX_PAGES_PER_CU 30.0
#endif
constexpr double kMediumMaxPagesPerCu = PG_MEDIUM_MAX_PAGES_PER_CU;

// KV heads (waves) per workgroup when a plan has more items than CUs.
#ifndef PG_MULTI_ROUND_WAVES
#define PG_MULTI_ROUND_WAVES 4
#endif
constexpr int kMultiRoundWaves = PG_MULTI_ROUND_WAVES;

struct WorkItem {
  int32_t request;
  int32_t kind;        // PG_KV_INT8, PG_KV_FP16 or PG_KV_HETEROGENEOUS
  int32_t segment;     // 0 primary, 1 tail
  int32_t page_begin;  // absolute index into the segment's page-index array
  int32_t page_end;    // exclusive
  int32_t last_page;   // absolute index of the segment's final page for the request
  int32_t item_in_request;  // position of this item among its request's items
  int32_t items_in_request; // number of items of the request
  int32_t request_page_begin;  // absolute index of the request's first page in the segment
  int32_t page_weight;  // the planner's weight per page: 2 for FP16 pages planned beside INT8 ones
  int32_t reserved[2];
};
static_assert(sizeof(WorkItem) == 48, "work item layout");

// Work item ``i`` of a one-request plan: the FP16 tail segment's items
// first, then the primary segment's; segment pages [base, base + n) in c
// nearly equal chunks (the first n % c one page longer), as the planner
// cuts them.  constexpr, so the partial kernel calls it as well.
constexpr WorkItem closed_form_item(int i, int items, int tail_items, int tail_begin,
                                    int tail_pages, int primary_begin, int primary_pages,
                                    int primary_kind) {
  const bool tail = i < tail_items;
  const int n = tail ? tail_pages : primary_pages;
  const int c = tail ? tail_items : items - tail_items;
  const int k = tail ? i : i - tail_items;
  const int base = tail ? tail_begin : primary_begin;
  const int q = n / c;
  const int r = n % c;
  WorkItem it{};
  it.request = 0;
  it.kind = tail ? PG_KV_FP16 : primary_kind;
  it.segment = tail ? 1 : 0;
  it.page_begin = base + k * q + (k < r ? k : r);
  it.page_end = it.page_begin + q + (k < r ? 1 : 0);
  it.last_page = base + n - 1;
  it.item_in_request = i;
  it.items_in_request = items;
  it.request_page_begin = base;
  it.page_weight = tail && primary_kind == PG_KV_INT8 ? 2 : 1;
  return it;
}

// KV heads (waves) per workgroup of the partial kernel for ``items`` work
// items on ``num_cus`` CUs.
int waves_per_block_for(int hkv, int64_t items, int64_t num_cus);

// Host half of the planner: validates the batch and cuts it into work items
// (``items``, ``item_ptr`` [B+1]).  Fills ``p``; the caller checks the
// workspace size and copies the work list to the device.
int32_t build_plan(const int32_t* host_indptr, const int32_t* host_last_page_len,
                   int32_t batch_size, int32_t primary_kind, const int32_t* host_tail_indptr,
                   const int32_t* host_tail_last_len, int32_t num_qo_heads, int32_t num_kv_heads,
                   int32_t head_dim, int32_t page_size, int32_t split_pages,
                   int32_t tail_split_pages, int32_t exact_tail_pages_hint, int32_t num_cus,
                   std::vector<WorkItem>& items, std::vector<int32_t>& item_ptr,
                   pg_decode_plan_t& p);

// Device dispatch order of a plan's items: with more items than CUs
// (several rounds of workgroups), the heaviest items first, by the weight
// the planner gave them (pages x page_weight: FP16 pages, the tail's or a
// heterogeneous table's hinted exact pages, weigh twice INT8 pages), so that
// the last round holds the lightest ones.  Stable; an item's partial row
// comes from its request and item_in_request, not from its position, so any
// order gives the same results.  The host-visible work list stays in request
// order.
void order_for_dispatch(std::vector<WorkItem>& items, int32_t num_cus);

}  // namespace pg
