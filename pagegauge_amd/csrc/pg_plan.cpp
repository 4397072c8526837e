// The decode split planner (host only): validation, the balanced and fixed
// splits, the closed-form description and the workspace layout.  The device
// copy of the work list is pg_decode_plan in pg_decode.hip.
#include "pg_plan.h"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

namespace pg {
namespace {

int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

}  // namespace

// KV heads (waves) per workgroup.  All of a page's heads in one workgroup
// keep its 16 KiB of codes on one CU (the best layout once the items fill
// most CUs); with fewer items the heads are split over several workgroups
// so that every CU gets work (a 4K-token request: 64 items in two-wave
// workgroups).
int waves_per_block_for(int hkv, int64_t items, int64_t num_cus) {
  int w = kMaxWavesPerBlock;
  while (w > 1 && hkv % w) w >>= 1;
  if (items > num_cus) {
    // More items than CUs: the items run in rounds, and at two waves per
    // SIMD (the partial kernel's registers) one 8-wave workgroup fills a CU,
    // so each item's start-up and drain leave its CU idle.  Narrower
    // workgroups put two items on each CU that overlap each other's
    // start-up (faster on every multi-round batch timed, B16 x 16K to 256
    // ragged requests); with at most one item per CU the width made no
    // difference (B8 ragged, B1 128K).
    while (w > kMultiRoundWaves && hkv % (w >> 1) == 0) w >>= 1;
    return w;
  }
  if (items * 10 >= num_cus * 7) return w;
  while (w > 2 && items * (hkv / w) < num_cus && hkv % (w >> 1) == 0) w >>= 1;
  return w;
}

void order_for_dispatch(std::vector<WorkItem>& items, int32_t num_cus) {
  const int64_t cus = num_cus > 0 ? num_cus : 256;
  if (static_cast<int64_t>(items.size()) <= cus) return;
  auto weight = [](const WorkItem& it) { return (it.page_end - it.page_begin) * it.page_weight; };
  std::stable_sort(items.begin(), items.end(), [&](const WorkItem& a, const WorkItem& b) {
    return weight(a) > weight(b);
  });
}

}  // namespace pg

using namespace pg;

extern "C" int64_t pg_decode_workspace_bytes(int32_t batch_size, int32_t num_qo_heads,
                                             int64_t total_items, int64_t max_items_per_request) {
  if (batch_size <= 0 || num_qo_heads <= 0 || total_items <= 0 || max_items_per_request <= 0)
    return 0;
  int64_t bytes = align_up(total_items * static_cast<int64_t>(sizeof(WorkItem)), 256);
  bytes += align_up((batch_size + 1) * static_cast<int64_t>(sizeof(int32_t)), 256);
  bytes += align_up(static_cast<int64_t>(batch_size) * num_qo_heads * max_items_per_request *
                        (kHeadDim + 2) * 4, 256);
  return bytes;
}

extern "C" int32_t pg_select_split_pages(int64_t total_pages, int32_t batch_size,
                                         int32_t num_kv_heads, int32_t bytes_per_page,
                                         int32_t num_cus) {
  // The balanced planner's pages per work item for ``batch_size`` requests
  // sharing ``total_pages`` pages evenly (INT8 pages for 4096 bytes per
  // (page, KV head) of K+V, FP16 pages for 8192), no tail segment.
  clear_error();
  if (total_pages <= 0 || batch_size <= 0 || num_kv_heads <= 0) {
    fail(PG_ERROR_INVALID_ARGUMENT, "pages, batch size and KV heads must be positive");
    return 0;
  }
  if (bytes_per_page != 4096 && bytes_per_page != 8192) {
    fail(PG_ERROR_INVALID_ARGUMENT, "bytes_per_page must be 4096 (INT8) or 8192 (FP16)");
    return 0;
  }
  if (total_pages > INT32_MAX) {
    fail(PG_ERROR_UNSUPPORTED, "total_pages must fit in int32");
    return 0;
  }
  pg_decode_plan_t p{};
  const int32_t rc = guarded([&]() -> int32_t {
    std::vector<int32_t> indptr(static_cast<size_t>(batch_size) + 1);
    const int64_t per = total_pages / batch_size, extra = total_pages % batch_size;
    indptr[0] = 0;
    for (int32_t b = 0; b < batch_size; ++b)
      indptr[b + 1] = static_cast<int32_t>(indptr[b] + per + (b < extra ? 1 : 0));
    const std::vector<int32_t> last(static_cast<size_t>(batch_size), kPageSize);
    std::vector<WorkItem> items;
    std::vector<int32_t> item_ptr;
    return build_plan(indptr.data(), last.data(), batch_size,
                      bytes_per_page == 4096 ? PG_KV_INT8 : PG_KV_FP16, nullptr, nullptr,
                      kGqa * num_kv_heads, num_kv_heads, kHeadDim, kPageSize, 0, 0, 0, num_cus,
                      items, item_ptr, p);
  });
  return rc == PG_OK ? p.split_pages : 0;
}

namespace pg {

int32_t build_plan(const int32_t* host_indptr, const int32_t* host_last_page_len,
                   int32_t batch_size, int32_t primary_kind, const int32_t* host_tail_indptr,
                   const int32_t* host_tail_last_len, int32_t num_qo_heads, int32_t num_kv_heads,
                   int32_t head_dim, int32_t page_size, int32_t split_pages,
                   int32_t tail_split_pages, int32_t exact_tail_pages_hint, int32_t num_cus,
                   std::vector<WorkItem>& items, std::vector<int32_t>& item_ptr,
                   pg_decode_plan_t& p) {
  if (!host_indptr || !host_last_page_len)
    return fail(PG_ERROR_INVALID_ARGUMENT, "null plan argument");
  if (batch_size <= 0) return fail(PG_ERROR_INVALID_ARGUMENT, "batch size must be positive");
  if (head_dim != kHeadDim) return fail(PG_ERROR_UNSUPPORTED, "head dimension must be 128");
  if (page_size != kPageSize) return fail(PG_ERROR_UNSUPPORTED, "page size must be 16");
  if (num_kv_heads <= 0 || num_qo_heads != kGqa * num_kv_heads)
    return fail(PG_ERROR_UNSUPPORTED, "the decode kernel requires GQA group size 4");
  if (num_kv_heads > 64) return fail(PG_ERROR_UNSUPPORTED, "at most 64 KV heads");
  if (primary_kind != PG_KV_INT8 && primary_kind != PG_KV_FP16 &&
      primary_kind != PG_KV_HETEROGENEOUS)
    return fail(PG_ERROR_INVALID_ARGUMENT, "kv kind must be INT8, FP16 or heterogeneous");
  if (primary_kind == PG_KV_HETEROGENEOUS && host_tail_indptr != nullptr)
    return fail(PG_ERROR_INVALID_ARGUMENT, "a heterogeneous plan has one unified page table");
  if ((host_tail_indptr == nullptr) != (host_tail_last_len == nullptr))
    return fail(PG_ERROR_INVALID_ARGUMENT, "tail indptr and last_page_len go together");
  if (exact_tail_pages_hint < 0)
    return fail(PG_ERROR_INVALID_ARGUMENT, "exact_tail_pages_hint must be non-negative");
  if (exact_tail_pages_hint > 0 && primary_kind != PG_KV_HETEROGENEOUS)
    return fail(PG_ERROR_INVALID_ARGUMENT, "exact_tail_pages_hint applies to heterogeneous plans");
  // work items address indices[indptr[0] ..]: a negative start would read
  // before the page table
  if (host_indptr[0] < 0) return fail(PG_ERROR_INVALID_ARGUMENT, "indptr[0] must be non-negative");
  if (host_tail_indptr && host_tail_indptr[0] < 0)
    return fail(PG_ERROR_INVALID_ARGUMENT, "tail indptr[0] must be non-negative");

  for (int b = 0; b < batch_size; ++b) {
    const int64_t n = static_cast<int64_t>(host_indptr[b + 1]) - host_indptr[b];
    if (n < 0) return fail(PG_ERROR_INVALID_ARGUMENT, "indptr must be non-decreasing");
    if (n > 0 && (host_last_page_len[b] < 1 || host_last_page_len[b] > kPageSize))
      return fail(PG_ERROR_INVALID_ARGUMENT, "last_page_len must lie in [1, 16]");
    if (host_tail_indptr) {
      const int64_t tn = static_cast<int64_t>(host_tail_indptr[b + 1]) - host_tail_indptr[b];
      if (tn < 0) return fail(PG_ERROR_INVALID_ARGUMENT, "tail indptr must be non-decreasing");
      if (tn > 0 && (host_tail_last_len[b] < 1 || host_tail_last_len[b] > kPageSize))
        return fail(PG_ERROR_INVALID_ARGUMENT, "tail last_page_len must lie in [1, 16]");
    }
  }
  // Segments of the batch; FP16 pages stream twice the bytes of INT8 pages.
  // ``first`` / ``last``: the request's first and last page in the segment's
  // page table (a heterogeneous table split by the hint keeps both).
  struct Segment {
    int request, kind, seg, begin, end;
    double weight;
    int first, last;
  };
  std::vector<Segment> segments;
  for (int b = 0; b < batch_size; ++b) {
    if (host_tail_indptr && host_tail_indptr[b + 1] > host_tail_indptr[b])
      segments.push_back({b, PG_KV_FP16, 1, host_tail_indptr[b], host_tail_indptr[b + 1],
                          primary_kind == PG_KV_INT8 ? 2.0 : 1.0, host_tail_indptr[b],
                          host_tail_indptr[b + 1] - 1});
    const int begin = host_indptr[b], end = host_indptr[b + 1];
    if (end <= begin) continue;
    // heterogeneous table: its last exact_tail_pages_hint pages are expected
    // to be FP16 exact pages at run time; they are planned as FP16 pages (own
    // items, first, twice the weight).  Balance only: the kernel reads
    // old_kv_len at run time, so any boundary is handled correctly.
    const int exact = std::min(exact_tail_pages_hint, end - begin);
    if (exact > 0)
      segments.push_back({b, primary_kind, 0, end - exact, end, 2.0, begin, end - 1});
    if (end - exact > begin)
      segments.push_back({b, primary_kind, 0, begin, end - exact, 1.0, begin, end - 1});
  }
  std::vector<int> chunks(segments.size(), 0);
  bool medium = false;
  if (split_pages > 0) {
    // fixed split (FlashInfer fixed_split_size semantics): pages per work item
    if (tail_split_pages <= 0)
      tail_split_pages = primary_kind == PG_KV_INT8 ? std::max(1, (split_pages + 1) / 2) : split_pages;
    for (size_t i = 0; i < segments.size(); ++i) {
      const int n = segments[i].end - segments[i].begin;
      const int size = std::min(segments[i].seg == 0 ? split_pages : tail_split_pages, kMaxChunkPages);
      chunks[i] = (n + size - 1) / size;
    }
  } else {
    // Balanced plan: the smallest per-item load ``cap`` (weighted pages) for
    // which the whole batch fits in one workgroup per CU; every segment is
    // cut into nearly equal chunks of at most kMaxChunkPages pages.
    const int64_t target = std::max<int64_t>(num_cus > 0 ? num_cus : 256, 1);
    const int64_t min_chunk = kMinChunkPages;
    auto count_for = [&](double cap, std::vector<int>* out) {
      int64_t total = 0;
      for (size_t i = 0; i < segments.size(); ++i) {
        const int n = segments[i].end - segments[i].begin;
        const int64_t by_cap = static_cast<int64_t>(std::ceil(n * segments[i].weight / cap - 1e-9));
        const int64_t by_size = (n + kMaxChunkPages - 1) / kMaxChunkPages;
        const int64_t most = std::max<int64_t>(1, n / min_chunk);
        const int64_t c = std::max<int64_t>({1, by_size, std::min(by_cap, most)});
        if (out) (*out)[i] = static_cast<int>(c);
        total += c;
      }
      return total;
    };
    double lo = 1e-3, hi = 1.0;
    for (const Segment& sg : segments) hi += (sg.end - sg.begin) * sg.weight;
    // Measured on MI355X (B=1 sweeps from 4K to 160K tokens, B=4 and B=8):
    // * large (>= 30 pages per CU): 16-page chunks beat finer ones, because
    //   each work item pays a fixed start-up (page ids, then the first
    //   group), on up to one 8-wave workgroup per CU;
    // * medium (3..30 pages per CU): about 7/16 of the CUs in items, each
    //   split over two half-height workgroups (one wave per SIMD), so every
    //   wave pipelines 2..16 groups (16K: 12.6 against 13.9 us; 64K: 29.2
    //   against 31.3 us; 112K: 45.1 against 47.8 us); past 30 the 64-page
    //   item cap needs more than 128 items, a second wave of workgroups;
    // * small: chunks down to one PV group for parallelism.
    const double per_cu = hi / static_cast<double>(target);
    medium = per_cu >= 3.0 && per_cu < kMediumMaxPagesPerCu;
    const int64_t item_target = medium ? std::max<int64_t>(1, target * 7 / 16) : target;
    lo = per_cu >= kMediumMaxPagesPerCu ? kLargeBatchMinChunk : 1e-3;
    if (count_for(hi, nullptr) <= item_target) {
      for (int iter = 0; iter < 64; ++iter) {
        const double mid = 0.5 * (lo + hi);
        if (count_for(mid, nullptr) <= item_target) hi = mid; else lo = mid;
      }
    }
    count_for(hi, &chunks);
  }

  items.clear();
  item_ptr.assign(batch_size + 1, 0);
  int max_per_request = 0;
  split_pages = 0;
  tail_split_pages = 0;
  size_t next = 0;
  for (int b = 0; b < batch_size; ++b) {
    // A request's items are contiguous; its FP16 tail items come first so
    // they start in the first wave of workgroups beside the INT8 chunks.
    item_ptr[b] = static_cast<int32_t>(items.size());
    for (; next < segments.size() && segments[next].request == b; ++next) {
      const Segment& sg = segments[next];
      const int n = sg.end - sg.begin;
      const int c = chunks[next];
      int start = sg.begin;
      for (int k = 0; k < c; ++k) {
        const int size = n / c + (k < n % c ? 1 : 0);
        items.push_back(WorkItem{b, sg.kind, sg.seg, start, start + size, sg.last,
                                 static_cast<int32_t>(items.size()) - item_ptr[b], 0, sg.first,
                                 static_cast<int32_t>(sg.weight), {0, 0}});
        start += size;
        if (sg.seg == 0) split_pages = std::max(split_pages, size);
        else tail_split_pages = std::max(tail_split_pages, size);
      }
    }
    const int in_request = static_cast<int>(items.size()) - item_ptr[b];
    for (size_t k = item_ptr[b]; k < items.size(); ++k) items[k].items_in_request = in_request;
    max_per_request = std::max(max_per_request, in_request);
  }
  item_ptr[batch_size] = static_cast<int32_t>(items.size());
  if (max_per_request > kMaxItemsPerRequest)
    return fail(PG_ERROR_UNSUPPORTED, "too many splits per request; raise split_pages");
  const int64_t n_items = std::max<int64_t>(1, static_cast<int64_t>(items.size()));
  const int64_t needed =
      pg_decode_workspace_bytes(batch_size, num_qo_heads, n_items, std::max(1, max_per_request));

  p = pg_decode_plan_t{};
  p.batch_size = batch_size;
  p.num_qo_heads = num_qo_heads;
  p.num_kv_heads = num_kv_heads;
  p.head_dim = head_dim;
  p.page_size = page_size;
  p.primary_kind = primary_kind;
  p.has_tail = host_tail_indptr != nullptr;
  p.split_pages = split_pages;
  p.tail_split_pages = tail_split_pages;
  p.num_items = static_cast<int32_t>(items.size());
  p.num_items_primary = 0;
  for (const WorkItem& it : items) p.num_items_primary += it.segment == 0;
  p.max_items_per_request = max_per_request;
  p.waves_per_block = waves_per_block_for(num_kv_heads, static_cast<int64_t>(items.size()),
                                          num_cus > 0 ? num_cus : 256);
  if (medium) {
    // two workgroups per item: the largest allowed divisor of Hkv below Hkv
    int w = kMaxWavesPerBlock;
    while (w > 1 && num_kv_heads % w) w >>= 1;
    if (w == num_kv_heads && w > 1) w >>= 1;
    p.waves_per_block = w;
  }
  // One request: describe the items in closed form when the formula gives
  // exactly the table (the kernel then skips the work-item load).
  if (batch_size == 1 && !items.empty()) {
    p.cf_tail_items = static_cast<int32_t>(items.size()) - p.num_items_primary;
    if (host_tail_indptr) {
      p.cf_tail_begin = host_tail_indptr[0];
      p.cf_tail_pages = host_tail_indptr[1] - host_tail_indptr[0];
    }
    p.cf_primary_begin = host_indptr[0];
    p.cf_primary_pages = host_indptr[1] - host_indptr[0];
    bool same = p.num_items_primary > 0 || p.cf_tail_items > 0;
    for (size_t i = 0; same && i < items.size(); ++i) {
      const WorkItem cf = closed_form_item(static_cast<int>(i), p.num_items, p.cf_tail_items,
                                           p.cf_tail_begin, p.cf_tail_pages, p.cf_primary_begin,
                                           p.cf_primary_pages, primary_kind);
      same = std::memcmp(&cf, &items[i], sizeof(WorkItem)) == 0;
    }
    p.closed_form = same ? 1 : 0;
    if (!same) {
      p.cf_tail_items = p.cf_tail_begin = p.cf_tail_pages = 0;
      p.cf_primary_begin = p.cf_primary_pages = 0;
    }
  }
  p.items_offset = 0;
  p.item_ptr_offset = align_up(n_items * static_cast<int64_t>(sizeof(WorkItem)), 256);
  p.partial_offset = p.item_ptr_offset + align_up((batch_size + 1) * 4, 256);
  p.workspace_bytes = needed;
  return PG_OK;
}

}  // namespace pg

extern "C" int32_t pg_decode_plan_host(const int32_t* host_indptr,
                                       const int32_t* host_last_page_len, int32_t batch_size,
                                       int32_t primary_kind, const int32_t* host_tail_indptr,
                                       const int32_t* host_tail_last_len, int32_t num_qo_heads,
                                       int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                       int32_t split_pages, int32_t tail_split_pages,
                                       int32_t exact_tail_pages_hint, int32_t num_cus,
                                       pg_decode_plan_t* plan, int32_t* items_out,
                                       int64_t items_capacity, int32_t* item_ptr_out) {
  clear_error();
  if (!plan) return fail(PG_ERROR_INVALID_ARGUMENT, "null plan argument");
  return guarded([&]() -> int32_t {
    std::vector<WorkItem> items;
    std::vector<int32_t> item_ptr;
    pg_decode_plan_t p{};
    const int32_t rc = build_plan(host_indptr, host_last_page_len, batch_size, primary_kind,
                                  host_tail_indptr, host_tail_last_len, num_qo_heads,
                                  num_kv_heads, head_dim, page_size, split_pages,
                                  tail_split_pages, exact_tail_pages_hint, num_cus, items,
                                  item_ptr, p);
    if (rc != PG_OK) return rc;
    *plan = p;
    if (items_out) {
      if (items_capacity < static_cast<int64_t>(items.size()))
        return fail(PG_ERROR_INVALID_ARGUMENT, "work-item buffer too small: need " +
                                                   std::to_string(items.size()) + " items");
      if (!items.empty()) std::memcpy(items_out, items.data(), items.size() * sizeof(WorkItem));
    }
    if (item_ptr_out)
      std::memcpy(item_ptr_out, item_ptr.data(), item_ptr.size() * sizeof(int32_t));
    return PG_OK;
  });
}
