// Host-side fuzz of the decode planner (pg_decode_plan_host), built with
// AddressSanitizer and UndefinedBehaviorSanitizer by tests/test_planner_sanitized.py.
// Random batches, page tables, kinds, splits, hints and CU counts, plus
// malformed inputs; every accepted plan is checked against the work-item
// contract of include/pagegauge_hip.h:
//   * each request's items are contiguous (item_ptr) and number
//     ``items of the request``, with in-request indices 0..n-1;
//   * per segment, the items tile [indptr[b], indptr[b+1]) in order, each
//     1..64 pages, and name the segment's last position;
//   * a closed-form plan reproduces every item from the formula the kernel
//     uses (tail items first, then the primary segment's);
//   * rejected inputs leave a message in pg_last_error().
// pg_select_split_pages is called on random uniform batches as well.
// Usage: planner_fuzz <seed> <iterations>; prints
// "ok <plans> <rejections> <closed-form plans>".
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "pagegauge_hip.h"
#include "pg_plan.h"

namespace {

int failures = 0;

void check(bool cond, const char* what, int iteration) {
  if (!cond) {
    std::fprintf(stderr, "iteration %d: %s\n", iteration, what);
    if (++failures > 20) std::exit(1);
  }
}

constexpr int kFields = 12;   // int32 per work item (include/pagegauge_hip.h)

struct Item {
  int request, kind, segment, begin, end, last, index, count, request_begin;
};

}  // namespace

int main(int argc, char** argv) {
  const unsigned long seed = argc > 1 ? std::strtoul(argv[1], nullptr, 10) : 1;
  const int iterations = argc > 2 ? std::atoi(argv[2]) : 2000;
  std::mt19937_64 rng(seed);
  auto uniform = [&](int lo, int hi) { return std::uniform_int_distribution<int>(lo, hi)(rng); };
  int plans = 0, rejected = 0, closed = 0;

  for (int iter = 0; iter < iterations; ++iter) {
    const int batch = uniform(1, 12);
    const int kind = uniform(0, 2);                       // PG_KV_INT8, FP16, HETEROGENEOUS
    const bool tail = kind != PG_KV_HETEROGENEOUS && uniform(0, 3) > 0;
    const int max_pages = uniform(0, 3) == 0 ? 4000 : 300;
    std::vector<int32_t> indptr(batch + 1, 0), last(batch), tail_indptr(batch + 1, 0),
        tail_last(batch);
    indptr[0] = uniform(0, 3) == 0 ? uniform(0, 50) : 0;   // tables need not start at 0
    tail_indptr[0] = uniform(0, 3) == 0 ? uniform(0, 50) : 0;
    for (int b = 0; b < batch; ++b) {
      indptr[b + 1] = indptr[b] + (uniform(0, 9) == 0 ? 0 : uniform(1, max_pages));
      last[b] = uniform(1, 16);
      tail_indptr[b + 1] = tail_indptr[b] + (uniform(0, 5) == 0 ? 0 : uniform(1, 16));
      tail_last[b] = uniform(1, 16);
    }
    // malformed inputs, about one call in six
    const int corrupt = uniform(0, 11);
    if (corrupt == 0) last[uniform(0, batch - 1)] = uniform(0, 1) ? 0 : 17;
    if (corrupt == 1) indptr[0] = -uniform(1, 5);
    if (corrupt == 2 && batch > 1) std::swap(indptr[1], indptr[batch]);
    if (corrupt == 3) tail_indptr[0] = -1;
    if (corrupt == 4) tail_last[uniform(0, batch - 1)] = 0;
    const int split = uniform(0, 2) == 0 ? uniform(1, 80) : 0;
    const int tail_split = uniform(0, 3) == 0 ? uniform(1, 20) : 0;
    const int hint = kind == PG_KV_HETEROGENEOUS && uniform(0, 1) ? uniform(1, 20) : 0;
    const int cus = uniform(0, 4) == 0 ? uniform(1, 600) : 256;
    const int hkv = uniform(0, 7) == 0 ? uniform(1, 16) : 8;

    pg_decode_plan_t plan;
    std::memset(&plan, 0, sizeof(plan));
    const int32_t* tp = tail ? tail_indptr.data() : nullptr;
    const int32_t* tl = tail ? tail_last.data() : nullptr;
    int rc = pg_decode_plan_host(indptr.data(), last.data(), batch, kind, tp, tl, 4 * hkv, hkv,
                                 128, 16, split, tail_split, hint, cus, &plan, nullptr, 0, nullptr);
    // the documented rules: tables start at a non-negative offset, never
    // decrease, and a non-empty request's last page holds 1..16 tokens
    bool valid = indptr[0] >= 0 && (!tail || tail_indptr[0] >= 0);
    for (int b = 0; b < batch; ++b) {
      if (indptr[b + 1] < indptr[b]) valid = false;
      if (indptr[b + 1] > indptr[b] && (last[b] < 1 || last[b] > 16)) valid = false;
      if (tail && tail_indptr[b + 1] > tail_indptr[b] && (tail_last[b] < 1 || tail_last[b] > 16))
        valid = false;
    }
    check((rc == 0) == valid, valid ? "a valid table was rejected" : "a malformed table was accepted",
          iter);
    if (rc != 0) {
      ++rejected;
      check(std::strlen(pg_last_error()) > 0, "a rejected plan leaves a message", iter);
      continue;
    }
    const int n_items = plan.num_items;   // 0 when every request is empty
    check(n_items >= 0, "a plan has a non-negative item count", iter);
    std::vector<int32_t> raw(kFields * static_cast<size_t>(n_items) + kFields, -7);
    std::vector<int32_t> item_ptr(batch + 1, -7);
    rc = pg_decode_plan_host(indptr.data(), last.data(), batch, kind, tp, tl, 4 * hkv, hkv, 128,
                             16, split, tail_split, hint, cus, &plan, raw.data(), n_items,
                             item_ptr.data());
    check(rc == 0, "the second plan call succeeds", iter);
    if (rc != 0) continue;
    ++plans;
    check(raw[kFields * n_items] == -7, "no item is written past num_items", iter);
    check(plan.waves_per_block >= 1 && hkv % plan.waves_per_block == 0,
          "waves per block divide the KV heads", iter);
    // (an empty plan still reserves one item and one partial row per head)
    check(plan.workspace_bytes ==
              pg_decode_workspace_bytes(batch, 4 * hkv, std::max(1, n_items),
                                        std::max(1, plan.max_items_per_request)),
          "workspace bytes follow pg_decode_workspace_bytes", iter);
    std::vector<Item> items(n_items);
    for (int i = 0; i < n_items; ++i) {
      const int32_t* r = &raw[kFields * i];
      items[i] = {r[0], r[1], r[2], r[3], r[4], r[5], r[6], r[7], r[8]};
    }
    check(item_ptr[0] == 0 && item_ptr[batch] == n_items, "item_ptr spans the items", iter);
    int most = 0;
    for (int b = 0; b < batch; ++b) {
      const int lo = item_ptr[b], hi = item_ptr[b + 1];
      check(lo <= hi, "item_ptr is non-decreasing", iter);
      most = std::max(most, hi - lo);
      // pages each segment still has to cover, in order
      int next0 = indptr[b], next1 = tail ? tail_indptr[b] : 0;
      for (int i = lo; i < hi; ++i) {
        const Item& it = items[i];
        check(it.request == b, "an item names its request", iter);
        check(it.index == i - lo && it.count == hi - lo, "in-request index and count", iter);
        check(it.end - it.begin >= 1 && it.end - it.begin <= 64, "items hold 1..64 pages", iter);
        check(it.request_begin == (it.segment == 1 ? tail_indptr[b] : indptr[b]),
              "an item names its request's first position", iter);
        if (it.segment == 1) {
          check(tail && it.kind == PG_KV_FP16, "tail items are FP16", iter);
          check(it.begin == next1, "tail items tile the tail table in order", iter);
          check(it.last == tail_indptr[b + 1] - 1, "tail items name the tail's last page", iter);
          next1 = it.end;
        } else {
          check(it.segment == 0 && it.kind == kind, "primary items have the plan's kind", iter);
          check(it.last == indptr[b + 1] - 1, "primary items name the segment's last page", iter);
          if (hint == 0) {   // (a hinted table plans its last pages first: checked below)
            check(it.begin == next0, "primary items tile the table in order", iter);
            next0 = it.end;
          }
        }
      }
      if (hint == 0) check(next0 == indptr[b + 1], "the primary table is covered", iter);
      if (tail) check(next1 == tail_indptr[b + 1], "the tail table is covered", iter);
    }
    check(most == plan.max_items_per_request, "max items per request", iter);
    if (hint > 0) {
      // every page of each table exactly once
      for (int b = 0; b < batch; ++b) {
        std::vector<int> seen(indptr[b + 1] - indptr[b], 0);
        for (int i = item_ptr[b]; i < item_ptr[b + 1]; ++i)
          for (int p = items[i].begin; p < items[i].end; ++p) ++seen[p - indptr[b]];
        for (int s : seen) check(s == 1, "hinted plans cover every page once", iter);
      }
    }
    if (plan.closed_form) {
      ++closed;
      check(batch == 1, "closed form is for one request", iter);
      const int tail_items = plan.cf_tail_items;
      for (int i = 0; i < n_items; ++i) {
        const bool t = i < tail_items;
        const int c = t ? tail_items : n_items - tail_items;
        const int k = t ? i : i - tail_items;
        const int n = t ? plan.cf_tail_pages : plan.cf_primary_pages;
        const int base = t ? plan.cf_tail_begin : plan.cf_primary_begin;
        const int begin = base + k * (n / c) + std::min(k, n % c);
        const int size = n / c + (k < n % c ? 1 : 0);
        check(items[i].begin == begin && items[i].end == begin + size,
              "the closed form reproduces the item", iter);
        check(items[i].segment == (t ? 1 : 0), "closed-form items keep their segment", iter);
      }
    }
    // the device dispatch order (pg_decode_plan): a permutation of the work
    // list; past one item per CU heaviest first, otherwise request order
    std::vector<pg::WorkItem> order(n_items);
    if (n_items > 0) std::memcpy(order.data(), raw.data(), n_items * sizeof(pg::WorkItem));
    const std::vector<pg::WorkItem> listed = order;
    pg::order_for_dispatch(order, cus);
    // the weight the planner gave each item, derived here from the tables:
    // FP16 tail pages beside INT8 ones, and a hinted table's last pages, x2
    auto weight = [&](const pg::WorkItem& it) {
      int per_page = 1;
      if (it.segment == 1 && kind == PG_KV_INT8) per_page = 2;
      if (it.segment == 0 && hint > 0) {
        const int end = indptr[it.request + 1];
        if (it.page_begin >= end - std::min(hint, end - indptr[it.request])) per_page = 2;
      }
      return (it.page_end - it.page_begin) * per_page;
    };
    for (int i = 0; i < n_items; ++i)
      check(order[i].page_weight * (order[i].page_end - order[i].page_begin) == weight(order[i]),
            "an item carries the weight it was planned with", iter);
    if (n_items <= cus) {
      check(n_items == 0 || std::memcmp(order.data(), listed.data(),
                                        n_items * sizeof(pg::WorkItem)) == 0,
            "one-round plans keep request order", iter);
    } else {
      for (int i = 1; i < n_items; ++i)
        check(weight(order[i - 1]) >= weight(order[i]), "heaviest items first", iter);
    }
    auto by_request = [](const pg::WorkItem& a, const pg::WorkItem& b) {
      return a.request != b.request ? a.request < b.request : a.item_in_request < b.item_in_request;
    };
    std::vector<pg::WorkItem> x = order, y = listed;
    std::sort(x.begin(), x.end(), by_request);
    std::sort(y.begin(), y.end(), by_request);
    check(n_items == 0 || std::memcmp(x.data(), y.data(), n_items * sizeof(pg::WorkItem)) == 0,
          "the dispatch order is a permutation of the work list", iter);
  }
  // pg_select_split_pages over random uniform batches (and invalid arguments)
  for (int iter = 0; iter < iterations / 4; ++iter) {
    const int64_t pages = uniform(0, 9) == 0 ? uniform(-5, 0) : uniform(1, 400000);
    const int batch = uniform(0, 9) == 0 ? uniform(-2, 0) : uniform(1, 600);
    const int bytes = uniform(0, 9) == 0 ? uniform(0, 9000) : (uniform(0, 1) ? 4096 : 8192);
    const int split = pg_select_split_pages(pages, batch, 8, bytes, uniform(0, 600));
    const bool valid = pages > 0 && batch > 0 && (bytes == 4096 || bytes == 8192);
    check(split >= 0 && split <= 64, "a split lies in 0..64", iter);
    if (!valid) check(split == 0 && std::strlen(pg_last_error()) > 0, "bad arguments give 0", iter);
    if (split == 0) check(std::strlen(pg_last_error()) > 0, "a zero split leaves a message", iter);
  }
  if (failures) return 1;
  std::printf("ok %d %d %d\n", plans, rejected, closed);
  return 0;
}
