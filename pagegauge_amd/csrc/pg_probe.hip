// HBM read probes for gfx950: the bandwidth a plain read reaches on this
// device, the denominator against which the decode kernels are judged
// beside the 8 TB/s specification.  Not part of the decode path.
//
//  * linear_read_kernel: a grid-stride read of one contiguous buffer,
//    16 bytes per lane per load, eight nontemporal loads in flight per lane;
//  * page_walk_kernel: the pages of a CSR page table (any order), each read
//    as one contiguous block of K codes and one of V codes by a whole
//    workgroup (the most favourable way to stream this cache's layout);
//  * decode_walk_kernel: the same pages read the way the INT8 decode kernel
//    reads them (work items of consecutive table entries, one wave per KV
//    head, 4-page groups with 1 or 2 groups in flight), loads only, so
//    that the decode kernel can be set against the stream of its own
//    access pattern; ``mode`` varies the lane pattern of the loads.
// Loaded values are folded into a register and written only under a
// condition that depends on them, so no load can be removed; workgroup b
// writes sink[b] only, and every entry point checks that the sink holds an
// entry per workgroup of its grid.
//
// Built into libpagegauge_bench.so (include/pagegauge_bench.h), bench.py's
// measurement library, not into the product library.
#include "pg_common.h"

#include <hip/hip_ext.h>

#include <string>

namespace pg {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kProbeThreads = 256;

__global__ __launch_bounds__(kProbeThreads) void linear_read_kernel(const v4i* src, int64_t count,
                                                                    int32_t* sink) {
  v4i acc = {0, 0, 0, 0};
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kProbeThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x;
  for (; i + 7 * stride < count; i += 8 * stride) {
    v4i x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= x[u];
  }
  for (; i < count; i += stride) acc ^= __builtin_nontemporal_load(src + i);
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x5a17c3e1) sink[blockIdx.x] = acc.x;
}

// Block b reads pages [b * pages_per_block, ...) of the table: K block then
// V block of each page, ``page_bytes`` each (16 tokens x Hkv x 128 codes).
__global__ __launch_bounds__(kProbeThreads) void page_walk_kernel(const int8_t* k_pages,
                                                                  const int8_t* v_pages,
                                                                  const int32_t* indices,
                                                                  int32_t pages, int32_t per_block,
                                                                  int32_t page_bytes,
                                                                  int32_t* sink) {
  const int begin = blockIdx.x * per_block;
  const int end = min(begin + per_block, pages);
  const int vectors = page_bytes / 16;
  v4i acc = {0, 0, 0, 0};
  for (int p = begin; p < end; ++p) {
    const int64_t page = indices[p];
    const v4i* k = reinterpret_cast<const v4i*>(k_pages + page * page_bytes);
    const v4i* v = reinterpret_cast<const v4i*>(v_pages + page * page_bytes);
    for (int i = threadIdx.x; i < vectors; i += kProbeThreads) acc ^= k[i] ^ v[i];
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x5a17c3e1) sink[blockIdx.x] = acc.x;
}

// Loads of one 4-page group for one wave: 8 x 16 B of K and 16 x 8 B of V
// per lane (the decode kernel's register footprint).
struct WalkGroup {
  v4i k[4][2];
  uint32_t v[16][2];
};

template <typename T>
__device__ __forceinline__ void walk_pin(T& x) {
  T value = x;
  asm volatile("" : "+v"(value));
  x = value;
}

// Work item b covers table entries [b * pages_per_item, +pages_per_item);
// wave w of workgroup (b, y) reads KV head y * heads_per_block + w.  Lane
// (kg = lane / 16, m16 = lane % 16) offsets within a (page, head), for 8 KV
// heads of 128 codes (1 KiB rows):
//   mode 0 (the decode kernel's): K bytes 16 kg.. and 64 + 16 kg.. of token
//          row m16; V 8 bytes of dims 8 m16.. of token rows 4 kg + t;
//   mode 1: whole 128-byte head rows, 8 rows per instruction;
//   mode 2: the workgroup's waves read whole pages as contiguous 1 KiB per
//          instruction (every byte of the page once; heads_per_block 8).
template <int kDepth, int kMode>
__global__ __launch_bounds__(512) void decode_walk_kernel(const int8_t* k_pages,
                                                          const int8_t* v_pages,
                                                          const int32_t* indices,
                                                          int32_t pages_per_item,
                                                          int32_t heads_per_block, int32_t* sink) {
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int head = blockIdx.y * heads_per_block + wave;
  const int m16 = lane & 15;
  const int kg = lane >> 4;
  const int begin = blockIdx.x * pages_per_item;
  const int my_page = indices[begin + min(lane, pages_per_item - 1)];
  const uint32_t k_off = kMode == 0 ? m16 * 1024 + head * 128 + 16 * kg
                         : kMode == 1 ? (lane >> 3) * 1024 + head * 128 + 16 * (lane & 7)
                                      : wave * 2048 + 16 * lane;
  const uint32_t k_step = kMode == 0 ? 64 : kMode == 1 ? 8192 : 1024;
  const uint32_t v_off = kMode == 0 ? 4 * kg * 1024 + head * 128 + 8 * m16 : k_off;
  v4i acc = {0, 0, 0, 0};
  WalkGroup buf[kDepth];
  auto issue = [&](int g, WalkGroup& d) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t p = __builtin_amdgcn_readlane(my_page, 4 * g + i);
      const int8_t* kp = k_pages + p * 16384;
      d.k[i][0] = *reinterpret_cast<const v4i*>(kp + k_off);
      d.k[i][1] = *reinterpret_cast<const v4i*>(kp + k_off + k_step);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t p = __builtin_amdgcn_readlane(my_page, 4 * g + i);
      const int8_t* vp = v_pages + p * 16384;
      if (kMode == 0) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const uint2 x = *reinterpret_cast<const uint2*>(vp + v_off + t * 1024);
          d.v[4 * i + t][0] = x.x;
          d.v[4 * i + t][1] = x.y;
        }
      } else {
        const v4i a0 = *reinterpret_cast<const v4i*>(vp + v_off);
        const v4i a1 = *reinterpret_cast<const v4i*>(vp + v_off + k_step);
        d.v[4 * i][0] = a0.x;
        d.v[4 * i][1] = a0.y;
        d.v[4 * i + 1][0] = a0.z;
        d.v[4 * i + 1][1] = a0.w;
        d.v[4 * i + 2][0] = a1.x;
        d.v[4 * i + 2][1] = a1.y;
        d.v[4 * i + 3][0] = a1.z;
        d.v[4 * i + 3][1] = a1.w;
      }
    }
  };
  auto consume = [&](WalkGroup& c) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      walk_pin(c.k[i][0]);
      walk_pin(c.k[i][1]);
      acc ^= c.k[i][0] ^ c.k[i][1];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      walk_pin(c.v[i][0]);
      walk_pin(c.v[i][1]);
      acc.x ^= static_cast<int>(c.v[i][0]);
      acc.y ^= static_cast<int>(c.v[i][1]);
    }
  };
  const int groups = pages_per_item / 4;
#pragma unroll
  for (int d = 0; d < kDepth; ++d)
    if (d < groups) issue(d, buf[d]);
  for (int g = 0; g < groups; g += kDepth) {
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      if (g + d < groups) {
        consume(buf[d]);
        if (g + d + kDepth < groups) issue(g + d + kDepth, buf[d]);
      }
    }
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x5a17c3e1) sink[blockIdx.x] = acc.x;
}

}  // namespace
}  // namespace pg

using namespace pg;

// Launches on ``stream``; with events, the dispatch itself stamps them
// (its begin and end, the interval a kernel trace reports).
template <typename Kernel, typename... Args>
int32_t probe_launch(Kernel kernel, int32_t blocks, void* stream, void* start_event,
                     void* stop_event, const char* what, Args... args) {
  if (start_event || stop_event) {
    hipExtLaunchKernelGGL(kernel, dim3(blocks), dim3(kProbeThreads), 0, as_stream(stream),
                          static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event),
                          0, args...);
  } else {
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kProbeThreads), 0, as_stream(stream), args...);
  }
  return check_launch(what);
}

namespace {
int32_t check_sink(int64_t blocks, int64_t sink_len) {
  if (blocks > sink_len)
    return fail(PG_ERROR_INVALID_ARGUMENT,
                "the sink needs an entry per workgroup (" + std::to_string(blocks) + " > " +
                    std::to_string(sink_len) + ")");
  return PG_OK;
}
}  // namespace

extern "C" int32_t pg_probe_linear_read(const void* src, int64_t bytes, int32_t* sink,
                                        int64_t sink_len, int32_t blocks, void* start_event,
                                        void* stop_event, void* stream) {
  clear_error();
  if (!src || !sink) return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if (bytes < 16 || bytes % 16 || reinterpret_cast<uintptr_t>(src) % 16)
    return fail(PG_ERROR_INVALID_ARGUMENT, "the read must be a 16-byte aligned multiple of 16 bytes");
  if (blocks < 1) return fail(PG_ERROR_INVALID_ARGUMENT, "blocks must be positive");
  if (int32_t rc = check_sink(blocks, sink_len)) return rc;
  return probe_launch(linear_read_kernel, blocks, stream, start_event, stop_event,
                      "probe_linear_read", static_cast<const v4i*>(src), bytes / 16, sink);
}

extern "C" int32_t pg_probe_decode_walk(const void* k_pages, const void* v_pages,
                                        const int32_t* indices, int32_t pages,
                                        int32_t pages_per_item, int32_t heads_per_block,
                                        int32_t depth, int32_t mode, int32_t* sink,
                                        int64_t sink_len, void* start_event, void* stop_event,
                                        void* stream) {
  clear_error();
  if (!k_pages || !v_pages || !indices || !sink)
    return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if (pages_per_item < 4 || pages_per_item > 64 || pages_per_item % 4 || pages < pages_per_item ||
      pages % pages_per_item)
    return fail(PG_ERROR_INVALID_ARGUMENT,
                "pages must be whole items of 4..64 pages (a multiple of 4 each)");
  if (heads_per_block != 4 && heads_per_block != 8)
    return fail(PG_ERROR_INVALID_ARGUMENT, "heads_per_block must be 4 or 8 (of 8 KV heads)");
  if (depth < 1 || depth > 2) return fail(PG_ERROR_INVALID_ARGUMENT, "depth must be 1 or 2");
  if (mode < 0 || mode > 2 || (mode == 2 && heads_per_block != 8))
    return fail(PG_ERROR_INVALID_ARGUMENT, "mode must be 0, 1, or 2 with 8 heads per block");
  const dim3 grid(pages / pages_per_item, 8 / heads_per_block);
  if (int32_t rc = check_sink(grid.x, sink_len)) return rc;   // sink[blockIdx.x]
  const dim3 block(kWave * heads_per_block);
  hipEvent_t start = static_cast<hipEvent_t>(start_event);
  hipEvent_t stop = static_cast<hipEvent_t>(stop_event);
  const int8_t* k = static_cast<const int8_t*>(k_pages);
  const int8_t* v = static_cast<const int8_t*>(v_pages);
#define PG_WALK_CASE(D, M)                                                                    \
  if (depth == D && mode == M) {                                                             \
    hipExtLaunchKernelGGL((decode_walk_kernel<D, M>), grid, block, 0, as_stream(stream), start, \
                          stop, 0, k, v, indices, pages_per_item, heads_per_block, sink);      \
    return check_launch("probe_decode_walk");                                                \
  }
  PG_WALK_CASE(1, 0) PG_WALK_CASE(2, 0)
  PG_WALK_CASE(1, 1) PG_WALK_CASE(2, 1)
  PG_WALK_CASE(1, 2) PG_WALK_CASE(2, 2)
#undef PG_WALK_CASE
  return fail(PG_ERROR_INVALID_ARGUMENT, "unsupported probe configuration");
}

extern "C" int32_t pg_probe_page_walk(const void* k_pages, const void* v_pages,
                                      const int32_t* indices, int32_t pages,
                                      int32_t pages_per_block, int32_t page_bytes,
                                      int32_t* sink, int64_t sink_len, void* start_event,
                                      void* stop_event, void* stream) {
  clear_error();
  if (!k_pages || !v_pages || !indices || !sink)
    return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if (pages < 1 || pages_per_block < 1 || page_bytes < 16 || page_bytes % 16)
    return fail(PG_ERROR_INVALID_ARGUMENT, "pages, pages per block and page bytes must be positive");
  const int32_t blocks = (pages + pages_per_block - 1) / pages_per_block;
  if (int32_t rc = check_sink(blocks, sink_len)) return rc;
  return probe_launch(page_walk_kernel, blocks, stream, start_event, stop_event, "probe_page_walk",
                      static_cast<const int8_t*>(k_pages), static_cast<const int8_t*>(v_pages),
                      indices, pages, pages_per_block, page_bytes, sink);
}
