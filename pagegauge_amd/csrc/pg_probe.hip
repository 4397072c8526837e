// HBM read probes for gfx950: the bandwidth a plain read reaches on this
// device, the denominator against which the decode kernels are judged
// beside the 8 TB/s specification.  Not part of the decode path.
//
//  * linear_read_kernel: a grid-stride read of one contiguous buffer,
//    16 bytes per lane per load, eight nontemporal loads in flight per lane;
//  * page_walk_kernel: the pages of a CSR page table (any order), each read
//    as one contiguous block of K codes and one of V codes by a whole
//    workgroup (the most favourable way to stream this cache's layout).
// Loaded values are folded into a register and written only under a
// condition that depends on them, so no load can be removed.
#include "pg_common.h"

#include <hip/hip_ext.h>

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

extern "C" int32_t pg_probe_linear_read(const void* src, int64_t bytes, int32_t* sink,
                                        int32_t blocks, void* start_event, void* stop_event,
                                        void* stream) {
  clear_error();
  if (!src || !sink) return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if (bytes < 16 || bytes % 16 || reinterpret_cast<uintptr_t>(src) % 16)
    return fail(PG_ERROR_INVALID_ARGUMENT, "the read must be a 16-byte aligned multiple of 16 bytes");
  if (blocks < 1) return fail(PG_ERROR_INVALID_ARGUMENT, "blocks must be positive");
  return probe_launch(linear_read_kernel, blocks, stream, start_event, stop_event,
                      "probe_linear_read", static_cast<const v4i*>(src), bytes / 16, sink);
}

extern "C" int32_t pg_probe_page_walk(const void* k_pages, const void* v_pages,
                                      const int32_t* indices, int32_t pages,
                                      int32_t pages_per_block, int32_t page_bytes,
                                      int32_t* sink, void* start_event, void* stop_event,
                                      void* stream) {
  clear_error();
  if (!k_pages || !v_pages || !indices || !sink)
    return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if (pages < 1 || pages_per_block < 1 || page_bytes < 16 || page_bytes % 16)
    return fail(PG_ERROR_INVALID_ARGUMENT, "pages, pages per block and page bytes must be positive");
  const int32_t blocks = (pages + pages_per_block - 1) / pages_per_block;
  return probe_launch(page_walk_kernel, blocks, stream, start_event, stop_event, "probe_page_walk",
                      static_cast<const int8_t*>(k_pages), static_cast<const int8_t*>(v_pages),
                      indices, pages, pages_per_block, page_bytes, sink);
}
