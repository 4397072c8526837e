// Cache-update kernels (K2 family) for gfx950: fused RoPE + FP16 append,
// fused RoPE + centered append + completed-page INT8 finalize (static,
// device-scalar and per-request positions), the per-request paged append /
// append-finalize, and the bulk completed-page quantizer.
//
// Everything here must be bit-exact against the reference arithmetic
// (tests/page_gauge_append_extension.cu:148-383,
// scripts/benchmark_page_gauge_overheads.py:23-205): FP16 products and sums
// round separately (no FMA contraction: this file is built with
// -ffp-contract=off and the pragma below), FP32 division is IEEE (HIP's
// default correctly rounded division), and the sign-symmetric
// floor(q + 0.5f) rounding is evaluated in float32 exactly as written.
//
// Layout per launch: one wave64 per (request, head row); lane l owns the two
// adjacent dimensions 2l and 2l+1, so every row access is one coalesced
// 256-byte (FP16) or 128-byte (INT8) transaction per wave.
#pragma clang fp contract(off)

#include "pg_common.h"

#include <mutex>

namespace pg {
namespace {

constexpr int kWavesPerBlock = 4;

struct UpdateParams {
  const uint16_t* query;
  const uint16_t* key;
  const uint16_t* value;
  const uint16_t* cosine;
  const uint16_t* sine;
  const uint16_t* key_center;
  const uint16_t* value_center;
  int64_t center_batch_stride;
  uint16_t* rotated_query;
  uint16_t* key_pages;    // FP16 pages (plain append) or the exact ring
  uint16_t* value_pages;
  int8_t* key_codes;
  int8_t* value_codes;
  uint16_t* key_scales;
  uint16_t* value_scales;
  int64_t query_batch_stride;
  int64_t key_batch_stride;
  int64_t value_batch_stride;
  int batch_size;
  int query_heads;
  int kv_heads;
  int pages_per_request;       // FP16 cache pages, or exact ring pages E
  int exact_sink_pages;
  int code_pages_per_request;
  int host_position;
  const int32_t* device_position;  // scalar position (graph replay)
  const int32_t* positions;        // per-request positions
  const int32_t* exact_page_ids;   // per-request exact page of the position (serving tables)
  const int32_t* code_page_ids;    // per-request code page of the position
  int64_t num_exact_pages;         // pool sizes for the explicit ids (out of range: no-op)
  int64_t num_code_pages;
  int64_t rope_row_stride;
  int rope_rows;
  int row_blocks;                  // blocks per request
};

struct Half2Bits {
  uint16_t lo, hi;
};

__device__ __forceinline__ Half2Bits load_pair(const uint16_t* base) {
  const uint32_t bits = *reinterpret_cast<const uint32_t*>(base);
  return {static_cast<uint16_t>(bits & 0xffffu), static_cast<uint16_t>(bits >> 16)};
}

__device__ __forceinline__ void store_pair(uint16_t* base, uint16_t lo, uint16_t hi) {
  *reinterpret_cast<uint32_t*>(base) = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
}

__device__ __forceinline__ _Float16 bits_to_h(uint16_t b) { return __builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ uint16_t h_to_bits(_Float16 h) { return __builtin_bit_cast(uint16_t, h); }

// One RoPE element: rn16(rn16(x*c) + rn16(partner*s)).  The partner's sign is
// flipped by XOR for the first half (tests/page_gauge_append_extension.cu:154-160).
__device__ __forceinline__ uint16_t rope_element(uint16_t x, uint16_t partner, uint16_t c,
                                                 uint16_t s, bool flip) {
  if (flip) partner ^= 0x8000u;
  const _Float16 primary = bits_to_h(x) * bits_to_h(c);
  const _Float16 secondary = bits_to_h(partner) * bits_to_h(s);
  const _Float16 sum = primary + secondary;
  return h_to_bits(sum);
}

// Rotates dims (2*lane, 2*lane+1) of a 128-wide row.
__device__ __forceinline__ Half2Bits rope_pair(const uint16_t* row, const uint16_t* cosine,
                                               const uint16_t* sine, int lane) {
  const int d = 2 * lane;
  const bool first_half = d < kHeadDim / 2;
  const int partner_d = first_half ? d + kHeadDim / 2 : d - kHeadDim / 2;
  const Half2Bits x = load_pair(row + d);
  const Half2Bits partner = load_pair(row + partner_d);
  const Half2Bits c = load_pair(cosine + d);
  const Half2Bits s = load_pair(sine + d);
  return {rope_element(x.lo, partner.lo, c.lo, s.lo, first_half),
          rope_element(x.hi, partner.hi, c.hi, s.hi, first_half)};
}

// fp16(float(a) - float(b)) with a float32 subtraction (:316-325).
__device__ __forceinline__ uint16_t centered(uint16_t a, uint16_t b) {
  const float diff = half_bits_to_float(a) - half_bits_to_float(b);
  return __half_as_ushort(__float2half_rn(diff));
}

__device__ __forceinline__ int8_t sign_symmetric_code(float quotient) {
  int code;
  if (quotient >= 0.0f) {
    code = static_cast<int>(floorf(quotient + 0.5f));
  } else {
    code = -static_cast<int>(floorf(-quotient + 0.5f));
  }
  code = max(-127, min(127, code));
  return static_cast<int8_t>(code);
}

__device__ __forceinline__ uint16_t stored_scale(float maximum) {
  return __half_as_ushort(__float2half_rn(fmaxf(maximum / 127.0f, 0x1p-20f)));
}

// Quantises one completed (page, head) block of 16 rows.  ``rows`` points at
// the FP16 block (row stride ``row_stride`` elements); row ``current_token``
// is taken from registers (``cur``) instead of memory, all others are read
// back.  Writes 16 code rows and the scale.  Lane owns dims 2*lane, 2*lane+1.
__device__ __forceinline__ void finalize_block(const uint16_t* rows, int64_t row_stride,
                                               int current_token, Half2Bits cur,
                                               int8_t* code_rows, uint16_t* scale_out,
                                               int lane) {
  Half2Bits page[kPageSize];
  float local_max = 0.0f;
#pragma unroll
  for (int t = 0; t < kPageSize; ++t) {
    page[t] = t == current_token ? cur : load_pair(rows + t * row_stride + 2 * lane);
    local_max = fmaxf(local_max, fabsf(half_bits_to_float(page[t].lo)));
    local_max = fmaxf(local_max, fabsf(half_bits_to_float(page[t].hi)));
  }
  const float maximum = wave_max(local_max);
  const uint16_t scale_bits = stored_scale(maximum);
  if (lane == 0) *scale_out = scale_bits;
  const float scale = half_bits_to_float(scale_bits);
#pragma unroll
  for (int t = 0; t < kPageSize; ++t) {
    const int8_t c0 = sign_symmetric_code(half_bits_to_float(page[t].lo) / scale);
    const int8_t c1 = sign_symmetric_code(half_bits_to_float(page[t].hi) / scale);
    *reinterpret_cast<uint16_t*>(code_rows + t * row_stride + 2 * lane) =
        static_cast<uint16_t>(static_cast<uint8_t>(c0)) |
        static_cast<uint16_t>(static_cast<uint16_t>(static_cast<uint8_t>(c1)) << 8);
  }
}

template <bool kPageGauge>
__global__ __launch_bounds__(kWave * kWavesPerBlock) void rope_append_kernel(UpdateParams p) {
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int request = blockIdx.x / p.row_blocks;
  const int row = (blockIdx.x % p.row_blocks) * kWavesPerBlock + wave;
  if (request >= p.batch_size || row >= p.query_heads + p.kv_heads) return;

  int position;
  bool dynamic;
  if (p.positions != nullptr) {
    position = p.positions[request];
    dynamic = true;
  } else if (p.device_position != nullptr) {
    position = p.device_position[0];
    dynamic = true;
  } else {
    position = p.host_position;
    dynamic = false;
  }
  const bool explicit_pages = p.exact_page_ids != nullptr;
  const int capacity = explicit_pages ? INT32_MAX
                                      : (kPageGauge ? p.code_pages_per_request : p.pages_per_request) *
                                            kPageSize;
  if (position < 0 || position >= capacity || (dynamic && position >= p.rope_rows)) return;
  const uint16_t* cosine = p.cosine;
  const uint16_t* sine = p.sine;
  if (dynamic) {
    cosine += static_cast<int64_t>(position) * p.rope_row_stride;
    sine += static_cast<int64_t>(position) * p.rope_row_stride;
  }
  const int page = position / kPageSize;
  const int token = position % kPageSize;

  if (row < p.query_heads) {
    const uint16_t* q = p.query + request * p.query_batch_stride + row * kHeadDim;
    const Half2Bits r = rope_pair(q, cosine, sine, lane);
    store_pair(p.rotated_query + (static_cast<int64_t>(request) * p.query_heads + row) * kHeadDim +
                   2 * lane,
               r.lo, r.hi);
    return;
  }
  const int head = row - p.query_heads;
  const uint16_t* k = p.key + request * p.key_batch_stride + head * kHeadDim;
  const uint16_t* v = p.value + request * p.value_batch_stride + head * kHeadDim;
  const Half2Bits rk = rope_pair(k, cosine, sine, lane);
  const Half2Bits rv = load_pair(v + 2 * lane);
  const int64_t row_stride = static_cast<int64_t>(p.kv_heads) * kHeadDim;

  if constexpr (!kPageGauge) {
    const int64_t physical = static_cast<int64_t>(request) * p.pages_per_request + page;
    const int64_t dst = ((physical * kPageSize + token) * p.kv_heads + head) * kHeadDim + 2 * lane;
    store_pair(p.key_pages + dst, rk.lo, rk.hi);
    store_pair(p.value_pages + dst, rv.lo, rv.hi);
  } else {
    int64_t exact_page, code_page;
    if (explicit_pages) {
      exact_page = p.exact_page_ids[request];
      code_page = p.code_page_ids[request];
      if (exact_page < 0 || code_page < 0 || exact_page >= p.num_exact_pages ||
          code_page >= p.num_code_pages)
        return;                                          // row not scheduled / out of the pools
    } else {
      const int tail_pages = p.pages_per_request - p.exact_sink_pages;
      const int local = page < p.exact_sink_pages ? page : p.exact_sink_pages + page % tail_pages;
      exact_page = static_cast<int64_t>(request) * p.pages_per_request + local;
      code_page = static_cast<int64_t>(request) * p.code_pages_per_request + page;
    }
    const uint16_t* kc = p.key_center + request * p.center_batch_stride + head * kHeadDim + 2 * lane;
    const uint16_t* vc = p.value_center + request * p.center_batch_stride + head * kHeadDim + 2 * lane;
    const Half2Bits ckc = load_pair(kc);
    const Half2Bits cvc = load_pair(vc);
    const Half2Bits ck = {centered(rk.lo, ckc.lo), centered(rk.hi, ckc.hi)};
    const Half2Bits cv = {centered(rv.lo, cvc.lo), centered(rv.hi, cvc.hi)};
    const int64_t page_base = (exact_page * kPageSize * p.kv_heads + head) * kHeadDim;
    store_pair(p.key_pages + page_base + token * row_stride + 2 * lane, ck.lo, ck.hi);
    store_pair(p.value_pages + page_base + token * row_stride + 2 * lane, cv.lo, cv.hi);
    if (token != kPageSize - 1) return;
    // The completed page is quantised in the same launch
    // (tests/page_gauge_append_extension.cu:327-382).
    const int64_t code_base = (code_page * kPageSize * p.kv_heads + head) * kHeadDim;
    finalize_block(p.key_pages + page_base, row_stride, token, ck, p.key_codes + code_base,
                   p.key_scales + code_page * p.kv_heads + head, lane);
    finalize_block(p.value_pages + page_base, row_stride, token, cv, p.value_codes + code_base,
                   p.value_scales + code_page * p.kv_heads + head, lane);
  }
}

// Per-request paged append (Triton append_kv / append_finalize_page_gauge,
// scripts/benchmark_page_gauge_overheads.py:86-205).  One wave per
// (request, head); page ids outside [0, num_pages) and offsets outside
// [0, 16) are skipped.
struct PagedParams {
  const uint16_t* key;
  const uint16_t* value;
  const uint16_t* key_center;
  const uint16_t* value_center;
  uint16_t* key_pages;
  uint16_t* value_pages;
  int8_t* key_codes;
  int8_t* value_codes;
  uint16_t* key_scales;
  uint16_t* value_scales;
  const int32_t* page_ids;
  const int32_t* page_offsets;
  int batch_size;
  int heads;
  int num_pages;
};

template <bool kFinalize>
__global__ __launch_bounds__(kWave * kWavesPerBlock) void paged_append_kernel(PagedParams p) {
  const int lane = threadIdx.x % kWave;
  const int item = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  if (item >= p.batch_size * p.heads) return;
  const int request = item / p.heads;
  const int head = item % p.heads;
  const int page = p.page_ids[request];
  const int token = p.page_offsets[request];
  if (page < 0 || page >= p.num_pages || token < 0 || token >= kPageSize) return;
  const int64_t row_stride = static_cast<int64_t>(p.heads) * kHeadDim;
  const int64_t src = (static_cast<int64_t>(request) * p.heads + head) * kHeadDim + 2 * lane;
  const int64_t page_base = (static_cast<int64_t>(page) * kPageSize * p.heads + head) * kHeadDim;
  const Half2Bits k = load_pair(p.key + src);
  const Half2Bits v = load_pair(p.value + src);
  if constexpr (!kFinalize) {
    store_pair(p.key_pages + page_base + token * row_stride + 2 * lane, k.lo, k.hi);
    store_pair(p.value_pages + page_base + token * row_stride + 2 * lane, v.lo, v.hi);
  } else {
    const Half2Bits kc = load_pair(p.key_center + head * kHeadDim + 2 * lane);
    const Half2Bits vc = load_pair(p.value_center + head * kHeadDim + 2 * lane);
    const Half2Bits ck = {centered(k.lo, kc.lo), centered(k.hi, kc.hi)};
    const Half2Bits cv = {centered(v.lo, vc.lo), centered(v.hi, vc.hi)};
    store_pair(p.key_pages + page_base + token * row_stride + 2 * lane, ck.lo, ck.hi);
    store_pair(p.value_pages + page_base + token * row_stride + 2 * lane, cv.lo, cv.hi);
    if (token != kPageSize - 1) return;
    finalize_block(p.key_pages + page_base, row_stride, token, ck, p.key_codes + page_base,
                   p.key_scales + static_cast<int64_t>(page) * p.heads + head, lane);
    finalize_block(p.value_pages + page_base, row_stride, token, cv, p.value_codes + page_base,
                   p.value_scales + static_cast<int64_t>(page) * p.heads + head, lane);
  }
}

// Bulk quantizer: one wave per (page, head); float32-centered values (not
// rounded to FP16), scale and sign-symmetric codes as the finalize
// (scripts/benchmark_page_gauge_overheads.py:23-83), or with ``half_even``
// the round-half-even codes of the K1 driver's quantize_page_gauge
// (scripts/benchmark_flashinfer_page_affine_int8.py:256-278: torch.round of
// the float32 quotient).  ``value`` may be null (one tensor).
struct QuantizeParams {
  const uint16_t* key;
  const uint16_t* value;
  const uint16_t* key_center;
  const uint16_t* value_center;
  int8_t* key_codes;
  int8_t* value_codes;
  uint16_t* key_scales;
  uint16_t* value_scales;
  int64_t num_pages;
  int heads;
  int64_t key_token_stride;     // elements between token rows of the source
  int64_t value_token_stride;
  // Optional exact ring (prefill): page i is also stored centered in FP16 at
  // ring page exact_map[i] when exact_map[i] >= 0.
  const int32_t* exact_map;
  uint16_t* exact_key;
  uint16_t* exact_value;
  int half_even;
};

// Round-half-even of the quotient (v_rndne_f32 under the default rounding
// mode), clamped to [-127, 127].
__device__ __forceinline__ int8_t half_even_code(float quotient) {
  return static_cast<int8_t>(fminf(fmaxf(rintf(quotient), -127.0f), 127.0f));
}

// ``src`` rows are ``src_stride`` elements apart, code rows ``row_stride``.
// With ``ring`` set, the FP16-rounded centered rows are also written there
// (row stride ``row_stride``), as the reference's prefill stores exact pages.
__device__ __forceinline__ void quantize_block(const uint16_t* src, int64_t src_stride,
                                               const uint16_t* center, int64_t row_stride,
                                               int8_t* codes, uint16_t* scale_out,
                                               uint16_t* ring, int lane, bool half_even) {
  const Half2Bits c = load_pair(center + 2 * lane);
  const float c0 = half_bits_to_float(c.lo);
  const float c1 = half_bits_to_float(c.hi);
  float lo[kPageSize];
  float hi[kPageSize];
  float local_max = 0.0f;
#pragma unroll
  for (int t = 0; t < kPageSize; ++t) {
    const Half2Bits x = load_pair(src + t * src_stride + 2 * lane);
    lo[t] = half_bits_to_float(x.lo) - c0;
    hi[t] = half_bits_to_float(x.hi) - c1;
    local_max = fmaxf(local_max, fmaxf(fabsf(lo[t]), fabsf(hi[t])));
    if (ring != nullptr)
      store_pair(ring + t * row_stride + 2 * lane, __half_as_ushort(__float2half_rn(lo[t])),
                 __half_as_ushort(__float2half_rn(hi[t])));
  }
  const float maximum = wave_max(local_max);
  const uint16_t scale_bits = stored_scale(maximum);
  if (lane == 0) *scale_out = scale_bits;
  const float scale = half_bits_to_float(scale_bits);
#pragma unroll
  for (int t = 0; t < kPageSize; ++t) {
    const float d0 = lo[t] / scale;
    const float d1 = hi[t] / scale;
    const int8_t q0 = half_even ? half_even_code(d0) : sign_symmetric_code(d0);
    const int8_t q1 = half_even ? half_even_code(d1) : sign_symmetric_code(d1);
    *reinterpret_cast<uint16_t*>(codes + t * row_stride + 2 * lane) =
        static_cast<uint16_t>(static_cast<uint8_t>(q0)) |
        static_cast<uint16_t>(static_cast<uint16_t>(static_cast<uint8_t>(q1)) << 8);
  }
}

__global__ __launch_bounds__(kWave * kWavesPerBlock) void quantize_pages_kernel(QuantizeParams p) {
  const int lane = threadIdx.x % kWave;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  if (item >= p.num_pages * p.heads) return;
  const int64_t page = item / p.heads;
  const int head = static_cast<int>(item % p.heads);
  const int64_t row_stride = static_cast<int64_t>(p.heads) * kHeadDim;
  const int64_t base = (page * kPageSize * p.heads + head) * kHeadDim;
  const int32_t ring_page = p.exact_map != nullptr ? p.exact_map[page] : -1;
  const int64_t ring_base = (static_cast<int64_t>(ring_page) * kPageSize * p.heads + head) * kHeadDim;
  quantize_block(p.key + page * kPageSize * p.key_token_stride + head * kHeadDim,
                 p.key_token_stride, p.key_center + head * kHeadDim, row_stride,
                 p.key_codes + base, p.key_scales + item,
                 ring_page >= 0 ? p.exact_key + ring_base : nullptr, lane, p.half_even != 0);
  if (p.value != nullptr)
    quantize_block(p.value + page * kPageSize * p.value_token_stride + head * kHeadDim,
                   p.value_token_stride, p.value_center + head * kHeadDim, row_stride,
                   p.value_codes + base, p.value_scales + item,
                   ring_page >= 0 ? p.exact_value + ring_base : nullptr, lane, p.half_even != 0);
}

// Exact per-(head, dim) token mean.  Every FP16 value is an integer multiple
// of 2^-24, so the column sums are kept exactly as int64 counts of 2^-24 and
// the result does not depend on the reduction order.  Launch 1 sums the
// tokens of one chunk per block; launch 2 adds the chunk sums and rounds
// f16(f32(f64(sum * 2^-24) / tokens)).
constexpr int kCenterChunk = 64;          // tokens per partial-sum block
constexpr int kCenterThreads = 256;       // 2 columns per thread -> 512 columns per block
constexpr int64_t kCenterMaxTokens = int64_t{1} << 22;  // |sum| < 2^40 * 2^22 fits in int64

__device__ __forceinline__ int64_t half_to_fixed24(uint16_t h) {
  const int e = (h >> 10) & 0x1f;
  const int64_t m = h & 0x3ff;
  const int64_t magnitude = e == 0 ? m : ((1024 + m) << (e - 1));
  return (h & 0x8000u) ? -magnitude : magnitude;
}

struct CenterParams {
  const uint16_t* source[2];   // key, value: [tokens, heads, 128] rows
  int64_t token_stride[2];
  uint16_t* center[2];         // [heads, 128]
  int64_t* partial;            // [2][chunks][heads*128]
  int64_t tokens;
  int columns;                 // heads * 128
  int chunks;
};

__global__ __launch_bounds__(kCenterThreads) void center_partial_kernel(CenterParams p) {
  const int which = blockIdx.z;
  const int column = (blockIdx.x * kCenterThreads + threadIdx.x) * 2;
  if (column >= p.columns) return;
  const int64_t begin = static_cast<int64_t>(blockIdx.y) * kCenterChunk;
  const int64_t end = min(begin + kCenterChunk, p.tokens);
  const uint16_t* src = p.source[which] + column;
  const int64_t stride = p.token_stride[which];
  int64_t s0 = 0, s1 = 0;
#pragma unroll 8
  for (int64_t t = begin; t < end; ++t) {
    const Half2Bits x = load_pair(src + t * stride);
    s0 += half_to_fixed24(x.lo);
    s1 += half_to_fixed24(x.hi);
  }
  int64_t* out = p.partial + (static_cast<int64_t>(which) * p.chunks + blockIdx.y) * p.columns + column;
  out[0] = s0;
  out[1] = s1;
}

__global__ __launch_bounds__(kCenterThreads) void center_finalize_kernel(CenterParams p) {
  const int which = blockIdx.y;
  const int column = blockIdx.x * kCenterThreads + threadIdx.x;
  if (column >= p.columns) return;
  const int64_t* in = p.partial + static_cast<int64_t>(which) * p.chunks * p.columns + column;
  int64_t total = 0;
  for (int c = 0; c < p.chunks; ++c) total += in[static_cast<int64_t>(c) * p.columns];
  const double mean = (static_cast<double>(total) * 0x1p-24) / static_cast<double>(p.tokens);
  p.center[which][column] = __half_as_ushort(__float2half_rn(static_cast<float>(mean)));
}

int32_t check_common(int batch, int query_heads, int kv_heads) {
  if (batch <= 0) return fail(PG_ERROR_INVALID_ARGUMENT, "Q/K/V batch sizes must match and be positive");
  if (query_heads <= 0 || kv_heads <= 0)
    return fail(PG_ERROR_INVALID_ARGUMENT, "head counts must be positive");
  return PG_OK;
}

int32_t launch_rope_append(UpdateParams p, bool page_gauge, hipStream_t stream) {
  p.row_blocks = (p.query_heads + p.kv_heads + kWavesPerBlock - 1) / kWavesPerBlock;
  const int64_t blocks = static_cast<int64_t>(p.batch_size) * p.row_blocks;
  if (blocks > 0x7fffffff) return fail(PG_ERROR_INVALID_ARGUMENT, "batch too large");
  if (page_gauge) {
    hipLaunchKernelGGL(rope_append_kernel<true>, dim3(static_cast<unsigned>(blocks)),
                       dim3(kWave * kWavesPerBlock), 0, stream, p);
  } else {
    hipLaunchKernelGGL(rope_append_kernel<false>, dim3(static_cast<unsigned>(blocks)),
                       dim3(kWave * kWavesPerBlock), 0, stream, p);
  }
  return check_launch(page_gauge ? "rope_append_page_gauge" : "rope_append_fp16");
}

int32_t launch_quantize(const QuantizeParams& p, hipStream_t stream, const char* what) {
  const int64_t waves = p.num_pages * p.heads;
  const int64_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  if (blocks > 0x7fffffff) return fail(PG_ERROR_INVALID_ARGUMENT, "too many pages");
  hipLaunchKernelGGL(quantize_pages_kernel, dim3(static_cast<unsigned>(blocks)),
                     dim3(kWave * kWavesPerBlock), 0, stream, p);
  return check_launch(what);
}

}  // namespace
}  // namespace pg

using namespace pg;

extern "C" int32_t pg_rope_append_fp16(const void* query, const void* key, const void* value,
                                       const void* cosine, const void* sine, void* rotated_query,
                                       void* key_pages, void* value_pages,
                                       int64_t query_batch_stride, int64_t key_batch_stride,
                                       int64_t value_batch_stride, int32_t batch_size,
                                       int32_t query_heads, int32_t kv_heads,
                                       int32_t pages_per_request, int32_t host_position,
                                       const int32_t* device_position, int64_t rope_row_stride,
                                       int32_t rope_rows, void* stream) {
  clear_error();
  if (int32_t rc = check_common(batch_size, query_heads, kv_heads)) return rc;
  if (!query || !key || !value || !cosine || !sine || !rotated_query || !key_pages || !value_pages)
    return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if (pages_per_request <= 0)
    return fail(PG_ERROR_INVALID_ARGUMENT, "FP16 cache pages must divide evenly across requests");
  if (device_position == nullptr && host_position < 0)
    return fail(PG_ERROR_INVALID_ARGUMENT, "position must be non-negative");
  if (device_position != nullptr && rope_rows <= 0)
    return fail(PG_ERROR_INVALID_ARGUMENT,
                "dynamic RoPE tables must be matching [positions,128] tensors");
  UpdateParams p{};
  p.query = static_cast<const uint16_t*>(query);
  p.key = static_cast<const uint16_t*>(key);
  p.value = static_cast<const uint16_t*>(value);
  p.cosine = static_cast<const uint16_t*>(cosine);
  p.sine = static_cast<const uint16_t*>(sine);
  p.rotated_query = static_cast<uint16_t*>(rotated_query);
  p.key_pages = static_cast<uint16_t*>(key_pages);
  p.value_pages = static_cast<uint16_t*>(value_pages);
  p.query_batch_stride = query_batch_stride;
  p.key_batch_stride = key_batch_stride;
  p.value_batch_stride = value_batch_stride;
  p.batch_size = batch_size;
  p.query_heads = query_heads;
  p.kv_heads = kv_heads;
  p.pages_per_request = pages_per_request;
  p.code_pages_per_request = pages_per_request;
  p.host_position = host_position;
  p.device_position = device_position;
  p.rope_row_stride = rope_row_stride;
  p.rope_rows = rope_rows;
  return launch_rope_append(p, false, as_stream(stream));
}

namespace {

int32_t page_gauge_checks(int32_t exact_pages_per_request, int32_t exact_sink_pages,
                          int32_t code_pages_per_request) {
  if (exact_sink_pages < 0)
    return fail(PG_ERROR_INVALID_ARGUMENT, "exact prefix page count must be nonnegative");
  if (exact_pages_per_request <= exact_sink_pages)
    return fail(PG_ERROR_INVALID_ARGUMENT, "exact cache must retain at least one tail-ring page");
  if (exact_sink_pages >= code_pages_per_request)
    return fail(PG_ERROR_INVALID_ARGUMENT, "exact prefix exceeds the logical cache capacity");
  return PG_OK;
}

UpdateParams page_gauge_params(const void* query, const void* key, const void* value,
                               const void* cosine, const void* sine, const void* key_center,
                               const void* value_center, int64_t center_batch_stride,
                               void* rotated_query, void* exact_key_pages,
                               void* exact_value_pages, int8_t* key_codes, int8_t* value_codes,
                               void* key_scales, void* value_scales, int64_t qbs, int64_t kbs,
                               int64_t vbs, int32_t batch_size, int32_t query_heads,
                               int32_t kv_heads, int32_t exact_pages_per_request,
                               int32_t exact_sink_pages, int32_t code_pages_per_request) {
  UpdateParams p{};
  p.query = static_cast<const uint16_t*>(query);
  p.key = static_cast<const uint16_t*>(key);
  p.value = static_cast<const uint16_t*>(value);
  p.cosine = static_cast<const uint16_t*>(cosine);
  p.sine = static_cast<const uint16_t*>(sine);
  p.key_center = static_cast<const uint16_t*>(key_center);
  p.value_center = static_cast<const uint16_t*>(value_center);
  p.center_batch_stride = center_batch_stride;
  p.rotated_query = static_cast<uint16_t*>(rotated_query);
  p.key_pages = static_cast<uint16_t*>(exact_key_pages);
  p.value_pages = static_cast<uint16_t*>(exact_value_pages);
  p.key_codes = key_codes;
  p.value_codes = value_codes;
  p.key_scales = static_cast<uint16_t*>(key_scales);
  p.value_scales = static_cast<uint16_t*>(value_scales);
  p.query_batch_stride = qbs;
  p.key_batch_stride = kbs;
  p.value_batch_stride = vbs;
  p.batch_size = batch_size;
  p.query_heads = query_heads;
  p.kv_heads = kv_heads;
  p.pages_per_request = exact_pages_per_request;
  p.exact_sink_pages = exact_sink_pages;
  p.code_pages_per_request = code_pages_per_request;
  return p;
}

bool any_null(std::initializer_list<const void*> pointers) {
  for (const void* ptr : pointers)
    if (ptr == nullptr) return true;
  return false;
}

}  // namespace

extern "C" int32_t pg_rope_append_page_gauge(
    const void* query, const void* key, const void* value, const void* cosine, const void* sine,
    const void* key_center, const void* value_center, int64_t center_batch_stride,
    void* rotated_query, void* exact_key_pages, void* exact_value_pages, int8_t* key_codes,
    int8_t* value_codes, void* key_scales, void* value_scales, int64_t query_batch_stride,
    int64_t key_batch_stride, int64_t value_batch_stride, int32_t batch_size,
    int32_t query_heads, int32_t kv_heads, int32_t exact_pages_per_request,
    int32_t exact_sink_pages, int32_t code_pages_per_request, int32_t host_position,
    const int32_t* device_position, int64_t rope_row_stride, int32_t rope_rows, void* stream) {
  clear_error();
  if (int32_t rc = check_common(batch_size, query_heads, kv_heads)) return rc;
  if (any_null({query, key, value, cosine, sine, key_center, value_center, rotated_query,
                exact_key_pages, exact_value_pages, key_codes, value_codes, key_scales,
                value_scales}))
    return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if (int32_t rc = page_gauge_checks(exact_pages_per_request, exact_sink_pages,
                                     code_pages_per_request))
    return rc;
  if (device_position == nullptr && host_position < 0)
    return fail(PG_ERROR_INVALID_ARGUMENT, "position must be non-negative");
  if (device_position == nullptr && host_position / kPageSize >= code_pages_per_request)
    return fail(PG_ERROR_INVALID_ARGUMENT,
                "position exceeds the per-request PageGauge cache capacity");
  if (device_position != nullptr && rope_rows <= 0)
    return fail(PG_ERROR_INVALID_ARGUMENT,
                "dynamic RoPE tables must be matching [positions,128] tensors");
  UpdateParams p = page_gauge_params(
      query, key, value, cosine, sine, key_center, value_center, center_batch_stride,
      rotated_query, exact_key_pages, exact_value_pages, key_codes, value_codes, key_scales,
      value_scales, query_batch_stride, key_batch_stride, value_batch_stride, batch_size,
      query_heads, kv_heads, exact_pages_per_request, exact_sink_pages, code_pages_per_request);
  p.host_position = host_position;
  p.device_position = device_position;
  p.rope_row_stride = rope_row_stride;
  p.rope_rows = rope_rows;
  return launch_rope_append(p, true, as_stream(stream));
}

extern "C" int32_t pg_rope_append_page_gauge_positions(
    const void* query, const void* key, const void* value, const void* cosine, const void* sine,
    const int32_t* positions, const void* key_center, const void* value_center,
    int64_t center_batch_stride, void* rotated_query, void* exact_key_pages,
    void* exact_value_pages, int8_t* key_codes, int8_t* value_codes, void* key_scales,
    void* value_scales, int64_t query_batch_stride, int64_t key_batch_stride,
    int64_t value_batch_stride, int32_t batch_size, int32_t query_heads, int32_t kv_heads,
    int32_t exact_pages_per_request, int32_t exact_sink_pages, int32_t code_pages_per_request,
    int64_t rope_row_stride, int32_t rope_rows, void* stream) {
  clear_error();
  if (int32_t rc = check_common(batch_size, query_heads, kv_heads)) return rc;
  if (any_null({query, key, value, cosine, sine, positions, key_center, value_center,
                rotated_query, exact_key_pages, exact_value_pages, key_codes, value_codes,
                key_scales, value_scales}))
    return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if (int32_t rc = page_gauge_checks(exact_pages_per_request, exact_sink_pages,
                                     code_pages_per_request))
    return rc;
  if (rope_rows <= 0)
    return fail(PG_ERROR_INVALID_ARGUMENT,
                "dynamic RoPE tables must be matching [positions,128] tensors");
  UpdateParams p = page_gauge_params(
      query, key, value, cosine, sine, key_center, value_center, center_batch_stride,
      rotated_query, exact_key_pages, exact_value_pages, key_codes, value_codes, key_scales,
      value_scales, query_batch_stride, key_batch_stride, value_batch_stride, batch_size,
      query_heads, kv_heads, exact_pages_per_request, exact_sink_pages, code_pages_per_request);
  p.positions = positions;
  p.rope_row_stride = rope_row_stride;
  p.rope_rows = rope_rows;
  return launch_rope_append(p, true, as_stream(stream));
}

extern "C" int32_t pg_rope_append_page_gauge_slots(
    const void* query, const void* key, const void* value, const void* cosine, const void* sine,
    const int32_t* positions, const int32_t* exact_page_ids, const int32_t* code_page_ids,
    const void* key_center, const void* value_center, int64_t center_batch_stride,
    void* rotated_query, void* exact_key_pages, void* exact_value_pages, int8_t* key_codes,
    int8_t* value_codes, void* key_scales, void* value_scales, int64_t query_batch_stride,
    int64_t key_batch_stride, int64_t value_batch_stride, int32_t batch_size,
    int32_t query_heads, int32_t kv_heads, int64_t num_exact_pages, int64_t num_code_pages,
    int64_t rope_row_stride, int32_t rope_rows, void* stream) {
  clear_error();
  if (int32_t rc = check_common(batch_size, query_heads, kv_heads)) return rc;
  if (num_exact_pages <= 0 || num_code_pages <= 0)
    return fail(PG_ERROR_INVALID_ARGUMENT, "exact and code page pools must be non-empty");
  if (any_null({query, key, value, cosine, sine, positions, exact_page_ids, code_page_ids,
                key_center, value_center, rotated_query, exact_key_pages, exact_value_pages,
                key_codes, value_codes, key_scales, value_scales}))
    return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if (rope_rows <= 0)
    return fail(PG_ERROR_INVALID_ARGUMENT,
                "dynamic RoPE tables must be matching [positions,128] tensors");
  UpdateParams p = page_gauge_params(
      query, key, value, cosine, sine, key_center, value_center, center_batch_stride,
      rotated_query, exact_key_pages, exact_value_pages, key_codes, value_codes, key_scales,
      value_scales, query_batch_stride, key_batch_stride, value_batch_stride, batch_size,
      query_heads, kv_heads, 1, 0, 1);
  p.positions = positions;
  p.exact_page_ids = exact_page_ids;
  p.code_page_ids = code_page_ids;
  p.num_exact_pages = num_exact_pages;
  p.num_code_pages = num_code_pages;
  p.rope_row_stride = rope_row_stride;
  p.rope_rows = rope_rows;
  return launch_rope_append(p, true, as_stream(stream));
}

namespace {

int32_t launch_paged(PagedParams p, bool finalize, hipStream_t stream, const char* what) {
  const int64_t waves = static_cast<int64_t>(p.batch_size) * p.heads;
  const int64_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  if (finalize) {
    hipLaunchKernelGGL(paged_append_kernel<true>, dim3(static_cast<unsigned>(blocks)),
                       dim3(kWave * kWavesPerBlock), 0, stream, p);
  } else {
    hipLaunchKernelGGL(paged_append_kernel<false>, dim3(static_cast<unsigned>(blocks)),
                       dim3(kWave * kWavesPerBlock), 0, stream, p);
  }
  return check_launch(what);
}

}  // namespace

extern "C" int32_t pg_append_kv(const void* key, const void* value, void* key_pages,
                                void* value_pages, const int32_t* page_ids,
                                const int32_t* page_offsets, int32_t batch_size, int32_t heads,
                                int32_t num_pages, void* stream) {
  clear_error();
  if (batch_size <= 0 || heads <= 0 || num_pages <= 0)
    return fail(PG_ERROR_INVALID_ARGUMENT, "batch, heads and pages must be positive");
  if (any_null({key, value, key_pages, value_pages, page_ids, page_offsets}))
    return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  PagedParams p{};
  p.key = static_cast<const uint16_t*>(key);
  p.value = static_cast<const uint16_t*>(value);
  p.key_pages = static_cast<uint16_t*>(key_pages);
  p.value_pages = static_cast<uint16_t*>(value_pages);
  p.page_ids = page_ids;
  p.page_offsets = page_offsets;
  p.batch_size = batch_size;
  p.heads = heads;
  p.num_pages = num_pages;
  return launch_paged(p, false, as_stream(stream), "append_kv");
}

extern "C" int32_t pg_append_finalize_page_gauge(
    const void* key, const void* value, const void* key_center, const void* value_center,
    void* exact_key_pages, void* exact_value_pages, int8_t* key_codes, int8_t* value_codes,
    void* key_scales, void* value_scales, const int32_t* page_ids, const int32_t* page_offsets,
    int32_t batch_size, int32_t heads, int32_t num_pages, void* stream) {
  clear_error();
  if (batch_size <= 0 || heads <= 0 || num_pages <= 0)
    return fail(PG_ERROR_INVALID_ARGUMENT, "batch, heads and pages must be positive");
  if (any_null({key, value, key_center, value_center, exact_key_pages, exact_value_pages,
                key_codes, value_codes, key_scales, value_scales, page_ids, page_offsets}))
    return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  PagedParams p{};
  p.key = static_cast<const uint16_t*>(key);
  p.value = static_cast<const uint16_t*>(value);
  p.key_center = static_cast<const uint16_t*>(key_center);
  p.value_center = static_cast<const uint16_t*>(value_center);
  p.key_pages = static_cast<uint16_t*>(exact_key_pages);
  p.value_pages = static_cast<uint16_t*>(exact_value_pages);
  p.key_codes = key_codes;
  p.value_codes = value_codes;
  p.key_scales = static_cast<uint16_t*>(key_scales);
  p.value_scales = static_cast<uint16_t*>(value_scales);
  p.page_ids = page_ids;
  p.page_offsets = page_offsets;
  p.batch_size = batch_size;
  p.heads = heads;
  p.num_pages = num_pages;
  return launch_paged(p, true, as_stream(stream), "append_finalize_page_gauge");
}

extern "C" int32_t pg_quantize_completed_kv_pages(const void* key, const void* value,
                                                  const void* key_center,
                                                  const void* value_center, int8_t* key_codes,
                                                  int8_t* value_codes, void* key_scales,
                                                  void* value_scales, int64_t num_pages,
                                                  int32_t heads, void* stream) {
  clear_error();
  if (num_pages <= 0 || heads <= 0)
    return fail(PG_ERROR_INVALID_ARGUMENT, "pages and heads must be positive");
  if (any_null({key, value, key_center, value_center, key_codes, value_codes, key_scales,
                value_scales}))
    return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  QuantizeParams p{};
  p.key = static_cast<const uint16_t*>(key);
  p.value = static_cast<const uint16_t*>(value);
  p.key_center = static_cast<const uint16_t*>(key_center);
  p.value_center = static_cast<const uint16_t*>(value_center);
  p.key_codes = key_codes;
  p.value_codes = value_codes;
  p.key_scales = static_cast<uint16_t*>(key_scales);
  p.value_scales = static_cast<uint16_t*>(value_scales);
  p.num_pages = num_pages;
  p.heads = heads;
  p.key_token_stride = p.value_token_stride = static_cast<int64_t>(heads) * kHeadDim;
  return launch_quantize(p, as_stream(stream), "quantize_completed_kv_pages");
}

extern "C" int32_t pg_quantize_page_gauge(const void* values, const void* center,
                                          int8_t* codes, void* scales, int64_t num_pages,
                                          int32_t heads, void* stream) {
  clear_error();
  if (num_pages <= 0 || heads <= 0)
    return fail(PG_ERROR_INVALID_ARGUMENT, "pages and heads must be positive");
  if (any_null({values, center, codes, scales}))
    return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  QuantizeParams p{};
  p.key = static_cast<const uint16_t*>(values);
  p.key_center = static_cast<const uint16_t*>(center);
  p.key_codes = codes;
  p.key_scales = static_cast<uint16_t*>(scales);
  p.num_pages = num_pages;
  p.heads = heads;
  p.key_token_stride = static_cast<int64_t>(heads) * kHeadDim;
  p.half_even = 1;
  return launch_quantize(p, as_stream(stream), "quantize_page_gauge");
}

extern "C" int32_t pg_prefill_page_gauge(const void* key, int64_t key_token_stride,
                                         const void* value, int64_t value_token_stride,
                                         const void* key_center, const void* value_center,
                                         int8_t* key_codes, int8_t* value_codes,
                                         void* key_scales, void* value_scales,
                                         const int32_t* exact_page_map, void* exact_key_pages,
                                         void* exact_value_pages, int64_t num_pages,
                                         int32_t heads, void* stream) {
  clear_error();
  if (num_pages <= 0 || heads <= 0)
    return fail(PG_ERROR_INVALID_ARGUMENT, "pages and heads must be positive");
  if (any_null({key, value, key_center, value_center, key_codes, value_codes, key_scales,
                value_scales}))
    return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if (exact_page_map != nullptr && (exact_key_pages == nullptr || exact_value_pages == nullptr))
    return fail(PG_ERROR_INVALID_ARGUMENT, "an exact page map needs exact key/value pages");
  const int64_t row = static_cast<int64_t>(heads) * kHeadDim;
  if (key_token_stride < row || value_token_stride < row || key_token_stride % 2 ||
      value_token_stride % 2)
    return fail(PG_ERROR_INVALID_ARGUMENT,
                "token strides must be even and cover heads*128 elements");
  QuantizeParams p{};
  p.key = static_cast<const uint16_t*>(key);
  p.value = static_cast<const uint16_t*>(value);
  p.key_center = static_cast<const uint16_t*>(key_center);
  p.value_center = static_cast<const uint16_t*>(value_center);
  p.key_codes = key_codes;
  p.value_codes = value_codes;
  p.key_scales = static_cast<uint16_t*>(key_scales);
  p.value_scales = static_cast<uint16_t*>(value_scales);
  p.num_pages = num_pages;
  p.heads = heads;
  p.key_token_stride = key_token_stride;
  p.value_token_stride = value_token_stride;
  p.exact_map = exact_page_map;
  p.exact_key = static_cast<uint16_t*>(exact_key_pages);
  p.exact_value = static_cast<uint16_t*>(exact_value_pages);
  return launch_quantize(p, as_stream(stream), "prefill_page_gauge");
}

extern "C" int64_t pg_token_major_centers_workspace_bytes(int64_t tokens, int32_t heads) {
  if (tokens <= 0 || heads <= 0) return 0;
  const int64_t chunks = (tokens + kCenterChunk - 1) / kCenterChunk;
  return 2 * chunks * heads * kHeadDim * static_cast<int64_t>(sizeof(int64_t));
}

namespace {

// Both center entry points: checks, then the chunk-sum and finalize launches
// with the chunk sums in ``partial`` (2 * chunks * heads * 128 int64).
int32_t launch_centers(const void* key, int64_t key_token_stride, const void* value,
                       int64_t value_token_stride, int64_t tokens, int32_t heads,
                       void* key_center, void* value_center, int64_t* partial,
                       int64_t partial_bytes, hipStream_t stream) {
  if (tokens <= 0 || heads <= 0)
    return fail(PG_ERROR_INVALID_ARGUMENT, "token-major K/V must contain tokens and heads");
  if (tokens > kCenterMaxTokens)
    return fail(PG_ERROR_INVALID_ARGUMENT, "at most 4194304 tokens per center reduction");
  if (any_null({key, value, key_center, value_center, partial}))
    return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  const int64_t row = static_cast<int64_t>(heads) * kHeadDim;
  if (key_token_stride < row || value_token_stride < row || key_token_stride % 2 ||
      value_token_stride % 2)
    return fail(PG_ERROR_INVALID_ARGUMENT,
                "token strides must be even and cover heads*128 elements");
  if (partial_bytes < pg_token_major_centers_workspace_bytes(tokens, heads))
    return fail(PG_ERROR_WORKSPACE, "center workspace too small");
  CenterParams p{};
  p.source[0] = static_cast<const uint16_t*>(key);
  p.source[1] = static_cast<const uint16_t*>(value);
  p.token_stride[0] = key_token_stride;
  p.token_stride[1] = value_token_stride;
  p.center[0] = static_cast<uint16_t*>(key_center);
  p.center[1] = static_cast<uint16_t*>(value_center);
  p.partial = partial;
  p.tokens = tokens;
  p.columns = static_cast<int>(row);
  p.chunks = static_cast<int>((tokens + kCenterChunk - 1) / kCenterChunk);
  const unsigned column_blocks = static_cast<unsigned>((row / 2 + kCenterThreads - 1) / kCenterThreads);
  hipLaunchKernelGGL(center_partial_kernel, dim3(column_blocks, p.chunks, 2), dim3(kCenterThreads),
                     0, stream, p);
  int32_t rc = check_launch("token_major_centers");
  if (rc != PG_OK) return rc;
  const unsigned finalize_blocks = static_cast<unsigned>((row + kCenterThreads - 1) / kCenterThreads);
  hipLaunchKernelGGL(center_finalize_kernel, dim3(finalize_blocks, 2), dim3(kCenterThreads), 0,
                     stream, p);
  return check_launch("token_major_centers");
}

}  // namespace

extern "C" int32_t pg_token_major_centers(const void* key, int64_t key_token_stride,
                                          const void* value, int64_t value_token_stride,
                                          int64_t tokens, int32_t heads, void* key_center,
                                          void* value_center, void* workspace,
                                          int64_t workspace_bytes, void* stream) {
  clear_error();
  return launch_centers(key, key_token_stride, value, value_token_stride, tokens, heads,
                        key_center, value_center, static_cast<int64_t*>(workspace),
                        workspace_bytes, as_stream(stream));
}

// ---------------------------------------------------------------------------
// No-allocation variant: the chunk sums live in ``scratch``, a file-scope
// device array.  Every GPU the library runs on holds its own copy (8 MiB)
// until the process ends.  On the host, ``scratch`` names a host-side stand-in,
// not device memory: the device address of each GPU's copy comes from
// hipGetSymbolAddress, taken once per device with that device current, and
// only that address is ever handed to a kernel.
// ---------------------------------------------------------------------------
namespace pg {
namespace {

constexpr int64_t kCenterScratchBytes = int64_t{8} << 20;
static __device__ __align__(256) int64_t scratch[kCenterScratchBytes / sizeof(int64_t)];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_address[kMaxScratchDevices] = {};

// Device address of this GPU's ``scratch`` (the current device, which must
// be the stream's).
int32_t center_scratch(hipStream_t stream, int64_t** address) {
  int device = -1;
  if (hipGetDevice(&device) != hipSuccess)
    return fail(PG_ERROR_LAUNCH, "hipGetDevice failed");
  if (stream != nullptr) {
    int stream_device = -1;
    if (hipStreamGetDevice(stream, &stream_device) != hipSuccess)
      return fail(PG_ERROR_INVALID_ARGUMENT, "hipStreamGetDevice failed");
    if (stream_device != device)
      return fail(PG_ERROR_INVALID_ARGUMENT,
                  "the stream belongs to another device than the current one");
  }
  if (device < 0 || device >= kMaxScratchDevices)
    return fail(PG_ERROR_UNSUPPORTED, "device ordinal beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_address[device] == nullptr) {
    void* ptr = nullptr;
    const hipError_t status = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (status != hipSuccess || ptr == nullptr)
      return fail(PG_ERROR_LAUNCH, std::string("hipGetSymbolAddress(scratch) failed: ") +
                                       hipGetErrorString(status));
    g_scratch_address[device] = ptr;
  }
  *address = static_cast<int64_t*>(g_scratch_address[device]);
  return PG_OK;
}

}  // namespace
}  // namespace pg

extern "C" int64_t pg_token_major_centers_noalloc_max_bytes(void) { return kCenterScratchBytes; }

extern "C" int32_t pg_token_major_centers_noalloc(const void* key, int64_t key_token_stride,
                                                  const void* value, int64_t value_token_stride,
                                                  int64_t tokens, int32_t heads,
                                                  void* key_center, void* value_center,
                                                  void* stream) {
  clear_error();
  const int64_t need = pg_token_major_centers_workspace_bytes(tokens, heads);
  if (need > kCenterScratchBytes)
    return fail(PG_ERROR_WORKSPACE,
                "the no-allocation center reduction holds at most 8 MiB of chunk sums "
                "(tokens/64 rounded up x heads <= 4096); this call needs " +
                    std::to_string(need) + " bytes");
  int64_t* partial = nullptr;
  if (int32_t rc = center_scratch(as_stream(stream), &partial)) return rc;
  return launch_centers(key, key_token_stride, value, value_token_stride, tokens, heads,
                        key_center, value_center, partial, kCenterScratchBytes,
                        as_stream(stream));
}
