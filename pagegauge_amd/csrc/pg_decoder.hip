// Decoder-step projections for gfx950: y = W x with the neighbouring
// element-wise work fused in, for batch-1..4 decode steps.
//
// One launch replaces, per projection of a Mistral decoder layer
// (scripts/benchmark_page_gauge_transformer.py:2754-2805):
//   * MistralRMSNorm of the input (float32 mean of squares, rsqrt, FP16
//     product with the norm weight) -- prologue;
//   * F.linear with FP16 weights and float32 accumulation;
//   * SiLU(gate) * up of the fused gate/up projection -- epilogue: the
//     workgroup that computes gate row i also computes up row i + n/2;
//   * the residual add (FP16 output of the projection, then an FP16 add) --
//     epilogue;
//   * for the QKV projection, the decode step's cache update
//     (rope_append_page_gauge_dynamic / rope_append_fp16_dynamic of
//     tests/page_gauge_append_extension.cu without its page finalize): each
//     workgroup computes rows d and d + 64 of one head, rotates query and key
//     rows, centers key and value rows and writes them into their ring slot
//     -- epilogue.  The completed page's INT8 finalize runs in the decode's
//     FP16 tail pass (pg_decode_run_finalize).
//
// The work is HBM-bound weight streaming (M = batch <= 4): every weight byte
// is read once.  A workgroup (4 waves; 7 for the 14336-wide down
// projection, whose 4-chunk waves fit occupancy 5) owns a group of rows; the
// 512-element chunks of a row are split over its waves (kC consecutive
// chunks each), a
// lane reads 16 bytes of every chunk (a wave covers 1 KiB per load
// instruction, fully coalesced), and every weight load of the group is issued
// before anything else, the input included.  Each wave then loads only its
// own slice of the input into registers; the RMSNorm needs one cross-wave sum
// of squares through LDS.  Products use v_dot2_f32_f16; the wave sums meet in
// LDS and one lane per output row applies the epilogue.
#include "pg_common.h"

namespace pg {
namespace {

typedef _Float16 v8h_t __attribute__((ext_vector_type(8)));
typedef uint32_t v4u_t __attribute__((ext_vector_type(4)));

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;
constexpr int kChunk = 512;          // elements per wave-wide 16-byte load
constexpr int kUnroll = 4;           // chunks in flight per row (generic kernel)
constexpr int kMaxBatch = 4;
#ifndef PG_GEMV_MAX_BLOCKS
#define PG_GEMV_MAX_BLOCKS 2048
#endif
constexpr int kMaxBlocks = PG_GEMV_MAX_BLOCKS;   // grid cap (grid-stride beyond it)
constexpr size_t kMaxStagedBytes = 64 * 1024;   // generic kernel: input staged in LDS
// Output rows per workgroup of the blocked kernels (k = 4096 with n <= 8192
// or larger; k = 14336).  A SwiGLU workgroup loads twice as many rows.
#ifndef PG_GEMV_ROWS_4096
#define PG_GEMV_ROWS_4096 2
#endif
#ifndef PG_GEMV_ROWS_4096_LARGE
#define PG_GEMV_ROWS_4096_LARGE 4
#endif
#ifndef PG_GEMV_ROWS_14336
#define PG_GEMV_ROWS_14336 4
#endif
// Waves per workgroup for k = 14336 (28 chunks of 512 split evenly).
#ifndef PG_GEMV_WAVES_14336
#define PG_GEMV_WAVES_14336 7
#endif

// Cache update of a decode step, applied to the QKV projection's output.
struct AppendArgs {
  int query_heads;
  int kv_heads;
  const uint16_t* cosine;      // [rope_rows, 128] FP16
  const uint16_t* sine;
  int64_t rope_row_stride;
  int rope_rows;
  const int32_t* positions;    // device, positions[b * position_stride]
  int position_stride;
  uint16_t* rotated_query;     // [batch, query_heads, 128]
  uint16_t* key_pages;         // FP16 pages [pages, 16, kv_heads, 128] or the exact ring
  uint16_t* value_pages;
  const uint16_t* key_center;  // [batch, kv_heads, 128] (stride center_batch_stride); null:
  const uint16_t* value_center;//   plain FP16 pages, no centering
  int64_t center_batch_stride;
  int pages_per_request;       // FP16 pages, or exact ring pages (sink + tail) per request
  int sink_pages;              // fixed prefix pages of the ring
  int capacity_tokens;         // positions at or past it (or the RoPE table) are skipped
};

struct GemvArgs {
  const uint16_t* weight;      // [n, k] row-major FP16
  const uint16_t* x;           // [batch, x_stride]
  int64_t x_stride;
  const uint16_t* norm_weight; // [k] or null
  float eps;
  int swiglu;                  // out[i] = silu(y[i]) * y[i + n/2], i < n/2
  const uint16_t* residual;    // [batch, residual_stride] or null; may alias out
  int64_t residual_stride;
  void* out;                   // [batch, out_stride] FP16 (or float32 if out_f32)
  int64_t out_stride;
  int out_f32;
  int n;                       // weight rows
  int out_rows;                // n, or n/2 with swiglu
  int k;
  int iterations;
  AppendArgs append;
};

__device__ __forceinline__ float h2f(uint16_t b) { return half_bits_to_float(b); }
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }

// Eight FP16 products summed into a float32 accumulator (4 x v_dot2_f32_f16).
// The halves are taken from a whole-vector bit cast: bit-casting a single
// element of an ext_vector (w[e]) miscompiles on this clang (element 0 is
// used for every e).
__device__ __forceinline__ float dot8(v4u_t w, v4u_t x, float acc) {
  const v8h_t wh = __builtin_bit_cast(v8h_t, w);
  const v8h_t xh = __builtin_bit_cast(v8h_t, x);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(wh, wh, 0, 1),
                               __builtin_shufflevector(xh, xh, 0, 1), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(wh, wh, 2, 3),
                               __builtin_shufflevector(xh, xh, 2, 3), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(wh, wh, 4, 5),
                               __builtin_shufflevector(xh, xh, 4, 5), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(wh, wh, 6, 7),
                               __builtin_shufflevector(xh, xh, 6, 7), acc, false);
  return acc;
}

// Sum of squares of 8 FP16 values in float32.
__device__ __forceinline__ float squares8(v4u_t x) {
  const v8h_t h = __builtin_bit_cast(v8h_t, x);
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float f = static_cast<float>(h[e]);
    s += f * f;
  }
  return s;
}

// MistralRMSNorm of 8 values: fp16(w * fp16(x * inv)).
__device__ __forceinline__ v4u_t normalize8(v4u_t x, v4u_t w, float inv) {
  const v8h_t xh = __builtin_bit_cast(v8h_t, x);
  const v8h_t wh = __builtin_bit_cast(v8h_t, w);
  v8h_t r;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float n = static_cast<float>(static_cast<_Float16>(static_cast<float>(xh[e]) * inv));
    r[e] = static_cast<_Float16>(static_cast<float>(wh[e]) * n);
  }
  return __builtin_bit_cast(v4u_t, r);
}

// torch: F.silu(gate) (float32 math, FP16 result) * up (an FP16 product).
__device__ __forceinline__ float swiglu(float gate, float up) {
  const float act = h2f(f2h(gate / (1.0f + expf(-gate))));
  return h2f(f2h(act * up));
}

// Writes one output element: FP16 projection value (or the SwiGLU of two),
// plus the residual in FP16, widened to float32 if requested.
__device__ __forceinline__ void store_output(const GemvArgs& a, int b, int row, float y0, float y1) {
  float y = h2f(f2h(y0));
  if (a.swiglu) y = swiglu(y, h2f(f2h(y1)));
  if (a.residual != nullptr) y = h2f(f2h(h2f(a.residual[b * a.residual_stride + row]) + y));
  if (a.out_f32)
    static_cast<float*>(a.out)[b * a.out_stride + row] = y;
  else
    static_cast<uint16_t*>(a.out)[b * a.out_stride + row] = f2h(y);
}

// Weight row of the block's r-th loaded row: output rows row0.. (and, with
// SwiGLU, the matching up rows n/2 + row0..); rows past the end are clamped
// (loaded, never stored).  With the append epilogue the block's two rows are
// dims d and d + 64 of one 128-row head, d = (row0 / 2) % 64.
template <int kR, bool kRope>
__device__ __forceinline__ int loaded_row(const GemvArgs& a, int row0, int r) {
  if constexpr (kRope) {
    const int pair = row0 / 2;
    return (pair / 64) * kHeadDim + pair % 64 + 64 * r;
  }
  const int out_row = min(row0 + (r % kR), a.out_rows - 1);
  return r < kR ? out_row : out_row + a.out_rows;
}

__device__ __forceinline__ _Float16 bits_h(uint16_t b) { return __builtin_bit_cast(_Float16, b); }

// rn16(rn16(x*c) + rn16(partner*s)), the partner negated for the first half
// (the rounding sequence of tests/page_gauge_append_extension.cu:154-160).
__device__ __forceinline__ uint16_t rope_element(uint16_t x, uint16_t partner, uint16_t c,
                                                 uint16_t s, bool flip) {
#pragma clang fp contract(off)
  if (flip) partner ^= 0x8000u;
  const _Float16 primary = bits_h(x) * bits_h(c);
  const _Float16 secondary = bits_h(partner) * bits_h(s);
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(primary + secondary));
}

// fp16(float(a) - float(b))
__device__ __forceinline__ uint16_t centered(uint16_t a, uint16_t b) {
  return f2h(h2f(a) - h2f(b));
}

// Epilogue inputs of one (batch row, head pair), loaded at kernel start so
// that their latency hides under the weight stream.
struct AppendInputs {
  int position;
  bool valid;
  uint16_t cos_lo, cos_hi, sin_lo, sin_hi, center_lo, center_hi;
};

__device__ __forceinline__ AppendInputs append_inputs(const GemvArgs& g, int b, int pair) {
  const AppendArgs& a = g.append;
  AppendInputs in{};
  in.position = a.positions[b * a.position_stride];
  in.valid = in.position >= 0 && in.position < a.capacity_tokens && in.position < a.rope_rows;
  if (!in.valid) return in;
  const int h = pair / 64;
  const int d = pair % 64;
  if (h < a.query_heads + a.kv_heads) {
    const int64_t row = static_cast<int64_t>(in.position) * a.rope_row_stride;
    in.cos_lo = a.cosine[row + d];
    in.cos_hi = a.cosine[row + d + 64];
    in.sin_lo = a.sine[row + d];
    in.sin_hi = a.sine[row + d + 64];
  }
  if (h >= a.query_heads && a.key_center != nullptr) {
    const bool value = h >= a.query_heads + a.kv_heads;
    const int head = h - a.query_heads - (value ? a.kv_heads : 0);
    const uint16_t* center = (value ? a.value_center : a.key_center) + b * a.center_batch_stride +
                             head * kHeadDim;
    in.center_lo = center[d];
    in.center_hi = center[d + 64];
  }
  return in;
}

// Append epilogue for batch row b: y_lo / y_hi are dims d and d + 64 of
// head h of the QKV output (query heads, then key heads, then value heads).
__device__ void append_pair(const GemvArgs& g, int b, int pair, float y_lo, float y_hi,
                            const AppendInputs& in) {
  const AppendArgs& a = g.append;
  if (!in.valid) return;
  const int position = in.position;
  const int h = pair / 64;
  const int d = pair % 64;
  uint16_t lo = f2h(y_lo);
  uint16_t hi = f2h(y_hi);
  if (h < a.query_heads + a.kv_heads) {
    const uint16_t r_lo = rope_element(lo, hi, in.cos_lo, in.sin_lo, true);
    const uint16_t r_hi = rope_element(hi, lo, in.cos_hi, in.sin_hi, false);
    lo = r_lo;
    hi = r_hi;
  }
  if (h < a.query_heads) {
    uint16_t* q = a.rotated_query + (static_cast<int64_t>(b) * a.query_heads + h) * kHeadDim;
    q[d] = lo;
    q[d + 64] = hi;
    return;
  }
  const bool value = h >= a.query_heads + a.kv_heads;
  const int head = h - a.query_heads - (value ? a.kv_heads : 0);
  const int page = position / kPageSize;
  const int token = position % kPageSize;
  int64_t physical;
  if (a.key_center == nullptr) {
    physical = static_cast<int64_t>(b) * a.pages_per_request + page;
  } else {
    const int tail_pages = a.pages_per_request - a.sink_pages;
    const int local = page < a.sink_pages ? page : a.sink_pages + page % tail_pages;
    physical = static_cast<int64_t>(b) * a.pages_per_request + local;
    lo = centered(lo, in.center_lo);
    hi = centered(hi, in.center_hi);
  }
  uint16_t* dst = (value ? a.value_pages : a.key_pages) +
                  ((physical * kPageSize + token) * a.kv_heads + head) * kHeadDim;
  dst[d] = lo;
  dst[d + 64] = hi;
}

template <int kR, int kLoad, int kC, bool kRope>
__device__ __forceinline__ void load_rows(const GemvArgs& a, int row0, int wave, int lane,
                                          v4u_t (&wr)[kLoad][kC]) {
#pragma unroll
  for (int r = 0; r < kLoad; ++r) {
    const int row = loaded_row<kR, kRope>(a, row0, r);
    const uint16_t* w = a.weight + static_cast<int64_t>(row) * a.k + (wave * kC) * kChunk + lane * 8;
#pragma unroll
    for (int c = 0; c < kC; ++c)
      wr[r][c] = __builtin_nontemporal_load(reinterpret_cast<const v4u_t*>(w + c * kChunk));
  }
}

// Blocked kernel: k = kWaves * kC * 512.  kR output rows per workgroup
// (2*kR weight rows with SwiGLU); grid-stride over row groups when the grid
// is capped.  kRope: the append epilogue (kR = 2, rows d and d + 64 of a head).
template <int kBatch, int kR, int kC, bool kSwiglu, bool kRope = false, int kWaves = kGemvWaves>
__global__ __launch_bounds__(kWave * kWaves) void decoder_gemv_kernel(GemvArgs a) {
  static_assert(!kRope || (kR == 2 && !kSwiglu), "the append epilogue pairs two rows");
  constexpr int kLoad = kSwiglu ? 2 * kR : kR;
  __shared__ float partial[kWaves][kBatch][kLoad];
  __shared__ float squares[kWaves][kBatch];
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  v4u_t wr[kLoad][kC];
  int row0 = blockIdx.x * kR;
  if (row0 < a.out_rows) load_rows<kR, kLoad, kC, kRope>(a, row0, wave, lane, wr);
  AppendInputs append_in{};
  if constexpr (kRope) {
    // the row pair's RoPE / center inputs, loaded beside its weights
    if (threadIdx.x < kBatch && row0 < a.out_rows) append_in = append_inputs(a, threadIdx.x, row0 / 2);
  }

  // this wave's slice of the input, in registers
  v4u_t xv[kBatch][kC];
#pragma unroll
  for (int b = 0; b < kBatch; ++b) {
#pragma unroll
    for (int c = 0; c < kC; ++c)
      xv[b][c] = *reinterpret_cast<const v4u_t*>(a.x + b * a.x_stride + (wave * kC + c) * kChunk +
                                                lane * 8);
  }
  if (a.norm_weight != nullptr) {
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      float ss = 0.0f;
#pragma unroll
      for (int c = 0; c < kC; ++c) ss += squares8(xv[b][c]);
      ss = wave_sum(ss);
      if (lane == 0) squares[wave][b] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      float total = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) total += squares[w][b];
      const float inv = rsqrtf(total / static_cast<float>(a.k) + a.eps);
#pragma unroll
      for (int c = 0; c < kC; ++c) {
        const v4u_t g = *reinterpret_cast<const v4u_t*>(a.norm_weight + (wave * kC + c) * kChunk +
                                                       lane * 8);
        xv[b][c] = normalize8(xv[b][c], g, inv);
      }
    }
  }

  for (int it = 0; it < a.iterations; ++it, row0 += gridDim.x * kR) {
    if (row0 >= a.out_rows) break;                         // uniform over the block
    if (it > 0) {
      load_rows<kR, kLoad, kC, kRope>(a, row0, wave, lane, wr);
      if constexpr (kRope) {
        if (threadIdx.x < kBatch) append_in = append_inputs(a, threadIdx.x, row0 / 2);
      }
    }
    float acc[kBatch][kLoad];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
#pragma unroll
      for (int r = 0; r < kLoad; ++r) acc[b][r] = 0.0f;
    }
#pragma unroll
    for (int c = 0; c < kC; ++c) {
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
#pragma unroll
        for (int r = 0; r < kLoad; ++r) acc[b][r] = dot8(wr[r][c], xv[b][c], acc[b][r]);
      }
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
#pragma unroll
      for (int r = 0; r < kLoad; ++r) {
        const float total = wave_sum(acc[b][r]);
        if (lane == 0) partial[wave][b][r] = total;
      }
    }
    __syncthreads();
    if (kRope && threadIdx.x < kBatch) {
      const int b = threadIdx.x;
      float y0 = 0.0f, y1 = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        y0 += partial[w][b][0];
        y1 += partial[w][b][1];
      }
      append_pair(a, b, row0 / 2, y0, y1, append_in);
    } else if (!kRope && threadIdx.x < kBatch * kR) {
      const int b = threadIdx.x / kR;
      const int r = threadIdx.x % kR;
      const int row = row0 + r;
      if (row < a.out_rows) {
        float y0 = 0.0f, y1 = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          y0 += partial[w][b][r];
          if (kSwiglu) y1 += partial[w][b][kR + r];
        }
        store_output(a, b, row, y0, y1);
      }
    }
    __syncthreads();                               // partial[] is reused next iteration
  }
}

// Any k (a multiple of 512): the input staged in LDS (with the RMSNorm
// applied), one wave per output row pair (loaded rows i, i+1) or, with
// SwiGLU, per output row (loaded rows i and i + n/2), chunks streamed four
// at a time.
template <int kBatch>
__global__ __launch_bounds__(kGemvThreads) void decoder_gemv_generic_kernel(GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];   // [kBatch][k]
  __shared__ float squares[kGemvWaves];
  const int k = a.k;
  for (int b = 0; b < kBatch; ++b) {
    const uint16_t* src = a.x + b * a.x_stride;
    uint16_t* dst = xs + b * k;
    float ss = 0.0f;
    for (int i = threadIdx.x * 8; i < k; i += kGemvThreads * 8) {
      const v4u_t v = *reinterpret_cast<const v4u_t*>(src + i);
      ss += squares8(v);
      *reinterpret_cast<v4u_t*>(dst + i) = v;
    }
    if (a.norm_weight != nullptr) {
      ss = wave_sum(ss);
      __syncthreads();
      if (threadIdx.x % kWave == 0) squares[threadIdx.x / kWave] = ss;
      __syncthreads();
      float total = 0.0f;
      for (int w = 0; w < kGemvWaves; ++w) total += squares[w];
      const float inv = rsqrtf(total / static_cast<float>(k) + a.eps);
      for (int i = threadIdx.x * 8; i < k; i += kGemvThreads * 8) {
        const v4u_t g = *reinterpret_cast<const v4u_t*>(a.norm_weight + i);
        *reinterpret_cast<v4u_t*>(dst + i) = normalize8(*reinterpret_cast<v4u_t*>(dst + i), g, inv);
      }
    }
  }
  __syncthreads();
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int chunks = k / kChunk;
  const int per_wave = a.swiglu ? 1 : 2;           // output rows per wave
  for (int it = 0; it < a.iterations; ++it) {
    const int row0 = ((it * gridDim.x + blockIdx.x) * kGemvWaves + wave) * per_wave;
    if (row0 >= a.out_rows) break;
    const int second = a.swiglu ? row0 + a.out_rows : min(row0 + 1, a.out_rows - 1);
    const uint16_t* w0 = a.weight + static_cast<int64_t>(row0) * k + lane * 8;
    const uint16_t* w1 = a.weight + static_cast<int64_t>(second) * k + lane * 8;
    float acc[kBatch][2];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) acc[b][0] = acc[b][1] = 0.0f;
    for (int j = 0; j < chunks; j += kUnroll) {
      v4u_t wr[kUnroll][2];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        if (j + u < chunks) {
          wr[u][0] = __builtin_nontemporal_load(reinterpret_cast<const v4u_t*>(w0 + (j + u) * kChunk));
          wr[u][1] = __builtin_nontemporal_load(reinterpret_cast<const v4u_t*>(w1 + (j + u) * kChunk));
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        if (j + u < chunks) {
#pragma unroll
          for (int b = 0; b < kBatch; ++b) {
            const v4u_t xv = *reinterpret_cast<const v4u_t*>(xs + b * k + (j + u) * kChunk + lane * 8);
            acc[b][0] = dot8(wr[u][0], xv, acc[b][0]);
            acc[b][1] = dot8(wr[u][1], xv, acc[b][1]);
          }
        }
      }
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const float y0 = wave_sum(acc[b][0]);
      const float y1 = wave_sum(acc[b][1]);
      if (lane == 0) {
        if (a.swiglu) {
          store_output(a, b, row0, y0, y1);
        } else {
          store_output(a, b, row0, y0, 0.0f);
          if (row0 + 1 < a.out_rows) store_output(a, b, row0 + 1, y1, 0.0f);
        }
      }
    }
  }
}

template <int kBatch>
int32_t launch_gemv(GemvArgs a, hipStream_t s) {
  const int chunks = a.k / kChunk;
  auto blocked = [&](auto kernel, int rows, int waves = kGemvWaves) {
    int64_t blocks = (static_cast<int64_t>(a.out_rows) + rows - 1) / rows;
    a.iterations = static_cast<int>((blocks + kMaxBlocks - 1) / kMaxBlocks);
    blocks = (blocks + a.iterations - 1) / a.iterations;
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(kWave * waves), 0, s, a);
  };
  if (chunks == 8 && !a.swiglu) {                 // k = 4096
    if (a.out_rows > 8192)
      blocked(decoder_gemv_kernel<kBatch, PG_GEMV_ROWS_4096_LARGE, 2, false>, PG_GEMV_ROWS_4096_LARGE);
    else
      blocked(decoder_gemv_kernel<kBatch, PG_GEMV_ROWS_4096, 2, false>, PG_GEMV_ROWS_4096);
  } else if (chunks == 8) {
    blocked(decoder_gemv_kernel<kBatch, PG_GEMV_ROWS_4096, 2, true>, PG_GEMV_ROWS_4096);
  } else if (chunks == 28 && !a.swiglu) {         // k = 14336
    static_assert(28 % PG_GEMV_WAVES_14336 == 0, "k = 14336 splits into whole chunks per wave");
    constexpr int kWaves14336 = PG_GEMV_WAVES_14336;
    blocked(decoder_gemv_kernel<kBatch, PG_GEMV_ROWS_14336, 28 / kWaves14336, false, false,
                                kWaves14336>,
            PG_GEMV_ROWS_14336, kWaves14336);
  } else {
    const size_t lds = static_cast<size_t>(kBatch) * a.k * sizeof(uint16_t);
    if (lds > kMaxStagedBytes)
      return fail(PG_ERROR_UNSUPPORTED, "batch * input width exceeds the 32768-element LDS staging");
    const int per_wave = a.swiglu ? 1 : 2;
    const int64_t waves = (static_cast<int64_t>(a.out_rows) + per_wave - 1) / per_wave;
    int64_t blocks = (waves + kGemvWaves - 1) / kGemvWaves;
    a.iterations = static_cast<int>((blocks + kMaxBlocks - 1) / kMaxBlocks);
    blocks = (waves + static_cast<int64_t>(kGemvWaves) * a.iterations - 1) /
             (static_cast<int64_t>(kGemvWaves) * a.iterations);
    hipLaunchKernelGGL(decoder_gemv_generic_kernel<kBatch>, dim3(static_cast<unsigned>(blocks)),
                       dim3(kGemvThreads), lds, s, a);
  }
  return check_launch("decoder_gemv");
}

// Greedy token selection: torch.argmax over each row of float32 logits
// (the first index of the maximum; NaN counts as the largest value).
constexpr int kArgmaxThreads = 1024;
constexpr int kArgmaxUnroll = 8;     // float4 loads in flight per thread

__device__ __forceinline__ bool argmax_better(float v, int i, float bv, int bi) {
  const bool nan = v != v, bnan = bv != bv;
  if (nan != bnan) return nan;
  if (!nan && v != bv) return v > bv;
  return i < bi;
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float* x, int n,
                                                                 int64_t row_stride,
                                                                 int64_t* out) {
  __shared__ float best_v[kArgmaxThreads / kWave];
  __shared__ int best_i[kArgmaxThreads / kWave];
  const float* row = x + blockIdx.x * row_stride;
  float bv = -__builtin_huge_valf();
  int bi = n;                                     // any real index beats it on ties
  const int vec = (reinterpret_cast<uintptr_t>(row) % 16 == 0) ? n / 4 : 0;
  // kArgmaxUnroll float4 loads per thread are issued before any is compared
  // (a 32768-entry row is one such round); the selection is a total order,
  // so the visiting order does not change the result
  for (int base = 0; base < vec; base += kArgmaxThreads * kArgmaxUnroll) {
    float4 v[kArgmaxUnroll];
#pragma unroll
    for (int u = 0; u < kArgmaxUnroll; ++u) {
      const int j = base + u * kArgmaxThreads + threadIdx.x;
      v[u] = j < vec ? reinterpret_cast<const float4*>(row)[j] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < kArgmaxUnroll; ++u) {
      const int j = base + u * kArgmaxThreads + threadIdx.x;
      if (j >= vec) continue;
      const float e[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (argmax_better(e[t], 4 * j + t, bv, bi)) { bv = e[t]; bi = 4 * j + t; }
    }
  }
  for (int i = 4 * vec + threadIdx.x; i < n; i += kArgmaxThreads)
    if (argmax_better(row[i], i, bv, bi)) { bv = row[i]; bi = i; }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, kWave);
    const int oi = __shfl_xor(bi, off, kWave);
    if (argmax_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  const int wave = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) {
    best_v[wave] = bv;
    best_i[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgmaxThreads / kWave; ++w)
      if (argmax_better(best_v[w], best_i[w], bv, bi)) { bv = best_v[w]; bi = best_i[w]; }
    out[blockIdx.x] = bi < n ? bi : 0;
  }
}

#ifndef PG_QKV_MAX_BLOCKS
#define PG_QKV_MAX_BLOCKS PG_GEMV_MAX_BLOCKS
#endif

template <int kBatch>
int32_t launch_qkv_append(GemvArgs a, hipStream_t s) {
  // one row pair per workgroup and iteration; past the grid cap each
  // workgroup takes several pairs (the input RMSNorm is then computed once
  // per workgroup for all of them)
  int64_t blocks = a.out_rows / 2;
  a.iterations = static_cast<int>((blocks + PG_QKV_MAX_BLOCKS - 1) / PG_QKV_MAX_BLOCKS);
  blocks = (blocks + a.iterations - 1) / a.iterations;
  hipLaunchKernelGGL((decoder_gemv_kernel<kBatch, 2, 2, false, true>),
                     dim3(static_cast<unsigned>(blocks)), dim3(kGemvThreads), 0, s, a);
  return check_launch("decoder_qkv_rope_append");
}

}  // namespace
}  // namespace pg

using namespace pg;

extern "C" int32_t pg_decoder_gemv(const void* weight, int32_t n, int32_t k, const void* x,
                                   int64_t x_stride, int32_t batch, const void* norm_weight,
                                   float eps, int32_t swiglu, const void* residual,
                                   int64_t residual_stride, void* out, int64_t out_stride,
                                   int32_t out_f32, void* stream) {
  clear_error();
  if (weight == nullptr || x == nullptr || out == nullptr)
    return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if (n <= 0 || k <= 0 || k % kChunk)
    return fail(PG_ERROR_INVALID_ARGUMENT, "rows must be positive and the input width a multiple of 512");
  if (batch < 1 || batch > kMaxBatch)
    return fail(PG_ERROR_UNSUPPORTED, "decoder projections take a batch of 1 to 4 rows");
  if (swiglu && n % 2)
    return fail(PG_ERROR_INVALID_ARGUMENT, "a SwiGLU projection needs gate and up rows (even n)");
  const int out_rows = swiglu ? n / 2 : n;
  if (x_stride < k || x_stride % 8 || (residual != nullptr && residual_stride < out_rows) ||
      out_stride < out_rows)
    return fail(PG_ERROR_INVALID_ARGUMENT, "row strides must cover the rows (input stride a multiple of 8)");
  GemvArgs a{};
  a.weight = static_cast<const uint16_t*>(weight);
  a.x = static_cast<const uint16_t*>(x);
  a.x_stride = x_stride;
  a.norm_weight = static_cast<const uint16_t*>(norm_weight);
  a.eps = eps;
  a.swiglu = swiglu;
  a.residual = static_cast<const uint16_t*>(residual);
  a.residual_stride = residual_stride;
  a.out = out;
  a.out_stride = out_stride;
  a.out_f32 = out_f32;
  a.n = n;
  a.out_rows = out_rows;
  a.k = k;
  hipStream_t s = as_stream(stream);
  switch (batch) {
    case 1: return launch_gemv<1>(a, s);
    case 2: return launch_gemv<2>(a, s);
    case 3: return launch_gemv<3>(a, s);
    default: return launch_gemv<4>(a, s);
  }
}

extern "C" int32_t pg_decoder_qkv_rope_append(
    const void* weight, int32_t k, const void* x, int64_t x_stride, int32_t batch,
    const void* norm_weight, float eps, int32_t query_heads, int32_t kv_heads, const void* cosine,
    const void* sine, int64_t rope_row_stride, int32_t rope_rows, const int32_t* positions,
    int32_t position_stride, void* rotated_query, void* key_pages, void* value_pages,
    const void* key_center, const void* value_center, int64_t center_batch_stride,
    int32_t pages_per_request, int32_t sink_pages, int32_t capacity_tokens, void* stream) {
  clear_error();
  if (weight == nullptr || x == nullptr || cosine == nullptr || sine == nullptr ||
      positions == nullptr || rotated_query == nullptr || key_pages == nullptr ||
      value_pages == nullptr)
    return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if ((key_center == nullptr) != (value_center == nullptr))
    return fail(PG_ERROR_INVALID_ARGUMENT, "key and value centers go together");
  if (k != 8 * kChunk)
    return fail(PG_ERROR_UNSUPPORTED, "the QKV append projection takes a 4096-wide input");
  if (batch < 1 || batch > kMaxBatch)
    return fail(PG_ERROR_UNSUPPORTED, "decoder projections take a batch of 1 to 4 rows");
  if (query_heads <= 0 || kv_heads <= 0 || query_heads % kv_heads)
    return fail(PG_ERROR_INVALID_ARGUMENT, "query heads must be a positive multiple of KV heads");
  if (x_stride < k || x_stride % 8 || rope_row_stride < kHeadDim || rope_rows <= 0 ||
      position_stride < 0)
    return fail(PG_ERROR_INVALID_ARGUMENT, "row strides must cover the rows (input stride a multiple of 8)");
  if (pages_per_request <= 0 || sink_pages < 0 ||
      (key_center != nullptr && sink_pages >= pages_per_request) || capacity_tokens < 0 ||
      (key_center == nullptr && capacity_tokens > pages_per_request * kPageSize))
    return fail(PG_ERROR_INVALID_ARGUMENT, "invalid page geometry");
  if (key_center != nullptr && center_batch_stride < static_cast<int64_t>(kv_heads) * kHeadDim &&
      batch > 1)
    return fail(PG_ERROR_INVALID_ARGUMENT, "center batch stride must cover the KV heads");
  GemvArgs a{};
  a.weight = static_cast<const uint16_t*>(weight);
  a.x = static_cast<const uint16_t*>(x);
  a.x_stride = x_stride;
  a.norm_weight = static_cast<const uint16_t*>(norm_weight);
  a.eps = eps;
  a.n = (query_heads + 2 * kv_heads) * kHeadDim;
  a.out_rows = a.n;
  a.k = k;
  AppendArgs& p = a.append;
  p.query_heads = query_heads;
  p.kv_heads = kv_heads;
  p.cosine = static_cast<const uint16_t*>(cosine);
  p.sine = static_cast<const uint16_t*>(sine);
  p.rope_row_stride = rope_row_stride;
  p.rope_rows = rope_rows;
  p.positions = positions;
  p.position_stride = position_stride;
  p.rotated_query = static_cast<uint16_t*>(rotated_query);
  p.key_pages = static_cast<uint16_t*>(key_pages);
  p.value_pages = static_cast<uint16_t*>(value_pages);
  p.key_center = static_cast<const uint16_t*>(key_center);
  p.value_center = static_cast<const uint16_t*>(value_center);
  p.center_batch_stride = center_batch_stride;
  p.pages_per_request = pages_per_request;
  p.sink_pages = sink_pages;
  p.capacity_tokens = capacity_tokens;
  hipStream_t s = as_stream(stream);
  switch (batch) {
    case 1: return launch_qkv_append<1>(a, s);
    case 2: return launch_qkv_append<2>(a, s);
    case 3: return launch_qkv_append<3>(a, s);
    default: return launch_qkv_append<4>(a, s);
  }
}

extern "C" int32_t pg_argmax_f32(const float* x, int32_t rows, int32_t n, int64_t row_stride,
                                 int64_t* out, void* stream) {
  clear_error();
  if (x == nullptr || out == nullptr) return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if (rows < 1 || n < 1 || row_stride < n)
    return fail(PG_ERROR_INVALID_ARGUMENT, "argmax needs rows of at least one element");
  hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(kArgmaxThreads), 0, as_stream(stream), x, n,
                     row_stride, out);
  return check_launch("argmax");
}
