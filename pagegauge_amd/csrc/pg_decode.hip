// Paged decode for gfx950: page-affine INT8 pages + FP16 (tail) pages,
// split-KV partial softmax, base-2 LSE combine and value-center restore.
//
// Reference semantics: the PageGauge FA2 patch (page scale applied to the
// score after the QK contraction and to the value contraction,
// patches/flashinfer-0.6.17-page-gauge-int8.patch:157-249), FlashInfer's
// split merge, merge_state_in_place and add_(output_center)
// (scripts/benchmark_flashinfer_page_affine_int8.py:566-602).
//
// Design (MI355X-native, no dequantisation):
//  * One workgroup per work item (request, segment, page range); one wave64
//    per KV head; the 4 GQA query heads of a KV head share every K/V load.
//  * INT8 pages never leave the integer domain.  The query of each head is
//    turned into a 23-bit fixed-point integer (per-head power-of-two scale)
//    and split into three balanced radix-256 digits; the 4 heads x 3 digits
//    form 12 rows of one v_mfma_i32_16x16x64_i8, whose B operand is the raw
//    K code bytes.  QK is therefore exact integer arithmetic.  The same trick
//    runs PV: probabilities (already multiplied by the V page scale, fixed
//    point per 4-page group) become 3 digits per head, the V code bytes are
//    transposed in registers (v_perm) into token-major MFMA operands, and one
//    i8 MFMA per 16 output dims covers 4 pages.  Scores and partial outputs
//    are recombined from the digit rows in float32.
//  * FP16 pages (the exact tail ring, or plain FP16 pages for the same-way
//    comparison kernel) use v_mfma_f32_16x16x32_f16 for QK (query head h on
//    row 4h so every lane owns one (head, token) score) and
//    v_mfma_f32_16x16x16_f16 for PV, with each probability carried as an
//    FP16 hi/lo pair on rows 4h and 4h+1 (about 22 significant bits).
//  * Softmax state per (head): running max m (uniform across the 16 lanes of
//    a head's row), lane-partial sums l, and 8 output dims per lane.  Base-2
//    scores s*sm_scale*log2(e) (FlashInfer convention).
//  * Each work item writes an unnormalised partial (o[128], m, l) per query
//    head; the combine kernel merges a request's partials with the base-2 LSE
//    merge, divides, adds the value center and writes out/lse.
#include "pg_common.h"
#include "pg_plan.h"

#include <hip/hip_ext.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

namespace pg {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kGroupPages = 4;          // INT8 pages per PV MFMA (k = 64 tokens)
// QK contraction unit of the INT8 path: 0 = i8 MFMA (the product), 1 = VALU
// v_dot4_i32_i8 over the same query digits (an alternative build for the
// MFMA-vs-VALU comparison; same integer results).
#ifndef PG_QK_VALU
#define PG_QK_VALU 0
#endif
#if PG_QK_VALU
// P digits (1 KiB), query digit rows [4 heads][3 digits][128 B], and the
// group's K rows [4 pages][16 tokens][144 B] (rows padded by 16 B).
constexpr int kQDigitBytes = 4 * 3 * 128;
constexpr int kKRowPitch = 144;
constexpr int kLdsPerWave = 1024 + kQDigitBytes + kGroupPages * 16 * kKRowPitch;
#else
constexpr int kLdsPerWave = 1024;       // INT8 P digits: [4 pages][4 heads][4 digit rows][16 tokens]
#endif
constexpr int kCombineThreads = 256;
constexpr float kNegInf = -__builtin_huge_valf();

// Phase trace of the partial kernel (PG_TRACE builds only, an alternative
// build for bench.py --trace; the product compiles none of it).  Each wave
// records s_memrealtime (100 MHz) marks into the lanes of one register and
// writes them as one 64-word row when it ends.  A mark placed after a load
// reads a register that load fills, so it waits for the load as the
// kernel's own consume points do.  Lanes of the row:
#ifndef PG_TRACE
#define PG_TRACE 0
#endif
constexpr int kTraceStart = 0;      // first instruction of the wave
constexpr int kTraceIds = 1;        // page ids of the chunk arrived
constexpr int kTraceIssued = 2;     // first group's K/V loads issued
constexpr int kTraceScales = 3;     // page scales arrived
constexpr int kTraceK = 4;          // + g: K codes of group g (FP16: page g) arrived, g < 16
constexpr int kTraceV = 20;         // + g: V codes of INT8 group g arrived
constexpr int kTraceDone = 36;      // + g: group g's PV products issued
constexpr int kTraceEnd = 52;       // softmax state final, before the partial write
constexpr int kTraceXcc = 53;       // XCC_ID hardware register
constexpr int kTraceHwId = 54;      // HW_ID hardware register (CU, SIMD, wave slot)
constexpr int kTraceItem = 55;      // (blockIdx.x << 8) | kv head
constexpr int kTraceKind = 56;      // work item kind
constexpr int kTracePages = 57;     // pages of the chunk
constexpr int kTraceSlots = 16;     // traced groups (FP16 pages) per wave
// The combine kernel's waves write rows of the same shape after the partial
// kernel's rows (lanes 53-55 as above, lane 56 = kTraceCombineKind):
constexpr int kCTraceMeta = 1;      // value-center bits and the item range arrived
constexpr int kCTraceRows = 2;      // the partial rows (o, m, l) arrived
constexpr int kCTraceMax = 3;       // the block's maximum read back after its barrier
constexpr int kCTraceSums = 4;      // the block's sums read back after their barrier
constexpr int kCTraceEnd = 5;       // outputs stored
constexpr uint32_t kTraceCombineKind = 100;
// Alternative build for the trace's before/after only: the page-scale loads
// in the conditional form the kernel had before (each compiled to a branch
// that waits for its load before the next one leaves).
#ifndef PG_CONDITIONAL_SCALE_LOADS
#define PG_CONDITIONAL_SCALE_LOADS 0
#endif
// Alternative build for the A/B only: the KV heads of an item's workgroups
// interleaved (workgroup y of Y takes heads y, y + Y, ...) instead of in
// blocks.
#ifndef PG_INTERLEAVED_HEADS
#define PG_INTERLEAVED_HEADS 0
#endif
// Alternative build for the A/B: each K load instruction reads whole
// 128-byte rows (8 rows per instruction) and a DPP rotation hands each lane
// its MFMA operand, instead of 16 half rows per instruction.
#ifndef PG_FULL_LINE_K
#define PG_FULL_LINE_K 0
#endif

struct DecodeArgs {
  const uint16_t* query;
  int64_t query_batch_stride;
  const void* k_cache;
  const void* v_cache;
  const uint16_t* k_scale;
  const uint16_t* v_scale;
  const int32_t* indices;
  const int32_t* last_page_len;
  const uint16_t* tail_k;
  const uint16_t* tail_v;
  const int32_t* tail_indices;
  const int32_t* tail_last_len;
  const int32_t* old_kv_len;   // heterogeneous plans: INT8 tokens per request (page aligned)
  const WorkItem* items;
  float* partial_o;   // [items][Hq][128]
  float* partial_m;   // [items][Hq]
  float* partial_l;   // [items][Hq]
  int num_qo_heads;
  int num_kv_heads;
  int waves_per_block;
  int max_items;      // partial rows per (request, head)
  float sm_scale_log2;
  // one-request plans: work items from the block index (no item load)
  int closed_form;
  int cf_items;
  int cf_tail_items;
  int cf_tail_begin;
  int cf_tail_pages;
  int cf_primary_begin;
  int cf_primary_pages;
  int cf_primary_kind;
  // decode-step finalize: the FP16 tail pass quantises the page that the
  // token at finalize_positions[request * finalize_position_stride] completed
  const int32_t* finalize_positions;
  int finalize_position_stride;
  int code_pages_per_request;
  int8_t* finalize_k_codes;
  int8_t* finalize_v_codes;
  uint16_t* finalize_k_scale;
  uint16_t* finalize_v_scale;
#if PG_TRACE
  uint32_t* trace;    // [waves of the grid][64] words, or null
#endif
};

// Per-lane softmax/output state of one KV head (4 query heads).
// Lane l owns head h = l/16; o[nb] is output dim 8*(l%16) + nb.
struct HeadState {
  float m;
  float l;
  float o[8];
#if PG_TRACE
  uint32_t trace;   // lane i: trace word i
#endif
};

#if PG_TRACE
// ``word``: the wave's trace register (lane i holds trace word i)
__device__ __forceinline__ void trace_put(uint32_t& word, int slot, uint32_t value) {
  word = static_cast<int>(threadIdx.x % kWave) == slot ? value : word;
}
__device__ __forceinline__ void trace_mark(uint32_t& word, int slot) {
  uint64_t t;
  asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t) : : "memory");
  trace_put(word, slot, static_cast<uint32_t>(t));
}
__device__ __forceinline__ void trace_mark_after(uint32_t& word, int slot, uint32_t loaded) {
  uint64_t t;
  asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t) : "v"(loaded) : "memory");
  trace_put(word, slot, static_cast<uint32_t>(t));
}
__device__ __forceinline__ uint32_t trace_hwreg_xcc() {
  uint32_t x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return x;
}
__device__ __forceinline__ uint32_t trace_hwreg_id() {
  uint32_t x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(x));
  return x;
}
#define PG_TRACE_MARK(st, slot) trace_mark((st).trace, (slot))
#define PG_TRACE_AFTER(st, slot, loaded) trace_mark_after((st).trace, (slot), static_cast<uint32_t>(loaded))
#define PG_TRACE_PUT(st, slot, value) trace_put((st).trace, (slot), static_cast<uint32_t>(value))
#else
#define PG_TRACE_MARK(st, slot) ((void)0)
#define PG_TRACE_AFTER(st, slot, loaded) ((void)0)
#define PG_TRACE_PUT(st, slot, value) ((void)0)
#endif

// Full-line K loads (PG_FULL_LINE_K): lane m16 < 8 holds (own MFMA 0 data,
// MFMA 0 data of lane m16 + 8), lane m16 >= 8 (MFMA 1 data of lane m16 - 8,
// own MFMA 1 data); one 8-lane rotation within each 16-lane row sends each
// lane the half its partner holds for it.
__device__ __forceinline__ void swap_k_halves(v4i (&k)[2], bool upper) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const int send = upper ? k[0][w] : k[1][w];
    const int got = __builtin_amdgcn_mov_dpp(send, 0x128, 0xf, 0xf, false);   // row_ror:8
    k[0][w] = upper ? got : k[0][w];
    k[1][w] = upper ? k[1][w] : got;
  }
}

// 4x4 byte transpose: r[k] holds 4 dims of token k; returns c[j] holding
// dim j of tokens 0..3.  v_perm_b32(hi, lo, sel) picks byte sel_i of the
// 8-byte value {hi:lo} (bytes 0-3 = lo) for result byte i.
__device__ __forceinline__ void transpose4x4(const uint32_t r[4], uint32_t c[4]) {
  const uint32_t t0 = __builtin_amdgcn_perm(r[1], r[0], 0x05010400u);  // r0.b0 r1.b0 r0.b1 r1.b1
  const uint32_t t1 = __builtin_amdgcn_perm(r[1], r[0], 0x07030602u);  // r0.b2 r1.b2 r0.b3 r1.b3
  const uint32_t t2 = __builtin_amdgcn_perm(r[3], r[2], 0x05010400u);
  const uint32_t t3 = __builtin_amdgcn_perm(r[3], r[2], 0x07030602u);
  c[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);  // r0.b0 r1.b0 r2.b0 r3.b0
  c[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
  c[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
  c[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

// Pins ``x`` in registers at this point: uses after it cannot be hoisted
// above it, and the wait for its load is placed here (not earlier).
template <typename T>
__device__ __forceinline__ void consume_point(T& x) {
  T value = x;
  asm volatile("" : "+v"(value));
  x = value;
}

// Exponent e with 0 < v < 2^e (v > 0); 0 for v == 0.
__device__ __forceinline__ int ceil_exponent(float v) {
  int e = 0;
  if (v > 0.0f) frexpf(v, &e);
  return e;
}

__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct Int8Group {
  v4i k[4][2];      // K codes of page i: bytes 16*kg.. and 64+16*kg.. of token lane%16
  v2u v[16];        // V codes [page i][t]: dims 8*(lane%16).. of token 4*(lane/16)+t
};

// Balanced radix-256 digits of |x| < 2^22 in one step: with
// y = (x + 0x808080) ^ 0x808080, bytes 0, 1, 2 of y are the int8 digits
// d2, d1, d0 of x = 65536*d0 + 256*d1 + d2 (each in [-128, 127]).
__device__ __forceinline__ uint32_t digit_bytes(int x) {
  return static_cast<uint32_t>(x + 0x808080) ^ 0x808080u;
}

// Recombination of the three digit rows of an accumulator:
// 65536*acc.x + 256*acc.y + acc.z for |acc.x|, |acc.y|, |acc.z| < 2^24.
// Each row converts to float exactly, and the fused multiply-add rounds
// 256*acc.y + acc.z once, so the low part is the correctly rounded value of
// the exact integer.  That integer can exceed int32: the PV accumulators of
// a 64-page item sum up to 16 groups of 64 tokens x 128 x 127 < 2^24 per
// row, i.e. 256*acc.y up to 2^32.
__device__ __forceinline__ float from_digits(v4i acc) {
  const float low = fmaf(static_cast<float>(acc.y), 256.0f, static_cast<float>(acc.z));
  return static_cast<float>(acc.x) * 65536.0f + low;
}

// Online-softmax update for chunks whose first step has a visible token (so
// the running max is finite from then on and no -inf - -inf arises): masked
// scores are -inf and give p = 0, the first step's alpha is exp2(-inf) = 0.
// exp2 is the hardware v_exp_f32; results below 2^-126 flush to zero, which
// is negligible against the row maximum's 1.
template <int kCount>
__device__ __forceinline__ float softmax_update_fast(HeadState& st, const float s[kCount],
                                                     float p[kCount]) {
  float local = s[0];
#pragma unroll
  for (int i = 1; i < kCount; ++i) local = fmaxf(local, s[i]);
  const float m_new = fmaxf(st.m, row16_max(local));
  const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < kCount; ++i) {
    p[i] = __builtin_amdgcn_exp2f(s[i] - m_new);
    sum += p[i];
  }
  st.l = st.l * alpha + sum;
  st.m = m_new;
  return alpha;
}

// ---------------------------------------------------------------------------
// INT8 page-affine chunk: pages [it.page_begin, it.page_end) of one request,
// KV head ``kv``, in groups of 4 pages.  kRowStride is the byte distance of
// two token rows (Hkv*128) when known at compile time, else 0.
//
// Fixed point: the query of head h is rounded to a 23-bit integer
// q_int = rint(q * 2^qe) (|q_int| < 2^22) and split into balanced radix-256
// digits q_int = 65536*d0 + 256*d1 + d2; A rows 4h, 4h+1, 4h+2 of the QK MFMA
// hold them, row 4h+3 is zero.  Scores are
// (65536*C[4h] + 256*C[4h+1] + C[4h+2]) * 2^-qe * sm_scale*log2(e) * sK, an
// exact integer dot product up to the final float conversion.  Probabilities
// use the same three digits relative to the chunk's largest V page scale:
// P_int = rint(p * sV * 2^pe) < 2^22.
//
// PV contraction order: k-block j (lanes 16j..16j+15 of the B operand) holds
// tokens 4j..4j+3 of the group's 4 pages, k = 16j + 4t + i for token 4j+t of
// page i.  Each V load therefore reads one page (a uniform base address) and
// the P digits of one lane's four pages pack into one dword per digit.
// ---------------------------------------------------------------------------
template <int kRowStride>
__device__ __forceinline__ void int8_chunk(const DecodeArgs& a, const WorkItem& it, int kv,
                                           int lane, uint8_t* lds, HeadState& st,
                                           const int* preloaded_page = nullptr) {
  const int hkv = a.num_kv_heads;
  const int m16 = lane & 15;
  const int kg = lane >> 4;
  const int a_head = m16 >> 2;   // A-operand row 4h+c -> head h, digit c
  const int a_digit = m16 & 3;
  const int64_t row_stride = kRowStride ? kRowStride : static_cast<int64_t>(hkv) * kHeadDim;
  const int64_t page_stride = row_stride * kPageSize;
  const int8_t* kc = static_cast<const int8_t*>(a.k_cache) + kv * kHeadDim;
  const int8_t* vc = static_cast<const int8_t*>(a.v_cache) + kv * kHeadDim;

  const int begin = it.page_begin;
  const int count = it.page_end - it.page_begin;   // 1..64 (planner bound)
  const int last_slot = it.last_page - begin;      // slot of the segment's final page (may be >= count)
  const int groups = (count + kGroupPages - 1) / kGroupPages;

  // Chunk metadata, one lane per page slot: physical page and K/V page scales.
  // ``preloaded_page``: this lane's entry of a wider range starting at the
  // same page, loaded by the caller before the chunk's end was known; lanes
  // past the chunk take its last page by a select, as the clamp gives them.
  const int my_page =
      preloaded_page ? (lane < count ? *preloaded_page
                                     : __builtin_amdgcn_readlane(*preloaded_page, count - 1))
                     : a.indices[begin + min(lane, count - 1)];

  // ---- query (A operand of QK): dims 16*kg + 64*j + b, b = 0..15
  const uint16_t* q = a.query + it.request * a.query_batch_stride +
                      static_cast<int64_t>(kv * kGqa + a_head) * kHeadDim;
  v8h qraw[2][2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    qraw[j][0] = *reinterpret_cast<const v8h*>(q + 16 * kg + 64 * j);
    qraw[j][1] = *reinterpret_cast<const v8h*>(q + 16 * kg + 64 * j + 8);
  }
  const int last_len = it.segment == 0 ? a.last_page_len[it.request] : a.tail_last_len[it.request];

  // Page scales of every lane's slot, loaded unconditionally: a slot past
  // the chunk end holds the chunk's last page (the clamp above), whose scales
  // no score reads and whose V scale is already in the chunk maximum.  Both
  // loads leave together right after the index arrives and are converted
  // only after the first group's K/V loads are issued (a conditional load
  // compiles to a branch that waits for each load in turn, which put two
  // more round trips in front of the first K/V load).
#if PG_CONDITIONAL_SCALE_LOADS
  const float sk_early = lane < count ? half_bits_to_float(a.k_scale[static_cast<int64_t>(my_page) * hkv + kv]) : 0.0f;
  const float sv_early = lane < count ? half_bits_to_float(a.v_scale[static_cast<int64_t>(my_page) * hkv + kv]) : 0.0f;
  uint32_t sk_raw = 0u, sv_raw = 0u;
#else
  uint32_t sk_raw = a.k_scale[static_cast<int64_t>(my_page) * hkv + kv];
  uint32_t sv_raw = a.v_scale[static_cast<int64_t>(my_page) * hkv + kv];
#endif

  // Loads: a uniform page base plus a fixed 32-bit lane offset.  Slots past
  // the chunk end re-read its last page: their scores are masked to -inf and
  // their probabilities (hence digits) are zero.
  Int8Group buf[2];
#if PG_FULL_LINE_K
  // whole 128-byte K rows per instruction: the first load of a page takes
  // rows 0-7 (lanes m16 < 8 their own dims 16kg.., lanes m16 >= 8 dims
  // 64 + 16kg.. of row m16 - 8), the second rows 8-15; swap_k_halves then
  // trades the halves between lanes 8 apart
  const uint32_t k_off = static_cast<uint32_t>((m16 & 7) * row_stride + (m16 & 8) * 8 + 16 * kg);
  const uint32_t k_off_second = static_cast<uint32_t>(k_off + 8 * row_stride);
#else
  const uint32_t k_off = static_cast<uint32_t>(m16 * row_stride + 16 * kg);
  const uint32_t k_off_second = k_off + 64;
#endif
  const uint32_t v_off = static_cast<uint32_t>(4 * kg * row_stride + 8 * m16);
  auto issue = [&](int g, Int8Group& dst) {
    const int8_t* kp[kGroupPages];
    const int8_t* vp[kGroupPages];
#pragma unroll
    for (int i = 0; i < kGroupPages; ++i) {
      const int page = __builtin_amdgcn_readlane(my_page, min(g * kGroupPages + i, count - 1));
      kp[i] = kc + static_cast<int64_t>(page) * page_stride;
      vp[i] = vc + static_cast<int64_t>(page) * page_stride;
    }
#pragma unroll
    for (int i = 0; i < kGroupPages; ++i) {
      dst.k[i][0] = *reinterpret_cast<const v4i*>(kp[i] + k_off);
      dst.k[i][1] = *reinterpret_cast<const v4i*>(kp[i] + k_off_second);
    }
#pragma unroll
    for (int i = 0; i < kGroupPages; ++i)
#pragma unroll
      for (int t = 0; t < 4; ++t)
        dst.v[4 * i + t] = *reinterpret_cast<const v2u*>(vp[i] + v_off + t * row_stride);
  };
  PG_TRACE_AFTER(st, kTraceIds, my_page);
  issue(0, buf[0]);
  PG_TRACE_MARK(st, kTraceIssued);
  PG_TRACE_PUT(st, kTracePages, count);

  // ---- query digits (overlaps the first group's loads)
  float qmax = 0.0f;
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int b = 0; b < 8; ++b) qmax = fmaxf(qmax, fabsf(static_cast<float>(qraw[j][h][b])));
  // max over the 16 lanes sharing a_head (lane bits 0,1,4,5)
  qmax = fmaxf(qmax, __shfl_xor(qmax, 1, kWave));
  qmax = fmaxf(qmax, __shfl_xor(qmax, 2, kWave));
  qmax = fmaxf(qmax, __shfl_xor(qmax, 16, kWave));
  qmax = fmaxf(qmax, __shfl_xor(qmax, 32, kWave));
  const int q_exp = 22 - ceil_exponent(qmax);   // |q| * 2^q_exp < 2^22
  // this lane's digit is byte 2 - a_digit of the digit bytes (row 3 is zero);
  // the selector packs it from two words into bytes 0, 1 (0x0c selects zero)
  const uint32_t q_byte = a_digit == 3 ? 0u : static_cast<uint32_t>(2 - a_digit);
  const uint32_t q_sel = q_byte | ((q_byte + 4u) << 8) | 0x0c0c0000u;
  v4i qd[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    int packed[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t y[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int e = 4 * w + b;
        const float qf = static_cast<float>(qraw[j][e >> 3][e & 7]);
        y[b] = digit_bytes(static_cast<int>(rintf(ldexpf(qf, q_exp))));
      }
      // byte b of the word = the selected digit byte of y[b]
      const uint32_t lo = __builtin_amdgcn_perm(y[1], y[0], q_sel);
      const uint32_t hi = __builtin_amdgcn_perm(y[3], y[2], q_sel);
      packed[w] = a_digit == 3 ? 0 : static_cast<int>(lo | (hi << 16));
    }
    qd[j] = v4i{packed[0], packed[1], packed[2], packed[3]};
  }
  // score scale for this lane's C row (head kg): 2^-q_exp(head kg) * sm_scale*log2e
  const float qscale = ldexpf(a.sm_scale_log2, -__shfl(q_exp, 4 * kg, kWave));
  // the V scale's chunk maximum fixes the probability fixed point for the
  // whole chunk
  consume_point(sk_raw);
  consume_point(sv_raw);
  PG_TRACE_AFTER(st, kTraceScales, sv_raw);
#if PG_CONDITIONAL_SCALE_LOADS
  const float my_sk = sk_early;
  const float my_sv = sv_early;
#else
  const float my_sk = half_bits_to_float(static_cast<uint16_t>(sk_raw));
  const float my_sv = half_bits_to_float(static_cast<uint16_t>(sv_raw));
#endif
  float vmax = my_sv;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) vmax = fmaxf(vmax, __shfl_xor(vmax, off, kWave));
  const int p_exp = 22 - ceil_exponent(vmax);      // p*sV*2^p_exp < 2^22 since p <= 1
  const float inv_p = ldexpf(1.0f, -p_exp);
  const float my_svu = ldexpf(my_sv, p_exp);       // sV * 2^p_exp of this lane's page slot

#if PG_QK_VALU
  // query digit rows for the VALU contraction: row 3h+c holds digit c of head h
  uint8_t* q_lds = lds + 1024;
  uint8_t* k_lds = lds + 1024 + kQDigitBytes;
  if (a_digit < 3) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
      *reinterpret_cast<v4i*>(q_lds + (a_head * 3 + a_digit) * 128 + 16 * kg + 64 * j) = qd[j];
  }
#endif
  // zero the wave's digit buffer once: digit row 3 of every head stays zero
  *reinterpret_cast<uint4*>(lds + 16 * lane) = uint4{0u, 0u, 0u, 0u};
  wave_lds_fence();
  // P digit writes: lane (head kg, token m16) -> rows 4*kg + c of k-block m16/4,
  // bytes 4*(m16%4) .. +3 (pages 0..3)
  uint32_t* p_dst = reinterpret_cast<uint32_t*>(lds + ((m16 >> 2) * 16 + 4 * kg) * 16 + 4 * (m16 & 3));
  const v4i* p_src = reinterpret_cast<const v4i*>(lds + (kg * 16 + m16) * 16);

  // PV partial sums stay in the MFMA accumulators (exact int32) while the
  // running max is unchanged; they are folded into st.o when it rises and at
  // the end.  Per digit row and group the sum is below 64 tokens * 128 * 127
  // < 2^20, so 16 groups (the 64-page chunk bound) stay below 2^24: each row
  // is exact in float, and from_digits recombines the rows in float (256 x
  // the middle row alone can pass 2^31).
  v4i pv[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) pv[nb] = v4i{0, 0, 0, 0};
  auto fold = [&](float scale) {
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      st.o[nb] = (st.o[nb] + from_digits(pv[nb]) * inv_p) * scale;
      pv[nb] = v4i{0, 0, 0, 0};
    }
  };

  auto compute = [&](int g, Int8Group& cur) {
#pragma unroll
    for (int i = 0; i < kGroupPages; ++i) {
      consume_point(cur.k[i][0]);
      consume_point(cur.k[i][1]);
    }
    if (PG_TRACE && g < kTraceSlots) PG_TRACE_AFTER(st, kTraceK + g, cur.k[kGroupPages - 1][1][3]);
#if PG_FULL_LINE_K
#pragma unroll
    for (int i = 0; i < kGroupPages; ++i) swap_k_halves(cur.k[i], m16 >= 8);
#endif
    // ---- QK: exact integer dot products
    float s[kGroupPages];
    float svu[kGroupPages];
#if PG_QK_VALU
    // the K rows go through LDS so that lane (head kg, token m16) sees the
    // whole row of its token; 3 digit dots per page with v_dot4_i32_i8
    int dots[kGroupPages][3];
#pragma unroll
    for (int i = 0; i < kGroupPages; ++i) {
      *reinterpret_cast<v4i*>(k_lds + (i * 16 + m16) * kKRowPitch + 16 * kg) = cur.k[i][0];
      *reinterpret_cast<v4i*>(k_lds + (i * 16 + m16) * kKRowPitch + 64 + 16 * kg) = cur.k[i][1];
#pragma unroll
      for (int c = 0; c < 3; ++c) dots[i][c] = 0;
    }
    wave_lds_fence();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v4i qv[3];
#pragma unroll
      for (int c = 0; c < 3; ++c) qv[c] = *reinterpret_cast<const v4i*>(q_lds + (kg * 3 + c) * 128 + 16 * j);
#pragma unroll
      for (int i = 0; i < kGroupPages; ++i) {
        const v4i kr = *reinterpret_cast<const v4i*>(k_lds + (i * 16 + m16) * kKRowPitch + 16 * j);
#pragma unroll
        for (int c = 0; c < 3; ++c)
#pragma unroll
          for (int w = 0; w < 4; ++w) dots[i][c] = __builtin_amdgcn_sdot4(qv[c][w], kr[w], dots[i][c], false);
      }
    }
    wave_lds_fence();
#endif
#pragma unroll
    for (int i = 0; i < kGroupPages; ++i) {
#if PG_QK_VALU
      const v4i acc = {dots[i][0], dots[i][1], dots[i][2], 0};
#else
      v4i acc = {0, 0, 0, 0};
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qd[0], cur.k[i][0], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qd[1], cur.k[i][1], acc, 0, 0, 0);
#endif
      const int slot = g * kGroupPages + i;
      const int ls = min(slot, count - 1);
      const float sk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_sk), ls));
      svu[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_svu), ls));
      // visible tokens of this slot: 16, last_len on the segment's final
      // page, 0 past the chunk end (uniform)
      const int lim = slot < count ? (slot == last_slot ? last_len : kPageSize) : 0;
      const float score = from_digits(acc) * (qscale * sk);
      s[i] = m16 < lim ? score : kNegInf;
    }
    float p[kGroupPages];
    const float alpha = softmax_update_fast<kGroupPages>(st, s, p);
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) fold(alpha);

    // ---- P digits: one dword per digit row holds this token's 4 pages
    uint32_t y[4];
#pragma unroll
    for (int i = 0; i < kGroupPages; ++i) y[i] = digit_bytes(static_cast<int>(rintf(p[i] * svu[i])));
    uint32_t dig[4];
    transpose4x4(y, dig);          // dig[b] = digit byte b of pages 0..3
    p_dst[0] = dig[2];             // row 4h:   d0 (weight 65536)
    p_dst[4] = dig[1];             // row 4h+1: d1 (weight 256)
    p_dst[8] = dig[0];             // row 4h+2: d2
    wave_lds_fence();
    const v4i pa = *p_src;
    wave_lds_fence();

    // ---- PV: V bytes of token 4*kg+t of the 4 pages transposed to one
    // dword per output dim; n-block nb covers output dim 8*(lane%16) + nb
#pragma unroll
    for (int i = 0; i < 16; ++i) consume_point(cur.v[i]);
    if (PG_TRACE && g < kTraceSlots) PG_TRACE_AFTER(st, kTraceV + g, cur.v[15][1]);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      uint32_t cols[4][4];   // [dim j][token t]
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t r[4] = {cur.v[t][half], cur.v[4 + t][half], cur.v[8 + t][half],
                               cur.v[12 + t][half]};
        uint32_t c[4];
        transpose4x4(r, c);
#pragma unroll
        for (int j = 0; j < 4; ++j) cols[j][t] = c[j];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const v4i bop = {static_cast<int>(cols[j][0]), static_cast<int>(cols[j][1]),
                         static_cast<int>(cols[j][2]), static_cast<int>(cols[j][3])};
        pv[4 * half + j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, bop, pv[4 * half + j], 0, 0, 0);
      }
    }
    if (PG_TRACE && g < kTraceSlots) PG_TRACE_MARK(st, kTraceDone + g);
  };

  // Software pipeline: the loads of group g+1 are in flight while group g is
  // computed; consume_point keeps the compiler from pulling g+1's uses (and
  // their waits) into iteration g, and places the wait for V after QK and
  // the softmax.  The steady-state loop has no branches around loads; the
  // last one or two groups are peeled.
  int g = 0;
  for (; g + 2 < groups; g += 2) {
    issue(g + 1, buf[1]);
    compute(g, buf[0]);
    issue(g + 2, buf[0]);
    compute(g + 1, buf[1]);
  }
  if (g + 1 < groups) {
    issue(g + 1, buf[1]);
    compute(g, buf[0]);
    compute(g + 1, buf[1]);
  } else {
    compute(g, buf[0]);
  }
  fold(1.0f);
}

// ---------------------------------------------------------------------------
// FP16 chunk (tail ring or plain FP16 pages), one page per step.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t word_of(v4u v, int i) { return v[i]; }

// Sign-symmetric rounding of x / scale to [-127, 127] and the stored page
// scale fp16(max(|x|max / 127, 2^-20)): the cache update's finalize
// (tests/page_gauge_append_extension.cu:327-382).
__device__ __forceinline__ uint32_t symmetric_code_byte(float quotient) {
  int code = quotient >= 0.0f ? static_cast<int>(floorf(quotient + 0.5f))
                              : -static_cast<int>(floorf(-quotient + 0.5f));
  code = max(-127, min(127, code));
  return static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(code)));
}

__device__ __forceinline__ uint16_t finalize_scale_bits(float maximum) {
  return __half_as_ushort(__float2half_rn(fmaxf(maximum / 127.0f, 0x1p-20f)));
}

// Codes of 8 FP16 values (two dwords of 4 codes).
__device__ __forceinline__ v2u codes8(const _Float16 (&x)[8], float scale) {
  uint32_t w[2] = {0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e)
    w[e >> 2] |= symmetric_code_byte(static_cast<float>(x[e]) / scale) << (8 * (e & 3));
  return v2u{w[0], w[1]};
}

// Finalize of one completed page from the FP16 pass's registers: k[j] holds
// K row m16, dims 32j + 8kg .. +7; v[r] holds V row 4kg + r, dims 8*m16 .. +7
// (the whole 16 x 128 block of this wave's head).  Writes the INT8 codes and
// the two page scales of code page ``page`` of ``request``.
__device__ void finalize_page(const DecodeArgs& a, int request, int page, int kv, int lane,
                              const v8h (&k)[4], const v4u (&v)[4]) {
  const int m16 = lane & 15;
  const int kg = lane >> 4;
  _Float16 kx[4][8], vx[4][8];
  float kmax = 0.0f, vmax = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const v8h kb = k[j];
    const v8h vb = __builtin_bit_cast(v8h, v[j]);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      kx[j][e] = kb[e];
      vx[j][e] = vb[e];
      kmax = fmaxf(kmax, fabsf(static_cast<float>(kx[j][e])));
      vmax = fmaxf(vmax, fabsf(static_cast<float>(vx[j][e])));
    }
  }
  const uint16_t k_bits = finalize_scale_bits(wave_max(kmax));
  const uint16_t v_bits = finalize_scale_bits(wave_max(vmax));
  const float k_scale = half_bits_to_float(k_bits);
  const float v_scale = half_bits_to_float(v_bits);
  const int hkv = a.num_kv_heads;
  const int64_t row_stride = static_cast<int64_t>(hkv) * kHeadDim;
  const int64_t code_page = static_cast<int64_t>(request) * a.code_pages_per_request + page;
  int8_t* kc = a.finalize_k_codes + (code_page * kPageSize + m16) * row_stride + kv * kHeadDim + 8 * kg;
  int8_t* vc = a.finalize_v_codes + (code_page * kPageSize + 4 * kg) * row_stride + kv * kHeadDim +
               8 * m16;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    *reinterpret_cast<v2u*>(kc + 32 * j) = codes8(kx[j], k_scale);
    *reinterpret_cast<v2u*>(vc + j * row_stride) = codes8(vx[j], v_scale);
  }
  if (lane == 0) {
    a.finalize_k_scale[code_page * hkv + kv] = k_bits;
    a.finalize_v_scale[code_page * hkv + kv] = v_bits;
  }
}

// kStrided: ``subs`` waves share one (request, KV head), and wave ``sub``
// takes pages sub, sub + subs, ... of the range into its own state (the
// caller merges the states); otherwise the wave takes every page.
template <bool kStrided = false>
__device__ __forceinline__ void fp16_pages(const DecodeArgs& a, int request, const uint16_t* kpages,
                                           const uint16_t* vpages, const int32_t* indices,
                                           int begin, int end, int last_page, int last_len,
                                           int kv, int lane, uint8_t* lds, HeadState& st,
                                           int sub = 0, int subs = 1) {
  if (!kStrided) {
    sub = 0;
    subs = 1;
  }
  const int hkv = a.num_kv_heads;
  const int m16 = lane & 15;
  const int kg = lane >> 4;
  const int64_t row_stride = static_cast<int64_t>(hkv) * kHeadDim;  // elements
  const uint16_t* kp = kpages + kv * kHeadDim;
  const uint16_t* vp = vpages + kv * kHeadDim;
  const int count = end - begin;        // 1..64 (planner bound)
  const int last_slot = last_page - begin;
  // Unconditional loads (a lane past the range re-reads its last page id;
  // every lane reads its head's query row): a conditional load compiles to
  // a branch that waits for it before the next load can leave.
  const int my_page = indices[begin + min(lane, count - 1)];
  // the decode step's position, when this pass finalizes a completed page:
  // loaded here (from a valid address either way) and consumed at the last
  // page, where a load would be one more round trip
  const bool finalizing = a.finalize_positions != nullptr;
  const int32_t* position_at =
      finalizing ? a.finalize_positions + request * a.finalize_position_stride : indices + begin;
  int finalize_position = *position_at;

  // Q operand: head h on row 4h; lanes of other rows hold zeros.
  v8h qa[4];
  const bool q_row = (m16 & 3) == 0;
  const uint16_t* q = a.query + request * a.query_batch_stride +
                      static_cast<int64_t>(kv * kGqa + (m16 >> 2)) * kHeadDim;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const v8h row = *reinterpret_cast<const v8h*>(q + 32 * j + 8 * kg);
    qa[j] = q_row ? row : v8h{0, 0, 0, 0, 0, 0, 0, 0};
  }
  uint16_t* plds = reinterpret_cast<uint16_t*>(lds);   // [4 heads][2 parts][16 tokens] fp16

  struct Fp16Page {
    v8h k[4];    // K row of token lane%16: halves 32*j + 8*kg .. +7
    v4u v[4];    // V: dims 8*m16 .. +7 of tokens 4*kg + k
  };
  Fp16Page buf[2];
  auto issue = [&](int local, Fp16Page& dst) {
    const int page = __builtin_amdgcn_readlane(my_page, sub + local * subs);
    const uint16_t* kbase = kp + (static_cast<int64_t>(page) * kPageSize + m16) * row_stride + 8 * kg;
#pragma unroll
    for (int j = 0; j < 4; ++j) dst.k[j] = *reinterpret_cast<const v8h*>(kbase + 32 * j);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint16_t* vbase =
          vp + (static_cast<int64_t>(page) * kPageSize + 4 * kg + k) * row_stride + 8 * m16;
      dst.v[k] = *reinterpret_cast<const v4u*>(vbase);
    }
  };

  // PV sums accumulate in the MFMA accumulators (rows 4h: hi part, 4h+1: lo
  // part) and are folded into st.o when the running max rises and at the end.
  v4f pv[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) pv[nb] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  auto fold = [&](float scale) {
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      st.o[nb] = (st.o[nb] + pv[nb].x + pv[nb].y) * scale;
      pv[nb] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };

  auto compute = [&](int local, Fp16Page& cur) {
    const int slot = sub + local * subs;
#pragma unroll
    for (int j = 0; j < 4; ++j) consume_point(cur.k[j]);
#pragma unroll
    for (int k = 0; k < 4; ++k) consume_point(cur.v[k]);
    if (PG_TRACE && local < kTraceSlots) PG_TRACE_AFTER(st, kTraceK + local, cur.v[3][3]);
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[j], cur.k[j], acc, 0, 0, 0);
    if (finalizing && slot == last_slot) {
      // the step's token completed this (the segment's last) page
      consume_point(finalize_position);
      const int position = finalize_position;
      if (position >= 0 && position % kPageSize == kPageSize - 1 &&
          position / kPageSize < a.code_pages_per_request)
        finalize_page(a, request, position / kPageSize, kv, lane, cur.k, cur.v);
    }
    const int lim = slot == last_slot ? last_len : kPageSize;
    if (lim < kPageSize) {
      // rows past the last token: zero V so that p = 0 cannot meet a NaN or
      // Inf left in unused ring rows
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (4 * kg + k >= lim) cur.v[k] = v4u{0u, 0u, 0u, 0u};
    }
    const float score = acc.x * a.sm_scale_log2;
    float s[1] = {m16 < lim ? score : kNegInf};
    float p[1];
    const float alpha = softmax_update_fast<1>(st, s, p);
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) fold(alpha);

    // P as an FP16 hi/lo pair (p = hi + lo to ~22 bits) -> LDS [head][part][token];
    // A operand rows 4h (hi) and 4h+1 (lo) read 4 tokens each, rows 4h+2/3 are 0.
    const _Float16 p_hi = static_cast<_Float16>(p[0]);
    const _Float16 p_lo = static_cast<_Float16>(p[0] - static_cast<float>(p_hi));
    plds[(kg * 2) * 16 + m16] = __builtin_bit_cast(uint16_t, p_hi);
    plds[(kg * 2 + 1) * 16 + m16] = __builtin_bit_cast(uint16_t, p_lo);
    wave_lds_fence();
    v4h pa = v4h{0, 0, 0, 0};
    if ((m16 & 3) < 2)
      pa = *reinterpret_cast<const v4h*>(plds + ((m16 >> 2) * 2 + (m16 & 1)) * 16 + 4 * kg);
    wave_lds_fence();

#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      const int dw = nb >> 1;
      const uint32_t sel = (nb & 1) ? 0x07060302u : 0x05040100u;
      // (token 4kg, token 4kg+1) and (4kg+2, 4kg+3) halves of dim 8*m16+nb
      const uint32_t p01 = __builtin_amdgcn_perm(word_of(cur.v[1], dw), word_of(cur.v[0], dw), sel);
      const uint32_t p23 = __builtin_amdgcn_perm(word_of(cur.v[3], dw), word_of(cur.v[2], dw), sel);
      const v4h bop = __builtin_shufflevector(__builtin_bit_cast(v2h, p01),
                                              __builtin_bit_cast(v2h, p23), 0, 1, 2, 3);
      pv[nb] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, bop, pv[nb], 0, 0, 0);
    }
  };

  const int local_count = kStrided ? (count - sub + subs - 1) / subs : count;   // this wave's pages
  if (kStrided && local_count <= 0) return;
  PG_TRACE_AFTER(st, kTraceIds, my_page);
  issue(0, buf[0]);
  PG_TRACE_MARK(st, kTraceIssued);
  PG_TRACE_PUT(st, kTracePages, count);
  int slot = 0;
  for (; slot + 2 < local_count; slot += 2) {
    issue(slot + 1, buf[1]);
    compute(slot, buf[0]);
    issue(slot + 2, buf[0]);
    compute(slot + 1, buf[1]);
  }
  if (slot + 1 < local_count) {
    issue(slot + 1, buf[1]);
    compute(slot, buf[0]);
    compute(slot + 1, buf[1]);
  } else {
    compute(slot, buf[0]);
  }
  fold(1.0f);
}

// ---------------------------------------------------------------------------
// Combine: block (request*Hq + head, dim quarter); 256 threads = 32 item rows
// x 8 float4 columns, so one pass loads 32 partials of 32 dims in parallel.
// ---------------------------------------------------------------------------
constexpr int kCombineRows = 32;
constexpr int kCombineCols = 8;      // float4 columns = 32 dims
constexpr int kCombineInRegs = 8;   // item rows per thread held in registers (256 items)

struct CombineArgs {
  const float* partial_o;
  const float* partial_m;
  const float* partial_l;
  const int32_t* item_ptr;
  const uint16_t* value_center;
  int64_t center_batch_stride;
  uint16_t* out;
  float* lse;
  int num_qo_heads;
  int max_items;
  int uniform_items;   // > 0: every request has this many items (no item_ptr read)
#if PG_TRACE
  uint32_t* trace;     // [waves of the combine grid][64] words, or null
#endif
};

__device__ __forceinline__ void fma4(float4& acc, float w, const float4& v) {
  acc.x += w * v.x;
  acc.y += w * v.y;
  acc.z += w * v.z;
  acc.w += w * v.w;
}

// The output of a combine: total * inv + center as one f32 fma, rounded to
// f32 and then to FP16.  The empty asm makes the f32 value opaque, so that
// the compiler cannot fold the FP16 rounding into a mixed-precision fma (one
// rounding) in one combine kernel and not in the other: with it both return
// the same bits for the same partials.
__device__ __forceinline__ float combine_output(float total, float inv, float center) {
  float o = __builtin_fmaf(total, inv, center);
  asm volatile("" : "+v"(o));
  return o;
}

// Merges the partials of (request, query head) for dims 32*quarter.. +31 and
// writes out/lse; ``tid`` in [0, 256).  Every wave works alone (no LDS, no
// barrier): wave w owns float4 columns 2w and 2w + 1.
//
// One memory round trip: the partial rows are loaded for the plan's largest
// item count while the request's own count is loaded; rows past the count
// are dropped by selects (they may hold anything).  DPP row q of a wave holds
// column 2w + q/2 and the item rows of half h = q % 2: lane i of the row
// accumulates rows i + 16h + 32k, k = 0, 1, ... in order, and the row's 16
// lanes reduce by DPP rotations (the tree that row16_sum forms at lane 0).
// The two halves of a column sit 16 lanes apart, so the maximum over all
// rows and the sum of the two half totals take one swap of 16 lanes each.
// That is the association combine_rows_kernel also keeps: per item w*o (one
// rounding), the 16-lane tree over each half, then the sum of the halves.
__device__ __forceinline__ void combine_unit(const CombineArgs& a, int row_head, int quarter,
                                             int tid, uint32_t& trace) {
  const int request = row_head / a.num_qo_heads;
  const int qh = row_head % a.num_qo_heads;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int q = lane >> 4;
  const int c = 2 * wave + (q >> 1);
  const int r = (lane & 15) + 16 * (q & 1);
  const int dim = 32 * quarter + 4 * c;
  const int64_t base = static_cast<int64_t>(row_head) * a.max_items;
  const float* pm = a.partial_m + base;
  const float* pl = a.partial_l + base;
  const float* po = a.partial_o + base * kHeadDim + dim;

  // The value center: every lane loads the 8-byte slice of its column
  // unconditionally (with no center, the first 8 bytes of this row's
  // partials, whose bits are dropped) and converts it only after the partial
  // rows are requested.  A conditional load compiles to a branch that waits
  // for it, which put a whole round trip in front of the partial loads.
  const bool has_center = a.value_center != nullptr;
  const uint16_t* cv = has_center
                           ? a.value_center + request * a.center_batch_stride +
                                 (qh / kGqa) * kHeadDim + dim
                           : reinterpret_cast<const uint16_t*>(a.partial_o + base * kHeadDim);
  uint2 center_bits = *reinterpret_cast<const uint2*>(cv);
  // the request's item count, used only after the rows are requested
  int item_begin = a.item_ptr[request];
  int item_end = a.item_ptr[request + 1];
  float4 ov[kCombineInRegs];
  float mv[kCombineInRegs], lv[kCombineInRegs];
#pragma unroll
  for (int k = 0; k < kCombineInRegs; ++k) {
    const int j = r + k * kCombineRows;
    const bool planned = j < a.max_items;
    ov[k] = planned ? *reinterpret_cast<const float4*>(po + static_cast<int64_t>(j) * kHeadDim)
                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    mv[k] = planned ? pm[j] : kNegInf;
    lv[k] = planned ? pl[j] : 0.0f;
  }
  consume_point(center_bits.x);   // waits for the center and the count here, the rows in flight
  consume_point(center_bits.y);
  consume_point(item_begin);
  consume_point(item_end);
#if PG_TRACE
  trace_mark_after(trace, kCTraceMeta, center_bits.y ^ static_cast<uint32_t>(item_end));
  trace_mark_after(trace, kCTraceRows, __float_as_uint(ov[kCombineInRegs - 1].w));
  trace_mark_after(trace, kCTraceRows, __float_as_uint(mv[kCombineInRegs - 1]));
  trace_mark_after(trace, kCTraceRows, __float_as_uint(lv[kCombineInRegs - 1]));
#endif
  const int count = a.uniform_items > 0 ? a.uniform_items : item_end - item_begin;
  float center4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (has_center) {
    center4[0] = half_bits_to_float(static_cast<uint16_t>(center_bits.x));
    center4[1] = half_bits_to_float(static_cast<uint16_t>(center_bits.x >> 16));
    center4[2] = half_bits_to_float(static_cast<uint16_t>(center_bits.y));
    center4[3] = half_bits_to_float(static_cast<uint16_t>(center_bits.y >> 16));
  }
  float local_max = kNegInf;
#pragma unroll
  for (int k = 0; k < kCombineInRegs; ++k) {
    const bool in = r + k * kCombineRows < count;
    mv[k] = in ? mv[k] : kNegInf;
    local_max = fmaxf(local_max, mv[k]);
  }
  for (int j = r + kCombineInRegs * kCombineRows; j < count; j += kCombineRows)
    local_max = fmaxf(local_max, pm[j]);
  local_max = row16_max(local_max);
  // the other half's maximum, 16 lanes away (the maximum is exact in any order)
  const float m = fmaxf(local_max, __shfl_xor(local_max, 16, kWave));
#if PG_TRACE
  trace_mark_after(trace, kCTraceMax, __float_as_uint(m));
#endif

  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  float lsum = 0.0f;
#pragma unroll
  for (int k = 0; k < kCombineInRegs; ++k) {
    const bool in = r + k * kCombineRows < count;
    const float w = (in && mv[k] != kNegInf) ? __builtin_amdgcn_exp2f(mv[k] - m) : 0.0f;
    if (in) {
      fma4(acc, w, ov[k]);
      lsum += w * lv[k];
    }
  }
  for (int j = r + kCombineInRegs * kCombineRows; j < count; j += kCombineRows) {
    const float mj = pm[j];
    const float w = mj == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(mj - m);
    fma4(acc, w, *reinterpret_cast<const float4*>(po + static_cast<int64_t>(j) * kHeadDim));
    lsum += w * pl[j];
  }
  acc.x = row16_sum(acc.x);
  acc.y = row16_sum(acc.y);
  acc.z = row16_sum(acc.z);
  acc.w = row16_sum(acc.w);
  lsum = row16_sum(lsum);
  // half 0 + half 1 (IEEE addition commutes, so both rows of the pair hold
  // the same bits); lane 0 of each row holds its 16-lane tree
  const float4 total = make_float4(acc.x + __shfl_xor(acc.x, 16, kWave),
                                   acc.y + __shfl_xor(acc.y, 16, kWave),
                                   acc.z + __shfl_xor(acc.z, 16, kWave),
                                   acc.w + __shfl_xor(acc.w, 16, kWave));
  const float l = lsum + __shfl_xor(lsum, 16, kWave);
#if PG_TRACE
  trace_mark_after(trace, kCTraceSums, __float_as_uint(l) ^ __float_as_uint(total.x));
#endif
  if ((lane & 31) == 0) {
    // lane 0 of DPP row 0 (column 2w) and of row 2 (column 2w + 1)
    const bool empty = !(l > 0.0f);
    const float inv = empty ? 0.0f : 1.0f / l;
    const float o4[4] = {combine_output(total.x, inv, center4[0]),
                         combine_output(total.y, inv, center4[1]),
                         combine_output(total.z, inv, center4[2]),
                         combine_output(total.w, inv, center4[3])};
    uint16_t* out = a.out + static_cast<int64_t>(row_head) * kHeadDim + dim;
    *reinterpret_cast<__half2*>(out) = __floats2half2_rn(o4[0], o4[1]);
    *reinterpret_cast<__half2*>(out + 2) = __floats2half2_rn(o4[2], o4[3]);
    if (tid == 0 && quarter == 0 && a.lse != nullptr)
      a.lse[row_head] = empty ? kNegInf : log2f(l) + m;
  }
}

__global__ __launch_bounds__(kCombineThreads) void combine_kernel(CombineArgs a) {
  uint32_t trace = 0;
#if PG_TRACE
  trace_mark(trace, kTraceStart);
#endif
  combine_unit(a, blockIdx.x, blockIdx.y, threadIdx.x, trace);
#if PG_TRACE
  if (a.trace != nullptr) {
    trace_mark(trace, kCTraceEnd);
    trace_put(trace, kTraceXcc, trace_hwreg_xcc());
    trace_put(trace, kTraceHwId, trace_hwreg_id());
    trace_put(trace, kTraceItem, (blockIdx.x << 8) | blockIdx.y);
    trace_put(trace, kTraceKind, kTraceCombineKind);
    const int64_t w = (static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x) *
                          (kCombineThreads / kWave) + threadIdx.x / kWave;
    a.trace[w * kWave + threadIdx.x % kWave] = trace;
  }
#endif
}

// ---------------------------------------------------------------------------
// Combine for plans of at most 32 items per request (large batches of short
// requests): one wave per (request, query head) row, lane l holding dims 2l
// and 2l + 1, four rows per workgroup, no LDS and no barrier.  The grid is a
// quarter of the rows instead of four workgroups per row, so a batch of
// thousands of rows fits in one wave of workgroups.
//
// The sums keep combine_unit's association, so both kernels return the same
// bits for the same partials (and a request's output does not depend on
// which kernel its batch selects): per item w*o (one rounding), the 16-row
// tree of row16_sum over items 0-15 and over items 16-31 (at a DPP row's
// lane 0: pairs 8 apart, then 4, 2 and 1 apart; IEEE addition commutes, so
// the rotation direction does not matter), then their sum.
// ---------------------------------------------------------------------------
constexpr int kCombineRowsMaxItems = kCombineRows;   // 32
// Below this many (request, query head) rows the four-workgroup kernel's
// wider spread of loads wins over the row kernel's one wave per row (cold
// calls: the four-workgroup kernel was faster up to B8, the row kernel from
// B16 on, by more the larger the batch).
#ifndef PG_COMBINE_ROWS_MIN_ROWS
#define PG_COMBINE_ROWS_MIN_ROWS 512
#endif
constexpr int kCombineRowsMinRows = PG_COMBINE_ROWS_MIN_ROWS;
constexpr int kCombineRowsPerBlock = kCombineThreads / kWave;

// lane 0 of row16_sum over a[0..15]
__device__ __forceinline__ float tree16(const float* a) {
  float s1[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) s1[i] = a[i] + a[i + 8];
  float s2[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) s2[i] = s1[i] + s1[i + 4];
  return (s2[0] + s2[2]) + (s2[1] + s2[3]);
}

// kSlots (8, 16 or 32) >= the plan's largest item count: item rows past it
// enter the trees as the +0 terms combine_unit's empty rows give.
template <int kSlots>
__global__ __launch_bounds__(kCombineThreads) void combine_rows_kernel(CombineArgs a, int rows) {
  static_assert(kSlots <= kCombineRowsMaxItems, "one 32-row pass");
  const int row_head = blockIdx.x * kCombineRowsPerBlock + static_cast<int>(threadIdx.x) / kWave;
  if (row_head >= rows) return;   // whole waves
  const int lane = threadIdx.x % kWave;
  const int request = row_head / a.num_qo_heads;
  const int qh = row_head % a.num_qo_heads;
  const int64_t base = static_cast<int64_t>(row_head) * a.max_items;
  const float* pm = a.partial_m + base;
  const float* pl = a.partial_l + base;
  const float* po = a.partial_o + base * kHeadDim + 2 * lane;

  // the value center, loaded unconditionally and converted after the
  // partial rows are requested (as in combine_unit)
  const bool has_center = a.value_center != nullptr;
  uint32_t center_bits = *(has_center
                               ? reinterpret_cast<const uint32_t*>(
                                     a.value_center + request * a.center_batch_stride +
                                     (qh / kGqa) * kHeadDim + 2 * lane)
                               : reinterpret_cast<const uint32_t*>(po));
  int item_begin = a.item_ptr[request];
  int item_end = a.item_ptr[request + 1];
  float2 ov[kSlots];
  float mv[kSlots], lv[kSlots];
#pragma unroll
  for (int j = 0; j < kSlots; ++j) {
    const bool planned = j < a.max_items;
    ov[j] = planned ? *reinterpret_cast<const float2*>(po + static_cast<int64_t>(j) * kHeadDim)
                    : make_float2(0.0f, 0.0f);
    mv[j] = planned ? pm[j] : kNegInf;
    lv[j] = planned ? pl[j] : 0.0f;
  }
  consume_point(center_bits);
  consume_point(item_begin);
  consume_point(item_end);
  const int count = a.uniform_items > 0 ? a.uniform_items : item_end - item_begin;
  float center2[2] = {0.0f, 0.0f};
  if (has_center) {
    center2[0] = half_bits_to_float(static_cast<uint16_t>(center_bits));
    center2[1] = half_bits_to_float(static_cast<uint16_t>(center_bits >> 16));
  }
  float m = kNegInf;
#pragma unroll
  for (int j = 0; j < kSlots; ++j) {
    mv[j] = j < count ? mv[j] : kNegInf;
    m = fmaxf(m, mv[j]);
  }
  float tx[kCombineRowsMaxItems], ty[kCombineRowsMaxItems], tl[kCombineRowsMaxItems];
#pragma unroll
  for (int j = 0; j < kCombineRowsMaxItems; ++j) {
    float x = 0.0f, y = 0.0f, l = 0.0f;
    if (j < kSlots && j < count) {
      const float w = mv[j] != kNegInf ? __builtin_amdgcn_exp2f(mv[j] - m) : 0.0f;
      x += w * ov[j].x;
      y += w * ov[j].y;
      l += w * lv[j];
    }
    tx[j] = x;
    ty[j] = y;
    tl[j] = l;
  }
  const float total_x = tree16(tx) + tree16(tx + 16);
  const float total_y = tree16(ty) + tree16(ty + 16);
  const float l = tree16(tl) + tree16(tl + 16);
  const bool empty = !(l > 0.0f);
  const float inv = empty ? 0.0f : 1.0f / l;
  uint16_t* out = a.out + static_cast<int64_t>(row_head) * kHeadDim + 2 * lane;
  *reinterpret_cast<__half2*>(out) = __floats2half2_rn(combine_output(total_x, inv, center2[0]),
                                                       combine_output(total_y, inv, center2[1]));
  if (lane == 0 && a.lse != nullptr) a.lse[row_head] = empty ? kNegInf : log2f(l) + m;
}

template <int kSlots>
void launch_combine_rows(const CombineArgs& c, int rows, void* stream, void* stop_event) {
  const dim3 grid((rows + kCombineRowsPerBlock - 1) / kCombineRowsPerBlock);
  if (stop_event) {
    hipExtLaunchKernelGGL(combine_rows_kernel<kSlots>, grid, dim3(kCombineThreads), 0,
                          as_stream(stream), nullptr, static_cast<hipEvent_t>(stop_event), 0, c,
                          rows);
  } else {
    hipLaunchKernelGGL(combine_rows_kernel<kSlots>, grid, dim3(kCombineThreads), 0,
                       as_stream(stream), c, rows);
  }
}

__device__ __forceinline__ void init_state(HeadState& st) {
  st.m = kNegInf;
  st.l = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) st.o[i] = 0.0f;
#if PG_TRACE
  st.trace = 0;
#endif
}

__global__ __launch_bounds__(kWave * kMaxWavesPerBlock) void decode_partial_kernel(DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_all[kMaxWavesPerBlock * kLdsPerWave];
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  HeadState st;
  init_state(st);
  PG_TRACE_MARK(st, kTraceStart);
  // KV heads in blocks: workgroup y of an item reads the contiguous part
  // y*W*128 .. (y+1)*W*128 of every token row (W waves per workgroup)
#if PG_INTERLEAVED_HEADS
  const int kv = wave * static_cast<int>(gridDim.y) + static_cast<int>(blockIdx.y);
#else
  const int kv = blockIdx.y * a.waves_per_block + wave;
#endif
  const WorkItem it = a.closed_form
                          ? closed_form_item(blockIdx.x, a.cf_items, a.cf_tail_items, a.cf_tail_begin,
                                             a.cf_tail_pages, a.cf_primary_begin, a.cf_primary_pages,
                                             a.cf_primary_kind)
                          : a.items[blockIdx.x];
  uint8_t* lds = lds_all + wave * kLdsPerWave;
  if (it.kind == PG_KV_INT8) {
    if (a.num_kv_heads == 8)
      int8_chunk<8 * kHeadDim>(a, it, kv, lane, lds, st);
    else
      int8_chunk<0>(a, it, kv, lane, lds, st);
  } else if (it.kind == PG_KV_HETEROGENEOUS) {
    // One unified table: the request's first old_kv_len/16 pages are INT8
    // codes, the rest index the FP16 exact pages.  The boundary is read at run
    // time; an item that straddles it runs both paths into one state.  The
    // item's page ids leave with the boundary's load (not after it): the
    // INT8 part takes its entries from them.
    const int item_page = a.indices[it.page_begin + min(lane, it.page_end - it.page_begin - 1)];
    const int boundary = min(max(it.request_page_begin + a.old_kv_len[it.request] / kPageSize,
                                 it.page_begin), it.page_end);
    if (boundary > it.page_begin) {
      WorkItem old_part = it;
      old_part.page_end = boundary;
      if (a.num_kv_heads == 8)
        int8_chunk<8 * kHeadDim>(a, old_part, kv, lane, lds, st, &item_page);
      else
        int8_chunk<0>(a, old_part, kv, lane, lds, st, &item_page);
    }
    if (boundary < it.page_end)
      fp16_pages(a, it.request, a.tail_k, a.tail_v, a.indices, boundary, it.page_end, it.last_page,
                 a.last_page_len[it.request], kv, lane, lds, st);
  } else if (it.segment == 0) {
    fp16_pages(a, it.request, static_cast<const uint16_t*>(a.k_cache),
               static_cast<const uint16_t*>(a.v_cache), a.indices, it.page_begin, it.page_end,
               it.last_page, a.last_page_len[it.request], kv, lane, lds, st);
  } else {
    fp16_pages(a, it.request, a.tail_k, a.tail_v, a.tail_indices, it.page_begin, it.page_end,
               it.last_page, a.tail_last_len[it.request], kv, lane, lds, st);
  }
  PG_TRACE_MARK(st, kTraceEnd);
  // partial write: lane (head l/16, n = l%16) owns dims 8n..8n+7.  Layout
  // [request][qo head][item of the request][128] so a combine block reads one
  // (request, head) as a contiguous run.
  const float l_row = row16_sum(st.l);
  const int qh = kv * kGqa + (lane >> 4);
  const int n = lane & 15;
  const int64_t row = (static_cast<int64_t>(it.request) * a.num_qo_heads + qh) * a.max_items +
                      it.item_in_request;
  float* o = a.partial_o + row * kHeadDim + 8 * n;
  *reinterpret_cast<float4*>(o) = make_float4(st.o[0], st.o[1], st.o[2], st.o[3]);
  *reinterpret_cast<float4*>(o + 4) = make_float4(st.o[4], st.o[5], st.o[6], st.o[7]);
  if (n == 0) {
    a.partial_m[row] = st.m;
    a.partial_l[row] = l_row;
  }
#if PG_TRACE
  if (a.trace != nullptr) {
    PG_TRACE_PUT(st, kTraceXcc, trace_hwreg_xcc());
    PG_TRACE_PUT(st, kTraceHwId, trace_hwreg_id());
    PG_TRACE_PUT(st, kTraceItem, (blockIdx.x << 8) | kv);
    PG_TRACE_PUT(st, kTraceKind, it.kind);
    const int64_t w = (static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x) * a.waves_per_block + wave;
    a.trace[w * kWave + lane] = st.trace;
  }
#endif
}

// ---------------------------------------------------------------------------
// merge_state_in_place and the fused exact-tail merge.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kWave) void merge_state_kernel(uint16_t* v, float* s, const uint16_t* vo,
                                                            const float* so, const uint8_t* mask,
                                                            int heads, int head_dim) {
  const int row_head = blockIdx.x;
  const int row = row_head / heads;
  if (mask != nullptr && mask[row] == 0) return;
  const float sa = s[row_head];
  const float sb = so[row_head];
  const float mx = fmaxf(sa, sb);
  const float wa = (sa == kNegInf) ? 0.0f : exp2f(sa - mx);
  const float wb = (sb == kNegInf) ? 0.0f : exp2f(sb - mx);
  const float den = wa + wb;
  for (int d = threadIdx.x; d < head_dim; d += kWave) {
    const int64_t i = static_cast<int64_t>(row_head) * head_dim + d;
    const float a = half_bits_to_float(v[i]);
    const float b = half_bits_to_float(vo[i]);
    const float o = den > 0.0f ? (wa * a + wb * b) / den : 0.0f;
    v[i] = __half_as_ushort(__float2half_rn(o));
  }
  __syncthreads();
  if (threadIdx.x == 0) s[row_head] = den > 0.0f ? log2f(den) + mx : kNegInf;
}

struct TailMergeArgs {
  DecodeArgs base;
  const uint16_t* exact_k;
  const uint16_t* exact_v;
  const int32_t* page_indices;
  const int32_t* last_len;
  uint16_t* old_output;
  float* old_lse;
  const uint16_t* value_center;
  int64_t center_batch_stride;
  int pages_per_request;
  int subs;             // waves per KV head (each takes every subs-th page)
};

// One workgroup per (request, group of KV heads); ``subs`` waves per head walk
// interleaved pages of the tail (the walk is latency-bound: a wave's pages
// are a dependent chain of loads), and their states meet in LDS before the
// merge with the old output.
__global__ __launch_bounds__(kWave * kMaxWavesPerBlock) void tail_merge_kernel(TailMergeArgs t) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_all[kMaxWavesPerBlock * kLdsPerWave];
  __shared__ float sub_state[kMaxWavesPerBlock][10][kWave];
  const DecodeArgs& a = t.base;
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int request = blockIdx.x;
  const int head_slot = wave % a.waves_per_block;
  const int sub = wave / a.waves_per_block;
  const int kv = blockIdx.y * a.waves_per_block + head_slot;
  HeadState st;
  init_state(st);
  // The old state and the value center of this lane's 8 dims are loaded
  // first, unconditionally (every sub-wave, only sub-wave 0 uses them), and
  // consumed after the walk: loaded there, they were one more round trip
  // at the end.
  const int qh = kv * kGqa + (lane >> 4);
  const int n = lane & 15;
  const int64_t row = static_cast<int64_t>(request) * a.num_qo_heads + qh;
  uint16_t* o = t.old_output + row * kHeadDim + 8 * n;
  const uint16_t* c = t.value_center + request * t.center_batch_stride + kv * kHeadDim + 8 * n;
  v4u old_bits = *reinterpret_cast<const v4u*>(o);
  v4u center_bits = *reinterpret_cast<const v4u*>(c);
  float old_lse = t.old_lse[row];
  const int begin = request * t.pages_per_request;
  const int end = begin + t.pages_per_request;
  fp16_pages<true>(a, request, t.exact_k, t.exact_v, t.page_indices, begin, end, end - 1,
                   t.last_len[request], kv, lane, lds_all + wave * kLdsPerWave, st, sub, t.subs);
  // every wave waits for its early loads here, long after they arrived (a
  // wave that leaves below does not leave with loads in flight)
  consume_point(old_bits);
  consume_point(center_bits);
  consume_point(old_lse);
  if (t.subs > 1) {
    sub_state[wave][0][lane] = st.m;
    sub_state[wave][1][lane] = st.l;
#pragma unroll
    for (int i = 0; i < 8; ++i) sub_state[wave][2 + i][lane] = st.o[i];
    __syncthreads();
    if (sub != 0) return;
    float mx = st.m;
    for (int j = 1; j < t.subs; ++j) mx = fmaxf(mx, sub_state[j * a.waves_per_block + head_slot][0][lane]);
    float l = 0.0f;
    float o[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (mx != kNegInf) {
      for (int j = 0; j < t.subs; ++j) {
        const int w = j * a.waves_per_block + head_slot;
        const float mj = sub_state[w][0][lane];
        const float f = mj == kNegInf ? 0.0f : exp2f(mj - mx);
        l += sub_state[w][1][lane] * f;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] += sub_state[w][2 + i][lane] * f;
      }
    }
    st.m = mx;
    st.l = l;
#pragma unroll
    for (int i = 0; i < 8; ++i) st.o[i] = o[i];
  }
  const float l_row = row16_sum(st.l);
  const float mx = fmaxf(old_lse, st.m);
  const float w_old = (old_lse == kNegInf) ? 0.0f : exp2f(old_lse - mx);
  const float w_new = (st.m == kNegInf) ? 0.0f : exp2f(st.m - mx);
  const float den = w_old + w_new * l_row;
  const float inv = den > 0.0f ? 1.0f / den : 0.0f;
  v4u merged_bits;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t word = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int nb = 2 * i + h;
      const float old_v = half_bits_to_float(static_cast<uint16_t>(old_bits[i] >> (16 * h)));
      const float center = half_bits_to_float(static_cast<uint16_t>(center_bits[i] >> (16 * h)));
      const float merged = (w_old * old_v + w_new * st.o[nb]) * inv + center;
      word |= static_cast<uint32_t>(__half_as_ushort(__float2half_rn(merged))) << (16 * h);
    }
    merged_bits[i] = word;
  }
  *reinterpret_cast<v4u*>(o) = merged_bits;
  if (n == 0) t.old_lse[row] = den > 0.0f ? log2f(den) + mx : kNegInf;
}

}  // namespace
}  // namespace pg

using namespace pg;

extern "C" int32_t pg_decode_plan(const int32_t* host_indptr, const int32_t* host_last_page_len,
                                  int32_t batch_size, int32_t primary_kind,
                                  const int32_t* host_tail_indptr,
                                  const int32_t* host_tail_last_len, int32_t num_qo_heads,
                                  int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                  int32_t split_pages, int32_t tail_split_pages,
                                  int32_t exact_tail_pages_hint, int32_t num_cus, void* workspace,
                                  int64_t workspace_bytes, pg_decode_plan_t* plan, void* stream) {
  clear_error();
  if (!plan || !workspace) return fail(PG_ERROR_INVALID_ARGUMENT, "null plan argument");
  std::vector<WorkItem> items;
  std::vector<int32_t> item_ptr;
  pg_decode_plan_t p{};
  const int32_t rc = guarded([&]() -> int32_t {
    return build_plan(host_indptr, host_last_page_len, batch_size, primary_kind,
                      host_tail_indptr, host_tail_last_len, num_qo_heads, num_kv_heads, head_dim,
                      page_size, split_pages, tail_split_pages, exact_tail_pages_hint, num_cus,
                      items, item_ptr, p);
  });
  if (rc != PG_OK) return rc;
  if (p.workspace_bytes > workspace_bytes)
    return fail(PG_ERROR_WORKSPACE, "decode workspace too small: need " +
                                        std::to_string(p.workspace_bytes) + " bytes, have " +
                                        std::to_string(workspace_bytes));

  order_for_dispatch(items, num_cus);
  hipStream_t s = as_stream(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  if (!items.empty()) {
    if (hipMemcpyAsync(ws + p.items_offset, items.data(), items.size() * sizeof(WorkItem),
                       hipMemcpyHostToDevice, s) != hipSuccess)
      return fail(PG_ERROR_LAUNCH, "plan copy failed");
  }
  if (hipMemcpyAsync(ws + p.item_ptr_offset, item_ptr.data(), item_ptr.size() * sizeof(int32_t),
                     hipMemcpyHostToDevice, s) != hipSuccess)
    return fail(PG_ERROR_LAUNCH, "plan copy failed");
  if (hipStreamSynchronize(s) != hipSuccess) return fail(PG_ERROR_LAUNCH, "plan copy sync failed");
  *plan = p;
  return PG_OK;
}

namespace {

#if PG_TRACE
// Trace buffer of the partial kernel (pg_trace_set_buffer); used by a launch
// only when it holds a 64-word row for every wave of the grid.
uint32_t* g_trace = nullptr;
int64_t g_trace_bytes = 0;
#endif

struct PartialViews {
  float* o;
  float* m;
  float* l;
};

PartialViews partial_views(const pg_decode_plan_t* plan, void* workspace) {
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const int64_t rows = static_cast<int64_t>(plan->batch_size) * plan->num_qo_heads *
                      std::max(1, plan->max_items_per_request);
  PartialViews v;
  v.o = reinterpret_cast<float*>(ws + plan->partial_offset);
  v.m = v.o + rows * kHeadDim;
  v.l = v.m + rows;
  return v;
}

}  // namespace

namespace {

// Decode-step finalize of pg_decode_run_finalize (positions null: none).
struct FinalizeSpec {
  const int32_t* positions = nullptr;
  int position_stride = 0;
  int code_pages_per_request = 0;
};

int32_t launch_partial(const pg_decode_plan_t* plan, const void* query,
                       int64_t query_batch_stride, const void* k_cache, const void* v_cache,
                       const void* k_scale, const void* v_scale, const int32_t* indices,
                       const int32_t* last_page_len, const void* tail_k, const void* tail_v,
                       const int32_t* tail_indices, const int32_t* tail_last_len, float sm_scale,
                       void* workspace, void* stream, void* start_event, void* stop_event,
                       const int32_t* old_kv_len = nullptr, FinalizeSpec finalize = {}) {
  clear_error();
  if (!plan || !query || !workspace) return fail(PG_ERROR_INVALID_ARGUMENT, "null run argument");
  if ((plan->primary_kind == PG_KV_HETEROGENEOUS) != (old_kv_len != nullptr))
    return fail(PG_ERROR_INVALID_ARGUMENT,
                "old_kv_len goes with (and only with) a heterogeneous plan");
  if (plan->num_items_primary > 0) {
    if (!k_cache || !v_cache || !indices || !last_page_len)
      return fail(PG_ERROR_INVALID_ARGUMENT, "primary segment tensors missing");
    if (plan->primary_kind != PG_KV_FP16 && (!k_scale || !v_scale))
      return fail(PG_ERROR_INVALID_ARGUMENT, "INT8 pages need k_scale and v_scale");
    if (plan->primary_kind == PG_KV_HETEROGENEOUS && (!tail_k || !tail_v))
      return fail(PG_ERROR_INVALID_ARGUMENT, "heterogeneous pages need the exact K/V pages");
  }
  if (plan->num_items > plan->num_items_primary &&
      (!tail_k || !tail_v || !tail_indices || !tail_last_len))
    return fail(PG_ERROR_INVALID_ARGUMENT, "tail segment tensors missing");
  if (!(sm_scale > 0.0f) || !__builtin_isfinite(sm_scale))
    return fail(PG_ERROR_INVALID_ARGUMENT, "sm_scale must be positive and finite");
  if (plan->num_items == 0) return PG_OK;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const PartialViews pv = partial_views(plan, workspace);
  DecodeArgs a{};
  a.query = static_cast<const uint16_t*>(query);
  a.query_batch_stride = query_batch_stride;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.k_scale = static_cast<const uint16_t*>(k_scale);
  a.v_scale = static_cast<const uint16_t*>(v_scale);
  a.indices = indices;
  a.last_page_len = last_page_len;
  a.tail_k = static_cast<const uint16_t*>(tail_k);
  a.tail_v = static_cast<const uint16_t*>(tail_v);
  a.tail_indices = tail_indices;
  a.tail_last_len = tail_last_len;
  a.old_kv_len = old_kv_len;
  a.items = reinterpret_cast<const WorkItem*>(ws + plan->items_offset);
  a.partial_o = pv.o;
  a.partial_m = pv.m;
  a.partial_l = pv.l;
  a.num_qo_heads = plan->num_qo_heads;
  a.num_kv_heads = plan->num_kv_heads;
  a.waves_per_block = plan->waves_per_block;
  if (a.waves_per_block < 1 || a.waves_per_block > kMaxWavesPerBlock ||
      plan->num_kv_heads % a.waves_per_block)
    return fail(PG_ERROR_INVALID_ARGUMENT, "plan has an invalid waves_per_block");
  a.max_items = std::max(1, plan->max_items_per_request);
  a.sm_scale_log2 = sm_scale * 1.4426950408889634f;
  if (finalize.positions != nullptr) {
    if (plan->primary_kind == PG_KV_FP16 || !k_cache || !v_cache || !k_scale || !v_scale)
      return fail(PG_ERROR_INVALID_ARGUMENT, "the finalize writes into INT8 code pages and scales");
    if (finalize.code_pages_per_request <= 0 || finalize.position_stride < 0)
      return fail(PG_ERROR_INVALID_ARGUMENT, "finalize needs positive code pages per request");
    a.finalize_positions = finalize.positions;
    a.finalize_position_stride = finalize.position_stride;
    a.code_pages_per_request = finalize.code_pages_per_request;
    a.finalize_k_codes = static_cast<int8_t*>(const_cast<void*>(k_cache));
    a.finalize_v_codes = static_cast<int8_t*>(const_cast<void*>(v_cache));
    a.finalize_k_scale = static_cast<uint16_t*>(const_cast<void*>(k_scale));
    a.finalize_v_scale = static_cast<uint16_t*>(const_cast<void*>(v_scale));
  }
  if (plan->closed_form) {
    if (plan->batch_size != 1 || plan->cf_tail_items < 0 || plan->cf_tail_items > plan->num_items ||
        plan->cf_tail_pages < plan->cf_tail_items || plan->cf_tail_pages < 0 ||
        plan->cf_primary_pages < plan->num_items - plan->cf_tail_items ||
        (plan->cf_tail_items == 0) != (plan->cf_tail_pages == 0) ||
        (plan->num_items - plan->cf_tail_items == 0) != (plan->cf_primary_pages == 0))
      return fail(PG_ERROR_INVALID_ARGUMENT, "plan has an inconsistent closed-form description");
    a.closed_form = 1;
    a.cf_items = plan->num_items;
    a.cf_tail_items = plan->cf_tail_items;
    a.cf_tail_begin = plan->cf_tail_begin;
    a.cf_tail_pages = plan->cf_tail_pages;
    a.cf_primary_begin = plan->cf_primary_begin;
    a.cf_primary_pages = plan->cf_primary_pages;
    a.cf_primary_kind = plan->primary_kind;
  }
  const dim3 grid(plan->num_items, plan->num_kv_heads / a.waves_per_block);
#if PG_TRACE
  a.trace = static_cast<int64_t>(grid.x) * grid.y * a.waves_per_block * kWave * 4 <= g_trace_bytes
                ? g_trace : nullptr;
#endif
  if (start_event || stop_event) {
    // The events take the dispatch's own begin/end timestamps.
    hipExtLaunchKernelGGL(decode_partial_kernel, grid, dim3(kWave * a.waves_per_block), 0,
                          as_stream(stream), static_cast<hipEvent_t>(start_event),
                          static_cast<hipEvent_t>(stop_event), 0, a);
  } else {
    hipLaunchKernelGGL(decode_partial_kernel, grid, dim3(kWave * a.waves_per_block), 0,
                       as_stream(stream), a);
  }
  return check_launch("decode_partial");
}

int32_t launch_combine(const pg_decode_plan_t* plan, const void* value_center,
                       int64_t center_batch_stride, void* out, float* lse, void* workspace,
                       void* stream, void* stop_event) {
  clear_error();
  if (!plan || !out || !workspace) return fail(PG_ERROR_INVALID_ARGUMENT, "null run argument");
  const PartialViews pv = partial_views(plan, workspace);
  CombineArgs c{};
  c.partial_o = pv.o;
  c.partial_m = pv.m;
  c.partial_l = pv.l;
  c.item_ptr = reinterpret_cast<const int32_t*>(static_cast<uint8_t*>(workspace) +
                                                plan->item_ptr_offset);
  c.value_center = static_cast<const uint16_t*>(value_center);
  c.center_batch_stride = center_batch_stride;
  c.out = static_cast<uint16_t*>(out);
  c.lse = lse;
  c.num_qo_heads = plan->num_qo_heads;
  c.max_items = std::max(1, plan->max_items_per_request);
  // every request has the same number of items (always so for one request)
  c.uniform_items = plan->num_items == plan->batch_size * plan->max_items_per_request
                        ? plan->max_items_per_request : 0;
  const int rows = plan->batch_size * plan->num_qo_heads;
  if (c.max_items <= kCombineRowsMaxItems && rows >= kCombineRowsMinRows) {
    if (c.max_items <= 8) {
      launch_combine_rows<8>(c, rows, stream, stop_event);
    } else if (c.max_items <= 16) {
      launch_combine_rows<16>(c, rows, stream, stop_event);
    } else {
      launch_combine_rows<32>(c, rows, stream, stop_event);
    }
    return check_launch("decode_combine");
  }
  const dim3 grid(rows, kHeadDim / 32);
#if PG_TRACE
  // combine rows follow the partial kernel's rows (one per wave of its grid)
  const int64_t partial_words = static_cast<int64_t>(plan->num_items) * plan->num_kv_heads * kWave;
  const int64_t combine_words = static_cast<int64_t>(grid.x) * grid.y * (kCombineThreads / kWave) * kWave;
  c.trace = (partial_words + combine_words) * 4 <= g_trace_bytes ? g_trace + partial_words : nullptr;
#endif
  if (stop_event) {
    hipExtLaunchKernelGGL(combine_kernel, grid, dim3(kCombineThreads), 0, as_stream(stream),
                          nullptr, static_cast<hipEvent_t>(stop_event), 0, c);
  } else {
    hipLaunchKernelGGL(combine_kernel, grid, dim3(kCombineThreads), 0, as_stream(stream), c);
  }
  return check_launch("decode_combine");
}

int32_t run_decode(const pg_decode_plan_t* plan, const void* query, int64_t query_batch_stride,
                   const void* k_cache, const void* v_cache, const void* k_scale,
                   const void* v_scale, const int32_t* indices, const int32_t* last_page_len,
                   const void* tail_k, const void* tail_v, const int32_t* tail_indices,
                   const int32_t* tail_last_len, const void* value_center,
                   int64_t center_batch_stride, void* out, float* lse, float sm_scale,
                   void* workspace, void* stream, void* start_event, void* stop_event,
                   const int32_t* old_kv_len = nullptr, FinalizeSpec finalize = {}) {
  if (int32_t rc = launch_partial(plan, query, query_batch_stride, k_cache, v_cache, k_scale,
                                  v_scale, indices, last_page_len, tail_k, tail_v, tail_indices,
                                  tail_last_len, sm_scale, workspace, stream, start_event, nullptr,
                                  old_kv_len, finalize))
    return rc;
  return launch_combine(plan, value_center, center_batch_stride, out, lse, workspace, stream,
                        stop_event);
}

}  // namespace

extern "C" int32_t pg_decode_run_partial(const pg_decode_plan_t* plan, const void* query,
                                         int64_t query_batch_stride, const void* k_cache,
                                         const void* v_cache, const void* k_scale,
                                         const void* v_scale, const int32_t* indices,
                                         const int32_t* last_page_len, const void* tail_k,
                                         const void* tail_v, const int32_t* tail_indices,
                                         const int32_t* tail_last_len, float sm_scale,
                                         void* workspace, void* stream) {
  return launch_partial(plan, query, query_batch_stride, k_cache, v_cache, k_scale, v_scale,
                        indices, last_page_len, tail_k, tail_v, tail_indices, tail_last_len,
                        sm_scale, workspace, stream, nullptr, nullptr);
}

extern "C" int32_t pg_decode_run_partial_timed(
    const pg_decode_plan_t* plan, const void* query, int64_t query_batch_stride,
    const void* k_cache, const void* v_cache, const void* k_scale, const void* v_scale,
    const int32_t* indices, const int32_t* last_page_len, const void* tail_k, const void* tail_v,
    const int32_t* tail_indices, const int32_t* tail_last_len, float sm_scale, void* workspace,
    void* stream, void* start_event, void* stop_event) {
  return launch_partial(plan, query, query_batch_stride, k_cache, v_cache, k_scale, v_scale,
                        indices, last_page_len, tail_k, tail_v, tail_indices, tail_last_len,
                        sm_scale, workspace, stream, start_event, stop_event);
}

extern "C" int32_t pg_decode_run_combine(const pg_decode_plan_t* plan, const void* value_center,
                                         int64_t center_batch_stride, void* out, float* lse,
                                         void* workspace, void* stream) {
  return launch_combine(plan, value_center, center_batch_stride, out, lse, workspace, stream,
                        nullptr);
}

extern "C" int32_t pg_decode_run(const pg_decode_plan_t* plan, const void* query,
                                 int64_t query_batch_stride, const void* k_cache,
                                 const void* v_cache, const void* k_scale, const void* v_scale,
                                 const int32_t* indices, const int32_t* last_page_len,
                                 const void* tail_k, const void* tail_v,
                                 const int32_t* tail_indices, const int32_t* tail_last_len,
                                 const void* value_center, int64_t center_batch_stride, void* out,
                                 float* lse, float sm_scale, void* workspace, void* stream) {
  return run_decode(plan, query, query_batch_stride, k_cache, v_cache, k_scale, v_scale, indices,
                    last_page_len, tail_k, tail_v, tail_indices, tail_last_len, value_center,
                    center_batch_stride, out, lse, sm_scale, workspace, stream, nullptr, nullptr);
}

extern "C" int32_t pg_decode_run_timed(const pg_decode_plan_t* plan, const void* query,
                                       int64_t query_batch_stride, const void* k_cache,
                                       const void* v_cache, const void* k_scale,
                                       const void* v_scale, const int32_t* indices,
                                       const int32_t* last_page_len, const void* tail_k,
                                       const void* tail_v, const int32_t* tail_indices,
                                       const int32_t* tail_last_len, const void* value_center,
                                       int64_t center_batch_stride, void* out, float* lse,
                                       float sm_scale, void* workspace, void* stream,
                                       void* start_event, void* stop_event) {
  return run_decode(plan, query, query_batch_stride, k_cache, v_cache, k_scale, v_scale, indices,
                    last_page_len, tail_k, tail_v, tail_indices, tail_last_len, value_center,
                    center_batch_stride, out, lse, sm_scale, workspace, stream, start_event,
                    stop_event);
}

extern "C" int32_t pg_decode_run_heterogeneous(
    const pg_decode_plan_t* plan, const void* query, int64_t query_batch_stride,
    const void* k_codes, const void* v_codes, const void* k_scale, const void* v_scale,
    const void* exact_k, const void* exact_v, const int32_t* indices,
    const int32_t* last_page_len, const int32_t* old_kv_len, const void* value_center,
    int64_t center_batch_stride, void* out, float* lse, float sm_scale, void* workspace,
    void* stream) {
  clear_error();
  if (!old_kv_len) return fail(PG_ERROR_INVALID_ARGUMENT, "old_kv_len is required");
  return run_decode(plan, query, query_batch_stride, k_codes, v_codes, k_scale, v_scale, indices,
                    last_page_len, exact_k, exact_v, nullptr, nullptr, value_center,
                    center_batch_stride, out, lse, sm_scale, workspace, stream, nullptr, nullptr,
                    old_kv_len);
}

extern "C" int32_t pg_decode_run_finalize(
    const pg_decode_plan_t* plan, const void* query, int64_t query_batch_stride,
    const void* k_cache, const void* v_cache, const void* k_scale, const void* v_scale,
    const int32_t* indices, const int32_t* last_page_len, const void* tail_k, const void* tail_v,
    const int32_t* tail_indices, const int32_t* tail_last_len, const void* value_center,
    int64_t center_batch_stride, void* out, float* lse, float sm_scale, void* workspace,
    const int32_t* positions, int32_t position_stride, int32_t code_pages_per_request,
    void* stream) {
  clear_error();
  if (!positions) return fail(PG_ERROR_INVALID_ARGUMENT, "finalize positions are required");
  FinalizeSpec f;
  f.positions = positions;
  f.position_stride = position_stride;
  f.code_pages_per_request = code_pages_per_request;
  return run_decode(plan, query, query_batch_stride, k_cache, v_cache, k_scale, v_scale, indices,
                    last_page_len, tail_k, tail_v, tail_indices, tail_last_len, value_center,
                    center_batch_stride, out, lse, sm_scale, workspace, stream, nullptr, nullptr,
                    nullptr, f);
}

extern "C" int32_t pg_decode_run_heterogeneous_finalize(
    const pg_decode_plan_t* plan, const void* query, int64_t query_batch_stride,
    const void* k_codes, const void* v_codes, const void* k_scale, const void* v_scale,
    const void* exact_k, const void* exact_v, const int32_t* indices,
    const int32_t* last_page_len, const int32_t* old_kv_len, const void* value_center,
    int64_t center_batch_stride, void* out, float* lse, float sm_scale, void* workspace,
    const int32_t* positions, int32_t position_stride, int32_t code_pages_per_request,
    void* stream) {
  clear_error();
  if (!old_kv_len) return fail(PG_ERROR_INVALID_ARGUMENT, "old_kv_len is required");
  if (!positions) return fail(PG_ERROR_INVALID_ARGUMENT, "finalize positions are required");
  FinalizeSpec f;
  f.positions = positions;
  f.position_stride = position_stride;
  f.code_pages_per_request = code_pages_per_request;
  return run_decode(plan, query, query_batch_stride, k_codes, v_codes, k_scale, v_scale, indices,
                    last_page_len, exact_k, exact_v, nullptr, nullptr, value_center,
                    center_batch_stride, out, lse, sm_scale, workspace, stream, nullptr, nullptr,
                    old_kv_len, f);
}

extern "C" int32_t pg_merge_state_in_place(void* v, float* s, const void* v_other,
                                           const float* s_other, const uint8_t* mask,
                                           int32_t rows, int32_t heads, int32_t head_dim,
                                           void* stream) {
  clear_error();
  if (!v || !s || !v_other || !s_other) return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if (rows <= 0 || heads <= 0 || head_dim <= 0)
    return fail(PG_ERROR_INVALID_ARGUMENT, "merge_state shapes must be positive");
  hipLaunchKernelGGL(merge_state_kernel, dim3(rows * heads), dim3(kWave), 0, as_stream(stream),
                     static_cast<uint16_t*>(v), s, static_cast<const uint16_t*>(v_other), s_other,
                     mask, heads, head_dim);
  return check_launch("merge_state_in_place");
}

extern "C" int32_t pg_exact_tail_merge_center(const void* query, const void* exact_key_pages,
                                              const void* exact_value_pages,
                                              const int32_t* exact_page_indices,
                                              const int32_t* exact_last_page_len,
                                              void* old_output, float* old_lse,
                                              const void* value_center,
                                              int64_t center_batch_stride, int32_t batch_size,
                                              int32_t query_heads, int32_t kv_heads,
                                              int32_t pages_per_request, float sm_scale,
                                              void* stream) {
  clear_error();
  if (!query || !exact_key_pages || !exact_value_pages || !exact_page_indices ||
      !exact_last_page_len || !old_output || !old_lse || !value_center)
    return fail(PG_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if (batch_size <= 0) return fail(PG_ERROR_INVALID_ARGUMENT, "batch size must be positive");
  if (query_heads <= 0 || kv_heads <= 0 || query_heads % kv_heads != 0)
    return fail(PG_ERROR_INVALID_ARGUMENT, "query heads must be a positive multiple of KV heads");
  if (query_heads / kv_heads != kGqa)
    return fail(PG_ERROR_UNSUPPORTED, "the fused exact-tail kernel currently requires GQA group size 4");
  if (kv_heads > 64) return fail(PG_ERROR_UNSUPPORTED, "at most 64 KV heads");
  if (pages_per_request <= 0 || pages_per_request > 16)
    return fail(PG_ERROR_INVALID_ARGUMENT, "the fused exact tail supports 1..16 pages per request");
  if (!(sm_scale > 0.0f) || !__builtin_isfinite(sm_scale))
    return fail(PG_ERROR_INVALID_ARGUMENT, "sm_scale must be positive and finite");
  TailMergeArgs t{};
  t.base.query = static_cast<const uint16_t*>(query);
  t.base.query_batch_stride = static_cast<int64_t>(query_heads) * kHeadDim;
  t.base.num_qo_heads = query_heads;
  t.base.num_kv_heads = kv_heads;
  // one KV head per group of sub-waves: up to kMaxWavesPerBlock waves walk
  // the tail's pages of one head in parallel
  t.base.waves_per_block = 1;
  t.subs = std::min(pages_per_request, kMaxWavesPerBlock);
  t.base.sm_scale_log2 = sm_scale * 1.4426950408889634f;
  t.exact_k = static_cast<const uint16_t*>(exact_key_pages);
  t.exact_v = static_cast<const uint16_t*>(exact_value_pages);
  t.page_indices = exact_page_indices;
  t.last_len = exact_last_page_len;
  t.old_output = static_cast<uint16_t*>(old_output);
  t.old_lse = old_lse;
  t.value_center = static_cast<const uint16_t*>(value_center);
  t.center_batch_stride = center_batch_stride;
  t.pages_per_request = pages_per_request;
  const dim3 grid(batch_size, kv_heads / t.base.waves_per_block);
  hipLaunchKernelGGL(tail_merge_kernel, grid, dim3(kWave * t.base.waves_per_block * t.subs), 0,
                     as_stream(stream), t);
  return check_launch("exact_tail_merge_center");
}

#if PG_TRACE
// Trace builds only (bench.py --trace): the device buffer the partial
// kernel writes its per-wave phase rows into; null or 0 bytes turns the
// trace off.  A launch whose grid needs more rows than fit writes none.
extern "C" int32_t pg_trace_set_buffer(void* device_words, int64_t bytes) {
  clear_error();
  if (bytes < 0 || (bytes > 0 && device_words == nullptr))
    return fail(PG_ERROR_INVALID_ARGUMENT, "trace buffer needs a pointer and a nonnegative size");
  g_trace = static_cast<uint32_t*>(device_words);
  g_trace_bytes = device_words ? bytes : 0;
  return PG_OK;
}
#endif
