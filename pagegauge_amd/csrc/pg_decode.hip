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

#include <algorithm>
#include <vector>

namespace pg {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned char u8x4 __attribute__((ext_vector_type(4)));

constexpr int kGroupPages = 4;          // INT8 pages per PV MFMA (k = 64 tokens)
constexpr int kMaxWavesPerBlock = 8;
constexpr int kLdsPerWave = 1024;       // INT8 P digits: [4 pages][4 heads][4 digits][16 tokens]
constexpr int kCombineThreads = 256;
constexpr int kMaxItemsPerRequest = 4096;
constexpr float kNegInf = -__builtin_huge_valf();

struct WorkItem {
  int32_t request;
  int32_t kind;        // PG_KV_INT8 or PG_KV_FP16
  int32_t segment;     // 0 primary, 1 tail
  int32_t page_begin;  // absolute index into the segment's page-index array
  int32_t page_end;    // exclusive
  int32_t last_page;   // absolute index of the segment's final page for the request
  int32_t pad0;
  int32_t pad1;
};
static_assert(sizeof(WorkItem) == 32, "work item layout");

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
  const WorkItem* items;
  float* partial_o;   // [items][Hq][128]
  float* partial_m;   // [items][Hq]
  float* partial_l;   // [items][Hq]
  int num_qo_heads;
  int num_kv_heads;
  int waves_per_block;
  float sm_scale_log2;
};

// Per-lane softmax/output state of one KV head (4 query heads).
// Lane l owns head h = l/16; o[nb] is output dim 64*(nb/4) + 4*(l%16) + nb%4.
struct HeadState {
  float m;
  float l;
  float o[8];
};

__device__ __forceinline__ uint32_t bits_of(u8x4 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ u8x4 bytes_of(uint32_t v) { return __builtin_bit_cast(u8x4, v); }

// 4x4 byte transpose: r[k] holds 4 dims of token k; returns c[j] holding
// dim j of tokens 0..3.
__device__ __forceinline__ void transpose4x4(const uint32_t r[4], uint32_t c[4]) {
  const u8x4 a = bytes_of(r[0]), b = bytes_of(r[1]), cc = bytes_of(r[2]), d = bytes_of(r[3]);
  const u8x4 t0 = __builtin_shufflevector(a, b, 0, 4, 1, 5);
  const u8x4 t1 = __builtin_shufflevector(a, b, 2, 6, 3, 7);
  const u8x4 t2 = __builtin_shufflevector(cc, d, 0, 4, 1, 5);
  const u8x4 t3 = __builtin_shufflevector(cc, d, 2, 6, 3, 7);
  c[0] = bits_of(__builtin_shufflevector(t0, t2, 0, 1, 4, 5));
  c[1] = bits_of(__builtin_shufflevector(t0, t2, 2, 3, 6, 7));
  c[2] = bits_of(__builtin_shufflevector(t1, t3, 0, 1, 4, 5));
  c[3] = bits_of(__builtin_shufflevector(t1, t3, 2, 3, 6, 7));
}

// Balanced radix-256 digits of |x| <= 2^22: x = d0*2^16 + d1*2^8 + d2.
__device__ __forceinline__ void balanced_digits(int x, int& d0, int& d1, int& d2) {
  d2 = ((x + 128) & 255) - 128;
  const int r = (x - d2) >> 8;
  d1 = ((r + 128) & 255) - 128;
  d0 = (r - d1) >> 8;
}

__device__ __forceinline__ int select_digit(int x, int which) {
  int d0, d1, d2;
  balanced_digits(x, d0, d1, d2);
  return which == 0 ? d0 : (which == 1 ? d1 : (which == 2 ? d2 : 0));
}

// Exponent e with 0 < v < 2^e (v > 0); 0 for v == 0.
__device__ __forceinline__ int ceil_exponent(float v) {
  int e = 0;
  if (v > 0.0f) frexpf(v, &e);
  return e;
}

__device__ __forceinline__ float combine_digits(v4i acc) {
  return static_cast<float>(acc.x) * 65536.0f + static_cast<float>(acc.y) * 256.0f +
         static_cast<float>(acc.z);
}

__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Online-softmax update for one lane holding ``count`` scores of head row
// lane/16.  Returns alpha (rescale of the previous state) and writes p[].
template <int kCount>
__device__ __forceinline__ float softmax_update(HeadState& st, const float s[kCount],
                                                float p[kCount]) {
  float local = s[0];
#pragma unroll
  for (int i = 1; i < kCount; ++i) local = fmaxf(local, s[i]);
  const float group_max = row16_max(local);
  const float m_new = fmaxf(st.m, group_max);
  if (m_new == kNegInf) {  // nothing visible yet in this row
#pragma unroll
    for (int i = 0; i < kCount; ++i) p[i] = 0.0f;
    return 1.0f;
  }
  const float alpha = exp2f(st.m - m_new);  // exp2(-inf) = 0 on the first visible group
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < kCount; ++i) {
    p[i] = exp2f(s[i] - m_new);
    sum += p[i];
  }
  st.l = st.l * alpha + sum;
  st.m = m_new;
  return alpha;
}

__device__ __forceinline__ int clamp_page_slot(int slot, int begin, int end) {
  return slot < end ? slot : end - 1;
}

// ---------------------------------------------------------------------------
// INT8 page-affine chunk: pages [it.page_begin, it.page_end) of one request,
// KV head ``kv``.  Groups of 4 pages; loads of group g+1 are issued before
// group g is computed.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void int8_chunk(const DecodeArgs& a, const WorkItem& it, int kv,
                                           int lane, uint8_t* lds, HeadState& st) {
  const int hkv = a.num_kv_heads;
  const int m16 = lane & 15;
  const int kg = lane >> 4;
  const int a_head = m16 >> 2;   // A-operand row 4h+c -> head h, digit c
  const int a_digit = m16 & 3;
  const int64_t row_stride = static_cast<int64_t>(hkv) * kHeadDim;   // one token row (bytes)
  const int8_t* kc = static_cast<const int8_t*>(a.k_cache) + kv * kHeadDim;
  const int8_t* vc = static_cast<const int8_t*>(a.v_cache) + kv * kHeadDim;

  // ---- query digits (A operand of QK): dims 16*kg + 64*j + b, b = 0..15
  const uint16_t* q = a.query + it.request * a.query_batch_stride +
                      static_cast<int64_t>(kv * kGqa + a_head) * kHeadDim;
  float qv[2][16];
  float qmax = 0.0f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint4 lo = *reinterpret_cast<const uint4*>(q + 16 * kg + 64 * j);
    const uint4 hi = *reinterpret_cast<const uint4*>(q + 16 * kg + 64 * j + 8);
    const uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      qv[j][2 * b] = half_bits_to_float(static_cast<uint16_t>(w[b] & 0xffffu));
      qv[j][2 * b + 1] = half_bits_to_float(static_cast<uint16_t>(w[b] >> 16));
      qmax = fmaxf(qmax, fmaxf(fabsf(qv[j][2 * b]), fabsf(qv[j][2 * b + 1])));
    }
  }
  // max over the 16 lanes sharing a_head (lane bits 0,1,4,5)
  qmax = fmaxf(qmax, __shfl_xor(qmax, 1, kWave));
  qmax = fmaxf(qmax, __shfl_xor(qmax, 2, kWave));
  qmax = fmaxf(qmax, __shfl_xor(qmax, 16, kWave));
  qmax = fmaxf(qmax, __shfl_xor(qmax, 32, kWave));
  const int q_exp = 22 - ceil_exponent(qmax);   // |q| * 2^q_exp < 2^22
  v4i qd[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    uint32_t packed[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t word = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int qi = static_cast<int>(rintf(ldexpf(qv[j][4 * w + b], q_exp)));
        const int digit = select_digit(qi, a_digit);
        word |= (static_cast<uint32_t>(digit) & 0xffu) << (8 * b);
      }
      packed[w] = word;
    }
    qd[j] = v4i{static_cast<int>(packed[0]), static_cast<int>(packed[1]),
                static_cast<int>(packed[2]), static_cast<int>(packed[3])};
  }
  // score scale for this lane's C row (head kg): 2^-q_exp(head kg) * sm_scale*log2e
  const int q_exp_row = __shfl(q_exp, 4 * kg, kWave);
  const float qscale = ldexpf(a.sm_scale_log2, -q_exp_row);

  // zero the wave's digit buffer once: digit row 3 of every head stays zero
  *reinterpret_cast<uint4*>(lds + 16 * lane) = uint4{0u, 0u, 0u, 0u};
  wave_lds_fence();

  const int begin = it.page_begin;
  const int end = it.page_end;
  const int last_page = it.last_page;
  const int last_len = it.segment == 0 ? a.last_page_len[it.request] : a.tail_last_len[it.request];
  const int32_t* indices = a.indices;
  const int groups = (end - begin + kGroupPages - 1) / kGroupPages;

  // group buffers
  v4i kb[kGroupPages][2];
  uint32_t vb[2][kPageSize];
  int page_id[kGroupPages];

  auto issue = [&](int g, v4i (&kbuf)[kGroupPages][2], uint32_t (&vbuf)[2][kPageSize],
                   int (&ids)[kGroupPages]) {
    // Slots past the chunk end keep a valid page id (for the scale loads) but
    // load nothing; their scores are masked to -inf.
#pragma unroll
    for (int i = 0; i < kGroupPages; ++i) {
      const int slot = clamp_page_slot(begin + g * kGroupPages + i, begin, end);
      ids[i] = indices[slot];
    }
#pragma unroll
    for (int i = 0; i < kGroupPages; ++i) {
      if (begin + g * kGroupPages + i < end) {
        const int8_t* base =
            kc + (static_cast<int64_t>(ids[i]) * kPageSize + m16) * row_stride + 16 * kg;
        kbuf[i][0] = *reinterpret_cast<const v4i*>(base);
        kbuf[i][1] = *reinterpret_cast<const v4i*>(base + 64);
      } else {
        kbuf[i][0] = v4i{0, 0, 0, 0};
        kbuf[i][1] = v4i{0, 0, 0, 0};
      }
    }
    // V: this lane reads page kg of the group, dims 4*m16 (+64), all 16 tokens
    int my_page = ids[0];
#pragma unroll
    for (int i = 1; i < kGroupPages; ++i) my_page = kg == i ? ids[i] : my_page;
    if (begin + g * kGroupPages + kg < end) {
      const int8_t* vbase = vc + static_cast<int64_t>(my_page) * kPageSize * row_stride + 4 * m16;
#pragma unroll
      for (int t = 0; t < kPageSize; ++t) {
        vbuf[0][t] = *reinterpret_cast<const uint32_t*>(vbase + t * row_stride);
        vbuf[1][t] = *reinterpret_cast<const uint32_t*>(vbase + t * row_stride + 64);
      }
    } else {
#pragma unroll
      for (int t = 0; t < kPageSize; ++t) {
        vbuf[0][t] = 0u;
        vbuf[1][t] = 0u;
      }
    }
  };

  if (groups > 0) issue(0, kb, vb, page_id);
  for (int g = 0; g < groups; ++g) {
    v4i kn[kGroupPages][2];
    uint32_t vn[2][kPageSize];
    int next_id[kGroupPages];
    if (g + 1 < groups) issue(g + 1, kn, vn, next_id);

    // ---- QK: exact integer scores, recombined in float
    float s[kGroupPages];
    float sv[kGroupPages];
#pragma unroll
    for (int i = 0; i < kGroupPages; ++i) {
      v4i acc = {0, 0, 0, 0};
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qd[0], kb[i][0], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qd[1], kb[i][1], acc, 0, 0, 0);
      const int slot = begin + g * kGroupPages + i;
      const float sk = half_bits_to_float(a.k_scale[static_cast<int64_t>(page_id[i]) * hkv + kv]);
      bool valid = slot < end;
      sv[i] = valid ? half_bits_to_float(a.v_scale[static_cast<int64_t>(page_id[i]) * hkv + kv]) : 0.0f;
      if (slot == last_page && m16 >= last_len) valid = false;
      s[i] = valid ? combine_digits(acc) * (qscale * sk) : kNegInf;
    }
    float p[kGroupPages];
    const float alpha = softmax_update<kGroupPages>(st, s, p);

    // ---- P digits (fixed point relative to the group's largest V scale)
    float vmax = sv[0];
#pragma unroll
    for (int i = 1; i < kGroupPages; ++i) vmax = fmaxf(vmax, sv[i]);
    const int p_exp = 22 - ceil_exponent(vmax);   // p*sV*2^p_exp < 2^22 since p <= 1
#pragma unroll
    for (int i = 0; i < kGroupPages; ++i) {
      const int pi = static_cast<int>(rintf(ldexpf(p[i] * sv[i], p_exp)));
      int d0, d1, d2;
      balanced_digits(pi, d0, d1, d2);
      uint8_t* row = lds + ((i * 4 + kg) * 4) * 16 + m16;   // [page i][head kg][digit][token]
      row[0] = static_cast<uint8_t>(d0);
      row[16] = static_cast<uint8_t>(d1);
      row[32] = static_cast<uint8_t>(d2);
    }
    wave_lds_fence();
    // A operand: lane (row 4h+c, page kg): 16 token digits
    const v4i pa = *reinterpret_cast<const v4i*>(lds + ((kg * 4 + a_head) * 4 + a_digit) * 16);
    wave_lds_fence();

    // ---- PV: V code bytes transposed to token-major operands
    const float inv_p = ldexpf(1.0f, -p_exp);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      uint32_t cols[4][4];   // [dim j][token quad]
#pragma unroll
      for (int tq = 0; tq < 4; ++tq) {
        uint32_t c[4];
        transpose4x4(&vb[half][4 * tq], c);
#pragma unroll
        for (int j = 0; j < 4; ++j) cols[j][tq] = c[j];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const v4i bop = {static_cast<int>(cols[j][0]), static_cast<int>(cols[j][1]),
                         static_cast<int>(cols[j][2]), static_cast<int>(cols[j][3])};
        v4i acc = {0, 0, 0, 0};
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, bop, acc, 0, 0, 0);
        const int nb = half * 4 + j;
        st.o[nb] = st.o[nb] * alpha + combine_digits(acc) * inv_p;
      }
    }

    if (g + 1 < groups) {
#pragma unroll
      for (int i = 0; i < kGroupPages; ++i) {
        kb[i][0] = kn[i][0];
        kb[i][1] = kn[i][1];
        page_id[i] = next_id[i];
      }
#pragma unroll
      for (int t = 0; t < kPageSize; ++t) {
        vb[0][t] = vn[0][t];
        vb[1][t] = vn[1][t];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// FP16 chunk (tail ring or plain FP16 pages), one page per step.
// ---------------------------------------------------------------------------
__device__ __forceinline__ v2h pair_of(uint32_t lo_token, uint32_t hi_token, int upper) {
  const v2h a = __builtin_bit_cast(v2h, lo_token);
  const v2h b = __builtin_bit_cast(v2h, hi_token);
  return upper ? __builtin_shufflevector(a, b, 1, 3) : __builtin_shufflevector(a, b, 0, 2);
}

__device__ __forceinline__ void fp16_pages(const DecodeArgs& a, int request, const uint16_t* kpages,
                                           const uint16_t* vpages, const int32_t* indices,
                                           int begin, int end, int last_page, int last_len,
                                           int kv, int lane, uint8_t* lds, HeadState& st) {
  const int hkv = a.num_kv_heads;
  const int m16 = lane & 15;
  const int kg = lane >> 4;
  const int64_t row_stride = static_cast<int64_t>(hkv) * kHeadDim;  // elements
  const uint16_t* kp = kpages + kv * kHeadDim;
  const uint16_t* vp = vpages + kv * kHeadDim;

  // Q operand: head h on row 4h; lanes of other rows hold zeros.
  v8h qa[4];
  const bool q_row = (m16 & 3) == 0;
  const uint16_t* q = a.query + request * a.query_batch_stride +
                      static_cast<int64_t>(kv * kGqa + (m16 >> 2)) * kHeadDim;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (q_row) {
      qa[j] = *reinterpret_cast<const v8h*>(q + 32 * j + 8 * kg);
    } else {
      qa[j] = v8h{0, 0, 0, 0, 0, 0, 0, 0};
    }
  }
  uint16_t* plds = reinterpret_cast<uint16_t*>(lds);   // [4 heads][16 tokens] fp16

  v8h kb[4];
  uint32_t vb[4][2][2];   // [token k][half][dword]
  auto issue = [&](int slot, v8h (&kbuf)[4], uint32_t (&vbuf)[4][2][2]) {
    const int page = indices[slot];
    const uint16_t* kbase = kp + (static_cast<int64_t>(page) * kPageSize + m16) * row_stride + 8 * kg;
#pragma unroll
    for (int j = 0; j < 4; ++j) kbuf[j] = *reinterpret_cast<const v8h*>(kbase + 32 * j);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint16_t* vbase =
          vp + (static_cast<int64_t>(page) * kPageSize + 4 * kg + k) * row_stride + 4 * m16;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const uint2 w = *reinterpret_cast<const uint2*>(vbase + 64 * half);
        vbuf[k][half][0] = w.x;
        vbuf[k][half][1] = w.y;
      }
    }
  };

  if (begin < end) issue(begin, kb, vb);
  for (int slot = begin; slot < end; ++slot) {
    v8h kn[4];
    uint32_t vn[4][2][2];
    if (slot + 1 < end) issue(slot + 1, kn, vn);

    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[j], kb[j], acc, 0, 0, 0);
    bool valid = true;
    if (slot == last_page && m16 >= last_len) valid = false;
    float s[1] = {valid ? acc.x * a.sm_scale_log2 : kNegInf};
    float p[1];
    const float alpha = softmax_update<1>(st, s, p);

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
    for (int half = 0; half < 2; ++half) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int dw = j >> 1;
        const int upper = j & 1;
        const v2h p01 = pair_of(vb[0][half][dw], vb[1][half][dw], upper);
        const v2h p23 = pair_of(vb[2][half][dw], vb[3][half][dw], upper);
        const v4h bop = __builtin_shufflevector(p01, p23, 0, 1, 2, 3);
        v4f o = {0.0f, 0.0f, 0.0f, 0.0f};
        o = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, bop, o, 0, 0, 0);
        const int nb = half * 4 + j;
        st.o[nb] = st.o[nb] * alpha + (o.x + o.y);
      }
    }

    if (slot + 1 < end) {
#pragma unroll
      for (int j = 0; j < 4; ++j) kb[j] = kn[j];
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          vb[k][half][0] = vn[k][half][0];
          vb[k][half][1] = vn[k][half][1];
        }
    }
  }
}

__device__ __forceinline__ void init_state(HeadState& st) {
  st.m = kNegInf;
  st.l = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) st.o[i] = 0.0f;
}

__global__ __launch_bounds__(kWave * kMaxWavesPerBlock) void decode_partial_kernel(DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_all[kMaxWavesPerBlock * kLdsPerWave];
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int kv = blockIdx.y * a.waves_per_block + wave;
  const WorkItem it = a.items[blockIdx.x];
  uint8_t* lds = lds_all + wave * kLdsPerWave;
  HeadState st;
  init_state(st);
  if (it.kind == PG_KV_INT8) {
    int8_chunk(a, it, kv, lane, lds, st);
  } else if (it.segment == 0) {
    fp16_pages(a, it.request, static_cast<const uint16_t*>(a.k_cache),
               static_cast<const uint16_t*>(a.v_cache), a.indices, it.page_begin, it.page_end,
               it.last_page, a.last_page_len[it.request], kv, lane, lds, st);
  } else {
    fp16_pages(a, it.request, a.tail_k, a.tail_v, a.tail_indices, it.page_begin, it.page_end,
               it.last_page, a.tail_last_len[it.request], kv, lane, lds, st);
  }
  // partial write: lane (head l/16, n = l%16) owns dims 4n..4n+3 and 64+4n..64+4n+3
  const float l_row = row16_sum(st.l);
  const int qh = kv * kGqa + (lane >> 4);
  const int n = lane & 15;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * a.num_qo_heads + qh;
  float* o = a.partial_o + row * kHeadDim;
  *reinterpret_cast<float4*>(o + 4 * n) = make_float4(st.o[0], st.o[1], st.o[2], st.o[3]);
  *reinterpret_cast<float4*>(o + 64 + 4 * n) = make_float4(st.o[4], st.o[5], st.o[6], st.o[7]);
  if (n == 0) {
    a.partial_m[row] = st.m;
    a.partial_l[row] = l_row;
  }
}

// ---------------------------------------------------------------------------
// Combine: one block per (request, query head).
// ---------------------------------------------------------------------------
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
};

__device__ __forceinline__ float block_reduce(float v, float* scratch, bool is_max) {
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  v = is_max ? wave_max(v) : wave_sum(v);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float r = scratch[0];
  for (int w = 1; w < kCombineThreads / kWave; ++w) r = is_max ? fmaxf(r, scratch[w]) : r + scratch[w];
  return r;
}

__global__ __launch_bounds__(kCombineThreads) void combine_kernel(CombineArgs a) {
  __shared__ float weights[kMaxItemsPerRequest];
  __shared__ float scratch[kCombineThreads / kWave];
  __shared__ float2 partial_acc[kCombineThreads / kWave][kWave];
  const int request = blockIdx.x / a.num_qo_heads;
  const int qh = blockIdx.x % a.num_qo_heads;
  const int begin = a.item_ptr[request];
  const int count = a.item_ptr[request + 1] - begin;
  const int tid = threadIdx.x;

  float local_max = kNegInf;
  for (int i = tid; i < count; i += kCombineThreads)
    local_max = fmaxf(local_max, a.partial_m[static_cast<int64_t>(begin + i) * a.num_qo_heads + qh]);
  const float m = block_reduce(local_max, scratch, true);
  float local_sum = 0.0f;
  for (int i = tid; i < count; i += kCombineThreads) {
    const int64_t row = static_cast<int64_t>(begin + i) * a.num_qo_heads + qh;
    const float mi = a.partial_m[row];
    const float w = (mi == kNegInf) ? 0.0f : exp2f(mi - m);
    weights[i] = w;
    local_sum += w * a.partial_l[row];
  }
  const float l = block_reduce(local_sum, scratch, false);   // includes a __syncthreads

  const int wave = tid / kWave;
  const int lane = tid % kWave;
  float2 acc = make_float2(0.0f, 0.0f);
  for (int i = wave; i < count; i += kCombineThreads / kWave) {
    const float w = weights[i];
    if (w != 0.0f) {
      const float2 o = *reinterpret_cast<const float2*>(
          a.partial_o + (static_cast<int64_t>(begin + i) * a.num_qo_heads + qh) * kHeadDim + 2 * lane);
      acc.x += w * o.x;
      acc.y += w * o.y;
    }
  }
  partial_acc[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    float2 total = partial_acc[0][lane];
    for (int w = 1; w < kCombineThreads / kWave; ++w) {
      total.x += partial_acc[w][lane].x;
      total.y += partial_acc[w][lane].y;
    }
    const bool empty = !(l > 0.0f);
    float ox = empty ? 0.0f : total.x / l;
    float oy = empty ? 0.0f : total.y / l;
    if (a.value_center != nullptr) {
      const int kv = qh / kGqa;
      const uint16_t* c = a.value_center + request * a.center_batch_stride + kv * kHeadDim + 2 * lane;
      ox += half_bits_to_float(c[0]);
      oy += half_bits_to_float(c[1]);
    }
    const __half2 h = __floats2half2_rn(ox, oy);
    *reinterpret_cast<__half2*>(a.out + (static_cast<int64_t>(request) * a.num_qo_heads + qh) * kHeadDim +
                                2 * lane) = h;
    if (lane == 0 && a.lse != nullptr)
      a.lse[static_cast<int64_t>(request) * a.num_qo_heads + qh] = empty ? kNegInf : log2f(l) + m;
  }
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
};

__global__ __launch_bounds__(kWave * kMaxWavesPerBlock) void tail_merge_kernel(TailMergeArgs t) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_all[kMaxWavesPerBlock * kLdsPerWave];
  const DecodeArgs& a = t.base;
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int request = blockIdx.x;
  const int kv = blockIdx.y * a.waves_per_block + wave;
  HeadState st;
  init_state(st);
  const int begin = request * t.pages_per_request;
  const int end = begin + t.pages_per_request;
  fp16_pages(a, request, t.exact_k, t.exact_v, t.page_indices, begin, end, end - 1,
             t.last_len[request], kv, lane, lds_all + wave * kLdsPerWave, st);
  const float l_row = row16_sum(st.l);
  const int qh = kv * kGqa + (lane >> 4);
  const int n = lane & 15;
  const int64_t row = static_cast<int64_t>(request) * a.num_qo_heads + qh;
  const float old_lse = t.old_lse[row];
  const float mx = fmaxf(old_lse, st.m);
  const float w_old = (old_lse == kNegInf) ? 0.0f : exp2f(old_lse - mx);
  const float w_new = (st.m == kNegInf) ? 0.0f : exp2f(st.m - mx);
  const float den = w_old + w_new * l_row;
  const float inv = den > 0.0f ? 1.0f / den : 0.0f;
  uint16_t* o = t.old_output + row * kHeadDim;
  const uint16_t* c = t.value_center + request * t.center_batch_stride + kv * kHeadDim;
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) {
    const int d = 64 * (nb >> 2) + 4 * n + (nb & 3);
    const float merged = (w_old * half_bits_to_float(o[d]) + w_new * st.o[nb]) * inv +
                         half_bits_to_float(c[d]);
    o[d] = __half_as_ushort(__float2half_rn(merged));
  }
  if (n == 0) t.old_lse[row] = den > 0.0f ? log2f(den) + mx : kNegInf;
}

int waves_per_block_for(int hkv) {
  for (int w = kMaxWavesPerBlock; w > 1; w >>= 1)
    if (hkv % w == 0) return w;
  return 1;
}

int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

}  // namespace
}  // namespace pg

using namespace pg;

extern "C" int64_t pg_decode_workspace_bytes(int32_t batch_size, int32_t num_qo_heads,
                                             int64_t max_items) {
  if (batch_size <= 0 || num_qo_heads <= 0 || max_items <= 0) return 0;
  int64_t bytes = align_up(max_items * static_cast<int64_t>(sizeof(WorkItem)), 256);
  bytes += align_up((batch_size + 1) * static_cast<int64_t>(sizeof(int32_t)), 256);
  bytes += align_up(max_items * num_qo_heads * static_cast<int64_t>(kHeadDim + 2) * 4, 256);
  return bytes;
}

extern "C" int32_t pg_select_split_pages(int64_t total_pages, int32_t batch_size,
                                         int32_t num_kv_heads, int32_t bytes_per_page,
                                         int32_t num_cus) {
  // One workgroup carries all KV heads of a page range, so the number of
  // workgroups is the number of page chunks.  A 512-thread block of eight
  // KV-head waves occupies two waves per SIMD, i.e. one block per CU at a
  // time: aim for one chunk per CU so the whole decode is a single wave of
  // workgroups.  Chunks never shrink below 4 pages (one PV MFMA group).
  // ``total_pages`` is weighted in units of ``bytes_per_page``.
  (void)num_kv_heads;
  (void)bytes_per_page;
  if (total_pages <= 0) return kGroupPages;
  if (num_cus <= 0) num_cus = 256;
  const int64_t target_items = std::max<int64_t>(num_cus, batch_size);
  int64_t split = (total_pages + target_items - 1) / target_items;
  split = std::max<int64_t>(split, kGroupPages);
  return static_cast<int32_t>(std::min<int64_t>(split, 1 << 20));
}

extern "C" int32_t pg_decode_plan(const int32_t* host_indptr, const int32_t* host_last_page_len,
                                  int32_t batch_size, int32_t primary_kind,
                                  const int32_t* host_tail_indptr,
                                  const int32_t* host_tail_last_len, int32_t num_qo_heads,
                                  int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                  int32_t split_pages, int32_t tail_split_pages, int32_t num_cus,
                                  void* workspace, int64_t workspace_bytes, pg_decode_plan_t* plan,
                                  void* stream) {
  clear_error();
  if (!host_indptr || !host_last_page_len || !plan || !workspace)
    return fail(PG_ERROR_INVALID_ARGUMENT, "null plan argument");
  if (batch_size <= 0) return fail(PG_ERROR_INVALID_ARGUMENT, "batch size must be positive");
  if (head_dim != kHeadDim) return fail(PG_ERROR_UNSUPPORTED, "head dimension must be 128");
  if (page_size != kPageSize) return fail(PG_ERROR_UNSUPPORTED, "page size must be 16");
  if (num_kv_heads <= 0 || num_qo_heads != kGqa * num_kv_heads)
    return fail(PG_ERROR_UNSUPPORTED, "the decode kernel requires GQA group size 4");
  if (num_kv_heads > 64) return fail(PG_ERROR_UNSUPPORTED, "at most 64 KV heads");
  if (primary_kind != PG_KV_INT8 && primary_kind != PG_KV_FP16)
    return fail(PG_ERROR_INVALID_ARGUMENT, "kv kind must be INT8 or FP16");
  if ((host_tail_indptr == nullptr) != (host_tail_last_len == nullptr))
    return fail(PG_ERROR_INVALID_ARGUMENT, "tail indptr and last_page_len go together");

  int64_t primary_pages = 0, tail_pages = 0;
  for (int b = 0; b < batch_size; ++b) {
    const int64_t n = static_cast<int64_t>(host_indptr[b + 1]) - host_indptr[b];
    if (n < 0) return fail(PG_ERROR_INVALID_ARGUMENT, "indptr must be non-decreasing");
    if (n > 0 && (host_last_page_len[b] < 1 || host_last_page_len[b] > kPageSize))
      return fail(PG_ERROR_INVALID_ARGUMENT, "last_page_len must lie in [1, 16]");
    primary_pages += n;
    if (host_tail_indptr) {
      const int64_t tn = static_cast<int64_t>(host_tail_indptr[b + 1]) - host_tail_indptr[b];
      if (tn < 0) return fail(PG_ERROR_INVALID_ARGUMENT, "tail indptr must be non-decreasing");
      if (tn > 0 && (host_tail_last_len[b] < 1 || host_tail_last_len[b] > kPageSize))
        return fail(PG_ERROR_INVALID_ARGUMENT, "tail last_page_len must lie in [1, 16]");
      tail_pages += tn;
    }
  }
  const int primary_bytes = primary_kind == PG_KV_INT8 ? 4096 : 8192;
  if (split_pages <= 0) {
    // FP16 tail pages cost twice the bytes of INT8 pages
    const int64_t weighted = primary_pages + (primary_kind == PG_KV_INT8 ? 2 : 1) * tail_pages;
    split_pages = pg_select_split_pages(weighted, batch_size, num_kv_heads, primary_bytes, num_cus);
  }
  if (tail_split_pages <= 0) {
    // an FP16 page streams twice the bytes of an INT8 page
    tail_split_pages = primary_kind == PG_KV_INT8 ? std::max(1, (split_pages + 1) / 2) : split_pages;
  }

  std::vector<WorkItem> items;
  std::vector<int32_t> item_ptr(batch_size + 1, 0);
  int max_per_request = 0;
  for (int b = 0; b < batch_size; ++b) {
    // Tail (FP16) items of a request come first so they start in the first
    // wave of workgroups next to the INT8 chunks instead of trailing them.
    item_ptr[b] = static_cast<int32_t>(items.size());
    if (host_tail_indptr) {
      const int tb = host_tail_indptr[b], te = host_tail_indptr[b + 1];
      for (int s = tb; s < te; s += tail_split_pages)
        items.push_back(WorkItem{b, PG_KV_FP16, 1, s, std::min(te, s + tail_split_pages), te - 1, 0, 0});
    }
    const int pb = host_indptr[b], pe = host_indptr[b + 1];
    for (int s = pb; s < pe; s += split_pages)
      items.push_back(WorkItem{b, primary_kind, 0, s, std::min(pe, s + split_pages), pe - 1, 0, 0});
    max_per_request = std::max(max_per_request, static_cast<int>(items.size()) - item_ptr[b]);
  }
  item_ptr[batch_size] = static_cast<int32_t>(items.size());
  if (max_per_request > kMaxItemsPerRequest)
    return fail(PG_ERROR_UNSUPPORTED, "too many splits per request; raise split_pages");
  const int64_t n_items = std::max<int64_t>(1, static_cast<int64_t>(items.size()));
  const int64_t needed = pg_decode_workspace_bytes(batch_size, num_qo_heads, n_items);
  if (needed > workspace_bytes)
    return fail(PG_ERROR_WORKSPACE, "decode workspace too small: need " + std::to_string(needed) +
                                        " bytes, have " + std::to_string(workspace_bytes));

  pg_decode_plan_t p{};
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
  p.items_offset = 0;
  p.item_ptr_offset = align_up(n_items * static_cast<int64_t>(sizeof(WorkItem)), 256);
  p.partial_offset = p.item_ptr_offset + align_up((batch_size + 1) * 4, 256);
  p.workspace_bytes = needed;

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

struct PartialViews {
  float* o;
  float* m;
  float* l;
};

PartialViews partial_views(const pg_decode_plan_t* plan, void* workspace) {
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const int64_t n_items = std::max<int64_t>(1, plan->num_items);
  PartialViews v;
  v.o = reinterpret_cast<float*>(ws + plan->partial_offset);
  v.m = v.o + n_items * plan->num_qo_heads * kHeadDim;
  v.l = v.m + n_items * plan->num_qo_heads;
  return v;
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
  clear_error();
  if (!plan || !query || !workspace) return fail(PG_ERROR_INVALID_ARGUMENT, "null run argument");
  if (plan->num_items_primary > 0) {
    if (!k_cache || !v_cache || !indices || !last_page_len)
      return fail(PG_ERROR_INVALID_ARGUMENT, "primary segment tensors missing");
    if (plan->primary_kind == PG_KV_INT8 && (!k_scale || !v_scale))
      return fail(PG_ERROR_INVALID_ARGUMENT, "INT8 pages need k_scale and v_scale");
  }
  if (plan->num_items > plan->num_items_primary &&
      (!tail_k || !tail_v || !tail_indices || !tail_last_len))
    return fail(PG_ERROR_INVALID_ARGUMENT, "tail segment tensors missing");
  if (!(sm_scale > 0.0f) || !__builtin_isfinite(sm_scale))
    return fail(PG_ERROR_INVALID_ARGUMENT, "sm_scale must be positive and finite");
  if (plan->num_items == 0) return PG_OK;
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
  a.items = reinterpret_cast<const WorkItem*>(static_cast<uint8_t*>(workspace) + plan->items_offset);
  a.partial_o = pv.o;
  a.partial_m = pv.m;
  a.partial_l = pv.l;
  a.num_qo_heads = plan->num_qo_heads;
  a.num_kv_heads = plan->num_kv_heads;
  a.waves_per_block = waves_per_block_for(plan->num_kv_heads);
  a.sm_scale_log2 = sm_scale * 1.4426950408889634f;
  const dim3 grid(plan->num_items, plan->num_kv_heads / a.waves_per_block);
  hipLaunchKernelGGL(decode_partial_kernel, grid, dim3(kWave * a.waves_per_block), 0,
                     as_stream(stream), a);
  return check_launch("decode_partial");
}

extern "C" int32_t pg_decode_run_combine(const pg_decode_plan_t* plan, const void* value_center,
                                         int64_t center_batch_stride, void* out, float* lse,
                                         void* workspace, void* stream) {
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
  hipLaunchKernelGGL(combine_kernel, dim3(plan->batch_size * plan->num_qo_heads),
                     dim3(kCombineThreads), 0, as_stream(stream), c);
  return check_launch("decode_combine");
}

extern "C" int32_t pg_decode_run(const pg_decode_plan_t* plan, const void* query,
                                 int64_t query_batch_stride, const void* k_cache,
                                 const void* v_cache, const void* k_scale, const void* v_scale,
                                 const int32_t* indices, const int32_t* last_page_len,
                                 const void* tail_k, const void* tail_v,
                                 const int32_t* tail_indices, const int32_t* tail_last_len,
                                 const void* value_center, int64_t center_batch_stride, void* out,
                                 float* lse, float sm_scale, void* workspace, void* stream) {
  if (int32_t rc = pg_decode_run_partial(plan, query, query_batch_stride, k_cache, v_cache,
                                         k_scale, v_scale, indices, last_page_len, tail_k, tail_v,
                                         tail_indices, tail_last_len, sm_scale, workspace, stream))
    return rc;
  return pg_decode_run_combine(plan, value_center, center_batch_stride, out, lse, workspace,
                               stream);
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
  t.base.waves_per_block = waves_per_block_for(kv_heads);
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
  hipLaunchKernelGGL(tail_merge_kernel, grid, dim3(kWave * t.base.waves_per_block), 0,
                     as_stream(stream), t);
  return check_launch("exact_tail_merge_center");
}
