/*
 * C restatement of the PageGauge compressed-KV decode path.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (as a second, independent engine
 * beside the numpy oracle) and by bench.py's CPU-baseline leg.  The product
 * library never links or calls it.
 *
 * FP16 arithmetic is emulated with this file's own IEEE binary16 rounding
 * (round-to-nearest-even from double, subnormals kept); FP32 arithmetic uses
 * C float with IEEE semantics (build without -ffast-math, with
 * -ffp-contract=off).  Citations are relative to the PageGauge reference tree.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define PG_PAGE 16
#define PG_DIM 128
#define PG_HALF 64

/* ---- binary16 helpers (own implementation, IEEE 754 RN-even) ---------- */

static double half_to_double(uint16_t h) {
  const int sign = (h >> 15) & 1;
  const int exponent = (h >> 10) & 0x1f;
  const int mantissa = h & 0x3ff;
  double value;
  if (exponent == 0) {
    value = ldexp((double)mantissa, -24);
  } else if (exponent == 31) {
    value = mantissa ? NAN : INFINITY;
  } else {
    value = ldexp((double)(mantissa | 0x400), exponent - 25);
  }
  return sign ? -value : value;
}

static float half_to_float(uint16_t h) { return (float)half_to_double(h); }

/* Round a double to binary16, nearest-even.  Exact for every double: the
 * scaled significand is split into integer and remainder parts with exact
 * double arithmetic (ldexp/floor are exact). */
static uint16_t double_to_half(double x) {
  if (isnan(x)) return 0x7e00;
  uint16_t sign = signbit(x) ? 0x8000 : 0;
  double a = fabs(x);
  if (a == 0.0) return sign;
  if (isinf(a)) return sign | 0x7c00;
  int e;
  frexp(a, &e);          /* a = f * 2^e, f in [0.5,1) */
  int exponent = e - 1;  /* a in [2^exponent, 2^(exponent+1)) */
  if (exponent < -14) exponent = -14; /* subnormal range: fixed quantum 2^-24 */
  const double quantum = ldexp(1.0, exponent - 10);
  const double scaled = a / quantum; /* exact: power-of-two division */
  double integral = floor(scaled);
  const double rest = scaled - integral;
  if (rest > 0.5 || (rest == 0.5 && fmod(integral, 2.0) != 0.0)) integral += 1.0;
  /* integral in [0, 2048]; renormalise */
  double value = integral * quantum;
  if (value >= 65520.0) return sign | 0x7c00;
  if (value == 0.0) return sign;
  if (value < ldexp(1.0, -14)) {
    return sign | (uint16_t)integral; /* subnormal: mantissa = value / 2^-24 */
  }
  frexp(value, &e);
  exponent = e - 1;
  const int mantissa = (int)(ldexp(value, -exponent) * 1024.0 - 1024.0);
  return sign | (uint16_t)(((exponent + 15) << 10) | mantissa);
}

static uint16_t float_to_half(float x) { return double_to_half((double)x); }

uint16_t pgo_double_to_half(double x) { return double_to_half(x); }
double pgo_half_to_double(uint16_t h) { return half_to_double(h); }

/* ---- A1 RoPE (tests/page_gauge_append_extension.cu:148-180) ------------ */

static uint16_t rope_element(const uint16_t* x, const uint16_t* c, const uint16_t* s, int d) {
  uint16_t partner = d < PG_HALF ? (uint16_t)(x[d + PG_HALF] ^ 0x8000u) : x[d - PG_HALF];
  const uint16_t p1 = double_to_half(half_to_double(x[d]) * half_to_double(c[d]));
  const uint16_t p2 = double_to_half(half_to_double(partner) * half_to_double(s[d]));
  return double_to_half(half_to_double(p1) + half_to_double(p2));
}

/* rows x [rows][128] -> y, shared cos/sin rows. */
void pgo_rope_rotate(const uint16_t* x, const uint16_t* c, const uint16_t* s, uint16_t* y,
                     int64_t rows) {
  for (int64_t r = 0; r < rows; ++r)
    for (int d = 0; d < PG_DIM; ++d) y[r * PG_DIM + d] = rope_element(x + r * PG_DIM, c, s, d);
}

/* ---- A3 scale and codes (tests/page_gauge_append_extension.cu:333-382) - */

static uint16_t scale_from_max(float maximum) {
  volatile float quotient = maximum / 127.0f; /* IEEE float division */
  float clamped = quotient > 0x1p-20f ? quotient : 0x1p-20f;
  return float_to_half(clamped);
}

static int8_t code_from_quotient(float q) {
  int code;
  if (q >= 0.0f) {
    volatile float shifted = q + 0.5f;
    code = (int)floorf(shifted);
  } else {
    volatile float shifted = -q + 0.5f;
    code = -(int)floorf(shifted);
  }
  if (code > 127) code = 127;
  if (code < -127) code = -127;
  return (int8_t)code;
}

/* One [16][heads][128] fp16 page -> codes (same layout) + scales[heads]. */
void pgo_finalize_page(const uint16_t* page, int heads, int8_t* codes, uint16_t* scales) {
  for (int h = 0; h < heads; ++h) {
    float maximum = 0.0f;
    for (int t = 0; t < PG_PAGE; ++t)
      for (int d = 0; d < PG_DIM; ++d) {
        const float v = fabsf(half_to_float(page[((int64_t)t * heads + h) * PG_DIM + d]));
        if (v > maximum) maximum = v;
      }
    const uint16_t stored = scale_from_max(maximum);
    scales[h] = stored;
    const float scale = half_to_float(stored);
    for (int t = 0; t < PG_PAGE; ++t)
      for (int d = 0; d < PG_DIM; ++d) {
        const int64_t i = ((int64_t)t * heads + h) * PG_DIM + d;
        volatile float quotient = half_to_float(page[i]) / scale;
        codes[i] = code_from_quotient(quotient);
      }
  }
}

/* ---- a14 bulk quantizer (scripts/benchmark_page_gauge_overheads.py:23-83) */

void pgo_quantize_completed(const uint16_t* values, const uint16_t* center, int64_t pages,
                            int heads, int8_t* codes, uint16_t* scales) {
  float* centered = (float*)malloc(sizeof(float) * PG_PAGE * PG_DIM);
  for (int64_t p = 0; p < pages; ++p)
    for (int h = 0; h < heads; ++h) {
      float maximum = 0.0f;
      for (int t = 0; t < PG_PAGE; ++t)
        for (int d = 0; d < PG_DIM; ++d) {
          const int64_t i = ((p * PG_PAGE + t) * heads + h) * PG_DIM + d;
          volatile float v = half_to_float(values[i]) - half_to_float(center[h * PG_DIM + d]);
          centered[t * PG_DIM + d] = v;
          if (fabsf(v) > maximum) maximum = fabsf(v);
        }
      const uint16_t stored = scale_from_max(maximum);
      scales[p * heads + h] = stored;
      const float scale = half_to_float(stored);
      for (int t = 0; t < PG_PAGE; ++t)
        for (int d = 0; d < PG_DIM; ++d) {
          const int64_t i = ((p * PG_PAGE + t) * heads + h) * PG_DIM + d;
          volatile float quotient = centered[t * PG_DIM + d] / scale;
          codes[i] = code_from_quotient(quotient);
        }
    }
  free(centered);
}

/* ---- A4 decode (scripts/benchmark_flashinfer_page_affine_int8.py:566-602)
 *
 * Dense float32 restatement of the segmented path: dequantise each INT8 page
 * (code * page scale), join the centered FP16 tail, softmax over all tokens of
 * the request, add the value center.  Two passes per (request, query head):
 * scores, then exp2-weights and the weighted value sum.  Outputs fp16 out and
 * float32 base-2 lse.  Single-threaded; this is the timed CPU baseline.
 */
void pgo_decode_page_gauge(const uint16_t* query, int batch, int hq, int hkv,
                           const int8_t* k_codes, const int8_t* v_codes,
                           const uint16_t* k_scale, const uint16_t* v_scale,
                           const int32_t* indptr, const int32_t* indices,
                           const int32_t* last_page_len,
                           const uint16_t* tail_k, const uint16_t* tail_v,
                           const int32_t* tail_indptr, const int32_t* tail_indices,
                           const int32_t* tail_last_len, const uint16_t* value_center,
                           int center_batched, float sm_scale, uint16_t* out, float* lse) {
  const int group = hq / hkv;
  const float scale_log2 = sm_scale * 1.4426950408889634f;
  int64_t max_tokens = 0;
  for (int b = 0; b < batch; ++b) {
    int64_t tokens = (int64_t)(indptr[b + 1] - indptr[b]) * PG_PAGE;
    if (tail_indptr) tokens += (int64_t)(tail_indptr[b + 1] - tail_indptr[b]) * PG_PAGE;
    if (tokens > max_tokens) max_tokens = tokens;
  }
  float* scores = (float*)malloc(sizeof(float) * (size_t)(max_tokens > 0 ? max_tokens : 1) * group);
  float qf[8][PG_DIM];
  float acc[8][PG_DIM];
  float kd[PG_DIM];
  for (int b = 0; b < batch; ++b) {
    for (int kv = 0; kv < hkv; ++kv) {
      for (int g = 0; g < group; ++g)
        for (int d = 0; d < PG_DIM; ++d)
          qf[g][d] = half_to_float(query[((int64_t)b * hq + kv * group + g) * PG_DIM + d]);
      /* pass 1: scores */
      int64_t n = 0;
      for (int seg = 0; seg < 2; ++seg) {
        const int32_t* ip = seg == 0 ? indptr : tail_indptr;
        const int32_t* ix = seg == 0 ? indices : tail_indices;
        const int32_t* ll = seg == 0 ? last_page_len : tail_last_len;
        if (!ip) continue;
        for (int32_t e = ip[b]; e < ip[b + 1]; ++e) {
          const int64_t page = ix[e];
          const int tokens = e == ip[b + 1] - 1 ? ll[b] : PG_PAGE;
          const float sk = seg == 0 ? half_to_float(k_scale[page * hkv + kv]) : 1.0f;
          for (int t = 0; t < tokens; ++t) {
            const int64_t base = ((page * PG_PAGE + t) * hkv + kv) * PG_DIM;
            if (seg == 0)
              for (int d = 0; d < PG_DIM; ++d) kd[d] = (float)k_codes[base + d] * sk;
            else
              for (int d = 0; d < PG_DIM; ++d) kd[d] = half_to_float(tail_k[base + d]);
            for (int g = 0; g < group; ++g) {
              float s = 0.0f;
              for (int d = 0; d < PG_DIM; ++d) s += qf[g][d] * kd[d];
              scores[n * group + g] = s * scale_log2;
            }
            ++n;
          }
        }
      }
      /* pass 2: softmax and values */
      float m[8], l[8];
      for (int g = 0; g < group; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
        for (int64_t i = 0; i < n; ++i) if (scores[i * group + g] > m[g]) m[g] = scores[i * group + g];
        for (int d = 0; d < PG_DIM; ++d) acc[g][d] = 0.0f;
      }
      n = 0;
      for (int seg = 0; seg < 2; ++seg) {
        const int32_t* ip = seg == 0 ? indptr : tail_indptr;
        const int32_t* ix = seg == 0 ? indices : tail_indices;
        const int32_t* ll = seg == 0 ? last_page_len : tail_last_len;
        if (!ip) continue;
        for (int32_t e = ip[b]; e < ip[b + 1]; ++e) {
          const int64_t page = ix[e];
          const int tokens = e == ip[b + 1] - 1 ? ll[b] : PG_PAGE;
          const float sv = seg == 0 ? half_to_float(v_scale[page * hkv + kv]) : 1.0f;
          for (int t = 0; t < tokens; ++t) {
            const int64_t base = ((page * PG_PAGE + t) * hkv + kv) * PG_DIM;
            if (seg == 0)
              for (int d = 0; d < PG_DIM; ++d) kd[d] = (float)v_codes[base + d] * sv;
            else
              for (int d = 0; d < PG_DIM; ++d) kd[d] = half_to_float(tail_v[base + d]);
            for (int g = 0; g < group; ++g) {
              const float w = exp2f(scores[n * group + g] - m[g]);
              l[g] += w;
              for (int d = 0; d < PG_DIM; ++d) acc[g][d] += w * kd[d];
            }
            ++n;
          }
        }
      }
      for (int g = 0; g < group; ++g) {
        const int qh = kv * group + g;
        for (int d = 0; d < PG_DIM; ++d) {
          float o = n > 0 ? acc[g][d] / l[g] : 0.0f;
          if (value_center) {
            const int64_t c = ((int64_t)(center_batched ? b : 0) * hkv + kv) * PG_DIM + d;
            o += half_to_float(value_center[c]);
          }
          out[((int64_t)b * hq + qh) * PG_DIM + d] = float_to_half(o);
        }
        lse[(int64_t)b * hq + qh] = n > 0 ? log2f(l[g]) + m[g] : -INFINITY;
      }
    }
  }
  free(scores);
}
