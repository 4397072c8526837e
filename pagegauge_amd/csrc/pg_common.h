// Shared definitions of the PageGauge MI355X (gfx950) library.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <string>

#include "pg_host.h"

namespace pg {

inline int32_t check_launch(const char* what) {
  hipError_t status = hipGetLastError();
  if (status != hipSuccess) {
    return fail(PG_ERROR_LAUNCH, std::string(what) + ": " + hipGetErrorString(status));
  }
  return PG_OK;
}

inline hipStream_t as_stream(void* stream) { return reinterpret_cast<hipStream_t>(stream); }

// -- device helpers ------------------------------------------------------

__device__ __forceinline__ float half_bits_to_float(uint16_t bits) {
  return __half2float(__ushort_as_half(bits));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, kWave));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, kWave);
  return v;
}

// Reductions over the 16 lanes of one DPP row (lanes 16*r .. 16*r+15):
// rotations by 8, 4, 2, 1 within the row leave every lane with the result.
template <int kRor>
__device__ __forceinline__ float row_ror(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x120 + kRor, 0xf, 0xf, false));
}

__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, row_ror<8>(v));
  v = fmaxf(v, row_ror<4>(v));
  v = fmaxf(v, row_ror<2>(v));
  v = fmaxf(v, row_ror<1>(v));
  return v;
}

__device__ __forceinline__ float row16_sum(float v) {
  v += row_ror<8>(v);
  v += row_ror<4>(v);
  v += row_ror<2>(v);
  v += row_ror<1>(v);
  return v;
}

}  // namespace pg
