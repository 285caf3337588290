// Shared device/host helpers for the gfx950 block-FP8 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fp8_blockwise.h"

namespace fp8b {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

// Largest finite float8_e4m3fn value (0x7E / 0xFE).
constexpr float kFp8Max = 448.0f;
// Lower bound applied to a group's amax before the scale is formed, so an
// all-zero group quantises to zeros with a small finite scale instead of 0/0.
constexpr float kAmaxFloor = 1e-10f;
// float8_e4m3fn NaN byte written for non-finite inputs.
constexpr uint8_t kFp8NaN = 0x7F;

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// fp32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  __bf16 b = (__bf16)f;
  return __builtin_bit_cast(uint16_t, b);
}

// Two fp32 -> two packed bf16 (low half = a).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return (uint32_t)f32_to_bf16_bits(a) | ((uint32_t)f32_to_bf16_bits(b) << 16);
}

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  _Float16 ha = (_Float16)a, hb = (_Float16)b;
  return (uint32_t)__builtin_bit_cast(uint16_t, ha) |
         ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}

// Exact float8_e4m3fn -> fp32 decode (OCP E4M3: bias 7, no inf, S.1111.111 = NaN).
__device__ __forceinline__ float fp8e4m3_to_f32(uint32_t b) {
  const uint32_t sign = (b & 0x80u) << 24;
  const uint32_t e = (b >> 3) & 0xFu;
  const uint32_t m = b & 0x7u;
  float v;
  if (e == 0) {
    v = (float)m * 0x1p-9f;
  } else if (e == 15 && m == 7) {
    v = __uint_as_float(0x7FC00000u);
  } else {
    v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  }
  return __uint_as_float(__float_as_uint(v) | sign);
}

// Max over the 16 lanes of each DPP row (lanes 16r..16r+15) of an unsigned
// value; every lane of the row receives the result.
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
  // quad_perm [1,0,3,2] : xor 1
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  // quad_perm [2,3,0,1] : xor 2
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  // row_half_mirror : lane i <-> 7-i within each half-row
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  // row_mirror : lane i <-> 15-i within the row
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  return v;
}

// Max over the 4 lanes of each DPP quad (lanes 4q..4q+3) of an unsigned
// value; every lane of the quad receives the result.
__device__ __forceinline__ uint32_t row4_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  return v;
}

// Max over the 8 lanes of each DPP half-row (lanes 8h..8h+7) of an unsigned
// value; every lane of the half-row receives the result.
__device__ __forceinline__ uint32_t row8_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  return v;
}

// Per-thread last-error text for the C ABI.
void set_error(const char* msg);

}  // namespace fp8b
