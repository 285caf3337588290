// Device helpers of the per-token-group float8_e4m3fn quantiser, shared by
// the act-quant kernels and the GEMM that quantises bf16 activations itself.
// Numerics (the contract written in include/fp8_blockwise.h):
//   amax  = max |x| over the group, taken as the max of the 15-bit magnitude
//           patterns of the bf16 inputs, so NaN (pattern > 0x7F80) wins;
//   scale = max(amax, 1e-10) / 448 as one IEEE fp32 division;
//   q     = e4m3fn(x / scale) rounded to nearest even.
//   NaN group -> scale NaN, q = 0x7F; +inf group -> scale +inf, q = signed
//   zero for finite x and 0x7F for +-inf.
#pragma once

#include "common.h"

namespace fp8b {

// x / s rounded to nearest even, for a group scale s > 0 (normal, finite)
// and |x| <= 448 s, given recip = RN(1/s) from one IEEE division per group.
// Markstein's theorem: q0 = RN(x * recip) is within one ulp of x/s, so
// r = x - q0*s is exact in one FMA and RN(q0 + r*recip) = RN(x/s). The sign
// is copied from x so that -0 stays -0 (q0 + r*recip would give +0). Below
// the fp32 normal range the quotient may differ from IEEE division in its
// last bits, but every such value converts to a signed fp8 zero.
__device__ __forceinline__ float div_by_scale(float x, float s, float recip) {
  const float q0 = x * recip;
  const float r = fmaf(-q0, s, x);
  return __builtin_copysignf(fmaf(r, recip, q0), x);
}

// Quantise 8 values held by one lane of a 16-lane group of 128.
// `mag` is the max over this lane's 8 bf16 magnitude patterns.
__device__ __forceinline__ void quant_row16_8(const float v[8], uint32_t mag,
                                              uint32_t& w0, uint32_t& w1,
                                              float& scale) {
  const uint32_t gmag = row16_max_u32(mag);
  if (gmag < 0x7F80u) {
    const float amax = fmaxf(bf16_to_f32(gmag), kAmaxFloor);
    scale = amax / kFp8Max;
    const float recip = 1.0f / scale;
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = div_by_scale(v[i], scale, recip);
    int p0 = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
    p0 = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], p0, true);
    int p1 = __builtin_amdgcn_cvt_pk_fp8_f32(y[4], y[5], 0, false);
    p1 = __builtin_amdgcn_cvt_pk_fp8_f32(y[6], y[7], p1, true);
    w0 = (uint32_t)p0;
    w1 = (uint32_t)p1;
  } else {
    const bool is_nan = gmag > 0x7F80u;
    scale = is_nan ? __uint_as_float(0x7FC00000u) : __uint_as_float(0x7F800000u);
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t u = __float_as_uint(v[i]);
      const bool nonfinite = (u & 0x7FFFFFFFu) >= 0x7F800000u;
      b[i] = (is_nan || nonfinite) ? kFp8NaN : ((u >> 24) & 0x80u);
    }
    w0 = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
    w1 = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
  }
}

// Unpack 8 bf16 (one 16-byte load) into fp32 values and the max magnitude.
__device__ __forceinline__ uint32_t unpack_bf16x8(const v4i raw, float v[8]) {
  uint32_t mag = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = (uint32_t)raw[i];
    const uint32_t lo = w & 0xFFFFu, hi = w >> 16;
    v[2 * i] = bf16_to_f32(lo);
    v[2 * i + 1] = bf16_to_f32(hi);
    mag = max(mag, max(lo & 0x7FFFu, hi & 0x7FFFu));
  }
  return mag;
}

}  // namespace fp8b
