// Device helpers of the per-token-group float8_e4m3fn quantiser and of the
// gated SiLU, shared by the act-quant and silu kernels, the GEMM that
// quantises bf16 activations itself and the gate/up GEMM whose epilogue
// applies SiLU(gate)*up and quantises the result.
// Numerics (the contract written in include/fp8_blockwise.h):
//   amax  = max |x| over the group, taken as the max of the 15-bit magnitude
//           patterns of the bf16 inputs, so NaN (pattern > 0x7F80) wins;
//   scale = max(amax, 1e-10) / 448, rounded as one IEEE fp32 division is
//           (computed without one: scale_from_amax);
//   q     = e4m3fn(x / scale) rounded to nearest even.
//   NaN group -> scale NaN, q = 0x7F; +inf group -> scale +inf, q = signed
//   zero for finite x and 0x7F for +-inf.
#pragma once

#include "common.h"

namespace fp8b {

// x / s rounded to nearest even, for a group scale s > 0 (normal, finite)
// and |x| <= 448 s, given recip = RN(1/s) from one IEEE division per group.
// Markstein's theorem: q0 = RN(x * recip) is within one ulp of x/s, so the
// residual is exact in one FMA and RN(q0 + r*recip) = RN(x/s). The residual
// is formed negated, n = q0*s - x, and enters the last FMA through the
// operand's negation: for x = -0, n = +0 and q0 - n*recip = -0 + -0 = -0,
// where the residual x - q0*s (+0) would give +0, so the sign of x survives
// without a copysign. Below the fp32 normal range the quotient may differ
// from IEEE division in its last bits, but every such value converts to a
// signed fp8 zero (tests/fastdiv_check.c checks every bf16 x and amax).
__device__ __forceinline__ float div_by_scale(float x, float s, float recip) {
  const float q0 = x * recip;
  const float n = fmaf(q0, s, -x);
  return fmaf(-n, recip, q0);
}

// scale = amax / 448 rounded to nearest even without a division: with
// c = RN(1/448), q0 = RN(amax*c) is within an ulp of the quotient, the
// residual amax - q0*448 is exact in one FMA, and RN(q0 + r*c) is the
// correctly rounded quotient (Markstein). Bit-identical to the IEEE division
// for every amax the kernels form (every finite bf16 magnitude, floored at
// 1e-10): checked exhaustively in tests/scale_recip_check.c.
__device__ __forceinline__ float scale_from_amax(float amax) {
  constexpr float c = 0x1.24924ap-9f;  // RN(1/448)
  const float q0 = amax * c;
  const float r = fmaf(-q0, kFp8Max, amax);
  return fmaf(r, c, q0);
}

// RN(1/s) for a group scale: v_rcp_f32 is within one ulp of 1/s, and one
// Newton step y + y*(1 - s*y) (the residual exact in an FMA) then rounds to
// the correctly rounded reciprocal for every s whose mantissa is not all
// ones; no scale_from_amax() result has one. Both facts are checked
// exhaustively in tests/scale_recip_check.c.
__device__ __forceinline__ float recip_of_scale(float s) {
  const float y = __builtin_amdgcn_rcpf(s);
  return fmaf(fmaf(-s, y, 1.0f), y, y);
}

// e4m3fn codes of 8 values of a finite group (scale s, recip = RN(1/s)),
// packed little-endian into two words.
__device__ __forceinline__ void quant8_finite(const float v[8], float scale, float recip,
                                              uint32_t& w0, uint32_t& w1) {
  float y[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = div_by_scale(v[i], scale, recip);
  // (the first convert of a word keeps the old high half, which the second
  // one overwrites: any register serves as the old value)
  int p0 = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], __float_as_int(y[0]), false);
  p0 = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], p0, true);
  int p1 = __builtin_amdgcn_cvt_pk_fp8_f32(y[4], y[5], __float_as_int(y[4]), false);
  p1 = __builtin_amdgcn_cvt_pk_fp8_f32(y[6], y[7], p1, true);
  w0 = (uint32_t)p0;
  w1 = (uint32_t)p1;
}

// Codes and scale of 8 values of a group whose amax is NaN (is_nan) or +inf:
// NaN group -> every code 0x7F, scale NaN; +inf group -> 0x7F for the +-inf
// values, signed zero for the finite ones, scale +inf.
__device__ __forceinline__ void quant8_nonfinite(const float v[8], bool is_nan, uint32_t& w0,
                                                 uint32_t& w1, float& scale) {
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

// Quantise 8 values held by one lane of a 16-lane group of 128.
// `mag` is the max over this lane's 8 bf16 magnitude patterns.
__device__ __forceinline__ void quant_row16_8(const float v[8], uint32_t mag,
                                              uint32_t& w0, uint32_t& w1,
                                              float& scale) {
  const uint32_t gmag = row16_max_u32(mag);
  if (gmag < 0x7F80u) {
    const float amax = fmaxf(bf16_to_f32(gmag), kAmaxFloor);
    scale = scale_from_amax(amax);
    quant8_finite(v, scale, recip_of_scale(scale), w0, w1);
  } else {
    quant8_nonfinite(v, gmag > 0x7F80u, w0, w1, scale);
  }
}

// Quantise 16 values held by one lane of an 8-lane group of 128 (a DPP
// half-row): the arithmetic of quant_row16_8 on twice the values per lane.
// `mag` is the max over this lane's 16 bf16 magnitude patterns; w[0..3] are
// the 16 codes, little-endian.
__device__ __forceinline__ void quant_row8_16(const float v[16], uint32_t mag, uint32_t w[4],
                                              float& scale) {
  const uint32_t gmag = row8_max_u32(mag);
  if (gmag < 0x7F80u) {
    const float amax = fmaxf(bf16_to_f32(gmag), kAmaxFloor);
    scale = scale_from_amax(amax);
    const float recip = recip_of_scale(scale);
    quant8_finite(v, scale, recip, w[0], w[1]);
    quant8_finite(v + 8, scale, recip, w[2], w[3]);
  } else {
    quant8_nonfinite(v, gmag > 0x7F80u, w[0], w[1], scale);
    quant8_nonfinite(v + 8, gmag > 0x7F80u, w[2], w[3], scale);
  }
}

// Quantise 32 values held by one lane of a 4-lane group of 128 (a DPP
// quad): the arithmetic of quant_row16_8 on four times the values per lane.
// `mag` is the max over this lane's 32 bf16 magnitude patterns; w[0..7] are
// the 32 codes, little-endian.
__device__ __forceinline__ void quant_row4_32(const float v[32], uint32_t mag, uint32_t w[8],
                                              float& scale) {
  const uint32_t gmag = row4_max_u32(mag);
  if (gmag < 0x7F80u) {
    const float amax = fmaxf(bf16_to_f32(gmag), kAmaxFloor);
    scale = scale_from_amax(amax);
    const float recip = recip_of_scale(scale);
#pragma unroll
    for (int i = 0; i < 4; ++i) quant8_finite(v + 8 * i, scale, recip, w[2 * i], w[2 * i + 1]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      quant8_nonfinite(v + 8 * i, gmag > 0x7F80u, w[2 * i], w[2 * i + 1], scale);
  }
}

// Max over the 8 bf16 magnitude patterns of one 16-byte load: sign bits
// cleared, then packed 16-bit maxima (v_pk_max_u16).
__device__ __forceinline__ uint32_t max_mag_bf16x8(const v4i raw) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  u16x2 h[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) h[i] = __builtin_bit_cast(u16x2, (uint32_t)raw[i] & 0x7FFF7FFFu);
  const u16x2 m = __builtin_elementwise_max(__builtin_elementwise_max(h[0], h[1]),
                                            __builtin_elementwise_max(h[2], h[3]));
  return max((uint32_t)m[0], (uint32_t)m[1]);
}

// Unpack 8 bf16 (one 16-byte load) into fp32 values and the max magnitude.
__device__ __forceinline__ uint32_t unpack_bf16x8(const v4i raw, float v[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = (uint32_t)raw[i];
    v[2 * i] = __uint_as_float(w << 16);
    v[2 * i + 1] = __uint_as_float(w & 0xFFFF0000u);
  }
  return max_mag_bf16x8(raw);
}

// silu(a) in fp32 (silu_f32), and silu(a) * b with the reference's rounding
// points (silu_mul_bits): silu in fp32, rounded to bf16, multiplied by the
// bf16 `up` value in fp32, rounded to bf16.
// silu(a) = a / (1 + e^-a) is evaluated with the hardware v_exp_f32 and
// v_rcp_f32 instead of expf and an IEEE division (~25 instructions per
// element, which bound the fused quantiser: 55 -> 41 us at [3001, 28672]).
// Accuracy: e^-a = 2^t with t = -a log2(e) split into the rounded product and
// its exact residual (fma) plus the low part of log2(e), the residual applied
// to first order; the reciprocal gets one Newton step. The fp32 silu is then
// within a few ulps of the division's. Overflow and non-finite inputs give
// what the division gives (e^-a = inf -> -0 for finite a, -inf -> NaN,
// NaN -> NaN); for a in about [-88.7, -87.3] the reciprocal is subnormal and
// may flush, giving -0 where the division gives |silu| < 1e-36.
__device__ __forceinline__ float silu_f32(float a) {
  constexpr float kLog2eHi = 1.4426950216293335f;   // log2(e) rounded to fp32
  constexpr float kLog2eLo = 1.925962989091e-08f;   // log2(e) - kLog2eHi
  constexpr float kLn2 = 0.6931471805599453f;
  const float t = -a * kLog2eHi;
  const float r = fmaf(-a, kLog2eHi, -t) - a * kLog2eLo;  // t's residual
  const float e0 = __builtin_amdgcn_exp2f(t);
  // (the correction and the Newton step only where they are finite: an
  // infinite t or e0 makes r or the step NaN)
  const bool e_fin = __builtin_isfinite(t) && e0 < __builtin_inff();
  const float e = e_fin ? fmaf(e0, r * kLn2, e0) : e0;
  const float y = 1.0f + e;
  const float inv0 = __builtin_amdgcn_rcpf(y);
  const float inv = y < __builtin_inff() ? fmaf(inv0, fmaf(-y, inv0, 1.0f), inv0) : inv0;
  return a * inv;
}

__device__ __forceinline__ uint32_t silu_mul_bits(uint32_t gate_bits, uint32_t up_bits) {
  const float silu = silu_f32(bf16_to_f32(gate_bits));
  const float silu_b = bf16_to_f32(f32_to_bf16_bits(silu));
  return f32_to_bf16_bits(silu_b * bf16_to_f32(up_bits));
}

// silu_mul_bits for |gate| < 64 (bf16 magnitude pattern below 0x4280): then
// |t| < 93, so t, e^-a and 1 + e^-a are finite and both guarded corrections
// of silu_mul_bits apply; this is the same arithmetic without the guards.
constexpr uint32_t kSiluFastMag = 0x4280u;  // bf16 pattern of 64.0
__device__ __forceinline__ uint32_t silu_mul_bits_small(uint32_t gate_bits, uint32_t up_bits) {
  constexpr float kLog2eHi = 1.4426950216293335f;
  constexpr float kLog2eLo = 1.925962989091e-08f;
  constexpr float kLn2 = 0.6931471805599453f;
  const float a = bf16_to_f32(gate_bits);
  const float t = -a * kLog2eHi;
  const float r = fmaf(-a, kLog2eHi, -t) - a * kLog2eLo;
  const float e0 = __builtin_amdgcn_exp2f(t);
  const float y = 1.0f + fmaf(e0, r * kLn2, e0);
  const float inv0 = __builtin_amdgcn_rcpf(y);
  const float silu = a * fmaf(inv0, fmaf(-y, inv0, 1.0f), inv0);
  const float silu_b = bf16_to_f32(f32_to_bf16_bits(silu));
  return f32_to_bf16_bits(silu_b * bf16_to_f32(up_bits));
}

// True when every active lane of the wave has pred set (wave-uniform).
__device__ __forceinline__ bool wave_all(bool pred) {
  return __builtin_amdgcn_ballot_w64(!pred) == 0;
}

// SiLU(gate)*up of 8 packed bf16 pairs (one 16-byte load of each): packed
// bf16 results, their fp32 values in v. Takes the guard-free form when every
// gate of the wave is below 64 in magnitude (the same bits either way).
__device__ __forceinline__ v4i silu_mul_bf16x8(const v4i g, const v4i u, float v[8]) {
  v4i h;
  if (wave_all(max_mag_bf16x8(g) < kSiluFastMag)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t gw = (uint32_t)g[i], uw = (uint32_t)u[i];
      const uint32_t lo = silu_mul_bits_small(gw & 0xFFFFu, uw & 0xFFFFu);
      const uint32_t hi = silu_mul_bits_small(gw >> 16, uw >> 16);
      v[2 * i] = bf16_to_f32(lo);
      v[2 * i + 1] = bf16_to_f32(hi);
      h[i] = (int)(lo | (hi << 16));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t gw = (uint32_t)g[i], uw = (uint32_t)u[i];
      const uint32_t lo = silu_mul_bits(gw & 0xFFFFu, uw & 0xFFFFu);
      const uint32_t hi = silu_mul_bits(gw >> 16, uw >> 16);
      v[2 * i] = bf16_to_f32(lo);
      v[2 * i + 1] = bf16_to_f32(hi);
      h[i] = (int)(lo | (hi << 16));
    }
  }
  return h;
}

}  // namespace fp8b
