// Per-token-group float8_e4m3fn quantisation and gated SiLU for gfx950.
//
// Layout: x is bf16 row-major [M,K]; every row is cut into groups of `group`
// consecutive elements. A group of 128 bf16 is 256 contiguous bytes, read by
// 16 lanes (one DPP row) with one 16-byte load each, so a wavefront covers
// four groups per load instruction and the whole wave's request is 1 KiB of
// consecutive memory when the four groups sit in one row. fp16 and fp32
// inputs take the typed kernels further down (same contract on the fp32
// values of x).
//
// Numerics (the contract written in include/fp8_blockwise.h):
//   amax  = max |x| over the group, taken as the max of the 15-bit magnitude
//           patterns of the bf16 inputs, so NaN (pattern > 0x7F80) wins;
//   scale = max(amax, 1e-10) / 448 rounded as one IEEE fp32 division;
//   q     = e4m3fn(x / scale) with the quotient rounded as IEEE fp32
//           division, then the gfx950 OCP fp8 convert (round to nearest
//           even). |x/scale| <= 448 * (1 + 2^-23) for finite groups, which
//           the convert rounds into range.
// The kernels form the scale, its reciprocal and the quotients without
// division instructions (quant.h); the results are the IEEE ones, checked
// over their whole input domain in tests/scale_recip_check.c and
// tests/fastdiv_check.c.
//   NaN group -> scale NaN, q = 0x7F; +inf group -> scale +inf, q = signed
//   zero for finite x and 0x7F for +-inf.
#include "common.h"
#include "quant.h"

#include <algorithm>

namespace fp8b {

// Fast path: group = 128, K % 128 == 0, 16-byte aligned rows of x, 8-byte
// aligned rows of q. 16 lanes per group (one 16-byte load each). Block
// (bx, by) quantises groups bx*16U .. bx*16U + 16U - 1 of rows by,
// by + gridDim.y, ...: 16-lane row r of the block takes groups
// bx*16U + r + 16u, u < U, and issues all U loads before converting any.
// The row is uniform over the block, so its base addresses are scalar and
// each lane adds a 32-bit offset (no per-lane index division).
// For U > 1 the block's 16U scales of a row go through LDS and leave as one
// contiguous store (16U lanes) instead of U four-float stores per wave;
// two LDS slots alternate between rows, so one barrier per row suffices.
// (R: 16-lane rows per block, 16 here and 16, 8 or 4 in the SiLU kernel;
// a block column holds R*U groups and 16-lane row r takes r + R*u.)
template <int R>
__device__ __forceinline__ void store_group_scale(float* sc, uint32_t u, float scale) {
  if ((threadIdx.x & 15u) == 0) sc[(threadIdx.x >> 4) + (uint32_t)R * u] = scale;
}

template <int N>
__device__ __forceinline__ void flush_group_scales(const float* sc, float* sr, int64_t ssg,
                                                   uint32_t groups_per_row) {
  __syncthreads();
  const uint32_t g = blockIdx.x * (uint32_t)N + threadIdx.x;
  if (threadIdx.x < (uint32_t)N && g < groups_per_row) sr[(int64_t)g * ssg] = sc[threadIdx.x];
}

template <int U>
__global__ void __launch_bounds__(256)
act_quant_g128_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                      uint8_t* __restrict__ q, int64_t ldq,
                      float* __restrict__ s, int64_t ssm, int64_t ssg,
                      uint32_t rows, uint32_t groups_per_row) {
  const uint32_t sub = threadIdx.x & 15u;
  const uint32_t g0 = blockIdx.x * 16u * U + (threadIdx.x >> 4);
  __shared__ float sc[2][16 * U];
  uint32_t par = 0;
  for (uint32_t m = blockIdx.y; m < rows; m += gridDim.y, par ^= 1u) {
    const uint16_t* xr = x + (int64_t)m * ldx;
    v4i raw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t g = min(g0 + 16u * u, groups_per_row - 1);  // uniform per 16-lane row
      raw[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(xr + g * 128u + sub * 8u));
    }
    uint8_t* qr = q + (int64_t)m * ldq;
    float* sr = s + (int64_t)m * ssm;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t g = g0 + 16u * u;
      if (g >= groups_per_row) break;  // uniform across the 16-lane group
      float v[8];
      const uint32_t mag = unpack_bf16x8(raw[u], v);
      uint32_t w0, w1;
      float scale;
      quant_row16_8(v, mag, w0, w1, scale);
      v2i packed;
      packed[0] = (int)w0;
      packed[1] = (int)w1;
      __builtin_nontemporal_store(packed, reinterpret_cast<v2i*>(qr + g * 128u + sub * 8u));
      if constexpr (U == 1) {
        if (sub == 0) sr[(int64_t)g * ssg] = scale;
      } else {
        store_group_scale<16>(sc[par], u, scale);
      }
    }
    if constexpr (U > 1) flush_group_scales<16 * U>(sc[par], sr, ssg, groups_per_row);
  }
}

// Rows of fewer than 16 groups (K below 2048): the 16-lane rows of a block
// take consecutive (row, group) pairs of the flattened [M x groups_per_row]
// index space, so none idles (the row-mapped kernel leaves 16 - groups of
// its 16). Same arithmetic per group.
__global__ void __launch_bounds__(256)
act_quant_g128_flat_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                           uint8_t* __restrict__ q, int64_t ldq,
                           float* __restrict__ s, int64_t ssm, int64_t ssg,
                           uint32_t slots, uint32_t groups_per_row) {
  const uint32_t sub = threadIdx.x & 15u;
  const uint32_t slot = blockIdx.x * 16u + (threadIdx.x >> 4);
  if (slot >= slots) return;  // uniform across the 16-lane row
  const uint32_t m = slot / groups_per_row, g = slot - m * groups_per_row;
  const v4i raw = __builtin_nontemporal_load(
      reinterpret_cast<const v4i*>(x + (int64_t)m * ldx + g * 128u + sub * 8u));
  float v[8];
  const uint32_t mag = unpack_bf16x8(raw, v);
  uint32_t w0, w1;
  float scale;
  quant_row16_8(v, mag, w0, w1, scale);
  v2i packed;
  packed[0] = (int)w0;
  packed[1] = (int)w1;
  __builtin_nontemporal_store(packed,
                              reinterpret_cast<v2i*>(q + (int64_t)m * ldq + g * 128u + sub * 8u));
  if (sub == 0) s[(int64_t)m * ssm + (int64_t)g * ssg] = scale;
}

// Groups per block column of the fast kernels: 16*U with U in {4, 2, 1}.
// 1 when there are few groups in all (decode: spread them over as many CUs
// as possible); else 4 or 2 when that divides the groups of a row (no idle
// 16-lane rows at the row's end). Other rows still take 4 or 2: the loads
// each lane has in flight count for more than the idle rows of the last
// column. U = 4 when the row fits one 64-group column that U = 2 would need
// two columns for, 2 otherwise. Measured (graph replays over 4 input sets,
// M x K bf16): 8192 x 7168 29.0 us at U = 4, 30.9 at U = 2, 35.4 at U = 1;
// 4096 x 14336 30.0 us at U = 2, 30.7 at U = 4, 33.3 at U = 1. Blocks of 8
// or 4 16-lane rows that split such rows exactly measured level or slower
// here (4096 x 14336 30.4 us at 8 rows x 2 or 7 groups, 8192 x 7168 30.4
// at 8 x 7).
inline int g128_unroll(int64_t rows, int64_t gpr) {
  if (rows * gpr < 16 * 1024) return 1;
  if (gpr % 64 == 0) return 4;
  if (gpr % 32 == 0) return 2;
  return gpr > 32 && gpr < 64 ? 4 : 2;
}

// Block shape of silu_mul_quant_g128_kernel: R 16-lane rows of U groups.
// A lane loads two vectors per group (gate and up), so U = 2 already keeps
// four loads in flight; rows whose group count is a multiple of 8 (but not
// of 64) take U = 2 and the largest R of 16, 8, 4 that splits the row
// exactly, the rest the act-quant shape (R = 16, U from g128_unroll).
// Measured (graph replays over 4 input sets, M x 2d bf16 in): d = 14336
// (112 groups) 3001 rows 39.3 us at R = 8 against 40.4 at 16 x 1 (one
// group per lane, no idle rows), 4096 rows 51.7 against 54.1; d = 7168 (56 groups) 8192
// rows 52.3 at R = 4 against 53.2 at 16 x 4 with 8 idle rows, 1024 rows 8.8
// against 9.5; 16 x 7 and 8 x 7 (one or two blocks per row) level or slower.
inline void silu_quant_shape(int64_t rows, int64_t gpr, int& R, int& U) {
  R = 16;
  U = g128_unroll(rows, gpr);
  if (rows * gpr < 16 * 1024 || gpr % 64 == 0 || gpr % 8 != 0) return;
  U = 2;
  R = (gpr / 2) % 16 == 0 ? 16 : (gpr / 2) % 8 == 0 ? 8 : 4;
}

// Scalar reference-shaped path for any group size, ragged K or unaligned
// rows: one thread walks one group serially.
__device__ __forceinline__ uint8_t quant_scalar(float xv, uint32_t gmag, float scale) {
  if (gmag > 0x7F80u) return kFp8NaN;
  if (gmag == 0x7F80u) {
    const uint32_t u = __float_as_uint(xv);
    if ((u & 0x7FFFFFFFu) >= 0x7F800000u) return kFp8NaN;
    return (uint8_t)((u >> 24) & 0x80u);
  }
  const float y = xv / scale;
  return (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(y, 0.0f, 0, false) & 0xFF);
}

__device__ __forceinline__ float scale_from_mag(uint32_t gmag) {
  if (gmag > 0x7F80u) return __uint_as_float(0x7FC00000u);
  if (gmag == 0x7F80u) return __uint_as_float(0x7F800000u);
  return fmaxf(bf16_to_f32(gmag), kAmaxFloor) / kFp8Max;
}

__global__ void __launch_bounds__(64)
act_quant_generic_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                         uint8_t* __restrict__ q, int64_t ldq,
                         float* __restrict__ s, int64_t ssm, int64_t ssg,
                         int64_t M, int64_t K, int64_t group, int64_t groups_per_row) {
  const int64_t gi = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (gi >= M * groups_per_row) return;
  const int64_t m = gi / groups_per_row;
  const int64_t g = gi - m * groups_per_row;
  const int64_t k0 = g * group;
  const int64_t k1 = min(k0 + group, K);
  const uint16_t* xr = x + m * ldx;
  uint32_t gmag = 0;
  for (int64_t k = k0; k < k1; ++k) gmag = max(gmag, (uint32_t)(xr[k] & 0x7FFFu));
  const float scale = scale_from_mag(gmag);
  uint8_t* qr = q + m * ldq;
  for (int64_t k = k0; k < k1; ++k) qr[k] = quant_scalar(bf16_to_f32(xr[k]), gmag, scale);
  s[m * ssm + g * ssg] = scale;
}

// 8 outputs per thread; requires d % 8 == 0 and 16-byte aligned rows.
__global__ void __launch_bounds__(256)
silu_and_mul_vec_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                        uint16_t* __restrict__ out, int64_t ldo,
                        uint32_t chunks, uint32_t chunks_per_row, int64_t d) {
  const uint32_t ci = blockIdx.x * 256u + threadIdx.x;
  if (ci >= chunks) return;
  const uint32_t m = ci / chunks_per_row;
  const uint32_t c = ci - m * chunks_per_row;
  const uint16_t* xr = x + (int64_t)m * ldx + c * 8u;
  const v4i g = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(xr));
  const v4i u = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(xr + d));
  float v[8];
  const v4i o = silu_mul_bf16x8(g, u, v);
  __builtin_nontemporal_store(o, reinterpret_cast<v4i*>(out + (int64_t)m * ldo + c * 8u));
}

__global__ void __launch_bounds__(256)
silu_and_mul_generic_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                            uint16_t* __restrict__ out, int64_t ldo, int64_t M, int64_t d) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= M * d) return;
  const int64_t m = i / d, j = i - m * d;
  out[m * ldo + j] = (uint16_t)silu_mul_bits(x[m * ldx + j], x[m * ldx + d + j]);
}

// Element type codes of the typed silu_and_mul (fp8b_dtype values).
template <int T> __device__ __forceinline__ float load_as_f32(const void* p, int64_t i) {
  if constexpr (T == FP8B_F32) return static_cast<const float*>(p)[i];
  else if constexpr (T == FP8B_F16) return (float)static_cast<const _Float16*>(p)[i];
  else return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}
// f rounded to the element type T (round to nearest even), as an fp32 value.
template <int T> __device__ __forceinline__ float round_to(float f) {
  if constexpr (T == FP8B_F32) return f;
  else if constexpr (T == FP8B_F16) return (float)(_Float16)f;
  else return bf16_to_f32(f32_to_bf16_bits(f));
}
template <int T> __device__ __forceinline__ void store_from_f32(void* p, int64_t i, float f) {
  if constexpr (T == FP8B_F32) static_cast<float*>(p)[i] = f;
  else if constexpr (T == FP8B_F16) static_cast<_Float16*>(p)[i] = (_Float16)f;
  else static_cast<uint16_t*>(p)[i] = (uint16_t)f32_to_bf16_bits(f);
}

// Act-quant of fp16 or fp32 inputs (the bf16 kernels above cover bf16). A
// magnitude pattern is the element's bits without the sign: 15 of them for
// fp16 (infinity 0x7C00), 31 for fp32 (0x7F800000); NaN patterns lie above
// infinity, so the group's max pattern carries a NaN. The scale and its
// reciprocal are formed by IEEE division once per group.
template <int T> struct TypedInf;
template <> struct TypedInf<FP8B_F16> { static constexpr uint32_t value = 0x7C00u; };
template <> struct TypedInf<FP8B_F32> { static constexpr uint32_t value = 0x7F800000u; };

template <int T> __device__ __forceinline__ uint32_t mag_bits(const void* p, int64_t i) {
  if constexpr (T == FP8B_F32) return static_cast<const uint32_t*>(p)[i] & 0x7FFFFFFFu;
  else return static_cast<const uint16_t*>(p)[i] & 0x7FFFu;
}
template <int T> __device__ __forceinline__ float mag_value(uint32_t mag) {
  if constexpr (T == FP8B_F32) return __uint_as_float(mag);
  else return (float)__builtin_bit_cast(_Float16, (uint16_t)mag);
}
// Scale of a finite group: max(amax, 1e-10) / 448, one IEEE division.
template <int T> __device__ __forceinline__ float typed_scale(uint32_t gmag) {
  return fmaxf(mag_value<T>(gmag), kAmaxFloor) / kFp8Max;
}

// Group 128, K % 128 == 0, 16-byte aligned rows of x, 8-byte aligned rows of
// q: 16 lanes per group (8 elements a lane: one 16-byte load of fp16, two of
// fp32) over the flattened (row, group) index space; a block takes 16*U
// consecutive slots, its 16-lane row r the slots r + 16u (u < U), all loads
// issued before any conversion. Quotients by div_by_scale from the IEEE
// reciprocal (correctly rounded, Markstein).
template <int T>
__device__ __forceinline__ uint32_t load8_typed(const void* x, int64_t e0, float v[8]) {
  uint32_t mag = 0;
  if constexpr (T == FP8B_F32) {
    const v4i* p = reinterpret_cast<const v4i*>(static_cast<const float*>(x) + e0);
    const v4i r0 = __builtin_nontemporal_load(p);
    const v4i r1 = __builtin_nontemporal_load(p + 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = __int_as_float(r0[i]);
      v[4 + i] = __int_as_float(r1[i]);
      mag = max(mag, max((uint32_t)r0[i] & 0x7FFFFFFFu, (uint32_t)r1[i] & 0x7FFFFFFFu));
    }
  } else {
    const v4i r = __builtin_nontemporal_load(
        reinterpret_cast<const v4i*>(static_cast<const uint16_t*>(x) + e0));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w = (uint32_t)r[i];
      v[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
      v[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
      mag = max(mag, max(w & 0x7FFFu, (w >> 16) & 0x7FFFu));
    }
  }
  return mag;
}

template <int T, int U>
__global__ void __launch_bounds__(256)
act_quant_typed_g128_kernel(const void* __restrict__ x, int64_t ldx,
                            uint8_t* __restrict__ q, int64_t ldq,
                            float* __restrict__ s, int64_t ssm, int64_t ssg,
                            uint32_t slots, uint32_t groups_per_row) {
  const uint32_t sub = threadIdx.x & 15u;
  const uint32_t slot0 = blockIdx.x * 16u * U + (threadIdx.x >> 4);
  float v[U][8];
  uint32_t mag[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t slot = min(slot0 + 16u * u, slots - 1);  // uniform per 16-lane row
    const uint32_t m = slot / groups_per_row, g = slot - m * groups_per_row;
    mag[u] = load8_typed<T>(x, (int64_t)m * ldx + g * 128u + sub * 8u, v[u]);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t slot = slot0 + 16u * u;
    if (slot >= slots) break;  // uniform across the 16-lane row
    const uint32_t m = slot / groups_per_row, g = slot - m * groups_per_row;
    const uint32_t gmag = row16_max_u32(mag[u]);
    uint32_t w0, w1;
    float scale;
    if (gmag < TypedInf<T>::value) {
      scale = typed_scale<T>(gmag);
      quant8_finite(v[u], scale, 1.0f / scale, w0, w1);
    } else {
      quant8_nonfinite(v[u], gmag > TypedInf<T>::value, w0, w1, scale);
    }
    v2i packed;
    packed[0] = (int)w0;
    packed[1] = (int)w1;
    __builtin_nontemporal_store(
        packed, reinterpret_cast<v2i*>(q + (int64_t)m * ldq + g * 128u + sub * 8u));
    if (sub == 0) s[(int64_t)m * ssm + (int64_t)g * ssg] = scale;
  }
}

// Any group size, ragged K or unaligned rows: one thread walks one group,
// quotients by IEEE division.
template <int T>
__global__ void __launch_bounds__(64)
act_quant_typed_generic_kernel(const void* __restrict__ x, int64_t ldx,
                               uint8_t* __restrict__ q, int64_t ldq,
                               float* __restrict__ s, int64_t ssm, int64_t ssg,
                               int64_t M, int64_t K, int64_t group, int64_t groups_per_row) {
  const int64_t gi = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (gi >= M * groups_per_row) return;
  const int64_t m = gi / groups_per_row;
  const int64_t g = gi - m * groups_per_row;
  const int64_t k0 = g * group;
  const int64_t k1 = min(k0 + group, K);
  const int64_t row = m * ldx;
  uint32_t gmag = 0;
  for (int64_t k = k0; k < k1; ++k) gmag = max(gmag, mag_bits<T>(x, row + k));
  constexpr uint32_t kInf = TypedInf<T>::value;
  const float scale = gmag > kInf    ? __uint_as_float(0x7FC00000u)
                      : gmag == kInf ? __uint_as_float(0x7F800000u)
                                     : typed_scale<T>(gmag);
  uint8_t* qr = q + m * ldq;
  for (int64_t k = k0; k < k1; ++k) {
    const float xv = load_as_f32<T>(x, row + k);
    uint8_t code;
    if (gmag > kInf) {
      code = kFp8NaN;
    } else if (gmag == kInf) {
      const uint32_t u = __float_as_uint(xv);
      code = (u & 0x7FFFFFFFu) >= 0x7F800000u ? kFp8NaN : (uint8_t)((u >> 24) & 0x80u);
    } else {
      code = (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(xv / scale, 0.0f, 0, false) & 0xFF);
    }
    qr[k] = code;
  }
  s[m * ssm + g * ssg] = scale;
}

// silu_and_mul for any pair of element types (x of type TX, out of type TO):
// out = TO( TX( TX(silu(fp32 gate)) * up ) ), the rounding points of
// act.py:25-28 (silu.to(b.dtype) * b computed in fp32 and rounded to b's
// dtype, then .to(out.dtype)). One element per thread and step.
template <int TX, int TO>
__global__ void __launch_bounds__(256)
silu_and_mul_typed_kernel(const void* __restrict__ x, int64_t ldx, void* __restrict__ out,
                          int64_t ldo, int64_t M, int64_t d) {
  const int64_t n = M * d;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256) {
    const int64_t m = i / d, j = i - m * d;
    const float a = load_as_f32<TX>(x, m * ldx + j);
    const float b = load_as_f32<TX>(x, m * ldx + d + j);
    const float h = round_to<TX>(round_to<TX>(silu_f32(a)) * b);
    store_from_f32<TO>(out, m * ldo + j, h);
  }
}

// Fused silu_and_mul + group-128 quantisation: identical arithmetic to
// silu_and_mul_vec_kernel followed by act_quant_g128_kernel, without the
// bf16 round trip through memory. Requires d % 128 == 0. Blocks of R 16-lane
// rows (16R threads) map to (row, group) as in act_quant_g128_kernel with
// R*U groups per block column; each lane loads its 8 gate and 8 up values
// of U groups before converting any.
template <int U, int R>
__global__ void __launch_bounds__(256)
silu_mul_quant_g128_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                           uint8_t* __restrict__ q, int64_t ldq,
                           float* __restrict__ s, int64_t ssm, int64_t ssg,
                           uint32_t rows, uint32_t groups_per_row, int64_t d) {
  const uint32_t sub = threadIdx.x & 15u;
  const uint32_t g0 = blockIdx.x * (uint32_t)(R * U) + (threadIdx.x >> 4);
  __shared__ float sc[2][R * U];
  uint32_t par = 0;
  for (uint32_t m = blockIdx.y; m < rows; m += gridDim.y, par ^= 1u) {
    const uint16_t* xr = x + (int64_t)m * ldx;
    const uint16_t* ur_ = xr + d;
    v4i gr[U], ur[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t g = min(g0 + (uint32_t)R * u, groups_per_row - 1);  // uniform per 16-lane row
      gr[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(xr + g * 128u + sub * 8u));
      ur[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(ur_ + g * 128u + sub * 8u));
    }
    uint8_t* qr = q + (int64_t)m * ldq;
    float* sr = s + (int64_t)m * ssm;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t g = g0 + (uint32_t)R * u;
      if (g >= groups_per_row) break;  // uniform across the 16-lane group
      float v[8];
      const v4i h = silu_mul_bf16x8(gr[u], ur[u], v);
      uint32_t w0, w1;
      float scale;
      quant_row16_8(v, max_mag_bf16x8(h), w0, w1, scale);
      v2i packed;
      packed[0] = (int)w0;
      packed[1] = (int)w1;
      __builtin_nontemporal_store(packed, reinterpret_cast<v2i*>(qr + g * 128u + sub * 8u));
      if constexpr (U == 1) {
        if (sub == 0) sr[(int64_t)g * ssg] = scale;
      } else {
        store_group_scale<R>(sc[par], u, scale);
      }
    }
    if constexpr (U > 1) flush_group_scales<R * U>(sc[par], sr, ssg, groups_per_row);
  }
}

// silu_mul_quant_g128_kernel for rows of fewer than 16 groups (d below
// 2048), mapped as act_quant_g128_flat_kernel is.
__global__ void __launch_bounds__(256)
silu_mul_quant_g128_flat_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                uint8_t* __restrict__ q, int64_t ldq,
                                float* __restrict__ s, int64_t ssm, int64_t ssg,
                                uint32_t slots, uint32_t groups_per_row, int64_t d) {
  const uint32_t sub = threadIdx.x & 15u;
  const uint32_t slot = blockIdx.x * 16u + (threadIdx.x >> 4);
  if (slot >= slots) return;  // uniform across the 16-lane row
  const uint32_t m = slot / groups_per_row, g = slot - m * groups_per_row;
  const uint16_t* xg = x + (int64_t)m * ldx + g * 128u + sub * 8u;
  const v4i gr = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(xg));
  const v4i ur = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(xg + d));
  float v[8];
  const v4i h = silu_mul_bf16x8(gr, ur, v);
  uint32_t w0, w1;
  float scale;
  quant_row16_8(v, max_mag_bf16x8(h), w0, w1, scale);
  v2i packed;
  packed[0] = (int)w0;
  packed[1] = (int)w1;
  __builtin_nontemporal_store(packed,
                              reinterpret_cast<v2i*>(q + (int64_t)m * ldq + g * 128u + sub * 8u));
  if (sub == 0) s[(int64_t)m * ssm + (int64_t)g * ssg] = scale;
}

__global__ void __launch_bounds__(64)
silu_mul_quant_generic_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                              uint8_t* __restrict__ q, int64_t ldq,
                              float* __restrict__ s, int64_t ssm, int64_t ssg,
                              int64_t M, int64_t d, int64_t group, int64_t groups_per_row) {
  const int64_t gi = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (gi >= M * groups_per_row) return;
  const int64_t m = gi / groups_per_row;
  const int64_t g = gi - m * groups_per_row;
  const int64_t j0 = g * group;
  const int64_t j1 = min(j0 + group, d);
  const uint16_t* xr = x + m * ldx;
  uint32_t gmag = 0;
  for (int64_t j = j0; j < j1; ++j)
    gmag = max(gmag, silu_mul_bits(xr[j], xr[d + j]) & 0x7FFFu);
  const float scale = scale_from_mag(gmag);
  uint8_t* qr = q + m * ldq;
  for (int64_t j = j0; j < j1; ++j)
    qr[j] = quant_scalar(bf16_to_f32(silu_mul_bits(xr[j], xr[d + j])), gmag, scale);
  s[m * ssm + g * ssg] = scale;
}

}  // namespace fp8b

using namespace fp8b;

static inline bool aligned(const void* p, uintptr_t a) {
  return ((uintptr_t)p & (a - 1)) == 0;
}

static int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(what);
    return FP8B_ERR_LAUNCH;
  }
  return FP8B_OK;
}

extern "C" int fp8b_act_quant(const void* x, int64_t ldx, void* q, int64_t ldq,
                              float* s, int64_t s_stride_m, int64_t s_stride_g,
                              int64_t M, int64_t K, int64_t group, void* stream) {
  if (M < 0 || K < 0 || ldx < K || ldq < K) {
    set_error("fp8b_act_quant: bad dims (need M,K >= 0, ldx >= K, ldq >= K)");
    return FP8B_ERR_DIMS;
  }
  if (group != 32 && group != 64 && group != 128 && group != 256) {
    set_error("fp8b_act_quant: group must be 32, 64, 128 or 256");
    return FP8B_ERR_BLOCK;
  }
  if (M == 0 || K == 0) return FP8B_OK;
  if (!x || !q || !s) {
    set_error("fp8b_act_quant: null pointer");
    return FP8B_ERR_NULL;
  }
  const int64_t gpr = (K + group - 1) / group;
  hipStream_t st = (hipStream_t)stream;
  // (the fast kernel forms in-row offsets g * 128 in 32 bits)
  const bool fast = group == 128 && K % 128 == 0 && ldx % 8 == 0 && ldq % 8 == 0 &&
                    aligned(x, 16) && aligned(q, 8) && M * gpr < (int64_t(1) << 31) &&
                    K < (int64_t(1) << 32);
  if (fast && gpr < 16) {
    const int64_t slots = M * gpr;
    act_quant_g128_flat_kernel<<<(unsigned)((slots + 15) / 16), 256, 0, st>>>(
        (const uint16_t*)x, ldx, (uint8_t*)q, ldq, s, s_stride_m, s_stride_g, (uint32_t)slots,
        (uint32_t)gpr);
  } else if (fast) {
    const int U = g128_unroll(M, gpr);
    const dim3 grid((unsigned)((gpr + 16 * U - 1) / (16 * U)), (unsigned)std::min<int64_t>(M, 65535));
    auto launch = [&](auto kernel) {
      kernel<<<grid, 256, 0, st>>>((const uint16_t*)x, ldx, (uint8_t*)q, ldq, s, s_stride_m,
                                   s_stride_g, (uint32_t)M, (uint32_t)gpr);
    };
    if (U == 4) launch(act_quant_g128_kernel<4>);
    else if (U == 2) launch(act_quant_g128_kernel<2>);
    else launch(act_quant_g128_kernel<1>);
  } else {
    const int64_t groups = M * gpr;
    act_quant_generic_kernel<<<(unsigned)((groups + 63) / 64), 64, 0, st>>>(
        (const uint16_t*)x, ldx, (uint8_t*)q, ldq, s, s_stride_m, s_stride_g, M, K, group, gpr);
  }
  return check_launch("fp8b_act_quant: kernel launch failed");
}

extern "C" int fp8b_act_quant_typed(const void* x, int64_t ldx, int x_dtype, void* q,
                                    int64_t ldq, float* s, int64_t s_stride_m,
                                    int64_t s_stride_g, int64_t M, int64_t K, int64_t group,
                                    void* stream) {
  if (x_dtype != FP8B_F32 && x_dtype != FP8B_BF16 && x_dtype != FP8B_F16) {
    set_error("fp8b_act_quant_typed: x_dtype must be FP8B_F32, FP8B_BF16 or FP8B_F16");
    return FP8B_ERR_DTYPE;
  }
  if (x_dtype == FP8B_BF16)
    return fp8b_act_quant(x, ldx, q, ldq, s, s_stride_m, s_stride_g, M, K, group, stream);
  if (M < 0 || K < 0 || ldx < K || ldq < K) {
    set_error("fp8b_act_quant_typed: bad dims (need M,K >= 0, ldx >= K, ldq >= K)");
    return FP8B_ERR_DIMS;
  }
  if (group != 32 && group != 64 && group != 128 && group != 256) {
    set_error("fp8b_act_quant_typed: group must be 32, 64, 128 or 256");
    return FP8B_ERR_BLOCK;
  }
  if (M == 0 || K == 0) return FP8B_OK;
  if (!x || !q || !s) {
    set_error("fp8b_act_quant_typed: null pointer");
    return FP8B_ERR_NULL;
  }
  const int64_t gpr = (K + group - 1) / group;
  hipStream_t st = (hipStream_t)stream;
  const int64_t per16 = x_dtype == FP8B_F32 ? 4 : 8;  // elements per 16 bytes
  const bool fast = group == 128 && K % 128 == 0 && ldx % per16 == 0 && ldq % 8 == 0 &&
                    aligned(x, 16) && aligned(q, 8) && M * gpr < (int64_t(1) << 31) &&
                    K < (int64_t(1) << 32);
  if (fast) {
    // 32 bytes of x in flight per lane: two groups of fp16, one of fp32
    const int64_t slots = M * gpr;
    if (x_dtype == FP8B_F32)
      act_quant_typed_g128_kernel<FP8B_F32, 1><<<(unsigned)((slots + 15) / 16), 256, 0, st>>>(
          x, ldx, (uint8_t*)q, ldq, s, s_stride_m, s_stride_g, (uint32_t)slots, (uint32_t)gpr);
    else
      act_quant_typed_g128_kernel<FP8B_F16, 2><<<(unsigned)((slots + 31) / 32), 256, 0, st>>>(
          x, ldx, (uint8_t*)q, ldq, s, s_stride_m, s_stride_g, (uint32_t)slots, (uint32_t)gpr);
  } else {
    const unsigned blocks = (unsigned)((M * gpr + 63) / 64);
    if (x_dtype == FP8B_F32)
      act_quant_typed_generic_kernel<FP8B_F32><<<blocks, 64, 0, st>>>(
          x, ldx, (uint8_t*)q, ldq, s, s_stride_m, s_stride_g, M, K, group, gpr);
    else
      act_quant_typed_generic_kernel<FP8B_F16><<<blocks, 64, 0, st>>>(
          x, ldx, (uint8_t*)q, ldq, s, s_stride_m, s_stride_g, M, K, group, gpr);
  }
  return check_launch("fp8b_act_quant_typed: kernel launch failed");
}

extern "C" int fp8b_silu_and_mul(const void* x, int64_t ldx, void* out, int64_t ldo,
                                 int64_t M, int64_t d, void* stream) {
  if (M < 0 || d < 0 || ldx < 2 * d || ldo < d) {
    set_error("fp8b_silu_and_mul: bad dims (need ldx >= 2d, ldo >= d)");
    return FP8B_ERR_DIMS;
  }
  if (M == 0 || d == 0) return FP8B_OK;
  if (!x || !out) {
    set_error("fp8b_silu_and_mul: null pointer");
    return FP8B_ERR_NULL;
  }
  hipStream_t st = (hipStream_t)stream;
  const bool fast = d % 8 == 0 && ldx % 8 == 0 && ldo % 8 == 0 && aligned(x, 16) &&
                    aligned(out, 16) && M * (d / 8) < (int64_t(1) << 31);
  if (fast) {
    const uint32_t cpr = (uint32_t)(d / 8);
    const uint32_t chunks = (uint32_t)(M * cpr);
    silu_and_mul_vec_kernel<<<(chunks + 255u) / 256u, 256, 0, st>>>(
        (const uint16_t*)x, ldx, (uint16_t*)out, ldo, chunks, cpr, d);
  } else {
    const int64_t n = M * d;
    silu_and_mul_generic_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(
        (const uint16_t*)x, ldx, (uint16_t*)out, ldo, M, d);
  }
  return check_launch("fp8b_silu_and_mul: kernel launch failed");
}

namespace {
template <int TX>
void launch_silu_typed(const void* x, int64_t ldx, void* out, int64_t ldo, int out_dtype,
                       int64_t M, int64_t d, hipStream_t st) {
  const int64_t n = M * d;
  const unsigned blocks = (unsigned)std::min<int64_t>((n + 255) / 256, 65536);
  if (out_dtype == FP8B_F32)
    silu_and_mul_typed_kernel<TX, FP8B_F32><<<blocks, 256, 0, st>>>(x, ldx, out, ldo, M, d);
  else if (out_dtype == FP8B_F16)
    silu_and_mul_typed_kernel<TX, FP8B_F16><<<blocks, 256, 0, st>>>(x, ldx, out, ldo, M, d);
  else
    silu_and_mul_typed_kernel<TX, FP8B_BF16><<<blocks, 256, 0, st>>>(x, ldx, out, ldo, M, d);
}
}  // namespace

extern "C" int fp8b_silu_and_mul_typed(const void* x, int64_t ldx, int x_dtype, void* out,
                                       int64_t ldo, int out_dtype, int64_t M, int64_t d,
                                       void* stream) {
  auto dtype_ok = [](int t) { return t == FP8B_F32 || t == FP8B_BF16 || t == FP8B_F16; };
  if (!dtype_ok(x_dtype) || !dtype_ok(out_dtype)) {
    set_error("fp8b_silu_and_mul_typed: dtypes must be FP8B_F32, FP8B_BF16 or FP8B_F16");
    return FP8B_ERR_DTYPE;
  }
  if (x_dtype == FP8B_BF16 && out_dtype == FP8B_BF16)
    return fp8b_silu_and_mul(x, ldx, out, ldo, M, d, stream);
  if (M < 0 || d < 0 || ldx < 2 * d || ldo < d) {
    set_error("fp8b_silu_and_mul_typed: bad dims (need ldx >= 2d, ldo >= d)");
    return FP8B_ERR_DIMS;
  }
  if (M == 0 || d == 0) return FP8B_OK;
  if (!x || !out) {
    set_error("fp8b_silu_and_mul_typed: null pointer");
    return FP8B_ERR_NULL;
  }
  hipStream_t st = (hipStream_t)stream;
  if (x_dtype == FP8B_F32) launch_silu_typed<FP8B_F32>(x, ldx, out, ldo, out_dtype, M, d, st);
  else if (x_dtype == FP8B_F16) launch_silu_typed<FP8B_F16>(x, ldx, out, ldo, out_dtype, M, d, st);
  else launch_silu_typed<FP8B_BF16>(x, ldx, out, ldo, out_dtype, M, d, st);
  return check_launch("fp8b_silu_and_mul_typed: kernel launch failed");
}

extern "C" int fp8b_silu_and_mul_quant(const void* x, int64_t ldx, void* q, int64_t ldq,
                                       float* s, int64_t s_stride_m, int64_t s_stride_g,
                                       int64_t M, int64_t d, int64_t group, void* stream) {
  if (M < 0 || d < 0 || ldx < 2 * d || ldq < d) {
    set_error("fp8b_silu_and_mul_quant: bad dims (need ldx >= 2d, ldq >= d)");
    return FP8B_ERR_DIMS;
  }
  if (group != 32 && group != 64 && group != 128 && group != 256) {
    set_error("fp8b_silu_and_mul_quant: group must be 32, 64, 128 or 256");
    return FP8B_ERR_BLOCK;
  }
  if (M == 0 || d == 0) return FP8B_OK;
  if (!x || !q || !s) {
    set_error("fp8b_silu_and_mul_quant: null pointer");
    return FP8B_ERR_NULL;
  }
  const int64_t gpr = (d + group - 1) / group;
  hipStream_t st = (hipStream_t)stream;
  const bool fast = group == 128 && d % 128 == 0 && ldx % 8 == 0 && ldq % 8 == 0 &&
                    aligned(x, 16) && aligned(q, 8) && M * gpr < (int64_t(1) << 31) &&
                    d < (int64_t(1) << 31);
  if (fast && gpr < 16) {
    const int64_t slots = M * gpr;
    silu_mul_quant_g128_flat_kernel<<<(unsigned)((slots + 15) / 16), 256, 0, st>>>(
        (const uint16_t*)x, ldx, (uint8_t*)q, ldq, s, s_stride_m, s_stride_g, (uint32_t)slots,
        (uint32_t)gpr, d);
  } else if (fast) {
    int R, U;
    silu_quant_shape(M, gpr, R, U);
    const dim3 grid((unsigned)((gpr + R * U - 1) / (R * U)), (unsigned)std::min<int64_t>(M, 65535));
    auto launch = [&](auto kernel) {
      kernel<<<grid, 16 * R, 0, st>>>((const uint16_t*)x, ldx, (uint8_t*)q, ldq, s, s_stride_m,
                                      s_stride_g, (uint32_t)M, (uint32_t)gpr, d);
    };
    if (U == 4) launch(silu_mul_quant_g128_kernel<4, 16>);
    else if (U == 2 && R == 16) launch(silu_mul_quant_g128_kernel<2, 16>);
    else if (U == 2 && R == 8) launch(silu_mul_quant_g128_kernel<2, 8>);
    else if (U == 2) launch(silu_mul_quant_g128_kernel<2, 4>);
    else launch(silu_mul_quant_g128_kernel<1, 16>);
  } else {
    const int64_t groups = M * gpr;
    silu_mul_quant_generic_kernel<<<(unsigned)((groups + 63) / 64), 64, 0, st>>>(
        (const uint16_t*)x, ldx, (uint8_t*)q, ldq, s, s_stride_m, s_stride_g, M, d, group, gpr);
  }
  return check_launch("fp8b_silu_and_mul_quant: kernel launch failed");
}

namespace fp8b {

// 128x128 weight-block quantiser: one 256-thread workgroup per block. Wave w
// handles block rows 32w..32w+31; for each row its 64 lanes read two
// consecutive elements (coalesced 512 B of fp32 or 256 B of bf16 per row),
// so a lane holds 64 values in registers and the block is read once.
//   Bs[nb,kb] = max(amax_block, 1e-10) / 448 (IEEE), Wq = e4m3fn(W / Bs)
// with IEEE division and the gfx950 OCP convert (RNE); elements past N or K
// do not take part. NaN in a block propagates to its scale (as torch.amax
// does) and every element of that block becomes the e4m3fn NaN 0x7F; a
// block whose amax is +inf gets scale +inf, 0x7F for its +-inf elements and
// a signed zero (x / inf) for the finite ones, the act-quant policy.
template <typename T>
__device__ __forceinline__ float load_w(const T* p);

// Code of x in a block of scale +inf.
__device__ __forceinline__ uint32_t inf_block_code(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x7FFFFFFFu) == 0x7F800000u ? (uint32_t)kFp8NaN : (u >> 24) & 0x80u;
}
template <>
__device__ __forceinline__ float load_w<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_w<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }

// Max of a 256-thread block's values (the block max of 128x128 weights):
// DPP rows of 16, then the four rows, then the four waves through LDS.
__device__ __forceinline__ uint32_t block128_max_u32(uint32_t m, int lane, int wid) {
  m = row16_max_u32(m);
  m = max(m, (uint32_t)__builtin_amdgcn_readlane((int)m, 0));
  m = max(m, (uint32_t)__builtin_amdgcn_readlane((int)m, 16));
  m = max(m, (uint32_t)__builtin_amdgcn_readlane((int)m, 32));
  m = max(m, (uint32_t)__builtin_amdgcn_readlane((int)m, 48));
  __shared__ uint32_t wmax[4];
  if (lane == 0) wmax[wid] = m;
  __syncthreads();
  return max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3]));
}

template <typename T>
__device__ __forceinline__ void weight_quant_block128_body(
    const T* __restrict__ W, int64_t ldw, uint8_t* __restrict__ q, int64_t ldq,
    float* __restrict__ s, int64_t s_sn, int64_t s_sk, int64_t N, int64_t K) {
  const int nb = blockIdx.y, kb = blockIdx.x;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t n0 = (int64_t)nb * 128 + wid * 32, k = (int64_t)kb * 128 + 2 * lane;
  float v[32][2];
  float amax = 0.f;
  bool nan = false;
#pragma unroll
  for (int r = 0; r < 32; ++r) {
    const int64_t n = n0 + r;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const bool in = n < N && k + e < K;
      const float x = in ? load_w<T>(W + n * ldw + k + e) : 0.f;
      v[r][e] = x;
      nan |= x != x;
      amax = fmaxf(amax, fabsf(x));
    }
  }
  const uint32_t m =
      block128_max_u32(__float_as_uint(amax) | (nan ? 0x7FC00000u : 0u), lane, wid);
  const bool block_nan = m > 0x7F800000u;
  const bool block_inf = m == 0x7F800000u;
  const float scale = block_nan ? __uint_as_float(0x7FC00000u)
                                : fmaxf(__uint_as_float(m), kAmaxFloor) / kFp8Max;
#pragma unroll
  for (int r = 0; r < 32; ++r) {
    const int64_t n = n0 + r;
    if (n >= N) break;
    uint32_t b;
    if (block_nan) {
      b = (uint32_t)kFp8NaN | ((uint32_t)kFp8NaN << 8);
    } else if (block_inf) {
      b = inf_block_code(v[r][0]) | (inf_block_code(v[r][1]) << 8);
    } else {
      b = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v[r][0] / scale, v[r][1] / scale, 0, false) &
          0xFFFFu;
    }
    if (k + 1 < K) {
      *reinterpret_cast<uint16_t*>(q + n * ldq + k) = (uint16_t)b;
    } else if (k < K) {
      q[n * ldq + k] = (uint8_t)b;
    }
  }
  if (threadIdx.x == 0) s[(int64_t)nb * s_sn + (int64_t)kb * s_sk] = scale;
}

template <typename T>
__global__ void __launch_bounds__(256)
weight_quant_block128_kernel(const T* __restrict__ W, int64_t ldw, uint8_t* __restrict__ q,
                             int64_t ldq, float* __restrict__ s, int64_t s_sn, int64_t s_sk,
                             int64_t N, int64_t K) {
  weight_quant_block128_body<T>(W, ldw, q, ldq, s, s_sn, s_sk, N, K);
}

// Weights whose rows are 16-byte multiples (fp32: ldw % 4 == 0, bf16:
// ldw % 8 == 0; W 16-byte aligned) and q rows aligned to one lane's codes:
// the same block quantiser with 16-byte loads. A lane holds VPL = 16 /
// sizeof(T) consecutive columns of NL rows (a load instruction covers
// RPL = 64 * VPL / 128 rows of the block: 2 for fp32, 4 for bf16); each
// store writes VPL codes. Blocks on the matrix edge take the per-element
// kernel's path. Same max, same scale, same per-element IEEE division: same
// bits.
template <typename T>
__global__ void __launch_bounds__(256)
weight_quant_vec_kernel(const T* __restrict__ W, int64_t ldw, uint8_t* __restrict__ q,
                        int64_t ldq, float* __restrict__ s, int64_t s_sn, int64_t s_sk,
                        int64_t N, int64_t K) {
  constexpr int VPL = 16 / sizeof(T), LPR = 128 / VPL, RPL = 64 / LPR, NL = 32 / RPL;
  const int nb = blockIdx.y, kb = blockIdx.x;
  if ((int64_t)nb * 128 + 128 > N || (int64_t)kb * 128 + 128 > K) {
    weight_quant_block128_body<T>(W, ldw, q, ldq, s, s_sn, s_sk, N, K);
    return;
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t n0 = (int64_t)nb * 128 + wid * 32 + lane / LPR;
  const int64_t k = (int64_t)kb * 128 + (lane % LPR) * VPL;
  float v[NL][VPL];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const v4i raw = __builtin_nontemporal_load(
        reinterpret_cast<const v4i*>(W + (n0 + RPL * i) * ldw + k));
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t u = (uint32_t)raw[w];
      if constexpr (VPL == 4) {
        v[i][w] = __uint_as_float(u);
      } else {
        v[i][2 * w] = __uint_as_float(u << 16);
        v[i][2 * w + 1] = __uint_as_float(u & 0xFFFF0000u);
      }
    }
  }
  float amax = 0.f;
  bool nan = false;
#pragma unroll
  for (int i = 0; i < NL; ++i)
#pragma unroll
    for (int e = 0; e < VPL; ++e) {
      nan |= v[i][e] != v[i][e];
      amax = fmaxf(amax, fabsf(v[i][e]));
    }
  const uint32_t m =
      block128_max_u32(__float_as_uint(amax) | (nan ? 0x7FC00000u : 0u), lane, wid);
  const bool block_nan = m > 0x7F800000u;
  const bool block_inf = m == 0x7F800000u;
  const float scale = block_nan ? __uint_as_float(0x7FC00000u)
                                : fmaxf(__uint_as_float(m), kAmaxFloor) / kFp8Max;
  // bf16 weights: the quotients without division instructions, as the
  // act-quant kernels form them (div_by_scale with recip_of_scale; exact
  // for bf16 values and scales of bf16 magnitudes, checked exhaustively in
  // tests/fastdiv_check.c and tests/scale_recip_check.c); fp32 weights keep
  // the IEEE division.
  const float recip = recip_of_scale(scale);
  auto quot = [&](float x) {
    if constexpr (VPL == 8) return div_by_scale(x, scale, recip);
    else return x / scale;
  };
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    uint32_t b[VPL / 4];
#pragma unroll
    for (int c = 0; c < VPL / 4; ++c) {
      if (block_nan) {
        b[c] = 0x7F7F7F7Fu;
      } else if (block_inf) {
        b[c] = inf_block_code(v[i][4 * c]) | (inf_block_code(v[i][4 * c + 1]) << 8) |
               (inf_block_code(v[i][4 * c + 2]) << 16) | (inf_block_code(v[i][4 * c + 3]) << 24);
      } else {
        int p = __builtin_amdgcn_cvt_pk_fp8_f32(quot(v[i][4 * c]), quot(v[i][4 * c + 1]), 0,
                                                false);
        p = __builtin_amdgcn_cvt_pk_fp8_f32(quot(v[i][4 * c + 2]), quot(v[i][4 * c + 3]), p,
                                            true);
        b[c] = (uint32_t)p;
      }
    }
    uint8_t* dst = q + (n0 + RPL * i) * ldq + k;
    if constexpr (VPL == 4) {
      *reinterpret_cast<uint32_t*>(dst) = b[0];
    } else {
      v2i w2;
      w2[0] = (int)b[0];
      w2[1] = (int)b[1];
      *reinterpret_cast<v2i*>(dst) = w2;
    }
  }
  if (threadIdx.x == 0) s[(int64_t)nb * s_sn + (int64_t)kb * s_sk] = scale;
}

}  // namespace fp8b

extern "C" int fp8b_weight_quant(const void* W, int64_t ldw, int w_dtype, void* q, int64_t ldq,
                                 float* s, int64_t s_sn, int64_t s_sk, int64_t N, int64_t K,
                                 void* stream) {
  if (N < 0 || K < 0 || ldw < K || ldq < K) {
    set_error("fp8b_weight_quant: bad dims (need N,K >= 0, ldw >= K, ldq >= K)");
    return FP8B_ERR_DIMS;
  }
  if (w_dtype != FP8B_F32 && w_dtype != FP8B_BF16) {
    set_error("fp8b_weight_quant: W must be FP8B_F32 or FP8B_BF16");
    return FP8B_ERR_DTYPE;
  }
  if (N == 0 || K == 0) return FP8B_OK;
  if (!W || !q || !s) {
    set_error("fp8b_weight_quant: null pointer");
    return FP8B_ERR_NULL;
  }
  if ((ldq % 2 != 0 || !aligned(q, 2)) ) {
    set_error("fp8b_weight_quant: q rows must be 2-byte aligned (even ldq)");
    return FP8B_ERR_ALIGN;
  }
  const int64_t NB = (N + 127) / 128, KB = (K + 127) / 128;
  if (NB > 65535) {
    set_error("fp8b_weight_quant: N too large");
    return FP8B_ERR_DIMS;
  }
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)KB, (unsigned)NB);
  if (w_dtype == FP8B_F32 && ldw % 4 == 0 && aligned(W, 16) && ldq % 4 == 0 && aligned(q, 4))
    weight_quant_vec_kernel<float><<<grid, 256, 0, st>>>((const float*)W, ldw, (uint8_t*)q, ldq,
                                                         s, s_sn, s_sk, N, K);
  else if (w_dtype == FP8B_BF16 && ldw % 8 == 0 && aligned(W, 16) && ldq % 8 == 0 &&
           aligned(q, 8))
    weight_quant_vec_kernel<uint16_t><<<grid, 256, 0, st>>>(
        (const uint16_t*)W, ldw, (uint8_t*)q, ldq, s, s_sn, s_sk, N, K);
  else if (w_dtype == FP8B_F32)
    weight_quant_block128_kernel<float><<<grid, 256, 0, st>>>((const float*)W, ldw, (uint8_t*)q,
                                                              ldq, s, s_sn, s_sk, N, K);
  else
    weight_quant_block128_kernel<uint16_t><<<grid, 256, 0, st>>>(
        (const uint16_t*)W, ldw, (uint8_t*)q, ldq, s, s_sn, s_sk, N, K);
  return check_launch("fp8b_weight_quant: kernel launch failed");
}
