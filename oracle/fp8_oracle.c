/*
 * CPU restatement of the block-FP8 linear path -- TEST INFRASTRUCTURE ONLY.
 *
 * This file is the checker the GPU kernels are compared against. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. It is
 * never part of the product path.
 *
 * Built with -ffp-contract=off so every fp32 operation below rounds exactly
 * where it is written.
 *
 * Functions and what each follows:
 *   oracle_e4m3fn_from_f32 / _to_f32 : float8_e4m3fn (OCP E4M3, "fn": no inf,
 *       S.1111.111 = NaN) with round-to-nearest-even, NaN for |x| rounding to
 *       >= 480 -- the semantics of torch's Tensor.to(torch.float8_e4m3fn),
 *       which the reference's callers use to make A and B
 *       (scripts/rebench_llm.py:130).
 *   oracle_act_quant : per-token-group quantiser; no reference counterpart
 *       exists (the reference consumes pre-quantised A/As,
 *       finegrained-fp8-helion/torch-ext/finegrained_fp8_helion/fp8.py:5);
 *       contract: s = max(amax,1e-10)/448, q = e4m3fn(x/s).
 *   oracle_act_quant_f32 : the same contract on fp32 values (fp32 inputs,
 *       and fp16 inputs widened to fp32, which is exact).
 *   oracle_block_gemm : fp8.py:24-38 -- per K-block fp32 dot, then
 *       acc = acc + (dot * As[m,kb]) * Bs[n/bn,kb] in K-block order.
 *   oracle_dequant_matmul : finegrained-fp8-helion/bench.py:11-14
 *       generalised to 2-D Bs: (A*As) @ (B*Bs)^T with the scales expanded.
 *   oracle_silu_and_mul : activation-helion/.../act.py:20-28.
 *   oracle_quant_weight_block : 128x128 weight-block quantiser, the format of
 *       FP8 checkpoints' "weight" + "weight_scale_inv" (Bs = max(amax,1e-10)/448
 *       per block, Wq = e4m3fn(W/Bs)); no reference counterpart (the reference
 *       harness draws random fp8 weights, scripts/rebench_llm.py:130-131);
 *       non-finite blocks as act-quant: NaN -> Bs NaN, codes 0x7F; +inf ->
 *       Bs +inf, codes 0x7F for +-inf and signed zero for finite values.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float f32_from_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint32_t bits_from_f32(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

float oracle_bf16_to_f32(uint16_t b) { return f32_from_bits((uint32_t)b << 16); }

/* fp32 -> bf16, round to nearest even; NaN -> 0x7FC0 with the sign kept. */
uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u = bits_from_f32(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)(((u >> 16) & 0x8000u) | 0x7FC0u);
  const uint32_t lsb = (u >> 16) & 1u;
  u += 0x7FFFu + lsb;
  return (uint16_t)(u >> 16);
}

/* Round a non-negative value with at most 24 significant bits to the nearest
 * integer, ties to even (exact: done on the value's own bits). */
static double rne_int(double v) {
  double fl = floor(v);
  double diff = v - fl;
  if (diff > 0.5) return fl + 1.0;
  if (diff < 0.5) return fl;
  return fmod(fl, 2.0) == 0.0 ? fl : fl + 1.0;
}

uint8_t oracle_e4m3fn_from_f32(float f) {
  const uint32_t u = bits_from_f32(f);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  if (isnan(f)) return (uint8_t)(0x7F | sign);
  const double a = fabs((double)f);
  if (a >= 480.0) return (uint8_t)(0x7F | sign); /* includes inf */
  if (a < 0x1p-6) {
    /* subnormal grid: multiples of 2^-9; n == 8 is the smallest normal */
    const int n = (int)rne_int(a * 512.0);
    return (uint8_t)(n | sign);
  }
  int ex;
  (void)frexp(a, &ex);           /* a = fr * 2^ex, fr in [0.5, 1) */
  int E = ex - 1;                /* a in [2^E, 2^(E+1)) */
  int n = (int)rne_int(ldexp(a, 3 - E)); /* in [8, 16] */
  if (n == 16) {
    n = 8;
    E += 1;
  }
  const int code = ((E + 7) << 3) | (n - 8);
  if (code > 0x7E) return (uint8_t)(0x7F | sign); /* rounded to 480: NaN */
  return (uint8_t)(code | sign);
}

float oracle_e4m3fn_to_f32(uint8_t b) {
  const int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
  double v;
  if (e == 15 && m == 7) return s ? -NAN : NAN;
  if (e == 0)
    v = ldexp((double)m, -9);
  else
    v = ldexp(1.0 + m / 8.0, e - 7);
  return (float)(s ? -v : v);
}

/* x: bf16 bits [M, ldx]; q: [M, K] bytes; s: [M, ceil(K/group)] */
/* x is bf16 bits (is_f32 = 0) or fp32 values (is_f32 = 1). */
static float act_x(const void* x, int is_f32, int64_t i) {
  return is_f32 ? ((const float*)x)[i] : oracle_bf16_to_f32(((const uint16_t*)x)[i]);
}

static void act_quant_impl(const void* x, int is_f32, int64_t M, int64_t K, int64_t ldx,
                           int64_t group, uint8_t* q, float* s) {
  const int64_t G = (K + group - 1) / group;
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t g = 0; g < G; ++g) {
      const int64_t k0 = g * group, k1 = (k0 + group < K) ? k0 + group : K;
      float amax = 0.0f;
      int has_nan = 0;
      for (int64_t k = k0; k < k1; ++k) {
        const float v = act_x(x, is_f32, m * ldx + k);
        if (isnan(v)) has_nan = 1;
        else if (fabsf(v) > amax) amax = fabsf(v);
      }
      float scale;
      if (has_nan) {
        scale = NAN;
        for (int64_t k = k0; k < k1; ++k) q[m * K + k] = 0x7F;
      } else if (isinf(amax)) {
        scale = INFINITY;
        for (int64_t k = k0; k < k1; ++k) {
          const float v = act_x(x, is_f32, m * ldx + k);
          q[m * K + k] = isinf(v) ? 0x7F : (signbit(v) ? 0x80 : 0x00);
        }
      } else {
        const float am = amax < 1e-10f ? 1e-10f : amax;
        scale = am / 448.0f;
        for (int64_t k = k0; k < k1; ++k) {
          const float v = act_x(x, is_f32, m * ldx + k);
          q[m * K + k] = oracle_e4m3fn_from_f32(v / scale);
        }
      }
      s[m * G + g] = scale;
    }
  }
}

void oracle_act_quant(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int64_t group,
                      uint8_t* q, float* s) {
  act_quant_impl(x, 0, M, K, ldx, group, q, s);
}

void oracle_act_quant_f32(const float* x, int64_t M, int64_t K, int64_t ldx, int64_t group,
                          uint8_t* q, float* s) {
  act_quant_impl(x, 1, M, K, ldx, group, q, s);
}

/* A [M,K], B [N,K] fp8 bytes; As [M,KB], Bs [NB,KB] fp32 contiguous; C fp32 [M,N].
 * The per-block dot product of fp8 values is exact in double and rounded once
 * to fp32. */
void oracle_block_gemm(const uint8_t* A, const uint8_t* B, const float* As, const float* Bs,
                       int64_t M, int64_t N, int64_t K, int64_t bn, int64_t bk, float* C) {
  const int64_t KB = (K + bk - 1) / bk;
  float lut[256];
  for (int i = 0; i < 256; ++i) lut[i] = oracle_e4m3fn_to_f32((uint8_t)i);
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      float acc = 0.0f;
      for (int64_t kb = 0; kb < KB; ++kb) {
        const int64_t k0 = kb * bk, k1 = (k0 + bk < K) ? k0 + bk : K;
        double d = 0.0;
        for (int64_t k = k0; k < k1; ++k)
          d += (double)lut[A[m * K + k]] * (double)lut[B[n * K + k]];
        const float dot = (float)d;
        const float t = dot * As[m * KB + kb];
        const float u = t * Bs[(n / bn) * KB + kb];
        acc = acc + u;
      }
      C[m * N + n] = acc;
    }
  }
}

/* (A*As) @ (B*Bs)^T: dequantised fp32 operands, dot accumulated in double,
 * rounded once to fp32. */
void oracle_dequant_matmul(const uint8_t* A, const uint8_t* B, const float* As,
                           const float* Bs, int64_t M, int64_t N, int64_t K, int64_t bn,
                           int64_t bk, float* C) {
  const int64_t KB = (K + bk - 1) / bk;
  float lut[256];
  for (int i = 0; i < 256; ++i) lut[i] = oracle_e4m3fn_to_f32((uint8_t)i);
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      double d = 0.0;
      for (int64_t k = 0; k < K; ++k) {
        const float a = lut[A[m * K + k]] * As[m * KB + k / bk];
        const float b = lut[B[n * K + k]] * Bs[(n / bn) * KB + k / bk];
        d += (double)a * (double)b;
      }
      C[m * N + n] = (float)d;
    }
  }
}

/* x bf16 [M, 2d] -> out bf16 [M, d] */
void oracle_silu_and_mul(const uint16_t* x, int64_t M, int64_t d, uint16_t* out) {
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t j = 0; j < d; ++j) {
      const float a = oracle_bf16_to_f32(x[m * 2 * d + j]);
      const float sig = 1.0f / (1.0f + expf(-a));
      const float silu = a * sig;
      const float sb = oracle_bf16_to_f32(oracle_f32_to_bf16(silu));
      const float up = oracle_bf16_to_f32(x[m * 2 * d + d + j]);
      out[m * d + j] = oracle_f32_to_bf16(sb * up);
    }
  }
}

/* W fp32 [N,K] -> Wq [N,K] bytes, Bs [ceil(N/bn), ceil(K/bk)].
 * Non-finite blocks follow the act-quant policy above: a NaN anywhere in the
 * block gives Bs = NaN and every code 0x7F; otherwise an infinite amax gives
 * Bs = +inf, codes 0x7F for +-inf elements and a signed zero for finite
 * ones (x / inf). */
void oracle_quant_weight_block(const float* W, int64_t N, int64_t K, int64_t bn, int64_t bk,
                               uint8_t* Wq, float* Bs) {
  const int64_t NB = (N + bn - 1) / bn, KB = (K + bk - 1) / bk;
  for (int64_t nb = 0; nb < NB; ++nb) {
    for (int64_t kb = 0; kb < KB; ++kb) {
      const int64_t n0 = nb * bn, n1 = (n0 + bn < N) ? n0 + bn : N;
      const int64_t k0 = kb * bk, k1 = (k0 + bk < K) ? k0 + bk : K;
      float amax = 0.0f;
      int has_nan = 0;
      for (int64_t n = n0; n < n1; ++n)
        for (int64_t k = k0; k < k1; ++k) {
          const float v = W[n * K + k];
          if (isnan(v)) has_nan = 1;
          else if (fabsf(v) > amax) amax = fabsf(v);
        }
      if (has_nan) {
        Bs[nb * KB + kb] = NAN;
        for (int64_t n = n0; n < n1; ++n)
          for (int64_t k = k0; k < k1; ++k) Wq[n * K + k] = 0x7F;
        continue;
      }
      if (isinf(amax)) {
        Bs[nb * KB + kb] = INFINITY;
        for (int64_t n = n0; n < n1; ++n)
          for (int64_t k = k0; k < k1; ++k) {
            const float v = W[n * K + k];
            Wq[n * K + k] = isinf(v) ? 0x7F : (signbit(v) ? 0x80 : 0x00);
          }
        continue;
      }
      const float am = amax < 1e-10f ? 1e-10f : amax;
      const float sc = am / 448.0f;
      Bs[nb * KB + kb] = sc;
      for (int64_t n = n0; n < n1; ++n)
        for (int64_t k = k0; k < k1; ++k) Wq[n * K + k] = oracle_e4m3fn_from_f32(W[n * K + k] / sc);
    }
  }
}
