/* Exhaustive check of the act-quant division used by the GPU kernels
 * (hf_kernels_helion_amd/csrc/act_quant.hip, div_by_scale):
 *   y = RN(1/s); q0 = RN(x*y); n = fma(q0, s, -x); q = fma(-n, y, q0)
 * against IEEE x/s, for every finite bf16 x and every bf16 amax >= |x|, with
 * s = max(amax, 1e-10) / 448 as the kernels compute it. Every quotient that
 * differs from IEEE division must be below 2^-12 in magnitude (it converts to
 * a signed float8_e4m3fn zero either way, since e4m3fn's smallest subnormal
 * is 2^-9) and carry the sign of x.
 * Prints "pairs=N mismatches=M large=L sign=S"; L and S must be 0.
 * Build: gcc -O2 -ffp-contract=off -fopenmp fastdiv_check.c -lm */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float bf16(uint32_t b) {
  const uint32_t u = b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

int main(void) {
  long n = 0, mism = 0, large = 0, sign = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : n, mism, large, sign)
  for (int am = 0; am < 0x7F80; ++am) {
    const float amax = fmaxf(bf16((uint32_t)am), 1e-10f);
    const float s = amax / 448.0f;
    const float y = 1.0f / s;
    for (uint32_t xm = 0; xm <= (uint32_t)am; ++xm) {
      for (int sg = 0; sg < 2; ++sg) {
        const float x = bf16(xm | (sg ? 0x8000u : 0u));
        const float q = x / s;
        const float q0 = x * y;
        const float n2 = fmaf(q0, s, -x);
        const float f = fmaf(-n2, y, q0);
        ++n;
        if (bits(f) != bits(q)) {
          ++mism;
          if (fabsf(q) >= 0x1p-12f || fabsf(f) >= 0x1p-12f) ++large;
        }
        if ((bits(f) ^ bits(x)) & 0x80000000u) ++sign;
      }
    }
  }
  printf("pairs=%ld mismatches=%ld large=%ld sign=%ld\n", n, mism, large, sign);
  return (large == 0 && sign == 0) ? 0 : 1;
}
