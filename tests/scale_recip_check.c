/* Exhaustive checks of the division-free scale and reciprocal of the
 * act-quant kernels (hf_kernels_helion_amd/csrc/quant.h):
 *   scale_from_amax: c = RN(1/448); q0 = RN(amax*c); r = fma(-q0, 448, amax);
 *                    s = fma(r, c, q0)
 *     must equal the IEEE quotient amax / 448 for every amax the kernels form
 *     (every finite bf16 magnitude, floored at 1e-10);
 *   recip_of_scale:  y1 = fma(fma(-s, y0, 1), y0, y0) from any y0 within one
 *     ulp of 1/s (v_rcp_f32's documented accuracy)
 *     must equal RN(1/s). This is checked for every float mantissa (the step
 *     commutes with scaling by powers of two while 1/s stays normal): it
 *     fails only for the all-ones mantissa, which no scale above has.
 * Prints "scales=N scale_bad=A recips=M recip_bad_mantissas=B allones_scales=C";
 * A and C must be 0 and B may only name the all-ones mantissa.
 * Build: gcc -O2 -ffp-contract=off scale_recip_check.c -lm */
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
static float from_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

int main(void) {
  const float c = 0x1.24924ap-9f; /* the kernels' constant */
  if (bits(c) != bits(1.0f / 448.0f)) {
    printf("constant is not RN(1/448)\n");
    return 1;
  }
  long scales = 0, scale_bad = 0, allones = 0;
  for (uint32_t p = 0; p < 0x7F80u; ++p) {
    const float amax = fmaxf(bf16(p), 1e-10f);
    const float want = amax / 448.0f;
    const float q0 = amax * c;
    const float r = fmaf(-q0, 448.0f, amax);
    const float s = fmaf(r, c, q0);
    ++scales;
    if (bits(s) != bits(want)) ++scale_bad;
    if ((bits(want) & 0x7FFFFFu) == 0x7FFFFFu) ++allones;
  }
  long recips = 0, recip_bad = 0, bad_not_allones = 0;
  for (uint32_t m = 0; m < (1u << 23); ++m) {
    const float b = from_bits(0x3F800000u | m);
    const float want = 1.0f / b;
    const double exact = 1.0 / (double)b;
    int bad = 0;
    for (int d = -2; d <= 2; ++d) {
      const float y0 = from_bits(bits(want) + (uint32_t)d);
      const double ulp = ldexp(1.0, ilogb(y0) - 23);
      if (fabs((double)y0 - exact) > ulp) continue; /* not within one ulp */
      ++recips;
      const float y1 = fmaf(fmaf(-b, y0, 1.0f), y0, y0);
      if (bits(y1) != bits(want)) bad = 1;
    }
    if (bad) {
      ++recip_bad;
      if (m != 0x7FFFFFu) ++bad_not_allones;
    }
  }
  printf("scales=%ld scale_bad=%ld recips=%ld recip_bad_mantissas=%ld allones_scales=%ld\n",
         scales, scale_bad, recips, recip_bad, allones);
  return (scale_bad == 0 && allones == 0 && bad_not_allones == 0) ? 0 : 1;
}
