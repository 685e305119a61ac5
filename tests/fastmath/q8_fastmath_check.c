/* Exhaustive CPU check of two f32 identities the Q8_0 GEMV kernel relies on
 * (ferrum_amd/csrc/fkv_gemv.hip: div127, round_away). Both use only IEEE f32
 * multiply, add, fma and trunc, which the GPU computes identically:
 *   div127(a) = fma(fma(-a*c, 127, a), c, a*c), c = RN(1/127)  == a / 127
 *       for every a in [0, +Inf) (and +Inf mapped to +Inf separately);
 *   trunc(y + copysign(0.5 - 2^-25, y)) == round-half-away-from-zero(y)
 *       for every non-NaN f32 y.
 * Prints the mismatch counts; exit status 1 on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* Rust's f32::round: half away from zero. */
static float round_half_away(float y) {
  float t = truncf(y);
  return (fabsf(y - t) >= 0.5f) ? t + copysignf(1.0f, y) : t;
}

int main(void) {
  const float c = 1.0f / 127.0f;
  unsigned long long bad_div = 0, bad_rnd = 0;
  for (uint32_t i = 0; i < 0x7f800000u; i++) { /* finite a >= 0 */
    const float a = u2f(i);
    const float q = a * c;
    const float r = fmaf(-q, 127.0f, a);
    if (f2u(fmaf(r, c, q)) != f2u(a / 127.0f)) bad_div++;
    for (int s = 0; s < 2; s++) {
      const float y = s ? -a : a;
      if (f2u(truncf(y + copysignf(0.49999997f, y))) != f2u(round_half_away(y))) bad_rnd++;
    }
  }
  for (int s = 0; s < 2; s++) { /* +-Inf */
    const float y = s ? -INFINITY : INFINITY;
    if (f2u(truncf(y + copysignf(0.49999997f, y))) != f2u(round_half_away(y))) bad_rnd++;
  }
  printf("div127 %llu round %llu\n", bad_div, bad_rnd);
  return (bad_div || bad_rnd) ? 1 : 0;
}
