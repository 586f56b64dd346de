/* Exhaustive CPU check of the activation quantiser's fast arithmetic
 * (mlsys-contest-syfi-fully-agent_amd/csrc/quantize.hip, fast_pack4).
 *
 * TEST SUPPORT ONLY.  For every bf16 block maximum `amax` with bits in
 * [ab_lo, ab_hi) and every bf16 `x` with |x| <= amax (NaN excluded), the
 * kernel's fast quotient
 *     s = amax / 448, r = 1 / s  (correctly rounded),
 *     q = x * r,  q' = fma(fma(-s, q, x), r, q),  y = |q'| with the sign of x
 * must give the same e4m3 code as the CPU oracle's correctly rounded x / s
 * (orc_f32_to_e4m3(x / s), oracle/synth.c).  Every operation is a single IEEE
 * fp32 operation (built with -ffp-contract=off), the same ones the GPU kernel
 * issues, so the count carries over to the device.
 *
 * `variant` plants mistakes to show that the check can fail:
 *   0 the kernel's formula, 1 no correction step (y = x * r),
 *   2 no sign fix (y = q'). */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "../../oracle/oracle.h"

static float bf16(uint32_t b) {
  const uint32_t u = b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint64_t quant_fastpath_mismatches(uint32_t ab_lo, uint32_t ab_hi, int variant, uint64_t* pairs) {
  uint64_t bad = 0, tot = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : bad, tot)
  for (int64_t ab = ab_lo; ab < (int64_t)ab_hi; ++ab) {
    const float amax = bf16((uint32_t)ab);
    const float s = amax > 0.0f ? amax / 448.0f : 1.0f;
    const float r = 1.0f / s;
    for (uint32_t xb = 0; xb < 0x10000u; ++xb) {
      if ((xb & 0x7FFFu) > (uint32_t)ab) continue;
      const float x = bf16(xb);
      const float q = x * r;
      const float q2 = fmaf(fmaf(-s, q, x), r, q);
      const float y = variant == 1 ? q : variant == 2 ? q2 : copysignf(q2, x);
      ++tot;
      if (orc_f32_to_e4m3(y) != orc_f32_to_e4m3(x / s)) ++bad;
    }
  }
  if (pairs) *pairs = tot;
  return bad;
}
