/*
 * CPU ORACLE — TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Polynomial exp: the Cephes single-precision expf method (range reduction by
 * a two-part ln2, degree-5 polynomial, 2^n by exponent-field write) with the
 * reference's domain clauses (src/kernels/internal/exp_common.h:39-86):
 * x < lo flushes to +0, x > hi saturates, NaN passes through.
 * Inline so that each ISA TU compiles it under its own contraction rule, as the
 * reference's inline ExpF32Scalar is compiled into both its scalar and AVX2 TUs.
 */
#ifndef ORACLE_ORACLE_EXP_H_
#define ORACLE_ORACLE_EXP_H_

#include <math.h>
#include <stdint.h>
#include <string.h>

#define EXP_HI 88.3762626647949f
#define EXP_LO -87.3365478515625f
#define EXP_LOG2E 1.44269504088896341f
#define EXP_C1 0.693359375f
#define EXP_C2 -2.12194440e-4f
#define EXP_P0 1.9875691500e-4f
#define EXP_P1 1.3981999507e-3f
#define EXP_P2 8.3334519073e-3f
#define EXP_P3 4.1665795894e-2f
#define EXP_P4 1.6666665459e-1f
#define EXP_P5 5.0000001201e-1f

static inline float orc_exp_inline(float x) {
  if (x < EXP_LO) return 0.0f;
  x = (EXP_HI < x) ? EXP_HI : x; /* std::min(x, hi): NaN passes through */
  const float fx = floorf((EXP_LOG2E * x) + 0.5f);
  x -= fx * EXP_C1;
  x -= fx * EXP_C2;
  const float z = x * x;
  float y = EXP_P0;
  y = (y * x) + EXP_P1;
  y = (y * x) + EXP_P2;
  y = (y * x) + EXP_P3;
  y = (y * x) + EXP_P4;
  y = (y * x) + EXP_P5;
  y = (y * z) + x + 1.0f;
  const int32_t n = (int32_t)fx;
  const uint32_t bits = (uint32_t)(n + 127) << 23;
  float pow2n;
  memcpy(&pow2n, &bits, sizeof pow2n);
  return y * pow2n;
}

#endif /* ORACLE_ORACLE_EXP_H_ */
