/*
 * CPU ORACLE — TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * AVX2 translation unit: the 8-lane primitives of
 * src/kernels/avx2/attention.cpp:25-99 and the lane exp of
 * src/kernels/internal/avx2_exp.h:15-43, restated with intrinsics and driven
 * by the same control flow as the scalar TU (oracle_units.h). Built with
 * -mavx2 -mfma -mf16c -ffp-contract=fast: besides the explicit intrinsics,
 * GCC fuses the scalar tails and the inline scalar exp exactly as it does for
 * the reference's AVX2 TU (GCC contracts by default in C++, ISO mode included). This is the CPU baseline that
 * bench.py times beside the GPU.
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>

#include "oracle.h"
#include "oracle_internal.h"

#include "oracle_exp.h"

static inline __m256 exp8(__m256 x) {
  const __m256 flush = _mm256_cmp_ps(x, _mm256_set1_ps(EXP_LO), _CMP_LT_OQ);
  x = _mm256_min_ps(x, _mm256_set1_ps(EXP_HI));
  __m256 fx = _mm256_fmadd_ps(x, _mm256_set1_ps(EXP_LOG2E), _mm256_set1_ps(0.5f));
  fx = _mm256_floor_ps(fx);
  x = _mm256_fnmadd_ps(fx, _mm256_set1_ps(EXP_C1), x);
  x = _mm256_fnmadd_ps(fx, _mm256_set1_ps(EXP_C2), x);
  const __m256 z = _mm256_mul_ps(x, x);
  __m256 y = _mm256_set1_ps(EXP_P0);
  y = _mm256_fmadd_ps(y, x, _mm256_set1_ps(EXP_P1));
  y = _mm256_fmadd_ps(y, x, _mm256_set1_ps(EXP_P2));
  y = _mm256_fmadd_ps(y, x, _mm256_set1_ps(EXP_P3));
  y = _mm256_fmadd_ps(y, x, _mm256_set1_ps(EXP_P4));
  y = _mm256_fmadd_ps(y, x, _mm256_set1_ps(EXP_P5));
  y = _mm256_fmadd_ps(y, z, _mm256_add_ps(x, _mm256_set1_ps(1.0f)));
  __m256i n = _mm256_cvttps_epi32(fx);
  n = _mm256_slli_epi32(_mm256_add_epi32(n, _mm256_set1_epi32(127)), 23);
  const __m256 res = _mm256_mul_ps(y, _mm256_castsi256_ps(n));
  return _mm256_blendv_ps(res, _mm256_setzero_ps(), flush);
}

void orc_exp_avx2_array(const float* in, float* out, int64_t n) {
  for (int64_t i = 0; i + 8 <= n; i += 8)
    _mm256_storeu_ps(out + i, exp8(_mm256_loadu_ps(in + i)));
}

/* Horizontal sum: (lo + hi), movehdup, add, movehl, add_ss
 * (src/kernels/avx2/attention.cpp:25-34). */
static inline float hsum256(__m256 v) {
  __m128 lo = _mm256_castps256_ps128(v);
  const __m128 hi = _mm256_extractf128_ps(v, 1);
  lo = _mm_add_ps(lo, hi);
  __m128 shuf = _mm_movehdup_ps(lo);
  __m128 sums = _mm_add_ps(lo, shuf);
  shuf = _mm_movehl_ps(shuf, sums);
  sums = _mm_add_ss(sums, shuf);
  return _mm_cvtss_f32(sums);
}

static float ops_dot_score_row(const float* q, const float* k_block, int64_t n,
                               int64_t d, float scale, float* scores) {
  float row_max = -INFINITY;
  for (int64_t j = 0; j < n; ++j) {
    const float* k = k_block + j * d;
    __m256 acc = _mm256_setzero_ps();
    int64_t e = 0;
    for (; e + 8 <= d; e += 8)
      acc = _mm256_fmadd_ps(_mm256_loadu_ps(q + e), _mm256_loadu_ps(k + e), acc);
    float dot = hsum256(acc);
    for (; e < d; ++e) dot += q[e] * k[e];
    const float s = dot * scale;
    scores[j] = s;
    row_max = s > row_max ? s : row_max;
  }
  return row_max;
}

static float ops_exp_row_sum(float* scores, int64_t n, float m_new) {
  const __m256 vm = _mm256_set1_ps(m_new);
  __m256 vsum = _mm256_setzero_ps();
  int64_t j = 0;
  for (; j + 8 <= n; j += 8) {
    const __m256 e = exp8(_mm256_sub_ps(_mm256_loadu_ps(scores + j), vm));
    _mm256_storeu_ps(scores + j, e);
    vsum = _mm256_add_ps(vsum, e);
  }
  float sum = hsum256(vsum);
  for (; j < n; ++j) {
    const float e = orc_exp_inline(scores[j] - m_new);
    scores[j] = e;
    sum += e;
  }
  return sum;
}

static void ops_scale_row(float* out, float s, int64_t d) {
  const __m256 vs = _mm256_set1_ps(s);
  int64_t e = 0;
  for (; e + 8 <= d; e += 8)
    _mm256_storeu_ps(out + e, _mm256_mul_ps(_mm256_loadu_ps(out + e), vs));
  for (; e < d; ++e) out[e] *= s;
}

static void ops_axpy_row(float* out, float s, const float* x, int64_t d) {
  const __m256 vs = _mm256_set1_ps(s);
  int64_t e = 0;
  for (; e + 8 <= d; e += 8)
    _mm256_storeu_ps(out + e, _mm256_fmadd_ps(vs, _mm256_loadu_ps(x + e),
                                              _mm256_loadu_ps(out + e)));
  for (; e < d; ++e) out[e] += s * x[e];
}

#define ORC_UNITS(name) orc_avx2_##name
#include "oracle_units.h"
