/*
 * CPU ORACLE — TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * The online-softmax control flow shared by the scalar and AVX2 oracle TUs.
 * It restates, in C, the arithmetic order of:
 *   - PrefillUnitsImpl      src/kernels/internal/attention_common.h:95-155
 *   - DecodeGroupSlice /
 *     DecodeUnitsImpl       src/kernels/internal/attention_common.h:171-271
 *   - PagedDecodeGroupSlice src/kernels/internal/paged_attention_common.h:69-136
 *   - PagedDecodeUnitsImpl  src/kernels/internal/paged_attention_common.h:176-200
 * over a four-primitive ISA policy. The including TU defines, before including:
 *   static float ops_dot_score_row(q, k_block, n, d, scale, scores);
 *   static float ops_exp_row_sum(scores, n, m_new);
 *   static void  ops_scale_row(out, s, d);
 *   static void  ops_axpy_row(out, s, x, d);
 * and ORC_UNITS(name) that suffixes the emitted function names.
 * Block constants: 32 query rows per prefill unit, 64 keys per online-softmax
 * unit, decode group slices of <= 8 heads (attention_common.h:33-42).
 */
#include <math.h>
#include <stdint.h>

#include "oracle_exp.h"
#include "oracle_internal.h"

void ORC_UNITS(prefill_units)(const orc_prefill_args* a, int64_t u0,
                                     int64_t u1) {
  const int64_t d = a->d;
  const int64_t l_dim = a->l_dim;
  float scores[ORC_KB];
  for (int64_t unit = u0; unit < u1; ++unit) {
    const int64_t h = unit / a->num_qblocks;
    const int64_t qb = unit % a->num_qblocks;
    const int64_t hk = h / a->group;
    const int64_t q0 = qb * ORC_QB;
    const int64_t q1 = q0 + ORC_QB < a->t_dim ? q0 + ORC_QB : a->t_dim;
    const float* k_head = a->k + hk * l_dim * d;
    const float* v_head = a->v + hk * l_dim * d;
    for (int64_t t = q0; t < q1; ++t) {
      const float* q_vec = a->q + (t * a->heads + h) * d;
      float* out_vec = a->out + (t * a->heads + h) * d;
      for (int64_t e = 0; e < d; ++e) out_vec[e] = 0.0f;
      float run_max = -INFINITY;
      float run_den = 0.0f;
      const int64_t limit = a->past + t;
      for (int64_t kb = 0; kb <= limit; kb += ORC_KB) {
        const int64_t kb_len = ORC_MIN(ORC_KB, l_dim - kb);
        const int64_t n_valid = ORC_MIN(limit - kb + 1, kb_len);
        const float* k_block = k_head + kb * d;
        const float* v_block = v_head + kb * d;
        const float block_max =
            ops_dot_score_row(q_vec, k_block, n_valid, d, a->scale, scores);
        const float m_new = block_max > run_max ? block_max : run_max;
        const float alpha = orc_exp_inline(run_max - m_new);
        const float row_sum = ops_exp_row_sum(scores, n_valid, m_new);
        run_den = (run_den * alpha) + row_sum;
        ops_scale_row(out_vec, alpha, d);
        for (int64_t j = 0; j < n_valid; ++j)
          ops_axpy_row(out_vec, scores[j], v_block + j * d, d);
        run_max = m_new;
      }
      ops_scale_row(out_vec, 1.0f / run_den, d);
    }
  }
}

void ORC_UNITS(decode_units)(const orc_decode_args* a, int64_t u0,
                                    int64_t u1) {
  const int64_t d = a->d;
  const int64_t l_dim = a->l_dim;
  const int64_t group = a->group;
  const int64_t limit = l_dim - 1;
  float scores[ORC_KB];
  float run_max[ORC_GROUP_CHUNK];
  float run_den[ORC_GROUP_CHUNK];
  for (int64_t hk = u0; hk < u1; ++hk) {
    const float* k_head = a->k + hk * l_dim * d;
    const float* v_head = a->v + hk * l_dim * d;
    const int64_t hq_base = hk * group;
    for (int64_t g0 = 0; g0 < group; g0 += ORC_GROUP_CHUNK) {
      const int64_t gn = ORC_MIN(ORC_GROUP_CHUNK, group - g0);
      const int64_t hq0 = hq_base + g0;
      for (int64_t gi = 0; gi < gn; ++gi) {
        float* o = a->out + (hq0 + gi) * d;
        for (int64_t e = 0; e < d; ++e) o[e] = 0.0f;
        run_max[gi] = -INFINITY;
        run_den[gi] = 0.0f;
      }
      for (int64_t kb = 0; kb <= limit; kb += ORC_KB) {
        const int64_t kb_len = ORC_MIN(ORC_KB, l_dim - kb);
        const int64_t n_valid = ORC_MIN(limit - kb + 1, kb_len);
        const float* k_block = k_head + kb * d;
        const float* v_block = v_head + kb * d;
        for (int64_t gi = 0; gi < gn; ++gi) {
          const float* q_vec = a->q + (hq0 + gi) * d;
          float* o = a->out + (hq0 + gi) * d;
          const float block_max =
              ops_dot_score_row(q_vec, k_block, n_valid, d, a->scale, scores);
          const float m_new = block_max > run_max[gi] ? block_max : run_max[gi];
          const float alpha = orc_exp_inline(run_max[gi] - m_new);
          const float row_sum = ops_exp_row_sum(scores, n_valid, m_new);
          run_den[gi] = (run_den[gi] * alpha) + row_sum;
          ops_scale_row(o, alpha, d);
          for (int64_t j = 0; j < n_valid; ++j)
            ops_axpy_row(o, scores[j], v_block + j * d, d);
          run_max[gi] = m_new;
        }
      }
      for (int64_t gi = 0; gi < gn; ++gi)
        ops_scale_row(a->out + (hq0 + gi) * d, 1.0f / run_den[gi], d);
    }
  }
}

/* One group slice of the paged decode recurrence: identical to the decode
 * slice except that each 64-key unit's keys are read block by block through
 * the block table (whole blocks per unit since bs | 64). */
static void ORC_UNITS(paged_group_slice)(const orc_paged_args* a,
                                         int64_t head_off, int64_t hq0,
                                         int64_t gn, int64_t limit,
                                         float* scores, float* run_max,
                                         float* run_den) {
  const int64_t d = a->d;
  const int64_t bs = a->block_size;
  for (int64_t gi = 0; gi < gn; ++gi) {
    float* o = a->out + (hq0 + gi) * d;
    for (int64_t e = 0; e < d; ++e) o[e] = 0.0f;
    run_max[gi] = -INFINITY;
    run_den[gi] = 0.0f;
  }
  for (int64_t kb = 0; kb <= limit; kb += ORC_KB) {
    const int64_t kb_len = ORC_MIN(ORC_KB, a->length - kb);
    const int64_t n_valid = ORC_MIN(limit - kb + 1, kb_len);
    const int64_t lb0 = kb / bs;
    for (int64_t gi = 0; gi < gn; ++gi) {
      const float* q_vec = a->q + (hq0 + gi) * d;
      float* o = a->out + (hq0 + gi) * d;
      float block_max = -INFINITY;
      for (int64_t b = 0; b * bs < n_valid; ++b) {
        const int64_t phys = a->block_table[lb0 + b];
        const float* k_tile = a->k_slab + phys * a->block_stride + head_off;
        const int64_t n_b = ORC_MIN(bs, n_valid - b * bs);
        const float bmax =
            ops_dot_score_row(q_vec, k_tile, n_b, d, a->scale, scores + b * bs);
        block_max = bmax > block_max ? bmax : block_max;
      }
      const float m_new = block_max > run_max[gi] ? block_max : run_max[gi];
      const float alpha = orc_exp_inline(run_max[gi] - m_new);
      const float row_sum = ops_exp_row_sum(scores, n_valid, m_new);
      run_den[gi] = (run_den[gi] * alpha) + row_sum;
      ops_scale_row(o, alpha, d);
      for (int64_t b = 0; b * bs < n_valid; ++b) {
        const int64_t phys = a->block_table[lb0 + b];
        const float* v_tile = a->v_slab + phys * a->block_stride + head_off;
        const int64_t n_b = ORC_MIN(bs, n_valid - b * bs);
        for (int64_t p = 0; p < n_b; ++p)
          ops_axpy_row(o, scores[b * bs + p], v_tile + p * d, d);
      }
      run_max[gi] = m_new;
    }
  }
  for (int64_t gi = 0; gi < gn; ++gi)
    ops_scale_row(a->out + (hq0 + gi) * d, 1.0f / run_den[gi], d);
}

void ORC_UNITS(paged_decode_units)(const orc_paged_args* a, int64_t u0,
                                          int64_t u1) {
  const int64_t limit = a->length - 1;
  const int64_t head_span = a->block_size * a->d;
  float scores[ORC_KB];
  float run_max[ORC_GROUP_CHUNK];
  float run_den[ORC_GROUP_CHUNK];
  for (int64_t hk = u0; hk < u1; ++hk) {
    const int64_t head_off = hk * head_span;
    const int64_t hq_base = hk * a->group;
    for (int64_t g0 = 0; g0 < a->group; g0 += ORC_GROUP_CHUNK) {
      const int64_t gn = ORC_MIN(ORC_GROUP_CHUNK, a->group - g0);
      ORC_UNITS(paged_group_slice)(a, head_off, hq_base + g0, gn, limit, scores,
                                   run_max, run_den);
    }
  }
}
