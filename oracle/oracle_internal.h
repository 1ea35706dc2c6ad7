/*
 * CPU ORACLE — TEST INFRASTRUCTURE ONLY (see oracle.h). Internal types shared
 * by the oracle's translation units.
 */
#ifndef ORACLE_ORACLE_INTERNAL_H_
#define ORACLE_ORACLE_INTERNAL_H_

#include <stdint.h>

#include "oracle.h"

/* Block constants of src/kernels/internal/attention_common.h:33-42. */
#define ORC_QB 32
#define ORC_KB 64
#define ORC_GROUP_CHUNK 8
#define ORC_MIN(a, b) ((a) < (b) ? (a) : (b))

/* Flattened argument bundles (src/kernels/internal/attention_common.h:44-93,
 * src/kernels/internal/paged_attention_common.h:47-59). */
typedef struct {
  const float* q;
  const float* k;
  const float* v;
  float* out;
  int64_t t_dim, heads, d, l_dim, group, past, num_qblocks;
  float scale;
} orc_prefill_args;

typedef struct {
  const float* q;
  const float* k;
  const float* v;
  float* out;
  int64_t d, l_dim, group;
  float scale;
} orc_decode_args;

typedef struct {
  const float* q;
  const float* k_slab;
  const float* v_slab;
  const int32_t* block_table;
  float* out;
  int64_t d, length, group, block_size, block_stride;
  float scale;
} orc_paged_args;

/* Per-ISA unit walkers (emitted from oracle_units.h). */
void orc_scalar_prefill_units(const orc_prefill_args* a, int64_t u0, int64_t u1);
void orc_scalar_decode_units(const orc_decode_args* a, int64_t u0, int64_t u1);
void orc_scalar_paged_decode_units(const orc_paged_args* a, int64_t u0,
                                   int64_t u1);
void orc_avx2_prefill_units(const orc_prefill_args* a, int64_t u0, int64_t u1);
void orc_avx2_decode_units(const orc_decode_args* a, int64_t u0, int64_t u1);
void orc_avx2_paged_decode_units(const orc_paged_args* a, int64_t u0,
                                 int64_t u1);

/* Deterministic parallel_for (src/parallel/parallel_for.cpp): [0, n) cut into
 * ceil(n / grain) chunks of `grain` units (the cut depends only on n and
 * grain), executed by a persistent pool; the caller participates. */
typedef void (*orc_body_fn)(void* ctx, int64_t begin, int64_t end);
void orc_parallel_for(int64_t n, int64_t grain, orc_body_fn body, void* ctx);

#endif /* ORACLE_ORACLE_INTERNAL_H_ */
