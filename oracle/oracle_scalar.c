/*
 * CPU ORACLE — TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Scalar translation unit: seeded generators, bf16 narrowing, the polynomial
 * exp, the scalar attention primitives, the two-pass cpu::attention oracle,
 * KV scatter/gather, the deterministic thread pool and the public entries.
 * Built with -ffp-contract=off and no -mfma so that, like the reference's
 * scalar TU on the x86-64 baseline, no multiply-add is ever contracted.
 */
#define _GNU_SOURCE
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "oracle_internal.h"

/* ------------------------------------------------------------------------ */
/* mt19937_64 (the C++ standard's parameters, [rand.predef]) and the fills  */
/* of src/tensor/ops.cpp:205-224 (Rng) and :451-477 (fill_normal).          */
/* ------------------------------------------------------------------------ */
#define MT_N 312
#define MT_M 156
#define MT_UPPER 0xFFFFFFFF80000000ULL
#define MT_LOWER 0x000000007FFFFFFFULL

void orc_mt64_seed(orc_mt64* g, uint64_t seed) {
  g->mt[0] = seed;
  for (int i = 1; i < MT_N; ++i)
    g->mt[i] = 6364136223846793005ULL * (g->mt[i - 1] ^ (g->mt[i - 1] >> 62)) +
               (uint64_t)i;
  g->idx = MT_N;
}

uint64_t orc_mt64_next(orc_mt64* g) {
  if (g->idx >= MT_N) {
    for (int i = 0; i < MT_N; ++i) {
      const uint64_t x = (g->mt[i] & MT_UPPER) | (g->mt[(i + 1) % MT_N] & MT_LOWER);
      uint64_t xa = x >> 1;
      if (x & 1ULL) xa ^= 0xB5026F5AA96619E9ULL;
      g->mt[i] = g->mt[(i + MT_M) % MT_N] ^ xa;
    }
    g->idx = 0;
  }
  uint64_t y = g->mt[g->idx++];
  y ^= (y >> 29) & 0x5555555555555555ULL;
  y ^= (y << 17) & 0x71D67FFFEDA60000ULL;
  y ^= (y << 37) & 0xFFF7EEE000000000ULL;
  y ^= y >> 43;
  return y;
}

double orc_mt64_unit(orc_mt64* g) {
  return (double)(orc_mt64_next(g) >> 11) * 0x1.0p-53;
}

double orc_mt64_unit_nonzero(orc_mt64* g) {
  return (double)((orc_mt64_next(g) >> 11) + 1) * 0x1.0p-53;
}

void orc_fill_normal(float* out, int64_t n, double mean, double stddev,
                     uint64_t seed) {
  orc_mt64 g;
  orc_mt64_seed(&g, seed);
  const double two_pi = 6.283185307179586476925286766559;
  for (int64_t i = 0; i < n; i += 2) {
    const double u1 = orc_mt64_unit_nonzero(&g);
    const double u2 = orc_mt64_unit(&g);
    const double radius = sqrt(-2.0 * log(u1));
    const double angle = two_pi * u2;
    out[i] = (float)(mean + stddev * (radius * cos(angle)));
    if (i + 1 < n) out[i + 1] = (float)(mean + stddev * (radius * sin(angle)));
  }
}

void orc_fill_uniform(float* out, int64_t n, double low, double high,
                      uint64_t seed) {
  orc_mt64 g;
  orc_mt64_seed(&g, seed);
  const double extent = high - low;
  for (int64_t i = 0; i < n; ++i) out[i] = (float)(low + orc_mt64_unit(&g) * extent);
}

/* ------------------------------------------------------------------------ */
/* bf16 narrowing / widening (src/tensor/half.h:111-129).                   */
/* ------------------------------------------------------------------------ */
uint16_t orc_fp32_to_bf16_bits(float v) {
  uint32_t bits;
  memcpy(&bits, &v, sizeof bits);
  if ((bits & 0x7FFFFFFFu) > 0x7F800000u) {
    uint16_t r = (uint16_t)(bits >> 16);
    if ((r & 0x007Fu) == 0u) r |= 0x0040u;
    return r;
  }
  const uint32_t rounded = bits + 0x7FFFu + ((bits >> 16) & 1u);
  return (uint16_t)(rounded >> 16);
}

float orc_bf16_bits_to_fp32(uint16_t b) {
  const uint32_t bits = (uint32_t)b << 16;
  float f;
  memcpy(&f, &bits, sizeof f);
  return f;
}

void orc_fp32_to_bf16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_fp32_to_bf16_bits(in[i]);
}

void orc_bf16_to_fp32_array(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_bits_to_fp32(in[i]);
}

#include "oracle_exp.h"

float orc_exp_scalar(float x) { return orc_exp_inline(x); }

/* ------------------------------------------------------------------------ */
/* Scalar primitives (src/kernels/scalar/attention.cpp:20-58).              */
/* ------------------------------------------------------------------------ */
static float ops_dot_score_row(const float* q, const float* k_block, int64_t n,
                               int64_t d, float scale, float* scores) {
  float row_max = -INFINITY;
  for (int64_t j = 0; j < n; ++j) {
    const float* k = k_block + j * d;
    float dot = 0.0f;
    for (int64_t e = 0; e < d; ++e) dot += q[e] * k[e];
    const float s = dot * scale;
    scores[j] = s;
    row_max = s > row_max ? s : row_max;
  }
  return row_max;
}

static float ops_exp_row_sum(float* scores, int64_t n, float m_new) {
  float sum = 0.0f;
  for (int64_t j = 0; j < n; ++j) {
    const float e = orc_exp_scalar(scores[j] - m_new);
    scores[j] = e;
    sum += e;
  }
  return sum;
}

static void ops_scale_row(float* out, float s, int64_t d) {
  for (int64_t e = 0; e < d; ++e) out[e] *= s;
}

static void ops_axpy_row(float* out, float s, const float* x, int64_t d) {
  for (int64_t e = 0; e < d; ++e) out[e] += s * x[e];
}

#define ORC_UNITS(name) orc_scalar_##name
#include "oracle_units.h"

/* ------------------------------------------------------------------------ */
/* Deterministic thread pool. Persistent workers; one region at a time.     */
/* ------------------------------------------------------------------------ */
#define ORC_MAX_THREADS 256
static struct {
  pthread_mutex_t mu;
  pthread_cond_t work_cv;
  pthread_cond_t done_cv;
  int nthreads; /* including the caller */
  int started;  /* workers created */
  uint64_t generation;
  orc_body_fn body;
  void* ctx;
  int64_t n, grain, num_chunks;
  atomic_llong next_chunk;
  int active;
  pthread_t workers[ORC_MAX_THREADS];
} g_pool = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER,
            PTHREAD_COND_INITIALIZER, 1, 0, 0, 0, 0, 0, 0, 0, 0, 0, {0}};

static void run_chunks(void) {
  for (;;) {
    const long long c = atomic_fetch_add(&g_pool.next_chunk, 1);
    if (c >= g_pool.num_chunks) break;
    const int64_t begin = (int64_t)c * g_pool.grain;
    const int64_t end = ORC_MIN(begin + g_pool.grain, g_pool.n);
    g_pool.body(g_pool.ctx, begin, end);
  }
}

static void* worker_main(void* arg) {
  (void)arg;
  uint64_t seen = 0;
  for (;;) {
    pthread_mutex_lock(&g_pool.mu);
    while (g_pool.generation == seen) pthread_cond_wait(&g_pool.work_cv, &g_pool.mu);
    seen = g_pool.generation;
    pthread_mutex_unlock(&g_pool.mu);
    run_chunks();
    pthread_mutex_lock(&g_pool.mu);
    if (--g_pool.active == 0) pthread_cond_signal(&g_pool.done_cv);
    pthread_mutex_unlock(&g_pool.mu);
  }
  return NULL;
}

void orc_set_threads(int n) {
  if (n < 1) n = 1;
  if (n > ORC_MAX_THREADS) n = ORC_MAX_THREADS;
  pthread_mutex_lock(&g_pool.mu);
  while (g_pool.started < n - 1) {
    pthread_create(&g_pool.workers[g_pool.started], NULL, worker_main, NULL);
    pthread_detach(g_pool.workers[g_pool.started]);
    ++g_pool.started;
  }
  g_pool.nthreads = n;
  pthread_mutex_unlock(&g_pool.mu);
}

int orc_get_threads(void) { return g_pool.nthreads; }

void orc_parallel_for(int64_t n, int64_t grain, orc_body_fn body, void* ctx) {
  if (n <= 0) return;
  const int64_t num_chunks = (n + grain - 1) / grain;
  if (num_chunks <= 1 || g_pool.nthreads <= 1 || g_pool.started == 0) {
    body(ctx, 0, n);
    return;
  }
  pthread_mutex_lock(&g_pool.mu);
  g_pool.body = body;
  g_pool.ctx = ctx;
  g_pool.n = n;
  g_pool.grain = grain;
  g_pool.num_chunks = num_chunks;
  atomic_store(&g_pool.next_chunk, 0);
  /* Workers beyond nthreads-1 stay asleep only if never started; started
   * workers all join every region (they find no chunks when n is small). */
  g_pool.active = g_pool.started;
  ++g_pool.generation;
  pthread_cond_broadcast(&g_pool.work_cv);
  pthread_mutex_unlock(&g_pool.mu);
  run_chunks();
  pthread_mutex_lock(&g_pool.mu);
  while (g_pool.active > 0) pthread_cond_wait(&g_pool.done_cv, &g_pool.mu);
  pthread_mutex_unlock(&g_pool.mu);
}

/* ------------------------------------------------------------------------ */
/* Public attention entries (src/kernels/paged_attention.cpp:76-147,        */
/* src/kernels/attention.cpp:76-187).                                       */
/* ------------------------------------------------------------------------ */
typedef void (*paged_units_fn)(const orc_paged_args*, int64_t, int64_t);
typedef void (*prefill_units_fn)(const orc_prefill_args*, int64_t, int64_t);
typedef void (*decode_units_fn)(const orc_decode_args*, int64_t, int64_t);

static paged_units_fn paged_fn(int isa) {
  return isa == ORC_ISA_AVX2 ? orc_avx2_paged_decode_units
                             : orc_scalar_paged_decode_units;
}
static prefill_units_fn prefill_fn(int isa) {
  return isa == ORC_ISA_AVX2 ? orc_avx2_prefill_units : orc_scalar_prefill_units;
}
static decode_units_fn decode_fn(int isa) {
  return isa == ORC_ISA_AVX2 ? orc_avx2_decode_units : orc_scalar_decode_units;
}

static int bs_ok(int64_t bs) { return bs > 0 && ORC_KB % bs == 0; }

typedef struct {
  const orc_paged_args* a;
  paged_units_fn fn;
} paged_single_ctx;

static void paged_single_body(void* c, int64_t b, int64_t e) {
  const paged_single_ctx* p = (const paged_single_ctx*)c;
  p->fn(p->a, b, e);
}

int orc_paged_decode_f32(int isa, const float* q, const float* k_slab,
                         const float* v_slab, const int32_t* block_table,
                         int64_t num_blocks, int64_t length, int64_t heads,
                         int64_t kv_heads, int64_t d, int64_t block_size,
                         int64_t block_stride, float scale, float* out) {
  (void)num_blocks;
  if (!bs_ok(block_size)) return 2;
  const orc_paged_args a = {q, k_slab, v_slab, block_table, out, d, length,
                            heads / kv_heads, block_size, block_stride, scale};
  paged_single_ctx c = {&a, paged_fn(isa)};
  orc_parallel_for(kv_heads, 1, paged_single_body, &c);
  return 0;
}

typedef struct {
  const float* q;
  const float* k_slab;
  const float* v_slab;
  const int32_t* const* block_tables;
  const int64_t* lengths;
  float* out;
  int64_t heads, kv_heads, d, group, block_size, block_stride;
  float scale;
  paged_units_fn fn;
} paged_batched_ctx;

/* Unit u -> (sequence u / Hkv, kv head u % Hkv), each unit running the
 * single-sequence recurrence (src/kernels/paged_attention.cpp:51-72). */
static void paged_batched_body(void* c, int64_t begin, int64_t end) {
  const paged_batched_ctx* p = (const paged_batched_ctx*)c;
  const int64_t row = p->heads * p->d;
  for (int64_t u = begin; u < end; ++u) {
    const int64_t b = u / p->kv_heads;
    const int64_t hk = u % p->kv_heads;
    const orc_paged_args a = {p->q + b * row,       p->k_slab,
                              p->v_slab,            p->block_tables[b],
                              p->out + b * row,     p->d,
                              p->lengths[b],        p->group,
                              p->block_size,        p->block_stride,
                              p->scale};
    p->fn(&a, hk, hk + 1);
  }
}

int orc_paged_decode_batched_f32(int isa, const float* q, const float* k_slab,
                                 const float* v_slab,
                                 const int32_t* const* block_tables,
                                 const int64_t* lengths, int64_t num_seqs,
                                 int64_t heads, int64_t kv_heads, int64_t d,
                                 int64_t block_size, int64_t block_stride,
                                 float scale, float* out) {
  if (num_seqs == 0) return 0;
  if (!bs_ok(block_size)) return 2;
  paged_batched_ctx c = {q,       k_slab,   v_slab,           block_tables,
                         lengths, out,      heads,            kv_heads,
                         d,       heads / kv_heads, block_size, block_stride,
                         scale,   paged_fn(isa)};
  orc_parallel_for(num_seqs * kv_heads, 1, paged_batched_body, &c);
  return 0;
}

typedef struct {
  const orc_decode_args* a;
  decode_units_fn fn;
} decode_ctx;

static void decode_body(void* c, int64_t b, int64_t e) {
  const decode_ctx* p = (const decode_ctx*)c;
  p->fn(p->a, b, e);
}

void orc_decode_f32(int isa, const float* q, const float* k, const float* v,
                    float* out, int64_t heads, int64_t kv_heads, int64_t d,
                    int64_t l_dim, float scale) {
  const orc_decode_args a = {q, k, v, out, d, l_dim, heads / kv_heads, scale};
  decode_ctx c = {&a, decode_fn(isa)};
  orc_parallel_for(kv_heads, 1, decode_body, &c);
}

typedef struct {
  const orc_prefill_args* a;
  prefill_units_fn fn;
} prefill_ctx;

static void prefill_body(void* c, int64_t b, int64_t e) {
  const prefill_ctx* p = (const prefill_ctx*)c;
  p->fn(p->a, b, e);
}

void orc_prefill_f32(int isa, const float* q, const float* k, const float* v,
                     float* out, int64_t t_dim, int64_t heads, int64_t kv_heads,
                     int64_t d, int64_t l_dim, float scale) {
  const int64_t nqb = (t_dim + ORC_QB - 1) / ORC_QB;
  const orc_prefill_args a = {q,     k,     v,          out,
                              t_dim, heads, d,          l_dim,
                              heads / kv_heads, l_dim - t_dim, nqb, scale};
  prefill_ctx c = {&a, prefill_fn(isa)};
  orc_parallel_for(heads * nqb, 1, prefill_body, &c);
}

typedef struct {
  const float* q;
  const int32_t* cu;
  int64_t num_seqs;
  const float* const* k_seqs;
  const float* const* v_seqs;
  const int64_t* l_dims;
  float* out;
  int64_t heads, d, group;
  float scale;
  prefill_units_fn fn;
} varlen_ctx;

/* Sequence-major unit walk: sequence b owns H * ceil(T_b/32) units
 * (src/kernels/attention.cpp:76-108). */
static void varlen_body(void* c, int64_t unit_begin, int64_t unit_end) {
  const varlen_ctx* p = (const varlen_ctx*)c;
  int64_t base = 0;
  for (int64_t b = 0; b < p->num_seqs; ++b) {
    const int64_t t0 = p->cu[b];
    const int64_t t_dim = p->cu[b + 1] - t0;
    const int64_t nqb = (t_dim + ORC_QB - 1) / ORC_QB;
    const int64_t seq_end = base + p->heads * nqb;
    const int64_t lo = unit_begin > base ? unit_begin : base;
    const int64_t hi = unit_end < seq_end ? unit_end : seq_end;
    if (lo < hi) {
      const int64_t l_dim = p->l_dims[b];
      const orc_prefill_args a = {p->q + t0 * p->heads * p->d,
                                  p->k_seqs[b],
                                  p->v_seqs[b],
                                  p->out + t0 * p->heads * p->d,
                                  t_dim,
                                  p->heads,
                                  p->d,
                                  l_dim,
                                  p->group,
                                  l_dim - t_dim,
                                  nqb,
                                  p->scale};
      p->fn(&a, lo - base, hi - base);
    }
    base = seq_end;
  }
}

void orc_prefill_varlen_f32(int isa, const float* q, const int32_t* cu_seqlens,
                            int64_t num_seqs, const float* const* k_seqs,
                            const float* const* v_seqs, const int64_t* l_dims,
                            float* out, int64_t heads, int64_t kv_heads,
                            int64_t d, float scale) {
  int64_t total = 0;
  for (int64_t b = 0; b < num_seqs; ++b) {
    const int64_t t_dim = cu_seqlens[b + 1] - cu_seqlens[b];
    total += heads * ((t_dim + ORC_QB - 1) / ORC_QB);
  }
  varlen_ctx c = {q,   cu_seqlens, num_seqs, k_seqs,           v_seqs,
                  l_dims, out,     heads,    d,                heads / kv_heads,
                  scale, prefill_fn(isa)};
  orc_parallel_for(total, 1, varlen_body, &c);
}

/* ------------------------------------------------------------------------ */
/* KV scatter / gather (src/kernels/kv_scatter.cpp:27-61,                   */
/* src/kernels/kv_gather.cpp:42-89).                                        */
/* ------------------------------------------------------------------------ */
void orc_kv_scatter_f32(const float* src_k, const float* src_v,
                        const int64_t* slot_mapping, int64_t t_dim,
                        int64_t kv_heads, int64_t d, int64_t block_size,
                        float* k_slab, float* v_slab) {
  const int64_t head_stride = block_size * d;
  for (int64_t t = 0; t < t_dim; ++t) {
    const int64_t slot = slot_mapping[t];
    const int64_t block = slot / block_size;
    const int64_t p = slot % block_size;
    const int64_t dst_base = block * kv_heads * head_stride + p * d;
    const int64_t src_base = t * kv_heads * d;
    for (int64_t h = 0; h < kv_heads; ++h) {
      memcpy(k_slab + dst_base + h * head_stride, src_k + src_base + h * d,
             (size_t)d * sizeof(float));
      memcpy(v_slab + dst_base + h * head_stride, src_v + src_base + h * d,
             (size_t)d * sizeof(float));
    }
  }
}

void orc_kv_scatter_bf16(const float* src_k, const float* src_v,
                         const int64_t* slot_mapping, int64_t t_dim,
                         int64_t kv_heads, int64_t d, int64_t block_size,
                         uint16_t* k_slab, uint16_t* v_slab) {
  const int64_t head_stride = block_size * d;
  for (int64_t t = 0; t < t_dim; ++t) {
    const int64_t slot = slot_mapping[t];
    const int64_t block = slot / block_size;
    const int64_t p = slot % block_size;
    const int64_t dst_base = block * kv_heads * head_stride + p * d;
    const int64_t src_base = t * kv_heads * d;
    for (int64_t h = 0; h < kv_heads; ++h)
      for (int64_t e = 0; e < d; ++e) {
        k_slab[dst_base + h * head_stride + e] =
            orc_fp32_to_bf16_bits(src_k[src_base + h * d + e]);
        v_slab[dst_base + h * head_stride + e] =
            orc_fp32_to_bf16_bits(src_v[src_base + h * d + e]);
      }
  }
}

static int8_t q8(float x, float s) {
  if (s == 0.0f) return 0;
  const float inv = 1.0f / s;
  float y = rintf(x * inv);
  if (y > 127.0f) y = 127.0f;
  if (y < -127.0f) y = -127.0f;
  return (int8_t)y;
}

/* One (block, kv head) of one slab: new rows at offsets [off0, off0 + n). */
static void append_q8_tile(const float* src, int64_t src_row_stride, const int64_t* rows,
                           int64_t n, int64_t off0, int64_t d, int8_t* tile, float* scale) {
  float m = 0.0f;
  for (int64_t i = 0; i < n; ++i)
    for (int64_t e = 0; e < d; ++e) {
      const float a = fabsf(src[rows[i] * src_row_stride + e]);
      if (a > m) m = a;
    }
  const float s0 = off0 > 0 ? *scale : 0.0f;
  float s1 = s0;
  if (m > s0 * 127.0f) {
    s1 = m / 127.0f;
    for (int64_t r = 0; r < off0; ++r)
      for (int64_t e = 0; e < d; ++e) {
        const float x = (float)tile[r * d + e] * s0;
        tile[r * d + e] = q8(x, s1);
      }
  }
  for (int64_t i = 0; i < n; ++i)
    for (int64_t e = 0; e < d; ++e)
      tile[(off0 + i) * d + e] = q8(src[rows[i] * src_row_stride + e], s1);
  *scale = s1;
}

void orc_kv_append_int8(const float* src_k, const float* src_v, const int64_t* slot_mapping,
                        int64_t t_dim, int64_t kv_heads, int64_t d, int64_t block_size,
                        int8_t* k_slab, int8_t* v_slab, float* k_scale, float* v_scale) {
  int64_t* rows = (int64_t*)malloc(sizeof(int64_t) * (size_t)(block_size > 0 ? block_size : 1));
  char* done = (char*)calloc((size_t)(t_dim > 0 ? t_dim : 1), 1);
  for (int64_t t = 0; t < t_dim; ++t) {
    if (done[t]) continue;
    const int64_t block = slot_mapping[t] / block_size;
    /* every row of this call landing in `block`, in offset order */
    int64_t n = 0, off0 = block_size;
    for (int64_t u = t; u < t_dim; ++u)
      if (slot_mapping[u] / block_size == block) {
        const int64_t off = slot_mapping[u] % block_size;
        if (off < off0) off0 = off;
        done[u] = 1;
        rows[n++] = u;
      }
    /* order by offset (insertion sort; n <= block_size) */
    for (int64_t i = 1; i < n; ++i)
      for (int64_t j = i; j > 0 && slot_mapping[rows[j - 1]] > slot_mapping[rows[j]]; --j) {
        const int64_t x = rows[j];
        rows[j] = rows[j - 1];
        rows[j - 1] = x;
      }
    for (int64_t h = 0; h < kv_heads; ++h) {
      const int64_t tile = (block * kv_heads + h) * block_size * d;
      append_q8_tile(src_k + h * d, kv_heads * d, rows, n, off0, d, k_slab + tile,
                     k_scale + block * kv_heads + h);
      append_q8_tile(src_v + h * d, kv_heads * d, rows, n, off0, d, v_slab + tile,
                     v_scale + block * kv_heads + h);
    }
  }
  free(rows);
  free(done);
}

/* OCP FP8 E4M3 ("e4m3fn"): sign, 4 exponent bits (bias 7), 3 mantissa bits;
 * no infinities, 0x7F / 0xFF are NaN, 448 is the largest finite value. */
float orc_e4m3_to_fp32(uint8_t c) {
  const int e = (c >> 3) & 15, m = c & 7;
  float v;
  if (e == 15 && m == 7)
    v = NAN;
  else if (e == 0)
    v = ldexpf((float)m, -9); /* subnormal: m * 2^-9 */
  else
    v = ldexpf((float)(8 + m), e - 10); /* (1 + m/8) * 2^(e-7) */
  return (c & 0x80) ? -v : v;
}

uint8_t orc_fp32_to_e4m3(float x) {
  if (isnan(x)) return 0x7F;
  uint32_t bits;
  memcpy(&bits, &x, 4);
  const uint8_t sign = (uint8_t)((bits >> 24) & 0x80);
  const float a = fabsf(x);
  if (a >= 448.0f) return sign | 0x7E; /* saturate: [448, 464] rounds to 448 anyway */
  if (a < 0.015625f) {                 /* below 2^-6: subnormal steps of 2^-9 */
    /* a * 2^9 is exact; rint is round-to-nearest-even; 8 steps carry into the
     * smallest normal, whose code (exponent 1, mantissa 0) is 8 as well. */
    return sign | (uint8_t)rintf(a * 512.0f);
  }
  memcpy(&bits, &a, 4);
  int e = (int)(bits >> 23) - 127; /* 2^e <= a < 2^(e+1), -6 <= e <= 8 */
  uint32_t m = (bits & 0x7FFFFF) >> 20, rem = bits & 0xFFFFF;
  if (rem > 0x80000u || (rem == 0x80000u && (m & 1u))) ++m; /* to nearest, ties to even */
  if (m == 8u) {
    m = 0u;
    ++e;
  }
  return sign | (uint8_t)(((e + 7) << 3) | (int)m);
}

static uint8_t qf8(float x, float s) {
  if (s == 0.0f) return 0;
  const float inv = 1.0f / s;
  float y = x * inv;
  if (y > 448.0f) y = 448.0f;
  if (y < -448.0f) y = -448.0f;
  return orc_fp32_to_e4m3(y);
}

/* One (block, kv head) of one FP8 slab: new rows at offsets [off0, off0 + n). */
static void append_f8_tile(const float* src, int64_t src_row_stride, const int64_t* rows,
                           int64_t n, int64_t off0, int64_t d, uint8_t* tile, float* scale) {
  float m = 0.0f;
  for (int64_t i = 0; i < n; ++i)
    for (int64_t e = 0; e < d; ++e) {
      const float a = fabsf(src[rows[i] * src_row_stride + e]);
      if (a > m) m = a;
    }
  const float s0 = off0 > 0 ? *scale : 0.0f;
  float s1 = s0;
  if (m > s0 * 448.0f) {
    s1 = m / 448.0f;
    for (int64_t r = 0; r < off0; ++r)
      for (int64_t e = 0; e < d; ++e) {
        const float x = orc_e4m3_to_fp32(tile[r * d + e]) * s0;
        tile[r * d + e] = qf8(x, s1);
      }
  }
  for (int64_t i = 0; i < n; ++i)
    for (int64_t e = 0; e < d; ++e)
      tile[(off0 + i) * d + e] = qf8(src[rows[i] * src_row_stride + e], s1);
  *scale = s1;
}

/* The rows of one call grouped by destination block, in offset order (shared
 * by the INT8 and FP8 appends). Calls fn(block, rows, n, off0). */
static void for_each_block_group(const int64_t* slot_mapping, int64_t t_dim, int64_t block_size,
                                 void (*fn)(void*, int64_t, const int64_t*, int64_t, int64_t),
                                 void* ctx) {
  int64_t* rows = (int64_t*)malloc(sizeof(int64_t) * (size_t)(block_size > 0 ? block_size : 1));
  char* done = (char*)calloc((size_t)(t_dim > 0 ? t_dim : 1), 1);
  for (int64_t t = 0; t < t_dim; ++t) {
    if (done[t]) continue;
    const int64_t block = slot_mapping[t] / block_size;
    int64_t n = 0, off0 = block_size;
    for (int64_t u = t; u < t_dim; ++u)
      if (slot_mapping[u] / block_size == block) {
        const int64_t off = slot_mapping[u] % block_size;
        if (off < off0) off0 = off;
        done[u] = 1;
        rows[n++] = u;
      }
    for (int64_t i = 1; i < n; ++i)
      for (int64_t j = i; j > 0 && slot_mapping[rows[j - 1]] > slot_mapping[rows[j]]; --j) {
        const int64_t x = rows[j];
        rows[j] = rows[j - 1];
        rows[j - 1] = x;
      }
    fn(ctx, block, rows, n, off0);
  }
  free(rows);
  free(done);
}

struct f8_append_ctx {
  const float *src_k, *src_v;
  int64_t kv_heads, d, block_size;
  uint8_t *k_slab, *v_slab;
  float *k_scale, *v_scale;
};

static void f8_append_group(void* p, int64_t block, const int64_t* rows, int64_t n, int64_t off0) {
  const struct f8_append_ctx* c = (const struct f8_append_ctx*)p;
  for (int64_t h = 0; h < c->kv_heads; ++h) {
    const int64_t tile = (block * c->kv_heads + h) * c->block_size * c->d;
    append_f8_tile(c->src_k + h * c->d, c->kv_heads * c->d, rows, n, off0, c->d,
                   c->k_slab + tile, c->k_scale + block * c->kv_heads + h);
    append_f8_tile(c->src_v + h * c->d, c->kv_heads * c->d, rows, n, off0, c->d,
                   c->v_slab + tile, c->v_scale + block * c->kv_heads + h);
  }
}

void orc_kv_append_fp8(const float* src_k, const float* src_v, const int64_t* slot_mapping,
                       int64_t t_dim, int64_t kv_heads, int64_t d, int64_t block_size,
                       uint8_t* k_slab, uint8_t* v_slab, float* k_scale, float* v_scale) {
  struct f8_append_ctx c = {src_k, src_v, kv_heads, d, block_size, k_slab, v_slab, k_scale,
                            v_scale};
  for_each_block_group(slot_mapping, t_dim, block_size, f8_append_group, &c);
}

void orc_fp8_dequant(const uint8_t* slab, const float* scale, int64_t num_blocks,
                     int64_t kv_heads, int64_t block_size, int64_t d, float* out) {
  const int64_t tile = block_size * d;
  for (int64_t u = 0; u < num_blocks * kv_heads; ++u)
    for (int64_t i = 0; i < tile; ++i)
      out[u * tile + i] = orc_e4m3_to_fp32(slab[u * tile + i]) * scale[u];
}

void orc_int8_dequant(const int8_t* slab, const float* scale, int64_t num_blocks,
                      int64_t kv_heads, int64_t block_size, int64_t d, float* out) {
  const int64_t tile = block_size * d;
  for (int64_t u = 0; u < num_blocks * kv_heads; ++u)
    for (int64_t i = 0; i < tile; ++i) out[u * tile + i] = (float)slab[u * tile + i] * scale[u];
}

void orc_kv_gather_f32(const float* k_slab, const float* v_slab,
                       const int32_t* block_table, int64_t block_size,
                       int64_t length, int64_t kv_heads, int64_t d,
                       float* out_k, float* out_v) {
  if (length == 0) return;
  const int64_t nb = (length + block_size - 1) / block_size;
  const int64_t block_stride = kv_heads * block_size * d;
  const int64_t head_stride = block_size * d;
  for (int64_t u = 0; u < kv_heads * nb; ++u) {
    const int64_t h = u / nb;
    const int64_t b = u % nb;
    const int64_t base = b * block_size;
    const int64_t rows = ORC_MIN(block_size, length - base);
    const int64_t src = (int64_t)block_table[b] * block_stride + h * head_stride;
    const int64_t dst = h * length * d + base * d;
    memcpy(out_k + dst, k_slab + src, (size_t)(rows * d) * sizeof(float));
    memcpy(out_v + dst, v_slab + src, (size_t)(rows * d) * sizeof(float));
  }
}

/* ------------------------------------------------------------------------ */
/* Two-pass oracle (src/cpu/attention.cpp:40-177, src/cpu/softmax.cpp).     */
/* Rows are processed one at a time ([L] scores per row instead of the      */
/* reference's materialized [H*T, L] matrix); each row's arithmetic is the  */
/* same: ascending single-accumulator dots, -inf mask, max, expf(x - max),  */
/* ascending sum, multiply by 1/sum, ascending context sum over all L keys. */
/* ------------------------------------------------------------------------ */
typedef struct {
  const float* q;
  const float* k;
  const float* v;
  float* out;
  int64_t t_dim, heads, d, l_dim, group, past;
  float scale;
} attn_ctx;

static void attention_rows(void* c, int64_t begin, int64_t end) {
  const attn_ctx* a = (const attn_ctx*)c;
  float* row = (float*)malloc((size_t)a->l_dim * sizeof(float));
  for (int64_t r = begin; r < end; ++r) {
    const int64_t h = r / a->t_dim;
    const int64_t t = r % a->t_dim;
    const int64_t hk = h / a->group;
    const int64_t limit = a->past + t;
    const float* qv = a->q + (t * a->heads + h) * a->d;
    for (int64_t s = 0; s < a->l_dim; ++s) {
      if (s > limit) {
        row[s] = -INFINITY;
        continue;
      }
      const float* kv = a->k + (hk * a->l_dim + s) * a->d;
      float dot = 0.0f;
      for (int64_t e = 0; e < a->d; ++e) dot += qv[e] * kv[e];
      row[s] = dot * a->scale;
    }
    float row_max = row[0];
    for (int64_t j = 1; j < a->l_dim; ++j) row_max = row_max < row[j] ? row[j] : row_max;
    float sum = 0.0f;
    for (int64_t j = 0; j < a->l_dim; ++j) {
      const float e = expf(row[j] - row_max);
      row[j] = e;
      sum += e;
    }
    const float inv = 1.0f / sum;
    for (int64_t j = 0; j < a->l_dim; ++j) row[j] *= inv;
    float* ov = a->out + (t * a->heads + h) * a->d;
    for (int64_t e = 0; e < a->d; ++e) {
      float acc = 0.0f;
      for (int64_t s = 0; s < a->l_dim; ++s)
        acc += row[s] * a->v[(hk * a->l_dim + s) * a->d + e];
      ov[e] = acc;
    }
  }
  free(row);
}

int orc_cpu_attention(const float* q, const float* k, const float* v,
                      int64_t t_dim, int64_t heads, int64_t kv_heads, int64_t d,
                      int64_t l_dim, float scale, float* out) {
  if (t_dim < 1 || heads < 1 || d < 1 || kv_heads < 1 || l_dim < 1) return 2;
  if (heads % kv_heads != 0 || l_dim < t_dim) return 2;
  attn_ctx c = {q, k, v, out, t_dim, heads, d, l_dim, heads / kv_heads,
                l_dim - t_dim, scale};
  orc_parallel_for(heads * t_dim, 1, attention_rows, &c);
  return 0;
}


/* RoPE row kernels (src/kernels/scalar/rope.cpp RopeRows and
 * src/kernels/avx2/rope.cpp RopeRows). This file is built with
 * -ffp-contract=off, so `lo * c - hi * s` rounds both products, as the
 * reference's scalar kernel does; fmaf() spells out the AVX2 kernel's fused
 * forms (bit-exact against the reference build for d = 10, 64, 72, 128, 130). */
void orc_rope_apply_f32(int isa, float* x, int64_t t, int64_t hx, int64_t d,
                        const int32_t* positions, const float* cos, const float* sin) {
  const int64_t half = d / 2;
  const int64_t fused = isa == 1 ? half / 8 * 8 : 0;  /* AVX2: whole 8-lane groups */
  for (int64_t i = 0; i < t; ++i) {
    const int64_t p = positions[i];
    const float* cr = cos + p * half;
    const float* sr = sin + p * half;
    for (int64_t h = 0; h < hx; ++h) {
      float* v = x + (i * hx + h) * d;
      for (int64_t j = 0; j < half; ++j) {
        const float c = cr[j], s = sr[j], lo = v[j], hi = v[j + half];
        if (j < fused) {
          v[j] = fmaf(-hi, s, lo * c);
          v[j + half] = fmaf(lo, s, hi * c);
        } else if (isa == 1) {
          /* the AVX2 kernel's scalar tail, which its build contracts into
           * fma(lo, c, -(hi*s)) and fma(hi, c, lo*s) */
          v[j] = fmaf(lo, c, -(hi * s));
          v[j + half] = fmaf(hi, c, lo * s);
        } else {
          v[j] = (lo * c) - (hi * s);
          v[j + half] = (hi * c) + (lo * s);
        }
      }
    }
  }
}

/* ------------------------------------------------------------------------ */
/* Packed linear layer (kernels::PackWeightPanels / PackedGemm).            */
/* ------------------------------------------------------------------------ */
enum { ORC_NR = 16 }; /* kernels::kNr (src/kernels/gemm.h:39) */

void orc_pack_weight_panels_u16(const uint16_t* w, int64_t n, int64_t k, uint16_t* wp) {
  const int64_t panels = (n + ORC_NR - 1) / ORC_NR;
  for (int64_t p = 0; p < panels; ++p)
    for (int64_t kk = 0; kk < k; ++kk)
      for (int64_t r = 0; r < ORC_NR; ++r) {
        const int64_t row = p * ORC_NR + r;
        wp[(p * k + kk) * ORC_NR + r] = row < n ? w[row * k + kk] : 0;
      }
}

void orc_pack_weight_panels_f32(const float* w, int64_t n, int64_t k, float* wp) {
  const int64_t panels = (n + ORC_NR - 1) / ORC_NR;
  for (int64_t p = 0; p < panels; ++p)
    for (int64_t kk = 0; kk < k; ++kk)
      for (int64_t r = 0; r < ORC_NR; ++r) {
        const int64_t row = p * ORC_NR + r;
        wp[(p * k + kk) * ORC_NR + r] = row < n ? w[row * k + kk] : 0.0f;
      }
}

static float orc_bits_f32(uint32_t b) {
  float f;
  memcpy(&f, &b, sizeof(f));
  return f;
}

float orc_fp16_bits_to_fp32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exponent = (h >> 10) & 0x1Fu;
  const uint32_t mantissa = h & 0x03FFu;
  if (exponent == 0x1Fu) return orc_bits_f32(sign | 0x7F800000u | (mantissa << 13));
  if (exponent == 0u) {
    if (mantissa == 0u) return orc_bits_f32(sign);
    /* Subnormal: normalise on the leading set bit n (0..9): 1.xxx * 2^(n-24). */
    int nb = 31 - __builtin_clz(mantissa);
    const uint32_t exp32 = 103u + (uint32_t)nb;
    const uint32_t man32 = (mantissa << (23u - (uint32_t)nb)) & 0x007FFFFFu;
    return orc_bits_f32(sign | (exp32 << 23) | man32);
  }
  return orc_bits_f32(sign | ((exponent + 112u) << 23) | (mantissa << 13));
}

static float orc_widen(const void* wp, int dtype, int64_t i) {
  if (dtype == 0) return ((const float*)wp)[i];
  const uint16_t b = ((const uint16_t*)wp)[i];
  return dtype == 1 ? orc_bits_f32((uint32_t)b << 16) : orc_fp16_bits_to_fp32(b);
}

int orc_packed_gemm(const float* x, int64_t m, int64_t k, const void* wp, int dtype, int64_t n,
                    const float* bias, float* y) {
  if (m < 1 || k < 1 || n < 1 || dtype < 0 || dtype > 2) return 2;
  const int64_t panels = (n + ORC_NR - 1) / ORC_NR;
  for (int64_t mm = 0; mm < m; ++mm) {
    const float* x_row = x + mm * k;
    for (int64_t p = 0; p < panels; ++p) {
      float acc[ORC_NR] = {0};
      for (int64_t kk = 0; kk < k; ++kk) {
        const float a = x_row[kk];
        const int64_t base = (p * k + kk) * ORC_NR;
        for (int64_t r = 0; r < ORC_NR; ++r) acc[r] += a * orc_widen(wp, dtype, base + r);
      }
      const int64_t col0 = p * ORC_NR;
      const int64_t ncols = ORC_MIN(ORC_NR, n - col0);
      float* y_row = y + mm * n + col0;
      for (int64_t r = 0; r < ncols; ++r) y_row[r] = bias ? acc[r] + bias[col0 + r] : acc[r];
    }
  }
  return 0;
}
