/*
 * CPU ORACLE — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of mathcslearner/LLM-Inference-Engine's paged-attention
 * path, used as the checker for the HIP implementation and as the CPU baseline
 * leg of bench.py. Nothing in the product library links, loads or calls this
 * code; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg do.
 *
 * Pinning (each function lists what checks it):
 *   - orc_mt64_* / orc_fill_*      : mt19937_64 known answer (10000th output of
 *                                    seed 5489), reference fill_normal spec
 *                                    (src/tensor/ops.h:88-109).
 *   - orc_fp32_to_bf16_bits        : RNE + NaN quieting (src/tensor/half.h:112-124),
 *                                    checked exhaustively on sampled bit patterns
 *                                    against numpy/torch RNE and special cases.
 *   - orc_exp_scalar / avx2        : <= 2 ulp vs double exp over the domain,
 *                                    flush/saturate/NaN clauses
 *                                    (src/kernels/internal/exp_common.h:63-86),
 *                                    bit-exact vs oracle/_ref where built.
 *   - scalar/avx2 attention units  : bit-exact vs oracle/_ref (the reference's
 *                                    own kernels compiled from its sources);
 *                                    HF goldens (tests/golden); fp64 brute force.
 *   - orc_cpu_attention            : HF goldens at rtol/atol 1e-4; fp64 brute
 *                                    force; causal-mask and GQA closed forms.
 *   - orc_kv_scatter/gather        : independent slot closed form + round trip,
 *                                    bit-exact vs oracle/_ref.
 *   - orc_pack_weight_panels_* /    : bit-exact vs oracle/_ref (the reference's
 *     orc_packed_gemm                scalar GemmTile and PackWeightPanels);
 *                                    fp64 brute force on small shapes; fp16
 *                                    widening exhaustive vs numpy float16.
 *
 * Error convention: functions return 0 on success and a core::StatusCode value
 * (2 = InvalidArgument) where the reference CHECK-aborts on a programmer error
 * (so a test can observe the rejection without killing the process).
 */
#ifndef ORACLE_ORACLE_H_
#define ORACLE_ORACLE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_ISA_SCALAR = 0, ORC_ISA_AVX2 = 1 };

/* ---- threading: deterministic parallel_for over independent units ---- */
void orc_set_threads(int n);
int orc_get_threads(void);

/* ---- seeded generators (src/tensor/ops.cpp:205-224, :451-477) ---- */
typedef struct {
  uint64_t mt[312];
  int idx;
} orc_mt64;
void orc_mt64_seed(orc_mt64* g, uint64_t seed);
uint64_t orc_mt64_next(orc_mt64* g);
double orc_mt64_unit(orc_mt64* g);         /* [0,1): (x>>11) * 2^-53     */
double orc_mt64_unit_nonzero(orc_mt64* g); /* (0,1]: ((x>>11)+1) * 2^-53 */
void orc_fill_normal(float* out, int64_t n, double mean, double stddev,
                     uint64_t seed);
void orc_fill_uniform(float* out, int64_t n, double low, double high,
                      uint64_t seed);

/* ---- bf16 (src/tensor/half.h:111-129) ---- */
uint16_t orc_fp32_to_bf16_bits(float v);
float orc_bf16_bits_to_fp32(uint16_t b);
void orc_fp32_to_bf16_array(const float* in, uint16_t* out, int64_t n);
void orc_bf16_to_fp32_array(const uint16_t* in, float* out, int64_t n);

/* ---- vector exp (src/kernels/internal/exp_common.h:63-86,
 *      src/kernels/internal/avx2_exp.h:15-43) ---- */
float orc_exp_scalar(float x);
void orc_exp_avx2_array(const float* in, float* out, int64_t n); /* n % 8 == 0 */

/* ---- kernels-module attention entry points (src/kernels/paged_attention.h,
 *      src/kernels/attention.h) ---- */
int orc_paged_decode_f32(int isa, const float* q, const float* k_slab,
                         const float* v_slab, const int32_t* block_table,
                         int64_t num_blocks, int64_t length, int64_t heads,
                         int64_t kv_heads, int64_t d, int64_t block_size,
                         int64_t block_stride, float scale, float* out);
int orc_paged_decode_batched_f32(int isa, const float* q, const float* k_slab,
                                 const float* v_slab,
                                 const int32_t* const* block_tables,
                                 const int64_t* lengths, int64_t num_seqs,
                                 int64_t heads, int64_t kv_heads, int64_t d,
                                 int64_t block_size, int64_t block_stride,
                                 float scale, float* out);
void orc_decode_f32(int isa, const float* q, const float* k, const float* v,
                    float* out, int64_t heads, int64_t kv_heads, int64_t d,
                    int64_t l_dim, float scale);
void orc_prefill_f32(int isa, const float* q, const float* k, const float* v,
                     float* out, int64_t t_dim, int64_t heads, int64_t kv_heads,
                     int64_t d, int64_t l_dim, float scale);
void orc_prefill_varlen_f32(int isa, const float* q, const int32_t* cu_seqlens,
                            int64_t num_seqs, const float* const* k_seqs,
                            const float* const* v_seqs, const int64_t* l_dims,
                            float* out, int64_t heads, int64_t kv_heads,
                            int64_t d, float scale);

/* ---- rotary position embedding, in place (src/kernels/rope.h:13-36;
 *      src/kernels/scalar/rope.cpp, src/kernels/avx2/rope.cpp). x [t, hx, d]
 *      fp32, cos/sin [P, d/2], positions [t]. isa 0: the scalar row kernel
 *      (lo*c - hi*s with both products rounded); isa 1: the AVX2 row kernel
 *      (fma(-hi, s, lo*c) and fma(lo, s, hi*c) over whole 8-wide groups of
 *      the half; fma(lo, c, -(hi*s)) and fma(hi, c, lo*s) for the rest). ---- */
void orc_rope_apply_f32(int isa, float* x, int64_t t, int64_t hx, int64_t d,
                        const int32_t* positions, const float* cos, const float* sin);

/* ---- KV scatter / gather (src/kernels/kv_scatter.cpp:27-61,
 *      src/kernels/kv_gather.cpp:42-89) ---- */
void orc_kv_scatter_f32(const float* src_k, const float* src_v,
                        const int64_t* slot_mapping, int64_t t_dim,
                        int64_t kv_heads, int64_t d, int64_t block_size,
                        float* k_slab, float* v_slab);
/* bf16-storage variant: the same slot arithmetic, each element narrowed with
 * orc_fp32_to_bf16_bits (the reference pool is fp32-only; this is the defined
 * semantics of the bf16-KV configs). */
void orc_kv_scatter_bf16(const float* src_k, const float* src_v,
                         const int64_t* slot_mapping, int64_t t_dim,
                         int64_t kv_heads, int64_t d, int64_t block_size,
                         uint16_t* k_slab, uint16_t* v_slab);
/* ---- INT8 KV with per-(block, kv head) scales ----
 * The reference reserves this format (docs/design/paged-kv-cache.md:219-231:
 * INT8 slabs [num_blocks, Hkv, bs, d] plus fp32 per-block-per-head scales
 * beside them, dequantised inside the attention kernels) without implementing
 * it, so these semantics are this build's; they are pinned by closed forms
 * (round-trip error, requantisation bounds, fresh-block reset) in
 * tests/test_oracle.py, not against a reference output.
 *
 * Append: the rows landing in one block in one call are quantised together.
 * For each (block, kv head) and each of K and V: m = max |x| over the new
 * rows; the block's old scale s0 counts only when the first new row's offset
 * in the block is > 0 (offset 0 means a freshly allocated block). If
 * m > s0 * 127 the scale becomes m / 127 and the block's older rows are
 * requantised (x' = q * s0, then quantised with the new scale); otherwise the
 * scale stays. quant(x, s) = 0 if s == 0, else clamp(rint(x * (1 / s)), -127,
 * 127). All arithmetic is fp32 with round-to-nearest-even. Rows of one block
 * must arrive with consecutive offsets (tokens append in order). */
void orc_kv_append_int8(const float* src_k, const float* src_v, const int64_t* slot_mapping,
                        int64_t t_dim, int64_t kv_heads, int64_t d, int64_t block_size,
                        int8_t* k_slab, int8_t* v_slab, float* k_scale, float* v_scale);
/* FP8 KV (OCP E4M3, "e4m3fn": bias 7, 3 mantissa bits, no infinities,
 * 0x7F/0xFF NaN, largest finite 448) with the INT8 layout and scale rule:
 * the same append as orc_kv_append_int8 with 448 in place of 127 and
 * quant(x, s) = 0 if s == 0, else e4m3(clamp(x * (1 / s), -448, 448)).
 * e4m3(y) rounds to nearest, ties to even (subnormal steps of 2^-9 below
 * 2^-6); |y| >= 448 saturates to 448 and NaN encodes as 0x7F. No reference
 * implementation exists either; tests/test_oracle.py pins the conversions
 * against torch.float8_e4m3fn over every code and every midpoint, and the
 * append by closed forms. */
float orc_e4m3_to_fp32(uint8_t c);
uint8_t orc_fp32_to_e4m3(float x);
void orc_kv_append_fp8(const float* src_k, const float* src_v, const int64_t* slot_mapping,
                       int64_t t_dim, int64_t kv_heads, int64_t d, int64_t block_size,
                       uint8_t* k_slab, uint8_t* v_slab, float* k_scale, float* v_scale);
/* Dequantised fp32 copy of an FP8 slab: x = e4m3(q) * scale[block, head]. */
void orc_fp8_dequant(const uint8_t* slab, const float* scale, int64_t num_blocks,
                     int64_t kv_heads, int64_t block_size, int64_t d, float* out);
/* Dequantised fp32 copy of an INT8 slab: x = q * scale[block, head]. */
void orc_int8_dequant(const int8_t* slab, const float* scale, int64_t num_blocks,
                      int64_t kv_heads, int64_t block_size, int64_t d, float* out);

void orc_kv_gather_f32(const float* k_slab, const float* v_slab,
                       const int32_t* block_table, int64_t block_size,
                       int64_t length, int64_t kv_heads, int64_t d,
                       float* out_k, float* out_v);

/* ---- the two-pass oracle cpu::attention (src/cpu/attention.cpp:97-177,
 *      src/cpu/softmax.cpp:24-73). q [T,H,d], k/v [Hkv,L,d], out [T,H,d]. ---- */
int orc_cpu_attention(const float* q, const float* k, const float* v,
                      int64_t t_dim, int64_t heads, int64_t kv_heads, int64_t d,
                      int64_t l_dim, float scale, float* out);

/* ---- packed linear layer (the attention output's consumer, o_proj) ----
 * Weight dtype codes: 0 fp32, 1 bf16 bits, 2 fp16 bits.
 * kernels::PackWeightPanels (src/kernels/gemm.cpp:119-151): w [n, k] ->
 * wp [ceil(n/16), k, 16], wp[p, kk, r] = w[p*16 + r, kk], 0 past n. */
void orc_pack_weight_panels_u16(const uint16_t* w, int64_t n, int64_t k, uint16_t* wp);
void orc_pack_weight_panels_f32(const float* w, int64_t n, int64_t k, float* wp);
/* IEEE binary16 bits -> fp32 (src/tensor/half.h:84-109). */
float orc_fp16_bits_to_fp32(uint16_t h);
/* kernels::PackedGemm's scalar tile (src/kernels/scalar/gemm.cpp:21-41) and
 * store (src/kernels/internal/gemm_common.h:22-41): per output row and panel
 * a 16-wide fp32 accumulator summed in ascending k, bias added after. */
int orc_packed_gemm(const float* x, int64_t m, int64_t k, const void* wp, int dtype, int64_t n,
                    const float* bias, float* y);

#ifdef __cplusplus
}
#endif

#endif /* ORACLE_ORACLE_H_ */
