/*
 * ehip.h — C ABI of the MI355X (gfx950) paged-attention path.
 *
 * This is the single device boundary of the engine's attention hot path: the
 * host C++ (kvcache bookkeeping, step packing) and any foreign caller (ctypes,
 * cgo, JNI) call HIP only through these functions. Plain pointers and sizes;
 * no C++ or framework types cross it.
 *
 * Conventions
 *   - Every function returns an int status with the values of the reference's
 *     core::StatusCode (src/core/status.h:52-64): 0 OK, 2 InvalidArgument,
 *     5 FailedPrecondition, 7 ResourceExhausted, 8 OutOfMemory,
 *     9 Unimplemented, 11 Internal. On failure ehip_last_error() holds a
 *     message. Where the reference CHECK-aborts on a programmer error
 *     (block_size not dividing 64, src/kernels/paged_attention.cpp:88-91) this
 *     ABI returns InvalidArgument instead, so a foreign caller can recover.
 *   - Pointers named d_* are device (HBM) pointers, normally from
 *     ehip_malloc. Pointers named h_* are host memory; they are read before
 *     the call returns and may be reused immediately.
 *   - Compute calls are asynchronous on the context's stream (all-or-nothing:
 *     argument validation happens before anything is enqueued). ehip_sync()
 *     waits, and reports device-side range errors (a slot or block id outside
 *     the slab, which the kernels skip instead of touching memory out of
 *     bounds).
 *   - Slabs use the reference layout [slab_blocks, Hkv, bs, d]
 *     (docs/design/paged-kv-cache.md:146-160): block id `blk` at
 *     blk*block_stride elements, kv head `hk` at +hk*bs*d, slot p at +p*d.
 *     KV element type is fp32 or bf16 (bf16 = the reference's
 *     Fp32ToBf16Bits round-to-nearest-even, src/tensor/half.h:112-124).
 *   - Queries and outputs are fp32, [rows, H, d] contiguous. Softmax,
 *     running sums and accumulation are fp32 everywhere, and P.V is fp32 on
 *     the vector ALUs in every decode kernel. The q.k products differ by
 *     kernel: bf16-KV decode multiplies bf16 K by q split into bf16 hi + lo
 *     parts (q = hi + lo to about 2^-17 relative) on the matrix cores;
 *     fp32-KV decode at head_dim 64 splits q and K into three bf16 parts each
 *     and accumulates the six leading products on the matrix cores (what is
 *     left out is below 2^-24 of |q||k| per element), and is all-fp32 on the
 *     vector ALUs at other head sizes; INT8 KV forms exact integer q.k
 *     products of a three-digit int8 split of q; FP8 KV widens the E4M3 keys
 *     to bf16 (exact) and multiplies them by q in bf16 hi + lo parts. The
 *     causal prefill-chunk kernel rounds q and the probabilities P to bf16
 *     for its matrix-core products (fp32 accumulate). The parity bars these
 *     give are stated beside each test.
 *   - A context is used from one host thread at a time (the reference's
 *     single engine thread, src/runtime/engine.h:27-33).
 */
#ifndef EHIP_H_
#define EHIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  EHIP_OK = 0,
  EHIP_INVALID_ARGUMENT = 2,
  EHIP_FAILED_PRECONDITION = 5,
  EHIP_RESOURCE_EXHAUSTED = 7,
  EHIP_OUT_OF_MEMORY = 8,
  EHIP_UNIMPLEMENTED = 9,
  EHIP_INTERNAL = 11
};

/* KV element types. INT8 and FP8 slabs carry fp32 per-(block, kv head) scales
 * in separate [slab_blocks, kv_heads] arrays (one for K, one for V): the format
 * the reference reserves in docs/design/paged-kv-cache.md:219-231. FP8 is the
 * OCP E4M3 format (4 exponent bits with bias 7, 3 mantissa bits, largest
 * finite value 448, codes 0x7F / 0xFF NaN). */
enum { EHIP_KV_F32 = 0, EHIP_KV_BF16 = 1, EHIP_KV_INT8 = 2, EHIP_KV_FP8 = 3 };
/* Weight storage of the packed linear layer (the reference's PackedLinear
 * weight dtypes kFloat32 / kBFloat16 / kFloat16, src/model/packed_linear.h:31-36). */
enum { EHIP_WEIGHT_F32 = 0, EHIP_WEIGHT_BF16 = 1, EHIP_WEIGHT_F16 = 2 };

typedef struct ehip_ctx ehip_ctx;

/* Attention geometry of one model (constant across layers and steps).
 * Mirrors kvcache::CacheGeometry (src/kvcache/kv_cache.h:45-50) plus the
 * per-call scalars the reference kernels take (paged_attention.h:50-57). */
typedef struct {
  int32_t heads;        /* H (query heads)                                   */
  int32_t kv_heads;     /* Hkv; H % Hkv == 0, group g = H / Hkv              */
  int32_t head_dim;     /* d                                                 */
  int32_t block_size;   /* bs in {8,16,32,64} (src/kvcache/block_pool.cpp:28-31) */
  int32_t kv_dtype;     /* EHIP_KV_F32, _BF16, _INT8 or _FP8                 */
  int32_t reserved;     /* must be 0                                         */
  int64_t slab_blocks;  /* blocks in each slab (bounds every block id)       */
  int64_t block_stride; /* elements per block id; 0 = Hkv*bs*d               */
  float scale;          /* multiplies the finished q.k dot (HF order)        */
} ehip_geometry;

/* One scheduler step (ragged): B sequences, sequence b contributes T_b query
 * rows (1 for decode, a causal chunk for prefill) at the END of its context
 * of L_b tokens (post-append), i.e. at positions L_b-T_b .. L_b-1, and
 * attends keys [0, position] (src/kernels/attention.h:221-227 for chunks,
 * src/kernels/paged_attention.h:105-110 for T_b == 1). Rows are packed
 * sequence-major like engine::BatchInputs::cu_seqlens
 * (src/engine/batch.h:81-103). */
typedef struct {
  int32_t num_seqs;              /* B >= 0                                   */
  int32_t reserved;              /* must be 0                                */
  const int32_t* h_query_lens;   /* [B]   T_b >= 1                           */
  const int64_t* h_context_lens; /* [B]   L_b >= T_b (post-append)           */
  const int32_t* h_table_offsets;/* [B+1] CSR offsets into h_table_ids       */
  const int32_t* h_table_ids;    /* [offsets[B]] physical block ids, >= ceil(L_b/bs) per seq */
  const int64_t* h_slot_mapping; /* [sum T_b] slots of the appended tokens, or NULL */
} ehip_step_desc;

/* ------------------------------------------------------------ context ---- */
int ehip_init(int device, ehip_ctx** out);
int ehip_destroy(ehip_ctx* ctx);
/* Copies the last failure message (NUL-terminated, truncated to n). */
int ehip_last_error(const ehip_ctx* ctx, char* buf, size_t n);
/* Device count, without creating a context (0 when no GPU is visible). */
int ehip_device_count(int* out);
/* Waits for all enqueued work; returns InvalidArgument if a kernel skipped an
 * out-of-range slot or block id since the previous ehip_sync, and Internal
 * (after clearing them) if the persistent decode kernel's item-queue counters
 * were left non-zero, which only overlapping launches on one context cause. */
int ehip_sync(ehip_ctx* ctx);
/* Enqueue the context's work on a caller's HIP stream (a hipStream_t passed
 * as void*), or back on the context's own stream when NULL. The per-layer
 * calls (ehip_step_kv_append*, ehip_step_rope_kv_append,
 * ehip_step_attention*) then record into a graph the caller captures on that
 * stream: they enqueue kernels only (no allocation, copy, memset or
 * synchronisation), and the persistent decode kernel leaves its queue
 * counters zero, so a captured layer sequence replays without host work.
 * ehip_step_upload copies the step descriptor and is not captured.
 * Switching streams first waits (on the host) for the work already queued on
 * the current stream: a context has one descriptor arena, one split
 * workspace and one set of queue counters, so its launches must never run on
 * two streams at once. FailedPrecondition if the current stream is being
 * captured (end the capture first). No counterpart in the reference (its
 * kernels run on the calling thread). */
int ehip_set_stream(ehip_ctx* ctx, void* stream);

/* ------------------------------------------------------------ memory ----- */
/* HBM allocation, 256-byte aligned, zero-filled (the reference BlockPool
 * zero-fills its slabs, src/kvcache/block_pool.cpp:195-220). */
int ehip_malloc(ehip_ctx* ctx, int64_t bytes, void** d_out);
int ehip_free(ehip_ctx* ctx, void* d_ptr);
/* Blocking copies (stream-ordered behind all enqueued work). */
int ehip_copy_to_device(ehip_ctx* ctx, void* d_dst, const void* h_src, int64_t bytes);
int ehip_copy_to_host(ehip_ctx* ctx, void* h_dst, const void* d_src, int64_t bytes);
int ehip_copy_device(ehip_ctx* ctx, void* d_dst, const void* d_src, int64_t bytes);
/* Synthetic N(mean, std) fill on the device (counter-based hash + Box-Muller;
 * for benchmarks whose pools are too large to generate on the host).
 * dtype: EHIP_KV_F32 writes float, EHIP_KV_BF16 writes RNE bf16 bits,
 * EHIP_KV_FP8 writes E4M3 codes (RNE, saturated to +-448). */
int ehip_fill_normal(ehip_ctx* ctx, void* d_dst, int64_t n, int32_t dtype, float mean,
                     float stddev, uint64_t seed);

/* ---------------------------------------------------- seeded host fills --
 * The reference's deterministic fills (src/tensor/ops.h:88-109): engine
 * std::mt19937_64(seed), whose output sequence the C++ standard fixes.
 * Host memory only; no context needed. */
/* Outputs skip .. skip+n-1 of std::mt19937_64(seed) (raw 64-bit values; the
 * reference's uniforms are (x >> 11) * 2^-53, src/tensor/ops.cpp:205-224). */
int ehip_rng_u64(uint64_t seed, uint64_t skip, uint64_t* h_out, int64_t n);
/* tensor::fill_normal (src/tensor/ops.cpp:451-477) on n fp32 elements:
 * Box-Muller on consecutive engine outputs, u1 = ((x >> 11) + 1) * 2^-53,
 * u2 = (x >> 11) * 2^-53, z0 = r cos(2 pi u2), z1 = r sin(2 pi u2),
 * element = (float)(mean + stddev * z); an odd n drops the last z1. Filled on
 * several threads; the values do not depend on their number. */
int ehip_host_fill_normal(float* h_dst, int64_t n, double mean, double stddev, uint64_t seed);
/* Fp32ToBf16Bits (src/tensor/half.h:112-124) over n host elements. */
int ehip_host_fp32_to_bf16(const float* h_src, uint16_t* h_dst, int64_t n);

/* ------------------------------------------------------------ timing ----- */
/* HIP events on the context's stream (the stream every kernel runs on). */
int ehip_event_create(ehip_ctx* ctx, void** ev_out);
int ehip_event_destroy(ehip_ctx* ctx, void* ev);
int ehip_event_record(ehip_ctx* ctx, void* ev);
int ehip_event_elapsed_ms(ehip_ctx* ctx, void* ev_start, void* ev_end, float* ms_out);

/* ----------------------------------------- reference kernel entry points --
 * Device-pointer versions of the reference kernels-module API, same argument
 * meaning and order, plus the slab capacity (`slab_blocks`) that lets the
 * kernels bound every block id they dereference. */

/* kernels::KvScatterF32 (src/kernels/kv_scatter.h:47-50,
 * src/kernels/kv_scatter.cpp:27-61): token t's K/V rows (src [T, Hkv, d],
 * token-major) go to slot slot_mapping[t] = block*bs + p, head h at
 * ((block*Hkv + h)*bs + p)*d. Bit-exact copy. */
int ehip_kv_scatter_f32(ehip_ctx* ctx, const float* d_src_k, const float* d_src_v,
                        const int64_t* d_slot_mapping, int64_t t_dim, int64_t kv_heads,
                        int64_t d, int64_t block_size, int64_t slab_blocks, float* d_k_slab,
                        float* d_v_slab);
/* The same scatter into bf16 slabs; every element narrowed with the
 * reference's Fp32ToBf16Bits (src/tensor/half.h:112-124), bit-exact. */
int ehip_kv_scatter_bf16(ehip_ctx* ctx, const float* d_src_k, const float* d_src_v,
                         const int64_t* d_slot_mapping, int64_t t_dim, int64_t kv_heads,
                         int64_t d, int64_t block_size, int64_t slab_blocks,
                         uint16_t* d_k_slab, uint16_t* d_v_slab);

/* kernels::KvGatherF32 (src/kernels/kv_gather.h:55-58,
 * src/kernels/kv_gather.cpp:63-89): paged -> contiguous [Hkv, L, d]. */
int ehip_kv_gather_f32(ehip_ctx* ctx, const float* d_k_slab, const float* d_v_slab,
                       const int32_t* d_block_table, int64_t block_size, int64_t length,
                       int64_t kv_heads, int64_t d, int64_t slab_blocks, float* d_out_k,
                       float* d_out_v);

/* kernels::PagedDecodeAttentionF32 (src/kernels/paged_attention.h:50-57):
 * out[H,d] = softmax(scale * q.K^T) V over keys [0, length-1] read through
 * d_block_table. block_size must divide 64 (else InvalidArgument). */
int ehip_paged_decode_attention_f32(ehip_ctx* ctx, const float* d_q, const float* d_k_slab,
                                    const float* d_v_slab, const int32_t* d_block_table,
                                    int64_t num_blocks, int64_t length, int64_t heads,
                                    int64_t kv_heads, int64_t d, int64_t block_size,
                                    int64_t block_stride, int64_t slab_blocks, float scale,
                                    float* d_out);

/* kernels::PrefillAttentionF32 (src/kernels/attention.h:40-43): causal
 * attention of T query rows at positions L-T .. L-1 over a contiguous cache,
 * q/out [T, H, d], k/v [Hkv, L, d] head-major (kv head hk at hk*L*d). fp32. */
int ehip_prefill_attention_f32(ehip_ctx* ctx, const float* d_q, const float* d_k,
                               const float* d_v, float* d_out, int64_t t_dim, int64_t heads,
                               int64_t kv_heads, int64_t d, int64_t l_dim, float scale);
/* kernels::DecodeAttentionF32 (src/kernels/attention.h:71-73): the T = 1 case,
 * q/out [H, d], k/v [Hkv, L, d]. fp32. Both read the contiguous cache through
 * the paged kernels (an identity table over 16-key runs of each kv head). */
int ehip_decode_attention_f32(ehip_ctx* ctx, const float* d_q, const float* d_k, const float* d_v,
                              float* d_out, int64_t heads, int64_t kv_heads, int64_t d,
                              int64_t l_dim, float scale);

/* The attention output's consumer, o_proj (src/model/optimized_model.cpp:346:
 * layer.o_proj->forward(ctx, tmp), a PackedLinear).
 *
 * kernels::PackWeightPanels (src/kernels/gemm.h:61-64): d_w [n, k] row-major
 * (weight_dtype EHIP_WEIGHT_F32 = fp32, _BF16 / _F16 = 16-bit bit patterns)
 * repacked into the reference's panel layout d_wp [ceil(n/16), k, 16]:
 * Wp[p, kk, r] = W[p*16 + r, kk], 0 past n (a pure permute, same dtype).
 * d_wp holds ceil(n/16)*k*16 elements (kernels::PackedWeightElements). */
int ehip_pack_weight_panels(ehip_ctx* ctx, const void* d_w, int32_t weight_dtype, int64_t n,
                            int64_t k, void* d_wp);
/* kernels::PackedGemm (src/kernels/gemm.h:76-78): y[m, n] = x[m, k] W^T
 * (+ bias[n], added after the k sum) over the packed weight. x, bias, y fp32;
 * y fully overwritten. On the matrix cores x is cut into three bf16 planes
 * and the weight into the planes its type needs to be exact (1 bf16, 2 fp16,
 * 3 fp32); the products of planes whose indices sum to at most 2 are summed
 * in fp32 (what is left out is below 2^-24 of |x||w| per term). Within the
 * reference's GEMM tolerance (allclose rtol 1e-4, atol 1e-5 sqrt(k)) of its
 * scalar result; deterministic. Calls with few row tiles split k over
 * workgroups and add the partials in split order (a workspace the context
 * owns). d_bias may be null. */
int ehip_packed_gemm(ehip_ctx* ctx, const float* d_x, int64_t m, int64_t k, const void* d_wp,
                     int32_t weight_dtype, int64_t n, const float* d_bias, float* d_y);

/* kernels::PrefillAttentionVarlenF32 (src/kernels/attention.h:221-227), in the
 * reference's argument order: sequence b's query rows are [cu_seqlens[b],
 * cu_seqlens[b+1]) of d_q/d_out [sum T, H, d], attending causally over its
 * own contiguous head-major cache d_k_seqs[b] / d_v_seqs[b] ([Hkv, L_b, d],
 * L_b = h_l_dims[b] >= T_b: P_b = L_b - T_b cached keys, then the chunk's).
 * cu_seqlens, the pointer arrays and l_dims are host arrays (the K/V they
 * point at are device memory). Every sequence is validated before anything is
 * launched; then each runs through the paged kernels over an identity table,
 * as ehip_prefill_attention_f32 (one plan and launch per sequence: the step
 * path, ehip_step_upload + ehip_step_attention, is the one-launch route over
 * paged slabs). num_seqs == 0 is a no-op. fp32. */
int ehip_prefill_attention_varlen_f32(ehip_ctx* ctx, const float* d_q,
                                      const int32_t* h_cu_seqlens, int64_t num_seqs,
                                      const float* const* h_k_seqs,
                                      const float* const* h_v_seqs, const int64_t* h_l_dims,
                                      float* d_out, int64_t heads, int64_t kv_heads, int64_t d,
                                      float scale);

/* No counterpart in the reference: the allocation-free variant of
 * ehip_paged_decode_attention_f32 (same arguments and results), for callers
 * that cannot allocate device memory — code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc. Its one-row plan and split
 * partials live in a static per-device scratch array of 4 MiB, written by a
 * kernel (no allocation, copy or host staging per call); rows that would need
 * more (key splits x H x (d + 2) x 4 bytes of partials, plus the plan) get
 * ResourceExhausted. Every call on a device shares that device's array, and
 * eager calls run in call order whichever context or stream makes them (each
 * waits for the previous call's end through a per-device event). A call made
 * on a stream under graph capture is ordered only by its graph: replays of
 * it must not overlap eager calls on the same device. */
int ehip_paged_decode_attention_f32_noalloc(ehip_ctx* ctx, const float* d_q,
                                            const float* d_k_slab, const float* d_v_slab,
                                            const int32_t* d_block_table, int64_t num_blocks,
                                            int64_t length, int64_t heads, int64_t kv_heads,
                                            int64_t d, int64_t block_size, int64_t block_stride,
                                            int64_t slab_blocks, float scale, float* d_out);

/* kernels::PagedDecodeAttentionBatchedF32 (src/kernels/paged_attention.h:105-110):
 * B sequences over one shared slab pair. Like the reference, the tables are
 * host arrays of per-sequence pointers (h_block_tables[b] has
 * >= ceil(h_lengths[b]/bs) entries); they are packed into one CSR descriptor
 * and uploaded with a single copy. q/out [B, H, d]. B == 0 is a no-op. */
int ehip_paged_decode_attention_batched_f32(
    ehip_ctx* ctx, const float* d_q, const float* d_k_slab, const float* d_v_slab,
    const int32_t* const* h_block_tables, const int64_t* h_lengths, int64_t num_seqs,
    int64_t heads, int64_t kv_heads, int64_t d, int64_t block_size, int64_t block_stride,
    int64_t slab_blocks, float scale, float* d_out);
/* The bf16-KV variant of the batched decode (slabs hold bf16 bits). */
int ehip_paged_decode_attention_batched_bf16(
    ehip_ctx* ctx, const float* d_q, const uint16_t* d_k_slab, const uint16_t* d_v_slab,
    const int32_t* const* h_block_tables, const int64_t* h_lengths, int64_t num_seqs,
    int64_t heads, int64_t kv_heads, int64_t d, int64_t block_size, int64_t block_stride,
    int64_t slab_blocks, float scale, float* d_out);

/* ------------------------------------------------ step path (hot path) ----
 * One descriptor upload per scheduler step, then per layer one append and one
 * attention launch covering every sequence (decode rows and prefill chunks
 * alike). Replaces the per-sequence loops of OptimizedModel::BatchedAttention
 * (src/model/optimized_model.cpp:370-467) and PagedKvCache::append
 * (src/kvcache/paged_cache.cpp:62-123). Block tables are layer-independent
 * (src/kvcache/block_pool.h:22-24), so one upload serves every layer. */

/* Validates the step against the geometry, builds the work list (split-KV
 * partition, load-balanced order) and uploads it with one async copy. */
int ehip_step_upload(ehip_ctx* ctx, const ehip_geometry* geom, const ehip_step_desc* step);
/* Append the step's new K/V rows (src [sum T_b, Hkv, d] fp32) at the uploaded
 * slot mapping; slabs are fp32 or bf16 per geom.kv_dtype. */
int ehip_step_kv_append(ehip_ctx* ctx, const float* d_src_k, const float* d_src_v,
                        void* d_k_slab, void* d_v_slab);
/* RoPE fused into the append: rotates q [sum T_b, H, d] in place and each new
 * K row (src [sum T_b, Hkv, d] fp32) on its way into the slab, and appends V
 * unrotated. Row t of sequence b sits at position context_lens[b] -
 * query_lens[b] + t (the positions BatchAssembler hands the model,
 * src/engine/batch.cpp:70-76). d_cos/d_sin are [table_positions, d/2] fp32
 * (Rope::cos()/sin(), src/model/modules.h:185-207). Replaces the two
 * kernels::RopeApplyF32 calls before the append in OptimizedModel's layer
 * forward (src/model/optimized_model.cpp:284-291, kernels in
 * src/kernels/rope.h:34) plus ehip_step_kv_append; q and the slab rows equal
 * the reference AVX2 kernel's results bit for bit (bf16 slabs after
 * round-to-nearest-even). d_src_k is left unrotated. EHIP_INVALID_ARGUMENT
 * when a position is >= table_positions, as OptimizedModel::forward rejects
 * positions past max_position_embeddings (src/model/optimized_model.cpp:529-535). */
int ehip_step_rope_kv_append(ehip_ctx* ctx, float* d_q, const float* d_src_k,
                             const float* d_src_v, const float* d_cos, const float* d_sin,
                             int64_t table_positions, void* d_k_slab, void* d_v_slab);
/* Attention for every row of the step: q/out [sum T_b, H, d] fp32. */
int ehip_step_attention(ehip_ctx* ctx, const float* d_q, const void* d_k_slab,
                        const void* d_v_slab, float* d_out);
/* ehip_step_kv_append followed by ehip_step_attention, with the same results
 * bit for bit (the append into the slabs, the outputs). When every row of the
 * step is a decode row (T_b == 1) on bf16 slabs covered by the matrix-core
 * decode kernel, both run in one launch (plus the split merge): the work item
 * that ends at a row's last key stores that row's new K/V and uses them
 * directly; otherwise the two launches run in order. Together they stand for
 * PagedKvCache::append followed by the batched attention in the reference's
 * layer forward (src/model/optimized_model.cpp:370-467). */
int ehip_step_append_attention(ehip_ctx* ctx, const float* d_src_k, const float* d_src_v,
                               const float* d_q, void* d_k_slab, void* d_v_slab, float* d_out);
/* INT8 KV (geometry kv_dtype EHIP_KV_INT8): the append quantises the step's
 * new rows into int8 slabs with fp32 scales [slab_blocks, kv_heads] per slab
 * (requantising a block's older rows when a new row exceeds its range; a row
 * at offset 0 starts a fresh block), and the attention dequantises through
 * the scales. The reference reserves this format
 * (docs/design/paged-kv-cache.md:219-231: INT8 slabs plus per-block-per-head
 * scales, dequantised inside the attention kernels) without implementing it;
 * these entry points add the scale parameters to ehip_step_kv_append and
 * ehip_step_attention as that design says. Covered shapes: head_dim 64 or
 * 128, g in {1, 2, 4, 8}, block_size >= 16. */
int ehip_step_kv_append_int8(ehip_ctx* ctx, const float* d_src_k, const float* d_src_v,
                             void* d_k_slab, void* d_v_slab, float* d_k_scale, float* d_v_scale);
int ehip_step_attention_int8(ehip_ctx* ctx, const float* d_q, const void* d_k_slab,
                             const void* d_v_slab, const float* d_k_scale,
                             const float* d_v_scale, float* d_out);
/* FP8 KV (geometry kv_dtype EHIP_KV_FP8): the same per-(block, kv head)
 * scaled format and entry points as INT8, with E4M3 codes in place of int8:
 * scale = max|x| / 448 when a block's range grows, code = E4M3(x / scale) with
 * round to nearest even (NaN stays NaN, 0x7F). The reference reserves the
 * element type for its FP8 KV cache (tensor::DataType::kFP8E4M3,
 * src/tensor/dtype.h:39; docs/design/tensor.md:159) and the scaled-slab seam
 * (docs/design/paged-kv-cache.md:219-231) without implementing either.
 * Covered shapes as for INT8. */
int ehip_step_kv_append_fp8(ehip_ctx* ctx, const float* d_src_k, const float* d_src_v,
                            void* d_k_slab, void* d_v_slab, float* d_k_scale, float* d_v_scale);
int ehip_step_attention_fp8(ehip_ctx* ctx, const float* d_q, const void* d_k_slab,
                            const void* d_v_slab, const float* d_k_scale, const float* d_v_scale,
                            float* d_out);
/* Counts of the uploaded plan (rows, work items, split partials). */
int ehip_step_info(const ehip_ctx* ctx, int64_t* rows, int64_t* items, int64_t* partials);

/* ------------------------------------------------ host-only planning ------
 * The work-list builder behind ehip_step_upload, callable without a GPU (for
 * tests of the host logic). Fills the counts the plan would have: query rows,
 * work items (of which joint_items serve two to four rows sharing leading
 * blocks), split partial slots, the base split length and the key re-reads
 * the joint items save (each group's shared prefix times its members minus
 * one). Any out pointer may be NULL. */
int ehip_plan_counts(const ehip_geometry* geom, const ehip_step_desc* step, int64_t* rows,
                     int64_t* items, int64_t* partials, int32_t* split_tokens,
                     int64_t* joint_items, int64_t* shared_tokens);
/* The work list of the same plan, in dispatch order, for tests of the host
 * logic: eight int32 per item {row, joint rows 2..4 (-1 where absent),
 * key_begin, key_end, kv_head, split}. Writes at most cap items; *n gets the
 * item count. */
int ehip_plan_items(const ehip_geometry* geom, const ehip_step_desc* step, int32_t* out,
                    int64_t cap, int64_t* n);
/* The causal prefill-chunk items of the plan ehip_step_upload would build
 * (chunks of >= 16 rows on the matrix-core kernel), in dispatch order: nine
 * int32 per item {row_base, chunk_rows, past, q0, kv_head, split, key_begin,
 * key_end, nsplit of the item's rows (0: unsplit)}. Writes at most cap items;
 * *n gets the item count. */
int ehip_plan_prefill_items(const ehip_geometry* geom, const ehip_step_desc* step, int32_t* out,
                            int64_t cap, int64_t* n);

#ifdef __cplusplus
}
#endif

#endif /* EHIP_H_ */
