#include "kernels.h"

#include <cmath>

#include "device_buffer.h"

namespace ehip::host::kernels {

Status PagedDecodeAttentionF32(ehip_ctx* ctx, const float* q, const float* k_slab,
                               const float* v_slab, const int32_t* d_block_table,
                               int64_t num_blocks, int64_t length, int64_t heads,
                               int64_t kv_heads, int64_t d, int64_t block_size,
                               int64_t block_stride, int64_t slab_blocks, float scale,
                               float* out) {
  return FromRc(ctx, ehip_paged_decode_attention_f32(ctx, q, k_slab, v_slab, d_block_table,
                                                     num_blocks, length, heads, kv_heads, d,
                                                     block_size, block_stride, slab_blocks,
                                                     scale, out));
}

Status PagedDecodeAttentionBatchedF32(ehip_ctx* ctx, const float* q, const float* k_slab,
                                      const float* v_slab, const int32_t* const* block_tables,
                                      const int64_t* lengths, int64_t num_seqs, int64_t heads,
                                      int64_t kv_heads, int64_t d, int64_t block_size,
                                      int64_t block_stride, int64_t slab_blocks, float scale,
                                      float* out) {
  return FromRc(ctx, ehip_paged_decode_attention_batched_f32(
                         ctx, q, k_slab, v_slab, block_tables, lengths, num_seqs, heads,
                         kv_heads, d, block_size, block_stride, slab_blocks, scale, out));
}

Status PagedDecodeAttentionBatchedBf16(ehip_ctx* ctx, const float* q, const uint16_t* k_slab,
                                       const uint16_t* v_slab,
                                       const int32_t* const* block_tables,
                                       const int64_t* lengths, int64_t num_seqs, int64_t heads,
                                       int64_t kv_heads, int64_t d, int64_t block_size,
                                       int64_t block_stride, int64_t slab_blocks, float scale,
                                       float* out) {
  return FromRc(ctx, ehip_paged_decode_attention_batched_bf16(
                         ctx, q, k_slab, v_slab, block_tables, lengths, num_seqs, heads,
                         kv_heads, d, block_size, block_stride, slab_blocks, scale, out));
}

Status KvScatterF32(ehip_ctx* ctx, const float* src_k, const float* src_v,
                    const int64_t* d_slot_mapping, int64_t t_dim, int64_t kv_heads, int64_t d,
                    int64_t block_size, int64_t slab_blocks, float* k_slab, float* v_slab) {
  return FromRc(ctx, ehip_kv_scatter_f32(ctx, src_k, src_v, d_slot_mapping, t_dim, kv_heads, d,
                                         block_size, slab_blocks, k_slab, v_slab));
}

Status KvScatterBf16(ehip_ctx* ctx, const float* src_k, const float* src_v,
                     const int64_t* d_slot_mapping, int64_t t_dim, int64_t kv_heads, int64_t d,
                     int64_t block_size, int64_t slab_blocks, uint16_t* k_slab,
                     uint16_t* v_slab) {
  return FromRc(ctx, ehip_kv_scatter_bf16(ctx, src_k, src_v, d_slot_mapping, t_dim, kv_heads, d,
                                          block_size, slab_blocks, k_slab, v_slab));
}

Status KvGatherF32(ehip_ctx* ctx, const float* k_slab, const float* v_slab,
                   const int32_t* d_block_table, int64_t block_size, int64_t length,
                   int64_t kv_heads, int64_t d, int64_t slab_blocks, float* out_k,
                   float* out_v) {
  return FromRc(ctx, ehip_kv_gather_f32(ctx, k_slab, v_slab, d_block_table, block_size, length,
                                        kv_heads, d, slab_blocks, out_k, out_v));
}

float AttentionScale(int64_t head_dim) {
  return static_cast<float>(1.0 / std::sqrt(static_cast<double>(head_dim)));
}

}  // namespace ehip::host::kernels
