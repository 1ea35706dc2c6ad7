// The reference's kernel entry points (src/kernels/paged_attention.h:50-57,
// :105-110; kv_scatter.h:47-50; kv_gather.h:55-58) over device pointers, with
// the C ABI's return codes turned into Status. Arguments keep the reference's
// names and meaning; the additions are the context (stream + workspace),
// slab_blocks (the slab's block count, against which every block id and slot
// is checked on the device) and the bf16 slab variants.
#pragma once

#include <cstdint>

#include "ehip.h"
#include "status.h"

namespace ehip::host::kernels {

Status PagedDecodeAttentionF32(ehip_ctx* ctx, const float* q, const float* k_slab,
                               const float* v_slab, const int32_t* d_block_table,
                               int64_t num_blocks, int64_t length, int64_t heads,
                               int64_t kv_heads, int64_t d, int64_t block_size,
                               int64_t block_stride, int64_t slab_blocks, float scale, float* out);

// block_tables: host array of B host pointers (each sequence's ids).
Status PagedDecodeAttentionBatchedF32(ehip_ctx* ctx, const float* q, const float* k_slab,
                                      const float* v_slab, const int32_t* const* block_tables,
                                      const int64_t* lengths, int64_t num_seqs, int64_t heads,
                                      int64_t kv_heads, int64_t d, int64_t block_size,
                                      int64_t block_stride, int64_t slab_blocks, float scale,
                                      float* out);
Status PagedDecodeAttentionBatchedBf16(ehip_ctx* ctx, const float* q, const uint16_t* k_slab,
                                       const uint16_t* v_slab,
                                       const int32_t* const* block_tables,
                                       const int64_t* lengths, int64_t num_seqs, int64_t heads,
                                       int64_t kv_heads, int64_t d, int64_t block_size,
                                       int64_t block_stride, int64_t slab_blocks, float scale,
                                       float* out);

Status KvScatterF32(ehip_ctx* ctx, const float* src_k, const float* src_v,
                    const int64_t* d_slot_mapping, int64_t t_dim, int64_t kv_heads, int64_t d,
                    int64_t block_size, int64_t slab_blocks, float* k_slab, float* v_slab);
Status KvScatterBf16(ehip_ctx* ctx, const float* src_k, const float* src_v,
                     const int64_t* d_slot_mapping, int64_t t_dim, int64_t kv_heads, int64_t d,
                     int64_t block_size, int64_t slab_blocks, uint16_t* k_slab, uint16_t* v_slab);

Status KvGatherF32(ehip_ctx* ctx, const float* k_slab, const float* v_slab,
                   const int32_t* d_block_table, int64_t block_size, int64_t length,
                   int64_t kv_heads, int64_t d, int64_t slab_blocks, float* out_k, float* out_v);

// scale = (float)(1 / sqrt((double)d)), as the reference computes it
// (src/model/optimized_model.cpp:473-474).
float AttentionScale(int64_t head_dim);

}  // namespace ehip::host::kernels
