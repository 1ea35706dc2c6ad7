// CPU ORACLE — TEST INFRASTRUCTURE ONLY.
//
// An extern "C" front over the reference's own kernels (compiled from the
// sources under /root/reference/src by oracle/Makefile's `ref` target) so
// that tests can pin the C restatement bit-for-bit and bench.py can time the
// reference's AVX2 path as the CPU baseline. `isa` = 0 scalar, 1 AVX2 runs the
// per-ISA unit walker serially through the reference's detail seams
// (src/kernels/internal/attention_impl.h:53-94); `isa` = -1 calls the public,
// DefaultPool-threaded entry point (ISA chosen by the reference's dispatch).
#include <cstdint>

#include "kernels/attention.h"
#include "kernels/dispatch.h"
#include "kernels/internal/attention_common.h"
#include "kernels/internal/attention_impl.h"
#include "kernels/internal/exp_common.h"
#include "kernels/internal/paged_attention_common.h"
#include "kernels/kv_gather.h"
#include "kernels/kv_scatter.h"
#include "kernels/paged_attention.h"
#include "kernels/internal/rope_impl.h"
#include "kernels/gemm.h"
#include "kernels/internal/gemm_impl.h"
#include "tensor/dtype.h"
#include "kernels/rope.h"

namespace k = engine::kernels;
namespace ki = engine::kernels::internal;

namespace {
k::Isa ToIsa(int isa) { return isa == 1 ? k::Isa::kAvx2 : k::Isa::kScalar; }
}  // namespace

extern "C" {

int ref_selected_isa() { return static_cast<int>(k::SelectedIsa()); }

float ref_exp_scalar(float x) { return ki::ExpF32Scalar(x); }

// RoPE in place (src/kernels/rope.h:34-36): isa 0 / 1 runs that ISA's row
// kernel through the detail seam, -1 the public threaded entry point.
void ref_rope_apply_f32(int isa, float* x, std::int64_t t, std::int64_t hx, std::int64_t d,
                        const std::int32_t* positions, const float* cos, const float* sin) {
  if (isa < 0) {
    k::RopeApplyF32(x, t, hx, d, positions, cos, sin);
    return;
  }
  k::detail::RopeRowsVariant(ToIsa(isa))(x, t, hx, d, positions, cos, sin);
}

void ref_paged_decode_batched_f32(int isa, const float* q, const float* k_slab,
                                  const float* v_slab,
                                  const std::int32_t* const* block_tables,
                                  const std::int64_t* lengths,
                                  std::int64_t num_seqs, std::int64_t heads,
                                  std::int64_t kv_heads, std::int64_t d,
                                  std::int64_t block_size,
                                  std::int64_t block_stride, float scale,
                                  float* out) {
  if (isa < 0) {
    k::PagedDecodeAttentionBatchedF32(q, k_slab, v_slab, block_tables, lengths,
                                      num_seqs, heads, kv_heads, d, block_size,
                                      block_stride, scale, out);
    return;
  }
  const ki::PagedDecodeBatchedArgs a{.q = q,
                                     .k_slab = k_slab,
                                     .v_slab = v_slab,
                                     .block_tables = block_tables,
                                     .lengths = lengths,
                                     .out = out,
                                     .num_seqs = num_seqs,
                                     .heads = heads,
                                     .kv_heads = kv_heads,
                                     .d = d,
                                     .group = heads / kv_heads,
                                     .block_size = block_size,
                                     .block_stride = block_stride,
                                     .scale = scale};
  k::detail::PagedDecodeBatchedUnits(
      a, k::detail::PagedDecodeAttentionVariant(ToIsa(isa)), 0,
      num_seqs * kv_heads);
}

void ref_paged_decode_f32(int isa, const float* q, const float* k_slab,
                          const float* v_slab, const std::int32_t* block_table,
                          std::int64_t num_blocks, std::int64_t length,
                          std::int64_t heads, std::int64_t kv_heads,
                          std::int64_t d, std::int64_t block_size,
                          std::int64_t block_stride, float scale, float* out) {
  if (isa < 0) {
    k::PagedDecodeAttentionF32(q, k_slab, v_slab, block_table, num_blocks,
                               length, heads, kv_heads, d, block_size,
                               block_stride, scale, out);
    return;
  }
  const ki::PagedDecodeArgs a{.q = q,
                              .k_slab = k_slab,
                              .v_slab = v_slab,
                              .block_table = block_table,
                              .out = out,
                              .d = d,
                              .length = length,
                              .group = heads / kv_heads,
                              .block_size = block_size,
                              .block_stride = block_stride,
                              .scale = scale};
  k::detail::PagedDecodeAttentionVariant(ToIsa(isa))(a, 0, kv_heads);
}

void ref_prefill_varlen_f32(int isa, const float* q,
                            const std::int32_t* cu_seqlens,
                            std::int64_t num_seqs, const float* const* k_seqs,
                            const float* const* v_seqs,
                            const std::int64_t* l_dims, float* out,
                            std::int64_t heads, std::int64_t kv_heads,
                            std::int64_t d, float scale) {
  if (isa < 0) {
    k::PrefillAttentionVarlenF32(q, cu_seqlens, num_seqs, k_seqs, v_seqs,
                                 l_dims, out, heads, kv_heads, d, scale);
    return;
  }
  std::int64_t total = 0;
  for (std::int64_t b = 0; b < num_seqs; ++b) {
    const std::int64_t t = cu_seqlens[b + 1] - cu_seqlens[b];
    total += heads * ((t + ki::kAttnQb - 1) / ki::kAttnQb);
  }
  const ki::PrefillVarlenArgs a{.q = q,
                                .cu_seqlens = cu_seqlens,
                                .k_seqs = k_seqs,
                                .v_seqs = v_seqs,
                                .l_dims = l_dims,
                                .out = out,
                                .num_seqs = num_seqs,
                                .heads = heads,
                                .d = d,
                                .group = heads / kv_heads,
                                .scale = scale};
  k::detail::PrefillVarlenUnits(
      a, k::detail::PrefillAttentionVariant(ToIsa(isa)), 0, total);
}

void ref_decode_f32(int isa, const float* q, const float* kk, const float* v,
                    float* out, std::int64_t heads, std::int64_t kv_heads,
                    std::int64_t d, std::int64_t l_dim, float scale) {
  const ki::DecodeArgs a{.q = q,
                         .k = kk,
                         .v = v,
                         .out = out,
                         .d = d,
                         .l_dim = l_dim,
                         .group = heads / kv_heads,
                         .scale = scale};
  k::detail::DecodeAttentionVariant(ToIsa(isa))(a, 0, kv_heads);
}

void ref_kv_scatter_f32(const float* src_k, const float* src_v,
                        const std::int64_t* slot_mapping, std::int64_t t_dim,
                        std::int64_t kv_heads, std::int64_t d,
                        std::int64_t block_size, float* k_slab, float* v_slab) {
  k::KvScatterF32(src_k, src_v, slot_mapping, t_dim, kv_heads, d, block_size,
                  k_slab, v_slab);
}

void ref_kv_gather_f32(const float* k_slab, const float* v_slab,
                       const std::int32_t* block_table, std::int64_t block_size,
                       std::int64_t length, std::int64_t kv_heads,
                       std::int64_t d, float* out_k, float* out_v) {
  k::KvGatherF32(k_slab, v_slab, block_table, block_size, length, kv_heads, d,
                 out_k, out_v);
}

// Packed linear layer (src/kernels/gemm.h): the panel pack, and the GEMM with
// isa 0 = the scalar tile over every row and panel (bit-identical to a naive
// ascending-k loop), 1 = the AVX2 tile, -1 = the public threaded PackedGemm.
// dtype: 0 fp32, 1 bf16, 2 fp16.
void ref_pack_weight_panels_u16(const std::uint16_t* w, std::int64_t n, std::int64_t k,
                                std::uint16_t* wp) {
  k::PackWeightPanels(w, n, k, wp);
}
void ref_pack_weight_panels_f32(const float* w, std::int64_t n, std::int64_t k, float* wp) {
  k::PackWeightPanels(w, n, k, wp);
}
void ref_packed_gemm(int isa, int dtype, const float* x, std::int64_t m, std::int64_t kk,
                     const void* wp, std::int64_t n, const float* bias, float* y) {
  namespace t = engine::tensor;
  const t::DataType dt = dtype == 0 ? t::DataType::kFloat32
                         : dtype == 1 ? t::DataType::kBFloat16 : t::DataType::kFloat16;
  if (isa < 0) {
    k::PackedGemm(x, m, kk, wp, dt, n, bias, y);
    return;
  }
  const std::int64_t panels = k::PackedPanels(n);
  const auto* w16 = static_cast<const std::uint16_t*>(wp);
  const auto* w32 = static_cast<const float*>(wp);
  if (isa == 0) {
    if (dtype == 0) k::scalar::GemmTileF32(x, kk, n, w32, bias, y, 0, m, 0, panels);
    else if (dtype == 1) k::scalar::GemmTileBf16(x, kk, n, w16, bias, y, 0, m, 0, panels);
    else k::scalar::GemmTileF16(x, kk, n, w16, bias, y, 0, m, 0, panels);
  } else {
    if (dtype == 0) k::avx2::GemmTileF32(x, kk, n, w32, bias, y, 0, m, 0, panels);
    else if (dtype == 1) k::avx2::GemmTileBf16(x, kk, n, w16, bias, y, 0, m, 0, panels);
    else k::avx2::GemmTileF16(x, kk, n, w16, bias, y, 0, m, 0, panels);
  }
}

}  // extern "C"
