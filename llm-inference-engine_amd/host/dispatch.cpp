#include "dispatch.h"

#include <cstdlib>
#include <cstring>
#include <mutex>

#include "check.h"
#include "device_buffer.h"

namespace ehip::host::dispatch {
namespace {

std::mutex g_cpu_mu;
CpuKernels g_cpu;

Status CpuOnlyF32(const BlockPool& pool, const char* what) {
  if (pool.geometry().dtype == KvDtype::kFloat32) return Status::Ok();
  return Error(StatusCode::kUnimplemented,
               Format("%s: the CPU kernels read f32 slabs; this pool holds bf16", what));
}

Status Missing(const char* what) {
  return Error(StatusCode::kUnimplemented,
               Format("%s: no CPU kernel registered (dispatch::RegisterCpuKernels)", what));
}

}  // namespace

Forced ParseForced(const char* value) {
  Forced f;
  if (value == nullptr || value[0] == '\0') return f;
  f.set = true;
  if (std::strcmp(value, "hip") == 0) {
    f.device = Device::kHip;
    return f;
  }
  const bool cpu_isa = std::strcmp(value, "scalar") == 0 || std::strcmp(value, "neon") == 0 ||
                       std::strcmp(value, "avx2") == 0;
  EHIP_CHECK(cpu_isa, "ENGINE_FORCE_ISA=\"%s\" names no kernel set (scalar, neon, avx2 or hip)",
             value);
  f.device = Device::kCpu;
  return f;
}

Forced ProcessForced() {
  static const Forced forced = ParseForced(std::getenv("ENGINE_FORCE_ISA"));
  return forced;
}

Device Resolve(Forced forced, bool slabs_in_hbm) {
  const Device natural = slabs_in_hbm ? Device::kHip : Device::kCpu;
  if (!forced.set) return natural;
  EHIP_CHECK(forced.device == natural,
             "ENGINE_FORCE_ISA forces the %s kernels, which cannot read a pool whose slabs are "
             "in %s memory",
             DeviceName(forced.device).data(), slabs_in_hbm ? "device" : "host");
  return forced.device;
}

Device Select(const BlockPool& pool) { return Resolve(ProcessForced(), pool.device_resident()); }

void RegisterCpuKernels(const CpuKernels& kernels) {
  std::lock_guard<std::mutex> lock(g_cpu_mu);
  g_cpu = kernels;
}

CpuKernels RegisteredCpuKernels() {
  std::lock_guard<std::mutex> lock(g_cpu_mu);
  return g_cpu;
}

Status PagedDecodeBatched(ehip_ctx* ctx, const BlockPool& pool, int layer, const float* q,
                          const int32_t* const* block_tables, const int64_t* lengths,
                          int64_t num_seqs, int64_t heads, float scale, float* out) {
  const CacheGeometry& g = pool.geometry();
  if (Select(pool) == Device::kHip) {
    if (g.dtype == KvDtype::kBFloat16)
      return FromRc(ctx, ehip_paged_decode_attention_batched_bf16(
                             ctx, q, static_cast<const uint16_t*>(pool.k_slab(layer)),
                             static_cast<const uint16_t*>(pool.v_slab(layer)), block_tables,
                             lengths, num_seqs, heads, g.num_kv_heads, g.head_dim,
                             pool.block_size(), pool.block_stride(), pool.num_blocks(), scale,
                             out));
    return FromRc(ctx, ehip_paged_decode_attention_batched_f32(
                           ctx, q, static_cast<const float*>(pool.k_slab(layer)),
                           static_cast<const float*>(pool.v_slab(layer)), block_tables, lengths,
                           num_seqs, heads, g.num_kv_heads, g.head_dim, pool.block_size(),
                           pool.block_stride(), pool.num_blocks(), scale, out));
  }
  if (Status s = CpuOnlyF32(pool, "PagedDecodeBatched"); !s.ok()) return s;
  const CpuKernels cpu = RegisteredCpuKernels();
  if (cpu.paged_decode_batched_f32 == nullptr) return Missing("PagedDecodeBatched");
  if (num_seqs == 0) return Status::Ok();
  cpu.paged_decode_batched_f32(q, static_cast<const float*>(pool.k_slab(layer)),
                               static_cast<const float*>(pool.v_slab(layer)), block_tables,
                               lengths, num_seqs, heads, g.num_kv_heads, g.head_dim,
                               pool.block_size(), pool.block_stride(), scale, out);
  return Status::Ok();
}

Status PagedDecode(ehip_ctx* ctx, const BlockPool& pool, int layer, const float* q,
                   const int32_t* block_table, int64_t num_blocks, int64_t length, int64_t heads,
                   float scale, float* out) {
  const CacheGeometry& g = pool.geometry();
  if (Select(pool) == Device::kHip) {
    if (g.dtype != KvDtype::kFloat32)
      return Error(StatusCode::kUnimplemented,
                   "PagedDecode: the single-sequence entry point reads f32 slabs");
    return FromRc(ctx, ehip_paged_decode_attention_f32(
                           ctx, q, static_cast<const float*>(pool.k_slab(layer)),
                           static_cast<const float*>(pool.v_slab(layer)), block_table,
                           num_blocks, length, heads, g.num_kv_heads, g.head_dim,
                           pool.block_size(), pool.block_stride(), pool.num_blocks(), scale,
                           out));
  }
  if (Status s = CpuOnlyF32(pool, "PagedDecode"); !s.ok()) return s;
  const CpuKernels cpu = RegisteredCpuKernels();
  if (cpu.paged_decode_f32 == nullptr) return Missing("PagedDecode");
  cpu.paged_decode_f32(q, static_cast<const float*>(pool.k_slab(layer)),
                       static_cast<const float*>(pool.v_slab(layer)), block_table, num_blocks,
                       length, heads, g.num_kv_heads, g.head_dim, pool.block_size(),
                       pool.block_stride(), scale, out);
  return Status::Ok();
}

Status KvScatter(ehip_ctx* ctx, const BlockPool& pool, int layer, const float* src_k,
                 const float* src_v, const int64_t* slot_mapping, int64_t t_dim) {
  const CacheGeometry& g = pool.geometry();
  if (Select(pool) == Device::kHip) {
    if (g.dtype == KvDtype::kBFloat16)
      return FromRc(ctx, ehip_kv_scatter_bf16(ctx, src_k, src_v, slot_mapping, t_dim,
                                              g.num_kv_heads, g.head_dim, pool.block_size(),
                                              pool.num_blocks(),
                                              static_cast<uint16_t*>(pool.k_slab(layer)),
                                              static_cast<uint16_t*>(pool.v_slab(layer))));
    return FromRc(ctx, ehip_kv_scatter_f32(ctx, src_k, src_v, slot_mapping, t_dim,
                                           g.num_kv_heads, g.head_dim, pool.block_size(),
                                           pool.num_blocks(),
                                           static_cast<float*>(pool.k_slab(layer)),
                                           static_cast<float*>(pool.v_slab(layer))));
  }
  if (Status s = CpuOnlyF32(pool, "KvScatter"); !s.ok()) return s;
  const CpuKernels cpu = RegisteredCpuKernels();
  if (cpu.kv_scatter_f32 == nullptr) return Missing("KvScatter");
  if (t_dim == 0) return Status::Ok();
  cpu.kv_scatter_f32(src_k, src_v, slot_mapping, t_dim, g.num_kv_heads, g.head_dim,
                     pool.block_size(), static_cast<float*>(pool.k_slab(layer)),
                     static_cast<float*>(pool.v_slab(layer)));
  return Status::Ok();
}

}  // namespace ehip::host::dispatch
