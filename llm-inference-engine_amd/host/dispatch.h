// Where the attention path's kernels run: on the CPU, through the engine's
// own kernel table (the reference's scalar / NEON / AVX2 kernels behind its
// per-process ISA selection, src/kernels/dispatch.h:24-117), or on the GPU
// through the HIP C ABI.
//
// The HIP path is not one more ISA of the CPU kernel table: it reads slabs
// in HBM and needs a device context. So the device is chosen per pool, by
// where the pool's slabs live (host memory -> CPU, HBM -> HIP), and the
// process-wide ENGINE_FORCE_ISA keeps its meaning: a CPU ISA name (scalar,
// neon, avx2) pins the CPU kernels, the extra value "hip" pins the GPU. As in
// the reference's ResolveIsa (src/kernels/dispatch.cpp:85-115), a forced
// choice that cannot run aborts instead of falling back, so a forced run never
// silently measures something else; the variable is read once per process.
#pragma once

#include <cstdint>
#include <string_view>

#include "block_pool.h"
#include "ehip.h"
#include "status.h"

namespace ehip::host::dispatch {

enum class Device : uint8_t { kCpu, kHip };

constexpr std::string_view DeviceName(Device d) { return d == Device::kHip ? "hip" : "cpu"; }

// A parsed ENGINE_FORCE_ISA: unset (nullptr or empty) leaves the choice to
// the pool; "scalar" / "neon" / "avx2" force the CPU, "hip" the GPU; any
// other value aborts.
struct Forced {
  bool set = false;
  Device device = Device::kCpu;
};
Forced ParseForced(const char* value);
// ParseForced(getenv("ENGINE_FORCE_ISA")), evaluated once per process.
Forced ProcessForced();

// The device for a pool whose slabs are (or are not) in HBM; aborts when a
// forced device cannot read them (the CPU cannot dereference HBM slabs, the
// GPU path reads only HBM).
Device Resolve(Forced forced, bool slabs_in_hbm);
Device Select(const BlockPool& pool);

// The engine's CPU kernels for this path, with the reference's signatures
// (src/kernels/paged_attention.h:50-57, :105-110; src/kernels/kv_scatter.h:47-50).
// The engine registers its own once at start-up; an entry left null makes the
// CPU route return Unimplemented.
struct CpuKernels {
  void (*paged_decode_f32)(const float* q, const float* k_slab, const float* v_slab,
                           const int32_t* block_table, int64_t num_blocks, int64_t length,
                           int64_t heads, int64_t kv_heads, int64_t d, int64_t block_size,
                           int64_t block_stride, float scale, float* out) = nullptr;
  void (*paged_decode_batched_f32)(const float* q, const float* k_slab, const float* v_slab,
                                   const int32_t* const* block_tables, const int64_t* lengths,
                                   int64_t num_seqs, int64_t heads, int64_t kv_heads, int64_t d,
                                   int64_t block_size, int64_t block_stride, float scale,
                                   float* out) = nullptr;
  void (*kv_scatter_f32)(const float* src_k, const float* src_v, const int64_t* slot_mapping,
                         int64_t t_dim, int64_t kv_heads, int64_t d, int64_t block_size,
                         float* k_slab, float* v_slab) = nullptr;
};
void RegisterCpuKernels(const CpuKernels& kernels);
CpuKernels RegisteredCpuKernels();

// The path's calls over one layer of a pool, run on Select(pool). Pointers
// (q, out, K/V rows, slots) live where that device reads them: host memory
// for the CPU, HBM for the GPU (block_tables are host pointer arrays either
// way). ctx may be null on the CPU route. bf16 slabs run on the GPU only (the
// reference pool is fp32, src/kvcache/block_pool.cpp:41-46).
Status PagedDecodeBatched(ehip_ctx* ctx, const BlockPool& pool, int layer, const float* q,
                          const int32_t* const* block_tables, const int64_t* lengths,
                          int64_t num_seqs, int64_t heads, float scale, float* out);
Status PagedDecode(ehip_ctx* ctx, const BlockPool& pool, int layer, const float* q,
                   const int32_t* block_table, int64_t num_blocks, int64_t length, int64_t heads,
                   float scale, float* out);
Status KvScatter(ehip_ctx* ctx, const BlockPool& pool, int layer, const float* src_k,
                 const float* src_v, const int64_t* slot_mapping, int64_t t_dim);

}  // namespace ehip::host::dispatch
