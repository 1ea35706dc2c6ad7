// Read-bandwidth probes that price the decode kernels' roofline on the device
// they run on: a streaming read of a buffer, and the decode access pattern
// alone (random (block, kv head) tiles of a K and a V slab, no arithmetic).
// Measurement infrastructure for benchmarks (lib/libehip_probe.so), built
// apart from the attention library; the C entry points are in ehip_probe.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "ehip_probe.h"

namespace {

// The load policy the decode kernels use for K/V tiles (buffer-load aux
// bits): non-temporal at system coherence scope.
constexpr int kNtAux = 2 | 16;

// Grid-stride 16-byte reads of a buffer below 4 GiB; the xor keeps the
// loads live.
template <int AUX>
__global__ __launch_bounds__(256) void StreamRead(const uint4* __restrict__ p, uint32_t n,
                                                 uint32_t* __restrict__ sink) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint4*>(p), 0, n * 16u, 0x00020000);
  uint32_t acc = 0;
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint4 v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, i * 16u, 0, AUX));
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;  // practically never; keeps the loads
}

// One wavefront per item: `tiles` consecutive entries of the permuted block
// list, each read as the (block, head) tile of K and of V.
template <int AUX>
__global__ __launch_bounds__(64) void TileGather(const uint8_t* __restrict__ k,
                                                const uint8_t* __restrict__ v,
                                                const int32_t* __restrict__ blocks, int32_t n_items,
                                                int32_t tiles, int32_t kv_heads, int64_t block_bytes,
                                                int32_t tile_bytes, uint32_t* __restrict__ sink) {
  const int item = blockIdx.x;
  if (item >= n_items) return;
  const int lane = threadIdx.x;
  const int head = item % kv_heads;
  uint32_t acc = 0;
  for (int t = 0; t < tiles; ++t) {
    const int32_t b = blocks[(item / kv_heads) * tiles + t];
    const int64_t off = int64_t{b} * block_bytes + int64_t{head} * tile_bytes;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(k + off), 0, static_cast<uint32_t>(tile_bytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(v + off), 0, static_cast<uint32_t>(tile_bytes), 0x00020000);
    for (int o = lane * 16; o < tile_bytes; o += 64 * 16) {
      const uint4 x = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, o, 0, AUX));
      const uint4 y = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, o, 0, AUX));
      acc ^= x.x ^ x.y ^ x.z ^ x.w ^ y.x ^ y.y ^ y.z ^ y.w;
    }
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

// Scratch a probe owns for one call: a stream, two events and a sink word.
struct ProbeRun {
  hipStream_t stream = nullptr;
  hipEvent_t a = nullptr, b = nullptr;
  uint32_t* sink = nullptr;
  hipError_t e = hipSuccess;

  ProbeRun() {
    e = hipStreamCreateWithFlags(&stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&b);
    if (e == hipSuccess) e = hipMalloc(&sink, 256);
  }
  ~ProbeRun() {
    if (stream) (void)hipStreamSynchronize(stream);
    if (sink) (void)hipFree(sink);
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    if (stream) (void)hipStreamDestroy(stream);
  }

  // Best-of-reps rate of `launch` over `bytes` bytes.
  template <class F>
  int Time(double bytes, int32_t reps, F launch, float* gbps) {
    float best = 0.f;
    for (int r = 0; e == hipSuccess && r < reps; ++r) {
      e = hipEventRecord(a, stream);
      if (e == hipSuccess) {
        launch();
        e = hipGetLastError();
      }
      if (e == hipSuccess) e = hipEventRecord(b, stream);
      if (e == hipSuccess) e = hipEventSynchronize(b);
      float ms = 0.f;
      if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
      if (e == hipSuccess && ms > 0.f) best = std::max(best, static_cast<float>(bytes / ms / 1e6));
    }
    if (e != hipSuccess) return 11;
    *gbps = best;
    return 0;
  }
};

}  // namespace

extern "C" int ehip_probe_stream_read(const void* d_buf, int64_t bytes, int32_t nt, int32_t reps,
                                      float* gbps) {
  if (!d_buf || !gbps || reps < 1 || bytes < 16 || bytes >= (int64_t{1} << 32)) return 2;
  ProbeRun run;
  if (run.e != hipSuccess) return 11;
  const uint32_t n = static_cast<uint32_t>(bytes / 16);
  const dim3 grid(8192), block(256);
  return run.Time(static_cast<double>(n) * 16.0, reps, [&] {
    if (nt)
      hipLaunchKernelGGL(StreamRead<kNtAux>, grid, block, 0, run.stream,
                         static_cast<const uint4*>(d_buf), n, run.sink);
    else
      hipLaunchKernelGGL(StreamRead<0>, grid, block, 0, run.stream,
                         static_cast<const uint4*>(d_buf), n, run.sink);
  }, gbps);
}

extern "C" int ehip_probe_tile_gather(const void* d_k_slab, const void* d_v_slab,
                                      int64_t slab_blocks, const int32_t* h_blocks,
                                      int64_t n_blocks, int32_t tiles_per_item, int32_t kv_heads,
                                      int64_t block_bytes, int32_t tile_bytes, int32_t nt,
                                      int32_t reps, float* gbps) {
  if (!d_k_slab || !d_v_slab || !h_blocks || !gbps || reps < 1 || tiles_per_item < 1 ||
      kv_heads < 1 || tile_bytes < 16 || tile_bytes % 16 != 0 ||
      int64_t{tile_bytes} * kv_heads > block_bytes || n_blocks < tiles_per_item ||
      n_blocks / tiles_per_item * kv_heads > INT32_MAX)
    return 2;
  for (int64_t i = 0; i < n_blocks; ++i)
    if (h_blocks[i] < 0 || h_blocks[i] >= slab_blocks) return 2;
  ProbeRun run;
  if (run.e != hipSuccess) return 11;
  const int32_t items = static_cast<int32_t>(n_blocks / tiles_per_item * kv_heads);
  int32_t* d_blocks = nullptr;
  if (hipMalloc(&d_blocks, static_cast<size_t>(n_blocks) * 4) != hipSuccess) return 11;
  run.e = hipMemcpyAsync(d_blocks, h_blocks, static_cast<size_t>(n_blocks) * 4,
                         hipMemcpyHostToDevice, run.stream);
  const double bytes = 2.0 * items * tiles_per_item * tile_bytes;
  const auto* k = static_cast<const uint8_t*>(d_k_slab);
  const auto* v = static_cast<const uint8_t*>(d_v_slab);
  const int rc = run.Time(bytes, reps, [&] {
    if (nt)
      hipLaunchKernelGGL(TileGather<kNtAux>, dim3(items), dim3(64), 0, run.stream, k, v,
                         d_blocks, items, tiles_per_item, kv_heads, block_bytes, tile_bytes,
                         run.sink);
    else
      hipLaunchKernelGGL(TileGather<0>, dim3(items), dim3(64), 0, run.stream, k, v, d_blocks,
                         items, tiles_per_item, kv_heads, block_bytes, tile_bytes, run.sink);
  }, gbps);
  (void)hipStreamSynchronize(run.stream);
  (void)hipFree(d_blocks);
  return rc;
}
