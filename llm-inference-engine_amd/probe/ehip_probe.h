/*
 * ehip_probe.h — read-bandwidth probes for benchmarks (lib/libehip_probe.so).
 *
 * Measurement infrastructure only: they price the decode kernels' HBM
 * roofline on the device they run on and are not part of the attention path
 * or its C ABI (include/ehip.h). Each probe runs `reps` times on its own
 * stream on the current HIP device and writes the best rate, bytes read per
 * second in GB/s, to *gbps. Returns 0 on success, 2 for bad arguments and 11
 * for a HIP failure (the values of include/ehip.h's status codes).
 */
#ifndef EHIP_PROBE_H_
#define EHIP_PROBE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* A streaming pass over d_buf (16 <= bytes < 4 GiB, device memory); nt selects
 * the non-temporal load policy the decode kernels use. */
int ehip_probe_stream_read(const void* d_buf, int64_t bytes, int32_t nt, int32_t reps,
                           float* gbps);

/* The decode kernels' access pattern alone: each of
 * (n_blocks / tiles_per_item) * kv_heads wavefronts reads tiles_per_item
 * (block, head) tiles of tile_bytes from both slabs, at the block ids h_blocks
 * (host array, each < slab_blocks; a block is block_bytes long). */
int ehip_probe_tile_gather(const void* d_k_slab, const void* d_v_slab, int64_t slab_blocks,
                           const int32_t* h_blocks, int64_t n_blocks, int32_t tiles_per_item,
                           int32_t kv_heads, int64_t block_bytes, int32_t tile_bytes, int32_t nt,
                           int32_t reps, float* gbps);

#ifdef __cplusplus
}
#endif

#endif /* EHIP_PROBE_H_ */
