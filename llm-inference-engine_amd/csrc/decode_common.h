// Split-KV bookkeeping shared by the decode kernels: partial-slot indexing and
// the log-sum-exp merge of a (row, kv head) group's split partials.
#pragma once

#include "device_util.h"
#include "kernels.h"

namespace ehip {

__device__ __forceinline__ int64_t PartialIndex(const RowDesc& rd, int kv_heads, int hk,
                                                int nsplit, int split) {
  return int64_t{rd.split_base} * kv_heads + int64_t{hk} * nsplit + split;
}

// Log-sum-exp merge of one (row, kv head) group's split partials by one
// wavefront: M = max_s m_s, L = sum_s l_s 2^(m_s - M),
// out = (sum_s o_s 2^(m_s - M)) / L. Splits are combined in split order, so
// the result is deterministic.
__device__ inline void MergeSplits(const DecodeParams& p, int row, int hk, int64_t pbase, int nsplit) {
  const int lane = threadIdx.x & 63;
  const int g = p.group, d = p.d;
  float* out = p.out + (int64_t{row} * p.heads + int64_t{hk} * g) * d;
  for (int h = 0; h < g; ++h) {
    float M = -INFINITY;
    for (int s = 0; s < nsplit; ++s) M = fmaxf(M, p.part_ml[((pbase + s) * g + h) * 2]);
    float L = 0.f;
    for (int s = 0; s < nsplit; ++s) {
      const float* ml = p.part_ml + ((pbase + s) * g + h) * 2;
      L += ml[1] * Exp2(ml[0] - M);
    }
    const float inv = 1.0f / L;
    for (int e = lane; e < d; e += 64) {
      float acc = 0.f;
      for (int s = 0; s < nsplit; ++s) {
        const float w = Exp2(p.part_ml[((pbase + s) * g + h) * 2] - M);
        acc += w * p.part_o[((pbase + s) * g + h) * d + e];
      }
      out[int64_t{h} * d + e] = acc * inv;
    }
  }
}

}  // namespace ehip
