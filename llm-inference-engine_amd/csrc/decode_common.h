// Shared by the decode kernels: work-item decoding, the range's table slice,
// partial-slot indexing and the sequential split merge.
#pragma once

#include "device_util.h"
#include "kernels.h"

namespace ehip {

// Cache policy of the K/V tile loads (buffer-load aux bits): non-temporal (nt)
// at system coherence scope (sc1). Every tile is streamed once per launch; on
// MI355X this policy raised a measured gather of the decode pattern (random
// 4 KiB (block, head) tiles) from 5.98 to 6.52 TB/s.
constexpr int kKvLoadAux = 2 | 16;

__device__ __forceinline__ int64_t PartialIndex(const RowDesc& rd, int kv_heads, int hk,
                                                int split) {
  return int64_t{rd.split_base} * kv_heads + int64_t{hk} * rd.nsplit + split;
}

// Table entry j of a key range's logical blocks lb0, lb0 + 1, ... (lb0 =
// tb / bs), called with j = lane and j = 64 + lane for the range's two
// 64-block halves (ranges are at most 128 blocks): -1 past the range, -2 for
// an id outside the slab (ReportRejectedBlocks flags those at the end of the
// item). The load is unconditional and branch-free (lanes past the range
// re-read its last entry) so it issues together with the item's other loads.
__device__ __forceinline__ int LoadRangeTable(const DecodeParams& p, int table_off, int tb,
                                              int te, int j) {
  const int lb0 = tb / p.bs;
  const int nblk = (te - 1) / p.bs - lb0 + 1;  // <= 128
  const int raw = p.table[table_off + lb0 + min(j, nblk - 1)];
  const bool bad = raw < 0 || raw >= p.slab_blocks;
  return j < nblk ? (bad ? -2 : raw) : -1;
}

// Block id bi (< 128, wavefront-uniform) of a range's slice held as two
// per-lane halves.
__device__ __forceinline__ int RangeTableId(int tab, int tab2, int bi) {
  return __builtin_amdgcn_readlane(bi < 64 ? tab : tab2, bi & 63);
}

// Work-item and row descriptors are read-only for a launch. Read through the
// constant address space at a wavefront-uniform index they become scalar
// loads (s_load, counted by lgkmcnt): they land in scalar registers and do not
// wait behind the wavefront's outstanding vector loads and stores, which a
// vector load would (vmcnt retires in issue order).
template <class R>
__device__ __forceinline__ R ScalarRead(const R* base, int i) {
#if defined(__HIP_DEVICE_COMPILE__)
  return ((const __attribute__((address_space(4))) R*)base)[i];
#else
  return base[i];  // the host pass only type-checks device code
#endif
}

__device__ __forceinline__ void ReportRejectedBlocks(const DecodeParams& p, int tab) {
  if (__any(tab == -2) && (threadIdx.x & 63) == 0) atomicOr(p.err, kErrBlockRange);
}

// A work item decoded: its rows (one, or the members of a joint group; slots
// past nrows repeat row 0), kv head, key range and split slot.
struct ItemRef {
  int rows[kMaxJointRows];
  int nrows;
  int hk;
  int split;
  int tb;
  int te;
  int table_off;
  int first[4];  // block ids of the first four 16-token halves, or -1
  bool last;     // the range ends at its row's last key
};

__device__ __forceinline__ ItemRef DecodeItem(const WorkItem& it) {
  ItemRef r;
  r.rows[0] = it.row0;
  r.rows[1] = it.row1 >= 0 ? it.row1 : it.row0;
  r.rows[2] = r.rows[3] = it.row0;
  r.nrows = it.row1 >= 0 ? 2 : 1;
  r.hk = UnpackHk(it.hk_split);
  r.split = UnpackSplit(it.hk_split);
  r.last = IsLastRange(it.hk_split);
  r.tb = it.tok_begin;
  r.te = it.tok_end;
  r.table_off = it.table_off;
  r.first[0] = it.first_block0;
  r.first[1] = it.first_block1;
  r.first[2] = it.first_block2;
  r.first[3] = it.first_block3;
  return r;
}

// Rows 3 and 4 of a joint item of a plan with groups beyond pairs (the
// kernels that serve such groups read them; p.items_x is null otherwise).
__device__ __forceinline__ void AddItemRows(const DecodeParams& p, int64_t idx, ItemRef& r) {
  if (p.items_x == nullptr) return;
  const ItemRowsX x = p.items_x[idx];
  if (x.row2 >= 0) {
    r.rows[2] = x.row2;
    r.nrows = 3;
  }
  if (x.row3 >= 0) {
    r.rows[3] = x.row3;
    r.nrows = 4;
  }
}

// Row r of an item, by selects (a dynamic index into the rows array would
// put it in scratch memory).
__device__ __forceinline__ int ItemRow(const ItemRef& it, int r) {
  return r == 0 ? it.rows[0] : r == 1 ? it.rows[1] : r == 2 ? it.rows[2] : it.rows[3];
}

// Sequential log-sum-exp merge of one (row, kv head) group's split partials
// by one wavefront (the fallback for groups too long for the parallel merge):
// M = max_s m_s, L = sum_s l_s 2^(m_s - M), out = (sum_s o_s 2^(m_s - M)) / L.
// Splits are combined in split order, so the result is deterministic.
__device__ inline void MergeSplits(const DecodeParams& p, int row, int hk, int64_t pbase,
                                   int nsplit) {
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
