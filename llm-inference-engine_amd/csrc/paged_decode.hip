// Ragged paged decode attention for gfx950 (VALU path), and the split merge.
//
// Semantics: kernels::PagedDecodeAttention{,Batched}F32
// (src/kernels/paged_attention.h:50-57, :105-110): for a query row attending
// keys [0, L-1], out[h] = softmax(scale * q_h . K^T) V with K/V read through
// the block table, query head h reading kv head h / g. The reference runs the
// online recurrence of src/kernels/internal/paged_attention_common.h:69-136
// per (sequence, kv head); here one wavefront handles one (row, kv head, key
// range) work item and the ranges are merged by log-sum-exp rescaling.
//
// Wavefront layout (specialised kernel): LPT lanes hold one token's head_dim
// row, each lane E elements in 16-byte vectors, so each load instruction reads
// whole 128/256-byte row segments. TPR = 64/LPT tokens are processed per
// "row" of the wavefront and 32 tokens per tile. The g query heads of the kv
// head live in registers (fp32), so every K/V byte is read from HBM once for
// all g heads. A joint work item (two rows sharing the range's blocks) is
// processed one row after the other here; the MFMA kernel serves both rows
// from one pass.
//
// Softmax: scores are formed as dot * scale * log2(e) and exponentiated with
// the hardware exp2; the running max/sum are per 32-key tile, so alpha
// rescaling happens once per tile.
#include <cstdlib>
#include <cstring>

#include "decode_common.h"
#include "device_util.h"
#include "kernels.h"

namespace ehip {
namespace {

constexpr int kWavesPerBlock = 4;
// Steps with at most this many (row, kv head) units take the workgroup-per-unit
// kernel (4 or 8 wavefronts each, 2048 wavefronts at most).
constexpr int64_t kWgMaxUnits = 256;
// ... and only when no row needs more than this many 32-key tiles per
// wavefront: past that, the split-KV path (more wavefronts on a long row,
// merged by a second kernel) measured faster (C2: rows up to 2049 keys,
// 32.6 against 39.0 us per layer; C1: one 513-key row, 17.3 against 22.0 us).
constexpr int kWgMaxTilesPerWave = 6;

template <class KV>
struct KvT;
template <>
struct KvT<float> {
  static constexpr int EPV = 4;  // elements per 16-byte vector
};
template <>
struct KvT<uint16_t> {
  static constexpr int EPV = 8;
};

template <class KV>
__device__ __forceinline__ void Widen(const uint4 r, float* o);
template <>
__device__ __forceinline__ void Widen<float>(const uint4 r, float* o) {
  o[0] = __uint_as_float(r.x);
  o[1] = __uint_as_float(r.y);
  o[2] = __uint_as_float(r.z);
  o[3] = __uint_as_float(r.w);
}
template <>
__device__ __forceinline__ void Widen<uint16_t>(const uint4 r, float* o) {
  o[0] = Bf16Lo(r.x);
  o[1] = Bf16Hi(r.x);
  o[2] = Bf16Lo(r.y);
  o[3] = Bf16Hi(r.y);
  o[4] = Bf16Lo(r.z);
  o[5] = Bf16Hi(r.z);
  o[6] = Bf16Lo(r.w);
  o[7] = Bf16Hi(r.w);
}

__device__ __forceinline__ float KvAt(const float* p, int64_t i) { return p[i]; }
__device__ __forceinline__ float KvAt(const uint16_t* p, int64_t i) {
  return __uint_as_float(uint32_t{p[i]} << 16);
}

// ----------------------------------------------------------------------------
// Specialised kernel body: KV in {f32, bf16}, D in {64, 128}, G = g exactly.
template <class KV, int D, int G>
__device__ __forceinline__ void DecodeValuRow(const DecodeParams& p, int row, int hk, int tb,
                                              int te, int split, int table_off,
                                              float* lds_o = nullptr, float* lds_ml = nullptr) {
  constexpr int EPV = KvT<KV>::EPV;
  constexpr int LPT = (G * D / 8 > 64) ? 16 : 8;  // lanes per token row
  constexpr int E = D / LPT;                      // elements per lane
  constexpr int NV = E / EPV;                     // 16-byte vectors per lane
  constexpr int TPR = 64 / LPT;                   // tokens per wavefront row
  constexpr int ROWS = 32 / TPR;                  // rows per 32-token tile
  constexpr int VSPAN = D / NV;                   // elements spanned by one vector index
  static_assert(NV >= 1 && NV * EPV == E && E * LPT == D, "layout");

  const int lane = threadIdx.x & 63;
  const RowDesc rd = p.rows[row];
  const int tl = lane / LPT;
  const int sub = lane % LPT;
  const int bs = p.bs;

  float q[G][E];
  {
    const float* qp = p.q + (int64_t{row} * p.heads + int64_t{hk} * G) * D + sub * EPV;
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int c = 0; c < EPV; c += 4) {
          const float4 x = *reinterpret_cast<const float4*>(qp + h * D + v * VSPAN + c);
          q[h][v * EPV + c + 0] = x.x;
          q[h][v * EPV + c + 1] = x.y;
          q[h][v * EPV + c + 2] = x.z;
          q[h][v * EPV + c + 3] = x.w;
        }
  }

  const int lb0 = tb / bs;
  const int tab = LoadRangeTable(p, table_off, tb, te, lane);
  const int tab2 = LoadRangeTable(p, table_off, tb, te, 64 + lane);
  const KV* kbase = static_cast<const KV*>(p.k_slab) + int64_t{hk} * p.head_stride;
  const KV* vbase = static_cast<const KV*>(p.v_slab) + int64_t{hk} * p.head_stride;
  const int lane_off = (tl * D + sub * EPV) * static_cast<int>(sizeof(KV));

  float m[G], l[G], o[G][E];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) o[h][e] = 0.f;
  }

  // K/V of one 32-token tile; two of them ping-pong so the next tile's loads
  // are in flight while the current one is computed.
  struct VTile {
    uint4 k[ROWS][NV], v[ROWS][NV];
    int phys[ROWS];
  };
  auto load = [&](VTile& t, int t0) {
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      // One buffer descriptor per wavefront row of TPR tokens (they lie in
      // one block): it starts at the row group's first token and covers
      // only tokens inside the range, so tokens past the range end read as
      // zeros and a row group past the end (or on a rejected block id) reads
      // nothing at all. Loads are non-temporal: every tile streams once.
      const int j0 = t0 + r * TPR;  // wavefront-uniform
      const int ph = RangeTableId(tab, tab2, min(j0, te - 1) / bs - lb0);
      const bool ok = j0 < te && ph >= 0;
      t.phys[r] = ok ? ph : -1;
      const int64_t off = int64_t{ok ? ph : 0} * p.block_stride + int64_t{j0 & (bs - 1)} * D;
      const uint32_t range =
          ok ? static_cast<uint32_t>(min(TPR, te - j0) * D * static_cast<int>(sizeof(KV))) : 0u;
      const __amdgpu_buffer_rsrc_t rk =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<KV*>(kbase + off), 0, range, 0x00020000);
      const __amdgpu_buffer_rsrc_t rv =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<KV*>(vbase + off), 0, range, 0x00020000);
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const int vo = lane_off + v * VSPAN * static_cast<int>(sizeof(KV));
        t.k[r][v] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, vo, 0, kKvLoadAux));
        t.v[r][v] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, vo, 0, kKvLoadAux));
      }
    }
  };
  auto compute = [&](const VTile& t, int t0) {
    const bool partial = t0 + 32 > te;

    float s[ROWS][G];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      float kf[E];
#pragma unroll
      for (int v = 0; v < NV; ++v) Widen<KV>(t.k[r][v], kf + v * EPV);
      const bool valid = t.phys[r] >= 0 && (!partial || t0 + r * TPR + tl < te);
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) acc = fmaf(q[h][e], kf[e], acc);
        acc = SumGroup<LPT>(acc);
        s[r][h] = valid ? acc * p.scale_log2 : -INFINITY;
      }
    }

#pragma unroll
    for (int h = 0; h < G; ++h) {
      float mx = s[0][h];
#pragma unroll
      for (int r = 1; r < ROWS; ++r) mx = fmaxf(mx, s[r][h]);
      mx = MaxAcross<LPT>(mx);
      const float mn = fmaxf(m[h], mx);
      // A tile whose every key sits in a rejected block leaves mn at -inf;
      // keep alpha finite (and the state untouched) in that case.
      const float alpha = mn == -INFINITY ? 1.f : Exp2(m[h] - mn);
      m[h] = mn;
      float psum = 0.f;
#pragma unroll
      for (int r = 0; r < ROWS; ++r) {
        s[r][h] = mn == -INFINITY ? 0.f : Exp2(s[r][h] - mn);
        psum += s[r][h];
      }
      l[h] = l[h] * alpha + psum;
#pragma unroll
      for (int e = 0; e < E; ++e) o[h][e] *= alpha;
    }

#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      float vf[E];  // rows past the range end were read as zeros
#pragma unroll
      for (int v = 0; v < NV; ++v) Widen<KV>(t.v[r][v], vf + v * EPV);
#pragma unroll
      for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < E; ++e) o[h][e] = fmaf(s[r][h], vf[e], o[h][e]);
    }
  };
  // Double-buffered unless the shape's registers would spill (fp32, d = 128,
  // g >= 7 keeps one tile in flight at a time).
  constexpr bool kDouble = !(sizeof(KV) == 4 && D == 128 && G >= 7);
  VTile bufA;
  if constexpr (kDouble) {
    VTile bufB;
    load(bufA, tb);
    // A work item's range is never empty; loads past its end are empty.
    for (int t0 = tb;; t0 += 64) {
      load(bufB, t0 + 32);
      compute(bufA, t0);
      if (t0 + 32 >= te) break;
      load(bufA, t0 + 64);
      compute(bufB, t0 + 32);
      if (t0 + 64 >= te) break;
    }
  } else {
    for (int t0 = tb; t0 < te; t0 += 32) {
      load(bufA, t0);
      compute(bufA, t0);
    }
  }

  ReportRejectedBlocks(p, tab);
  ReportRejectedBlocks(p, tab2);
#pragma unroll
  for (int h = 0; h < G; ++h) {
    l[h] = SumAcross<LPT>(l[h]);
#pragma unroll
    for (int e = 0; e < E; ++e) o[h][e] = SumAcross<LPT>(o[h][e]);
  }

  if (lds_o) {  // a wavefront's share of a workgroup-wide range: unnormalised (o, m, l)
    if (tl == 0) {
      float* po = lds_o + sub * EPV;
#pragma unroll
      for (int h = 0; h < G; ++h)
#pragma unroll
        for (int v = 0; v < NV; ++v)
#pragma unroll
          for (int c = 0; c < EPV; ++c) po[h * D + v * VSPAN + c] = o[h][v * EPV + c];
    }
    if (lane == 0) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        lds_ml[h * 2 + 0] = m[h];
        lds_ml[h * 2 + 1] = l[h];
      }
    }
    return;
  }
  if (rd.nsplit == 1) {
    if (tl == 0) {
      float* op = p.out + (int64_t{row} * p.heads + int64_t{hk} * G) * D + sub * EPV;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float inv = 1.0f / l[h];
#pragma unroll
        for (int v = 0; v < NV; ++v)
#pragma unroll
          for (int c = 0; c < EPV; c += 4) {
            float4 x;
            x.x = o[h][v * EPV + c + 0] * inv;
            x.y = o[h][v * EPV + c + 1] * inv;
            x.z = o[h][v * EPV + c + 2] * inv;
            x.w = o[h][v * EPV + c + 3] * inv;
            *reinterpret_cast<float4*>(op + h * D + v * VSPAN + c) = x;
          }
      }
    }
    return;
  }

  const int64_t pidx = PartialIndex(rd, p.kv_heads, hk, split);
  if (tl == 0) {
    float* po = p.part_o + pidx * G * D + sub * EPV;
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int c = 0; c < EPV; c += 4) {
          float4 x;
          x.x = o[h][v * EPV + c + 0];
          x.y = o[h][v * EPV + c + 1];
          x.z = o[h][v * EPV + c + 2];
          x.w = o[h][v * EPV + c + 3];
          *reinterpret_cast<float4*>(po + h * D + v * VSPAN + c) = x;
        }
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      p.part_ml[(pidx * G + h) * 2 + 0] = m[h];
      p.part_ml[(pidx * G + h) * 2 + 1] = l[h];
    }
  }
}

template <class KV, int D, int G>
__global__ __launch_bounds__(kWavesPerBlock * 64) void DecodeValu(DecodeParams p) {
  // Wavefront-uniform (readfirstlane): the item and everything derived from
  // it live in scalar registers, so the K/V buffer descriptors are uniform.
  const int item_idx =
      blockIdx.x * kWavesPerBlock + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (item_idx >= p.n_items) return;
  ItemRef it = DecodeItem(p.items[item_idx]);
  AddItemRows(p, item_idx, it);
  for (int r = 0; r < it.nrows; ++r)
    DecodeValuRow<KV, D, G>(p, ItemRow(it, r), it.hk, it.tb, it.te, it.split, it.table_off);
}

// ----------------------------------------------------------------------------
// Small steps (few (row, kv head) units, as in single-sequence and 32-row fp32
// decode): one workgroup of NW wavefronts per unit. Each wavefront takes an
// equal run of whole 32-key tiles of the row and leaves its unnormalised
// (o, m, l) in LDS; after a barrier the workgroup merges them (the split
// merge's log-sum-exp, in wavefront order) and writes the row's output. One
// launch, no global partials and no merge kernel, and NW times the bytes in
// flight per row of the one-item-per-wavefront kernel.
template <class KV, int D, int G, int NW>
__global__ __launch_bounds__(NW * 64) void DecodeValuWg(DecodeParams p) {
  __shared__ float lds_o[NW * G * D];
  __shared__ float lds_ml[NW * G * 2];
  const int unit = blockIdx.x;
  const int row = unit / p.kv_heads;
  const int hk = unit - row * p.kv_heads;
  const RowDesc rd = p.rows[row];
  const int len = rd.length;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tiles = (len + 31) / 32;
  const int tb = (tiles * w) / NW * 32;
  const int te = min(len, (tiles * (w + 1)) / NW * 32);
  if (tb < te) {
    DecodeValuRow<KV, D, G>(p, row, hk, tb, te, 0, rd.table_off, lds_o + w * G * D,
                            lds_ml + w * G * 2);
  } else {
    const int lane = threadIdx.x & 63;
    for (int j = lane; j < G * D; j += 64) lds_o[w * G * D + j] = 0.f;
    if (lane < G) {
      lds_ml[(w * G + lane) * 2 + 0] = -INFINITY;
      lds_ml[(w * G + lane) * 2 + 1] = 0.f;
    }
  }
  __syncthreads();
  float* out = p.out + (int64_t{row} * p.heads + int64_t{hk} * G) * D;
  for (int j = threadIdx.x; j < G * D; j += NW * 64) {
    const int h = j / D;
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < NW; ++u) mx = fmaxf(mx, lds_ml[(u * G + h) * 2]);
    float lsum = 0.f, acc = 0.f;
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      const float mu = lds_ml[(u * G + h) * 2];
      const float wt = mu == -INFINITY ? 0.f : Exp2(mu - mx);
      lsum += lds_ml[(u * G + h) * 2 + 1] * wt;
      acc += wt * lds_o[u * G * D + j];
    }
    out[j] = acc * (1.0f / lsum);
  }
}

// ----------------------------------------------------------------------------
// Generic kernel: any d <= 256, any g (heads processed in chunks of 8, one
// pass over the range's keys per chunk). Lanes own head_dim elements
// e = lane + 64k; every key is one wavefront-wide dot product. Used for the
// shapes the specialised kernels do not cover.
template <class KV>
__device__ void DecodeGenericRow(const DecodeParams& p, int row, int hk, int tb, int te,
                                 int split) {
  constexpr int HC = 8;
  const int lane = threadIdx.x & 63;
  const RowDesc rd = p.rows[row];
  const int g = p.group, d = p.d, bs = p.bs;
  const KV* kslab = static_cast<const KV*>(p.k_slab) + int64_t{hk} * p.head_stride;
  const KV* vslab = static_cast<const KV*>(p.v_slab) + int64_t{hk} * p.head_stride;
  const int64_t pidx = PartialIndex(rd, p.kv_heads, hk, split);

  for (int h0 = 0; h0 < g; h0 += HC) {
    const int hc = min(HC, g - h0);
    float q[HC][4], o[HC][4], m[HC], l[HC];
    for (int h = 0; h < HC; ++h) {
      m[h] = -INFINITY;
      l[h] = 0.f;
      for (int k = 0; k < 4; ++k) {
        const int e = lane + 64 * k;
        q[h][k] = (h < hc && e < d)
                      ? p.q[(int64_t{row} * p.heads + int64_t{hk} * g + h0 + h) * d + e]
                      : 0.f;
        o[h][k] = 0.f;
      }
    }
    for (int j = tb; j < te; ++j) {
      const int phys = p.table[rd.table_off + j / bs];
      if (phys < 0 || phys >= p.slab_blocks) {
        if (lane == 0) atomicOr(p.err, kErrBlockRange);
        continue;
      }
      const int64_t off = int64_t{phys} * p.block_stride + int64_t{j % bs} * d;
      float kv[4], vv[4];
      for (int k = 0; k < 4; ++k) {
        const int e = lane + 64 * k;
        kv[k] = e < d ? KvAt(kslab, off + e) : 0.f;
        vv[k] = e < d ? KvAt(vslab, off + e) : 0.f;
      }
      for (int h = 0; h < HC; ++h) {
        if (h >= hc) break;
        float acc = 0.f;
        for (int k = 0; k < 4; ++k) acc = fmaf(q[h][k], kv[k], acc);
        const float s = WaveSum(acc) * p.scale_log2;
        const float mn = fmaxf(m[h], s);
        const float alpha = Exp2(m[h] - mn);
        const float pr = Exp2(s - mn);
        m[h] = mn;
        l[h] = l[h] * alpha + pr;
        for (int k = 0; k < 4; ++k) o[h][k] = fmaf(pr, vv[k], o[h][k] * alpha);
      }
    }
    for (int h = 0; h < hc; ++h) {
      if (rd.nsplit == 1) {
        const float inv = 1.0f / l[h];
        for (int k = 0; k < 4; ++k) {
          const int e = lane + 64 * k;
          if (e < d)
            p.out[(int64_t{row} * p.heads + int64_t{hk} * g + h0 + h) * d + e] = o[h][k] * inv;
        }
      } else {
        for (int k = 0; k < 4; ++k) {
          const int e = lane + 64 * k;
          if (e < d) p.part_o[(pidx * g + h0 + h) * d + e] = o[h][k];
        }
        if (lane == 0) {
          p.part_ml[(pidx * g + h0 + h) * 2 + 0] = m[h];
          p.part_ml[(pidx * g + h0 + h) * 2 + 1] = l[h];
        }
      }
    }
  }
}

template <class KV>
__global__ __launch_bounds__(kWavesPerBlock * 64) void DecodeGeneric(DecodeParams p) {
  // Wavefront-uniform (readfirstlane): the item and everything derived from
  // it live in scalar registers, so the K/V buffer descriptors are uniform.
  const int item_idx =
      blockIdx.x * kWavesPerBlock + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (item_idx >= p.n_items) return;
  ItemRef it = DecodeItem(p.items[item_idx]);
  AddItemRows(p, item_idx, it);
  for (int r = 0; r < it.nrows; ++r)
    DecodeGenericRow<KV>(p, ItemRow(it, r), it.hk, it.tb, it.te, it.split);
}

// ----------------------------------------------------------------------------
// Split merge. A (row, kv head) group with more than one split is merged by
// ceil(g*d / (256*EPT)) workgroups of 256 threads, EPT consecutive output
// elements of one head per thread (EPT = 4, 16-byte loads and stores, when d
// and the output allow it): the group's (max, sum) pairs are read into LDS in
// one parallel sweep, the g per-head weights 2^(m_s - M) / L are formed there,
// and each thread then sums its elements' split partials with independent
// loads, so a group costs a few memory round trips whatever its split count.
constexpr int kMergeThreads = 256;
constexpr int kMergeMaxPairs = 2048;  // nsplit * g held in LDS (16 KiB)

template <int EPT>
struct MergeVec;
template <>
struct MergeVec<1> {
  using T = float;
  __device__ static float Fma(float w, float x, float acc) { return fmaf(w, x, acc); }
};
template <>
struct MergeVec<4> {
  using T = float4;
  __device__ static float4 Fma(float w, float4 x, float4 acc) {
    return make_float4(fmaf(w, x.x, acc.x), fmaf(w, x.y, acc.y), fmaf(w, x.z, acc.z),
                       fmaf(w, x.w, acc.w));
  }
};

template <int EPT>
__global__ __launch_bounds__(kMergeThreads) void MergeSplitsKernel(DecodeParams p, int chunks) {
  using V = typename MergeVec<EPT>::T;
  __shared__ float2 ml[kMergeMaxPairs];
  const int64_t grp = blockIdx.x / chunks;
  const int chunk = static_cast<int>(blockIdx.x - grp * chunks);
  const int mi = static_cast<int>(grp / p.kv_heads);
  const int hk = static_cast<int>(grp - int64_t{mi} * p.kv_heads);
  const int row = p.merge_rows[mi];
  const RowDesc rd = p.rows[row];
  const int nsplit = rd.nsplit;
  if (nsplit <= 1) return;  // merge_rows holds split rows only
  const int64_t pbase = PartialIndex(rd, p.kv_heads, hk, 0);
  const int g = p.group, d = p.d;
  const int npairs = nsplit * g;
  const int tid = threadIdx.x;
  if (npairs > kMergeMaxPairs) {  // very long rows: one wavefront, sequential merge
    if (chunk == 0 && tid < 64) MergeSplits(p, row, hk, pbase, nsplit);
    return;
  }
  const int gd = g * d;
  const int j = (chunk * kMergeThreads + tid) * EPT;  // first element; d % EPT == 0
  const bool has = j < gd;
  const int h = has ? j / d : 0;
  const int gdv = gd / EPT;
  const V* po = reinterpret_cast<const V*>(p.part_o + pbase * gd + (has ? j : 0));
  // The partial outputs do not depend on the weights: the first kMergeBatch
  // of them are loaded together with the (max, sum) pairs.
  constexpr int kMergeBatch = 16;
  V ov[kMergeBatch];
#pragma unroll
  for (int s = 0; s < kMergeBatch; ++s)
    if (s < nsplit) ov[s] = po[int64_t{s} * gdv];
  const float2* src = reinterpret_cast<const float2*>(p.part_ml) + pbase * g;
  for (int i = tid; i < npairs; i += kMergeThreads) ml[i] = src[i];
  __syncthreads();
  if (tid < g) {
    float M = -INFINITY;
    for (int s = 0; s < nsplit; ++s) M = fmaxf(M, ml[s * g + tid].x);
    float L = 0.f;
    for (int s = 0; s < nsplit; ++s) L += ml[s * g + tid].y * Exp2(ml[s * g + tid].x - M);
    const float inv = 1.0f / L;
    for (int s = 0; s < nsplit; ++s) ml[s * g + tid].x = Exp2(ml[s * g + tid].x - M) * inv;
  }
  __syncthreads();
  if (!has) return;
  V acc{};
#pragma unroll
  for (int s = 0; s < kMergeBatch; ++s)
    if (s < nsplit) acc = MergeVec<EPT>::Fma(ml[s * g + h].x, ov[s], acc);
#pragma unroll 8
  for (int s = kMergeBatch; s < nsplit; ++s)
    acc = MergeVec<EPT>::Fma(ml[s * g + h].x, po[int64_t{s} * gdv], acc);
  *reinterpret_cast<V*>(p.out + (int64_t{row} * p.heads + int64_t{hk} * g) * d + j) = acc;
}

template <class KV>
hipError_t LaunchTyped(const DecodeParams& p, hipStream_t stream) {
  const dim3 grid((p.n_items + kWavesPerBlock - 1) / kWavesPerBlock);
  const dim3 block(kWavesPerBlock * 64);
  constexpr int EPV = KvT<KV>::EPV;
  const bool aligned = (reinterpret_cast<uintptr_t>(p.k_slab) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.v_slab) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.q) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.out) % 16 == 0) &&
                       (p.block_stride % EPV == 0);
#define EHIP_DECODE_CASE(DD, GG)                                              \
  if (p.d == DD && p.group == GG) {                                           \
    hipLaunchKernelGGL((DecodeValu<KV, DD, GG>), grid, block, 0, stream, p); \
    return hipGetLastError();                                                 \
  }
  if (aligned) {
    EHIP_DECODE_CASE(64, 1)
    EHIP_DECODE_CASE(64, 2)
    EHIP_DECODE_CASE(64, 4)
    EHIP_DECODE_CASE(64, 7)
    EHIP_DECODE_CASE(64, 8)
    EHIP_DECODE_CASE(128, 1)
    EHIP_DECODE_CASE(128, 2)
    EHIP_DECODE_CASE(128, 4)
    EHIP_DECODE_CASE(128, 7)
    EHIP_DECODE_CASE(128, 8)
  }
#undef EHIP_DECODE_CASE
  hipLaunchKernelGGL((DecodeGeneric<KV>), grid, block, 0, stream, p);
  return hipGetLastError();
}

// Workgroup-per-unit decode for small fp32 steps; false when it does not
// apply (too many units, a row longer than NW wavefronts' table slices, or a
// shape without a specialised kernel). Tuning::decode_wg = false turns it off.
bool LaunchSmallStep(const DecodeParams& p, const Tuning& tune, hipStream_t stream,
                     hipError_t* err) {
  if (!tune.decode_wg) return false;
  const int64_t units = int64_t{p.n_rows} * p.kv_heads;
  if (units < 1 || units > kWgMaxUnits) return false;
  const bool aligned = (reinterpret_cast<uintptr_t>(p.k_slab) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.v_slab) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.q) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.out) % 16 == 0) &&
                       (p.block_stride % 4 == 0);
  if (!aligned) return false;
  const dim3 grid(static_cast<uint32_t>(units));
  // A wavefront's run (at most len / NW + 32 keys, starting on a 32-key
  // boundary) must fit its 64-entry table slice.
#define EHIP_WG_CASE(DD, GG, NW)                                                           \
  if (p.d == DD && p.group == GG) {                                                        \
    if (p.max_length > int64_t{NW} * std::min(64 * p.bs - 32 - p.bs, kWgMaxTilesPerWave * 32)) \
      return false;                                                                        \
    hipLaunchKernelGGL((DecodeValuWg<float, DD, GG, NW>), grid, dim3(NW * 64), 0, stream, p); \
    *err = hipGetLastError();                                                              \
    return true;                                                                           \
  }
  // Eight wavefronts per workgroup keep the register budget of the
  // one-item kernels (two workgroup wavefronts per SIMD); the shapes that
  // would spill there take four.
  EHIP_WG_CASE(64, 1, 8)
  EHIP_WG_CASE(64, 2, 8)
  EHIP_WG_CASE(64, 4, 8)
  EHIP_WG_CASE(64, 7, 8)
  EHIP_WG_CASE(64, 8, 4)
  EHIP_WG_CASE(128, 1, 8)
  EHIP_WG_CASE(128, 2, 8)
  EHIP_WG_CASE(128, 7, 8)
  EHIP_WG_CASE(128, 8, 4)
#undef EHIP_WG_CASE
  return false;
}

hipError_t LaunchSplits(const DecodeParams& p, int kv_dtype, const Tuning& tune,
                        QueueState* queue, hipStream_t stream) {
  if (ScaledKv(kv_dtype)) {
    // No VALU fallback for INT8/FP8: the plan validation admits only the
    // shapes the MFMA kernel covers.
    hipError_t err = hipSuccess;
    if (LaunchDecodeQ8(p, kv_dtype == EHIP_KV_FP8, stream, &err)) return err;
    return hipErrorInvalidValue;
  }
  // The matrix-core kernel where it covers the shape (Tuning::decode_valu
  // selects the all-VALU kernels).
  hipError_t err = hipSuccess;
  if (LaunchDecodeMfma(p, kv_dtype, tune, queue, stream, &err)) return err;
  // Only the MFMA kernel performs a fused append; the caller checked coverage.
  if (p.new_k != nullptr) return hipErrorInvalidValue;
  if (kv_dtype != EHIP_KV_BF16) return LaunchTyped<float>(p, stream);
  return LaunchTyped<uint16_t>(p, stream);
}

}  // namespace

hipError_t LaunchDecode(const DecodeParams& p, int kv_dtype, const Tuning& tune,
                        QueueState* queue, hipStream_t stream) {
  // Small fp32 steps without prefill chunks: one workgroup per (row, kv head),
  // merged in LDS (the plan's split partials are not used). Not for a fused
  // append, which only the matrix-core kernel performs.
  if (kv_dtype == EHIP_KV_F32 && p.n_items > 0 && !p.has_prefill && p.new_k == nullptr) {
    hipError_t e = hipSuccess;
    if (LaunchSmallStep(p, tune, stream, &e)) return e;
  }
  // Split rows may come from prefill key splits alone (no decode items).
  hipError_t e = p.n_items > 0 ? LaunchSplits(p, kv_dtype, tune, queue, stream) : hipSuccess;
  if (e != hipSuccess || p.n_merge == 0) return e;
  // Only the rows that were split: a step dominated by prefill-chunk rows
  // (which need no merge) launches no idle merge blocks.
  const int64_t groups = int64_t{p.n_merge} * p.kv_heads;
  const int gd = p.group * p.d;
  // Four elements per thread for merges of 2^18 output elements or more,
  // where fewer instructions per element pay (merge kernel, rocprofv3: C4's
  // 2048 groups of 512 elements 7.8 -> 6.7 us, C5's 256 groups of 1024
  // 8.8 -> 8.5 us). Small merges keep one element per thread, whose extra
  // threads put more loads in flight at once (C2's 64 groups of 448: 4.7
  // against 5.0 us with four). The partial workspace is 256-byte aligned; the
  // output row offset is a multiple of d floats.
  const bool wide = groups * gd >= (int64_t{1} << 18);
  if (wide && p.d % 4 == 0 && reinterpret_cast<uintptr_t>(p.out) % 16 == 0) {
    const int chunks = (gd + 4 * kMergeThreads - 1) / (4 * kMergeThreads);
    hipLaunchKernelGGL(MergeSplitsKernel<4>, dim3(groups * chunks), dim3(kMergeThreads), 0,
                       stream, p, chunks);
  } else {
    const int chunks = (gd + kMergeThreads - 1) / kMergeThreads;
    hipLaunchKernelGGL(MergeSplitsKernel<1>, dim3(groups * chunks), dim3(kMergeThreads), 0,
                       stream, p, chunks);
  }
  return hipGetLastError();
}

}  // namespace ehip
