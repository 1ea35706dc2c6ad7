// Ragged paged decode attention for bf16 K/V on gfx950: QK^T on the matrix
// cores, softmax and PV on the vector ALUs in fp32.
//
// Same semantics and work partition as the VALU kernel (paged_decode.hip):
// one wavefront per (row, kv head, key split) work item, splits merged by
// log-sum-exp. What changes is where the arithmetic runs.
//
// QK^T: S[h][t] = sum_e Q[h][e] K[t][e] for the g query heads of the kv head
// and a 16-token block half, as v_mfma_f32_16x16x32_bf16 with A = Q (M = head,
// padded to 16) and B = K^T (N = token). The B operand of lane l is K row
// (l % 16), elements c*32 + (l/16)*8 .. +8 of chunk c: one 16-byte load per
// lane straight from the slab, no widening. Q is split into bf16 hi + lo
// parts (q = hi + lo to ~2^-17 relative) and both are multiplied, so the
// scores carry fp32-class accuracy while K stays in its stored bf16.
// Accumulator layout: lane l holds S[4*(l/16) + i][l % 16], i = 0..3.
//
// Softmax: online per 32-token tile (two MFMA halves): each 16-lane row
// reduces its heads' tile max with DPP; probabilities go through a small LDS
// buffer [token][head] to the PV layout.
//
// PV: lane l owns head_dim elements 8*(l % (d/8)) .. +8 of every other token
// row (d/8 lanes per row), accumulating o[h][e] in fp32 for all g heads; the
// token-parallel partial sums are reduced once at the end.
//
// K/V tiles are double-buffered in registers: the loads of tile k+1 are in
// flight while tile k is computed.
#include <cstdlib>
#include <cstring>

#include "decode_common.h"
#include "device_util.h"
#include "kernels.h"

namespace ehip {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

__device__ __forceinline__ bf16x8_t AsBf16x8(uint4 u) { return __builtin_bit_cast(bf16x8_t, u); }

__device__ __forceinline__ float ReadLane(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

// Max over each 16-lane row.
__device__ __forceinline__ float Max16(float x) {
  x = fmaxf(x, Dpp<0xB1>(x));
  x = fmaxf(x, Dpp<0x4E>(x));
  x = fmaxf(x, Dpp<0x141>(x));
  x = fmaxf(x, Dpp<0x128>(x));
  return x;
}

// TH 16-token halves of K and V (one MFMA N-tile each) for one tile.
template <int D, int TH>
struct Tile {
  static constexpr int NC = D / 32;
  static constexpr int PV_LPT = D / 8;
  static constexpr int PV_J = 16 * PV_LPT / 64;
  uint4 k[TH][NC];
  uint4 v[TH][PV_J];
  int phys[TH];
};

template <int D, int G, int TH>
__global__ __launch_bounds__(64) void DecodeMfmaBf16(DecodeParams p) {
  using T = Tile<D, TH>;
  constexpr int TT = 16 * TH;        // tokens per tile
  constexpr int NC = T::NC;          // MFMA k-chunks over head_dim
  constexpr int HR = (G + 3) / 4;    // 16-lane accumulator rows holding real heads
  constexpr int HP = HR * 4;         // heads padded to whole rows
  constexpr int PV_LPT = T::PV_LPT;  // PV lanes per token row
  constexpr int PV_TPI = 64 / PV_LPT;
  constexpr int PV_J = T::PV_J;
  static_assert(G >= 1 && G <= 16 && (D == 64 || D == 128), "shape");

  __shared__ float p_lds[TT * HP];

  const int lane = threadIdx.x;
  const int item_idx = blockIdx.x;
  if (item_idx >= p.n_items) return;
  const WorkItem it = p.items[item_idx];
  const RowDesc rd = p.rows[it.row];
  const int hk = it.kv_head;
  const int bs = p.bs;
  const int n = lane & 15;   // MFMA column (token of a half) / A row (head)
  const int kq = lane >> 4;  // MFMA k-group and accumulator row
  const int pv_e = (lane % PV_LPT) * 8;
  const int pv_t = lane / PV_LPT;

  // Q as MFMA A operands (hi and lo bf16 parts), zero for padding heads.
  bf16x8_t qa_hi[NC], qa_lo[NC];
  {
    const float* qp = p.q + (int64_t{it.row} * p.heads + int64_t{hk} * G) * D;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      uint32_t hi[4], lo[4];
      // Every lane loads (padding heads read head 0) and padding is zeroed
      // after, so no branch sits around the loads.
      const int hq = n < G ? n : 0;
      const float4 a = *reinterpret_cast<const float4*>(qp + hq * D + c * 32 + kq * 8);
      const float4 b = *reinterpret_cast<const float4*>(qp + hq * D + c * 32 + kq * 8 + 4);
      const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        const uint32_t h0 = Fp32ToBf16Bits(x[i]), h1 = Fp32ToBf16Bits(x[i + 1]);
        const uint32_t l0 = Fp32ToBf16Bits(x[i] - __uint_as_float(h0 << 16));
        const uint32_t l1 = Fp32ToBf16Bits(x[i + 1] - __uint_as_float(h1 << 16));
        hi[i / 2] = n < G ? (h0 | (h1 << 16)) : 0u;
        lo[i / 2] = n < G ? (l0 | (l1 << 16)) : 0u;
      }
      qa_hi[c] = AsBf16x8(make_uint4(hi[0], hi[1], hi[2], hi[3]));
      qa_lo[c] = AsBf16x8(make_uint4(lo[0], lo[1], lo[2], lo[3]));
    }
  }

  const int tb = it.split * rd.split_len;
  const int te = min(rd.length, tb + rd.split_len);
  const int lb0 = tb / bs;
  const int nblk = (te - 1) / bs - lb0 + 1;  // <= 64
  int tab = -1;
  if (lane < nblk) {
    tab = p.table[rd.table_off + lb0 + lane];
    if (tab < 0 || tab >= p.slab_blocks) {
      atomicOr(p.err, kErrBlockRange);
      tab = -1;
    }
  }
  const uint16_t* kbase = static_cast<const uint16_t*>(p.k_slab) + int64_t{hk} * bs * D;
  const uint16_t* vbase = static_cast<const uint16_t*>(p.v_slab) + int64_t{hk} * bs * D;
  const int bmask = bs - 1;
  const uint32_t tile_bytes = static_cast<uint32_t>(bs) * D * 2;  // one (block, head) tile
  // Per-lane byte offsets inside a (block, head) tile: loop-invariant.
  const int koff = (n * D + kq * 8) * 2;
  const int voff = (pv_t * D + pv_e) * 2;

  // K/V come in through buffer loads: the (block, head) tile base is a
  // scalar descriptor and each lane adds its fixed offset, so no 64-bit
  // address arithmetic sits between the loads and the compiler keeps the
  // next tile's loads in flight while the current one is computed. A half
  // beyond the split, or on a rejected block id, gets an empty descriptor:
  // its loads return zeros without touching memory, and it is masked.
  auto load = [&](T& t, int t0) {
#pragma unroll
    for (int h2 = 0; h2 < TH; ++h2) {
      const int th = t0 + 16 * h2;  // wavefront-uniform; a half lies in one block (bs >= 16)
      const int phys = __builtin_amdgcn_readlane(tab, min(th, te - 1) / bs - lb0);
      const bool ok = th < te && phys >= 0;
      t.phys[h2] = ok ? phys : -1;
      const int64_t boff = int64_t{ok ? phys : 0} * p.block_stride;
      const uint32_t range = ok ? tile_bytes : 0u;
      const __amdgpu_buffer_rsrc_t rk =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kbase + boff), 0, range, 0x00020000);
      const __amdgpu_buffer_rsrc_t rv =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vbase + boff), 0, range, 0x00020000);
      const int sbase = (th & bmask) * D * 2;
#pragma unroll
      for (int c = 0; c < NC; ++c)
        t.k[h2][c] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, koff + c * 64, sbase, 0));
#pragma unroll
      for (int j = 0; j < PV_J; ++j)
        t.v[h2][j] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, voff + j * PV_TPI * D * 2, sbase, 0));
    }
  };

  float m[4], lsum[4], o[G][8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    lsum[i] = 0.f;
  }
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[h][e] = 0.f;

  auto process = [&](const T& t, int t0) {
    f32x4_t acc[TH];
#pragma unroll
    for (int h2 = 0; h2 < TH; ++h2) {
      acc[h2] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const bf16x8_t kb = AsBf16x8(t.k[h2][c]);
        acc[h2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa_hi[c], kb, acc[h2], 0, 0, 0);
        acc[h2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa_lo[c], kb, acc[h2], 0, 0, 0);
      }
    }
    float s[TH][4];
#pragma unroll
    for (int h2 = 0; h2 < TH; ++h2) {
      const bool valid = t.phys[h2] >= 0 && t0 + 16 * h2 + n < te;
#pragma unroll
      for (int i = 0; i < 4; ++i) s[h2][i] = valid ? acc[h2][i] * p.scale_log2 : -INFINITY;
    }
    float alpha[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float mx = s[0][i];
#pragma unroll
      for (int h2 = 1; h2 < TH; ++h2) mx = fmaxf(mx, s[h2][i]);
      mx = Max16(mx);
      const float mn = fmaxf(m[i], mx);
      // An all-masked tile leaves mn at -inf: keep the state unchanged.
      alpha[i] = mn == -INFINITY ? 1.f : Exp2(m[i] - mn);
      m[i] = mn;
      float ps = 0.f;
#pragma unroll
      for (int h2 = 0; h2 < TH; ++h2) {
        s[h2][i] = mn == -INFINITY ? 0.f : Exp2(s[h2][i] - mn);
        ps += s[h2][i];
      }
      lsum[i] = lsum[i] * alpha[i] + ps;
    }
    if (kq < HR) {
#pragma unroll
      for (int h2 = 0; h2 < TH; ++h2)
        *reinterpret_cast<float4*>(&p_lds[(16 * h2 + n) * HP + 4 * kq]) =
            make_float4(s[h2][0], s[h2][1], s[h2][2], s[h2][3]);
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float a = ReadLane(alpha[h & 3], 16 * (h >> 2));
#pragma unroll
      for (int e = 0; e < 8; ++e) o[h][e] *= a;
    }
    const bool partial = t0 + TT > te;
#pragma unroll
    for (int h2 = 0; h2 < TH; ++h2) {
      if (t.phys[h2] < 0) continue;
#pragma unroll
      for (int j = 0; j < PV_J; ++j) {
        const int tt = 16 * h2 + j * PV_TPI + pv_t;
        const uint4 r = t.v[h2][j];
        float vf[8] = {Bf16Lo(r.x), Bf16Hi(r.x), Bf16Lo(r.y), Bf16Hi(r.y),
                       Bf16Lo(r.z), Bf16Hi(r.z), Bf16Lo(r.w), Bf16Hi(r.w)};
        if (partial && t0 + tt >= te) {
#pragma unroll
          for (int e = 0; e < 8; ++e) vf[e] = 0.f;  // stale rows never reach the sum
        }
        float pv[HP];
#pragma unroll
        for (int r4 = 0; r4 < HR; ++r4) {
          const float4 x = *reinterpret_cast<const float4*>(&p_lds[tt * HP + 4 * r4]);
          pv[4 * r4 + 0] = x.x;
          pv[4 * r4 + 1] = x.y;
          pv[4 * r4 + 2] = x.z;
          pv[4 * r4 + 3] = x.w;
        }
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
          for (int e = 0; e < 8; ++e) o[h][e] = fmaf(pv[h], vf[e], o[h][e]);
      }
    }
    __syncthreads();  // p_lds is rewritten by the next tile
  };

  T bufA, bufB;
  load(bufA, tb);
  for (int t0 = tb; t0 < te; t0 += 2 * TT) {
    load(bufB, t0 + TT);
    process(bufA, t0);
    if (t0 + TT >= te) break;
    load(bufA, t0 + 2 * TT);
    process(bufB, t0 + TT);
  }

  // Token-parallel partial sums -> per (head, element) totals.
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[h][e] = SumAcross<PV_LPT>(o[h][e]);
  float lrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) lrow[i] = SumGroup16(lsum[i]);

  if (it.nsplit == 1) {
    if (lane < PV_LPT) {
      float* op = p.out + (int64_t{it.row} * p.heads + int64_t{hk} * G) * D + pv_e;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float inv = 1.0f / ReadLane(lrow[h & 3], 16 * (h >> 2));
        *reinterpret_cast<float4*>(op + h * D) =
            make_float4(o[h][0] * inv, o[h][1] * inv, o[h][2] * inv, o[h][3] * inv);
        *reinterpret_cast<float4*>(op + h * D + 4) =
            make_float4(o[h][4] * inv, o[h][5] * inv, o[h][6] * inv, o[h][7] * inv);
      }
    }
    return;
  }
  const int64_t pidx = PartialIndex(rd, p.kv_heads, hk, it.nsplit, it.split);
  if (lane < PV_LPT) {
    float* po = p.part_o + pidx * G * D + pv_e;
#pragma unroll
    for (int h = 0; h < G; ++h) {
      *reinterpret_cast<float4*>(po + h * D) = make_float4(o[h][0], o[h][1], o[h][2], o[h][3]);
      *reinterpret_cast<float4*>(po + h * D + 4) =
          make_float4(o[h][4], o[h][5], o[h][6], o[h][7]);
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float mh = ReadLane(m[h & 3], 16 * (h >> 2));
    const float lh = ReadLane(lrow[h & 3], 16 * (h >> 2));
    if (lane == 0) {
      p.part_ml[(pidx * G + h) * 2 + 0] = mh;
      p.part_ml[(pidx * G + h) * 2 + 1] = lh;
    }
  }
}

}  // namespace

bool LaunchDecodeMfma(const DecodeParams& p, hipStream_t stream, hipError_t* err) {
  const bool aligned = (reinterpret_cast<uintptr_t>(p.k_slab) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.v_slab) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.q) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.out) % 16 == 0) &&
                       (p.block_stride % 8 == 0);
  if (!aligned || p.bs < 16) return false;
  const dim3 grid(p.n_items), block(64);
  // EHIP_DECODE_TILE=32 selects 32-token tiles (two MFMA halves per tile).
  const char* tile = std::getenv("EHIP_DECODE_TILE");
  const bool wide = tile && std::strcmp(tile, "32") == 0;
#define EHIP_MFMA_CASE(DD, GG)                                                     \
  if (p.d == DD && p.group == GG) {                                                \
    if (wide)                                                                      \
      hipLaunchKernelGGL((DecodeMfmaBf16<DD, GG, 2>), grid, block, 0, stream, p); \
    else                                                                           \
      hipLaunchKernelGGL((DecodeMfmaBf16<DD, GG, 1>), grid, block, 0, stream, p); \
    *err = hipGetLastError();                                                      \
    return true;                                                                   \
  }
  EHIP_MFMA_CASE(128, 1)
  EHIP_MFMA_CASE(128, 2)
  EHIP_MFMA_CASE(128, 4)
  EHIP_MFMA_CASE(128, 8)
  EHIP_MFMA_CASE(64, 1)
  EHIP_MFMA_CASE(64, 2)
  EHIP_MFMA_CASE(64, 4)
  EHIP_MFMA_CASE(64, 8)
#undef EHIP_MFMA_CASE
  return false;
}

}  // namespace ehip
