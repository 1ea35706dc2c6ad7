// INT8-KV paged decode for gfx950: per-(block, kv head) scales, one 64-lane
// wavefront per work item (row, kv head, key range).
//
// The slabs hold int8 K/V [slab_blocks, Hkv, bs, d] with fp32 scales
// [slab_blocks, Hkv] beside them (the layout the reference reserves for INT8
// KV, docs/design/paged-kv-cache.md:219-231). Attention is the same online
// softmax over the dequantised values x = q * scale as the fp32/bf16 paths
// (kernels::PagedDecodeAttentionBatchedF32, src/kernels/paged_attention.h:105-110):
//
//  * QK^T runs on v_mfma_f32_16x16x32_bf16. Lane (n, kq) loads D/4 bytes of
//    key row n in one piece (16 or 32 contiguous bytes); its 8-element chunk c
//    is bytes [8c, 8c + 8) of that piece, i.e. head-dim elements
//    kq * D/4 + 8c .. + 8. The query operands use the same permutation of the
//    head dimension, so the dot products are unchanged. int8 values widen to
//    bf16 exactly (|q| <= 127 fits bf16's 8-bit significand); Q is split into
//    bf16 hi + lo parts as in the bf16 kernel. The 16 keys of one MFMA half
//    lie in one block, so that half's score is scaled by the block's K scale
//    (times softmax scale and log2 e) after the MFMA.
//  * PV runs on the VALU in fp32: lane owns elements 4 * (lane % (D/4)) .. +4
//    of a token row (one 4-byte load), widened and multiplied by the half's V
//    scale; token groups are summed across lanes at the end.
//
// Rows past a key range read as zeros through bounded buffer descriptors and
// are masked; split results go through the same partial/merge path as the
// other decode kernels.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "decode_common.h"
#include "device_util.h"
#include "kernels.h"

namespace ehip {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

__device__ __forceinline__ float ReadLaneF(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

__device__ __forceinline__ float Max16F(float x) {
  x = fmaxf(x, Dpp<0xB1>(x));
  x = fmaxf(x, Dpp<0x4E>(x));
  x = fmaxf(x, Dpp<0x141>(x));
  x = fmaxf(x, Dpp<0x128>(x));
  return x;
}

// Signed byte k of w as float (exact).
__device__ __forceinline__ float ByteF(uint32_t w, int k) {
  return static_cast<float>(static_cast<int8_t>(w >> (8 * k)));
}

// Eight int8 (two dwords) widened to bf16: the bf16 of a small integer is the
// upper half of its fp32 bits (the lower half is zero), packed two per dword.
__device__ __forceinline__ bf16x8_t WidenQ8(uint32_t lo, uint32_t hi) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t src = i < 2 ? lo : hi;
    const uint32_t a = __float_as_uint(ByteF(src, (2 * i) & 3));
    const uint32_t b = __float_as_uint(ByteF(src, (2 * i + 1) & 3));
    w[i] = __builtin_amdgcn_perm(b, a, 0x07060302u);
  }
  return __builtin_bit_cast(bf16x8_t, make_uint4(w[0], w[1], w[2], w[3]));
}

template <int D, int TH>
struct TileQ8 {
  static constexpr int KB = D / 4;        // key bytes per lane per half
  static constexpr int KL = KB / 16;      // 16-byte key loads per lane per half
  static constexpr int VLPT = D / 4;      // PV lanes per token row (4 elements each)
  static constexpr int VT = 64 / VLPT;    // token rows per V load instruction
  static constexpr int VJ = 16 / VT;      // V loads per half
  uint4 k[TH][KL];
  uint32_t v[TH][VJ];
  float ks[TH], vs[TH];
  int phys[TH];
};

// QL: Q operands in LDS rather than registers. OCC: waves per SIMD.
template <int D, int G, int TH, bool QL, int OCC>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(OCC)))
void DecodeMfmaQ8(DecodeParams p) {
  using T = TileQ8<D, TH>;
  constexpr int TT = 16 * TH;
  constexpr int NC = D / 32;
  constexpr int KB = T::KB;
  constexpr int KL = T::KL;
  constexpr int VLPT = T::VLPT;
  constexpr int VT = T::VT;
  constexpr int VJ = T::VJ;
  constexpr int HR = (G + 3) / 4;
  constexpr int HP = HR * 4;
  static_assert(G >= 1 && G <= 8 && (D == 64 || D == 128), "shape");

  __shared__ float p_lds[TT * HP];
  __shared__ uint4 q_lds[QL ? 2 * NC * 64 : 1];

  const int lane = threadIdx.x;
  const int item_idx = blockIdx.x;
  if (item_idx >= p.n_items) return;
  const ItemRef it = DecodeItem(p.items[item_idx]);  // one row per item (no joint plans)
  const int row = it.rows[0];
  const int hk = it.hk;
  const int tb = it.tb, te = it.te;
  const int bs = p.bs;
  const int n = lane & 15;
  const int kq = lane >> 4;
  const int ev = (lane % VLPT) * 4;
  const int tv = lane / VLPT;
  const bool live = n < G;

  float4 qraw[NC][2];
  {
    const float* qp =
        p.q + (int64_t{row} * p.heads + int64_t{hk} * G + (live ? n : 0)) * D + kq * KB;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      qraw[c][0] = *reinterpret_cast<const float4*>(qp + c * 8);
      qraw[c][1] = *reinterpret_cast<const float4*>(qp + c * 8 + 4);
    }
  }
  const int lb0 = tb / bs;
  const int tab = LoadRangeTable(p, it.table_off, tb, te, lane);
  const int8_t* kbase = static_cast<const int8_t*>(p.k_slab) + int64_t{hk} * bs * D;
  const int8_t* vbase = static_cast<const int8_t*>(p.v_slab) + int64_t{hk} * bs * D;
  const int bmask = bs - 1;
  const int koff = n * D + kq * KB;
  const int voff = tv * D + ev;
  const uint32_t scale_range = static_cast<uint32_t>(
      p.slab_blocks * p.kv_heads * 4 < 0xFFFFFFFFll ? p.slab_blocks * p.kv_heads * 4 : 0xFFFFFFFFll);
  const __amdgpu_buffer_rsrc_t rks = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(p.k_scale), 0, scale_range, 0x00020000);
  const __amdgpu_buffer_rsrc_t rvs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(p.v_scale), 0, scale_range, 0x00020000);

  auto load = [&](T& t, int t0, bool given) {
#pragma unroll
    for (int h2 = 0; h2 < TH; ++h2) {
      const int th = t0 + 16 * h2;  // wavefront-uniform; a half lies in one block (bs >= 16)
      const int phys = given ? it.first[h2 > 0 ? 1 : 0]
                             : __builtin_amdgcn_readlane(tab, min(th, te - 1) / bs - lb0);
      const bool ok = th < te && phys >= 0;
      t.phys[h2] = ok ? phys : -1;
      const int64_t boff = int64_t{ok ? phys : 0} * p.block_stride + (th & bmask) * D;
      const uint32_t range = ok ? static_cast<uint32_t>(min(16, te - th) * D) : 0u;
      const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<int8_t*>(kbase + boff), 0, range, 0x00020000);
      const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<int8_t*>(vbase + boff), 0, range, 0x00020000);
#pragma unroll
      for (int i = 0; i < KL; ++i)
        t.k[h2][i] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, koff + 16 * i, 0, kKvLoadAux));
#pragma unroll
      for (int j = 0; j < VJ; ++j)
        t.v[h2][j] = __builtin_amdgcn_raw_buffer_load_b32(rv, voff + j * VT * D, 0, kKvLoadAux);
      // The block's scales (vector loads, so they count with the tile loads).
      const int so = ((ok ? phys : 0) * p.kv_heads + hk) * 4;
      t.ks[h2] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rks, so, 0, 0));
      t.vs[h2] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rvs, so, 0, 0));
    }
  };

  T bufA, bufB;
  if (it.first[0] >= 0)
    load(bufA, tb, true);
  else
    load(bufA, tb, false);

  bf16x8_t qa_hi[NC], qa_lo[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const float x[8] = {qraw[c][0].x, qraw[c][0].y, qraw[c][0].z, qraw[c][0].w,
                        qraw[c][1].x, qraw[c][1].y, qraw[c][1].z, qraw[c][1].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float xv = live ? x[i] : 0.f;
      const __bf16 hb = static_cast<__bf16>(xv);
      qa_hi[c][i] = hb;
      qa_lo[c][i] = static_cast<__bf16>(xv - static_cast<float>(hb));
    }
    if constexpr (QL) {
      q_lds[(2 * c) * 64 + lane] = __builtin_bit_cast(uint4, qa_hi[c]);
      q_lds[(2 * c + 1) * 64 + lane] = __builtin_bit_cast(uint4, qa_lo[c]);
    }
  }

  float m[4], lsum[4], o[G][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    lsum[i] = 0.f;
  }
#pragma unroll
  for (int h = 0; h < G; ++h) o[h][0] = o[h][1] = o[h][2] = o[h][3] = 0.f;

  auto process = [&](const T& t, int t0) {
    f32x4_t acc[TH];
#pragma unroll
    for (int h2 = 0; h2 < TH; ++h2) {
      acc[h2] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint4 w = t.k[h2][c / 2];
        const bf16x8_t kb = (c & 1) ? WidenQ8(w.z, w.w) : WidenQ8(w.x, w.y);
        const bf16x8_t qh = QL ? __builtin_bit_cast(bf16x8_t, q_lds[(2 * c) * 64 + lane]) : qa_hi[c];
        const bf16x8_t ql =
            QL ? __builtin_bit_cast(bf16x8_t, q_lds[(2 * c + 1) * 64 + lane]) : qa_lo[c];
        acc[h2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qh, kb, acc[h2], 0, 0, 0);
        acc[h2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ql, kb, acc[h2], 0, 0, 0);
      }
    }
    float s[TH][4];
#pragma unroll
    for (int h2 = 0; h2 < TH; ++h2) {
      const bool valid = t.phys[h2] >= 0 && t0 + 16 * h2 + n < te;
      const float sc = t.ks[h2] * p.scale_log2;
#pragma unroll
      for (int i = 0; i < 4; ++i) s[h2][i] = valid ? acc[h2][i] * sc : -INFINITY;
    }
    float alpha[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float mx = s[0][i];
#pragma unroll
      for (int h2 = 1; h2 < TH; ++h2) mx = fmaxf(mx, s[h2][i]);
      mx = Max16F(mx);
      const float mn = fmaxf(m[i], mx);
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
      const float a = ReadLaneF(alpha[h & 3], 16 * (h >> 2));
      o[h][0] *= a;
      o[h][1] *= a;
      o[h][2] *= a;
      o[h][3] *= a;
    }
#pragma unroll
    for (int h2 = 0; h2 < TH; ++h2) {
      if (t.phys[h2] < 0) continue;
      const float vsc = t.vs[h2];
#pragma unroll
      for (int j = 0; j < VJ; ++j) {
        const int tt = 16 * h2 + j * VT + tv;
        const uint32_t r = t.v[h2][j];
        const float v0 = ByteF(r, 0) * vsc, v1 = ByteF(r, 1) * vsc;
        const float v2 = ByteF(r, 2) * vsc, v3 = ByteF(r, 3) * vsc;
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
        for (int h = 0; h < G; ++h) {
          o[h][0] = fmaf(pv[h], v0, o[h][0]);
          o[h][1] = fmaf(pv[h], v1, o[h][1]);
          o[h][2] = fmaf(pv[h], v2, o[h][2]);
          o[h][3] = fmaf(pv[h], v3, o[h][3]);
        }
      }
    }
    __syncthreads();  // p_lds is rewritten by the next tile
  };

  for (int t0 = tb;; t0 += 2 * TT) {
    load(bufB, t0 + TT, false);
    process(bufA, t0);
    if (t0 + TT >= te) break;
    load(bufA, t0 + 2 * TT, false);
    process(bufB, t0 + TT);
    if (t0 + 2 * TT >= te) break;
  }

  ReportRejectedBlocks(p, tab);
  // Token groups of a V load hold partial sums of the same elements.
  if constexpr (VT > 1) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) o[h][e] = SumAcross<VLPT>(o[h][e]);
  }
  float lrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) lrow[i] = SumGroup16(lsum[i]);

  const RowDesc rd = p.rows[row];
  if (rd.nsplit == 1) {
    if (lane < VLPT) {
      float* op = p.out + (int64_t{row} * p.heads + int64_t{hk} * G) * D + ev;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float inv = 1.0f / ReadLaneF(lrow[h & 3], 16 * (h >> 2));
        *reinterpret_cast<float4*>(op + h * D) =
            make_float4(o[h][0] * inv, o[h][1] * inv, o[h][2] * inv, o[h][3] * inv);
      }
    }
    return;
  }
  const int64_t pidx = PartialIndex(rd, p.kv_heads, hk, it.split);
  if (lane < VLPT) {
    float* po = p.part_o + pidx * G * D + ev;
#pragma unroll
    for (int h = 0; h < G; ++h)
      *reinterpret_cast<float4*>(po + h * D) = make_float4(o[h][0], o[h][1], o[h][2], o[h][3]);
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float mh = ReadLaneF(m[h & 3], 16 * (h >> 2));
    const float lh = ReadLaneF(lrow[h & 3], 16 * (h >> 2));
    if (lane == 0) {
      p.part_ml[(pidx * G + h) * 2 + 0] = mh;
      p.part_ml[(pidx * G + h) * 2 + 1] = lh;
    }
  }
}

template <int D, int G>
void LaunchQ8Shape(const DecodeParams& p, hipStream_t stream) {
  constexpr bool QL = D * G >= 512;
  hipLaunchKernelGGL((DecodeMfmaQ8<D, G, 2, QL, 2>), dim3(p.n_items), dim3(64), 0, stream, p);
}

}  // namespace

bool LaunchDecodeQ8(const DecodeParams& p, hipStream_t stream, hipError_t* err) {
  const bool aligned = (reinterpret_cast<uintptr_t>(p.k_slab) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.v_slab) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.q) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.out) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.k_scale) % 4 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.v_scale) % 4 == 0) &&
                       (p.block_stride % 16 == 0);
  if (!aligned || p.bs < 16 || p.n_joint > 0) return false;
#define EHIP_Q8_CASE(DD, GG)           \
  if (p.d == DD && p.group == GG) {    \
    LaunchQ8Shape<DD, GG>(p, stream);  \
    *err = hipGetLastError();          \
    return true;                       \
  }
  EHIP_Q8_CASE(128, 1)
  EHIP_Q8_CASE(128, 2)
  EHIP_Q8_CASE(128, 4)
  EHIP_Q8_CASE(128, 8)
  EHIP_Q8_CASE(64, 1)
  EHIP_Q8_CASE(64, 2)
  EHIP_Q8_CASE(64, 4)
  EHIP_Q8_CASE(64, 8)
#undef EHIP_Q8_CASE
  return false;
}

}  // namespace ehip
