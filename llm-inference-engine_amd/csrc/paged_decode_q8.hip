// INT8- and FP8-KV paged decode for gfx950: per-(block, kv head) scales, one
// 64-lane wavefront per work item (row, kv head, key range).
//
// The slabs hold int8 or E4M3 K/V [slab_blocks, Hkv, bs, d] with fp32 scales
// [slab_blocks, Hkv] beside them (the layout the reference reserves for INT8
// KV, docs/design/paged-kv-cache.md:219-231). Attention is the same online
// softmax over the dequantised values x = q * scale as the fp32/bf16 paths
// (kernels::PagedDecodeAttentionBatchedF32, src/kernels/paged_attention.h:105-110):
//
//  * QK^T runs on v_mfma_i32_16x16x64_i8 with the int8 keys as they sit in
//    the slab: lane (n, kq) loads D/4 contiguous bytes of key row n, and its
//    16-byte chunk c covers head-dim elements kq * D/4 + 16c .. + 16. Each
//    query row is scaled by 127 / max|q| and split into three int8 digits,
//    q ~ s_q * (d1 + d2 / 128 + d3 / 16384) with |error| <= s_q / 32768, over
//    the same head-dim permutation, so three integer MFMAs per chunk give the
//    dot products exactly in int32 up to that query rounding. The 16 keys of
//    one MFMA half lie in one block: that half's scores are
//    (a1 + a2 / 128 + a3 / 16384) * s_q * k_scale * softmax scale * log2 e.
//  * PV runs on the VALU in fp32: lane owns elements 4 * (lane % (D/4)) .. +4
//    of a token row (one 4-byte load). The bytes are read as unsigned after
//    flipping their sign bits (u = q + 128, one v_cvt_f32_ubyte each) and
//    multiplied by p * v_scale (the half's V scale is folded into the
//    probability when it is written for the PV layout); the
//    128 * sum(p * v_scale) offset is taken out once per item; token groups
//    are summed across lanes at the end.
//
// FP8 (E4M3) slabs take the same loads, tiles, softmax and outputs; two steps
// differ:
//  * QK^T runs on v_mfma_f32_16x16x32_bf16: the lane's D/4 key bytes (the
//    same loads as INT8) are widened to bf16 with v_cvt_scalef32_pk_bf16_fp8
//    (two per instruction, scale 1: every E4M3 value is a bf16 value), and q
//    is split into bf16 hi + lo (q = hi + lo to ~2^-17 relative, as in the
//    bf16 decode kernel). The fp8 matrix-core form
//    (v_mfma_scale_f32_16x16x128_f8f6f4 over E4M3 digits of q) measured
//    1e-4..2e-4 relative output error where a CPU model of the digit split
//    alone gives ~1e-6, so it stays out.
//  * PV converts the V bytes with v_cvt_pk_f32_fp8 (two per instruction);
//    signed codes need no offset correction.
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

typedef __attribute__((ext_vector_type(4))) int i32x4_t;

// Lazy rescaling slack (log2 units): probabilities stay below 2^8.
constexpr float kRefSlack = 8.f;

// Byte k of w as an unsigned integer in float (v_cvt_f32_ubyte).
__device__ __forceinline__ float UByteF(uint32_t w, int k) {
  return static_cast<float>((w >> (8 * k)) & 0xFFu);
}

__device__ __forceinline__ uint32_t PackDigits(const int* d) {
  return (static_cast<uint32_t>(d[0]) & 0xFFu) | ((static_cast<uint32_t>(d[1]) & 0xFFu) << 8) |
         ((static_cast<uint32_t>(d[2]) & 0xFFu) << 16) | (static_cast<uint32_t>(d[3]) << 24);
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

// OCC: waves per SIMD. RMAX: rows per work item. A joint item (two rows over
// their shared prefix) puts the second row's g heads in MFMA rows g..2g-1, so
// its keys are read and multiplied once for both rows; only the PV work
// grows with the virtual heads.
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

// Eight E4M3 codes (two words) as eight bf16 values (exact).
__device__ __forceinline__ bf16x8_t Fp8x8ToBf16(uint32_t w0, uint32_t w1) {
  const bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(w0), 1.0f, false);
  const bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(w0), 1.0f, true);
  const bf16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(w1), 1.0f, false);
  const bf16x2_t d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(w1), 1.0f, true);
  return bf16x8_t{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

template <int D, int G, int TH, int OCC, int RMAX, bool F8>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(OCC)))
void DecodeMfmaQ8(DecodeParams p) {
  using T = TileQ8<D, TH>;
  constexpr int TT = 16 * TH;
  constexpr int KB = T::KB;
  constexpr int KL = T::KL;
  constexpr int VLPT = T::VLPT;
  constexpr int VT = T::VT;
  constexpr int VJ = T::VJ;
  constexpr int GV = G * RMAX;  // virtual heads, row-major over the item's rows
  constexpr int HR = (GV + 3) / 4;
  constexpr int HP = HR * 4;
  static_assert(G >= 1 && G <= 8 && GV <= 16 && (D == 64 || D == 128), "shape");

  __shared__ float p_lds[TT * HP];

  const int lane = threadIdx.x;
  const int item_idx = blockIdx.x;
  if (item_idx >= p.n_items) return;
  ItemRef it = DecodeItem(p.items[item_idx]);
  if constexpr (RMAX > 2) AddItemRows(p, item_idx, it);
  const int nrows = RMAX == 1 ? 1 : it.nrows;  // the host launches RMAX >= the plan's joint rows
  const int hk = it.hk;
  const int tb = it.tb, te = it.te;
  const int bs = p.bs;
  const int n = lane & 15;
  const int kq = lane >> 4;
  const int ev = (lane % VLPT) * 4;
  const int tv = lane / VLPT;
  const int vrow = n / G;  // this lane's row of the item (virtual head n)
  const bool live = n < GV && vrow < nrows;

  float qf[KB];  // this lane's query slice: virtual head n, elements kq * KB .. + KB
  {
    int qrow = it.rows[0];  // the lane's row by selects (no dynamic indexing)
#pragma unroll
    for (int rr = 1; rr < RMAX; ++rr) qrow = (live && vrow == rr) ? it.rows[rr] : qrow;
    const float* qp =
        p.q + (int64_t{qrow} * p.heads + int64_t{hk} * G + (live ? n % G : 0)) * D + kq * KB;
#pragma unroll
    for (int i = 0; i < KB; i += 4) {
      const float4 x = *reinterpret_cast<const float4*>(qp + i);
      qf[i] = x.x;
      qf[i + 1] = x.y;
      qf[i + 2] = x.z;
      qf[i + 3] = x.w;
    }
  }
  // The range's table slice, two block ids per lane (ranges up to 128 blocks).
  const int lb0 = tb / bs;
  const int nblk = (te - 1) / bs - lb0 + 1;
  auto table_at = [&](int j) {
    const int raw = p.table[it.table_off + lb0 + min(j, nblk - 1)];
    const bool bad = raw < 0 || raw >= p.slab_blocks;
    return j < nblk ? (bad ? -2 : raw) : -1;
  };
  const int tab = table_at(lane);
  const int tab2 = table_at(64 + lane);
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

  // gh >= 0: the halves' block ids come from the work item (its first four
  // halves; gh: the tile's first half); gh < 0: from the table slice.
  auto load = [&](T& t, int t0, int gh) {
#pragma unroll
    for (int h2 = 0; h2 < TH; ++h2) {
      const int th = t0 + 16 * h2;  // wavefront-uniform; a half lies in one block (bs >= 16)
      const int bi = min(th, te - 1) / bs - lb0;  // wavefront-uniform, < 128
      const int phys = gh >= 0 ? it.first[min(gh + h2, 3)]
                               : __builtin_amdgcn_readlane(bi < 64 ? tab : tab2, bi & 63);
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
  // The first two tiles go in flight at once; when the item carries their
  // block ids neither waits for the table slice.
  if (it.first[0] >= 0) {
    load(bufA, tb, 0);
    if (it.first[TT / 16] >= 0)
      load(bufB, tb + TT, TT / 16);
    else
      load(bufB, tb + TT, -1);
  } else {
    load(bufA, tb, -1);
    load(bufB, tb + TT, -1);
  }

  // Query operands: int8, three digits per 16-element chunk (KL chunks);
  // FP8 keys, bf16 hi + lo per 8-element chunk (KB / 8 chunks).
  constexpr int NC8 = KB / 8;
  constexpr float kQRange = 127.0f;
  i32x4_t qd[KL][F8 ? 1 : 3];
  bf16x8_t qh[F8 ? NC8 : 1], ql[F8 ? NC8 : 1];
  float sq4[4];  // s_q of the heads 4 * kq + i (this lane's accumulator rows)
  {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < KB; ++i) amax = fmaxf(amax, fabsf(qf[i]));
    amax = fmaxf(amax, ShflXor(amax, 16));
    amax = fmaxf(amax, ShflXor(amax, 32));
    const float inv = (live && amax > 0.f) ? kQRange / amax : 0.f;
    const float sq = F8 ? 1.0f : (live ? amax * (1.0f / kQRange) : 0.f);
    if constexpr (F8) {
#pragma unroll
      for (int c = 0; c < NC8; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float xv = live ? qf[8 * c + i] : 0.f;
          const __bf16 hb = static_cast<__bf16>(xv);
          qh[c][i] = hb;
          ql[c][i] = static_cast<__bf16>(xv - static_cast<float>(hb));
        }
    } else {
#pragma unroll
      for (int c = 0; c < KL; ++c) {
        uint32_t w[3][4];
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          int d1[4], d2[4], d3[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float x = qf[c * 16 + g4 * 4 + j] * inv;
            const float r1 = rintf(x);
            const float x2 = (x - r1) * 128.0f;
            const float r2 = rintf(x2);
            const float r3 = rintf((x2 - r2) * 128.0f);
            d1[j] = static_cast<int>(r1);
            d2[j] = static_cast<int>(r2);
            d3[j] = static_cast<int>(r3);
          }
          w[0][g4] = PackDigits(d1);
          w[1][g4] = PackDigits(d2);
          w[2][g4] = PackDigits(d3);
        }
#pragma unroll
        for (int dg = 0; dg < 3; ++dg)
          qd[c][dg] = i32x4_t{static_cast<int>(w[dg][0]), static_cast<int>(w[dg][1]),
                              static_cast<int>(w[dg][2]), static_cast<int>(w[dg][3])};
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      sq4[i] = __shfl(sq, 4 * kq + i);  // lane 4kq+i holds head 4kq+i (kq of that lane = 0)
  }

  float m[4], lsum[4], cofs[4], o[GV][4];  // cofs: sum of p * v_scale per head row
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    lsum[i] = 0.f;
    cofs[i] = 0.f;
  }
#pragma unroll
  for (int h = 0; h < GV; ++h) o[h][0] = o[h][1] = o[h][2] = o[h][3] = 0.f;

  auto process = [&](const T& t, int t0) {
    float s[TH][4];
#pragma unroll
    for (int h2 = 0; h2 < TH; ++h2) {
      float dot[4];
      if constexpr (F8) {
        f32x4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC8; ++c) {
          const uint4 w = t.k[h2][c / 2];
          const bf16x8_t kb = (c & 1) ? Fp8x8ToBf16(w.z, w.w) : Fp8x8ToBf16(w.x, w.y);
          a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qh[c], kb, a, 0, 0, 0);
          a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ql[c], kb, a, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) dot[i] = a[i];
      } else {
        i32x4_t a1 = {0, 0, 0, 0}, a2 = {0, 0, 0, 0}, a3 = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < KL; ++c) {
          const i32x4_t kb = __builtin_bit_cast(i32x4_t, t.k[h2][c]);
          a1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(qd[c][0], kb, a1, 0, 0, 0);
          a2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(qd[c][1], kb, a2, 0, 0, 0);
          a3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(qd[c][2], kb, a3, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
          dot[i] = fmaf(static_cast<float>(a3[i]), 1.0f / 16384.0f,
                        fmaf(static_cast<float>(a2[i]), 1.0f / 128.0f, static_cast<float>(a1[i])));
      }
      const bool valid = t.phys[h2] >= 0 && t0 + 16 * h2 + n < te;
      const float sc = t.ks[h2] * p.scale_log2;
#pragma unroll
      for (int i = 0; i < 4; ++i) s[h2][i] = valid ? dot[i] * (sq4[i] * sc) : -INFINITY;
    }
    // Lazy rescaling (FlashAttention-3, Shah et al. 2024): each head row
    // keeps a reference m (log2 units; -inf until the row meets a key) that
    // moves only when a tile's row max exceeds it by more than kRefSlack, so
    // probabilities stay below 2^kRefSlack and most tiles need neither the
    // row reduction nor the output rescale: each lane checks its own scores
    // and the wavefront takes the slow path when any lane must.
    bool need = false;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int h2 = 0; h2 < TH; ++h2) need = need || s[h2][i] > m[i] + kRefSlack;
    const bool rescale = __any(need);
    float alpha[4] = {1.f, 1.f, 1.f, 1.f};
    if (rescale) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float mx = s[0][i];
#pragma unroll
        for (int h2 = 1; h2 < TH; ++h2) mx = fmaxf(mx, s[h2][i]);
        mx = Max16F(mx);
        const bool mv = mx > m[i] + kRefSlack;  // the same in the row's 16 lanes
        alpha[i] = mv && m[i] != -INFINITY ? Exp2(m[i] - mx) : 1.f;
        m[i] = mv ? mx : m[i];
        lsum[i] *= alpha[i];
        if constexpr (!F8) cofs[i] *= alpha[i];
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float ps = 0.f, pc = 0.f;
#pragma unroll
      for (int h2 = 0; h2 < TH; ++h2) {
        const float pr = m[i] == -INFINITY ? 0.f : Exp2(s[h2][i] - m[i]);
        ps += pr;
        // The half's V scale rides on the probability (one multiply per
        // score here instead of one per V element in the PV loop).
        s[h2][i] = pr * t.vs[h2];
        if constexpr (!F8) pc += s[h2][i];
      }
      lsum[i] += ps;
      if constexpr (!F8) cofs[i] += pc;
    }
    if (kq < HR) {
#pragma unroll
      for (int h2 = 0; h2 < TH; ++h2)
        *reinterpret_cast<float4*>(&p_lds[(16 * h2 + n) * HP + 4 * kq]) =
            make_float4(s[h2][0], s[h2][1], s[h2][2], s[h2][3]);
    }
    __syncthreads();
    if (rescale) {
#pragma unroll
      for (int h = 0; h < GV; ++h) {
        if (h / G >= nrows) break;
        const float a = ReadLaneF(alpha[h & 3], 16 * (h >> 2));
        o[h][0] *= a;
        o[h][1] *= a;
        o[h][2] *= a;
        o[h][3] *= a;
      }
    }
#pragma unroll
    for (int h2 = 0; h2 < TH; ++h2) {
      if (t.phys[h2] < 0) continue;
#pragma unroll
      for (int j = 0; j < VJ; ++j) {
        const int tt = 16 * h2 + j * VT + tv;
        float v0, v1, v2, v3;
        if constexpr (F8) {
          const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(t.v[h2][j]), false);
          const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(t.v[h2][j]), true);
          v0 = lo[0];
          v1 = lo[1];
          v2 = hi[0];
          v3 = hi[1];
        } else {
          const uint32_t r = t.v[h2][j] ^ 0x80808080u;  // u = q + 128
          v0 = UByteF(r, 0);
          v1 = UByteF(r, 1);
          v2 = UByteF(r, 2);
          v3 = UByteF(r, 3);
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
        for (int h = 0; h < GV; ++h) {
          if (h / G >= nrows) break;
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
    process(bufA, t0);
    if (t0 + TT >= te) break;
    load(bufA, t0 + 2 * TT, -1);
    process(bufB, t0 + TT);
    if (t0 + 2 * TT >= te) break;
    load(bufB, t0 + 3 * TT, -1);
  }

  ReportRejectedBlocks(p, tab);
  ReportRejectedBlocks(p, tab2);
  // Token groups of a V load hold partial sums of the same elements.
  if constexpr (VT > 1) {
#pragma unroll
    for (int h = 0; h < GV; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) o[h][e] = SumAcross<VLPT>(o[h][e]);
  }
  float lrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) lrow[i] = SumGroup16(lsum[i]);
  if constexpr (!F8) {
    // The unsigned bytes carried +128: take 128 * sum(p * v_scale) out of
    // every element of each head.
    float crow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) crow[i] = 128.0f * SumGroup16(cofs[i]);
#pragma unroll
    for (int h = 0; h < GV; ++h) {
      const float c = ReadLaneF(crow[h & 3], 16 * (h >> 2));
#pragma unroll
      for (int e = 0; e < 4; ++e) o[h][e] -= c;
    }
  }

  // Each of the item's rows: its g heads are virtual heads rr * g .. + g.
#pragma unroll
  for (int rr = 0; rr < RMAX; ++rr) {
    if (rr >= nrows) break;
    const int row = it.rows[rr];
    const RowDesc rd = p.rows[row];
    if (rd.nsplit == 1) {
      if (lane < VLPT) {
        float* op = p.out + (int64_t{row} * p.heads + int64_t{hk} * G) * D + ev;
#pragma unroll
        for (int h = 0; h < G; ++h) {
          const int vh = rr * G + h;
          const float inv = 1.0f / ReadLaneF(lrow[vh & 3], 16 * (vh >> 2));
          *reinterpret_cast<float4*>(op + h * D) =
              make_float4(o[vh][0] * inv, o[vh][1] * inv, o[vh][2] * inv, o[vh][3] * inv);
        }
      }
      continue;
    }
    const int64_t pidx = PartialIndex(rd, p.kv_heads, hk, it.split);
    if (lane < VLPT) {
      float* po = p.part_o + pidx * G * D + ev;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const int vh = rr * G + h;
        *reinterpret_cast<float4*>(po + h * D) =
            make_float4(o[vh][0], o[vh][1], o[vh][2], o[vh][3]);
      }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const int vh = rr * G + h;
      const float mh = ReadLaneF(m[vh & 3], 16 * (vh >> 2));
      const float lh = ReadLaneF(lrow[vh & 3], 16 * (vh >> 2));
      if (lane == 0) {
        p.part_ml[(pidx * G + h) * 2 + 0] = mh;
        p.part_ml[(pidx * G + h) * 2 + 1] = lh;
      }
    }
  }
}

template <int D, int G, bool F8>
void LaunchQ8Shape(const DecodeParams& p, hipStream_t stream) {
  // 32-token tiles: 64-token tiles measured slower on C4 and C5.
  // Joint plans: 2g or 4g virtual heads (one wavefront per SIMD where they
  // reach 16 at d = 128, whose accumulators would spill at two).
  if (p.n_joint > 0 && p.joint_rows > 2) {
    if constexpr (4 * G <= 16) {
      constexpr int OCC = (D == 128 && 4 * G >= 16) ? 1 : 2;
      hipLaunchKernelGGL((DecodeMfmaQ8<D, G, 2, OCC, 4, F8>), dim3(p.n_items), dim3(64), 0,
                         stream, p);
    }
    return;
  }
  if (p.n_joint > 0) {
    constexpr int OCC = (D == 128 && 2 * G >= 16) ? 1 : 2;
    hipLaunchKernelGGL((DecodeMfmaQ8<D, G, 2, OCC, 2, F8>), dim3(p.n_items), dim3(64), 0, stream,
                       p);
    return;
  }
  hipLaunchKernelGGL((DecodeMfmaQ8<D, G, 2, 2, 1, F8>), dim3(p.n_items), dim3(64), 0, stream, p);
}

}  // namespace

bool LaunchDecodeQ8(const DecodeParams& p, bool fp8, hipStream_t stream, hipError_t* err) {
  const bool aligned = (reinterpret_cast<uintptr_t>(p.k_slab) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.v_slab) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.q) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.out) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.k_scale) % 4 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.v_scale) % 4 == 0) &&
                       (p.block_stride % 16 == 0);
  if (!aligned || p.bs < 16) return false;
  if (p.n_joint > 0 && p.joint_rows * p.group > 16) return false;  // the plan caps groups
#define EHIP_Q8_CASE(DD, GG)                                                      \
  if (p.d == DD && p.group == GG) {                                               \
    if (fp8)                                                                      \
      LaunchQ8Shape<DD, GG, true>(p, stream);                                     \
    else                                                                          \
      LaunchQ8Shape<DD, GG, false>(p, stream);                                    \
    *err = hipGetLastError();                                                     \
    return true;                                                                  \
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
