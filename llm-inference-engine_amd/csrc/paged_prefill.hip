// Causal prefill-chunk attention over the paged cache on the gfx950 matrix
// cores (bf16 inputs, fp32 accumulation).
//
// Semantics: kernels::PrefillAttentionVarlenF32 (src/kernels/attention.h:221-227,
// src/kernels/attention.cpp:153-187; recurrence
// src/kernels/internal/attention_common.h:95-155): chunk row t of a sequence
// with L cached keys (post-append) and T new rows sits at position
// P + t (P = L - T) and attends keys [0, P + t]. The reference gathers each
// sequence's K/V into a contiguous copy first (src/kvcache/paged_gather.cpp:16-49);
// here K/V are read through the block table directly.
//
// Work: one workgroup of 4 wavefronts per (sequence, kv head, 16 query rows);
// wavefront w owns query heads hk*g + w*HPW .. +HPW (HPW = g / 4) of those
// rows. Keys stream in 32-token tiles staged in LDS (double-buffered, loaded
// one tile ahead into registers):
//   - K row-major [token][d], rows padded by 16 bytes, so the MFMA A operand
//     (16 tokens x 8 elements per lane) is one conflict-free 16-byte read;
//   - V transposed [d][token'], token' a permutation that puts the 8 tokens a
//     lane contracts over next to each other, rows padded to 80 bytes, so
//     the PV B operand is one 16-byte read as well.
// S^T = K Q^T (v_mfma_f32_16x16x32_bf16, A = K, B = Q^T): lane l holds
// scores of tokens 4*(l/16) + i of each 16-token half for query row l % 16,
// which is exactly the A-operand layout P needs for O = P V once the two
// halves' token order is folded into the V permutation. The online softmax
// (max/sum per row) runs in fp32 across the 4 lanes that share a row.
#include <cstdlib>

#include "device_util.h"
#include "kernels.h"

namespace ehip {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int kQRows = 16;   // query rows per workgroup
constexpr int kTile = 32;    // keys per tile
constexpr int kWaves = 4;

__device__ __forceinline__ float ShflF(float x, int src_lane) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src_lane << 2, __float_as_int(x)));
}

// Position of token t (0..31) of a tile in the transposed V rows: the MFMA
// contraction index k = 8*kq + i of lane group kq covers tokens 4kq+i (i < 4)
// of the first half and 16+4kq+i-4 (i >= 4) of the second.
__device__ __forceinline__ int VPerm(int t) {
  return t < 16 ? (t >> 2) * 8 + (t & 3) : ((t - 16) >> 2) * 8 + 4 + (t & 3);
}

template <int D>
struct PrefillSmem {
  static constexpr int KROW = D * 2 + 16;      // bytes per K row (padded)
  static constexpr int VROW = kTile * 2 + 16;  // bytes per transposed V row (padded)
  static constexpr int KBYTES = kTile * KROW;
  static constexpr int VBYTES = D * VROW;
  static constexpr int BYTES = 2 * (KBYTES + VBYTES);  // double-buffered
};

template <int D, int G>
__global__ __launch_bounds__(kWaves * 64) void PrefillMfmaBf16(PrefillParams p) {
  constexpr int HPW = G / kWaves;     // query heads per wavefront
  constexpr int NC = D / 32;          // MFMA k-chunks over head_dim (QK^T)
  constexpr int NB = D / 16;          // 16-wide output column blocks (PV)
  using SM = PrefillSmem<D>;
  static_assert(G % kWaves == 0 && HPW >= 1, "g must be a multiple of 4");
  // Per thread per tile: 2 x 16-byte K loads and 2 x 16-byte V loads.
  constexpr int KV_VECS = kTile * D / 8;  // 16-byte vectors per tile (K or V)
  static_assert(KV_VECS == 2 * kWaves * 64, "tile / block shape");

  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = lane & 15;
  const int kq = lane >> 4;

  const PrefillItem it = p.items[blockIdx.x];
  const int hk = it.kv_head;
  const int P = it.past;       // cached keys before the chunk
  const int T = it.chunk;      // chunk rows
  const int q0 = it.q0;        // first chunk row of this block
  const int bs = p.bs;
  const int qn = min(kQRows, T - q0);        // live query rows of this block
  const int kend = P + q0 + qn;              // keys [0, kend) are attended by some row
  const int kdiag = P + q0;                  // keys < kdiag are seen by every row

  // Q^T as MFMA B operands (bf16, round-to-nearest-even): lane l holds
  // Q[row q0 + l%16][c*32 + 8*kq .. +8] for each of its heads.
  bf16x8_t qb[HPW][NC];
  {
    const int qr = q0 + min(n, qn - 1);
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
      const int head = hk * G + wave * HPW + hh;
      const float* qp = p.q + (int64_t{it.row_base + qr} * p.heads + head) * D + kq * 8;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const float4 a = *reinterpret_cast<const float4*>(qp + c * 32);
        const float4 b = *reinterpret_cast<const float4*>(qp + c * 32 + 4);
        const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) qb[hh][c][i] = static_cast<__bf16>(x[i]);
      }
    }
  }

  // Tile loads: thread -> (token pair, 8-element group) for V and (token,
  // 8-element group) for K, two of each per tile.
  const uint16_t* kslab = static_cast<const uint16_t*>(p.k_slab) + int64_t{hk} * bs * D;
  const uint16_t* vslab = static_cast<const uint16_t*>(p.v_slab) + int64_t{hk} * bs * D;
  constexpr int EG = D / 8;  // 8-element groups per row
  uint4 kr0, kr1, vr0, vr1;  // the next tile, two 16-byte vectors of K and of V
  bool bad = false;
  // Thread -> K vectors u = tid and tid + 256 (token u / EG, group u % EG);
  // V token pair vp = tid % 16 (tokens 2vp, 2vp + 1), group tid / 16.
  const int tk0 = tid / EG, tk1 = (tid + kWaves * 64) / EG, ek = tid % EG;
  const int vp = tid % 16, ev = tid / 16;
#define EHIP_PF_GLOAD(K0)                                                                    \
  do {                                                                                      \
    const int pk0 = min((K0) + tk0, kend - 1), pk1 = min((K0) + tk1, kend - 1);             \
    const int pv0 = min((K0) + 2 * vp, kend - 1), pv1 = min((K0) + 2 * vp + 1, kend - 1);    \
    int b0 = p.table[it.table_off + pk0 / bs], b1 = p.table[it.table_off + pk1 / bs];         \
    int b2 = p.table[it.table_off + pv0 / bs], b3 = p.table[it.table_off + pv1 / bs];         \
    if (b0 < 0 || b0 >= p.slab_blocks) { bad = true; b0 = 0; }                               \
    if (b1 < 0 || b1 >= p.slab_blocks) { bad = true; b1 = 0; }                               \
    if (b2 < 0 || b2 >= p.slab_blocks) { bad = true; b2 = 0; }                               \
    if (b3 < 0 || b3 >= p.slab_blocks) { bad = true; b3 = 0; }                               \
    kr0 = *reinterpret_cast<const uint4*>(kslab + int64_t{b0} * p.block_stride +             \
                                          (pk0 % bs) * D + ek * 8);                          \
    kr1 = *reinterpret_cast<const uint4*>(kslab + int64_t{b1} * p.block_stride +             \
                                          (pk1 % bs) * D + ek * 8);                          \
    vr0 = *reinterpret_cast<const uint4*>(vslab + int64_t{b2} * p.block_stride +             \
                                          (pv0 % bs) * D + ev * 8);                          \
    vr1 = *reinterpret_cast<const uint4*>(vslab + int64_t{b3} * p.block_stride +             \
                                          (pv1 % bs) * D + ev * 8);                          \
  } while (0)

  // Per head state. Scores/probabilities live in the S^T layout (row n =
  // l % 16); the output accumulators in the MFMA D layout (rows 4kq+i).
  f32x4_t o[HPW][NB];
  float m[HPW], l[HPW];
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh) {
    m[hh] = -INFINITY;
    l[hh] = 0.f;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) o[hh][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  const int qpos = P + q0 + n;  // this lane's query position (S^T layout)

  const int ntiles = (kend + kTile - 1) / kTile;
  const int vtp = VPerm(2 * vp);
  EHIP_PF_GLOAD(0);
  for (int tile = 0; tile < ntiles; ++tile) {
    const int buf = tile & 1;
    const int k0 = tile * kTile;
    {
      unsigned char* kw = smem + buf * (SM::KBYTES + SM::VBYTES);
      unsigned char* vw = kw + SM::KBYTES;
      *reinterpret_cast<uint4*>(kw + tk0 * SM::KROW + ek * 16) = kr0;
      *reinterpret_cast<uint4*>(kw + tk1 * SM::KROW + ek * 16) = kr1;
      // V: pack the token pair's elements into (t, t+1) dwords and write
      // them transposed, V^T[e][perm(t)], with perm(2vp + 1) = perm(2vp) + 1.
      const uint32_t a[4] = {vr0.x, vr0.y, vr0.z, vr0.w};
      const uint32_t b[4] = {vr1.x, vr1.y, vr1.z, vr1.w};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t lo = (a[w] & 0xFFFFu) | (b[w] << 16);       // element 2w
        const uint32_t hi = (a[w] >> 16) | (b[w] & 0xFFFF0000u);   // element 2w + 1
        const int e = ev * 8 + 2 * w;
        *reinterpret_cast<uint32_t*>(vw + e * SM::VROW + vtp * 2) = lo;
        *reinterpret_cast<uint32_t*>(vw + (e + 1) * SM::VROW + vtp * 2) = hi;
      }
    }
    __syncthreads();
    if (tile + 1 < ntiles) EHIP_PF_GLOAD(k0 + kTile);  // next tile in flight during compute
    const unsigned char* kb = smem + buf * (SM::KBYTES + SM::VBYTES);
    const unsigned char* vb = kb + SM::KBYTES;
    const bool diag = k0 + kTile > kdiag;  // some key of the tile is masked for some row

#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
      f32x4_t s[2];
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        s[h2] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const bf16x8_t ka = __builtin_bit_cast(
              bf16x8_t, *reinterpret_cast<const uint4*>(kb + (16 * h2 + n) * SM::KROW +
                                                        (c * 32 + kq * 8) * 2));
          s[h2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[hh][c], s[h2], 0, 0, 0);
        }
      }
      // s[h2][i] = score(token k0 + 16*h2 + 4*kq + i, query row n)
      float sv[8];
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kpos = k0 + 16 * h2 + 4 * kq + i;
          const bool ok = !diag || (kpos <= qpos && kpos < kend);
          sv[4 * h2 + i] = ok ? s[h2][i] * p.scale_log2 : -INFINITY;
        }
      float mx = sv[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) mx = fmaxf(mx, sv[i]);
      mx = fmaxf(mx, ShflF(mx, lane ^ 16));
      mx = fmaxf(mx, ShflF(mx, lane ^ 32));
      const float mn = fmaxf(m[hh], mx);
      const float alpha = mn == -INFINITY ? 1.f : Exp2(m[hh] - mn);
      m[hh] = mn;
      bf16x8_t pa;
      float ps = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float pv = mn == -INFINITY ? 0.f : Exp2(sv[i] - mn);
        ps += pv;
        pa[i] = static_cast<__bf16>(pv);
      }
      l[hh] = l[hh] * alpha + ps;  // lane-partial over this lane's tokens
      // Rescale the output rows (D layout: row 4kq+i) by their row's alpha,
      // which lives in lanes l % 16 == row.
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ar = ShflF(alpha, 4 * kq + i);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) o[hh][nb][i] *= ar;
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const bf16x8_t vbv = __builtin_bit_cast(
            bf16x8_t, *reinterpret_cast<const uint4*>(vb + (16 * nb + n) * SM::VROW + kq * 16));
        o[hh][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, vbv, o[hh][nb], 0, 0, 0);
      }
    }
  }

  // Row sums: each lane holds a partial over its tokens; the 4 lanes of a
  // row (l % 16 equal) together hold the row total.
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh) {
    float lt = l[hh];
    lt += ShflF(lt, lane ^ 16);
    lt += ShflF(lt, lane ^ 32);
    const int head = hk * G + wave * HPW + hh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * kq + i;  // D-layout row of register i
      const float inv = 1.0f / ShflF(lt, r);
      if (r < qn) {
        float* op = p.out + (int64_t{it.row_base + q0 + r} * p.heads + head) * D + n;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) op[16 * nb] = o[hh][nb][i] * inv;
      }
    }
  }
  if (__any(bad) && lane == 0) atomicOr(p.err, kErrBlockRange);
#undef EHIP_PF_GLOAD
}

}  // namespace

bool LaunchPrefillMfma(const PrefillParams& p, hipStream_t stream, hipError_t* err) {
  if (p.n_items == 0) {
    *err = hipSuccess;
    return true;
  }
  const dim3 grid(p.n_items), block(kWaves * 64);
#define EHIP_PREFILL_CASE(DD, GG)                                                        \
  if (p.d == DD && p.group == GG) {                                                      \
    hipLaunchKernelGGL((PrefillMfmaBf16<DD, GG>), grid, block, PrefillSmem<DD>::BYTES, \
                       stream, p);                                                       \
    *err = hipGetLastError();                                                            \
    return true;                                                                         \
  }
  EHIP_PREFILL_CASE(128, 4)
  EHIP_PREFILL_CASE(128, 8)
#undef EHIP_PREFILL_CASE
  return false;
}

bool PrefillSupported(int kv_dtype, int d, int group, int bs) {
  return kv_dtype == EHIP_KV_BF16 && d == 128 && (group == 4 || group == 8) && bs >= 16;
}

}  // namespace ehip
