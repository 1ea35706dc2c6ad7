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
// Work: one workgroup of 4 wavefronts per (sequence, kv head, M query rows);
// wavefront w owns 16 of those rows for 2 of the kv head's g query heads
// (g = 4: M = 32, two row groups x two head groups; g = 8: M = 16, four head
// groups). Each wavefront keeps 2 (row block, head) accumulator blocks, so
// every K and V operand read from LDS feeds two MFMAs.
// Keys stream in 32-token tiles that go from the slab straight into LDS
// (buffer_load ... lds, no staging registers) into three buffers, two tiles
// ahead of compute. K and V tiles are both row-major [token][d], 256-byte
// rows with their 16-byte chunks XOR-swizzled by 2 (row mod 8) (a load
// instruction writes 1 KiB of consecutive LDS, so rows cannot be padded).
// The MFMA A operand of K (16 tokens x 8 elements per lane, one 16-byte read)
// and the PV operand of V read with ds_read_b64_tr_b16 (two transposed 8-byte
// reads per lane: 4 tokens x 16 columns of 4 rows per 16-lane group) read the
// swizzled chunks.
// S^T = K Q^T (v_mfma_f32_16x16x32_bf16, A = K, B = Q^T): lane l holds
// scores of tokens 4*(l/16) + i of each 16-token half for query row l % 16,
// which is exactly the A-operand layout P needs for O = P V once the two
// halves' token order is folded into the V permutation. The online softmax
// (max/sum per row) runs in fp32 across the 4 lanes that share a row; the
// output rescale is skipped for a tile in which no row's running max moved.
#include <climits>

#include "decode_common.h"
#include "device_util.h"
#include "kernels.h"

namespace ehip {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int kTile = 32;    // keys per tile
constexpr float kRefSlack = 8.f;
constexpr int kWaves = 4;

// Query rows per workgroup for group size g when each wavefront keeps hb
// (head) accumulator blocks of 16 rows: 4 wavefronts over g / hb head groups.
constexpr int PrefillRows(int g, int hb) { return 16 * (kWaves / (g / hb)); }

// Accumulator blocks (heads) per wavefront: each K and V operand read from
// LDS feeds two MFMAs.
constexpr int kHeadsPerWave = 2;

// ds_read_b64_tr_b16: lane i of each 16-lane group receives element i % 4 of
// the 8 bytes addressed by lanes 4j + i / 4 of the group, for j = 0..3.
__device__ __forceinline__ bf16x4_t TransposedRead(const unsigned char* p) {
  typedef __attribute__((ext_vector_type(4))) short s16x4_t;
  const s16x4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4_t*)(p));
  return __builtin_bit_cast(bf16x4_t, r);
}

// Reductions over the 4 lanes of a row (l, l ^ 16, l ^ 32, l ^ 48) with the
// gfx950 swap permutes, without an LDS round trip. With both operands set to
// x, v_permlane32_swap leaves (x[l % 32], x[32 + l % 32]) in lane l and
// v_permlane16_swap leaves (x of the even row, x of the odd row) of the
// lane's row pair; combining the two gives every lane the same value.
template <typename Op>
__device__ __forceinline__ float RowReduce(float x, Op op) {
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = op(__uint_as_float(h[0]), __uint_as_float(h[1]));
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float RowMax(float x) {
  return RowReduce(x, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ float RowSum(float x) {
  return RowReduce(x, [](float a, float b) { return a + b; });
}

__device__ __forceinline__ float Max4(float a, float b, float c, float d) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b),
                                       __builtin_elementwise_maximum(c, d));
}

template <int D>
struct PrefillSmem {
  static constexpr int ROW = D * 2;  // bytes per K or V row (16-byte chunks XOR-swizzled)
  static constexpr int TILE = kTile * ROW;
};

// LDS byte offset of 16-byte chunk c of K/V row r inside a tile. The chunks of
// a row are XOR-swizzled by 2 (r mod 8): rows are 256 bytes apart (the tile
// loads write whole 1 KiB runs of LDS, so rows cannot be padded), and the
// swizzle spreads both MFMA operand reads (a 16-byte K read of 16 rows at
// one chunk; a transposed V read of 4 rows at two chunks) over the banks.
__device__ __forceinline__ int SwzOff(int r, int c) { return r * 256 + ((c ^ (2 * (r & 7))) << 4); }

// OCC: wavefronts per SIMD. 3 makes the register allocation fit 168 (a few
// values spilled outside the tile loop; the three 48 KiB tile buffers of
// three workgroups fit a CU's LDS). 2 leaves it unconstrained: it lands at
// 180-186 registers, and a target of 2 (182/178) measured 4% slower on C3.
template <int D, int G, int OCC>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(OCC == 3 ? 3 : 1)))
void PrefillMfmaBf16(PrefillParams p) {
  constexpr int HB = kHeadsPerWave;   // heads (accumulator blocks) per wavefront
  // Fold the softmax's scale and reference into the QK^T MFMA (one FMA less
  // per score), with IEEE maxima and pairwise row sums. Measured on MI355X:
  // at three workgroups per CU (issue-bound, the C5 re-prefill) 330 -> 323 us
  // per layer; at two (bound by the longest blocks' tile latency, C3's
  // chunks) 37.0 -> 39.0 us, so only there.
  constexpr bool kFold = OCC == 3;
  constexpr int NHG = G / HB;         // head groups
  constexpr int RG = kWaves / NHG;    // 16-row groups per workgroup
  constexpr int M = 16 * RG;          // query rows per workgroup
  constexpr int NC = D / 32;          // MFMA k-chunks over head_dim (QK^T)
  constexpr int NB = D / 16;          // 16-wide output column blocks (PV)
  using SM = PrefillSmem<D>;
  static_assert(G % HB == 0 && NHG >= 1 && kWaves % NHG == 0, "g must be 4 or 8");
  static_assert(M == PrefillRows(G, HB), "rows per workgroup");
  // Per thread per tile: 2 x 16-byte K loads and 2 x 16-byte V loads.
  constexpr int KV_VECS = kTile * D / 8;  // 16-byte vectors per tile (K or V)
  static_assert(KV_VECS == 2 * kWaves * 64, "tile / block shape");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = lane & 15;
  const int kq = lane >> 4;
  const int rg = wave % RG;   // this wavefront's 16-row group
  const int hgi = wave / RG;  // and head group

  const PrefillItem it = p.items[blockIdx.x];
  const int hk = UnpackHk(it.hk_split);
  const int split = UnpackSplit(it.hk_split);
  const int P = it.past;       // cached keys before the chunk
  const int T = it.chunk;      // chunk rows
  const int q0 = it.q0;        // first chunk row of this workgroup
  const int bs = p.bs;
  const int qn = min(M, T - q0);             // live query rows of the workgroup
  const int kend = P + q0 + qn;              // keys [0, kend) are attended by some row
  const int key0 = it.key_begin;             // this item's key range [key0, key1)
  const int key1 = it.key_end;
  const bool whole = key0 == 0 && key1 >= kend;  // else: partials for the split merge
  const int r0 = q0 + 16 * rg;               // this wavefront's first row
  const int qnw = min(16, max(0, T - r0));   // its live rows (0: nothing to compute)
  const int wend = min(P + r0 + qnw, key1);  // keys this wavefront's rows attend here

  // Q^T as MFMA B operands (bf16, round-to-nearest-even), in registers:
  // lane l holds Q[row r0 + l%16][c*32 + 8*kq .. +8] for each of its heads
  // (with kFold scaled by scale * log2(e) before the rounding, so the MFMA
  // leaves scores in the log2 units of the softmax). The fp32 rows are
  // loaded after the first tiles' block ids and converted after the first
  // tiles' K/V loads are issued (below).
  bf16x8_t qreg[HB][NC];
  float4 qraw[HB][NC][2];
  auto load_q = [&]() __attribute__((always_inline)) {
    const int qr = r0 + min(n, max(qnw, 1) - 1);
#pragma unroll
    for (int hh = 0; hh < HB; ++hh) {
      const int head = hk * G + hgi * HB + hh;
      const float* qp = p.q + (int64_t{it.row_base + min(qr, T - 1)} * p.heads + head) * D + kq * 8;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        qraw[hh][c][0] = *reinterpret_cast<const float4*>(qp + c * 32);
        qraw[hh][c][1] = *reinterpret_cast<const float4*>(qp + c * 32 + 4);
      }
    }
  };
  auto convert_q = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int hh = 0; hh < HB; ++hh)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const float4 a = qraw[hh][c][0], b = qraw[hh][c][1];
        const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        bf16x8_t qv;
#pragma unroll
        for (int i = 0; i < 8; ++i) qv[i] = static_cast<__bf16>(kFold ? x[i] * p.scale_log2 : x[i]);
        qreg[hh][c] = qv;
      }
  };

  // Tile loads: thread -> (token, 8-element group), two K and two V vectors
  // per tile, at the same slab offsets.
  const uint16_t* kslab = static_cast<const uint16_t*>(p.k_slab) + int64_t{hk} * bs * D;
  const uint16_t* vslab = static_cast<const uint16_t*>(p.v_slab) + int64_t{hk} * bs * D;
  constexpr int EG = D / 8;  // 8-element groups per row
  // K/V tiles go from the slab straight into LDS (buffer_load ... lds: no
  // staging registers), into three buffers, two tiles ahead of compute.
  static_assert(D == 128, "tile loads write 4 rows of 256 bytes per instruction");
  __shared__ __align__(16) unsigned char lt0[2 * SM::TILE];
  __shared__ __align__(16) unsigned char lt1[2 * SM::TILE];
  __shared__ __align__(16) unsigned char lt2[2 * SM::TILE];
  bool bad = false;
  // Thread -> K and V rows tk0 = tid / 16 and tk1 = tk0 + 16: one load
  // instruction of a wavefront writes the 1 KiB of rows 4w..4w+3 (then
  // 16+4w..), lane l the 16 bytes at 16 l, which hold chunk (l % 16) ^ 2 (row
  // mod 8) of its row: the lane reads that chunk from the slab.
  const int tk0 = tid / EG, tk1 = tk0 + kTile / 2, ek = tid % EG;
  // bs is a power of two: block index and slot by shift and mask. A 32-key
  // tile spans at most two blocks (bs >= 16, tiles start at multiples of
  // 32): their two ids are read once per wavefront and selected per thread,
  // and K/V are read through buffer descriptors with 32-bit byte offsets
  // (the host routes slabs of 4 GiB or more away from this kernel).
  const int bsh = __builtin_ctz(bs), bmask = bs - 1;
  // A tile's two block ids are loaded two tiles ahead of its K/V loads, by
  // vector loads that share the K/V loads' in-order counter (a scalar load
  // would be waited for right before the K/V loads, and while one is in
  // flight every LDS wait becomes a wait for it too).
  const __amdgpu_buffer_rsrc_t rt = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int32_t*>(p.table + it.table_off), 0, 0xFFFFFFFFu, 0x00020000);
  const uint32_t nblk = static_cast<uint32_t>(p.slab_blocks);
  const int last_blk = (key1 - 1) >> bsh;
  const uint32_t stride_b = static_cast<uint32_t>(p.block_stride) * 2u;
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kslab), 0, 0xFFFFFFFFu, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vslab), 0, 0xFFFFFFFFu, 0x00020000);
  const uint32_t ko = static_cast<uint32_t>((ek ^ (2 * (tk0 & 7))) * 16);
  // A whole tile starting at a multiple of 32 keys (the planner cuts key
  // ranges at multiples of 32; the load checks it): row tk0 sits in its
  // first block, at slot (k0 mod bs) + tk0; row tk1 in its second block at
  // slot tk0 when bs = 16, else in the first at slot (k0 mod bs) + tk1. So
  // each load offset is a wavefront-uniform part (block id x stride, plus
  // the tile's slot offset) and these per-thread parts: 2 VALU instructions
  // per tile instead of ~20. Measured on the three-per-CU instance (VALU
  // issue-bound): C5 re-prefill 316 -> 310 us; on the two-per-CU one
  // (latency-bound) C3 chunks 31.5 -> 31.9 us, so only there.
  const uint32_t c0 = static_cast<uint32_t>(tk0 * D * 2) + ko;
  const uint32_t c1 = static_cast<uint32_t>((bs == 16 ? tk0 : tk1) * D * 2) + ko;
#define EHIP_PF_IDLOAD(ID, K0)                                                               \
  do {                                                                                      \
    const int kb0 = min((K0) >> bsh, last_blk);                                             \
    ID##0 = __builtin_amdgcn_raw_buffer_load_b32(rt, static_cast<uint32_t>(kb0) * 4u, 0, 0); \
    ID##1 = __builtin_amdgcn_raw_buffer_load_b32(                                            \
        rt, static_cast<uint32_t>(min(kb0 + 1, last_blk)) * 4u, 0, 0);                      \
  } while (0)
#define EHIP_PF_LDSP(x) ((__attribute__((address_space(3))) void*)(x))
#define EHIP_PF_GLOAD(BUF, K0, ID)                                                             \
  do {                                                                                      \
    const int kb0 = min((K0) >> bsh, last_blk);                                             \
    int id0 = __builtin_amdgcn_readfirstlane(ID##0);                                         \
    int id1 = __builtin_amdgcn_readfirstlane(ID##1);                                         \
    const bool okb = static_cast<uint32_t>(id0) < nblk && static_cast<uint32_t>(id1) < nblk; \
    bad = bad | !okb;                                                                        \
    id0 = okb ? id0 : 0;                                                                     \
    id1 = okb ? id1 : 0;                                                                     \
    uint32_t a0, a1;                                                                         \
    if (OCC == 3 && (K0) + kTile <= key1 && ((K0) & (kTile - 1)) == 0) {                    \
      const uint32_t so = static_cast<uint32_t>(((K0) & bmask) * D * 2);                     \
      a0 = static_cast<uint32_t>(id0) * stride_b + so + c0;                                  \
      a1 = static_cast<uint32_t>(bs == 16 ? id1 : id0) * stride_b + so + c1;                 \
    } else {                                                                                 \
      /* The item's last tile: rows past its end read its last row. */                       \
      const int pk0 = min((K0) + tk0, key1 - 1), pk1 = min((K0) + tk1, key1 - 1);            \
      a0 = static_cast<uint32_t>((pk0 >> bsh) != kb0 ? id1 : id0) * stride_b +               \
           static_cast<uint32_t>((pk0 & bmask) * D * 2) + ko;                                \
      a1 = static_cast<uint32_t>((pk1 >> bsh) != kb0 ? id1 : id0) * stride_b +               \
           static_cast<uint32_t>((pk1 & bmask) * D * 2) + ko;                                \
    }                                                                                        \
    unsigned char* const lk = (BUF) + wave * 1024;                                           \
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, EHIP_PF_LDSP(lk), 16, a0, 0, 0, 0);        \
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, EHIP_PF_LDSP(lk + SM::TILE / 2), 16, a1, 0, \
                                             0, 0);                                         \
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, EHIP_PF_LDSP(lk + SM::TILE), 16, a0, 0, 0,  \
                                             0);                                            \
    __builtin_amdgcn_raw_ptr_buffer_load_lds(                                                \
        rv, EHIP_PF_LDSP(lk + SM::TILE + SM::TILE / 2), 16, a1, 0, 0, 0);                   \
  } while (0)

  // Per head state. Scores/probabilities live in the S^T layout (row n =
  // l % 16); the output accumulators in the MFMA D layout (rows 4kq+i).
  f32x4_t o[HB][NB];
  float ref[HB], l[HB];
#pragma unroll
  for (int hh = 0; hh < HB; ++hh) {
    ref[hh] = -INFINITY;
    l[hh] = 0.f;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) o[hh][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  const int qpos = P + r0 + n;  // this lane's query position (S^T layout)

  const int ntiles = (key1 - key0 + kTile - 1) / kTile;
  auto compute_tile = [&](int tile, const unsigned char* buf) __attribute__((always_inline)) {
    const int k0 = key0 + tile * kTile;
    // Wavefront-uniform: a tile wholly past this wavefront's last row (the
    // other row groups' diagonal) is skipped.
    if (k0 < wend) {
      const unsigned char* kb = buf;
      const unsigned char* vb = buf + SM::TILE;
      // Keys past this lane's query position (or past the workgroup's last
      // key) are masked.
      const bool diag = k0 + kTile > P + r0 || k0 + kTile > key1;
      const int lim = min(qpos, key1 - 1);

      // S^T for all heads: each K operand feeds HB MFMAs, each Q operand two
      // (the tile's halves). With kFold the accumulators start at -ref and Q
      // carries scale * log2(e), so they finish as the exponents of the
      // probabilities (score * scale * log2(e) - ref); otherwise one FMA per
      // score forms them.
      f32x4_t s[HB][2];
#pragma unroll
      for (int hh = 0; hh < HB; ++hh) {
        const float nr = !kFold || ref[hh] == -INFINITY ? 0.f : -ref[hh];
        s[hh][0] = s[hh][1] = f32x4_t{nr, nr, nr, nr};
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        bf16x8_t ka[2];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2)
          ka[h2] = __builtin_bit_cast(
              bf16x8_t, *reinterpret_cast<const uint4*>(kb + SwzOff(16 * h2 + n, 4 * c + kq)));
#pragma unroll
        for (int hh = 0; hh < HB; ++hh) {
          const bf16x8_t qv = qreg[hh][c];
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2)
            s[hh][h2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[h2], qv, s[hh][h2], 0, 0, 0);
        }
      }
      // s[hh][h2][i] = exponent of token k0 + 16*h2 + 4*kq + i for query row
      // n. Only tiles reaching the diagonal mask anything.
      if (diag) {
#pragma unroll
        for (int hh = 0; hh < HB; ++hh)
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (k0 + 16 * h2 + 4 * kq + i > lim) s[hh][h2][i] = -INFINITY;
      }
      // Lazy rescaling (FlashAttention-3, Shah et al. 2024): each row keeps a
      // reference ref (log2 units; -inf until the row meets a key) and the
      // probabilities are exp2(score * scale * log2e - ref). The reference
      // moves only when a tile's row max exceeds it by more than kRefSlack,
      // so probabilities stay below 2^kRefSlack and, for most tiles, neither
      // a row reduction nor an output rescale is needed: each lane checks its
      // own scores and the wavefront takes the slow path when any lane must.
      float t[HB][8], tmax[HB];
      bool need = false;
#pragma unroll
      for (int hh = 0; hh < HB; ++hh) {
        const float r = ref[hh] == -INFINITY ? 0.f : ref[hh];
#pragma unroll
        for (int j = 0; j < 8; ++j)  // masked scores stay -inf
          t[hh][j] = kFold ? s[hh][j >> 2][j & 3] : fmaf(s[hh][j >> 2][j & 3], p.scale_log2, -r);
        if constexpr (kFold) {
          // The MFMA results are not known to be canonical, so the IEEE
          // maximum (NaN-propagating: v_maximum3_f32 on gfx950) replaces
          // fmaxf, which would canonicalise each one first.
          const float m0 = Max4(t[hh][0], t[hh][1], t[hh][2], t[hh][3]);
          const float m1 = Max4(t[hh][4], t[hh][5], t[hh][6], t[hh][7]);
          tmax[hh] = __builtin_elementwise_maximum(m0, m1);
        } else {
          float tm = -INFINITY;  // FMA results: fmaxf chains become v_max3_f32
#pragma unroll
          for (int j = 0; j < 8; ++j) tm = fmaxf(tm, t[hh][j]);
          tmax[hh] = tm;
        }
        need = need || ref[hh] == -INFINITY || tmax[hh] > kRefSlack;
      }
      // The tile's V operands (two transposed reads per 16-column block) of
      // the first two blocks are requested ahead of the PV MFMAs, and each
      // PV step requests the block two ahead. With kFold the first two go
      // out here, before the softmax; on the two-per-CU instance issuing
      // them before the rescale branch measured slower (C3 37.0 -> 39.1 us),
      // so there they go out after it.
      const int vr = 4 * kq + (n >> 2);
      const unsigned char* vl = vb + (n & 1) * 8;
      auto vread = [&](int nb) __attribute__((always_inline)) {
        const int vo = SwzOff(vr, 2 * nb + ((n & 3) >> 1));
        const bf16x4_t v0 = TransposedRead(vl + vo);
        const bf16x4_t v1 = TransposedRead(vl + 16 * SM::ROW + vo);
        return __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
      };
      bf16x8_t vop[NB];
      if constexpr (kFold) {
        vop[0] = vread(0);
        vop[1] = vread(1);
      }
      if (__any(need)) {
        bool moved = false;
        float alpha[HB];
#pragma unroll
        for (int hh = 0; hh < HB; ++hh) {
          const float tr = RowMax(tmax[hh]);  // the row's max over the tile, from its reference
          const bool unset = ref[hh] == -INFINITY;
          const bool mv = tr != -INFINITY && (unset || tr > kRefSlack);
          const float d = mv ? tr : 0.f;
          alpha[hh] = unset ? 1.f : Exp2(-d);
          ref[hh] = mv ? (unset ? 0.f : ref[hh]) + tr : ref[hh];
          moved = moved || mv;
#pragma unroll
          for (int j = 0; j < 8; ++j) t[hh][j] -= d;
          l[hh] *= alpha[hh];
        }
        // Rescale the output (O^T: this lane's registers all belong to its
        // row n) by the row's alpha.
        if (__any(moved)) {
#pragma unroll
          for (int hh = 0; hh < HB; ++hh)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
              for (int i = 0; i < 4; ++i) o[hh][nb][i] *= alpha[hh];
        }
      }
      bf16x8_t pa[HB];
#pragma unroll
      for (int hh = 0; hh < HB; ++hh) {
        float pv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          pv[j] = Exp2(t[hh][j]);
          pa[hh][j] = static_cast<__bf16>(pv[j]);
        }
        // Lane-partial row sum over this lane's tokens: pairwise with kFold
        // (three dependent adds deep), in token order otherwise (measured
        // faster on the latency-bound two-per-CU instance).
        float ps = 0.f;
        if constexpr (kFold) {
          ps = ((pv[0] + pv[1]) + (pv[2] + pv[3])) + ((pv[4] + pv[5]) + (pv[6] + pv[7]));
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) ps += pv[j];
        }
        l[hh] += ps;
      }
      // O^T += V^T P^T: each V operand read once, HB MFMAs. The A operand of
      // lane (n, kq) is V[token][16nb + n] over tokens 4kq..4kq+3 and
      // 16+4kq..16+4kq+3 (the tokens its P values cover): two transposed
      // reads, in which lane s of each 16-lane group addresses token row
      // 4kq + s/4 (+16), columns 16nb + 4(s%4) .. +3, and lane n receives
      // column 16nb + n of the group's 4 rows. The B operand is P^T, which is
      // this lane's P values as they are (row n, the same 8 tokens).
      if constexpr (!kFold) {
        vop[0] = vread(0);
        vop[1] = vread(1);
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if (nb + 2 < NB) vop[nb + 2] = vread(nb + 2);
#pragma unroll
        for (int hh = 0; hh < HB; ++hh)
          o[hh][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop[nb], pa[hh], o[hh][nb], 0, 0, 0);
      }
    }
  };
  // Tile t goes to LDS buffer t % 3 (ids slot t % 3). Step t: wait until
  // this wavefront's loads of tile t have landed, barrier (every
  // wavefront's part of tile t is in LDS, and every wavefront is done
  // reading tile t - 1, whose buffer takes tile t + 2), compute tile t and
  // issue tile t + 2's loads and the block ids of tile t + 5 (in the order
  // below). At every wait the same vector memory operations follow tile t's
  // loads in issue order: the ids of tile t + 3, tile t + 1's four loads and
  // the ids of tile t + 4 (vmcnt retires them in order; the compiler
  // barriers keep that order).
  // Start: the first three tiles' block ids, then the query rows (neither
  // waits for the other), then tile 0's and tile 1's K/V once their ids are
  // in, then the queries' conversion. A C3 timeline of the start (entry to
  // the first tile in LDS, ~4.8 us at a launch's start) measured the same
  // with the rows loaded first: the first ids alone take 3.5-4 us to land.
  uint32_t idA0, idA1, idB0, idB1, idC0, idC1;  // block ids of each buffer's next tile
#define EHIP_PF_FENCE() asm volatile("" ::: "memory")
  EHIP_PF_IDLOAD(idA, key0);
  EHIP_PF_IDLOAD(idB, key0 + kTile);
  EHIP_PF_IDLOAD(idC, key0 + 2 * kTile);
  EHIP_PF_FENCE();
  load_q();
  EHIP_PF_FENCE();
  EHIP_PF_GLOAD(lt0, key0, idA);
  EHIP_PF_FENCE();
  EHIP_PF_IDLOAD(idA, key0 + 3 * kTile);
  EHIP_PF_FENCE();
  EHIP_PF_GLOAD(lt1, key0 + kTile, idB);
  EHIP_PF_FENCE();
  EHIP_PF_IDLOAD(idB, key0 + 4 * kTile);
  EHIP_PF_FENCE();
  __builtin_amdgcn_sched_barrier(0);
  convert_q();
  // Where a step issues tile t + 2's loads. On the two-per-CU instance
  // (bound by its longest blocks' walk) after computing tile t: right after
  // each barrier every wavefront of the workgroup would issue its loads at
  // once, and the later ones wait for the earlier ones to be accepted (a
  // per-tile C3 timeline put that at 0.28 of a 1.08 us step; C3 chunks
  // 35.3 -> 33.7 us). On the three-per-CU instance (issue-bound, three
  // workgroups' loads interleave anyway) before it, which keeps them two
  // tiles ahead (C5 re-prefill 314 against 316 us after).
  constexpr bool kLoadsAfter = OCC == 2;
#define EHIP_PF_LOADS(T, Y, IDY)                                        \
  do {                                                                  \
    EHIP_PF_FENCE();                                                    \
    EHIP_PF_GLOAD(Y, key0 + ((T) + 2) * kTile, IDY);                     \
    EHIP_PF_FENCE();                                                    \
    EHIP_PF_IDLOAD(IDY, key0 + ((T) + 5) * kTile);                       \
    EHIP_PF_FENCE();                                                    \
  } while (0)
#define EHIP_PF_STEP(T, X, Y, IDY)                                      \
  do {                                                                  \
    asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");       \
    if constexpr (!kLoadsAfter) EHIP_PF_LOADS(T, Y, IDY);               \
    compute_tile((T), (X));                                             \
  } while (0)
  // The walk ends with the item's last tile (before that step's loads when
  // they come after the tile). The loads stay unconditional otherwise, so the
  // count above holds at every step and the compiler's own waits stay exact
  // (the last steps load tiles past the item's end: its last rows again,
  // clamped).
  for (int tile = 0;; tile += 3) {
    EHIP_PF_STEP(tile, lt0, lt2, idC);
    if (tile + 1 >= ntiles) break;
    if constexpr (kLoadsAfter) EHIP_PF_LOADS(tile, lt2, idC);
    EHIP_PF_STEP(tile + 1, lt1, lt0, idA);
    if (tile + 2 >= ntiles) break;
    if constexpr (kLoadsAfter) EHIP_PF_LOADS(tile + 1, lt0, idA);
    EHIP_PF_STEP(tile + 2, lt2, lt1, idB);
    if (tile + 3 >= ntiles) break;
    if constexpr (kLoadsAfter) EHIP_PF_LOADS(tile + 2, lt1, idB);
  }
  // Loads past the item's end may still be in flight: they write this
  // workgroup's LDS, so they land before the workgroup ends.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#undef EHIP_PF_STEP
#undef EHIP_PF_LOADS
#undef EHIP_PF_FENCE
#undef EHIP_PF_LDSP

  // Row sums: each lane holds a partial over its tokens; the 4 lanes of a
  // row (l % 16 equal) together hold the row total. O^T puts output row n,
  // columns 16nb + 4kq .. +3 in lane (n, kq).
  if (whole) {
    // Normalised rows go out through LDS, so that each store instruction
    // writes two rows' 512-byte runs (whole 128-byte lines) rather than 16
    // rows' 64-byte pieces: a C3 timeline measured the epilogue at 1.96 ->
    // 0.94 us per workgroup with whole-line stores. The tile buffers are
    // free once every wavefront's loads have landed and its last tile is
    // computed (the barrier). Each wavefront stages one head at a time in
    // 8 KiB of them: rows 512 bytes apart, 16-byte chunk c of row r at
    // (c ^ r) (the 16 lanes of a write or read pass hit distinct banks).
    asm volatile("s_barrier" ::: "memory");
    unsigned char* const stage = (wave < 2 ? lt0 : lt1) + (wave & 1) * 8192;
#pragma unroll
    for (int hh = 0; hh < HB; ++hh) {
      const float inv = 1.0f / RowSum(l[hh]);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        *reinterpret_cast<float4*>(stage + n * 512 + (((4 * nb + kq) ^ n) & 31) * 16) =
            make_float4(o[hh][nb][0] * inv, o[hh][nb][1] * inv, o[hh][nb][2] * inv,
                        o[hh][nb][3] * inv);
      const int head = hk * G + hgi * HB + hh;
      const int c = lane & 31;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int row = 2 * j + (lane >> 5);
        const float4 v = *reinterpret_cast<const float4*>(stage + row * 512 + ((c ^ row) & 31) * 16);
        if (row < qnw)
          *reinterpret_cast<float4*>(p.out + (int64_t{it.row_base + r0 + row} * p.heads + head) * D +
                                     4 * c) = v;
      }
    }
  } else {
#pragma unroll
    for (int hh = 0; hh < HB; ++hh) {
      const float lt = RowSum(l[hh]);
      const int hg = hgi * HB + hh;  // head within the kv head's group
      if (n < qnw) {
        // Split partials: unnormalised output, the reference in log2 units
        // and the row sum, at the row's split slot.
        const RowDesc rd = p.rows[it.row_base + r0 + n];
        const int64_t pidx = PartialIndex(rd, p.kv_heads, hk, split);
        float* po = p.part_o + (pidx * G + hg) * D + 4 * kq;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          *reinterpret_cast<float4*>(po + 16 * nb) =
              make_float4(o[hh][nb][0], o[hh][nb][1], o[hh][nb][2], o[hh][nb][3]);
        if (kq == 0) {
          *reinterpret_cast<float2*>(p.part_ml + (pidx * G + hg) * 2) = make_float2(ref[hh], lt);
        }
      }
    }
  }
  if (__any(bad) && lane == 0) atomicOr(p.err, kErrBlockRange);
#undef EHIP_PF_GLOAD
#undef EHIP_PF_IDLOAD
}

}  // namespace

bool LaunchPrefillMfma(const PrefillParams& p, hipStream_t stream, hipError_t* err) {
  if (p.n_items == 0) {
    *err = hipSuccess;
    return true;
  }
  const dim3 grid(p.n_items), block(kWaves * 64);
  // Three workgroups per CU where the launch has work for several rounds of
  // them (the C5 re-prefill, 2048 workgroups: 277-278 us against 285 us at
  // two); two where it is bound by its longest blocks' walk (C3's 600
  // workgroups: 36.8 us at two against 38.6-39.6 us at three, the critical
  // blocks sharing their CU with more neighbours).
  static const int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 256;
    return n > 0 ? n : 256;
  }();
  const bool occ3 = p.n_items >= 4 * cus;
#define EHIP_PREFILL_CASE(DD, GG)                                                  \
  if (p.d == DD && p.group == GG) {                                                \
    if (occ3)                                                                      \
      hipLaunchKernelGGL((PrefillMfmaBf16<DD, GG, 3>), grid, block, 0, stream, p); \
    else                                                                           \
      hipLaunchKernelGGL((PrefillMfmaBf16<DD, GG, 2>), grid, block, 0, stream, p); \
    *err = hipGetLastError();                                                      \
    return true;                                                                   \
  }
  EHIP_PREFILL_CASE(128, 4)
  EHIP_PREFILL_CASE(128, 8)
#undef EHIP_PREFILL_CASE
  return false;
}

int PrefillRowsPerItem(int kv_dtype, int d, int group, int bs, int64_t slab_bytes) {
  if (kv_dtype != EHIP_KV_BF16 || d != 128 || (group != 4 && group != 8) || bs < 16) return 0;
  if (slab_bytes > int64_t{0xFFFFFFFF}) return 0;  // 32-bit K/V byte offsets
  return PrefillRows(group, kHeadsPerWave);
}

}  // namespace ehip
