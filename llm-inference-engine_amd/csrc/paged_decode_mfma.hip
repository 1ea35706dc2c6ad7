// Ragged paged decode attention for bf16 K/V on gfx950: QK^T on the matrix
// cores, softmax and PV on the vector ALUs in fp32.
//
// Same semantics and work partition as the VALU kernel (paged_decode.hip):
// one wavefront per (row(s), kv head, key range) work item, ranges merged by
// log-sum-exp. What changes is where the arithmetic runs.
//
// QK^T: S[m][t] = sum_e Q[m][e] K[t][e] for the "virtual heads" m of the item
// (the g query heads of the kv head, for each row of the item: a joint item
// serves two rows sharing the range's blocks from one pass over K/V) and a
// 16-token block half, as v_mfma_f32_16x16x32_bf16 with A = Q (M = virtual
// head, padded to 16) and B = K^T (N = token). The B operand of lane l is K
// row (l % 16), elements c*32 + (l/16)*8 .. +8 of chunk c: one 16-byte load
// per lane straight from the slab, no widening. Q is split into bf16 hi + lo
// parts (q = hi + lo to ~2^-17 relative) and both are multiplied, so the
// scores carry fp32-class accuracy while K stays in its stored bf16.
// Accumulator layout: lane l holds S[4*(l/16) + i][l % 16], i = 0..3.
//
// Softmax: online per tile (one or two MFMA halves): each 16-lane row reduces
// its virtual heads' tile max with DPP; probabilities go through a small LDS
// buffer [token][virtual head] to the PV layout.
//
// PV: lane l owns head_dim elements 2*(l % (d/2)) and +1 of every
// (128/d)-th token row (all rows for d = 128), accumulating o[m][e] in fp32
// for every virtual head; V arrives as one 4-byte load per lane per row group,
// so each load instruction reads whole 256-byte rows, and the accumulators
// take 2·GV registers (the token-parallel sums of d = 64 are reduced once at
// the end).
//
// K/V arrive through buffer loads whose descriptor is the (block, head) tile
// base, double-buffered in registers: the next tile's loads are in flight
// while the current one is computed.
#include <cstdlib>
#include <cstring>
#include <type_traits>

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
// Lazy rescaling slack (log2 units): probabilities stay below 2^8.
constexpr float kRefSlack = 8.f;

__device__ __forceinline__ float Max16(float x) {
  x = fmaxf(x, Dpp<0xB1>(x));
  x = fmaxf(x, Dpp<0x4E>(x));
  x = fmaxf(x, Dpp<0x141>(x));
  x = fmaxf(x, Dpp<0x128>(x));
  return x;
}

// TH 16-token halves of K and V (one MFMA N-tile each) for one tile. KV is
// the slab element: uint16_t (bf16) or float. A lane's K operand of a chunk
// is 8 elements (KW 16-byte vectors); its V pair is 4 or 8 bytes.
template <class KV, int D, int TH>
struct Tile {
  static constexpr int NC = D / 32;
  static constexpr int KW = sizeof(KV) / 2;  // 16-byte K vectors per lane per chunk
  static constexpr int VLPT = D / 2;    // PV lanes per token row (2 elements each)
  static constexpr int VT = 64 / VLPT;  // token rows per V load instruction
  static constexpr int VJ = 16 / VT;    // V loads per 16-token half
  using VW = std::conditional_t<sizeof(KV) == 4, uint2, uint32_t>;
  uint4 k[TH][NC][KW];
  VW v[TH][VJ];
  int phys[TH];
};

// Two V elements of a lane as floats.
__device__ __forceinline__ void VPair(uint32_t r, float& v0, float& v1) {
  v0 = Bf16Lo(r);
  v1 = Bf16Hi(r);
}
__device__ __forceinline__ void VPair(uint2 r, float& v0, float& v1) {
  v0 = __uint_as_float(r.x);
  v1 = __uint_as_float(r.y);
}

// Orders a wavefront's own LDS stores before its later reads (and the reads
// before later stores) within an item. A one-wavefront workgroup uses the
// workgroup barrier; with several wavefronts per item each wavefront walks
// its own tiles, so the order is kept at wavefront scope (LDS operations of
// one wavefront execute in issue order).
template <int WPI>
__device__ __forceinline__ void ItemSync() {
  if constexpr (WPI == 1) {
    __syncthreads();
  } else {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// KV: uint16_t (bf16 slabs; K is the MFMA B operand as stored) or float (fp32
// slabs, d = 64: Q and each K row are split into three bf16 parts and the six
// leading products are accumulated, so the scores keep fp32 accuracy; V stays
// fp32 on the VALU).
// QL: keep the Q operands in LDS (read per MFMA) instead of 8·NC registers,
// so the wide shapes fit two wavefronts per SIMD.
// OCC: wavefronts per SIMD the register allocation must allow.
// FUSE: the launch carries the step's new K/V rows (fused append); the
// instance without it has no append code at all.
// WPI: wavefronts per work item. With WPI > 1 (launches whose grid covers
// every item, no queue) the item's whole tiles are cut into WPI contiguous
// runs, one per wavefront of the workgroup; each wavefront keeps its own
// softmax state and the workgroup combines the WPI states in LDS
// (log-sum-exp, as the split merge does) before wavefront 0 stores the item's
// result: an item's latency is then its wavefronts' shorter walks, with no
// more split partials for the merge launch to read.
template <class KV, int D, int G, int RMAX, int TH, int NBUF, bool QL, int OCC, bool FUSE,
          int WPI = 1>
__global__ __launch_bounds__(64 * WPI) __attribute__((amdgpu_waves_per_eu(OCC)))
void DecodeMfma(DecodeParams p) {
  using T = Tile<KV, D, TH>;
  constexpr bool F32 = sizeof(KV) == 4;
  constexpr int KW = T::KW;
  constexpr int TT = 16 * TH;        // tokens per tile
  constexpr int GV = G * RMAX;       // virtual heads (row-major over the item's rows)
  constexpr int NC = T::NC;          // MFMA k-chunks over head_dim
  constexpr int HR = (GV + 3) / 4;   // 16-lane accumulator rows holding virtual heads
  constexpr int HP = HR * 4;         // virtual heads padded to whole rows
  constexpr int VLPT = T::VLPT;
  constexpr int VT = T::VT;
  constexpr int VJ = T::VJ;
  static_assert(GV >= 1 && GV <= 16 && (D == 64 || D == 128), "shape");
  static_assert(WPI == 1 || (!QL && NBUF == 2), "items over several wavefronts: Q in registers");

  __shared__ float p_lds_all[WPI][TT * HP];
  constexpr int NQ = F32 ? 3 : 2;  // bf16 parts of Q
  __shared__ uint4 q_lds[QL ? NQ * NC * 64 : 1];
  // Fused append: the row's new K row as stored (bf16 or fp32) and its V
  // pairs (element 2i, 2i + 1 per entry).
  __shared__ uint4 knew_lds[FUSE ? D * static_cast<int>(sizeof(KV)) / 16 : 1];
  __shared__ typename T::VW vnew_lds[FUSE ? D / 2 : 1];
  // The item's table slice (up to 128 block ids), per wavefront: read by
  // broadcast LDS loads when a tile's loads are issued, so no register holds
  // it through the item.
  __shared__ int tab_lds[WPI][128];

  const int lane = threadIdx.x & 63;
  const int wv = WPI > 1 ? static_cast<int>(threadIdx.x >> 6) : 0;  // wavefront of the item
  float* const p_lds = p_lds_all[wv];
  // Persistent wavefronts: a workgroup's first item is its index; each later
  // one comes by ticket from the workgroup's sub-queue. The ticket
  // is drawn when at most kDrawAhead keys of the current item remain: late
  // enough that items go to the wavefronts that free up first (longest-first
  // list scheduling: the queue hands out the short items last, so the
  // wavefronts finish together), early enough to hide the atomic's latency.
  // On its way out each wavefront counts itself in; the last one (which then
  // knows every ticket has been drawn) clears every counter for the next
  // launch, so a launch leaves them as it found them: zero. A launch whose
  // grid covers every item (each wavefront's first item is its only one)
  // touches no counter at all: no tickets, no count on the way out.
  // Descriptors come through the scalar unit: the rows' split slots and the
  // next item are requested together before the item's results are stored,
  // so neither waits behind outstanding vector memory operations (vmcnt
  // retires loads and stores in issue order).
  constexpr int kDrawAhead = 64;
  // Sub-queue q of nq serves items q, q + nq, ... in list order: the ones
  // below gridDim.x are first items (workgroup i starts with item i), the
  // rest go out by ticket, from the first such index at or above gridDim.x.
  const int nq = min(p.queues, static_cast<int>(gridDim.x));
  const bool queued = WPI == 1 && static_cast<int>(gridDim.x) < p.n_items;
  // Workgroup b runs on XCD b mod 8. Spread: sub-queue (b / 8) mod nq, served
  // by workgroups of every XCD (a grid of at least 8 nq workgroups gives
  // every sub-queue some); else b mod nq, one XCD's workgroups per sub-queue.
  const int q = (p.queue_spread && static_cast<int>(gridDim.x) >= 8 * nq)
                    ? (static_cast<int>(blockIdx.x) >> 3) % nq
                    : static_cast<int>(blockIdx.x) % nq;
  const int first_queued = q + nq * ((static_cast<int>(gridDim.x) - q + nq - 1) / nq);
  uint32_t* const my_queue = p.queue + q * kQueueStride;
  int item_idx = blockIdx.x;
  WorkItem wi;
  if (item_idx < p.n_items) wi = ScalarRead(p.items, item_idx);
  while (item_idx < p.n_items) {
  uint32_t ticket = 0;
  bool drawn = false;
  ItemRef it = DecodeItem(wi);
  if constexpr (RMAX > 2) AddItemRows(p, item_idx, it);
  const int nrows = it.nrows;  // <= RMAX (the host launches RMAX >= the plan's joint rows)
  const int hk = it.hk;
  const int tb = it.tb, te = it.te;
  const int bs = p.bs;
  const int n = lane & 15;   // MFMA column (token of a half) / A row (virtual head)
  const int kq = lane >> 4;  // MFMA k-group and accumulator row
  const int ev = (lane % VLPT) * 2;  // PV head_dim elements ev, ev + 1
  const int tv = lane / VLPT;        // PV token row within a load's row group

  // Everything the item needs is fetched at once: the range's table slice
  // (every row of the item reads the same blocks over [tb, te)) and the
  // queries; the first tile's K/V follow as soon as the table lands.
  const int vrow = n / G;  // item row of this lane's virtual head
  const bool live = n < GV && vrow < nrows;
  float4 qraw[NC][2];
  {
    // Every lane loads (padding lanes read a live head) and padding is
    // zeroed afterwards, so no branch sits around the loads.
    // The lane's row by selects (no dynamic indexing of the item's rows).
    int qrow = it.rows[0];
#pragma unroll
    for (int rr = 1; rr < RMAX; ++rr) qrow = (live && vrow == rr) ? it.rows[rr] : qrow;
    const int qh = live ? n % G : 0;
    const float* qp = p.q + (int64_t{qrow} * p.heads + int64_t{hk} * G + qh) * D + kq * 8;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      qraw[c][0] = *reinterpret_cast<const float4*>(qp + c * 32);
      qraw[c][1] = *reinterpret_cast<const float4*>(qp + c * 32 + 4);
    }
  }
  const int lb0 = tb / bs;
  const int tab = LoadRangeTable(p, it.table_off, tb, te, lane);
  const int tab2 = LoadRangeTable(p, it.table_off, tb, te, 64 + lane);
  const KV* kbase = static_cast<const KV*>(p.k_slab) + int64_t{hk} * p.head_stride;
  const KV* vbase = static_cast<const KV*>(p.v_slab) + int64_t{hk} * p.head_stride;
  const int bmask = bs - 1;
  constexpr int ES = static_cast<int>(sizeof(KV));
  // Per-lane byte offsets inside a (block, head) tile: loop-invariant.
  const int koff = (n * D + kq * 8) * ES;
  const int voff = (tv * D + ev) * ES;
  // Fused append: the item ending at its row's last key (position te - 1)
  // streams keys [tb, te - 1) from the slab and takes the new key from the
  // step's new rows in one more step after the loop.
  const bool fuse_item = FUSE && it.last;        // workgroup-uniform
  const bool fuse = fuse_item && wv == WPI - 1;  // the wavefront that appends
  const int newpos = te - 1;
  const int kend = fuse_item ? newpos : te;  // keys the tile loops read from the slab
  // This wavefront's slab keys [wtb, wte): the item's whole tiles in WPI runs.
  int wtb = tb, wte = kend;
  if constexpr (WPI > 1) {
    const int per = ((kend - tb + TT - 1) / TT + WPI - 1) / WPI;
    wtb = min(kend, tb + wv * per * TT);
    wte = min(kend, tb + (wv + 1) * per * TT);
  }

  // Each half's descriptor starts at its first token row and covers only the
  // rows inside the range: rows past the range end read as zeros (so stale
  // slab rows never reach the PV sums, whatever they hold), and a half beyond
  // the range, or on a rejected block id, gets an empty descriptor whose loads
  // return zeros without touching memory. Scores of such rows are masked.
  // gh >= 0: the halves' block ids come from the work item, which carries
  // the item's first four halves (gh: the tile's first half); gh < 0: from
  // the table slice.
  auto load = [&](T& t, int t0, int gh) {
#pragma unroll
    for (int h2 = 0; h2 < TH; ++h2) {
      const int th = t0 + 16 * h2;  // wavefront-uniform; a half lies in one block (bs >= 16)
      const int phys =
          gh >= 0 ? it.first[min(gh + h2, 3)]
                  : __builtin_amdgcn_readfirstlane(
                        tab_lds[wv][max(0, min(th, kend - 1) / bs - lb0)]);
      const bool ok = th < kend && phys >= 0;
      t.phys[h2] = ok ? phys : -1;
      const int64_t boff = int64_t{ok ? phys : 0} * p.block_stride + (th & bmask) * D;
      const uint32_t range = ok ? static_cast<uint32_t>(min(16, kend - th) * D * ES) : 0u;
      const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<KV*>(kbase + boff), 0, range, 0x00020000);
      const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<KV*>(vbase + boff), 0, range, 0x00020000);
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int w = 0; w < KW; ++w)
          t.k[h2][c][w] = __builtin_bit_cast(
              uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, koff + c * 32 * ES + w * 16, 0,
                                                           kKvLoadAux));
#pragma unroll
      for (int j = 0; j < VJ; ++j) {
        if constexpr (F32)
          t.v[h2][j] = __builtin_bit_cast(
              uint2, __builtin_amdgcn_raw_buffer_load_b64(rv, voff + j * VT * D * ES, 0, kKvLoadAux));
        else
          t.v[h2][j] = __builtin_amdgcn_raw_buffer_load_b32(rv, voff + j * VT * D * ES, 0, kKvLoadAux);
      }
    }
  };

  // The table slice into LDS (waiting for its two loads), rejected ids
  // flagged; no register keeps it afterwards.
  auto stash = [&]() {
    tab_lds[wv][lane] = tab;
    tab_lds[wv][64 + lane] = tab2;
    ReportRejectedBlocks(p, tab);
    ReportRejectedBlocks(p, tab2);
  };

  T bufA, bufB, bufC;
  // The first two tiles go in flight at once, while Q is split; when the
  // item carries their block ids neither waits for the table slice.
  if (wv == 0 && it.first[0] >= 0) {
    load(bufA, tb, 0);
    if (it.first[TT / 16] >= 0) {
      load(bufB, tb + TT, TT / 16);
      stash();
    } else {
      stash();
      load(bufB, tb + TT, -1);
    }
  } else {
    stash();
    load(bufA, wtb, -1);
    load(bufB, wtb + TT, -1);
  }

  // Fused append: the item ending at its row's last key stores that key's
  // new K/V rows at the row's slot for later steps (bf16 slabs: narrowed with
  // the reference's round-to-nearest-even; fp32: as given), and keeps them in
  // LDS for its last step (no other item reads that row, and this item never
  // loads it from the slab).
  if (fuse) {
    const int row = it.rows[0];
    const int pair = lane % (D / 2);
    const int64_t src = (int64_t{row} * p.kv_heads + hk) * D + 2 * pair;
    const float2 kx = *reinterpret_cast<const float2*>(p.new_k + src);
    const float2 vx = *reinterpret_cast<const float2*>(p.new_v + src);
    typename T::VW kp, vp;
    if constexpr (F32) {
      kp = make_uint2(__float_as_uint(kx.x), __float_as_uint(kx.y));
      vp = make_uint2(__float_as_uint(vx.x), __float_as_uint(vx.y));
    } else {
      kp = Fp32ToBf16Bits(kx.x) | (Fp32ToBf16Bits(kx.y) << 16);
      vp = Fp32ToBf16Bits(vx.x) | (Fp32ToBf16Bits(vx.y) << 16);
    }
    reinterpret_cast<typename T::VW*>(knew_lds)[pair] = kp;
    vnew_lds[pair] = vp;
    const int64_t slot = p.slots[row];
    if (slot >= 0 && slot < p.slab_blocks * bs) {
      const int64_t blk = slot / bs;
      const int64_t dst = blk * p.block_stride + int64_t{hk} * p.head_stride +
                          (slot - blk * bs) * D + 2 * pair;
      if (lane < D / 2) {
        KV* kslab = static_cast<KV*>(const_cast<void*>(p.k_slab));
        KV* vslab = static_cast<KV*>(const_cast<void*>(p.v_slab));
        *reinterpret_cast<typename T::VW*>(kslab + dst) = kp;
        *reinterpret_cast<typename T::VW*>(vslab + dst) = vp;
      }
    } else if (lane == 0) {
      atomicOr(p.err, kErrSlotRange);
    }
    ItemSync<WPI>();  // the LDS rows are read by the tile patch below
  }

  // Q as MFMA A operands in NQ bf16 parts (round-to-nearest-even narrowing of
  // the remainder, branch-free): q = q0 + q1 (bf16 K) or q0 + q1 + q2 (fp32
  // K); padding virtual heads are zero.
  bf16x8_t qa[NQ][NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const float x[8] = {qraw[c][0].x, qraw[c][0].y, qraw[c][0].z, qraw[c][0].w,
                        qraw[c][1].x, qraw[c][1].y, qraw[c][1].z, qraw[c][1].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float r = live ? x[i] : 0.f;
#pragma unroll
      for (int k = 0; k < NQ; ++k) {
        const __bf16 b = static_cast<__bf16>(r);
        qa[k][c][i] = b;
        r -= static_cast<float>(b);
      }
    }
    if constexpr (QL) {
#pragma unroll
      for (int k = 0; k < NQ; ++k) q_lds[(NQ * c + k) * 64 + lane] = __builtin_bit_cast(uint4, qa[k][c]);
    }
  }

  float m[4], lsum[4], o[GV][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    lsum[i] = 0.f;
  }
#pragma unroll
  for (int h = 0; h < GV; ++h) o[h][0] = o[h][1] = 0.f;

  auto process = [&](const T& t, int t0, int tend) {
    if (queued && !drawn && t0 + kDrawAhead >= tend) {  // wavefront-uniform
      drawn = true;
      if (lane == 0) ticket = atomicAdd(my_queue, 1u);
    }
    f32x4_t acc[TH];
#pragma unroll
    for (int h2 = 0; h2 < TH; ++h2) {
      acc[h2] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        bf16x8_t qp[NQ];
#pragma unroll
        for (int k = 0; k < NQ; ++k) qp[k] = QL ? AsBf16x8(q_lds[(NQ * c + k) * 64 + lane]) : qa[k][c];
        if constexpr (F32) {
          // K = k0 + k1 + k2 (bf16 parts of the fp32 row): the six products
          // of parts whose indices sum to at most 2, smallest first. What is
          // left out is below 2^-24 of |q||k| per element (a 2 x 2 split
          // leaves ~2^-17, too coarse for the fp32 reference's 1e-4 / 1e-5
          // elementwise criterion at logit scales ~4).
          const uint4 a = t.k[h2][c][0], b = t.k[h2][c][1];
          const float x[8] = {__uint_as_float(a.x), __uint_as_float(a.y), __uint_as_float(a.z),
                              __uint_as_float(a.w), __uint_as_float(b.x), __uint_as_float(b.y),
                              __uint_as_float(b.z), __uint_as_float(b.w)};
          bf16x8_t kp[3];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            float r = x[i];
#pragma unroll
            for (int k = 0; k < 3; ++k) {
              const __bf16 bb = static_cast<__bf16>(r);
              kp[k][i] = bb;
              r -= static_cast<float>(bb);
            }
          }
          acc[h2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qp[0], kp[2], acc[h2], 0, 0, 0);
          acc[h2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qp[1], kp[1], acc[h2], 0, 0, 0);
          acc[h2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qp[2], kp[0], acc[h2], 0, 0, 0);
          acc[h2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qp[0], kp[1], acc[h2], 0, 0, 0);
          acc[h2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qp[1], kp[0], acc[h2], 0, 0, 0);
          acc[h2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qp[0], kp[0], acc[h2], 0, 0, 0);
        } else {
          const bf16x8_t kb = AsBf16x8(t.k[h2][c][0]);
          acc[h2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qp[0], kb, acc[h2], 0, 0, 0);
          acc[h2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qp[1], kb, acc[h2], 0, 0, 0);
        }
      }
    }
    float s[TH][4];
#pragma unroll
    for (int h2 = 0; h2 < TH; ++h2) {
      const bool valid = t.phys[h2] >= 0 && t0 + 16 * h2 + n < tend;
#pragma unroll
      for (int i = 0; i < 4; ++i) s[h2][i] = valid ? acc[h2][i] * p.scale_log2 : -INFINITY;
    }
    // Lazy rescaling (FlashAttention-3, Shah et al. 2024): each head row
    // keeps a reference m (log2 units; -inf until the row meets a key) that
    // moves only when a tile's row max exceeds it by more than kRefSlack, so
    // probabilities stay below 2^kRefSlack and most tiles need neither the
    // row reduction nor the output rescale: each lane checks its own scores
    // and the wavefront takes the slow path when any lane must. (An
    // all-masked tile moves nothing.)
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
        mx = Max16(mx);
        const bool mv = mx > m[i] + kRefSlack;  // the same in the row's 16 lanes
        alpha[i] = mv && m[i] != -INFINITY ? Exp2(m[i] - mx) : 1.f;
        m[i] = mv ? mx : m[i];
        lsum[i] *= alpha[i];
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float ps = 0.f;
#pragma unroll
      for (int h2 = 0; h2 < TH; ++h2) {
        s[h2][i] = m[i] == -INFINITY ? 0.f : Exp2(s[h2][i] - m[i]);
        ps += s[h2][i];
      }
      lsum[i] += ps;
    }
    if (kq < HR) {
#pragma unroll
      for (int h2 = 0; h2 < TH; ++h2)
        *reinterpret_cast<float4*>(&p_lds[(16 * h2 + n) * HP + 4 * kq]) =
            make_float4(s[h2][0], s[h2][1], s[h2][2], s[h2][3]);
    }
    ItemSync<WPI>();
    if (rescale) {
#pragma unroll
      for (int h = 0; h < GV; ++h) {
        if (h / G >= nrows) break;
        const float a = ReadLane(alpha[h & 3], 16 * (h >> 2));
        o[h][0] *= a;
        o[h][1] *= a;
      }
    }
#pragma unroll
    for (int h2 = 0; h2 < TH; ++h2) {
      if (t.phys[h2] < 0) continue;
#pragma unroll
      for (int j = 0; j < VJ; ++j) {
        const int tt = 16 * h2 + j * VT + tv;
        float v0, v1;
        VPair(t.v[h2][j], v0, v1);
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
        for (int rr = 0; rr < RMAX; ++rr) {
          if (rr >= nrows) break;
#pragma unroll
          for (int h = rr * G; h < (rr + 1) * G; ++h) {
            o[h][0] = fmaf(pv[h], v0, o[h][0]);
            o[h][1] = fmaf(pv[h], v1, o[h][1]);
          }
        }
        // Keep the broadcast probability reads next to their use: hoisting
        // a whole tile's worth would cost 8·GV registers per token.
        if ((j & 3) == 3) __builtin_amdgcn_sched_barrier(0);
      }
    }
    ItemSync<WPI>();  // p_lds is rewritten by the next tile
  };

  // A work item's range is never empty (tb < te), so the loop has no entry
  // test for the compiler to sink the Q loads behind. NBUF - 1 tiles are in
  // flight while one is computed; loads past the range are empty.
  // (For a fused item whose range is the new key alone the loop's one tile
  // is empty: every score masked, the state unchanged.)
  if constexpr (NBUF == 2) {
    // (A wavefront's run is empty only when the item has fewer tiles than
    // WPI.)
    for (int t0 = wtb; WPI == 1 || wtb < wte; t0 += 2 * TT) {
      process(bufA, t0, kend);
      if (t0 + TT >= wte) break;
      load(bufA, t0 + 2 * TT, -1);
      process(bufB, t0 + TT, kend);
      if (t0 + 2 * TT >= wte) break;
      load(bufB, t0 + 3 * TT, -1);
    }
  } else {
    for (int t0 = tb;; t0 += 3 * TT) {
      load(bufC, t0 + 2 * TT, -1);
      process(bufA, t0, kend);
      if (t0 + TT >= kend) break;
      load(bufA, t0 + 3 * TT, -1);
      process(bufB, t0 + TT, kend);
      if (t0 + 2 * TT >= kend) break;
      load(bufB, t0 + 4 * TT, -1);
      process(bufC, t0 + 2 * TT, kend);
      if (t0 + 3 * TT >= kend) break;
    }
  }
  if (fuse) {
    // The new key as a one-row tile: row 0 of the first half, from LDS.
    T tn;
#pragma unroll
    for (int h2 = 0; h2 < TH; ++h2) {
      tn.phys[h2] = h2 == 0 ? 0 : -1;
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int w = 0; w < KW; ++w)
          tn.k[h2][c][w] = (h2 == 0 && n == 0) ? knew_lds[(c * 32 + kq * 8) * ES / 16 + w]
                                               : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
      for (int j = 0; j < VJ; ++j)
        tn.v[h2][j] = (h2 == 0 && j * VT + tv == 0) ? vnew_lds[lane % VLPT] : typename T::VW{};
    }
    process(tn, newpos, te);
  }

  // Token-parallel partial sums (d = 64) -> per (virtual head, element) totals.
  if constexpr (VT > 1) {
#pragma unroll
    for (int h = 0; h < GV; ++h) {
      o[h][0] = SumAcross<VLPT>(o[h][0]);
      o[h][1] = SumAcross<VLPT>(o[h][1]);
    }
  }
  float lrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) lrow[i] = SumGroup16(lsum[i]);
  if constexpr (WPI > 1) {
    // Combine the wavefronts' states: M = max_w m_w, L = sum_w l_w 2^(m_w - M),
    // O = sum_w o_w 2^(m_w - M) per virtual head. Every wavefront reaches
    // this barrier once (one item per workgroup); wavefront 0 goes on.
    __shared__ float ml_lds[WPI][GV][2];
    __shared__ float o_lds[WPI][GV][D];
#pragma unroll
    for (int h = 0; h < GV; ++h) {
      const float mh = ReadLane(m[h & 3], 16 * (h >> 2));
      const float lh = ReadLane(lrow[h & 3], 16 * (h >> 2));
      if (lane == 0) {
        ml_lds[wv][h][0] = mh;
        ml_lds[wv][h][1] = lh;
      }
      if (lane < VLPT) *reinterpret_cast<float2*>(&o_lds[wv][h][ev]) = make_float2(o[h][0], o[h][1]);
    }
    __syncthreads();
    if (wv != 0) return;
#pragma unroll
    for (int h = 0; h < GV; ++h) {
      float mx = -INFINITY;
#pragma unroll
      for (int w = 0; w < WPI; ++w) mx = fmaxf(mx, ml_lds[w][h][0]);
      float L = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
      for (int w = 0; w < WPI; ++w) {
        const float sc = mx == -INFINITY ? 0.f : Exp2(ml_lds[w][h][0] - mx);
        L += ml_lds[w][h][1] * sc;
        const float2 ow = *reinterpret_cast<const float2*>(&o_lds[w][h][ev]);
        o0 += ow.x * sc;
        o1 += ow.y * sc;
      }
      o[h][0] = o0;
      o[h][1] = o1;
      // Back into the per-row layout the stores read: lane 16 j, slot i holds
      // virtual head 4 j + i.
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if ((h & 3) == i && (h >> 2) == kq) {
          m[i] = mx;
          lrow[i] = L;
        }
    }
  }

  RowDesc rds[RMAX];
#pragma unroll
  for (int rr = 0; rr < RMAX; ++rr) rds[rr] = ScalarRead(p.rows, it.rows[rr]);
  item_idx = first_queued + nq * static_cast<int>(__builtin_amdgcn_readfirstlane(ticket));
  if (item_idx < p.n_items) wi = ScalarRead(p.items, item_idx);
#pragma unroll
  for (int rr = 0; rr < RMAX; ++rr) {
    if (rr >= nrows) break;
    const int row = it.rows[rr];
    const RowDesc rd = rds[rr];
    if (rd.nsplit == 1) {
      if (lane < VLPT) {
        float* op = p.out + (int64_t{row} * p.heads + int64_t{hk} * G) * D + ev;
#pragma unroll
        for (int h = 0; h < G; ++h) {
          const int v = rr * G + h;
          const float inv = 1.0f / ReadLane(lrow[v & 3], 16 * (v >> 2));
          *reinterpret_cast<float2*>(op + h * D) = make_float2(o[v][0] * inv, o[v][1] * inv);
        }
      }
      continue;
    }
    const int64_t pidx = PartialIndex(rd, p.kv_heads, hk, it.split);
    if (lane < VLPT) {
      float* po = p.part_o + pidx * G * D + ev;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const int v = rr * G + h;
        *reinterpret_cast<float2*>(po + h * D) = make_float2(o[v][0], o[v][1]);
      }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const int v = rr * G + h;
      const float mh = ReadLane(m[v & 3], 16 * (v >> 2));
      const float lh = ReadLane(lrow[v & 3], 16 * (v >> 2));
      if (lane == 0) {
        p.part_ml[(pidx * G + h) * 2 + 0] = mh;
        p.part_ml[(pidx * G + h) * 2 + 1] = lh;
      }
    }
  }
  }
  if (queued && lane == 0 && atomicAdd(p.queue_done, 1u) == gridDim.x - 1) {
    for (int k = 0; k < nq; ++k) atomicExch(p.queue + k * kQueueStride, 0u);
    atomicExch(p.queue_done, 0u);
  }
}

// Workgroups of THREADS threads a launch of kernel K keeps resident: its
// occupancy per CU times the CU count, queried once per (kernel, device).
template <auto K, int THREADS = 64>
int ResidentWaves() {
  constexpr int kDevices = 64;
  static int cached[kDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < kDevices && cached[dev] > 0) return cached[dev];
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, K, THREADS, 0) != hipSuccess)
    return 0;
  if (dev >= 0 && dev < kDevices) cached[dev] = cus * per_cu;
  return cus * per_cu;
}

// Launch knobs resolved from the context's tuning switches.
struct Knobs {
  bool wide;       // 32-key tiles (two MFMA halves)
  bool deep;       // three tiles in registers
  bool persist;    // persistent wavefronts drawing items from the queue
  int32_t slots;   // cap on persistent wavefronts (0: the resident count)
  bool split4;     // fp32 steps whose items fit one round: 4 wavefronts per item
};

template <auto K>
void LaunchPersistent(const DecodeParams& p, hipStream_t stream, const Knobs& kn) {
  int grid = p.n_items;
  if (kn.persist) {
    // Tuning::decode_slots caps the grid below the resident count (tests use
    // it to make every wavefront take many items from the queue).
    int slots = ResidentWaves<K>();
    if (kn.slots > 0 && (slots <= 0 || kn.slots < slots)) slots = kn.slots;
    if (slots > 0 && slots < grid) grid = slots;
  }
  hipLaunchKernelGGL(K, dim3(grid), dim3(64), 0, stream, p);
}

template <class KV, int D, int G, int RMAX, bool FUSE>
void LaunchShape(const DecodeParams& p, hipStream_t stream, const Knobs& kn) {
  // Two wavefronts per SIMD wherever the shape fits 256 registers without
  // spilling (the 16-virtual-head and triple-buffered 128-wide shapes do not).
  constexpr bool QL = D * G * RMAX >= 1024;
  constexpr int OCC = (D == 128 && G * RMAX >= 16) ? 1 : 2;
  constexpr int OCC3 = D == 128 ? 1 : 2;
  if constexpr (sizeof(KV) == 4) {
    // fp32 slabs: the default shape only (32-key tiles, two buffers). Three
    // buffers for small steps (all items in one round of resident wavefronts,
    // one per SIMD) measured the same on C2: 23.5 against 23.6 us per layer.
    // Steps of at least 256 items that all fit one round of 4-wavefront
    // workgroups (C2's 500) spread each item over 4 wavefronts: 22.4 against
    // 22.9 us per C2 layer (interleaved calls). C2's time is the memory
    // system serving one ~35 MB burst (~3.6 TB/s: 500 wavefronts see their
    // first tile 5.4 us into the launch, 2000 see it at 10.5 us), so the
    // shorter walks gain little; C1's 16 items lost 0.7 us and keep one
    // wavefront per item.
    if constexpr (!QL) {
      constexpr auto K4 = DecodeMfma<KV, D, G, RMAX, 2, 2, QL, OCC, FUSE, 4>;
      if (kn.split4 && p.n_items >= 256 && p.n_items <= ResidentWaves<K4, 256>()) {
        hipLaunchKernelGGL(K4, dim3(p.n_items), dim3(256), 0, stream, p);
        return;
      }
    }
    LaunchPersistent<DecodeMfma<KV, D, G, RMAX, 2, 2, QL, OCC, FUSE>>(p, stream, kn);
  } else {
    if (kn.wide && kn.deep)
      LaunchPersistent<DecodeMfma<KV, D, G, RMAX, 2, 3, QL, OCC3, FUSE>>(p, stream, kn);
    else if (kn.wide)
      LaunchPersistent<DecodeMfma<KV, D, G, RMAX, 2, 2, QL, OCC, FUSE>>(p, stream, kn);
    else if (kn.deep)
      LaunchPersistent<DecodeMfma<KV, D, G, RMAX, 1, 3, QL, OCC3, FUSE>>(p, stream, kn);
    else
      LaunchPersistent<DecodeMfma<KV, D, G, RMAX, 1, 2, QL, OCC, FUSE>>(p, stream, kn);
  }
}

template <class KV, int D, int G, int RMAX>
void LaunchShape(const DecodeParams& p, hipStream_t stream, const Knobs& kn) {
  if (p.new_k != nullptr)
    LaunchShape<KV, D, G, RMAX, true>(p, stream, kn);
  else
    LaunchShape<KV, D, G, RMAX, false>(p, stream, kn);
}

// Rows per item the kernel is instantiated for: 1, 2, or 4 for groups of three
// or four sharers (the plan caps a group at 16 / g rows, so 4 only for g <= 4).
template <class KV, int D, int G>
bool LaunchRows(const DecodeParams& p, hipStream_t stream, const Knobs& kn) {
  const int rows = p.n_joint > 0 ? p.joint_rows : 1;
  if constexpr (G <= 4) {
    if (rows > 2) {
      LaunchShape<KV, D, G, 4>(p, stream, kn);
      return true;
    }
  }
  if (rows > 2) return false;
  if (rows == 2)
    LaunchShape<KV, D, G, 2>(p, stream, kn);
  else
    LaunchShape<KV, D, G, 1>(p, stream, kn);
  return true;
}

}  // namespace

bool DecodeMfmaCovers(const DecodeParams& p, int kv_dtype, const Tuning& tune) {
  const bool f32 = kv_dtype == EHIP_KV_F32;
  if (!f32 && kv_dtype != EHIP_KV_BF16) return false;
  // 16-byte K/V vectors: bf16 rows start on 8-element, fp32 on 4-element
  // multiples of the slab base.
  const int64_t vec = f32 ? 4 : 8;
  const bool aligned = (reinterpret_cast<uintptr_t>(p.k_slab) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.v_slab) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.q) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(p.out) % 16 == 0) &&
                       (p.block_stride % vec == 0) && (p.head_stride % vec == 0);
  // fp32: head_dim 64 (the 128-wide fp32 tiles would not fit two wavefronts
  // per SIMD) and g in {1, 2, 4, 7, 8}; bf16: head_dim 64 or 128, g in {1, 2, 4, 8}.
  const bool shape = f32 ? (p.d == 64 && (p.group == 1 || p.group == 2 || p.group == 4 ||
                                          p.group == 7 || p.group == 8))
                         : ((p.d == 64 || p.d == 128) &&
                            (p.group == 1 || p.group == 2 || p.group == 4 || p.group == 8));
  return aligned && shape && p.bs >= 16 && !tune.decode_valu;
}

bool LaunchDecodeMfma(const DecodeParams& params, int kv_dtype, const Tuning& tune,
                      QueueState* queue, hipStream_t stream, hipError_t* err) {
  DecodeParams p = params;
  p.queue = queue->d_counters;
  p.queue_done = queue->d_done;
  p.queue_spread = tune.decode_qspread ? 1 : 0;
  p.queues = tune.decode_queues > 0 ? std::min(tune.decode_queues, kItemQueues) : kDefaultQueues;
  if (!DecodeMfmaCovers(p, kv_dtype, tune)) return false;
  // 32-token tiles (two MFMA halves per tile, double-buffered) measured best
  // on C4; decode_tile16 selects one half per tile (fewer registers),
  // decode_bufs3 three tiles in registers (two in flight), and
  // decode_persist = false one workgroup per item (the hardware dispatcher
  // hands out the items instead of the queue).
  const Knobs kn{!tune.decode_tile16, tune.decode_bufs3, tune.decode_persist, tune.decode_slots,
                 tune.decode_split4};
  bool ok = false;
#define EHIP_MFMA_CASE(KV, DD, GG) \
  else if (p.d == DD && p.group == GG) ok = LaunchRows<KV, DD, GG>(p, stream, kn);
  if (kv_dtype == EHIP_KV_F32) {
    if (false) {
    }
    EHIP_MFMA_CASE(float, 64, 1)
    EHIP_MFMA_CASE(float, 64, 2)
    EHIP_MFMA_CASE(float, 64, 4)
    EHIP_MFMA_CASE(float, 64, 7)
    EHIP_MFMA_CASE(float, 64, 8)
  } else {
    if (false) {
    }
    EHIP_MFMA_CASE(uint16_t, 128, 1)
    EHIP_MFMA_CASE(uint16_t, 128, 2)
    EHIP_MFMA_CASE(uint16_t, 128, 4)
    EHIP_MFMA_CASE(uint16_t, 128, 8)
    EHIP_MFMA_CASE(uint16_t, 64, 1)
    EHIP_MFMA_CASE(uint16_t, 64, 2)
    EHIP_MFMA_CASE(uint16_t, 64, 4)
    EHIP_MFMA_CASE(uint16_t, 64, 8)
  }
#undef EHIP_MFMA_CASE
  if (ok) *err = hipGetLastError();
  return ok;
}

}  // namespace ehip
