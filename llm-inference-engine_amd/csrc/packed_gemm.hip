// The attention output's consumer: the packed linear layer (o_proj) on the
// gfx950 matrix cores.
//
// Semantics: kernels::PackedGemm (src/kernels/gemm.h): y[m, n] = x[m, k] W^T
// (+ bias[n]) with fp32 activations, weights stored fp32, fp16 or bf16 in the
// reference's panel layout Wp[p, k, r] = W[p*16 + r, k] (zero past n), fp32
// accumulation, and the bias added once after the k sum
// (src/kernels/internal/gemm_common.h:22-41).
//
// Matrix-core form: every operand is cut into bf16 planes whose sum is the
// value. x (fp32) takes three (x = x0 + x1 + x2, each the RNE bf16 of what the
// earlier ones leave: about 2^-24 relative). Weights take as many as their
// type needs to be exact: one for bf16, two for fp16 (11 significant bits,
// inside bf16's exponent range), three for fp32. The products x_i W_j with
// i + j <= 2 run on v_mfma_f32_16x16x32_bf16, smallest first; the ones left
// out are below 2^-24 of |x||w| per term. A bf16 weight therefore costs three
// MFMAs per 32-k chunk and block, fp16 five, fp32 six.
//
// x is cut into its planes once per call by a pre-pass (SplitRows) that
// writes them zero-padded to whole 64 x 64 tiles, so every column tile reads
// ready operands instead of re-cutting x.
//
// Work: one workgroup of 4 wavefronts per (64 rows, BP panels, k range):
// BP = 16 (256 columns) for bf16 weights, 8 (128) for fp16 and fp32. Each k
// step of 64 stages x's three planes (rows padded to 72 elements so the 16
// lanes of an A-operand read hit distinct banks) and the panels' 64 rows (as
// the weight's planes, the panel layout as stored) in LDS; the next step's
// global loads are in flight meanwhile. A wavefront owns 32 rows x BP/2
// panels: 2 x BP/2 blocks of 16 x 16. The A operand of
// lane (n, q) is row n at k = 4q..4q+3 and 16+4q..16+4q+3 (two 8-byte reads);
// the B operand is the same k set of panel column n, read with
// ds_read_b64_tr_b16 from the [k][16] panel rows.
//
// Decode-shaped calls (few rows) have few tiles: the k range is then split
// over workgroups, each writing its fp32 partial block, and a second kernel
// adds the partials in split order, then the bias. Every output element is
// the same sums in the same order on every call: results are deterministic.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.h"

namespace ehip {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int kNr = 16;     // the reference's panel width (kernels::kNr)
constexpr int kBM = 64;     // rows per workgroup
constexpr int kBK = 64;     // k per step (two 32-k MFMA chunks)
constexpr int kXP = 3;      // bf16 planes of x
constexpr int kXRow = 72;   // bf16 elements per LDS row of an x plane (64 + 8)
constexpr int kThreads = 256;

template <int WT>
struct WeightType;
template <>
struct WeightType<EHIP_WEIGHT_F32> {
  using T = float;
  static constexpr int WP = 3;
};
template <>
struct WeightType<EHIP_WEIGHT_BF16> {
  using T = uint16_t;
  static constexpr int WP = 1;
};
template <>
struct WeightType<EHIP_WEIGHT_F16> {
  using T = uint16_t;
  static constexpr int WP = 2;
};

// A stored weight as fp32: exact for all three types (the reference's
// widening, src/tensor/half.h:84-109, :126-129).
template <int WT>
__device__ __forceinline__ float Widen(typename WeightType<WT>::T v) {
  if constexpr (WT == EHIP_WEIGHT_F32) {
    return v;
  } else if constexpr (WT == EHIP_WEIGHT_BF16) {
    return __uint_as_float(static_cast<uint32_t>(v) << 16);
  } else {
    return static_cast<float>(__builtin_bit_cast(_Float16, v));
  }
}

// v as P bf16 planes: plane i is the round-to-nearest-even bf16 of what the
// earlier planes leave.
template <int P>
__device__ __forceinline__ void Planes(float v, __bf16 (&out)[P]) {
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const __bf16 b = static_cast<__bf16>(v);
    out[i] = b;
    v -= static_cast<float>(b);
  }
}

// ds_read_b64_tr_b16: lane i of each 16-lane group receives element i % 4 of
// the 8 bytes addressed by lanes 4j + i / 4 of the group, for j = 0..3.
__device__ __forceinline__ bf16x4_t TransposedRead(const __bf16* p) {
  typedef __attribute__((ext_vector_type(4))) short s16x4_t;
  const s16x4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4_t*)(p));
  return __builtin_bit_cast(bf16x4_t, r);
}

template <int WT, int BP>
__global__ __launch_bounds__(kThreads) void PackedGemmMfma(GemmParams p) {
  using W = WeightType<WT>;
  using T = typename W::T;
  constexpr int WP = W::WP;
  constexpr int WE = 16 * static_cast<int>(sizeof(T)) / 16;  // 16-byte loads per panel row
  constexpr int kBP = BP;
  constexpr int NW = kBP / 2;          // panels per wavefront
  constexpr int KS = kThreads / kBP;   // threads per panel in the loads (k-row stride)
  constexpr int RPT = kBK / KS;        // panel rows a thread loads per step

  __shared__ __align__(16) __bf16 xs[kXP][kBM * kXRow];
  __shared__ __align__(16) __bf16 ws[WP][kBP * kBK * kNr];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n16 = lane & 15;
  const int q = lane >> 4;
  const int wr = wave >> 1;  // rows 32*wr .. +32 of the tile
  const int wc = wave & 1;   // panels NW*wc .. +NW of the tile
  const int64_t m0 = int64_t{blockIdx.y} * kBM;
  const int pb = static_cast<int>(blockIdx.x) * kBP;
  const int split = blockIdx.z;
  const int64_t kb = int64_t{split} * p.k_split;
  const int64_t ke = kb + p.k_split < p.k ? kb + p.k_split : p.k;

  // Global loads: 16 consecutive k from xk of x row xr in each plane (the
  // planes are zero-padded to whole tiles: no masks); panel rows wk and
  // wk + KS, ... (16 weights each) of panel wpp.
  const int xr = tid >> 2, xk = (tid & 3) * 16;
  // A tile's rows past m are never stored, and each output row depends on its
  // own x row only, so the x rows of wholly dead 32-row halves (a decode
  // call's m <= 32 in a 64-row tile) are neither loaded nor computed: x's
  // L2 -> CU traffic and the MFMA work halve there. Whether a thread's row
  // (and a wavefront's half) is live is uniform per wavefront.
  const int rows_live = static_cast<int>(p.m - m0 < kBM ? p.m - m0 : kBM);
  const bool x_live = (xr & ~31) < rows_live;
  const bool wave_live = 32 * wr < rows_live;
  const int64_t plane = p.m_pad * p.k_pad;
  const __bf16* xrow = reinterpret_cast<const __bf16*>(p.xp) + (m0 + xr) * p.k_pad;
  const int wpp = tid / KS, wk = tid % KS;  // panel wpp, k rows wk + KS * h
  const bool w_ok = pb + wpp < p.panels;
  const T* wpanel = static_cast<const T*>(p.wp) + (w_ok ? int64_t{pb + wpp} * p.k * kNr : 0);

  bf16x8_t xv[kXP][2];
  uint4 wv[RPT][WE];
  auto gload = [&](int64_t k0) {
    if (x_live) {
#pragma unroll
      for (int pl = 0; pl < kXP; ++pl)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          xv[pl][h] = *reinterpret_cast<const bf16x8_t*>(xrow + pl * plane + k0 + xk + 8 * h);
    }
#pragma unroll
    for (int h = 0; h < RPT; ++h) {
      const int64_t kw = k0 + wk + KS * h;
      const bool ok = w_ok && kw < ke;
      const uint4* src = reinterpret_cast<const uint4*>(wpanel + (ok ? kw : 0) * kNr);
#pragma unroll
      for (int i = 0; i < WE; ++i) wv[h][i] = ok ? src[i] : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto lstore = [&]() {
    if (x_live) {
#pragma unroll
      for (int pl = 0; pl < kXP; ++pl)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          *reinterpret_cast<bf16x8_t*>(&xs[pl][xr * kXRow + xk + 8 * h]) = xv[pl][h];
    }
    // Each panel row as WP planes: 16 weights, two 16-byte stores per plane.
#pragma unroll
    for (int hr = 0; hr < RPT; ++hr) {
      const T* w = reinterpret_cast<const T*>(wv[hr]);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        bf16x8_t wpl[WP];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if constexpr (WT == EHIP_WEIGHT_BF16) {
            wpl[0][i] = __builtin_bit_cast(__bf16, w[8 * h + i]);
          } else {
            __bf16 parts[WP];
            Planes<WP>(Widen<WT>(w[8 * h + i]), parts);
#pragma unroll
            for (int pl = 0; pl < WP; ++pl) wpl[pl][i] = parts[pl];
          }
        }
#pragma unroll
        for (int pl = 0; pl < WP; ++pl)
          *reinterpret_cast<bf16x8_t*>(&ws[pl][(wpp * kBK + wk + KS * hr) * kNr + 8 * h]) =
              wpl[pl];
      }
    }
  };

  f32x4_t acc[2][NW];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int cb = 0; cb < NW; ++cb) acc[rb][cb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&]() {
    if (!wave_live) return;
#pragma unroll
    for (int kc = 0; kc < kBK / 32; ++kc) {
    bf16x8_t a[2][kXP];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int row = 32 * wr + 16 * rb + n16;
#pragma unroll
      for (int pl = 0; pl < kXP; ++pl) {
        const __bf16* base = &xs[pl][row * kXRow + 32 * kc];
        const bf16x4_t lo = *reinterpret_cast<const bf16x4_t*>(base + 4 * q);
        const bf16x4_t hi = *reinterpret_cast<const bf16x4_t*>(base + 16 + 4 * q);
        a[rb][pl] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    }
#pragma unroll
    for (int cb = 0; cb < NW; ++cb) {
      const int panel = NW * wc + cb;
      bf16x8_t b[WP];
#pragma unroll
      for (int pl = 0; pl < WP; ++pl) {
        const __bf16* base =
            &ws[pl][(panel * kBK + 32 * kc + 4 * q + (n16 >> 2)) * kNr + 4 * (n16 & 3)];
        const bf16x4_t lo = TransposedRead(base);
        const bf16x4_t hi = TransposedRead(base + 16 * kNr);
        b[pl] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        // Products x_i W_j with i + j <= 2, smallest first.
#pragma unroll
        for (int s = 2; s >= 0; --s)
#pragma unroll
          for (int j = 0; j < WP; ++j) {
            const int i = s - j;
            if (i >= 0 && i < kXP)
              acc[rb][cb] =
                  __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[rb][i], b[j], acc[rb][cb], 0, 0, 0);
          }
      }
    }
    }
  };

  gload(kb);
  for (int64_t k0 = kb; k0 < ke; k0 += kBK) {
    __syncthreads();  // the previous step's operand reads are done
    lstore();
    __syncthreads();
    if (k0 + kBK < ke) gload(k0 + kBK);
    compute();
  }

  // acc[rb][cb][i] = y[row 32wr + 16rb + 4q + i][column of panel NW wc + cb, n16].
#pragma unroll
  for (int cb = 0; cb < NW; ++cb) {
    const int64_t col = int64_t{pb + NW * wc + cb} * kNr + n16;
    if (col >= p.n) continue;
    const float bias = (p.splits == 1 && p.bias) ? p.bias[col] : 0.f;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t row = m0 + 32 * wr + 16 * rb + 4 * q + i;
        if (row >= p.m) continue;
        if (p.splits == 1)
          p.y[row * p.n + col] = acc[rb][cb][i] + bias;
        else
          p.part[(int64_t{split} * p.m + row) * p.n + col] = acc[rb][cb][i];
      }
  }
}

// x [m, k] fp32 -> its three bf16 planes [3][m_pad][k_pad], zero past m and
// k; one thread per 8 consecutive elements of a padded row.
__global__ __launch_bounds__(256) void SplitRows(GemmParams p, __bf16* xp) {
  const int64_t groups = p.m_pad * (p.k_pad / 8);
  const int64_t g = int64_t{blockIdx.x} * 256 + threadIdx.x;
  if (g >= groups) return;
  const int64_t row = g / (p.k_pad / 8);
  const int64_t k0 = (g - row * (p.k_pad / 8)) * 8;
  float v[8];
  if (p.x_vec && row < p.m && k0 + 8 <= p.k) {
    const float4 a = *reinterpret_cast<const float4*>(p.x + row * p.k + k0);
    const float4 b = *reinterpret_cast<const float4*>(p.x + row * p.k + k0 + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (row < p.m && k0 + i < p.k) ? p.x[row * p.k + k0 + i] : 0.f;
  }
  bf16x8_t out[kXP];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    __bf16 parts[kXP];
    Planes<kXP>(v[i], parts);
#pragma unroll
    for (int pl = 0; pl < kXP; ++pl) out[pl][i] = parts[pl];
  }
  const int64_t plane = p.m_pad * p.k_pad;
#pragma unroll
  for (int pl = 0; pl < kXP; ++pl)
    *reinterpret_cast<bf16x8_t*>(xp + pl * plane + row * p.k_pad + k0) = out[pl];
}

// y = (partial 0 + partial 1 + ...) in split order, then + bias.
__global__ __launch_bounds__(256) void GemmSplitReduce(GemmParams p) {
  const int64_t total = p.m * p.n;
  const int64_t i = int64_t{blockIdx.x} * 256 + threadIdx.x;
  if (i >= total) return;
  float s = p.part[i];
  for (int sp = 1; sp < p.splits; ++sp) s += p.part[int64_t{sp} * total + i];
  if (p.bias) s += p.bias[i % p.n];
  p.y[i] = s;
}

// Wp[p, kk, r] = W[p*16 + r, kk] (0 past n): the reference's PackWeightPanels
// (src/kernels/gemm.h), one thread per (panel, k) row of 16.
template <class T>
__global__ __launch_bounds__(256) void PackPanels(const T* w, int64_t n, int64_t k, T* wp) {
  const int64_t panels = (n + kNr - 1) / kNr;
  const int64_t i = int64_t{blockIdx.x} * 256 + threadIdx.x;
  if (i >= panels * k) return;
  const int64_t pnl = i / k, kk = i - pnl * k;
  T* out = wp + i * kNr;
#pragma unroll
  for (int r = 0; r < kNr; ++r) {
    const int64_t row = pnl * kNr + r;
    out[r] = row < n ? w[row * k + kk] : T{};
  }
}

}  // namespace

void PlanPackedGemm(int64_t m, int64_t k, int64_t n, int weight_dtype, int cus, GemmParams* p) {
  // 16 panels (256 columns) per workgroup for bf16 weights and up to 256
  // rows: each x row is then staged for twice the columns (C4 o_proj 58.5 ->
  // 56 us, C5 63 -> 60 us). Taller calls keep 8 (C3's 2382 rows: 350 against
  // 365 us at 16), as do fp16 and fp32 weights, whose two or three weight
  // planes would not fit LDS at 16.
  const int kBP = (weight_dtype == EHIP_WEIGHT_BF16 && m <= 256) ? 16 : 8;
  p->group_panels = kBP;
  p->m = m;
  p->k = k;
  p->n = n;
  p->m_pad = (m + kBM - 1) / kBM * kBM;
  p->k_pad = (k + kBK - 1) / kBK * kBK;
  p->panels = (n + kNr - 1) / kNr;
  const int64_t tiles = ((m + kBM - 1) / kBM) * ((p->panels + kBP - 1) / kBP);
  const int64_t steps = (k + kBK - 1) / kBK;
  // Enough workgroups for one round at the tile's occupancy (two per CU for
  // the 256-column tile, about four otherwise: a workgroup keeps one step of
  // loads in flight, so the chip's share of them sets the bandwidth); each
  // split keeps at least 2 steps.
  const int64_t per_cu = kBP == 16 ? 2 : 4;
  int64_t splits = (per_cu * int64_t{cus} + tiles - 1) / tiles;
  splits = splits < 1 ? 1 : splits;
  const int64_t max_splits = steps / 2 > 1 ? steps / 2 : 1;
  splits = splits > max_splits ? max_splits : splits;
  splits = splits > 64 ? 64 : splits;
  const int64_t per = (steps + splits - 1) / splits;
  p->k_split = per * kBK;
  p->splits = static_cast<int32_t>((steps + per - 1) / per);
}

size_t PackedGemmPlaneBytes(const GemmParams& p) {
  return static_cast<size_t>(kXP) * static_cast<size_t>(p.m_pad) * static_cast<size_t>(p.k_pad) *
         sizeof(uint16_t);
}

hipError_t LaunchPackedGemm(const GemmParams& p, int weight_dtype, hipStream_t stream) {
  {
    const int64_t groups = p.m_pad * (p.k_pad / 8);
    hipLaunchKernelGGL(SplitRows, dim3(static_cast<uint32_t>((groups + 255) / 256)), dim3(256), 0,
                       stream, p, reinterpret_cast<__bf16*>(p.xp));
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  }
  const dim3 grid(static_cast<uint32_t>((p.panels + p.group_panels - 1) / p.group_panels),
                  static_cast<uint32_t>((p.m + kBM - 1) / kBM), static_cast<uint32_t>(p.splits));
  switch (weight_dtype) {
    case EHIP_WEIGHT_F32:
      hipLaunchKernelGGL((PackedGemmMfma<EHIP_WEIGHT_F32, 8>), grid, dim3(kThreads), 0, stream, p);
      break;
    case EHIP_WEIGHT_BF16:
      if (p.group_panels == 16)
        hipLaunchKernelGGL((PackedGemmMfma<EHIP_WEIGHT_BF16, 16>), grid, dim3(kThreads), 0, stream,
                           p);
      else
        hipLaunchKernelGGL((PackedGemmMfma<EHIP_WEIGHT_BF16, 8>), grid, dim3(kThreads), 0, stream,
                           p);
      break;
    case EHIP_WEIGHT_F16:
      hipLaunchKernelGGL((PackedGemmMfma<EHIP_WEIGHT_F16, 8>), grid, dim3(kThreads), 0, stream, p);
      break;
    default:
      return hipErrorInvalidValue;
  }
  if (hipError_t e = hipGetLastError(); e != hipSuccess || p.splits == 1) return e;
  const int64_t total = p.m * p.n;
  hipLaunchKernelGGL(GemmSplitReduce, dim3(static_cast<uint32_t>((total + 255) / 256)), dim3(256),
                     0, stream, p);
  return hipGetLastError();
}

hipError_t LaunchPackWeightPanels(const void* w, int weight_dtype, int64_t n, int64_t k, void* wp,
                                  hipStream_t stream) {
  const int64_t rows = (n + kNr - 1) / kNr * k;
  const dim3 grid(static_cast<uint32_t>((rows + 255) / 256));
  if (weight_dtype == EHIP_WEIGHT_F32)
    hipLaunchKernelGGL(PackPanels<float>, grid, dim3(256), 0, stream, static_cast<const float*>(w),
                       n, k, static_cast<float*>(wp));
  else
    hipLaunchKernelGGL(PackPanels<uint16_t>, grid, dim3(256), 0, stream,
                       static_cast<const uint16_t*>(w), n, k, static_cast<uint16_t*>(wp));
  return hipGetLastError();
}

}  // namespace ehip
