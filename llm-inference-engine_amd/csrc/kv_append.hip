// KV append (scatter), gather and synthetic fills for gfx950.
//
// Scatter semantics: kernels::KvScatterF32 (src/kernels/kv_scatter.cpp:27-61):
// token t's row for kv head h (src + (t*Hkv + h)*d) lands at slot
// s = slot_mapping[t], block s / bs, row s % bs, i.e. slab element
// ((block*Hkv + h)*bs + s % bs)*d. A pure copy (fp32) or the reference's
// round-to-nearest-even narrowing (bf16), so the result is bit-exact.
//
// One thread moves one 16-byte source vector (4 floats) of one (token, head)
// row; consecutive threads cover consecutive source bytes, so reads are fully
// coalesced and each row's destination is a contiguous 4*d (or 2*d) bytes.
#include "device_util.h"
#include "kernels.h"

namespace ehip {
namespace {

template <class KV>
__device__ __forceinline__ void Store4(KV* dst, float4 x);
template <>
__device__ __forceinline__ void Store4<float>(float* dst, float4 x) {
  *reinterpret_cast<float4*>(dst) = x;
}
template <>
__device__ __forceinline__ void Store4<uint16_t>(uint16_t* dst, float4 x) {
  uint2 w;
  w.x = Fp32ToBf16Bits(x.x) | (Fp32ToBf16Bits(x.y) << 16);
  w.y = Fp32ToBf16Bits(x.z) | (Fp32ToBf16Bits(x.w) << 16);
  *reinterpret_cast<uint2*>(dst) = w;
}

__device__ __forceinline__ void Store1(float* dst, float x) { *dst = x; }
__device__ __forceinline__ void Store1(uint16_t* dst, float x) {
  *dst = static_cast<uint16_t>(Fp32ToBf16Bits(x));
}
// E4M3 code of x saturated to +-448 (v_cvt_pk_fp8_f32 rounds to nearest even).
__device__ __forceinline__ void Store1(uint8_t* dst, float x) {
  const float c = fminf(fmaxf(x, -448.0f), 448.0f);
  *dst = static_cast<uint8_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c, c, 0, false) & 0xFF);
}

// d % 4 == 0 path.
template <class KV>
__global__ __launch_bounds__(256) void KvScatterVec(const float* __restrict__ src_k,
                                                    const float* __restrict__ src_v,
                                                    const int64_t* __restrict__ slots,
                                                    int64_t n_vec, int kv_heads, int d, int bs,
                                                    int64_t slab_blocks, KV* k_slab, KV* v_slab,
                                                    int32_t* err) {
  const int vpr = d >> 2;  // vectors per (token, head) row
  for (int64_t i = blockIdx.x * int64_t{blockDim.x} + threadIdx.x; i < n_vec;
       i += int64_t{gridDim.x} * blockDim.x) {
    const int64_t row = i / vpr;  // token * Hkv + head
    const int e = static_cast<int>(i - row * vpr) << 2;
    const int64_t t = row / kv_heads;
    const int h = static_cast<int>(row - t * kv_heads);
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= slab_blocks * bs) {
      atomicOr(err, kErrSlotRange);
      continue;
    }
    const int64_t block = slot / bs;
    const int64_t pos = slot - block * bs;
    const int64_t dst = ((block * kv_heads + h) * bs + pos) * d + e;
    const float4 kx = *reinterpret_cast<const float4*>(src_k + row * d + e);
    const float4 vx = *reinterpret_cast<const float4*>(src_v + row * d + e);
    Store4<KV>(k_slab + dst, kx);
    Store4<KV>(v_slab + dst, vx);
  }
}

template <class KV>
__global__ __launch_bounds__(256) void KvScatterScalar(const float* __restrict__ src_k,
                                                       const float* __restrict__ src_v,
                                                       const int64_t* __restrict__ slots,
                                                       int64_t n, int kv_heads, int d, int bs,
                                                       int64_t slab_blocks, KV* k_slab,
                                                       KV* v_slab, int32_t* err) {
  for (int64_t i = blockIdx.x * int64_t{blockDim.x} + threadIdx.x; i < n;
       i += int64_t{gridDim.x} * blockDim.x) {
    const int64_t row = i / d;
    const int e = static_cast<int>(i - row * d);
    const int64_t t = row / kv_heads;
    const int h = static_cast<int>(row - t * kv_heads);
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= slab_blocks * bs) {
      atomicOr(err, kErrSlotRange);
      continue;
    }
    const int64_t block = slot / bs;
    const int64_t pos = slot - block * bs;
    const int64_t dst = ((block * kv_heads + h) * bs + pos) * d + e;
    Store1(k_slab + dst, src_k[i]);
    Store1(v_slab + dst, src_v[i]);
  }
}

// Fused RoPE + KV append for the rows of one step: kernels::RopeApplyF32
// (src/kernels/rope.h:13-36, HF half rotation) on q in place and on each
// appended K row on its way into the slab (src/model/optimized_model.cpp
// applies RoPE to q and k, then PagedKvCache::append scatters k and v).
// Row r sits at position rows[r].length - 1. The pair (x[j], x[j + d/2]) is
// rotated as the reference's AVX2 row kernel does it:
//   out[j]       = fma(-x[j + d/2], sin, x[j] * cos)
//   out[j + d/2] = fma(x[j], sin, x[j + d/2] * cos)
// for the pairs in whole groups of 8, and as the compiled scalar tail of that
// kernel, fma(x[j], cos, -(x[j + d/2] * sin)) and fma(x[j + d/2], cos,
// x[j] * sin), for the rest, so q and the K slab match the reference
// bit for bit (the bf16 slab after its round-to-nearest-even). One thread handles W
// consecutive pairs of one (row, head): heads [0, H) are q, [H, H + Hkv) the
// k/v rows, whose v is copied unrotated. The source K rows are left as they
// were (the rotated rows live in the slab).
template <int W>
struct Pairs {
  float v[W];
};

template <int W>
__device__ __forceinline__ Pairs<W> LoadPairs(const float* p) {
  Pairs<W> r;
  if constexpr (W == 4) {
    const float4 x = *reinterpret_cast<const float4*>(p);
    r.v[0] = x.x, r.v[1] = x.y, r.v[2] = x.z, r.v[3] = x.w;
  } else {
#pragma unroll
    for (int w = 0; w < W; ++w) r.v[w] = p[w];
  }
  return r;
}

template <int W>
__device__ __forceinline__ void StorePairs(float* p, const Pairs<W>& r) {
  if constexpr (W == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(r.v[0], r.v[1], r.v[2], r.v[3]);
  } else {
#pragma unroll
    for (int w = 0; w < W; ++w) p[w] = r.v[w];
  }
}

template <class KV, int W>
__device__ __forceinline__ void StorePairs(KV* p, const Pairs<W>& r) {
  if constexpr (W == 4) {
    Store4<KV>(p, make_float4(r.v[0], r.v[1], r.v[2], r.v[3]));
  } else {
#pragma unroll
    for (int w = 0; w < W; ++w) Store1(p + w, r.v[w]);
  }
}

// Grid: x = query row (its position, slot and table entry are wavefront-
// uniform), y strides over the row's (head, pair group) items.
template <class KV, int W>
__global__ __launch_bounds__(256) void RopeKvAppend(
    float* __restrict__ q, const float* __restrict__ src_k, const float* __restrict__ src_v,
    const RowDesc* __restrict__ rows, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, const int64_t* __restrict__ slots, int heads, int kv_heads,
    int d, int bs, int64_t slab_blocks, KV* k_slab, KV* v_slab, int32_t* err) {
  const int half = d >> 1;
  const int fused = half & ~7;  // pairs the AVX2 kernel handles 8 at a time
  const int gpr = half / W;     // pair groups per head row
  const int per_row = (heads + kv_heads) * gpr;
  const int64_t r = blockIdx.x;
  const int64_t p = rows[r].length - 1;
  const int64_t slot = slots[r];
  for (int rem = blockIdx.y * blockDim.x + threadIdx.x; rem < per_row;
       rem += gridDim.y * blockDim.x) {
    const int hh = rem / gpr;
    const int j = (rem - hh * gpr) * W;
    const bool is_q = hh < heads;
    const float* x = is_q ? q + (r * heads + hh) * d : src_k + (r * kv_heads + (hh - heads)) * d;
    const Pairs<W> lo = LoadPairs<W>(x + j), hi = LoadPairs<W>(x + j + half);
    const Pairs<W> c = LoadPairs<W>(cos_t + p * half + j), s = LoadPairs<W>(sin_t + p * half + j);
    Pairs<W> ro, rh;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      if (j + w < fused) {
        ro.v[w] = fmaf(-hi.v[w], s.v[w], lo.v[w] * c.v[w]);
        rh.v[w] = fmaf(lo.v[w], s.v[w], hi.v[w] * c.v[w]);
      } else {
        ro.v[w] = fmaf(lo.v[w], c.v[w], -(hi.v[w] * s.v[w]));
        rh.v[w] = fmaf(hi.v[w], c.v[w], lo.v[w] * s.v[w]);
      }
    }
    if (is_q) {
      float* xq = q + (r * heads + hh) * d;
      StorePairs<W>(xq + j, ro);
      StorePairs<W>(xq + j + half, rh);
      continue;
    }
    const int h = hh - heads;
    if (slot < 0 || slot >= slab_blocks * bs) {
      atomicOr(err, kErrSlotRange);
      continue;
    }
    const int64_t block = slot / bs;
    const int64_t dst = ((block * kv_heads + h) * bs + (slot - block * bs)) * d;
    const float* xv = src_v + (r * kv_heads + h) * d;
    StorePairs<KV, W>(k_slab + dst + j, ro);
    StorePairs<KV, W>(k_slab + dst + j + half, rh);
    StorePairs<KV, W>(v_slab + dst + j, LoadPairs<W>(xv + j));
    StorePairs<KV, W>(v_slab + dst + j + half, LoadPairs<W>(xv + j + half));
  }
}

// INT8 / FP8 append with per-(block, kv head) scales. One wavefront per
// (append group, kv head): the group's rows land at consecutive offsets
// [off0, off0 + n) of one block. For K, then V: m = max |x| over the new rows;
// the stored scale counts only when off0 > 0 (offset 0 is a freshly allocated
// block, whatever an earlier owner left); if m exceeds R times that scale (R =
// 127 for int8, 448 for E4M3), the scale becomes m / R and the block's older
// rows are requantised. Each value is quant(x, s) = 0 if s == 0, else the code
// of y = x * (1 / s): int8 clamp(rint(y), -127, 127); E4M3 of clamp(y, -448,
// 448) rounded to nearest even (v_cvt_pk_fp8_f32 is exact RNE there), NaN
// giving 0x7F. All in fp32 with round-to-nearest-even, so the slabs and
// scales are bit-identical to the CPU restatement. Lanes handle 4 consecutive
// elements (d % 4 == 0).
__device__ __forceinline__ int32_t Q8(float x, float inv, bool zero) {
  if (zero) return 0;
  const float y = fminf(fmaxf(rintf(x * inv), -127.0f), 127.0f);
  return static_cast<int32_t>(y);
}

__device__ __forceinline__ uint32_t Pack4(int32_t a, int32_t b, int32_t c, int32_t e) {
  return (static_cast<uint32_t>(a) & 0xFFu) | ((static_cast<uint32_t>(b) & 0xFFu) << 8) |
         ((static_cast<uint32_t>(c) & 0xFFu) << 16) | (static_cast<uint32_t>(e) << 24);
}

// Four E4M3 codes of x * inv (zero: all 0).
__device__ __forceinline__ uint32_t PackF8(float4 x, float inv, bool zero) {
  const float y[4] = {x.x * inv, x.y * inv, x.z * inv, x.w * inv};
  float c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = fminf(fmaxf(y[i], -448.0f), 448.0f);
  uint32_t w = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c[0], c[1], 0, false));
  w = static_cast<uint32_t>(
      __builtin_amdgcn_cvt_pk_fp8_f32(c[2], c[3], static_cast<int>(w), true));
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (y[i] != y[i]) w = (w & ~(0xFFu << (8 * i))) | (0x7Fu << (8 * i));
  return zero ? 0u : w;
}

// The four values a stored word holds, times s.
template <bool F8>
__device__ __forceinline__ float4 Unpack4(uint32_t w, float s) {
  if constexpr (F8) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
    return make_float4(lo[0] * s, lo[1] * s, hi[0] * s, hi[1] * s);
  } else {
    return make_float4(static_cast<float>(static_cast<int8_t>(w)) * s,
                       static_cast<float>(static_cast<int8_t>(w >> 8)) * s,
                       static_cast<float>(static_cast<int8_t>(w >> 16)) * s,
                       static_cast<float>(static_cast<int8_t>(w >> 24)) * s);
  }
}

template <bool F8>
__device__ __forceinline__ uint32_t Quant4(float4 x, float inv, bool zero) {
  if constexpr (F8)
    return PackF8(x, inv, zero);
  else
    return Pack4(Q8(x.x, inv, zero), Q8(x.y, inv, zero), Q8(x.z, inv, zero), Q8(x.w, inv, zero));
}

template <bool F8>
__global__ __launch_bounds__(64) void AppendQ8(const float* __restrict__ src_k,
                                               const float* __restrict__ src_v,
                                               const Q8Group* __restrict__ groups,
                                               const int32_t* __restrict__ rows, int kv_heads,
                                               int d, int bs, int64_t slab_blocks,
                                               uint8_t* k_slab, uint8_t* v_slab, float* k_scale,
                                               float* v_scale, int32_t* err) {
  constexpr float kRange = F8 ? 448.0f : 127.0f;
  const int gi = blockIdx.x / kv_heads;
  const int h = blockIdx.x - gi * kv_heads;
  const int lane = threadIdx.x;
  const Q8Group gr = groups[gi];
  if (gr.block < 0 || gr.block >= slab_blocks || gr.off0 < 0 || gr.off0 + gr.n > bs) {
    if (lane == 0) atomicOr(err, kErrSlotRange);
    return;
  }
  const int64_t tile = (int64_t{gr.block} * kv_heads + h) * bs * d;
  const int d4 = d >> 2;
  const int ne4 = gr.n * d4;
  for (int which = 0; which < 2; ++which) {
    const float* src = which ? src_v : src_k;
    uint32_t* dst = reinterpret_cast<uint32_t*>((which ? v_slab : k_slab) + tile);
    float* sc = (which ? v_scale : k_scale) + int64_t{gr.block} * kv_heads + h;
    auto src4 = [&](int i) {
      const int r = rows[gr.row0 + i / d4];
      return *reinterpret_cast<const float4*>(src + (int64_t{r} * kv_heads + h) * d +
                                              (i % d4) * 4);
    };
    float m = 0.f;
    for (int i = lane; i < ne4; i += 64) {
      const float4 x = src4(i);
      m = fmaxf(m, fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w))));
    }
    m = WaveMax(m);
    const float s0 = gr.off0 > 0 ? *sc : 0.f;
    float s1 = s0;
    if (m > s0 * kRange) {
      s1 = m / kRange;
      const float inv = 1.0f / s1;
      const bool zero = s1 == 0.0f;
      for (int i = lane; i < gr.off0 * d4; i += 64)
        dst[i] = Quant4<F8>(Unpack4<F8>(dst[i], s0), inv, zero);
    }
    const float inv = 1.0f / s1;
    const bool zero = s1 == 0.0f;
    for (int i = lane; i < ne4; i += 64) dst[gr.off0 * d4 + i] = Quant4<F8>(src4(i), inv, zero);
    if (lane == 0) *sc = s1;
  }
}

// kernels::KvGatherF32 (src/kernels/kv_gather.cpp:42-89): out[h, j, :] is
// token j of kv head h, read through the table.
__global__ __launch_bounds__(256) void KvGather(const float* __restrict__ k_slab,
                                                const float* __restrict__ v_slab,
                                                const int32_t* __restrict__ table, int bs,
                                                int64_t length, int kv_heads, int d,
                                                int64_t slab_blocks, float* out_k, float* out_v,
                                                int32_t* err) {
  const int64_t n = int64_t{kv_heads} * length * d;
  for (int64_t i = blockIdx.x * int64_t{blockDim.x} + threadIdx.x; i < n;
       i += int64_t{gridDim.x} * blockDim.x) {
    const int64_t hj = i / d;
    const int e = static_cast<int>(i - hj * d);
    const int h = static_cast<int>(hj / length);
    const int64_t j = hj - int64_t{h} * length;
    const int64_t phys = table[j / bs];
    if (phys < 0 || phys >= slab_blocks) {
      atomicOr(err, kErrBlockRange);
      continue;
    }
    const int64_t src = ((phys * kv_heads + h) * bs + j % bs) * d + e;
    out_k[i] = k_slab[src];
    out_v[i] = v_slab[src];
  }
}

// Counter-based N(mean, std) fill: element pair i/2 hashes (seed, i/2) with
// splitmix64 into two uniforms and takes the Box-Muller cosine/sine branch.
__device__ __forceinline__ uint64_t SplitMix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

template <class KV>
__global__ __launch_bounds__(256) void FillNormal(KV* dst, int64_t n, float mean, float stddev,
                                                  uint64_t seed) {
  for (int64_t i = blockIdx.x * int64_t{blockDim.x} + threadIdx.x; i < n;
       i += int64_t{gridDim.x} * blockDim.x) {
    const uint64_t h = SplitMix64(seed * 0x2545F4914F6CDD1Dull + static_cast<uint64_t>(i >> 1));
    const float u1 = (static_cast<float>(h >> 40) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
    const float u2 = static_cast<float>((h >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);
    const float r = sqrtf(-2.0f * __logf(u1));
    const float z = (i & 1) ? r * __sinf(6.283185307f * u2) : r * __cosf(6.283185307f * u2);
    Store1(dst + i, mean + stddev * z);
  }
}

int GridFor(int64_t work, int block) {
  const int64_t g = (work + block - 1) / block;
  return static_cast<int>(g < 65536 ? (g < 1 ? 1 : g) : 65536);
}

}  // namespace

hipError_t LaunchAppendQ8(const float* src_k, const float* src_v, const Q8Group* groups,
                          int64_t n_groups, const int32_t* rows, int kv_heads, int d, int bs,
                          int64_t slab_blocks, void* k_slab, void* v_slab, float* k_scale,
                          float* v_scale, bool fp8, int32_t* err, hipStream_t stream) {
  if (n_groups <= 0) return hipSuccess;
  if (d % 4 != 0 || n_groups * kv_heads > 0x7FFFFFFF) return hipErrorInvalidValue;
  hipLaunchKernelGGL(fp8 ? AppendQ8<true> : AppendQ8<false>,
                     dim3(static_cast<uint32_t>(n_groups * kv_heads)), dim3(64), 0, stream,
                     src_k, src_v, groups, rows, kv_heads, d, bs, slab_blocks,
                     static_cast<uint8_t*>(k_slab), static_cast<uint8_t*>(v_slab), k_scale,
                     v_scale, err);
  return hipGetLastError();
}

hipError_t LaunchRopeKvAppend(float* q, const float* src_k, const float* src_v,
                              const RowDesc* rows, const float* cos_t, const float* sin_t,
                              const int64_t* slots, int64_t n_rows, int heads, int kv_heads,
                              int d, int bs, int64_t slab_blocks, void* k_slab, void* v_slab,
                              int kv_dtype, int32_t* err, hipStream_t stream) {
  const bool vec = (d % 8) == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(src_k) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(src_v) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(cos_t) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(sin_t) % 16 == 0;
  if (n_rows <= 0) return hipSuccess;
  if (n_rows > 0x7FFFFFFF) return hipErrorInvalidValue;
  const int64_t per_row = int64_t{heads + kv_heads} * (d / 2) / (vec ? 4 : 1);
  const int threads = per_row >= 256 ? 256 : static_cast<int>((per_row + 63) / 64 * 64);
  const int64_t ys = (per_row + threads - 1) / threads;
  const dim3 grid(static_cast<uint32_t>(n_rows), static_cast<uint32_t>(ys < 65535 ? ys : 65535)),
      block(threads);
#define EHIP_ROPE_LAUNCH(KV, W)                                                               \
  hipLaunchKernelGGL((RopeKvAppend<KV, W>), grid, block, 0, stream, q, src_k, src_v, rows,   \
                     cos_t, sin_t, slots, heads, kv_heads, d, bs, slab_blocks,                \
                     static_cast<KV*>(k_slab), static_cast<KV*>(v_slab), err)
  if (kv_dtype == EHIP_KV_BF16) {
    if (vec)
      EHIP_ROPE_LAUNCH(uint16_t, 4);
    else
      EHIP_ROPE_LAUNCH(uint16_t, 1);
  } else {
    if (vec)
      EHIP_ROPE_LAUNCH(float, 4);
    else
      EHIP_ROPE_LAUNCH(float, 1);
  }
#undef EHIP_ROPE_LAUNCH
  return hipGetLastError();
}

hipError_t LaunchKvScatter(const float* src_k, const float* src_v, const int64_t* slots,
                           int64_t t_dim, int32_t kv_heads, int32_t d, int32_t bs,
                           int64_t slab_blocks, void* k_slab, void* v_slab, int kv_dtype,
                           int32_t* err, hipStream_t stream) {
  if (t_dim == 0) return hipSuccess;
  const bool vec = (d % 4 == 0) && (reinterpret_cast<uintptr_t>(src_k) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(src_v) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(k_slab) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(v_slab) % 16 == 0);
  const int64_t n = t_dim * kv_heads * d;
  if (vec) {
    const int64_t nv = n / 4;
    if (kv_dtype == EHIP_KV_BF16)
      hipLaunchKernelGGL(KvScatterVec<uint16_t>, dim3(GridFor(nv, 256)), dim3(256), 0, stream,
                         src_k, src_v, slots, nv, kv_heads, d, bs, slab_blocks,
                         static_cast<uint16_t*>(k_slab), static_cast<uint16_t*>(v_slab), err);
    else
      hipLaunchKernelGGL(KvScatterVec<float>, dim3(GridFor(nv, 256)), dim3(256), 0, stream,
                         src_k, src_v, slots, nv, kv_heads, d, bs, slab_blocks,
                         static_cast<float*>(k_slab), static_cast<float*>(v_slab), err);
  } else {
    if (kv_dtype == EHIP_KV_BF16)
      hipLaunchKernelGGL(KvScatterScalar<uint16_t>, dim3(GridFor(n, 256)), dim3(256), 0, stream,
                         src_k, src_v, slots, n, kv_heads, d, bs, slab_blocks,
                         static_cast<uint16_t*>(k_slab), static_cast<uint16_t*>(v_slab), err);
    else
      hipLaunchKernelGGL(KvScatterScalar<float>, dim3(GridFor(n, 256)), dim3(256), 0, stream,
                         src_k, src_v, slots, n, kv_heads, d, bs, slab_blocks,
                         static_cast<float*>(k_slab), static_cast<float*>(v_slab), err);
  }
  return hipGetLastError();
}

hipError_t LaunchKvGather(const float* k_slab, const float* v_slab, const int32_t* table,
                          int32_t bs, int64_t length, int32_t kv_heads, int32_t d,
                          int64_t slab_blocks, float* out_k, float* out_v, int32_t* err,
                          hipStream_t stream) {
  const int64_t n = int64_t{kv_heads} * length * d;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(KvGather, dim3(GridFor(n, 256)), dim3(256), 0, stream, k_slab, v_slab,
                     table, bs, length, kv_heads, d, slab_blocks, out_k, out_v, err);
  return hipGetLastError();
}

hipError_t LaunchFillNormal(void* dst, int64_t n, int dtype, float mean, float stddev,
                            uint64_t seed, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  if (dtype == EHIP_KV_BF16)
    hipLaunchKernelGGL(FillNormal<uint16_t>, dim3(GridFor(n, 256)), dim3(256), 0, stream,
                       static_cast<uint16_t*>(dst), n, mean, stddev, seed);
  else if (dtype == EHIP_KV_FP8)
    hipLaunchKernelGGL(FillNormal<uint8_t>, dim3(GridFor(n, 256)), dim3(256), 0, stream,
                       static_cast<uint8_t*>(dst), n, mean, stddev, seed);
  else
    hipLaunchKernelGGL(FillNormal<float>, dim3(GridFor(n, 256)), dim3(256), 0, stream,
                       static_cast<float*>(dst), n, mean, stddev, seed);
  return hipGetLastError();
}

}  // namespace ehip
