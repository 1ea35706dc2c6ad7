// Device helpers shared by the gfx950 kernels: bf16 bit conversions, DPP and
// cross-row lane exchanges for 64-wide wavefronts, hardware exp2.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ehip {

// Reference Fp32ToBf16Bits (src/tensor/half.h:112-124): NaN keeps its sign and
// top payload bits and is quieted when the kept payload is empty; everything
// else rounds to nearest even on the 16 dropped bits (overflow carries into
// the exponent and lands on +-inf).
__device__ __forceinline__ uint32_t Fp32ToBf16Bits(float v) {
  const uint32_t bits = __float_as_uint(v);
  if ((bits & 0x7FFFFFFFu) > 0x7F800000u) {
    uint32_t r = bits >> 16;
    if ((r & 0x7Fu) == 0u) r |= 0x40u;
    return r;
  }
  return (bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float Bf16Lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float Bf16Hi(uint32_t pair) {
  return __uint_as_float(pair & 0xFFFF0000u);
}

// DPP lane exchange within rows of 16 lanes. CTRL values (gfx9 encoding):
// 0xB1 quad_perm[1,0,3,2] (xor 1), 0x4E quad_perm[2,3,0,1] (xor 2),
// 0x141 row_half_mirror (i <-> 7-i), 0x128 row_ror:8 (xor 8 within 16).
template <int CTRL>
__device__ __forceinline__ float Dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of 8 lanes: after xor1 and xor2 every lane holds its
// quad's sum; the half-row mirror pairs quad 0 with quad 1 (and 2 with 3).
__device__ __forceinline__ float SumGroup8(float x) {
  x += Dpp<0xB1>(x);
  x += Dpp<0x4E>(x);
  x += Dpp<0x141>(x);
  return x;
}
__device__ __forceinline__ float SumGroup16(float x) {
  x = SumGroup8(x);
  x += Dpp<0x128>(x);
  return x;
}

template <int LPT>
__device__ __forceinline__ float SumGroup(float x) {
  static_assert(LPT == 8 || LPT == 16, "lanes per token");
  if constexpr (LPT == 8) return SumGroup8(x);
  else return SumGroup16(x);
}

__device__ __forceinline__ float ShflXor(float x, int mask) {
  const int lane = __lane_id();
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(x)));
}

// Reductions across the lanes that differ only in the bits >= log2(STRIDE)
// (the "token lanes" of a wavefront whose low bits index a head-dim slice).
template <int STRIDE>
__device__ __forceinline__ float MaxAcross(float x) {
  if constexpr (STRIDE <= 8) x = fmaxf(x, Dpp<0x128>(x));
  if constexpr (STRIDE <= 16) x = fmaxf(x, ShflXor(x, 16));
  x = fmaxf(x, ShflXor(x, 32));
  return x;
}
template <int STRIDE>
__device__ __forceinline__ float SumAcross(float x) {
  if constexpr (STRIDE <= 8) x += Dpp<0x128>(x);
  if constexpr (STRIDE <= 16) x += ShflXor(x, 16);
  x += ShflXor(x, 32);
  return x;
}

__device__ __forceinline__ float WaveSum(float x) {
  x = SumGroup16(x);
  x += ShflXor(x, 16);
  x += ShflXor(x, 32);
  return x;
}
__device__ __forceinline__ float WaveMax(float x) {
  x = fmaxf(x, Dpp<0xB1>(x));
  x = fmaxf(x, Dpp<0x4E>(x));
  x = fmaxf(x, Dpp<0x141>(x));
  x = fmaxf(x, Dpp<0x128>(x));
  x = fmaxf(x, ShflXor(x, 16));
  x = fmaxf(x, ShflXor(x, 32));
  return x;
}

// Hardware base-2 exponential (v_exp_f32); exp2(-inf) = 0.
__device__ __forceinline__ float Exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;

}  // namespace ehip
