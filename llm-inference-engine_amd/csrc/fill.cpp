// Seeded host fills with the reference's determinism contract
// (src/tensor/ops.h:88-109, src/tensor/ops.cpp:205-224 and :451-477):
// std::mt19937_64, whose output sequence the C++ standard fixes; uniforms
// u = (x >> 11) * 2^-53 in [0, 1) and ((x >> 11) + 1) * 2^-53 in (0, 1];
// normals by Box-Muller on consecutive pairs of engine outputs, evaluated in
// double and narrowed once per element. Benchmarks and tests build their
// synthetic steps from these streams, so a seed names the same data on every
// machine with the same libm.
//
// Work is split over threads by pairs of engine outputs: a thread advances a
// copy of the engine past the pairs before its range (discard) and produces
// its range, so the result does not depend on the thread count.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <random>
#include <thread>
#include <vector>

#include "ehip.h"

namespace {

constexpr double kTwoPi = 2.0 * 3.141592653589793;  // 2 * std::numbers::pi
constexpr double kTwoM53 = 1.0 / 9007199254740992.0;  // 2^-53

// Threads for a fill of n elements: one per 4M elements, at most the
// hardware's (and 16, the CPU share of one GPU on a shared host).
int FillThreads(int64_t n) {
  const int64_t hw = std::max<int64_t>(1, std::thread::hardware_concurrency());
  return static_cast<int>(std::clamp<int64_t>(n / (int64_t{1} << 22), 1, std::min<int64_t>(hw, 16)));
}

template <class F>
void ParallelRanges(int64_t n, int threads, F fn) {
  if (threads <= 1) {
    fn(int64_t{0}, n);
    return;
  }
  std::vector<std::thread> pool;
  pool.reserve(static_cast<size_t>(threads));
  for (int t = 0; t < threads; ++t) {
    const int64_t lo = n * t / threads, hi = n * (t + 1) / threads;
    pool.emplace_back([=] { fn(lo, hi); });
  }
  for (auto& th : pool) th.join();
}

// Elements [e0, e1) of fill_normal(mean, stddev, seed): element 2p is the
// cosine branch of pair p, element 2p + 1 its sine branch; pair p uses engine
// outputs 2p and 2p + 1.
void NormalRange(float* dst, int64_t n, double mean, double stddev, uint64_t seed, int64_t e0,
                 int64_t e1) {
  std::mt19937_64 eng(seed);
  const int64_t p0 = e0 / 2;
  eng.discard(static_cast<unsigned long long>(2 * p0));
  for (int64_t e = 2 * p0; e < e1; e += 2) {
    const double u1 = static_cast<double>((eng() >> 11) + 1) * kTwoM53;
    const double u2 = static_cast<double>(eng() >> 11) * kTwoM53;
    const double radius = std::sqrt(-2.0 * std::log(u1));
    const double angle = kTwoPi * u2;
    const double z0 = radius * std::cos(angle);
    const double z1 = radius * std::sin(angle);
    if (e >= e0) dst[e] = static_cast<float>(mean + (stddev * z0));
    if (e + 1 < e1 && e + 1 < n) dst[e + 1] = static_cast<float>(mean + (stddev * z1));
  }
}

// The reference's Fp32ToBf16Bits (src/tensor/half.h:112-124): NaN keeps its
// sign and top payload bits, quieted when the kept payload is empty; every
// other value rounds to nearest even on the dropped 16 bits.
inline uint16_t ToBf16(float v) {
  uint32_t bits;
  static_assert(sizeof(bits) == sizeof(v), "float is 32 bits");
  __builtin_memcpy(&bits, &v, sizeof(bits));
  if ((bits & 0x7FFFFFFFu) > 0x7F800000u) {
    uint32_t r = bits >> 16;
    if ((r & 0x7Fu) == 0u) r |= 0x40u;
    return static_cast<uint16_t>(r);
  }
  return static_cast<uint16_t>((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
}

}  // namespace

extern "C" {

int ehip_rng_u64(uint64_t seed, uint64_t skip, uint64_t* h_out, int64_t n) {
  if (n < 0 || (n > 0 && !h_out)) return EHIP_INVALID_ARGUMENT;
  std::mt19937_64 eng(seed);
  eng.discard(static_cast<unsigned long long>(skip));
  for (int64_t i = 0; i < n; ++i) h_out[i] = eng();
  return EHIP_OK;
}

int ehip_host_fill_normal(float* h_dst, int64_t n, double mean, double stddev, uint64_t seed) {
  if (n < 0 || (n > 0 && !h_dst) || !std::isfinite(mean) || !std::isfinite(stddev) ||
      stddev < 0)
    return EHIP_INVALID_ARGUMENT;
  if (n == 0) return EHIP_OK;
  // Ranges start on pair boundaries so each pair is produced by one thread.
  const int64_t pairs = (n + 1) / 2;
  ParallelRanges(pairs, FillThreads(n), [&](int64_t p0, int64_t p1) {
    NormalRange(h_dst, n, mean, stddev, seed, 2 * p0, std::min(n, 2 * p1));
  });
  return EHIP_OK;
}

int ehip_host_fp32_to_bf16(const float* h_src, uint16_t* h_dst, int64_t n) {
  if (n < 0 || (n > 0 && (!h_src || !h_dst))) return EHIP_INVALID_ARGUMENT;
  ParallelRanges(n, FillThreads(n), [&](int64_t lo, int64_t hi) {
    for (int64_t i = lo; i < hi; ++i) h_dst[i] = ToBf16(h_src[i]);
  });
  return EHIP_OK;
}

}  // extern "C"
