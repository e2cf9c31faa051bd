// Seeded inputs of the benchmark harness (include/mi_bench.h).
#include "mi_bench.h"

#include <cmath>
#include <cstring>

namespace {

uint64_t step(uint64_t x) {
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  return x;
}

// XorShift64 is linear over GF(2)^64: a map is its 64 column images.
struct Gf2Map {
  uint64_t col[64];
  uint64_t apply(uint64_t x) const {
    uint64_t y = 0;
    for (int b = 0; b < 64; ++b)
      if ((x >> b) & 1u) y ^= col[b];
    return y;
  }
};

uint64_t advance(uint64_t state, uint64_t steps) {
  Gf2Map power;
  for (int b = 0; b < 64; ++b) power.col[b] = step(1ull << b);
  while (steps != 0) {
    if (steps & 1u) state = power.apply(state);
    Gf2Map sq;
    for (int b = 0; b < 64; ++b) sq.col[b] = power.apply(power.col[b]);
    power = sq;
    steps >>= 1;
  }
  return state;
}

double draw(uint64_t *state) {
  *state = step(*state);
  return (double)*state / 18446744073709551616.0;
}

// Round-to-nearest-even binary32 -> binary16.
uint16_t to_f16(float value) {
  uint32_t x;
  std::memcpy(&x, &value, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0));
  if (exp == 0) return (uint16_t)sign;
  const int e = (int)exp - 112;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e >= 1) {
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
  }
  man |= 0x800000u;
  const uint32_t shift = (uint32_t)(126 - (int)exp);
  if (shift >= 25) return (uint16_t)sign;
  uint32_t h = man >> shift;
  const uint32_t rem = man & ((1u << shift) - 1u), half = 1u << (shift - 1);
  if (rem > half || (rem == half && (h & 1u))) ++h;
  return (uint16_t)(sign | h);
}

}  // namespace

extern "C" void mi_bench_fill_normal_f16(uint64_t seed, uint16_t *out, size_t n,
                                         int32_t threads) {
  const uint64_t start = seed == 0 ? 0x9e3779b97f4a7c15ull : seed;
  if (threads < 1) threads = 1;
  if ((size_t)threads > n / 65536 + 1) threads = (int32_t)(n / 65536 + 1);
#pragma omp parallel for num_threads(threads) schedule(static, 1)
  for (int32_t w = 0; w < threads; ++w) {
    const size_t lo = n * (size_t)w / (size_t)threads;
    const size_t hi = n * (size_t)(w + 1) / (size_t)threads;
    uint64_t state = advance(start, 2 * (uint64_t)lo);
    for (size_t i = lo; i < hi; ++i) {
      const double u1 = draw(&state), u2 = draw(&state);
      const double z = std::sqrt(-2.0 * std::log(1.0 - u1)) * std::cos(2.0 * M_PI * u2);
      out[i] = to_f16((float)z);
    }
  }
}

extern "C" void mi_bench_fill_uniform_u32(uint64_t seed, uint32_t lo, uint32_t hi,
                                          uint32_t *out, size_t n) {
  uint64_t state = seed == 0 ? 0x9e3779b97f4a7c15ull : seed;
  const double span = (double)hi - (double)lo + 1.0;
  for (size_t i = 0; i < n; ++i) {
    const double value = std::floor(draw(&state) * span);
    out[i] = lo + (value >= span ? hi - lo : (uint32_t)value);
  }
}
