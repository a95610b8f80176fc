// fmx_synth.cpp -- seeded synthetic inputs (host memory).
//
// The reference loads real checkpoints; a benchmark of the MoE block needs
// inputs of the same shapes instead. Element i of (seed, stream) is
//   bf16(mean + std * sqrt(-2 ln u1) * cos(2 pi u2))
// with u1, u2 taken from splitmix64 of counters 2i and 2i+1 under a key
// derived from (seed, stream): a pure function of (seed, stream, i), so the
// output is the same for any thread count and any slice can be regenerated.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/fmx.h"

namespace {

inline uint64_t splitmix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// Round to nearest even from fp64 to bf16 (normal and subnormal ranges).
inline uint16_t f64_to_bf16_host(double d) {
  uint64_t u;
  std::memcpy(&u, &d, 8);
  const uint16_t sign = static_cast<uint16_t>((u >> 48) & 0x8000u);
  const uint64_t a = u & 0x7fffffffffffffffull;
  if (a > 0x7ff0000000000000ull) return 0x7fc0u;
  if (a >= 0x47f0000000000000ull) return sign | 0x7f80u;
  if (a < 0x3810000000000000ull) return sign | static_cast<uint16_t>(std::nearbyint(std::fabs(d) * 0x1p133));
  const uint64_t r = (a + 0x00000fffffffffffull + ((a >> 45) & 1u)) >> 45;
  return sign | static_cast<uint16_t>(r - (static_cast<uint64_t>(1023 - 127) << 7));
}

}  // namespace

extern "C" int fmx_synth_normal_bf16(uint16_t* out, int64_t n, uint64_t seed, uint64_t stream,
                                     double mean, double std_dev) {
  if (n < 0 || (!out && n > 0)) return FMX_ERR_ARG;
  const uint64_t key = splitmix64(seed ^ splitmix64(stream + 0x632be59bd9b4e019ull));
  const double two_pi = 6.283185307179586476925286766559;
  auto work = [&](int64_t b, int64_t e) {
    for (int64_t i = b; i < e; ++i) {
      const uint64_t h1 = splitmix64(key + 2 * static_cast<uint64_t>(i));
      const uint64_t h2 = splitmix64(key + 2 * static_cast<uint64_t>(i) + 1);
      const double u1 = (static_cast<double>(h1 >> 11) + 1.0) * 0x1p-53;  // (0, 1]
      const double u2 = static_cast<double>(h2 >> 11) * 0x1p-53;          // [0, 1)
      const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(two_pi * u2);
      out[i] = f64_to_bf16_host(mean + std_dev * z);
    }
  };
  unsigned nt = std::thread::hardware_concurrency();
  if (nt == 0) nt = 1;
  if (nt > 16) nt = 16;
  if (n < (1 << 16)) nt = 1;
  std::vector<std::thread> pool;
  const int64_t chunk = (n + nt - 1) / nt;
  for (unsigned t = 0; t < nt; ++t) {
    const int64_t b = t * chunk, e = std::min<int64_t>(n, b + chunk);
    if (b >= e) break;
    pool.emplace_back(work, b, e);
  }
  for (auto& th : pool) th.join();
  return FMX_OK;
}
