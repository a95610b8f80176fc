// fmx_synth.hip -- seeded synthetic inputs, in host or device memory.
//
// The reference loads real checkpoints; a benchmark of the MoE block needs
// inputs of the same shapes instead. Element i of (seed, stream) is
//   bf16(mean + std * sqrt(-2 ln u1) * cos(2 pi u2))
// with u1, u2 taken from splitmix64 of counters 2i and 2i+1 under a key
// derived from (seed, stream): a pure function of (seed, stream, i), so the
// output is the same for any thread count and any slice can be regenerated.
// The device version runs the same integer steps and the same fp64
// formula; its log and cos are the device library's, so it agrees with the
// host version except where a last-ulp difference of the fp64 value crosses
// a bf16 rounding boundary (about one element in 2^44).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/fmx.h"

namespace {

__host__ __device__ inline uint64_t splitmix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

__host__ __device__ inline uint64_t synth_key(uint64_t seed, uint64_t stream) {
  return splitmix64(seed ^ splitmix64(stream + 0x632be59bd9b4e019ull));
}

// Round to nearest even from fp64 to bf16 (normal and subnormal ranges), on
// the integer image of the double.
__host__ __device__ inline uint16_t f64_to_bf16_rne(double d, uint64_t u) {
  const uint16_t sign = static_cast<uint16_t>((u >> 48) & 0x8000u);
  const uint64_t a = u & 0x7fffffffffffffffull;
  if (a > 0x7ff0000000000000ull) return 0x7fc0u;
  if (a >= 0x47f0000000000000ull) return sign | 0x7f80u;
  if (a < 0x3810000000000000ull) return sign | static_cast<uint16_t>(rint(fabs(d) * 0x1p133));
  const uint64_t r = (a + 0x00000fffffffffffull + ((a >> 45) & 1u)) >> 45;
  return sign | static_cast<uint16_t>(r - (static_cast<uint64_t>(1023 - 127) << 7));
}

constexpr double kTwoPi = 6.283185307179586476925286766559;

__host__ __device__ inline double synth_uniform1(uint64_t key, int64_t i) {
  const uint64_t h1 = splitmix64(key + 2 * static_cast<uint64_t>(i));
  return (static_cast<double>(h1 >> 11) + 1.0) * 0x1p-53;  // (0, 1]
}
__host__ __device__ inline double synth_uniform2(uint64_t key, int64_t i) {
  const uint64_t h2 = splitmix64(key + 2 * static_cast<uint64_t>(i) + 1);
  return static_cast<double>(h2 >> 11) * 0x1p-53;          // [0, 1)
}

__global__ __launch_bounds__(256) void synth_kernel(uint16_t* out, int64_t n, uint64_t key,
                                                    double mean, double std_dev) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const double u1 = synth_uniform1(key, i), u2 = synth_uniform2(key, i);
    const double z = sqrt(-2.0 * log(u1)) * cos(kTwoPi * u2);
    const double v = mean + std_dev * z;
    out[i] = f64_to_bf16_rne(v, static_cast<uint64_t>(__double_as_longlong(v)));
  }
}

}  // namespace

extern "C" int fmx_synth_normal_bf16(uint16_t* out, int64_t n, uint64_t seed, uint64_t stream,
                                     double mean, double std_dev) {
  if (n < 0 || (!out && n > 0)) return FMX_ERR_ARG;
  const uint64_t key = synth_key(seed, stream);
  auto work = [&](int64_t b, int64_t e) {
    for (int64_t i = b; i < e; ++i) {
      const double u1 = synth_uniform1(key, i), u2 = synth_uniform2(key, i);
      const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(kTwoPi * u2);
      const double v = mean + std_dev * z;
      uint64_t u;
      std::memcpy(&u, &v, 8);
      out[i] = f64_to_bf16_rne(v, u);
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

extern "C" int fmx_synth_normal_bf16_device(void* out, int64_t n, uint64_t seed, uint64_t stream,
                                            double mean, double std_dev, fmx_stream s) {
  if (n < 0 || (!out && n > 0)) return FMX_ERR_ARG;
  if (n == 0) return FMX_OK;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 8192);
  hipLaunchKernelGGL(synth_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(s), static_cast<uint16_t*>(out), n,
                     synth_key(seed, stream), mean, std_dev);
  return hipGetLastError() == hipSuccess ? FMX_OK : FMX_ERR_HIP;
}
