// fmx_pack.hip -- load-time re-layout of 4-bit expert weights into the
// packed tile/unit blocks the decode kernels stream (layout: fmx_dev.hpp).
// Replaces, as the last load-time transform, the expert stacking of
// LlamaModel::build_moe_weight_cache (server/src/model.cpp:368-470).
#include "fmx_dev.hpp"

namespace fmx {

// ---------------------------------------------------------------- packing

// Nibble order inside a packed word: stored position i (i < 4) holds element
// 2i of the word's 8 and position i + 4 holds element 2i + 1, so that nib8
// (fmx_dev.hpp) yields the bf16 pairs (q_2i, q_2i+1): operands in natural
// element order, matching activation rows as they are stored.
__device__ inline uint32_t interleave_nibbles(uint32_t w) {
  uint32_t r = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r |= ((w >> (8 * i)) & 0xfu) << (4 * i);
    r |= ((w >> (8 * i + 4)) & 0xfu) << (4 * (i + 4));
  }
  return r;
}

// One thread per (expert, tile, unit, lane): the lane's 16 weight bytes of
// each matrix; lanes 0..15 also the (scale, bias) words of their row. Rows
// past the source's N and quantisation groups past its K pack as zero words
// with scale 0 and bias 0: weights of value 0 that pad a matrix to whole
// tiles and units.
__global__ void pack_kernel(PackArgs a) {
  const int64_t blk = blockIdx.x;  // (expert, tile, unit)
  const int lane = threadIdx.x;
  const int64_t per_exp = static_cast<int64_t>(a.nt) * a.nu;
  const int64_t e = blk / per_exp;
  const int64_t r = blk - e * per_exp;
  const int tile = static_cast<int>(r / a.nu), u = static_cast<int>(r - static_cast<int64_t>(tile) * a.nu);
  const int col = lane & 15, j = lane >> 4;
  const int K = a.k_src ? a.k_src : a.nu * 128, G = K / kGroup;
  const int64_t row = static_cast<int64_t>(tile) * 16 + col;
  const bool row_in = row < a.N;
  const int nm = a.w1 ? 2 : 1;
  const int BB = nm == 2 ? 2304 : 1152;
  uint8_t* dst = a.dst + e * a.dst_estride + (static_cast<int64_t>(tile) * a.nu + u) * BB;
  for (int mtx = 0; mtx < nm; ++mtx) {
    const uint32_t* w = mtx ? a.w1 : a.w0;
    const uint16_t* s = mtx ? a.s1 : a.s0;
    const uint16_t* bb = mtx ? a.b1 : a.b0;
    const uint32_t* wr = w + (e * a.N + row) * (K / 8) + u * 16;
    u32x4_t v;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // word 4q + j of the unit: k = 128 u + 8 (4q + j), in group 2u + (4q + j) / 8
      const bool in = row_in && 2 * u + (4 * q + j) / 8 < G;
      v[q] = in ? interleave_nibbles(wr[4 * q + j]) : 0u;
    }
    *reinterpret_cast<u32x4_t*>(dst + mtx * 1024 + 16 * lane) = v;
    if (lane < 16) {
      const int64_t g = (e * a.N + row) * G + 2 * u;
      const bool in0 = row_in && 2 * u < G, in1 = row_in && 2 * u + 1 < G;
      u32x2_t sb;
      sb[0] = (in0 ? static_cast<uint32_t>(s[g]) : 0u) | ((in1 ? static_cast<uint32_t>(s[g + 1]) : 0u) << 16);
      sb[1] = (in0 ? static_cast<uint32_t>(bb[g]) : 0u) | ((in1 ? static_cast<uint32_t>(bb[g + 1]) : 0u) << 16);
      *reinterpret_cast<u32x2_t*>(dst + nm * 1024 + mtx * 128 + 8 * col) = sb;
    }
  }
}

hipError_t launch_pack(const PackArgs& a, hipStream_t stream) {
  const int64_t blocks = a.n_exp * a.nt * a.nu;
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(pack_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kWave), 0, stream, a);
  return hipGetLastError();
}

}  // namespace fmx
