// fmx_elem.hip -- small kernels around the GEMMs: the top-k weighted
// combine with the gated shared expert, layout permutations, index
// broadcasting for gather_qmm, and the affine quantizer.
#include <algorithm>

#include "fmx_dev.hpp"

namespace fmx {

constexpr int kElemThreads = 256;

static inline unsigned grid_for(int64_t n, int per_block) {
  return static_cast<unsigned>((n + per_block - 1) / per_block);
}

// ------------------------------------------------------------------ combine
// y = sum(d_sorted[inv] * scores[..., None], -2)            model.cpp:782-784
//   + sigmoid(x . w_sg) * shared_expert(x)                   model.cpp:787-803
// Every MLX op's bf16 (F16: fp16) result is rounded as MLX rounds it; the
// k-sum accumulates in fp32 in slot order.
template <bool F16>
__global__ __launch_bounds__(kElemThreads) void combine_kernel(CombineArgs a) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kElemThreads + threadIdx.x;
  const int oct = a.H / 8;
  if (gid >= static_cast<int64_t>(a.T) * oct) return;
  const int t = static_cast<int>(gid / oct), o = static_cast<int>(gid % oct);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < a.k; ++j) {
    const int64_t ent = static_cast<int64_t>(t) * a.k + j;
    const uint32_t row = min(a.inv[ent], static_cast<uint32_t>(a.T * a.k - 1));
    const float s = Act<F16>::ld(a.scores[ent]);
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(a.d + static_cast<int64_t>(row) * a.H + o * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] += Act<F16>::rnd(Act<F16>::lo(v[i]) * s);
      acc[2 * i + 1] += Act<F16>::rnd(Act<F16>::hi(v[i]) * s);
    }
  }
  uint16_t outv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) outv[i] = Act<F16>::st(acc[i]);
  if (a.sd || a.sd_part) {
    const float g = a.sgate[t];
    float sdv[8];
    if (a.sd_part) {
      // shared down projection from its split-K partial sums, in slice order
#pragma unroll
      for (int i = 0; i < 8; ++i) sdv[i] = 0.0f;
      for (int ks = 0; ks < a.sd_ksplit; ++ks) {
        const float* p = a.sd_part + (static_cast<int64_t>(ks) * a.T + t) * a.H + o * 8;
        const f32x4_t lo = *reinterpret_cast<const f32x4_t*>(p);
        const f32x4_t hi = *reinterpret_cast<const f32x4_t*>(p + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sdv[i] += lo[i];
          sdv[4 + i] += hi[i];
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) sdv[i] = Act<F16>::rnd(sdv[i]);
    } else {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(a.sd + static_cast<int64_t>(t) * a.H + o * 8);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sdv[2 * i] = Act<F16>::lo(v[i]);
        sdv[2 * i + 1] = Act<F16>::hi(v[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float sh = Act<F16>::rnd(g * sdv[i]);
      outv[i] = Act<F16>::st(Act<F16>::ld(outv[i]) + sh);
    }
  }
  u32x4_t w;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = static_cast<uint32_t>(outv[2 * i]) | (static_cast<uint32_t>(outv[2 * i + 1]) << 16);
  *reinterpret_cast<u32x4_t*>(a.y + static_cast<int64_t>(t) * a.H + o * 8) = w;
}

hipError_t launch_combine(const CombineArgs& a, hipStream_t stream) {
  const int64_t n = static_cast<int64_t>(a.T) * (a.H / 8);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL((a.f16 ? combine_kernel<true> : combine_kernel<false>), dim3(grid_for(n, kElemThreads)),
                     dim3(kElemThreads), 0, stream, a);
  return hipGetLastError();
}

// Nemotron-H (nemotron_h.cpp:1096-1108): y = astype(sum(h * scores, -2),
// bf16) with h and the scores fp32 (the product and the k-sum in fp32, slot
// order, each operation rounded on its own: __fmul_rn / __fadd_rn keep the
// compiler from contracting them), then + shared (fp32 add), rounded to bf16.
__global__ __launch_bounds__(kElemThreads) void nh_combine_kernel(NhCombineArgs a) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kElemThreads + threadIdx.x;
  // the GEMMs that read the fp16-range flag have finished: clear it for the
  // next forward's router
  if (gid == 0 && a.clear) *a.clear = 0u;
  const int quads = a.H / 4;
  if (gid >= static_cast<int64_t>(a.T) * quads) return;
  const int t = static_cast<int>(gid / quads), o = static_cast<int>(gid % quads);
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < a.k; ++j) {
    const int64_t ent = static_cast<int64_t>(t) * a.k + j;
    const uint32_t row = min(a.inv[ent], static_cast<uint32_t>(a.T * a.k - 1));
    const float s = a.scores[ent];
    const f32x4_t v = *reinterpret_cast<const f32x4_t*>(a.d + static_cast<int64_t>(row) * a.H + o * 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = __fadd_rn(acc[i], __fmul_rn(v[i], s));
  }
  float out[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = round_bf16(acc[i]);
  if (a.sd) {
    const f32x4_t v = *reinterpret_cast<const f32x4_t*>(a.sd + static_cast<int64_t>(t) * a.H + o * 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = __fadd_rn(out[i], v[i]);
  }
  u32x2_t w;
  w[0] = static_cast<uint32_t>(f32_to_bf16(out[0])) | (static_cast<uint32_t>(f32_to_bf16(out[1])) << 16);
  w[1] = static_cast<uint32_t>(f32_to_bf16(out[2])) | (static_cast<uint32_t>(f32_to_bf16(out[3])) << 16);
  *reinterpret_cast<u32x2_t*>(a.y + static_cast<int64_t>(t) * a.H + o * 4) = w;
}

hipError_t launch_nh_combine(const NhCombineArgs& a, hipStream_t stream) {
  const int64_t n = static_cast<int64_t>(a.T) * (a.H / 4);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(nh_combine_kernel, dim3(grid_for(n, kElemThreads)), dim3(kElemThreads), 0,
                     stream, a);
  return hipGetLastError();
}

// ------------------------------------------------------------------ layouts
__global__ __launch_bounds__(kElemThreads) void permute_p8_kernel(const uint16_t* x, int64_t n_oct,
                                                                  uint16_t* xp) {
  const int64_t o = static_cast<int64_t>(blockIdx.x) * kElemThreads + threadIdx.x;
  if (o >= n_oct) return;
  const u32x4_t v = *reinterpret_cast<const u32x4_t*>(x + o * 8);
  u32x4_t p;
  p[0] = (v[0] & 0xffffu) | (v[2] << 16);
  p[1] = (v[0] >> 16) | (v[2] & 0xffff0000u);
  p[2] = (v[1] & 0xffffu) | (v[3] << 16);
  p[3] = (v[1] >> 16) | (v[3] & 0xffff0000u);
  *reinterpret_cast<u32x4_t*>(xp + o * 8) = p;
}

hipError_t launch_permute_p8(const uint16_t* x, int64_t rows, int64_t K, uint16_t* xp,
                             hipStream_t stream) {
  const int64_t n_oct = rows * (K / 8);
  if (n_oct == 0) return hipSuccess;
  hipLaunchKernelGGL(permute_p8_kernel, dim3(grid_for(n_oct, kElemThreads)), dim3(kElemThreads),
                     0, stream, x, n_oct, xp);
  return hipGetLastError();
}

__global__ __launch_bounds__(kElemThreads) void fill_u32_kernel(uint32_t* p, int64_t n, uint32_t v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kElemThreads + threadIdx.x;
  if (i < n) p[i] = v;
}

hipError_t launch_fill_u32(uint32_t* p, int64_t n, uint32_t v, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(fill_u32_kernel, dim3(grid_for(n, kElemThreads)), dim3(kElemThreads), 0,
                     stream, p, n, v);
  return hipGetLastError();
}

// bf16-valued fp32 -> bf16 bits (the value's upper half: exact); F16:
// fp16-valued fp32 -> fp16 bits (exact)
template <bool F16>
__global__ __launch_bounds__(kElemThreads) void f32_half_kernel(const float* src, int64_t n, uint16_t* dst) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kElemThreads + threadIdx.x;
  if (i < n) dst[i] = F16 ? f32_to_f16(src[i]) : static_cast<uint16_t>(__float_as_uint(src[i]) >> 16);
}

hipError_t launch_f32_bf16(const float* src, int64_t n, uint16_t* dst, hipStream_t stream, bool f16) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL((f16 ? f32_half_kernel<true> : f32_half_kernel<false>), dim3(grid_for(n, kElemThreads)),
                     dim3(kElemThreads), 0, stream, src, n, dst);
  return hipGetLastError();
}

// ------------------------------------------------------------------ gather_qmm indices
// MLX broadcasting of one index array: entry i of the flattened batch
__device__ inline void bcast_one(const BcastArgs& a, int64_t i) {
  uint32_t v;
  if (!a.src) {
    int64_t rem = i, off = 0;
    for (int d = a.ndim - 1; d >= 0; --d) {
      const int64_t c = rem % a.out_shape[d];
      rem /= a.out_shape[d];
      off += c * a.src_stride[d];
    }
    v = static_cast<uint32_t>(off);
  } else {
    int64_t rem = i, off = 0;
    for (int d = a.ndim - 1; d >= 0; --d) {
      const int64_t c = rem % a.out_shape[d];
      rem /= a.out_shape[d];
      off += c * a.src_stride[d];
    }
    v = a.is_i32 ? static_cast<uint32_t>(static_cast<const int32_t*>(a.src)[off])
                 : static_cast<const uint32_t*>(a.src)[off];
  }
  a.dst[i] = v;
  if (a.dst_rows)
    for (int m = 0; m < a.M; ++m) a.dst_rows[i * a.M + m] = v;
}

// ------------------------------------------------------------------ ops prologue
// Blocks [0, n_idx) broadcast the index arrays (one entry of each per
// thread); the n_ovf blocks after them copy x in a grid-stride loop and
// each writes its ovf word.
__global__ __launch_bounds__(kElemThreads) void ops_prologue_kernel(OpsPrologue a, int n_idx,
                                                                    int n_ovf) {
  __shared__ uint32_t s_ovf;
  if (static_cast<int>(blockIdx.x) < n_idx) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kElemThreads + threadIdx.x;
    if (i < a.lhs.n) bcast_one(a.lhs, i);
    if (i < a.rhs.n) bcast_one(a.rhs, i);
    return;
  }
  const int c = blockIdx.x - n_idx;
  if (threadIdx.x == 0) s_ovf = 0u;
  __syncthreads();
  bool ovf = false;
  for (int64_t o = static_cast<int64_t>(c) * kElemThreads + threadIdx.x; o < a.n_oct;
       o += static_cast<int64_t>(n_ovf) * kElemThreads) {
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(a.x + o * 8);
    if (a.x_f16) {  // already fp16: the Q8 order only (elements 0,2,4,6,1,3,5,7)
      u32x4_t q;
      q[0] = (v[0] & 0xffffu) | (v[1] << 16);
      q[1] = (v[2] & 0xffffu) | (v[3] << 16);
      q[2] = (v[0] >> 16) | (v[1] & 0xffff0000u);
      q[3] = (v[2] >> 16) | (v[3] & 0xffff0000u);
      *reinterpret_cast<u32x4_t*>(a.xq + o * 8) = q;
      continue;
    }
    u32x4_t p;
    p[0] = (v[0] & 0xffffu) | (v[2] << 16);
    p[1] = (v[0] >> 16) | (v[2] & 0xffff0000u);
    p[2] = (v[1] & 0xffffu) | (v[3] << 16);
    p[3] = (v[1] >> 16) | (v[3] & 0xffff0000u);
    *reinterpret_cast<u32x4_t*>(a.xp + o * 8) = p;
    *reinterpret_cast<u32x4_t*>(a.xq + o * 8) = bf16_chunk_to_f16_q8(v, ovf);
  }
  if (__ballot(ovf) && (threadIdx.x & 63) == 0) atomicOr(&s_ovf, 1u);
  __syncthreads();
  if (threadIdx.x == 0) a.ovf[c] = s_ovf;
}

int ops_prologue_ovf_words(int64_t n_oct) {
  return static_cast<int>(std::min<int64_t>(kOvfBlocks, (n_oct + kElemThreads - 1) / kElemThreads));
}

hipError_t launch_ops_prologue(const OpsPrologue& a, hipStream_t stream) {
  const int n_idx = static_cast<int>(grid_for(std::max(a.lhs.n, a.rhs.n), kElemThreads));
  const int n_ovf = ops_prologue_ovf_words(a.n_oct);
  if (n_idx + n_ovf == 0) return hipSuccess;
  hipLaunchKernelGGL(ops_prologue_kernel, dim3(n_idx + n_ovf), dim3(kElemThreads), 0, stream, a, n_idx,
                     n_ovf);
  return hipGetLastError();
}

// ------------------------------------------------------------------ quantization
// One thread per group of 64. Follows the affine quantizer of MLX (mode
// "affine"): scale = max((max - min)/15, 1e-7) signed toward the larger-
// magnitude edge, q0 = rint(edge/scale), and when q0 != 0 the scale is
// snapped to edge/q0 with bias = edge. Divisions are formed in fp64 and
// rounded to fp32, which is the correctly rounded fp32 quotient.
__device__ inline float div_rn(float a, float b) {
  return static_cast<float>(static_cast<double>(a) / static_cast<double>(b));
}

__global__ __launch_bounds__(kElemThreads) void quantize_kernel(const uint16_t* w, int64_t n_groups,
                                                                uint32_t* wq, uint16_t* s,
                                                                uint16_t* b) {
  const int64_t gi = static_cast<int64_t>(blockIdx.x) * kElemThreads + threadIdx.x;
  if (gi >= n_groups) return;
  const uint16_t* src = w + gi * kGroup;
  float v[kGroup];
#pragma unroll
  for (int c = 0; c < kGroup / 8; ++c) {
    const u32x4_t q = *reinterpret_cast<const u32x4_t*>(src + c * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[c * 8 + 2 * i] = __uint_as_float(q[i] << 16);
      v[c * 8 + 2 * i + 1] = __uint_as_float(q[i] & 0xffff0000u);
    }
  }
  float w_min = __builtin_huge_valf(), w_max = -__builtin_huge_valf();
#pragma unroll
  for (int i = 0; i < kGroup; ++i) {
    w_max = fmaxf(w_max, v[i]);
    w_min = fminf(w_min, v[i]);
  }
  const bool mask = fabsf(w_min) > fabsf(w_max);
  float scale = fmaxf(div_rn(w_max - w_min, 15.0f), 1e-7f);
  scale = mask ? scale : -scale;
  const float edge = mask ? w_min : w_max;
  const float q0 = rintf(div_rn(edge, scale));
  float bias = 0.0f;
  if (q0 != 0.0f) {
    scale = div_rn(edge, q0);
    bias = edge;
  }
  uint32_t* dst = wq + gi * (kGroup / 8);
#pragma unroll
  for (int p = 0; p < kGroup / 8; ++p) {
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float q = rintf(div_rn(v[p * 8 + i] - bias, scale));
      q = fminf(fmaxf(q, 0.0f), 15.0f);
      word |= static_cast<uint32_t>(q) << (4 * i);
    }
    dst[p] = word;
  }
  s[gi] = f32_to_bf16(scale);
  b[gi] = f32_to_bf16(bias);
}

hipError_t launch_quantize(const uint16_t* w, int64_t n_groups, uint32_t* wq, uint16_t* s,
                           uint16_t* b, hipStream_t stream) {
  if (n_groups == 0) return hipSuccess;
  hipLaunchKernelGGL(quantize_kernel, dim3(grid_for(n_groups, kElemThreads)), dim3(kElemThreads),
                     0, stream, w, n_groups, wq, s, b);
  return hipGetLastError();
}

// dequantize: out = s*q + b rounded to bf16 (mx::dequantize on bf16 scales)
__global__ __launch_bounds__(kElemThreads) void dequantize_kernel(const uint32_t* wq,
                                                                  const uint16_t* s,
                                                                  const uint16_t* b,
                                                                  int64_t n_words, uint16_t* out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kElemThreads + threadIdx.x;
  if (i >= n_words) return;
  const int64_t g = i / (kGroup / 8);
  const float sc = bf16_to_f32(s[g]), bi = bf16_to_f32(b[g]);
  const uint32_t w = wq[i];
  u32x4_t o;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    // two roundings (multiply, then add), never a contracted fma
    const float lo = __fadd_rn(__fmul_rn(sc, static_cast<float>((w >> (8 * p)) & 15u)), bi);
    const float hi = __fadd_rn(__fmul_rn(sc, static_cast<float>((w >> (8 * p + 4)) & 15u)), bi);
    o[p] = static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
  }
  *reinterpret_cast<u32x4_t*>(out + i * 8) = o;
}

hipError_t launch_dequantize(const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                             int64_t n_groups, uint16_t* out, hipStream_t stream) {
  const int64_t n_words = n_groups * (kGroup / 8);
  if (n_words == 0) return hipSuccess;
  hipLaunchKernelGGL(dequantize_kernel, dim3(grid_for(n_words, kElemThreads)), dim3(kElemThreads),
                     0, stream, wq, s, b, n_words, out);
  return hipGetLastError();
}

}  // namespace fmx
