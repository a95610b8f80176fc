// fmx_qgemm.hip -- grouped affine-4-bit GEMM on MFMA (the gather_qmm core).
//
// Computes, for every row r of every segment (rows sharing one expert e),
//   out[r, n] = sum_k x[r, k] * (s[e,n,g(k)] * q[e,n,k] + b[e,n,g(k)])
// i.e. mx::gather_qmm / mx::quantized_matmul with transpose=true, group 64,
// bits 4 (server/src/model.cpp:703-721, :741-747), optionally fused with the
// compiled SwiGLU of a gate/up pair (model.cpp:14-25, :715).
//
// Schedule (one workgroup = one segment x one 16-row output tile):
//   - the 4 waves split the K groups four ways; partial sums meet in LDS
//     and are added in wave order, so results are deterministic;
//   - per group of 64: each lane loads two packed words (16 nibbles) of its
//     output row, and the nibbles become bf16 values 128+q with one
//     AND/OR per pair (0x4300 | q is the bf16 bit pattern of 128+q);
//   - v_mfma_f32_16x16x32_bf16 forms P = x.(128+q) over the group and
//     X = x.1 (an all-ones operand); the group then adds s*P + (b-128s)*X,
//     which is the exact fp32 value of x.(s*q+b): weights are never rounded
//     to bf16;
//   - activations are stored in the P8 layout (fmx_common.hpp), so a word's
//     nibble pairs (q_i, q_{i+4}) meet consecutive activation pairs.
// Tokens are the MFMA's 16-row dimension: a decode segment of 1..16 rows is
// one M tile, larger segments loop over M tiles.
#include "fmx_kernels.hpp"

namespace fmx {

constexpr int kQThreads = 256;
constexpr int kQWaves = kQThreads / kWave;

__device__ inline bf16x8_t nibbles_as_bf16(uint32_t w) {
  u32x4_t d;
  d[0] = (w & 0x000f000fu) | 0x43004300u;
  d[1] = ((w >> 4) & 0x000f000fu) | 0x43004300u;
  d[2] = ((w >> 8) & 0x000f000fu) | 0x43004300u;
  d[3] = ((w >> 12) & 0x000f000fu) | 0x43004300u;
  return __builtin_bit_cast(bf16x8_t, d);
}

__device__ inline f32x4_t mfma16(const bf16x8_t& a, const bf16x8_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <bool DUAL>
__device__ void qgemm_tile(const QGemmProblem& P, int seg, int nt, float* s_red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, j = lane >> 4;
  const int64_t e =
      P.seg_exp ? static_cast<int64_t>(min(P.seg_exp[seg], static_cast<uint32_t>(P.n_exp - 1))) : 0;
  const int r0 = P.seg_off ? static_cast<int>(min(P.seg_off[seg], static_cast<uint32_t>(P.rows_max))) : 0;
  const int r1 = P.seg_off ? max(r0, static_cast<int>(min(P.seg_off[seg + 1],
                                                          static_cast<uint32_t>(P.rows_max))))
                           : P.rows_static;
  const int K = P.K, N = P.N, G = K / kGroup;
  const int n = nt * 16 + col;
  const int nc = n < N ? n : N - 1;

  const uint32_t* w0r = P.w0 + e * P.ew + static_cast<int64_t>(nc) * (K / 8) + 2 * j;
  const uint16_t* s0r = P.s0 + e * P.es + static_cast<int64_t>(nc) * G;
  const uint16_t* b0r = P.b0 + e * P.es + static_cast<int64_t>(nc) * G;
  const uint32_t* w1r = nullptr;
  const uint16_t *s1r = nullptr, *b1r = nullptr;
  if (DUAL) {
    w1r = P.w1 + e * P.ew + static_cast<int64_t>(nc) * (K / 8) + 2 * j;
    s1r = P.s1 + e * P.es + static_cast<int64_t>(nc) * G;
    b1r = P.b1 + e * P.es + static_cast<int64_t>(nc) * G;
  }
  const int gb = (G * wave) / kQWaves, ge = (G * (wave + 1)) / kQWaves;
  const u32x4_t ones_u = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, ones_u);
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};

  for (int mb = r0; mb < r1; mb += 16) {
    const int r = mb + col;
    const bool vm = r < r1;
    const uint16_t* xr = P.x;
    if (vm) {
      const int64_t xrow =
          P.row_map ? static_cast<int64_t>(min(P.row_map[r], static_cast<uint32_t>(P.x_rows - 1))) : r;
      xr = P.x + xrow * P.ldx + 16 * j;
    }
    f32x4_t acc0 = zero, acc1 = zero;
    for (int g = gb; g < ge; ++g) {
      u32x4_t a0 = {0u, 0u, 0u, 0u}, a1 = {0u, 0u, 0u, 0u};
      if (vm) {
        a0 = *reinterpret_cast<const u32x4_t*>(xr + g * kGroup);
        a1 = *reinterpret_cast<const u32x4_t*>(xr + g * kGroup + 8);
      }
      const u32x2_t q0 = *reinterpret_cast<const u32x2_t*>(w0r + g * 8);
      const float sc0 = bf16_to_f32(s0r[g]);
      const float bi0 = bf16_to_f32(b0r[g]);
      const bf16x8_t A0 = __builtin_bit_cast(bf16x8_t, a0);
      const bf16x8_t A1 = __builtin_bit_cast(bf16x8_t, a1);
      f32x4_t X = mfma16(A0, ones, zero);
      X = mfma16(A1, ones, X);
      f32x4_t P0 = mfma16(A0, nibbles_as_bf16(q0[0]), zero);
      P0 = mfma16(A1, nibbles_as_bf16(q0[1]), P0);
      const float c0 = __builtin_fmaf(-128.0f, sc0, bi0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc0[i] = __builtin_fmaf(sc0, P0[i], acc0[i]);
        acc0[i] = __builtin_fmaf(c0, X[i], acc0[i]);
      }
      if (DUAL) {
        const u32x2_t q1 = *reinterpret_cast<const u32x2_t*>(w1r + g * 8);
        const float sc1 = bf16_to_f32(s1r[g]);
        const float bi1 = bf16_to_f32(b1r[g]);
        f32x4_t P1 = mfma16(A0, nibbles_as_bf16(q1[0]), zero);
        P1 = mfma16(A1, nibbles_as_bf16(q1[1]), P1);
        const float c1 = __builtin_fmaf(-128.0f, sc1, bi1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc1[i] = __builtin_fmaf(sc1, P1[i], acc1[i]);
          acc1[i] = __builtin_fmaf(c1, X[i], acc1[i]);
        }
      }
    }
    // split-K partials meet in LDS; wave 0 adds them in wave order
    if (wave > 0) {
      float* dst = s_red + (wave - 1) * 8 * kWave;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dst[i * kWave + lane] = acc0[i];
        if (DUAL) dst[(4 + i) * kWave + lane] = acc1[i];
      }
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int w = 0; w < kQWaves - 1; ++w) {
        const float* srcp = s_red + w * 8 * kWave;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc0[i] += srcp[i * kWave + lane];
          if (DUAL) acc1[i] += srcp[(4 + i) * kWave + lane];
        }
      }
      if (n < N) {
        const int ncol = P.out_p8 ? ((n & ~7) | p8_slot(n & 7)) : n;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int rr = mb + 4 * j + i;  // MFMA output row of this lane
          if (rr >= r1) continue;
          const int64_t orow =
              P.out_map ? static_cast<int64_t>(min(P.out_map[rr], static_cast<uint32_t>(P.out_rows - 1)))
                        : rr;
          uint16_t v;
          if (DUAL)
            v = swiglu_bf16(round_bf16(acc0[i]), round_bf16(acc1[i]));
          else
            v = f32_to_bf16(acc0[i]);
          P.out[orow * P.ldo + ncol] = v;
        }
      }
    }
    __syncthreads();
  }
}

__device__ inline void qgemm_run(const QGemmProblem& P, int bid, float* s_red) {
  const int seg = bid / P.n_tiles, nt = bid % P.n_tiles;
  const int n_seg = P.seg_n ? static_cast<int>(min(*P.seg_n, static_cast<uint32_t>(P.max_seg))) : 1;
  if (seg >= n_seg) return;
  if (P.dual)
    qgemm_tile<true>(P, seg, nt, s_red);
  else
    qgemm_tile<false>(P, seg, nt, s_red);
}

__global__ __launch_bounds__(kQThreads) void qgemm_kernel(QGemmProblem p0, QGemmProblem p1,
                                                          int nblk0) {
  __shared__ float s_red[(kQWaves - 1) * 8 * kWave];
  const int bid = blockIdx.x;
  if (bid < nblk0)
    qgemm_run(p0, bid, s_red);
  else
    qgemm_run(p1, bid - nblk0, s_red);
}

hipError_t launch_qgemm(const QGemmProblem& p0, const QGemmProblem* p1, hipStream_t stream) {
  const int nblk0 = p0.max_seg * p0.n_tiles;
  const int nblk1 = p1 ? p1->max_seg * p1->n_tiles : 0;
  if (nblk0 + nblk1 == 0) return hipSuccess;
  QGemmProblem q1 = p1 ? *p1 : p0;
  hipLaunchKernelGGL(qgemm_kernel, dim3(nblk0 + nblk1), dim3(kQThreads), 0, stream, p0, q1,
                     nblk0);
  return hipGetLastError();
}

}  // namespace fmx
