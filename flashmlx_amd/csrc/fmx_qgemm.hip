// fmx_qgemm.hip -- grouped affine-4-bit GEMM on MFMA (the gather_qmm core).
//
// Computes, for every row r of every segment (rows sharing one expert e),
//   out[r, n] = sum_k x[r, k] * (s[e,n,g(k)] * q[e,n,k] + b[e,n,g(k)])
// i.e. mx::gather_qmm / mx::quantized_matmul with transpose=true, group 64,
// bits 4 (server/src/model.cpp:703-721, :741-747), optionally fused with the
// compiled SwiGLU of a gate/up pair (model.cpp:14-25, :715).
//
// Exact dequantisation. Nibbles become bf16 values 128+q with one AND/OR per
// pair (0x4300 | q is the bf16 bit pattern of 128+q). v_mfma_f32_16x16x32_bf16
// forms P = x.(128+q) over one group and X = x.1 (an all-ones operand); the
// group then adds s*P + (b - 128 s)*X, the exact fp32 value of x.(s*q + b):
// weights are never rounded to bf16.
//
// Schedule. A workgroup owns one segment (rows sharing an expert) x one tile
// of 16 output rows; its 4 waves split K and their partial sums meet in LDS,
// added in wave order (deterministic). The unit of work is two groups (128
// k) of the 16 rows: lane (c = l % 16, j = l / 16) loads the 16 bytes at
// words 4j..4j+3 of the unit in its row, so lanes j < 2 hold group 2u and
// lanes j >= 2 group 2u+1; the 4 lanes of a row read 64 contiguous bytes. An
// MFMA contracts 32 k across all four j, so each group's sum is formed with
// the weight operand zeroed on the other group's lanes: the conversion's
// AND mask and OR constant are per-lane values, which zero those lanes for
// free. Activation rows (P8 layout, fmx_common.hpp) are staged in LDS once
// per workgroup. Weight loads run two units ahead of the math. Global loads
// are unconditional from addresses clamped into their arrays (a load under a
// lane-divergent branch ends in a wait for all outstanding loads).
#include <algorithm>

#include "fmx_kernels.hpp"

namespace fmx {

constexpr int kQThreads = 256;
constexpr int kQWaves = kQThreads / kWave;
constexpr int kQRows = 16;                   // activation rows per MFMA tile
constexpr size_t kQStageBytes = 56 * 1024;   // LDS for staged activation rows

__device__ inline f32x4_t mfma16(const bf16x8_t& a, const bf16x8_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// the 8 nibbles of w as bf16 (128+q) pairs (q_i, q_{i+4}), or zeros where
// mask/magic are zero
__device__ inline bf16x8_t nibbles_as_bf16(uint32_t w, uint32_t mask, uint32_t magic) {
  u32x4_t d;
  d[0] = (w & mask) | magic;
  d[1] = ((w >> 4) & mask) | magic;
  d[2] = ((w >> 8) & mask) | magic;
  d[3] = ((w >> 12) & mask) | magic;
  return __builtin_bit_cast(bf16x8_t, d);
}

// Raw loads of one unit. Loaded values are only combined where they are
// used: touching a prefetched value right after its load would make the
// wave wait for it there.
template <bool DUAL, bool EVEN_G>
struct UnitLoad {
  u32x4_t q0, q1;  // 16 bytes of the packed row (gate / up)
  // scales and biases of groups 2u and 2u+1: with an even group count one
  // 32-bit load each (low half = group 2u); else separate 16-bit loads
  uint32_t s0, b0, s1, b1;
  uint16_t s0h, b0h, s1h, b1h;
  bool has_hi;
};

// Weights of expert e: uniform base pointers (scalar registers) plus 32-bit
// per-lane row offsets, so loads address as base + offset.
template <bool DUAL>
struct RowPtrs {
  const uint32_t* w0; const uint16_t* s0; const uint16_t* b0;
  const uint32_t* w1; const uint16_t* s1; const uint16_t* b1;
  int wo;  // row offset in words
  int so;  // row offset in scale elements
};

template <bool DUAL, bool EVEN_G>
__device__ inline UnitLoad<DUAL, EVEN_G> load_unit(int u, int G, int j, const RowPtrs<DUAL>& R) {
  UnitLoad<DUAL, EVEN_G> L;
  L.has_hi = EVEN_G || 2 * u + 1 < G;
  const int wo = R.wo + u * 16 + 4 * (L.has_hi ? j : (j & 1));  // inside the row either way
  L.q0 = *reinterpret_cast<const u32x4_t*>(R.w0 + wo);
  if (DUAL) L.q1 = *reinterpret_cast<const u32x4_t*>(R.w1 + wo);
  const int sl = R.so + 2 * u;
  if (EVEN_G) {
    L.s0 = *reinterpret_cast<const uint32_t*>(R.s0 + sl);
    L.b0 = *reinterpret_cast<const uint32_t*>(R.b0 + sl);
    if (DUAL) {
      L.s1 = *reinterpret_cast<const uint32_t*>(R.s1 + sl);
      L.b1 = *reinterpret_cast<const uint32_t*>(R.b1 + sl);
    }
  } else {
    const int sh = L.has_hi ? sl + 1 : sl;
    L.s0 = R.s0[sl];
    L.b0 = R.b0[sl];
    L.s0h = R.s0[sh];
    L.b0h = R.b0[sh];
    if (DUAL) {
      L.s1 = R.s1[sl];
      L.b1 = R.b1[sl];
      L.s1h = R.s1[sh];
      L.b1h = R.b1[sh];
    }
  }
  return L;
}

// (scale, bias) words of groups 2u | 2u+1 << 16; no second group: 0 for it
template <bool EVEN_G>
__device__ inline uint32_t pair_word(uint32_t lo, uint16_t hi, bool has_hi) {
  if (EVEN_G) return lo;
  return (lo & 0xffffu) | (has_hi ? static_cast<uint32_t>(hi) << 16 : 0u);
}

// acc += s_lo*P_lo + (b_lo-128 s_lo)*X_lo + s_hi*P_hi + (b_hi-128 s_hi)*X_hi
__device__ inline void unit_epilogue(f32x4_t& acc, uint32_t sp, uint32_t bp, const f32x4_t& Plo,
                                     const f32x4_t& Phi, const f32x4_t& Xlo, const f32x4_t& Xhi) {
  const float sl = __uint_as_float(sp << 16), sh = __uint_as_float(sp & 0xffff0000u);
  const float cl = __builtin_fmaf(-128.0f, sl, __uint_as_float(bp << 16));
  const float ch = __builtin_fmaf(-128.0f, sh, __uint_as_float(bp & 0xffff0000u));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc[i] = __builtin_fmaf(sl, Plo[i], acc[i]);
    acc[i] = __builtin_fmaf(cl, Xlo[i], acc[i]);
    acc[i] = __builtin_fmaf(sh, Phi[i], acc[i]);
    acc[i] = __builtin_fmaf(ch, Xhi[i], acc[i]);
  }
}

template <bool DUAL, bool EVEN_G>
__device__ void qgemm_tile(const QGemmProblem& P, int seg, int nt, int ks, uint16_t* s_x,
                           float* s_red) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, j = lane >> 4;
  const bool lo = j < 2;
  const int64_t e =
      P.seg_exp ? static_cast<int64_t>(min(P.seg_exp[seg], static_cast<uint32_t>(P.n_exp - 1))) : 0;
  const int r0 = P.seg_off ? static_cast<int>(min(P.seg_off[seg], static_cast<uint32_t>(P.rows_max))) : 0;
  const int r1 = P.seg_off ? max(r0, static_cast<int>(min(P.seg_off[seg + 1],
                                                          static_cast<uint32_t>(P.rows_max))))
                           : P.rows_static;
  const int K = P.K, N = P.N, G = K / kGroup, U = (G + 1) / 2;
  const int n = nt * 16 + col;
  const int nc = n < N ? n : N - 1;

  RowPtrs<DUAL> R;
  R.w0 = P.w0 + e * P.ew;
  R.s0 = P.s0 + e * P.es;
  R.b0 = P.b0 + e * P.es;
  if (DUAL) {
    R.w1 = P.w1 + e * P.ew;
    R.s1 = P.s1 + e * P.es;
    R.b1 = P.b1 + e * P.es;
  }
  R.wo = nc * (K / 8);
  R.so = nc * G;
  // this workgroup's units (K slice ks of ksplit), split four ways over its waves
  const int kb = (U * ks) / P.ksplit, ke = (U * (ks + 1)) / P.ksplit;
  const int ub = kb + ((ke - kb) * wave) / kQWaves, ue = kb + ((ke - kb) * (wave + 1)) / kQWaves;
  const int xs = (ke - kb) * 128 + 8;                     // LDS row stride (elements)
  const int kvalid = min((ke - kb) * 128, K - kb * 128);  // slice elements inside K

  // per-lane operand constants: zero on the other group's lanes
  const uint32_t m_lo = lo ? 0x000f000fu : 0u, c_lo = lo ? 0x43004300u : 0u;
  const uint32_t m_hi = lo ? 0u : 0x000f000fu, c_hi = lo ? 0u : 0x43004300u;
  const uint32_t o_lo = lo ? 0x3f803f80u : 0u, o_hi = lo ? 0u : 0x3f803f80u;
  const u32x4_t ones_lo_u = {o_lo, o_lo, o_lo, o_lo}, ones_hi_u = {o_hi, o_hi, o_hi, o_hi};
  const bf16x8_t ones_lo = __builtin_bit_cast(bf16x8_t, ones_lo_u);
  const bf16x8_t ones_hi = __builtin_bit_cast(bf16x8_t, ones_hi_u);
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
  const u32x4_t zero_u = {0u, 0u, 0u, 0u};

  for (int mb = r0; mb < r1; mb += P.rows_per_pass) {
    const int rows = min(P.rows_per_pass, r1 - mb);
    // 1. weight loads of the first two units (independent of the rows)
    // (unit indices are clamped into [0, U-1]: a wave with no units, or the
    // prefetch past its last unit, still reads inside the rows)
    UnitLoad<DUAL, EVEN_G> cur = load_unit<DUAL, EVEN_G>(min(ub, U - 1), G, j, R);
    UnitLoad<DUAL, EVEN_G> nxt = load_unit<DUAL, EVEN_G>(max(0, min(ub + 1, ue - 1)), G, j, R);

    // 2. stage the rows' K slice in LDS (16-byte pieces)
    {
      const int per_row = kvalid / 8;
      for (int i = tid; i < rows * per_row; i += kQThreads) {
        const int rr = i / per_row, pc = i - rr * per_row;
        const int64_t xrow = P.row_map
            ? static_cast<int64_t>(min(P.row_map[mb + rr], static_cast<uint32_t>(P.x_rows - 1)))
            : mb + rr;
        u32x4_t v = *reinterpret_cast<const u32x4_t*>(P.x + xrow * P.ldx + kb * 128 + pc * 8);
        if (P.x_natural) {  // natural order -> P8 (elements 0,4,1,5,2,6,3,7)
          const u32x4_t n = v;
          v[0] = (n[0] & 0xffffu) | (n[2] << 16);
          v[1] = (n[0] >> 16) | (n[2] & 0xffff0000u);
          v[2] = (n[1] & 0xffffu) | (n[3] << 16);
          v[3] = (n[1] >> 16) | (n[3] & 0xffff0000u);
        }
        *reinterpret_cast<u32x4_t*>(s_x + rr * xs + pc * 8) = v;
      }
    }
    __syncthreads();

    // 3. MFMAs, one unit at a time
    f32x4_t acc0 = zero, acc1 = zero;
    const bool vm = col < rows;
    const uint16_t* xl = s_x + min(col, rows - 1) * xs;
#pragma unroll 1
    for (int u = ub; u < ue; ++u) {
      const UnitLoad<DUAL, EVEN_G> nn = load_unit<DUAL, EVEN_G>(min(u + 2, ue - 1), G, j, R);
      const bool has_hi = 2 * u + 1 < G;
      const int xo = (u - kb) * 128 + 32 * (has_hi ? j : (j & 1));  // staged data either way
      bf16x8_t A[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xl + xo + 8 * a);
        A[a] = __builtin_bit_cast(bf16x8_t, vm ? v : zero_u);
      }
      f32x4_t Xlo = zero, Xhi = zero, Plo = zero, Phi = zero;
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        Xlo = mfma16(A[a], ones_lo, Xlo);
        Xhi = mfma16(A[a], ones_hi, Xhi);
      }
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        Plo = mfma16(A[a], nibbles_as_bf16(cur.q0[a], m_lo, c_lo), Plo);
        Phi = mfma16(A[a], nibbles_as_bf16(cur.q0[a], m_hi, c_hi), Phi);
      }
      unit_epilogue(acc0, pair_word<EVEN_G>(cur.s0, cur.s0h, cur.has_hi),
                    pair_word<EVEN_G>(cur.b0, cur.b0h, cur.has_hi), Plo, Phi, Xlo, Xhi);
      if (DUAL) {
        Plo = zero;
        Phi = zero;
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          Plo = mfma16(A[a], nibbles_as_bf16(cur.q1[a], m_lo, c_lo), Plo);
          Phi = mfma16(A[a], nibbles_as_bf16(cur.q1[a], m_hi, c_hi), Phi);
        }
        unit_epilogue(acc1, pair_word<EVEN_G>(cur.s1, cur.s1h, cur.has_hi),
                      pair_word<EVEN_G>(cur.b1, cur.b1h, cur.has_hi), Plo, Phi, Xlo, Xhi);
      }
      cur = nxt;
      nxt = nn;
    }

    // 4. the waves' partial sums meet in LDS; wave 0 adds them in wave order
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
          const int rl = 4 * j + i;  // MFMA output row of register i
          if (rl >= rows) continue;
          const int rr = mb + rl;
          const int64_t orow =
              P.out_map ? static_cast<int64_t>(min(P.out_map[rr], static_cast<uint32_t>(P.out_rows - 1)))
                        : rr;
          if (P.ksplit > 1) {
            P.out_part[(static_cast<int64_t>(ks) * P.out_rows + orow) * N + n] = acc0[i];
          } else {
            uint16_t v;
            if (DUAL)
              v = swiglu_bf16(round_bf16(acc0[i]), round_bf16(acc1[i]));
            else
              v = f32_to_bf16(acc0[i]);
            P.out[orow * P.ldo + ncol] = v;
          }
        }
      }
    }
    __syncthreads();
  }
}

template <bool DUAL, bool EVEN_G>
__device__ inline void qgemm_run(const QGemmProblem& P, int bid, uint16_t* s_x, float* s_red) {
  const int per_seg = P.n_tiles * P.ksplit;
  const int seg = bid / per_seg, rem = bid % per_seg;
  const int nt = rem / P.ksplit, ks = rem % P.ksplit;
  const int n_seg = P.seg_n ? static_cast<int>(min(*P.seg_n, static_cast<uint32_t>(P.max_seg))) : 1;
  if (seg >= n_seg) return;
  qgemm_tile<DUAL, EVEN_G>(P, seg, nt, ks, s_x, s_red);
}

// One grid for one or two problems of the same kind (both SwiGLU pairs or
// both single matrices, both with an even or both with an odd number of
// groups): blocks [0, nblk0) serve p0, the rest p1. Register budgets: 3
// waves/SIMD for SwiGLU pairs, 4 for single matrices.
template <bool DUAL, bool EVEN_G>
__global__ __launch_bounds__(kQThreads) __attribute__((amdgpu_waves_per_eu(DUAL ? 3 : 4, 8)))
void qgemm_kernel(QGemmProblem p0, QGemmProblem p1, int nblk0) {
  extern __shared__ __attribute__((aligned(16))) uint16_t s_x[];
  __shared__ float s_red[(kQWaves - 1) * 8 * kWave];
  const int bid = blockIdx.x;
  if (bid < nblk0)
    qgemm_run<DUAL, EVEN_G>(p0, bid, s_x, s_red);
  else
    qgemm_run<DUAL, EVEN_G>(p1, bid - nblk0, s_x, s_red);
}

// Rows staged per pass and the LDS they take: at most 16 (one MFMA tile),
// at most max_rows (the most rows a segment can hold), and within budget.
static size_t stage_plan(QGemmProblem& p) {
  const int G = p.K / kGroup, U = (G + 1) / 2;
  const int ukw = (U + p.ksplit - 1) / p.ksplit;  // most units a K slice holds
  const size_t row_bytes = static_cast<size_t>(ukw * 128 + 8) * 2;
  int rp = std::min(kQRows, std::max(1, p.max_rows_per_seg));
  while (rp > 1 && rp * row_bytes > kQStageBytes) --rp;
  p.rows_per_pass = rp;
  p.n_tiles = (p.N + 15) / 16;
  return rp * row_bytes;
}

static int blocks_of(const QGemmProblem& p) { return p.max_seg * p.n_tiles * p.ksplit; }

hipError_t launch_qgemm(const QGemmProblem& p0_, const QGemmProblem* p1_, hipStream_t stream) {
  QGemmProblem p0 = p0_;
  if (p0.ksplit < 1) p0.ksplit = 1;
  QGemmProblem p1 = p1_ ? *p1_ : p0;
  if (p1.ksplit < 1) p1.ksplit = 1;
  const bool even0 = ((p0.K / kGroup) & 1) == 0, even1 = ((p1.K / kGroup) & 1) == 0;
  if (p1_ && p1.dual != p0.dual) return hipErrorInvalidValue;
  if (p1_ && even1 != even0) {  // different kinds: two grids
    hipError_t err = launch_qgemm(p0_, nullptr, stream);
    return err != hipSuccess ? err : launch_qgemm(*p1_, nullptr, stream);
  }
  size_t lds = stage_plan(p0);
  if (p1_) lds = std::max(lds, stage_plan(p1));
  const int nblk0 = blocks_of(p0);
  const int nblk1 = p1_ ? blocks_of(p1) : 0;
  if (nblk0 + nblk1 == 0) return hipSuccess;
  const dim3 grid(nblk0 + nblk1), block(kQThreads);
  if (p0.dual && even0)
    hipLaunchKernelGGL((qgemm_kernel<true, true>), grid, block, lds, stream, p0, p1, nblk0);
  else if (p0.dual)
    hipLaunchKernelGGL((qgemm_kernel<true, false>), grid, block, lds, stream, p0, p1, nblk0);
  else if (even0)
    hipLaunchKernelGGL((qgemm_kernel<false, true>), grid, block, lds, stream, p0, p1, nblk0);
  else
    hipLaunchKernelGGL((qgemm_kernel<false, false>), grid, block, lds, stream, p0, p1, nblk0);
  return hipGetLastError();
}

}  // namespace fmx
