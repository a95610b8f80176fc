// fmx_prefill.hip -- the expert GEMMs of the MoE block for prefill batches
// (more than 16 tokens) on packed expert weights (layout: fmx_dev.hpp):
//
//   pf_gemm<true>   gate/up + SwiGLU: the routed experts over their sorted
//                   rows and the shared expert over all tokens, one grid
//   pf_gemm<false>  the down projections of both, one grid
//
// Reference: server/src/model.cpp:673-734 (switch_mlp: gather_qmm over the
// expert-sorted rows, SwiGLU at :715), :736-748 (shared expert MLP), :14-25
// (compiled SwiGLU).
//
// Work item = one pass x one column group. A pass is at most 64 rows that
// share an expert (the sort's pass table cuts every expert's segment of
// sorted rows into passes; the shared expert's passes are 64 consecutive
// tokens). A column group is 4 waves x 4 weight tiles of 16 rows: 128
// SwiGLU columns (2 gate/up tile pairs per wave) or 256 down columns. The
// workgroup walks K in 128-k units through a three-stage LDS ring that LDS
// DMA fills, with no registers held for loads in flight: per unit, the
// pass's activation rows (64 x 256 bytes, gathered through the row map) and
// each wave's four packed blocks (weight words, then all four blocks'
// scale/bias words in one piece). One barrier per unit; after it the unit
// two ahead is issued into the buffer that every wave finished with in the
// previous iteration.
//
// Activation rows sit in LDS as 16-byte chunks XOR-swizzled by row (chunk c
// of row r at slot c ^ (r & 15)), so the 16 lanes that read one k-slice of
// 16 rows hit 16 different slots: the MFMA operand reads are free of bank
// conflicts. The DMA writes a 1 KB piece (4 rows) per instruction and picks
// each lane's source chunk to match.
//
// Weights are dequantised in registers to bf16, s*q + b evaluated in fp32
// and rounded once, and multiplied against every 16-row tile of the pass
// with v_mfma_f32_16x16x32_bf16 (fp32 accumulation): the dequantisation is
// paid once per weight per pass, the MFMAs once per 16 rows.
#include "fmx_dev.hpp"

namespace fmx {

namespace {

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kPfThreads = 256;
constexpr int kPfWaves = kPfThreads / kWave;
constexpr int kPfMT = kPassRows / 16;                        // 16-row tiles per pass
constexpr int kPfABytes = kPassRows * 256;                   // a pass's rows, one unit
// a wave's share of one unit: the weight words of its blocks (4 KB: 2 pairs
// or 4 singles), then their (scale, bias) words (512 bytes) and 512 bytes
// that the idle half of the DMA wave writes
constexpr int kPfWaveBBytes = 4096 + 1024;
constexpr int kPfStageBytes = kPfABytes + kPfWaves * kPfWaveBBytes;
constexpr int kPfStages = 3;

template <bool DUAL>
constexpr int pf_nb() { return DUAL ? 2 : 4; }  // packed blocks per wave
// LDS DMA instructions one wave issues per unit: its row pieces, the 1 KB
// weight pieces of its blocks and one for all their (scale, bias) words.
// Every one runs with all lanes on: a DMA under a lane condition may be
// duplicated into both arms of a branch by the compiler, and the wait counts
// below count instructions.
template <bool DUAL>
constexpr int pf_insts() { return kPfMT + 4 + 1; }

__device__ inline void dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

__device__ inline uint32_t pack_bf16x2(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// The 8 weights of a packed word (element 2i at nibble position i, 2i + 1 at
// i + 4) as bf16(s*q + b) in natural element order. Masking the even and the
// odd nibble positions into bytes lets v_cvt_f32_ubyte{0..3} read each
// weight directly (bytes 0..3 of lo: elements 0, 4, 1, 5; of hi: 2, 6, 3, 7).
__device__ inline bf16x8_t dq8(uint32_t w, float s, float b) {
  uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
  // keeps the byte extracts below from folding into per-nibble bit-field
  // extracts (one more instruction per weight)
  asm volatile("" : "+v"(lo), "+v"(hi));
  auto q = [](uint32_t v, int i) { return static_cast<float>((v >> (8 * i)) & 0xffu); };
  u32x4_t d;
  d[0] = pack_bf16x2(__builtin_fmaf(s, q(lo, 0), b), __builtin_fmaf(s, q(lo, 2), b));
  d[1] = pack_bf16x2(__builtin_fmaf(s, q(hi, 0), b), __builtin_fmaf(s, q(hi, 2), b));
  d[2] = pack_bf16x2(__builtin_fmaf(s, q(lo, 1), b), __builtin_fmaf(s, q(lo, 3), b));
  d[3] = pack_bf16x2(__builtin_fmaf(s, q(hi, 1), b), __builtin_fmaf(s, q(hi, 3), b));
  return __builtin_bit_cast(bf16x8_t, d);
}

template <bool DUAL>
__global__ __launch_bounds__(kPfThreads) void pf_gemm(PfArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t s_pf[];
  constexpr int NB = pf_nb<DUAL>(), NM = DUAL ? 2 : 1;
  constexpr int BB = DUAL ? kBlockPair : kBlockSingle;
  constexpr int PER = pf_insts<DUAL>();

  int item = blockIdx.x;
  const bool second = item >= a.n_items0;
  if (second) item -= a.n_items0;
  const PfSet& P = second ? a.s1 : a.s0;
  const int pass = item / P.ng, ng = item - pass * P.ng;

  // ---- the pass: rows [row0, row0 + rows) of expert e
  int row0, rows;
  int64_t e = 0;
  if (P.pass_n) {
    const int np = min(static_cast<int>(*P.pass_n), P.max_pass);
    if (pass >= np) return;
    const u32x2_t t = *reinterpret_cast<const u32x2_t*>(P.pass_tab + 2 * pass);
    row0 = min(static_cast<int>(t[0]), P.rows_max);
    rows = min(min(static_cast<int>(t[1] >> 16), kPassRows), P.rows_max - row0);
    e = min(static_cast<int>(t[1] & 0xffffu), P.n_exp - 1);
  } else {
    row0 = pass * kPassRows;
    rows = min(kPassRows, P.rows_static - row0);
  }
  if (rows <= 0) return;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i16 = lane & 15, j = lane >> 4;
  const int nu = P.nu;

  // ---- sources: this wave's packed blocks (tiles past the matrix re-read
  // its last tile and are not stored) and its row pieces' lanes
  const int tile0 = (ng * kPfWaves + wave) * NB;
  const uint8_t* wexp = P.w + e * P.es;
  const uint8_t* bsrc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
    bsrc[b] = wexp + static_cast<int64_t>(min(tile0 + b, P.nt - 1)) * nu * BB;
  const uint16_t* asrc[kPfMT];
#pragma unroll
  for (int pc = 0; pc < kPfMT; ++pc) {
    const int r = 4 * (pc * kPfWaves + wave) + j;  // pass row of this lane's chunk
    const int rr = min(r, rows - 1);               // rows past the pass repeat its last
    int64_t xr = row0 + rr;
    if (P.row_map) xr = min(P.row_map[row0 + rr], static_cast<uint32_t>(P.x_rows - 1));
    asrc[pc] = P.x + xr * P.ldx + 8 * (i16 ^ (r & 15));
  }

  // the (scale, bias) piece: lane l < 32 fetches 16 bytes of block l / SBL's
  // 16 x 8 (single) or 2 x 16 x 8 (pair) bytes; lanes 32..63 repeat lanes
  // 0..31 into the spare 512 bytes
  constexpr int SBL = 32 / NB;  // lanes per block
  const int sbl = lane & 31;
  const int sb_blk = sbl / SBL, sb_off = NM * 1024 + 16 * (sbl % SBL);

  auto issue = [&](int u, int st) {
    uint8_t* sa = s_pf + st * kPfStageBytes;
#pragma unroll
    for (int pc = 0; pc < kPfMT; ++pc) dma16(asrc[pc] + u * 128, sa + (pc * kPfWaves + wave) * 1024);
    uint8_t* sb = sa + kPfABytes + wave * kPfWaveBBytes;
    const int64_t uo = static_cast<int64_t>(u) * BB;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int m = 0; m < NM; ++m) dma16(bsrc[b] + uo + m * 1024 + 16 * lane, sb + (b * NM + m) * 1024);
    const uint8_t* gs = bsrc[0] + uo + sb_off;
#pragma unroll
    for (int b = 1; b < NB; ++b)
      if (sb_blk == b) gs = bsrc[b] + uo + sb_off;
    dma16(gs, sb + 4096);
  };

  f32x4_t acc[kPfMT][NB][NM];
#pragma unroll
  for (int mt = 0; mt < kPfMT; ++mt)
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int m = 0; m < NM; ++m) acc[mt][b][m] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  issue(0, 0);
  if (nu > 1) issue(1, 1);
  for (int u = 0; u < nu; ++u) {
    // this wave's DMA of unit u has landed (only unit u + 1's may still be
    // in flight); after the barrier every wave's has, and every wave is done
    // with the buffer of unit u - 1
    if (u + 1 < nu)
      wait_vmcnt<PER>();
    else
      wait_vmcnt0();
    lds_dma_barrier();
    if (u + 2 < nu) issue(u + 2, (u + 2) % kPfStages);

    const uint8_t* sa = s_pf + (u % kPfStages) * kPfStageBytes;
    const uint8_t* sb = sa + kPfABytes + wave * kPfWaveBBytes;
    bf16x8_t B[NB][NM][4];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        const u32x4_t W = *reinterpret_cast<const u32x4_t*>(sb + (b * NM + m) * 1024 + 16 * lane);
        const u32x2_t sbw = *reinterpret_cast<const u32x2_t*>(sb + 4096 + b * (NM * 128) + m * 128 + 8 * i16);
        const float s0 = __uint_as_float(sbw[0] << 16), s1 = __uint_as_float(sbw[0] & 0xffff0000u);
        const float b0 = __uint_as_float(sbw[1] << 16), b1 = __uint_as_float(sbw[1] & 0xffff0000u);
        B[b][m][0] = dq8(W[0], s0, b0);
        B[b][m][1] = dq8(W[1], s0, b0);
        B[b][m][2] = dq8(W[2], s1, b1);
        B[b][m][3] = dq8(W[3], s1, b1);
      }
    }
#pragma unroll
    for (int mt = 0; mt < kPfMT; ++mt) {
      if (16 * mt >= rows) break;
      const uint8_t* ar = sa + (16 * mt + i16) * 256;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const bf16x8_t A = *reinterpret_cast<const bf16x8_t*>(ar + (((4 * q + j) ^ i16) << 4));
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int m = 0; m < NM; ++m) acc[mt][b][m] = mfma_bf16(A, B[b][m][q], acc[mt][b][m]);
      }
    }
  }

  // ---- epilogue: lane (i16, j) holds rows 4j + r of each 16-row tile, column i16
#pragma unroll
  for (int mt = 0; mt < kPfMT; ++mt) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int t = tile0 + b;
      if (t >= P.nt) continue;
      const int col = t * 16 + i16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * mt + 4 * j + r;
        if (row >= rows) continue;
        uint16_t v;
        if (DUAL)
          v = swiglu_bf16(round_bf16(acc[mt][b][0][r]), round_bf16(acc[mt][b][NM - 1][r]));
        else
          v = f32_to_bf16(acc[mt][b][0][r]);
        P.out[static_cast<int64_t>(row0 + row) * P.ldo + col] = v;
      }
    }
  }
}

}  // namespace

int pf_items(PfSet& s, bool dual) {
  const int per_group = kPfWaves * (dual ? pf_nb<true>() : pf_nb<false>());
  s.ng = (s.nt + per_group - 1) / per_group;
  const int passes = s.pass_n ? s.max_pass : (s.rows_static + kPassRows - 1) / kPassRows;
  return passes * s.ng;
}

size_t pf_lds_bytes() { return static_cast<size_t>(kPfStages) * kPfStageBytes; }

hipError_t launch_pf(const PfArgs& a, bool dual, hipStream_t stream) {
  const int n = a.n_items0 + a.n_items1;
  if (n == 0) return hipSuccess;
  if (dual)
    hipLaunchKernelGGL(pf_gemm<true>, dim3(n), dim3(kPfThreads), pf_lds_bytes(), stream, a);
  else
    hipLaunchKernelGGL(pf_gemm<false>, dim3(n), dim3(kPfThreads), pf_lds_bytes(), stream, a);
  return hipGetLastError();
}

}  // namespace fmx
