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
// tokens). A column group is 4 waves x 2 weight tiles of 16 rows: 64
// SwiGLU columns (one gate/up tile pair per wave) or 128 down columns. The
// workgroup walks K in 128-k units through a ring of LDS stages that LDS
// DMA fills, with no registers held for loads in flight: per unit, the
// pass's activation rows (its 16-row tiles x 256 bytes, gathered through
// the row map) and each wave's two packed blocks (weight words, then both
// blocks' scale/bias words in one 4-byte-per-lane piece). One barrier per
// unit; after it the unit kPfStages - 1 ahead is issued into the buffer
// that every wave finished with in the previous iteration. Two stages
// (50 KB) let three workgroups share a CU, so one's dequantisation
// overlaps the others' MFMAs and loads.
//
// Activation rows sit in LDS as 16-byte chunks XOR-swizzled by row (chunk c
// of row r at slot c ^ (r & 15)), so the 16 lanes that read one k-slice of
// 16 rows hit 16 different slots: the MFMA operand reads are free of bank
// conflicts. The DMA writes a 1 KB piece (4 rows) per instruction and picks
// each lane's source chunk to match.
//
// Arithmetic: the weights are dequantised once per pass into fp16 (s*q + b
// rounded once, 2^-11 relative) and multiplied with
// v_mfma_f32_16x16x32_f16 against fp16 copies of the activation rows
// (exact for bf16 magnitudes in [2^-14, 65536); smaller ones round to
// fp16's subnormal grid, at most 2^-25 off; the copies are written in the
// P8 layout, fmx_dev.hpp, by the router for x and by this gate/up grid for h).
// When a row holds a value outside fp16's range (the forward's flag word
// says so) the grid takes the exact bf16 path instead: nibbles become the
// bf16 values 128 + q, the MFMA forms P = x.(128+q) and X = x.1 per
// quantisation group in fp32, and each group adds s P + (b - 128 s) X to the
// accumulator. (Weights rounded to bf16, as MLX's GPU kernels stage them,
// cost 0.5 % relative L2 error of the block output at 512 tokens and put
// single elements outside the bf16 parity tolerance; fp16 weights cost
// 0.06 %.)
// A float16 block (io_f16) brings fp16 rows, scales and biases: the same
// fp16 arithmetic, SwiGLU and outputs rounded to fp16, never the exact path.
//
// The single-matrix grid also reads weights in MLX's own layout (words of
// 8 nibbles along K per row, scales and biases per row and group), for
// quantized_matmul and gather_qmm with more than 16 rows: lane (i16, j)
// moves words 4j..4j+3 of row i16 of the unit (the same 1 KB piece per
// block), the (scale, bias) DMA takes each row's two 4-byte pairs from the
// two arrays, and a lane reads its k-slice's word from the piece it sits in.
// An MLX word's nibbles convert in another order than a packed word's, so
// the rows come in matching copies: fp16 in the Q8 layout, bf16 in the P8
// layout (fmx_dev.hpp), and out_map scatters the sorted rows of gather_qmm
// back to their output rows.
#include <algorithm>

#include "fmx_dev.hpp"

namespace fmx {

namespace {

constexpr int kPfThreads = 256;
constexpr int kPfWaves = kPfThreads / kWave;
constexpr int kPfMT = kPassRows / 16;                        // 16-row tiles per pass
constexpr int kPfABytes = kPassRows * 256;                   // a pass's rows, one unit
constexpr int kPfStages = 2;
constexpr int kXcds = 8;  // MI355X: 8 XCDs, each with its own L2

// Packed blocks per wave: one gate/up pair or two single blocks (2 KB of
// weight words per unit), so a workgroup's two stages fit three workgroups
// in a CU's LDS.
template <bool DUAL>
constexpr int pf_nb() { return DUAL ? 1 : 2; }
template <bool DUAL>
constexpr int pf_nm() { return DUAL ? 2 : 1; }
// a wave's share of one unit: its 1 KB weight pieces, then the blocks'
// (scale, bias) words (256 bytes, one 4-byte DMA per lane)
template <bool DUAL>
constexpr int pf_wave_bbytes() { return pf_nb<DUAL>() * pf_nm<DUAL>() * 1024 + 256; }
template <bool DUAL>
constexpr int pf_stage_bytes() { return kPfABytes + kPfWaves * pf_wave_bbytes<DUAL>(); }

// LDS DMA instructions one wave issues per unit: its row pieces (one per
// 16-row tile the pass fills), the 1 KB weight pieces of its blocks and one
// for all their (scale, bias) words. Every one runs with all lanes on: a
// DMA under a lane condition may be duplicated into both arms of a branch by
// the compiler, and the wait counts below count instructions.

__device__ inline void dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}
__device__ inline void dma4(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 4, 0, 0);
}

// One unit's products: the pass's rows in LDS at sa (16-byte chunks
// XOR-swizzled by row), the wave's packed words W and (scale, bias) pairs
// SB, accumulated into acc.
template <bool DUAL, int MT, bool F16, bool MLX>
__device__ __attribute__((always_inline)) void pf_unit(const PfSet& P, const uint8_t* sa,
                                                       const u32x4_t (&W)[pf_nb<DUAL>()][pf_nm<DUAL>()],
                                                       const u32x2_t (&SB)[pf_nb<DUAL>()][pf_nm<DUAL>()],
                                                       f32x4_t (&acc)[MT][pf_nb<DUAL>()][pf_nm<DUAL>()], int i16,
                                                       int j) {
  constexpr int NB = pf_nb<DUAL>(), NM = pf_nm<DUAL>();
  if constexpr (F16) {
    // every activation operand of the unit is read up front (one LDS round
    // trip per unit, not one per k-slice)
    f16x8_t A[4][MT];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        A[q][mt] = *reinterpret_cast<const f16x8_t*>(sa + (16 * mt + i16) * 256 + (((4 * q + j) ^ i16) << 4));
    f16x2_t sc[NB][NM][2], bs[NB][NM][2];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        if (P.io_f16) {  // float16 scales and biases: the values as they are
          sc[b][m][0] = __builtin_bit_cast(f16x2_t, (SB[b][m][0] & 0xffffu) * 0x10001u);
          sc[b][m][1] = __builtin_bit_cast(f16x2_t, (SB[b][m][0] >> 16) * 0x10001u);
          bs[b][m][0] = __builtin_bit_cast(f16x2_t, (SB[b][m][1] & 0xffffu) * 0x10001u);
          bs[b][m][1] = __builtin_bit_cast(f16x2_t, (SB[b][m][1] >> 16) * 0x10001u);
        } else {
          sc[b][m][0] = f16_splat(__uint_as_float(SB[b][m][0] << 16));
          sc[b][m][1] = f16_splat(__uint_as_float(SB[b][m][0] & 0xffff0000u));
          bs[b][m][0] = f16_splat(__uint_as_float(SB[b][m][1] << 16));
          bs[b][m][1] = f16_splat(__uint_as_float(SB[b][m][1] & 0xffff0000u));
        }
      }
    __builtin_amdgcn_sched_barrier(0);
    // k-slice q (32 k) of quantisation group q / 2: the weights dequantised
    // once, multiplied against every 16-row tile of the pass
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          const f16x8_t B = dq8_f16(W[b][m][q], sc[b][m][q >> 1], bs[b][m][q >> 1]);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[mt][b][m] = mfma_f16(A[q][mt], B, acc[mt][b][m]);
        }
  } else {
    float sc[NB][NM][2], cb[NB][NM][2];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        sc[b][m][0] = __uint_as_float(SB[b][m][0] << 16);
        sc[b][m][1] = __uint_as_float(SB[b][m][0] & 0xffff0000u);
        cb[b][m][0] = __builtin_fmaf(-128.0f, sc[b][m][0], __uint_as_float(SB[b][m][1] << 16));
        cb[b][m][1] = __builtin_fmaf(-128.0f, sc[b][m][1], __uint_as_float(SB[b][m][1] & 0xffff0000u));
      }
    // exact dequantisation, one quantisation group (two k-slices) at a time:
    // P = x.(128+q) and X = x.1 by MFMA, then acc += s P + (b - 128 s) X
    // (the group's activation operands only are held, which keeps this
    // path within the register budget of the fp16 path)
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
    const u32x4_t ones_u = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
    const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, ones_u);
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      bf16x8_t A[4][MT];
#pragma unroll
      for (int q = 2 * g; q < 2 * g + 2; ++q)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          A[q][mt] = *reinterpret_cast<const bf16x8_t*>(sa + (16 * mt + i16) * 256 + (((4 * q + j) ^ i16) << 4));
      f32x4_t X[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) X[mt] = mfma_bf16(A[2 * g + 1][mt], ones, mfma_bf16(A[2 * g][mt], ones, zero));
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          const bf16x8_t B0 = nib8(W[b][m][2 * g]), B1 = nib8(W[b][m][2 * g + 1]);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const f32x4_t Pg = mfma_bf16(A[2 * g + 1][mt], B1, mfma_bf16(A[2 * g][mt], B0, zero));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              acc[mt][b][m][i] = __builtin_fmaf(sc[b][m][g], Pg[i], acc[mt][b][m][i]);
              acc[mt][b][m][i] = __builtin_fmaf(cb[b][m][g], X[mt][i], acc[mt][b][m][i]);
            }
          }
        }
    }
  }
}

// The work item's outputs from acc (rows [row0, row0 + rows), the wave's
// tiles from tile0, K slice ks).
template <bool DUAL, int MT, bool MLX>
__device__ __attribute__((always_inline)) void pf_epilogue(const PfSet& P,
                                                           f32x4_t (&acc)[MT][pf_nb<DUAL>()][pf_nm<DUAL>()],
                                                           int tile0, int row0, int rows, int ks, int i16, int j,
                                                           int lane, uint32_t* flag, uint32_t flag_out) {
  constexpr int NB = pf_nb<DUAL>(), NM = pf_nm<DUAL>();
  // ---- epilogue: lane (i16, j) holds rows 4j + r of each 16-row tile,
  // column i16; gate/up (and a relu^2 up projection) also writes its rows
  // in fp16 (P8 layout) for the down grid and flags values outside fp16's
  // range
  bool ovf = false;
  float* const out32 = P.out32 ? P.out32 + ks * P.part_stride : nullptr;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int t = tile0 + b;
      if (t >= P.nt) continue;
      const int col = t * 16 + i16;
      const int colh = (col & ~7) | p8_slot(col & 7);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * mt + 4 * j + r;
        if (row >= rows) continue;
        const int64_t orow =
            static_cast<int64_t>((MLX && P.out_map) ? min(P.out_map[row0 + row], static_cast<uint32_t>(P.rows_max - 1))
                                                    : row0 + row) * P.ldo;
        if (DUAL && P.io_f16) {  // a float16 block: fp16 SwiGLU, both copies fp16
          const uint16_t v = swiglu_f16(round_f16(acc[mt][b][0][r]), round_f16(acc[mt][b][NM - 1][r]));
          P.out[orow + col] = v;
          P.outh[orow + colh] = v;
        } else if (DUAL) {
          const uint16_t v = swiglu_bf16(round_bf16(acc[mt][b][0][r]), round_bf16(acc[mt][b][NM - 1][r]));
          P.out[orow + col] = v;
          ovf |= bf16_f16_overflow(v);
          P.outh[orow + colh] = static_cast<uint16_t>(bf16_to_f16_bits(v));
        } else if (out32) {
          out32[orow + col] = acc[mt][b][0][r];
        } else if (P.act) {
          // relu^2 of the bf16 product (Nemotron-H, nemotron_h.cpp:54-63):
          // exact in fp32; bf16 and fp16 copies for the down grid
          const float hv = fmaxf(round_bf16(acc[mt][b][0][r]), 0.0f);
          const float av = hv * hv;
          P.out[orow + col] = f32_to_bf16(av);
          ovf |= av >= 65504.0f;
          P.outh[orow + colh] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(av));
        } else if (P.io_f16) {
          P.out[orow + col] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(acc[mt][b][0][r]));
        } else {
          uint16_t v = f32_to_bf16(acc[mt][b][0][r]);
          if (P.bias) v = f32_to_bf16(bf16_to_f32(v) + bf16_to_f32(P.bias[col]));
          if (P.res)
            v = f32_to_bf16(bf16_to_f32(P.res[static_cast<int64_t>(row0 + row) * P.ldr + col]) + bf16_to_f32(v));
          P.out[orow + col] = v;
        }
      }
    }
  }
  if ((DUAL || P.act) && __ballot(ovf) && lane == 0) atomicOr(flag, flag_out);
}

// One work item: rows [row0, row0 + rows) (rows <= 16 MT) of expert e's
// weights, column group ng. MT (the 16-row tiles the rows fill) fixes how
// many row pieces each wave moves per unit, so the pass's rows are moved
// and multiplied once, without padding to kPassRows.
template <bool DUAL, int MT, bool F16, bool MLX>
__device__ __attribute__((always_inline)) void pf_item(const PfSet& P, int ng, int row0, int rows,
                                                       int64_t e, int ks, uint8_t* s_pf,
                                                       uint32_t* flag, uint32_t flag_out) {
  constexpr int NB = pf_nb<DUAL>(), NM = pf_nm<DUAL>();
  constexpr int BB = DUAL ? kBlockPair : kBlockSingle;
  constexpr int PA = (4 * MT + kPfWaves - 1) / kPfWaves;  // 4-row pieces per wave and unit
  constexpr int PER = PA + NB * NM + 1;                  // LDS DMA instructions per wave and unit
  constexpr int WB = pf_wave_bbytes<DUAL>(), SBO = NB * NM * 1024;  // wave's stage share, its sb offset
  constexpr int STAGE = pf_stage_bytes<DUAL>();
  static_assert(NB * NM * 128 == 256, "the blocks' (scale, bias) words fill one 4-byte DMA");
  static_assert(!MLX || !DUAL, "MLX-layout weights: single matrices only");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i16 = lane & 15, j = lane >> 4;
  // K slice ks of the set's ksplit: units [kb, kb + nu) of the P.nu
  const int kn = max(P.ksplit, 1);
  const int kb = (P.nu * ks) / kn;
  const int nu = (P.nu * (ks + 1)) / kn - kb;

  // ---- sources: this wave's packed blocks (tiles past the matrix re-read
  // its last tile and are not stored) and its row pieces' lanes
  const int tile0 = (ng * kPfWaves + wave) * NB;
  const uint8_t* wexp = MLX ? nullptr : P.w + e * P.es;
  const uint8_t* bsrc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if constexpr (MLX) {
      // MLX layout: lane (i16, j) moves words 4j .. 4j + 3 of the unit in
      // row i16 of the tile (64 contiguous bytes per row and unit)
      const int64_t row = static_cast<int64_t>(e) * P.nt * 16 + min(tile0 + b, P.nt - 1) * 16 + i16;
      bsrc[b] = reinterpret_cast<const uint8_t*>(P.mw + row * (P.nu * 16) + 16 * kb + 4 * j);
    } else {
      bsrc[b] = wexp + (static_cast<int64_t>(min(tile0 + b, P.nt - 1)) * P.nu + kb) * BB;
    }
  }
  const uint16_t* asrc[PA];
#pragma unroll
  for (int pc = 0; pc < PA; ++pc) {
    const int r = 4 * (pc * kPfWaves + wave) + j;  // pass row of this lane's chunk
    const int rr = min(r, rows - 1);               // rows past the pass repeat its last
    int64_t xr = row0 + rr;
    if (P.row_map) xr = min(P.row_map[row0 + rr], static_cast<uint32_t>(P.x_rows - 1));
    asrc[pc] = (F16 ? P.xh : P.x) + xr * P.ldx + 128 * kb + 8 * (i16 ^ (r & 15));
  }

  // the (scale, bias) piece: lane l fetches 4 bytes of block l / SBL's
  // 16 x 8 (single) or 2 x 16 x 8 (pair) bytes
  constexpr int SBL = kWave / NB;  // lanes per block
  const uint8_t* sb_src;
  if constexpr (MLX) {
    // the scale (even lanes) or bias (odd lanes) pair of groups 2u, 2u + 1
    // of row (lane % 32) / 2 of block lane / 32, at the place of the
    // packed block's (scale, bias) word
    const int64_t row = static_cast<int64_t>(e) * P.nt * 16 + min(tile0 + lane / SBL, P.nt - 1) * 16 +
                        (lane % SBL) / 2;
    sb_src = reinterpret_cast<const uint8_t*>((lane & 1 ? P.mb : P.ms) + row * (P.nu * 2) + 2 * kb);
  } else {
    sb_src = wexp + (static_cast<int64_t>(min(tile0 + lane / SBL, P.nt - 1)) * P.nu + kb) * BB + NM * 1024 +
             4 * (lane % SBL);
  }

  auto issue = [&](int u, int st) {
    uint8_t* sa = s_pf + st * STAGE;
#pragma unroll
    for (int pc = 0; pc < PA; ++pc) dma16(asrc[pc] + u * 128, sa + (pc * kPfWaves + wave) * 1024);
    uint8_t* sb = sa + kPfABytes + wave * WB;
    if constexpr (MLX) {
#pragma unroll
      for (int b = 0; b < NB; ++b) dma16(bsrc[b] + 64 * u, sb + b * 1024);
      dma4(sb_src + 4 * u, sb + SBO);
    } else {
      const int64_t uo = static_cast<int64_t>(u) * BB;
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int m = 0; m < NM; ++m) dma16(bsrc[b] + uo + m * 1024 + 16 * lane, sb + (b * NM + m) * 1024);
      dma4(sb_src + uo, sb + SBO);
    }
  };

  f32x4_t acc[MT][NB][NM];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int m = 0; m < NM; ++m) acc[mt][b][m] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // the ring: units u + 1 .. u + kPfStages - 2 are in flight while unit u
  // is multiplied; unit u + kPfStages - 1 is issued into the buffer of u - 1
#pragma unroll
  for (int st = 0; st < kPfStages - 1; ++st)
    if (st < nu) issue(st, st);
  for (int u = 0; u < nu; ++u) {
    // this wave's DMA of unit u has landed (only later units' may still be
    // in flight); after the barrier every wave's has, and every wave is done
    // with the buffer of unit u - 1
    const int ahead = min(kPfStages - 2, nu - 1 - u);
    if (ahead >= 2)
      wait_vmcnt<2 * PER>();
    else if (ahead == 1)
      wait_vmcnt<PER>();
    else
      wait_vmcnt0();
    lds_dma_barrier();
    if (u + kPfStages - 1 < nu) issue(u + kPfStages - 1, (u + kPfStages - 1) % kPfStages);

    const uint8_t* sa = s_pf + (u % kPfStages) * STAGE;
    const uint8_t* sb = sa + kPfABytes + wave * WB;
    // the unit's packed words and (scale, bias) pairs
    u32x4_t W[NB][NM];
    u32x2_t SB[NB][NM];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        if constexpr (MLX) {
          // word 4q + j of row i16 (k-slice q) sits in lane 16q + i16's piece
#pragma unroll
          for (int q = 0; q < 4; ++q)
            W[b][m][q] = *reinterpret_cast<const uint32_t*>(sb + b * 1024 + 256 * q + 16 * i16 + 4 * j);
        } else {
          W[b][m] = *reinterpret_cast<const u32x4_t*>(sb + (b * NM + m) * 1024 + 16 * lane);
        }
        SB[b][m] = *reinterpret_cast<const u32x2_t*>(sb + SBO + b * (NM * 128) + m * 128 + 8 * i16);
      }
    pf_unit<DUAL, MT, F16, MLX>(P, sa, W, SB, acc, i16, j);
  }
  pf_epilogue<DUAL, MT, MLX>(P, acc, tile0, row0, rows, ks, i16, j, lane, flag, flag_out);
}

// Block -> work item. The hardware dispatches block b to XCD b % 8, each
// XCD taking its blocks in order. Each XCD takes a contiguous eighth of the
// routed passes and runs all column groups of one pass back to back, so the
// pass's rows are fetched into that XCD's L2 once and an expert's further
// passes find its weights there; the shared expert's column
// groups go round-robin and an XCD runs all passes of one group back to
// back, so the group's weights are fetched once. Blocks past the work
// (padding, passes the sort did not fill) exit.
template <bool DUAL, bool MLX>
__device__ __attribute__((always_inline)) void pf_grid(const PfArgs& a, uint8_t* s_pf) {
  int b = blockIdx.x;
  const bool second = b >= a.n_items0;
  if (second) b -= a.n_items0;
  const PfSet& P = second ? a.s1 : a.s0;
  const int x = b % kXcds, l = b / kXcds;
  int pass, ng, ks = 0;
  if (P.pass_n) {
    // XCD x takes a contiguous range of the pass table, so an expert's
    // passes (consecutive in the table) run back to back on one L2; the
    // ranges differ in length by at most one pass
    const int npass = min(static_cast<int>(*P.pass_n), P.max_pass);
    const int lo = (x * npass) / kXcds, hi = ((x + 1) * npass) / kXcds;
    if (l / P.ng >= hi - lo) return;
    pass = lo + l / P.ng;
    ng = l % P.ng;
  } else {
    // XCD x runs every pass and K slice of one column group back to back
    const int pr = P.pass_rows > 0 ? min(P.pass_rows, kPassRows) : kPassRows;
    const int np = (P.rows_static + pr - 1) / pr;
    const int per = np * max(P.ksplit, 1);
    ng = x + kXcds * (l / per);
    pass = (l % per) % np;
    ks = (l % per) / np;
    if (ng >= P.ng) return;
  }

  // ---- the pass: rows [row0, row0 + rows) of expert e
  int row0, rows;
  int64_t e = 0;
  if (P.pass_n) {
    const int npass = min(static_cast<int>(*P.pass_n), P.max_pass);
    if (pass >= npass) return;
    const u32x2_t t = *reinterpret_cast<const u32x2_t*>(P.pass_tab + 2 * pass);
    row0 = min(static_cast<int>(t[0]), P.rows_max);
    rows = min(min(static_cast<int>(t[1] >> 16), kPassRows), P.rows_max - row0);
    e = min(static_cast<int>(t[1] & 0xffffu), P.n_exp - 1);
  } else {
    const int pr = P.pass_rows > 0 ? min(P.pass_rows, kPassRows) : kPassRows;
    row0 = pass * pr;
    rows = min(pr, P.rows_static - row0);
  }
  if (rows <= 0) return;
  // one call site per tile count and arithmetic: each inlined copy is
  // compiled on its own
  static_assert(kPfMT == 4, "row-tile dispatch below covers passes of up to 4 tiles");
  bool exact;
  if (MLX && a.n_flag > 1) {
    // OR of the copy kernel's per-block words (at most 4 per lane: one load)
    const int i = 4 * (threadIdx.x & 63);
    uint32_t v = 0;
    if (i < a.n_flag) {
      const u32x4_t f = *reinterpret_cast<const u32x4_t*>(a.f16_flag + i);
      v = f[0] | (i + 1 < a.n_flag ? f[1] : 0u) | (i + 2 < a.n_flag ? f[2] : 0u) | (i + 3 < a.n_flag ? f[3] : 0u);
    }
    exact = __ballot((v & a.flag_in) != 0) != 0;
  } else {
    exact = __builtin_amdgcn_readfirstlane(*a.f16_flag & a.flag_in) != 0;
  }
  if (exact) {
    switch ((rows + 15) / 16) {
      case 1: pf_item<DUAL, 1, false, MLX>(P, ng, row0, rows, e, ks, s_pf, a.f16_flag, a.flag_out); break;
      case 2: pf_item<DUAL, 2, false, MLX>(P, ng, row0, rows, e, ks, s_pf, a.f16_flag, a.flag_out); break;
      case 3: pf_item<DUAL, 3, false, MLX>(P, ng, row0, rows, e, ks, s_pf, a.f16_flag, a.flag_out); break;
      default: pf_item<DUAL, 4, false, MLX>(P, ng, row0, rows, e, ks, s_pf, a.f16_flag, a.flag_out); break;
    }
  } else {
    switch ((rows + 15) / 16) {
      case 1: pf_item<DUAL, 1, true, MLX>(P, ng, row0, rows, e, ks, s_pf, a.f16_flag, a.flag_out); break;
      case 2: pf_item<DUAL, 2, true, MLX>(P, ng, row0, rows, e, ks, s_pf, a.f16_flag, a.flag_out); break;
      case 3: pf_item<DUAL, 3, true, MLX>(P, ng, row0, rows, e, ks, s_pf, a.f16_flag, a.flag_out); break;
      default: pf_item<DUAL, 4, true, MLX>(P, ng, row0, rows, e, ks, s_pf, a.f16_flag, a.flag_out); break;
    }
  }
}

template <bool DUAL>
__global__ __launch_bounds__(kPfThreads) void pf_gemm(PfArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t s_pf[];
  pf_grid<DUAL, false>(a, s_pf);
}

// MLX-layout weights: the lane's word reads and row-map scatter take a few
// registers more, which would leave two waves per SIMD; held to three
__global__ __launch_bounds__(kPfThreads) __attribute__((amdgpu_waves_per_eu(3))) void pf_gemm_mlx(PfArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t s_pf[];
  pf_grid<false, true>(a, s_pf);
}

}  // namespace

int pf_items(PfSet& s, bool dual) {
  const int per_group = kPfWaves * (dual ? pf_nb<true>() : pf_nb<false>());
  s.ng = (s.nt + per_group - 1) / per_group;
  if (s.pass_n)  // pass-major per XCD
    return kXcds * s.ng * ((s.max_pass + kXcds - 1) / kXcds);
  const int pr = s.pass_rows > 0 ? std::min(s.pass_rows, kPassRows) : kPassRows;
  const int np = (s.rows_static + pr - 1) / pr;  // group-major per XCD
  return kXcds * np * max(s.ksplit, 1) * ((s.ng + kXcds - 1) / kXcds);
}

size_t pf_lds_bytes(bool dual) {
  return static_cast<size_t>(kPfStages) * (dual ? pf_stage_bytes<true>() : pf_stage_bytes<false>());
}

hipError_t launch_pf(const PfArgs& a, bool dual, hipStream_t stream) {
  const int n = a.n_items0 + a.n_items1;
  if (n == 0) return hipSuccess;
  // K slices only for static single-matrix sets with fp32 outputs
  for (const PfSet* s : {&a.s0, &a.s1})
    if (s->ksplit > 1 && (dual || s->pass_n || !s->out32 || s->ksplit > s->nu)) return hipErrorInvalidValue;
  // per-block flag words: at most 4 per lane, 16-byte aligned
  if (a.n_flag > 4 * kWave || (a.n_flag > 1 && (reinterpret_cast<uintptr_t>(a.f16_flag) & 15)))
    return hipErrorInvalidValue;
  // MLX-layout weights: single matrices, every set with items in that layout
  const bool mlx = (a.n_items0 ? a.s0.mw : a.s1.mw) != nullptr;
  if (mlx && (dual || (a.n_items0 && !a.s0.mw) || (a.n_items1 && !a.s1.mw))) return hipErrorInvalidValue;
  if (dual)
    hipLaunchKernelGGL(pf_gemm<true>, dim3(n), dim3(kPfThreads), pf_lds_bytes(true), stream, a);
  else if (mlx)
    hipLaunchKernelGGL(pf_gemm_mlx, dim3(n), dim3(kPfThreads), pf_lds_bytes(false), stream, a);
  else
    hipLaunchKernelGGL(pf_gemm<false>, dim3(n), dim3(kPfThreads), pf_lds_bytes(false), stream, a);
  return hipGetLastError();
}

}  // namespace fmx
