// fmx_dev.hpp -- device helpers shared by the router, sort and GEMM kernels
// (library-internal).
#pragma once

#include <type_traits>

#include "fmx_kernels.hpp"

extern "C" __device__ __attribute__((const)) double __ockl_wfred_max_f64(double);

namespace fmx {

// ------------------------------------------------------------------ lanes, scans

__device__ inline uint64_t lanes_below(int lane) {
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Exclusive scan of one value per thread over a workgroup of NT threads.
template <int NT>
__device__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* s_tmp, uint32_t* total) {
  constexpr int NW = NT / kWave;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t y = __shfl_up(x, d);
    if (lane >= d) x += y;
  }
  if (lane == kWave - 1) s_tmp[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t run = 0;
    for (int w = 0; w < NW; ++w) {
      const uint32_t t = s_tmp[w];
      s_tmp[w] = run;
      run += t;
    }
    s_tmp[NW] = run;
  }
  __syncthreads();
  const uint32_t r = s_tmp[wave] + x - v;
  if (total) *total = s_tmp[NW];
  __syncthreads();
  return r;
}

// Stable counting sort of n keys by value, by one workgroup of NT threads
// (every thread calls). Entries are cut into tiles of 64 (one per lane of a
// wave). Within a tile, the lanes holding an equal key are found with one
// ballot per key bit; a lane's rank among them is the popcount of the equal
// lanes below it. The per-(key, tile) counts, scanned in key-major order,
// give every (key, tile) its first output position, so
// position = base[key][tile] + rank. Keys >= E are treated as E - 1.
// `keys` may point to LDS or global memory.
// s_cnt: E * ceil(n/64) bytes of LDS; s_rank: n bytes; s_tmp: NT/64 + 1 words.
template <int NT>
__device__ void sort_block(const uint32_t* keys, int n, int k, int E, const SortOut& o,
                           uint8_t* s_cnt, uint8_t* s_rank, uint32_t* s_tmp) {
  constexpr int NW = NT / kWave;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n_tiles = (n + 63) / 64;
  const int total = E * n_tiles;
  const int nbits = E <= 1 ? 1 : 32 - __builtin_clz(static_cast<uint32_t>(E - 1));

  for (int i = tid; i < total; i += NT) s_cnt[i] = 0;
  __syncthreads();

  for (int tile = wave; tile < n_tiles; tile += NW) {
    const int i = tile * 64 + lane;
    const bool valid = i < n;
    uint32_t key = valid ? keys[i] : 0u;
    key = key < static_cast<uint32_t>(E) ? key : static_cast<uint32_t>(E - 1);
    uint64_t eq = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (key >> b) & 1u;
      const uint64_t m = __ballot(bit);
      eq &= bit ? m : ~m;
    }
    if (valid) {
      const int rank = __popcll(eq & lanes_below(lane));
      s_rank[i] = static_cast<uint8_t>(rank);
      if (rank == 0) s_cnt[key * n_tiles + tile] = static_cast<uint8_t>(__popcll(eq));
    }
  }
  __syncthreads();

  // key-major exclusive scan of the count table
  const int per = (total + NT - 1) / NT;
  const int beg = tid * per;
  const int end = min(beg + per, total);
  uint32_t local = 0;
  for (int j = beg; j < end; ++j) local += s_cnt[j];
  uint32_t run = block_exclusive_scan<NT>(local, s_tmp, nullptr);
  for (int j = beg; j < end; ++j) {
    o.base[j] = run;
    if (j % n_tiles == 0) o.offsets[j / n_tiles] = run;
    run += s_cnt[j];
  }
  if (tid == 0) o.offsets[E] = static_cast<uint32_t>(n);
  __syncthreads();

  for (int i = tid; i < n; i += NT) {
    uint32_t key = keys[i];
    key = key < static_cast<uint32_t>(E) ? key : static_cast<uint32_t>(E - 1);
    const uint32_t pos = o.base[key * n_tiles + i / 64] + s_rank[i];
    if (o.order) o.order[pos] = static_cast<uint32_t>(i);
    if (o.inv) o.inv[i] = pos;
    if (o.src) o.src[pos] = static_cast<uint32_t>(i / k);
    if (o.idx) o.idx[pos] = key;
  }

  // segment table of the non-empty keys, ascending, and the pass table
  // (each segment cut into passes of at most kPassRows rows)
  if (o.seg_off) {
    const int eper = (E + NT - 1) / NT;
    const int eb = tid * eper, ee = min(eb + eper, E);
    uint32_t cnt = 0, pcnt = 0;
    for (int e = eb; e < ee; ++e) {
      const uint32_t c = o.offsets[e + 1] - o.offsets[e];
      cnt += c ? 1u : 0u;
      pcnt += (c + kPassRows - 1) / kPassRows;
    }
    uint32_t U = 0, NP = 0;
    uint32_t u = block_exclusive_scan<NT>(cnt, s_tmp, &U);
    uint32_t p = block_exclusive_scan<NT>(pcnt, s_tmp, &NP);
    for (int e = eb; e < ee; ++e) {
      const uint32_t off = o.offsets[e], c = o.offsets[e + 1] - off;
      if (c) {
        if (o.seg_exp) o.seg_exp[u] = static_cast<uint32_t>(e);
        o.seg_off[u] = off;
        ++u;
        if (o.pass_tab) {
          for (uint32_t r = 0; r < c; r += kPassRows, ++p) {
            o.pass_tab[2 * p] = off + r;
            o.pass_tab[2 * p + 1] = static_cast<uint32_t>(e) | (min(c - r, static_cast<uint32_t>(kPassRows)) << 16);
          }
        }
      }
    }
    if (tid == 0) {
      o.seg_off[U] = static_cast<uint32_t>(n);
      if (o.seg_n) *o.seg_n = U;
      if (o.pass_n) *o.pass_n = NP;
    }
  }
}

// ------------------------------------------------------------------ exact dot products

// Row moves of the DPP (gfx9 encodings): row_shr:n (lane i of a 16-lane row
// takes lane i - n of its row), row_bcast:15 (lane 15 of each row to the
// next row), row_bcast:31 (lane 31 to rows 2 and 3); the row mask selects
// the rows written. Lanes without a source, and rows outside the mask, keep
// `old`.
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr4 = 0x114, kDppRowShr8 = 0x118;
constexpr int kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;

template <int CTRL, int ROWS = 0xf>
__device__ inline uint32_t dpp_mov(uint32_t old, uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(static_cast<int>(old), static_cast<int>(v), CTRL, ROWS, 0xf, false));
}
template <int CTRL, int ROWS = 0xf>
__device__ inline float dpp_mov(float old, float v) {
  return __uint_as_float(dpp_mov<CTRL, ROWS>(__float_as_uint(old), __float_as_uint(v)));
}
template <int CTRL, int ROWS = 0xf>
__device__ inline double dpp_mov(double old, double v) {
  const uint64_t o = static_cast<uint64_t>(__double_as_longlong(old));
  const uint64_t x = static_cast<uint64_t>(__double_as_longlong(v));
  const uint32_t lo = dpp_mov<CTRL, ROWS>(static_cast<uint32_t>(o), static_cast<uint32_t>(x));
  const uint32_t hi = dpp_mov<CTRL, ROWS>(static_cast<uint32_t>(o >> 32), static_cast<uint32_t>(x >> 32));
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}

// Pairwise tree over each block of B consecutive lanes (B a power of two,
// 1..64), adjacent lanes first: the block's result lands in its last lane
// (the other lanes hold partial values). op(v, ident) must be v. For a sum
// over 64 lanes this is the association of the butterfly s_l <- s_l +
// s_(l xor w), w = 1, 2, .., 32: every pair's operands are the same.
template <int B, typename T, typename Op>
__device__ inline T tree_to_last(T v, T ident, Op op) {
  static_assert(B >= 1 && B <= 64 && (B & (B - 1)) == 0, "B: a power of two <= 64");
  if constexpr (B >= 2) v = op(v, dpp_mov<kDppRowShr1>(ident, v));
  if constexpr (B >= 4) v = op(v, dpp_mov<kDppRowShr2>(ident, v));
  if constexpr (B >= 8) v = op(v, dpp_mov<kDppRowShr4>(ident, v));
  if constexpr (B >= 16) v = op(v, dpp_mov<kDppRowShr8>(ident, v));
  if constexpr (B >= 32) v = op(v, dpp_mov<kDppRowBcast15, 0xa>(ident, v));
  if constexpr (B >= 64) v = op(v, dpp_mov<kDppRowBcast31, 0xc>(ident, v));
  return v;
}

__device__ inline double readlane_f64(double v, int l) {
  const uint64_t x = static_cast<uint64_t>(__double_as_longlong(v));
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(x), l);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(x >> 32), l);
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}

// Wave-wide results of the tree, in every lane
__device__ inline float wave_max_f32(float v) {
  v = tree_to_last<64>(v, -__builtin_huge_valf(), [](float a, float b) { return fmaxf(a, b); });
  return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 63));
}
__device__ inline uint32_t wave_max_u32(uint32_t v) {
  v = tree_to_last<64>(v, 0u, [](uint32_t a, uint32_t b) { return max(a, b); });
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}
__device__ inline double wave_sum_f64(double v) {
  return readlane_f64(tree_to_last<64>(v, 0.0, [](double a, double b) { return a + b; }), 63);
}

// Reduce-scatter of N = 2^P doubles over the 64 lanes of a wave: butterfly
// steps w = 32, 16, .. pair the values up, then a DPP tree sums each block
// of 64 / N lanes; afterwards the last lane of block b (lane
// (b + 1) * 64 / N - 1) holds the wave-wide total of value b. The router's
// partial sums are exact, so the association order is free.
template <int N>
__device__ inline double reduce_scatter64(double (&v)[N], int lane) {
  constexpr int P = N == 1 ? 0 : N == 2 ? 1 : N == 4 ? 2 : N == 8 ? 3 : N == 16 ? 4 : N == 32 ? 5 : 6;
  static_assert((1 << P) == N && P <= 6, "N must be a power of two <= 64");
#pragma unroll
  for (int s = 0; s < P; ++s) {
    const int w = 32 >> s;
    const bool up = (lane & w) != 0;
    const int half = N >> (s + 1);
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      if (i < half) {
        // bitwise select of two loaded values: a lane-dependent array index
        // would move v[] to scratch memory
        const uint64_t lo = __double_as_longlong(v[i]);
        const uint64_t hi = __double_as_longlong(v[i + half]);
        const uint64_t m = up ? ~0ull : 0ull;
        const double send = __longlong_as_double((lo & m) | (hi & ~m));
        const double keep = __longlong_as_double((hi & m) | (lo & ~m));
        v[i] = keep + __shfl_xor(send, w);
      }
    }
  }
  return tree_to_last<(64 >> P)>(v[0], 0.0, [](double a, double b) { return a + b; });
}

// Whether lane holds a reduce_scatter64<N> total
template <int N>
__device__ inline bool rs64_holder(int lane) {
  return (lane & (64 / N - 1)) == 64 / N - 1;
}

// ------------------------------------------------------------------ router rows

// Eight consecutive weights (elements 8 ch .. 8 ch + 7) of a router row, held
// raw until used: a 16-byte bf16 chunk, or one 4-bit word with its group's
// scale and bias (RouterRows). get(j) is weight j as an exact double: for the
// quantized form s*q + b of bf16 s, b and q in 0..15 (MLX's dequantised
// value, model.cpp:758-760), whose product and sum are exact in fp64.
// F16: the row, or the scales and biases, in float16 (s*q + b of fp16 s, b
// is exact in fp64 too).
struct RChunk {
  u32x4_t v;  // the bf16 (fp16) chunk, or v[0] = the 4-bit word
  float s, b;
  bool q;
  template <bool F16 = false>
  __device__ inline double get(int j) const {
    if (q) return __builtin_fma(static_cast<double>(s), static_cast<double>((v[0] >> (4 * j)) & 15u),
                                static_cast<double>(b));
    const uint32_t w = v[j >> 1];
    return static_cast<double>((j & 1) ? Act<F16>::hi(w) : Act<F16>::lo(w));
  }
};

template <bool F16 = false>
__device__ inline RChunk load_rchunk(const RouterRows& r, int64_t row, int H, int ch) {
  RChunk c;
  c.q = r.s != nullptr;
  if (c.q) {
    c.v = u32x4_t{static_cast<const uint32_t*>(r.w)[row * (H / 8) + ch], 0u, 0u, 0u};
    const int64_t g = row * (H / 64) + ch / 8;
    c.s = Act<F16>::ld(r.s[g]);
    c.b = Act<F16>::ld(r.b[g]);
  } else {
    c.v = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(r.w) + row * H + ch * 8);
    c.s = c.b = 0.0f;
  }
  return c;
}

// ------------------------------------------------------------------ LDS staging

// One row of K bf16 (K a multiple of 8) -> LDS by LDS DMA: each
// global_load_lds_dwordx4 moves a wave's 64 x 16 bytes (a 1 KB piece of the
// row) straight into LDS, with no registers and no wait at the issuing point;
// in a last, partial piece the lanes past the row's end do not take part.
// Called by one whole wave (dst must be wave-uniform). CPOL is the loads'
// cache policy: kCpolDevice (sc1) reads data that other workgroups of the
// same grid wrote with device-scope stores.
constexpr int kCpolDevice = 16;
template <int CPOL = 0>
__device__ inline void dma_row(const uint16_t* src, int K, uint16_t* s_dst, int lane) {
  for (int pc = 0; pc * 512 < K; ++pc) {
    if (pc * 512 + 8 * lane < K)
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(src + pc * 512 + 8 * lane),
                                       (__attribute__((address_space(3))) void*)(s_dst + pc * 512),
                                       16, 0, CPOL);
  }
}

// Rows [T][K] of bf16 (row stride ld elements) -> LDS rows of stride xs
// elements: waves wave, wave + nw, ... take the rows in turn (wave must be
// wave-uniform). The caller waits (wait_vmcnt0) and barriers before any wave
// reads the rows.
__device__ inline void dma_rows(const uint16_t* src, int64_t ld, int T, int K, uint16_t* s_dst, int xs,
                                int wave, int nw, int lane) {
  for (int t = wave; t < T; t += nw) dma_row(src + t * ld, K, s_dst + t * xs, lane);
}

// s_waitcnt vmcnt(N), other counters untouched (gfx9 encoding: vmcnt[3:0] |
// expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14]). Vector memory loads
// complete in issue order, so vmcnt(N) right after N loads means that every
// older load, e.g. an LDS DMA issued before them, has landed.
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ inline void wait_vmcnt0() { wait_vmcnt<0>(); }
// s_waitcnt lgkmcnt(0) alone (vmcnt and expcnt at their maximum: no wait)
__device__ inline void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14)); }

// Workgroup barrier for LDS written by LDS DMA that every wave has already
// waited for (wait_vmcnt): s_barrier alone, with compiler-level memory
// barriers around it, so that no fence adds a wait for the loads still in
// flight (the fences of __syncthreads drain vmcnt to 0).
__device__ inline void lds_dma_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Workgroup barrier for data in LDS only: waits for this wave's LDS
// operations (lgkmcnt), not for its global stores in flight, which the
// fence of __syncthreads would drain as well.
__device__ inline void lds_barrier() {
  asm volatile("" ::: "memory");
  wait_lgkmcnt0();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ------------------------------------------------------------------ packed 4-bit tiles
//
// Packed layout (fmx_pack_expert_weights). A matrix [N, K] is cut into tiles
// of 16 rows and units of 128 k (two quantisation groups). Block (tile, unit)
// holds, for lane l = 16*j + c of a wave, the 16 bytes of row 16*tile + c
// that the lane feeds to four v_mfma_f32_16x16x32_bf16 as its B operand:
// words 4a + j (a = 0..3) of the unit, i.e. k = 32a + 8j .. 32a + 8j + 7.
// MFMAs a = 0, 1 then cover group 0 of the unit and a = 2, 3 group 1, so
// every group's partial sum is formed without masking. Within each word the
// nibbles are re-ordered (element 2i at position i, element 2i + 1 at
// position i + 4) so that nib8 below yields the elements in natural order and
// activation rows are used exactly as stored. After the 1024 weight
// bytes come 16 x 8 bytes of (scale g0 | scale g1 << 16, bias g0 | bias g1 <<
// 16) per row. A SwiGLU pair stores gate and up blocks side by side:
// [gate w | up w | gate sb | up sb], 2304 bytes. The blocks of a tile are
// consecutive (unit-major within the tile), tiles follow each other, and
// experts follow each other.
//
// Exact dequantisation: nibbles become the bf16 values 128 + q (exact); per
// group the products P = x.(128+q) and X = x.1 (an all-ones operand) are
// formed in fp32 by the MFMA, and acc += s * P + (b - 128 s) * X is the
// fp32 value of x.(s*q + b): weights are never rounded to bf16.

constexpr int kBlockSingle = 1152;
constexpr int kBlockPair = 2304;

__device__ inline f32x4_t mfma_bf16(const bf16x8_t& a, const bf16x8_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 8 nibbles -> bf16 pairs (128 + p_i, 128 + p_{i+4}), i = 0..3, where p_i is
// the nibble at position i (for a packed word: elements 2i and 2i + 1)
__device__ inline bf16x8_t nib8(uint32_t w) {
  u32x4_t d;
  d[0] = (w & 0x000f000fu) | 0x43004300u;
  d[1] = ((w >> 4) & 0x000f000fu) | 0x43004300u;
  d[2] = ((w >> 8) & 0x000f000fu) | 0x43004300u;
  d[3] = ((w >> 12) & 0x000f000fu) | 0x43004300u;
  return __builtin_bit_cast(bf16x8_t, d);
}

// ------------------------------------------------------------------ fp16 operands (prefill)
//
// The prefill GEMMs multiply in fp16: a weight s*q + b rounded once to fp16
// (11 significant bits) is within 2^-11 relative of its exact value, an
// eighth of bf16's rounding error. A bf16 activation converts to fp16
// exactly when its magnitude lies in [2^-14, 65536); below 2^-14 fp16 is
// subnormal (steps of 2^-24), so smaller values round to that grid (an
// absolute error of at most 2^-25; magnitudes under 2^-25 become 0).
// Activations at or above 65536 (and inf/NaN) raise a flag that sends the
// GEMM to the exact bf16 path instead.
//
// P8 layout (p8_slot): the 8 elements e0..e7 of a 16-byte activation chunk are
// stored as e0 e4 e1 e5 e2 e6 e3 e7, the order in which dq8_f16 delivers the
// 8 weights of a packed word, so that A and B operands pair up by position.

// A byte 0..15 is the FP8 (E4M3) encoding of q * 2^-9 (the subnormal and the
// first normal binade are evenly spaced); v_cvt_scalef32_pk_f16_fp8 with the
// power-of-two scale 2^9 turns two such bytes into the exact fp16 values q.
constexpr float kFp8Q = 512.0f;

// The 8 weights of a packed word (element 2i at nibble position i, 2i + 1 at
// i + 4) as fp16(s*q + b) in P8 layout: masking the even and the odd nibble
// positions into bytes gives lo = elements 0, 4, 1, 5 and hi = 2, 6, 3, 7;
// each pair is converted by one instruction and scaled by one packed fp16
// fma (a single rounding of s*q + b).
__device__ inline f16x8_t dq8_f16(uint32_t w, f16x2_t s, f16x2_t b) {
  const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
  const f16x2_t q04 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, kFp8Q, false);
  const f16x2_t q15 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, kFp8Q, true);
  const f16x2_t q26 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, kFp8Q, false);
  const f16x2_t q37 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, kFp8Q, true);
  const f16x2_t d0 = __builtin_elementwise_fma(q04, s, b);
  const f16x2_t d1 = __builtin_elementwise_fma(q15, s, b);
  const f16x2_t d2 = __builtin_elementwise_fma(q26, s, b);
  const f16x2_t d3 = __builtin_elementwise_fma(q37, s, b);
  return f16x8_t{d0[0], d0[1], d1[0], d1[1], d2[0], d2[1], d3[0], d3[1]};
}

// (s, s) as fp16 from a bf16 (exact for |s| in [2^-17, 65504])
__device__ inline f16x2_t f16_splat(float s) {
  const _Float16 h = static_cast<_Float16>(s);
  return f16x2_t{h, h};
}

__device__ inline f32x4_t mfma_f16(const f16x8_t& a, const f16x8_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// |v| >= 65536 (or inf/NaN) for a bf16 bit pattern: outside fp16's range
__device__ inline bool bf16_f16_overflow(uint32_t h) { return (h & 0x7fffu) >= 0x4780u; }

// fp16 bits of a bf16 value (round to nearest even: exact for magnitudes in
// [2^-14, 65536), on fp16's subnormal grid below)
__device__ inline uint32_t bf16_to_f16_bits(uint32_t h) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(__uint_as_float(h << 16)));
}

// A 16-byte chunk of 8 bf16 (natural order) as 8 fp16 in P8 layout; ovf is
// set when an element is outside fp16's range.
__device__ inline u32x4_t bf16_chunk_to_f16_p8(u32x4_t v, bool& ovf) {
  uint32_t e[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    e[2 * i] = v[i] & 0xffffu;
    e[2 * i + 1] = v[i] >> 16;
  }
  u32x4_t o;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    ovf = ovf || bf16_f16_overflow(e[m]) || bf16_f16_overflow(e[m + 4]);
    o[m] = bf16_to_f16_bits(e[m]) | (bf16_to_f16_bits(e[m + 4]) << 16);
  }
  return o;
}

// The same chunk as 8 fp16 in the Q8 layout (elements 0,2,4,6,1,3,5,7): the
// order in which dq8_f16 delivers an MLX-layout word's weights (element i
// at nibble position i).
__device__ inline u32x4_t bf16_chunk_to_f16_q8(u32x4_t v, bool& ovf) {
  uint32_t e[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    e[2 * i] = v[i] & 0xffffu;
    e[2 * i + 1] = v[i] >> 16;
  }
  constexpr int q8[8] = {0, 2, 4, 6, 1, 3, 5, 7};
  u32x4_t o;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t lo = e[q8[2 * m]], hi = e[q8[2 * m + 1]];
    ovf = ovf || bf16_f16_overflow(lo) || bf16_f16_overflow(hi);
    o[m] = bf16_to_f16_bits(lo) | (bf16_to_f16_bits(hi) << 16);
  }
  return o;
}

// ------------------------------------------------------------------ operands of either dtype
//
// Decode tiles multiply in the activation dtype: bf16 operands on
// v_mfma_f32_16x16x32_bf16, or fp16 ones (a float16 block) on
// v_mfma_f32_16x16x32_f16, with the same exact dequantisation. The nibble
// operands 128 + q are exact in fp16 too (0x5800 | q << 3), and so is a
// product x.(128 + q) of an fp16 x (11 + 8 significant bits) in fp32.

template <bool F16>
using act8_t = typename std::conditional<F16, f16x8_t, bf16x8_t>::type;

__device__ inline f32x4_t mfma16(const bf16x8_t& a, const bf16x8_t& b, const f32x4_t& c) { return mfma_bf16(a, b, c); }
__device__ inline f32x4_t mfma16(const f16x8_t& a, const f16x8_t& b, const f32x4_t& c) { return mfma_f16(a, b, c); }

// nib8 with fp16 pairs
__device__ inline f16x8_t nib8_f16(uint32_t w) {
  u32x4_t d;
  d[0] = ((w << 3) & 0x00780078u) | 0x58005800u;
  d[1] = ((w >> 1) & 0x00780078u) | 0x58005800u;
  d[2] = ((w >> 5) & 0x00780078u) | 0x58005800u;
  d[3] = ((w >> 9) & 0x00780078u) | 0x58005800u;
  return __builtin_bit_cast(f16x8_t, d);
}

template <bool F16>
__device__ inline act8_t<F16> nib8_dt(uint32_t w) {
  if constexpr (F16)
    return nib8_f16(w);
  else
    return nib8(w);
}

// eight ones (bf16 0x3f80, fp16 0x3c00)
template <bool F16>
__device__ inline act8_t<F16> ones8() {
  const uint32_t o = F16 ? 0x3c003c00u : 0x3f803f80u;
  return __builtin_bit_cast(act8_t<F16>, u32x4_t{o, o, o, o});
}

template <bool DUAL>
struct PkUnit {
  u32x4_t w0, w1;    // packed words (gate / up)
  u32x2_t sb0, sb1;  // (s g0 | s g1 << 16, b g0 | b g1 << 16)
};

// vector memory instructions one pk_load issues
template <bool DUAL>
constexpr int pk_load_insts() { return DUAL ? 4 : 2; }

// The loads are non-temporal: a decode forward reads each weight once, and
// without the hint the weight stream evicts from the L2 and the last-level
// cache what the next kernels need at once (their code, the routing
// tables, rows and flags), so every later kernel's first instructions and
// loads went out to HBM (measured: Qwen1.5-MoE decode batch 1 21.9 -> 20.4
// us per layer, the 24-layer stack's batch-1 step 1.25 -> 1.18 ms).
template <bool DUAL>
__device__ inline PkUnit<DUAL> pk_load(const uint8_t* blk, int lane) {
  PkUnit<DUAL> L;
  const int col = lane & 15;
  L.w0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(blk + 16 * lane));
  if (DUAL) {
    L.w1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(blk + 1024 + 16 * lane));
    L.sb0 = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(blk + 2048 + 8 * col));
    L.sb1 = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(blk + 2048 + 128 + 8 * col));
  } else {
    L.sb0 = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(blk + 1024 + 8 * col));
  }
  return L;
}

// acc[i] += s0 P0 + (b0 - 128 s0) X0 + s1 P1 + (b1 - 128 s1) X1 (scales and
// biases in the activation dtype)
template <bool F16 = false>
__device__ inline void pk_epi(f32x4_t& acc, const u32x2_t& sb, const f32x4_t& P0, const f32x4_t& P1,
                              const f32x4_t& X0, const f32x4_t& X1) {
  const float s0 = Act<F16>::lo(sb[0]), s1 = Act<F16>::hi(sb[0]);
  const float c0 = __builtin_fmaf(-128.0f, s0, Act<F16>::lo(sb[1]));
  const float c1 = __builtin_fmaf(-128.0f, s1, Act<F16>::hi(sb[1]));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc[i] = __builtin_fmaf(s0, P0[i], acc[i]);
    acc[i] = __builtin_fmaf(c0, X0[i], acc[i]);
    acc[i] = __builtin_fmaf(s1, P1[i], acc[i]);
    acc[i] = __builtin_fmaf(c1, X1[i], acc[i]);
  }
}

// One unit: A[a] (a = 0..3) are the lane's activation operands for k =
// 32a + 8j .. +7 (P8 order); accumulates into acc0 (and acc1 for a pair).
template <bool DUAL, bool F16 = false>
__device__ inline void pk_unit(const PkUnit<DUAL>& L, const act8_t<F16> (&A)[4], f32x4_t& acc0,
                               f32x4_t& acc1) {
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
  const act8_t<F16> ones = ones8<F16>();
  const f32x4_t X0 = mfma16(A[1], ones, mfma16(A[0], ones, zero));
  const f32x4_t X1 = mfma16(A[3], ones, mfma16(A[2], ones, zero));
  {
    const f32x4_t P0 = mfma16(A[1], nib8_dt<F16>(L.w0[1]), mfma16(A[0], nib8_dt<F16>(L.w0[0]), zero));
    const f32x4_t P1 = mfma16(A[3], nib8_dt<F16>(L.w0[3]), mfma16(A[2], nib8_dt<F16>(L.w0[2]), zero));
    pk_epi<F16>(acc0, L.sb0, P0, P1, X0, X1);
  }
  if (DUAL) {
    const f32x4_t P0 = mfma16(A[1], nib8_dt<F16>(L.w1[1]), mfma16(A[0], nib8_dt<F16>(L.w1[0]), zero));
    const f32x4_t P1 = mfma16(A[3], nib8_dt<F16>(L.w1[3]), mfma16(A[2], nib8_dt<F16>(L.w1[2]), zero));
    pk_epi<F16>(acc1, L.sb1, P0, P1, X0, X1);
  }
}

// The four A operands of one unit from an LDS row (P8 layout): xu points at
// the unit's first element of the lane's row, plus 8*j.
template <bool F16 = false>
__device__ inline void lds_a(const uint16_t* xu, act8_t<F16> (&A)[4]) {
#pragma unroll
  for (int a = 0; a < 4; ++a) A[a] = *reinterpret_cast<const act8_t<F16>*>(xu + 32 * a);
}

// ------------------------------------------------------------------ decode tiles
//
// Workgroups of kDecThreads threads (4 waves) that multiply one 16-row tile
// over K split in four quarters, all of a quarter's loads in flight at once.

// LDS row stride (elements) of staged activation rows of length K
__host__ __device__ inline int xstride(int K) { return K + 8; }

constexpr int kDecWaves = kDecThreads / kWave;
constexpr int kDecQuadRedBytes = (kDecWaves - 1) * 8 * kWave * 4;  // quad_reduce's LDS

// Units [u0, u1) (u1 - u0 <= NU) of one 16-row tile (blocks of BB bytes from
// tile_base), all loads in flight together, against activation rows in LDS
// (xl: the lane's row plus 8*j). The rows' LDS DMA is the caller's last
// memory operation before this call: right after the weight loads, vmcnt
// (their count) proves the DMA complete while they stay in flight, and
// the units are multiplied as their loads land.
template <bool DUAL, int NU, bool F16 = false>
__device__ inline void tile_units_lds(const uint8_t* tile_base, int u0, int u1, const uint16_t* xl,
                                      int lane, f32x4_t& acc0, f32x4_t& acc1) {
  constexpr int BB = DUAL ? kBlockPair : kBlockSingle;
  PkUnit<DUAL> L[NU];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int d = 0; d < NU; ++d) L[d] = pk_load<DUAL>(tile_base + min(u0 + d, u1 - 1) * BB, lane);
  __builtin_amdgcn_sched_barrier(0);
  wait_vmcnt<NU * pk_load_insts<DUAL>()>();
  lds_dma_barrier();
#pragma unroll
  for (int d = 0; d < NU; ++d) {
    if (u0 + d < u1) {
      act8_t<F16> A[4];
      lds_a<F16>(xl + (u0 + d) * 128, A);
      pk_unit<DUAL, F16>(L[d], A, acc0, acc1);
    }
  }
}

// Waves 1..3 hand their partial sums over K quarters 1..3 to wave 0 through
// LDS (s_red: 3 x 8 x 64 floats); wave 0 adds them in wave order.
__device__ inline void quad_reduce(f32x4_t& acc0, f32x4_t& acc1, int wave, int lane, float* s_red) {
  if (wave > 0) {
    float* slot = s_red + (wave - 1) * 8 * kWave;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      slot[i * kWave + lane] = acc0[i];
      slot[(4 + i) * kWave + lane] = acc1[i];
    }
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int w = 0; w < kDecWaves - 1; ++w) {
      const float* slot = s_red + w * 8 * kWave;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc0[i] += slot[i * kWave + lane];
        acc1[i] += slot[(4 + i) * kWave + lane];
      }
    }
  }
}

// ------------------------------------------------------------------ Nemotron-H selection
// (nemotron_h.cpp:1017-1050)

// fp32 ordering key: larger floats give larger keys (zeros of either sign
// give the key of +0)
__device__ inline uint32_t f32_key(float f) {
  const uint32_t u = f == 0.0f ? 0u : __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ inline uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int w = 32; w >= 1; w >>= 1) {
    const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), w);
    const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), w);
    const uint64_t o = (static_cast<uint64_t>(hi) << 32) | lo;
    v = o > v ? o : v;
  }
  return v;
}

// One token by one wave: orig = fp32(sigmoid(logit)) (fp64 with exp_det,
// rounded once); sel = orig + correction bias (fp32); with groups, each
// group's score is the sum of its two largest sel, the topk_group best
// groups stay (ties: lower group) and the others' sel become 0; the k
// largest sel are selected (ties: lower expert; slot order sel desc, index
// asc); scores = orig of the selected, / (slot-order sum + 1e-20) when
// renormalising, * scaling, every operation in fp32. lrow: the token's E
// bf16 logits (global or LDS); lane j < k writes slot j to inds_out,
// scores_out and (non-null) inds_lds. E <= 64 * NPER, n_group <= 64.
template <int NPER>
__device__ void nh_select_wave(const uint16_t* lrow, int E, int k, int norm, int n_group, int topk_group,
                               float scaling, const float* cbias, int lane, uint32_t* inds_out,
                               float* scores_out, uint32_t* inds_lds) {
  constexpr int kMaxExpertsPerLane = NPER;
  const int nblk = (E + kWave - 1) / kWave;  // wave-uniform
  float orig[kMaxExpertsPerLane], sel[kMaxExpertsPerLane];
#pragma unroll
  for (int i = 0; i < kMaxExpertsPerLane; ++i) {
    const int e = lane + 64 * i;
    orig[i] = 0.0f;
    sel[i] = -__builtin_huge_valf();
    if (i < nblk && e < E) {
      const double l = static_cast<double>(bf16_to_f32(lrow[e]));
      orig[i] = static_cast<float>(1.0 / (1.0 + exp_det(-l)));
      sel[i] = cbias ? orig[i] + cbias[e] : orig[i];
    }
  }
  if (n_group > 1) {
    const int G = E / n_group;
    // lane g ends with group g's score (n_group <= 64)
    float my_gs = -__builtin_huge_valf();
    for (int g = 0; g < n_group; ++g) {
      float m1 = -__builtin_huge_valf(), m2 = -__builtin_huge_valf();
#pragma unroll
      for (int i = 0; i < kMaxExpertsPerLane; ++i) {
        const int e = lane + 64 * i;
        if (i < nblk && e < E && e / G == g) {
          if (sel[i] > m1) {
            m2 = m1;
            m1 = sel[i];
          } else if (sel[i] > m2) {
            m2 = sel[i];
          }
        }
      }
      // merge the lanes' two largest
#pragma unroll
      for (int w = 32; w >= 1; w >>= 1) {
        const float o1 = __shfl_xor(m1, w), o2 = __shfl_xor(m2, w);
        const float hi = fmaxf(m1, o1), lo = fmaxf(fminf(m1, o1), fmaxf(m2, o2));
        m1 = hi;
        m2 = lo;
      }
      if (lane == g) my_gs = m1 + m2;
    }
    // the topk_group groups that argpartition's (value asc, index asc) order
    // leaves last stay: group score desc, then index desc (equal scores: the
    // lower group is zeroed first)
    bool keep = false;
    uint64_t gkey = lane < n_group ? (static_cast<uint64_t>(f32_key(my_gs)) << 32) | static_cast<uint32_t>(lane + 1)
                                   : 0ull;
    for (int r = 0; r < topk_group; ++r) {
      const uint64_t best = wave_max_u64(gkey);
      if (gkey == best && lane < n_group) {
        keep = true;
        gkey = 0ull;
      }
    }
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; ++i) {
      const int e = lane + 64 * i;
      const int g = min(e, E - 1) / G;
      const bool kept = __shfl(static_cast<int>(keep), g) != 0;
      if (i < nblk && e < E && !kept) sel[i] = 0.0f;
    }
  }
  uint64_t key[kMaxExpertsPerLane];
#pragma unroll
  for (int i = 0; i < kMaxExpertsPerLane; ++i) {
    const int e = lane + 64 * i;
    key[i] = (i < nblk && e < E)
                 ? (static_cast<uint64_t>(f32_key(sel[i])) << 32) | (0xffffffffu - static_cast<uint32_t>(e))
                 : 0ull;
  }
  float my_sc = 0.0f, den = 0.0f;
  for (int j = 0; j < k; ++j) {
    uint64_t best = 0ull;
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; ++i)
      if (i < nblk) best = key[i] > best ? key[i] : best;
    best = wave_max_u64(best);
    const uint32_t e = 0xffffffffu - static_cast<uint32_t>(best);
    float o = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; ++i) {
      if (i < nblk && key[i] == best) key[i] = 0ull;
      if (i == static_cast<int>(e >> 6)) o = orig[i];
    }
    o = __shfl(o, static_cast<int>(e & 63u));  // the winner's lane holds its orig
    den = __fadd_rn(den, o);
    if (lane == j) {
      my_sc = o;
      inds_out[j] = e;
      if (inds_lds) inds_lds[j] = e;
    }
  }
  if (lane < k) {
    float sc = my_sc;
    if (norm && k > 1) sc = sc / __fadd_rn(den, 1e-20f);
    scores_out[lane] = __fmul_rn(sc, scaling);
  }
}

constexpr int kNormThreads = 256;
constexpr int kNormMaxChunks = 4;  // 16-byte chunks per thread: H <= 8192

// ------------------------------------------------------------------ RMSNorm
//
// RMSNorm arithmetic (mx::fast::rms_norm, model.cpp:486-488), shared by
// rmsnorm_kernel, the decode projections' fused norms and K1's so that all
// give the same bits (kNormThreads threads over a row): x = bf16(x + delta) element by element; the sum of squares
// in fp64, each thread over its chunks c = tid + kNormThreads q in order,
// then the wave's butterfly and the waves in order; r = 1 / sqrt(ss / H +
// eps) in fp64; out = bf16(bf16(x * r) * w).
__device__ inline u32x4_t norm_add(u32x4_t x, const u32x4_t& d) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t lo = f32_to_bf16(bf16_to_f32(x[m] & 0xffffu) + bf16_to_f32(d[m] & 0xffffu));
    const uint32_t hi = f32_to_bf16(bf16_to_f32(x[m] >> 16) + bf16_to_f32(d[m] >> 16));
    x[m] = lo | (hi << 16);
  }
  return x;
}
__device__ inline double norm_sq(const u32x4_t& x, double ss) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const double lo = bf16_to_f32(x[m] & 0xffffu), hi = bf16_to_f32(x[m] >> 16);
    ss += lo * lo;
    ss += hi * hi;
  }
  return ss;
}
__device__ inline double norm_wave_sum(double ss) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
  return ss;
}
__device__ inline double norm_r(const double* s_red_row, int H, float eps) {
  double tot = 0.0;
#pragma unroll
  for (int w = 0; w < kNormThreads / kWave; ++w) tot += s_red_row[w];
  return 1.0 / sqrt(tot / static_cast<double>(H) + static_cast<double>(eps));
}
__device__ inline u32x4_t norm_apply(const u32x4_t& x, const u32x4_t& wv, double r) {
  u32x4_t o;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    uint32_t e2[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const double xv = bf16_to_f32((x[m] >> (16 * hf)) & 0xffffu);
      const uint16_t n = f64_to_bf16(xv * r);
      e2[hf] = f64_to_bf16(static_cast<double>(bf16_to_f32(n)) *
                           static_cast<double>(bf16_to_f32((wv[m] >> (16 * hf)) & 0xffffu)));
    }
    o[m] = e2[0] | (e2[1] << 16);
  }
  return o;
}

// The norm of T <= MAXT rows (row stride ld) of H elements into LDS rows of
// stride xs elements, by kNormThreads threads, chunk c of a row to thread c
// mod kNormThreads as in rmsnorm_kernel (the same bits); s_red: MAXT x
// (kNormThreads / kWave) doubles. The raw rows go to LDS with the sums of
// squares and are normalised there in place (no row held in registers).
// Every thread calls; ends with a barrier.
template <int MAXT>
__device__ inline void norm_rows_lds(const uint16_t* x, int64_t ld, const uint16_t* w, float eps, int T, int H,
                                     uint16_t* s_dst, int xs, double* s_red) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nch = H / 8;
  u32x4_t wv[kNormMaxChunks];
  double ss[MAXT];
#pragma unroll
  for (int q = 0; q < kNormMaxChunks; ++q) {
    const int c = tid + q * kNormThreads;
    if (c < nch) wv[q] = reinterpret_cast<const u32x4_t*>(w)[c];
  }
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    ss[t] = 0.0;
    if (t >= T) continue;
#pragma unroll
    for (int q = 0; q < kNormMaxChunks; ++q) {
      const int c = tid + q * kNormThreads;
      if (c >= nch) break;
      const u32x4_t v = reinterpret_cast<const u32x4_t*>(x + static_cast<int64_t>(t) * ld)[c];
      *reinterpret_cast<u32x4_t*>(s_dst + t * xs + 8 * c) = v;
      ss[t] = norm_sq(v, ss[t]);
    }
  }
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    if (t >= T) continue;
    const double sw = norm_wave_sum(ss[t]);
    if (lane == 0) s_red[t * (kNormThreads / kWave) + wave] = sw;
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    if (t >= T) continue;
    const double r = norm_r(s_red + t * (kNormThreads / kWave), H, eps);
#pragma unroll
    for (int q = 0; q < kNormMaxChunks; ++q) {
      const int c = tid + q * kNormThreads;
      if (c >= nch) break;
      u32x4_t* p = reinterpret_cast<u32x4_t*>(s_dst + t * xs + 8 * c);
      *p = norm_apply(*p, wv[q], r);
    }
  }
  __syncthreads();
}

}  // namespace fmx
