// fmx_decode.hip -- the MoE block for decode batches (T <= 16 tokens) on
// packed expert weights, in three kernels:
//
//   K1  router: logits in column workgroups; the last of them to finish
//       derives softmax, top-k, the sort and the routed-expert tables
//       |  shared expert gate/up + SwiGLU (routing-independent, streams
//       meanwhile)
//   K2  routed experts' gate/up + SwiGLU tiles
//   K3  per 16 columns of H: the down projections of every routed expert and
//       of the shared expert, then the top-k weighted combine and the gated
//       shared add, written straight to y
//
// Reference: server/src/model.cpp:750-807 (moe_block), :673-734 (switch_mlp:
// gather_qmm gate/up/down, SwiGLU), :736-748 (shared_expert_mlp), :14-25
// (compiled SwiGLU), :757-775 (router), :682-700 (sort).
//
// Rows of every MFMA tile are indexed by token: a token selects an expert at
// most once, so expert e's tile rows are the tokens that routed to it and no
// gather or sort is needed for the products. The only cross-workgroup
// handoff inside a kernel is K1's router (release/acquire fences in a few
// dozen workgroups); everything else meets at kernel boundaries.
#include <algorithm>

#include "fmx_dev.hpp"

namespace fmx {

namespace {

// LDS row stride (elements) of staged activation rows of length K
__host__ __device__ inline int xstride(int K) { return K + 8; }

constexpr int kDecWaves = kDecThreads / kWave;
constexpr int kRouterColsPerWg = 2;  // two columns per router workgroup, H halves per wave

// Units [u0, u1) (u1 - u0 <= NU) of one 16-row tile (blocks of BB bytes from
// tile_base), all loads in flight together, against activation rows in LDS
// (xl: the lane's row plus 8*j). The rows' LDS DMA is the caller's last
// memory operation before this call: right after the weight loads, vmcnt
// (their count) proves the DMA complete while they stay in flight, and
// the units are multiplied as their loads land.
template <bool DUAL, int NU>
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
      bf16x8_t A[4];
      lds_a(xl + (u0 + d) * 128, A);
      pk_unit<DUAL>(L[d], A, acc0, acc1);
    }
  }
}

// Waves 2p and 2p+1 of a workgroup compute tile pair slot p over K halves 0
// and 1; the second half's partial sums reach the first through LDS (s_red:
// 2 x 8 x 64 floats).
__device__ inline void pair_reduce(f32x4_t& acc0, f32x4_t& acc1, int wave, int lane, float* s_red) {
  float* slot = s_red + (wave >> 1) * 8 * kWave;
  if (wave & 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      slot[i * kWave + lane] = acc0[i];
      slot[(4 + i) * kWave + lane] = acc1[i];
    }
  }
  __syncthreads();
  if (!(wave & 1)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc0[i] += slot[i * kWave + lane];
      acc1[i] += slot[(4 + i) * kWave + lane];
    }
  }
}

// ---------------------------------------------------------------- K1: router

// Softmax (fp64, exp_det, fixed-order normaliser) and top-k of token t by
// one wave, as model.cpp:764-775 with the renormalisation of
// moe-support-plan.md:319-322: the k largest bf16 probabilities, ties to the
// lower expert index, slots ordered (probability desc, index asc).
// lrow: the token's E (+1) logits in LDS.
template <int NPER>
__device__ void route_token(const DecodeArgs& a, int t, const uint16_t* lrow, int lane, uint32_t* s_inds) {
  const int E = a.E;
  double lv[NPER];
  double m = -__builtin_huge_val();
#pragma unroll
  for (int i = 0; i < NPER; ++i) {
    const int e = lane + 64 * i;
    lv[i] = e < E ? static_cast<double>(bf16_to_f32(lrow[e])) : -__builtin_huge_val();
    m = fmax(m, lv[i]);
  }
  m = __ockl_wfred_max_f64(m);
  // lane l sums e = l, l + 64, ... in turn; six butterfly steps then give
  // every lane the same total
  double ex[NPER];
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < NPER; ++i) {
    const int e = lane + 64 * i;
    ex[i] = e < E ? exp_det(lv[i] - m) : 0.0;
    s += ex[i];
  }
#pragma unroll
  for (int w = 32; w >= 1; w >>= 1) s += __shfl_xor(s, w);
  uint32_t key[NPER];
#pragma unroll
  for (int i = 0; i < NPER; ++i) {
    const int e = lane + 64 * i;
    key[i] = 0u;
    if (e < E) {
      const uint16_t p = f64_to_bf16(ex[i] / s);
      if (a.probs) a.probs[static_cast<int64_t>(t) * E + e] = p;
      // probabilities are >= 0: their bf16 patterns order like their values
      key[i] = (static_cast<uint32_t>(p) << 16) | (0xffffu - static_cast<uint32_t>(e));
    }
  }
  float sc_sum = 0.0f;
  uint32_t my_key = 0u;
  for (int j = 0; j < a.k; ++j) {
    uint32_t best = 0u;
#pragma unroll
    for (int i = 0; i < NPER; ++i) best = max(best, key[i]);
    best = __ockl_wfred_max_u32(best);
#pragma unroll
    for (int i = 0; i < NPER; ++i)
      if (key[i] == best) key[i] = 0u;
    sc_sum += bf16_to_f32(static_cast<uint16_t>(best >> 16));  // fp32, slot order
    if (lane == j) my_key = best;
  }
  if (lane < a.k) {
    const uint32_t e = 0xffffu - (my_key & 0xffffu);
    uint16_t sc = static_cast<uint16_t>(my_key >> 16);
    if (a.norm) {
      const double den = static_cast<double>(round_bf16(sc_sum));
      sc = f32_to_bf16(static_cast<float>(static_cast<double>(bf16_to_f32(sc)) / den));
    }
    s_inds[t * a.k + lane] = e;
    a.inds[t * a.k + lane] = e;
    a.scores[t * a.k + lane] = sc;
  }
  if (lane == 0 && a.wsg) a.sgate[t] = sigmoid_bf16(bf16_to_f32(lrow[E]));
}

// The last router workgroup: routing of every token, the ascending list of
// routed experts (seg) and each expert's token -> slot row (slots).
template <int NPER>
__device__ void route_finish(const DecodeArgs& a, uint16_t* s_lg) {
  __shared__ uint32_t s_inds[kDecMaxT * kDecMaxK];
  __shared__ uint32_t s_seg[kDecMaxE + 1];
  __shared__ uint16_t s_segof[kDecMaxE];
  __shared__ uint8_t s_used[kDecMaxE];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int T = a.T, E = a.E, k = a.k, n = T * k;
  const int ld = E + 1;
  // every token's logits -> LDS in one round trip
  for (int i = tid; i < T * ld; i += kDecThreads) s_lg[i] = a.logits[i];
  for (int e = tid; e < E; e += kDecThreads) s_used[e] = 0;
  __syncthreads();
  for (int t = wave; t < T; t += kDecWaves) route_token<NPER>(a, t, s_lg + t * ld, lane, s_inds);
  __syncthreads();
  for (int i = tid; i < n; i += kDecThreads) s_used[s_inds[i]] = 1;
  __syncthreads();
  if (wave == 0) {
    uint32_t U = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      const bool used = e < E && s_used[e];
      const uint64_t b = __ballot(used);
      if (used) {
        const uint32_t u = U + static_cast<uint32_t>(__popcll(b & lanes_below(lane)));
        s_seg[1 + u] = static_cast<uint32_t>(e);
        s_segof[e] = static_cast<uint16_t>(u);
      }
      U += static_cast<uint32_t>(__popcll(b));
    }
    if (lane == 0) s_seg[0] = U;
  }
  __syncthreads();
  const int U = static_cast<int>(s_seg[0]);
  for (int i = tid; i <= U; i += kDecThreads) a.seg[i] = s_seg[i];
  // slot table, one byte per (expert u, token t): written as whole words
  for (int i = tid; i < U * (kDecMaxT / 4); i += kDecThreads) {
    const int u = i / (kDecMaxT / 4), t0 = 4 * (i - u * (kDecMaxT / 4));
    uint32_t word = 0xffffffffu;
    for (int q = 0; q < 4; ++q) {
      const int t = t0 + q;
      if (t >= T) continue;
      for (int j = 0; j < k; ++j)
        if (s_segof[s_inds[t * k + j]] == u) word = (word & ~(0xffu << (8 * q))) | (static_cast<uint32_t>(j) << (8 * q));
    }
    reinterpret_cast<uint32_t*>(a.slots)[i] = word;
  }
}

// Router columns 2*wg, 2*wg + 1 (column E: the shared-expert gate row) for
// every token: logits = x . w_c in fp64 (bf16 products are exact in fp32,
// their sum is exact in fp64 and so independent of order), rounded once to
// bf16 (model.cpp:762, :792-799). Waves 2c, 2c+1 take the two halves of H;
// every lane's partial sum of every token goes to LDS and 16 threads per
// (column, token) add them up.
template <int NPER>
__device__ void dec_router(const DecodeArgs& a, int wg, uint16_t* s_x, double* s_lp) {
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = a.H, T = a.T, E = a.E, xs = xstride(H);
  const int ncols = E + (a.wsg ? 1 : 0);
  const int c = min(wg * kRouterColsPerWg + (wave >> 1), ncols - 1);
  const int hh = wave & 1, half_oct = H / 16;
  const uint16_t* wrow = c < E ? a.wr + static_cast<int64_t>(c) * H : a.wsg;
  dma_rows(a.x, H, T, H, s_x, xs, wave, kDecWaves, lane);
  u32x4_t wv[kDecRouterChunks];
#pragma unroll
  for (int i = 0; i < kDecRouterChunks; ++i) {
    const int ch = hh * half_oct + min(lane + 64 * i, half_oct - 1);
    wv[i] = *reinterpret_cast<const u32x4_t*>(wrow + ch * 8);
  }
  wait_vmcnt0();
  __syncthreads();
  double wd[kDecRouterChunks * 8];
#pragma unroll
  for (int i = 0; i < kDecRouterChunks; ++i) {
    const bool ok = lane + 64 * i < half_oct;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      wd[8 * i + 2 * q] = ok ? static_cast<double>(__uint_as_float(wv[i][q] << 16)) : 0.0;
      wd[8 * i + 2 * q + 1] = ok ? static_cast<double>(__uint_as_float(wv[i][q] & 0xffff0000u)) : 0.0;
    }
  }
#pragma unroll 1
  for (int t = 0; t < T; ++t) {
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < kDecRouterChunks; ++i) {
      const int ch = hh * half_oct + min(lane + 64 * i, half_oct - 1);
      const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(s_x + t * xs + ch * 8);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc = __builtin_fma(static_cast<double>(__uint_as_float(xv[q] << 16)), wd[8 * i + 2 * q], acc);
        acc = __builtin_fma(static_cast<double>(__uint_as_float(xv[q] & 0xffff0000u)), wd[8 * i + 2 * q + 1], acc);
      }
    }
    s_lp[(t * kDecWaves + wave) * kWave + lane] = acc;
  }
  __syncthreads();
  // (column cc, token t) <- 16 threads, each adding 8 of its 128 partials
  for (int g = tid >> 4; g < kRouterColsPerWg * T; g += kDecThreads / 16) {
    const int cc = g / T, t = g - cc * T, r = tid & 15;
    const double* p = s_lp + (t * kDecWaves + 2 * cc) * kWave;
    double v = 0.0;
#pragma unroll
    for (int q = 0; q < 8; ++q) v += p[r * 8 + q];
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1) v += __shfl_xor(v, w);
    const int col = wg * kRouterColsPerWg + cc;
    if (r == 0 && col < ncols) {
      uint16_t l = f64_to_bf16(v);
      if (col < E && a.lbias)
        l = f64_to_bf16(static_cast<double>(bf16_to_f32(l)) + static_cast<double>(bf16_to_f32(a.lbias[col])));
      a.logits[static_cast<int64_t>(t) * (E + 1) + col] = l;
    }
  }
  // the last router workgroup to arrive sees every logit (release by each,
  // acquire by the last) and finishes the routing
  __syncthreads();
  if (tid == 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    s_last = atomicAdd(a.counter, 1u) == static_cast<uint32_t>(a.n_rt - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  route_finish<NPER>(a, s_x);
  if (tid == 0) *a.counter = 0u;  // every router workgroup has arrived
}

// Shared expert gate/up + SwiGLU for tile pair `pair` (model.cpp:741-747):
// hs[t, n] = swiglu(x_t . Wg[n], x_t . Wu[n]) for every token.
__device__ void dec_shared_gu(const DecodeArgs& a, int pair, uint16_t* s_x, float* s_red) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = a.H, T = a.T, Is = a.Is, xs = xstride(H);
  const int nu = H / 128, half = (nu + 1) / 2;
  const int tile = 2 * pair + (wave >> 1);
  const int u0 = (wave & 1) ? half : 0, u1 = (wave & 1) ? nu : half;
  const int m = lane & 15, j = lane >> 4;
  const uint16_t* xl = s_x + min(m, T - 1) * xs + 8 * j;
  f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
  dma_rows(a.x, H, T, H, s_x, xs, wave, kDecWaves, lane);
  tile_units_lds<true, 8>(a.sgu + static_cast<int64_t>(tile) * nu * kBlockPair, u0, u1, xl, lane, acc0, acc1);
  pair_reduce(acc0, acc1, wave, lane, s_red);
  if (wave & 1) return;
  const int n = tile * 16 + m;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 4 * j + i;
    if (t < T)
      a.hs[static_cast<int64_t>(t) * Is + n] = swiglu_bf16(round_bf16(acc0[i]), round_bf16(acc1[i]));
  }
}

// LDS: [router lane partials (16 x 4 x 64 doubles) or the pair reduction]
// then the staged activation rows.
template <int NPER>
__global__ __launch_bounds__(kDecThreads) void dec_k1(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int wg = blockIdx.x;
  if (wg < a.n_rt) {
    double* s_lp = reinterpret_cast<double*>(smem);
    uint16_t* s_x = reinterpret_cast<uint16_t*>(smem + kDecRouterLpBytes);
    dec_router<NPER>(a, wg, s_x, s_lp);
  } else {
    float* s_red = reinterpret_cast<float*>(smem);
    uint16_t* s_x = reinterpret_cast<uint16_t*>(smem + kDecRouterLpBytes);
    dec_shared_gu(a, wg - a.n_rt, s_x, s_red);
  }
}

// ---------------------------------------------------------------- K2: routed gate/up

// Tile pair `pair` of routed expert number u (model.cpp:703-712, :715):
// h[t*k + slot, n] = swiglu(x_t . Wg_e[n], x_t . Wu_e[n]) for the tokens t
// whose slot `slot` selected expert e.
__device__ void dec_sort(const DecodeArgs& a) {
  // switch_mlp's sort of the flattened indices (model.cpp:682-700), for the
  // routing accessors; the decode products do not need it
  __shared__ uint32_t s_inds[kDecMaxT * kDecMaxK];
  __shared__ uint8_t s_cnt[kDecMaxE * (kDecMaxT * kDecMaxK / 64)];
  __shared__ uint8_t s_rank[kDecMaxT * kDecMaxK];
  __shared__ uint32_t s_tmp[kDecWaves + 1];
  const int n = a.T * a.k;
  for (int i = threadIdx.x; i < n; i += kDecThreads) s_inds[i] = min(a.inds[i], static_cast<uint32_t>(a.E - 1));
  __syncthreads();
  sort_block<kDecThreads>(s_inds, n, a.k, a.E, a.sort, s_cnt, s_rank, s_tmp);
}

__global__ __launch_bounds__(kDecThreads) void dec_k2(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  float* s_red = reinterpret_cast<float*>(smem);
  uint16_t* s_x = reinterpret_cast<uint16_t*>(smem + kDecRouterLpBytes);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int T = a.T, k = a.k, H = a.H, I = a.I, xs = xstride(H);
  if (blockIdx.x == a.max_seg * a.gu_pairs) {
    dec_sort(a);
    return;
  }
  const int u = blockIdx.x / a.gu_pairs, pair = blockIdx.x - u * a.gu_pairs;
  // routing tables first: a workgroup without an expert leaves before it
  // starts any LDS DMA
  const int U = static_cast<int>(min(a.seg[0], static_cast<uint32_t>(a.max_seg)));
  if (u >= U) return;  // workgroup-uniform
  const int e = static_cast<int>(min(a.seg[1 + u], static_cast<uint32_t>(a.E - 1)));
  const uint32_t* srow = reinterpret_cast<const uint32_t*>(a.slots + u * kDecMaxT);
  const uint32_t slot4 = srow[lane & 3];  // slots of tokens 4*(lane&3) .. +3
  // activation rows -> LDS (DMA), in flight with the weight loads
  dma_rows(a.x, H, T, H, s_x, xs, wave, kDecWaves, lane);
  const int nu = H / 128, half = (nu + 1) / 2;
  const int tile = 2 * pair + (wave >> 1);
  const int u0 = (wave & 1) ? half : 0, u1 = (wave & 1) ? nu : half;
  const int m = lane & 15, j = lane >> 4;
  const uint16_t* xl = s_x + min(m, T - 1) * xs + 8 * j;
  f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
  tile_units_lds<true, 8>(a.gu + static_cast<int64_t>(e) * a.gu_es + static_cast<int64_t>(tile) * nu * kBlockPair,
                          u0, u1, xl, lane, acc0, acc1);
  pair_reduce(acc0, acc1, wave, lane, s_red);
  if (wave & 1) return;
  const int n = tile * 16 + m;
  // lane 16j + c holds rows 4j..4j+3: their slots are the bytes of word j
  const uint32_t my_slots = __shfl(slot4, j);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 4 * j + i;
    const uint32_t slot = (my_slots >> (8 * i)) & 0xffu;
    if (t < T && slot < static_cast<uint32_t>(k))
      a.h[static_cast<int64_t>(t * k + slot) * I + n] = swiglu_bf16(round_bf16(acc0[i]), round_bf16(acc1[i]));
  }
}

// ---------------------------------------------------------------- K3: down projections

constexpr int kDnTiles = 4;  // 16-row tiles of H per K3 workgroup (one per wave)
constexpr int kDnMaxUnits = 16;

// Routed expert number u, columns 64*cb .. 64*cb + 63 of H (model.cpp:718-721):
// d[t*k + slot, n] = h[t*k + slot] . Wd_e[n] for the tokens t that selected
// expert e. Wave w computes tile 4*cb + w over the whole of I in one batch of
// loads; the tokens' h rows are staged in LDS (rows indexed by token).
__device__ void dec_down_routed(const DecodeArgs& a, int u, int cb, uint16_t* s_a) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int T = a.T, k = a.k, H = a.H, I = a.I, xs = xstride(I);
  const int U = static_cast<int>(min(a.seg[0], static_cast<uint32_t>(a.max_seg)));
  if (u >= U) return;  // workgroup-uniform
  const int e = static_cast<int>(min(a.seg[1 + u], static_cast<uint32_t>(a.E - 1)));
  const uint32_t* srow = reinterpret_cast<const uint32_t*>(a.slots + u * kDecMaxT);
  const uint32_t slot4 = srow[lane & 3];
  // tokens' h rows -> LDS rows t (rows of tokens that did not select e stay
  // unset: their products land in output rows that are never stored)
  for (int t = wave; t < T; t += kDecWaves) {
    const uint32_t slot = (__shfl(slot4, t >> 2) >> (8 * (t & 3))) & 0xffu;
    if (slot < static_cast<uint32_t>(k)) dma_row(a.h + static_cast<int64_t>(t * k + slot) * I, I, s_a + t * xs, lane);
  }
  const int nu = I / 128, tile = kDnTiles * cb + wave;
  const uint8_t* tb = a.dn + static_cast<int64_t>(e) * a.dn_es + static_cast<int64_t>(tile) * nu * kBlockSingle;
  const int m = lane & 15, j = lane >> 4;
  const uint16_t* xl = s_a + min(m, T - 1) * xs + 8 * j;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f}, unused = acc;
  tile_units_lds<false, kDnMaxUnits>(tb, 0, nu, xl, lane, acc, unused);
  const int n = tile * 16 + m;
  const uint32_t my_slots = __shfl(slot4, j);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 4 * j + i;
    const uint32_t slot = (my_slots >> (8 * i)) & 0xffu;
    if (t < T && slot < static_cast<uint32_t>(k))
      a.d[static_cast<int64_t>(t * k + slot) * H + n] = f32_to_bf16(acc[i]);
  }
}

// Shared expert down projection, columns 64*cb .. +63, K slice ks of
// kDecSdSplit (model.cpp:746-747): fp32 partial sums sd_part[ks][t][n].
__device__ void dec_down_shared(const DecodeArgs& a, int cb, int ks, uint16_t* s_a) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int T = a.T, H = a.H, Is = a.Is;
  const int nu_all = Is / 128;
  const int ub = (nu_all * ks) / kDecSdSplit, ue = (nu_all * (ks + 1)) / kDecSdSplit, nu = ue - ub;
  const int kk = nu * 128, xs = xstride(kk);
  dma_rows(a.hs + ub * 128, Is, T, kk, s_a, xs, wave, kDecWaves, lane);
  const int tile = kDnTiles * cb + wave;
  const uint8_t* tb = a.sdn + (static_cast<int64_t>(tile) * nu_all + ub) * kBlockSingle;
  const int m = lane & 15, j = lane >> 4;
  const uint16_t* xl = s_a + min(m, T - 1) * xs + 8 * j;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f}, unused = acc;
  tile_units_lds<false, kDnMaxUnits>(tb, 0, nu, xl, lane, acc, unused);
  const int n = tile * 16 + m;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 4 * j + i;
    if (t < T) a.sd_part[(static_cast<int64_t>(ks) * T + t) * H + n] = acc[i];
  }
}

__global__ __launch_bounds__(kDecThreads) void dec_k3(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint16_t* s_a = reinterpret_cast<uint16_t*>(smem);
  const int nblk = a.H / (16 * kDnTiles);
  const int wg = blockIdx.x, n_routed = a.max_seg * nblk;
  if (wg < n_routed)
    dec_down_routed(a, wg / nblk, wg - (wg / nblk) * nblk, s_a);
  else
    dec_down_shared(a, (wg - n_routed) / kDecSdSplit, (wg - n_routed) % kDecSdSplit, s_a);
}

// ---------------------------------------------------------------- K4: combine

// y = sum over slots (fp32, slot order) of bf16(d * score) -> bf16
//   + bf16(sigmoid(gate) * bf16(shared down, K slices added in order)) -> bf16
// (model.cpp:782-803); one thread per 8 columns of a token.
__global__ __launch_bounds__(kDecThreads) void dec_k4(DecodeArgs a) {
  const int oct = a.H / 8;
  const int g = blockIdx.x * kDecThreads + threadIdx.x;
  if (g >= a.T * oct) return;
  const int t = g / oct, o = g - t * oct;
  // every load first (one round trip), then the arithmetic in slot order
  u32x4_t dv[kDecMaxK];
  uint16_t sv[kDecMaxK];
#pragma unroll
  for (int q = 0; q < kDecMaxK; ++q) {
    const int qq = min(q, a.k - 1);
    dv[q] = *reinterpret_cast<const u32x4_t*>(a.d + static_cast<int64_t>(t * a.k + qq) * a.H + o * 8);
    sv[q] = a.scores[t * a.k + qq];
  }
  f32x4_t sp[2 * kDecSdSplit];
  if (a.Is > 0) {
#pragma unroll
    for (int ks = 0; ks < kDecSdSplit; ++ks) {
      const float* p = a.sd_part + (static_cast<int64_t>(ks) * a.T + t) * a.H + o * 8;
      sp[2 * ks] = *reinterpret_cast<const f32x4_t*>(p);
      sp[2 * ks + 1] = *reinterpret_cast<const f32x4_t*>(p + 4);
    }
  }
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < kDecMaxK; ++q) {
    if (q < a.k) {
      const float sc = bf16_to_f32(sv[q]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] += round_bf16(__uint_as_float(dv[q][i] << 16) * sc);
        acc[2 * i + 1] += round_bf16(__uint_as_float(dv[q][i] & 0xffff0000u) * sc);
      }
    }
  }
  float yv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) yv[i] = round_bf16(acc[i]);
  if (a.Is > 0) {
    float sd[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < kDecSdSplit; ++ks) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sd[i] += sp[2 * ks][i];
        sd[4 + i] += sp[2 * ks + 1][i];
      }
    }
    const float gt = a.sgate[t];
#pragma unroll
    for (int i = 0; i < 8; ++i) yv[i] += round_bf16(gt * round_bf16(sd[i]));
  }
  u32x4_t w;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = static_cast<uint32_t>(f32_to_bf16(yv[2 * i])) | (static_cast<uint32_t>(f32_to_bf16(yv[2 * i + 1])) << 16);
  *reinterpret_cast<u32x4_t*>(a.y + static_cast<int64_t>(t) * a.H + o * 8) = w;
}

}  // namespace

// ---------------------------------------------------------------- host side

static size_t k12_lds(const DecodeArgs& a) {
  return kDecRouterLpBytes + static_cast<size_t>(a.T) * xstride(a.H) * 2;
}

static size_t k3_lds(const DecodeArgs& a) {
  const int nu_s = a.Is / 128;
  const int kk_s = ((nu_s + kDecSdSplit - 1) / kDecSdSplit) * 128;
  return static_cast<size_t>(a.T) * xstride(std::max(a.I, kk_s)) * 2;
}

bool decode_plan(DecodeArgs& a) {
  const int nu_i = a.I / 128, nu_s = a.Is / 128;
  if (a.T < 1 || a.T > kDecMaxT || a.k < 1 || a.k > kDecMaxK || a.E < 1 || a.E > kDecMaxE ||
      a.H % 512 || a.I % 128 || a.Is % 128 || a.H > kDecRouterChunks * kWave * 16 ||
      a.H / 128 > 16 || nu_i > kDnMaxUnits ||
      (nu_s + kDecSdSplit - 1) / kDecSdSplit > kDnMaxUnits || (a.Is > 0 && nu_s < kDecSdSplit) ||
      a.H % (16 * kDnTiles))
    return false;
  a.n_rt = (a.E + (a.Is > 0 ? 1 : 0) + kRouterColsPerWg - 1) / kRouterColsPerWg;
  a.n_sgu = a.Is / 32;
  a.max_seg = std::min(a.E, a.T * a.k);
  a.gu_pairs = a.I / 32;
  return k12_lds(a) <= 160 * 1024 && k3_lds(a) <= 160 * 1024;
}

hipError_t launch_decode_k1(const DecodeArgs& a, hipStream_t stream) {
  const dim3 grid(a.n_rt + a.n_sgu), block(kDecThreads);
  if (a.E <= 64)
    hipLaunchKernelGGL(dec_k1<1>, grid, block, k12_lds(a), stream, a);
  else if (a.E <= 128)
    hipLaunchKernelGGL(dec_k1<2>, grid, block, k12_lds(a), stream, a);
  else
    hipLaunchKernelGGL(dec_k1<4>, grid, block, k12_lds(a), stream, a);
  return hipGetLastError();
}

hipError_t launch_decode_k2(const DecodeArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(dec_k2, dim3(a.max_seg * a.gu_pairs + 1), dim3(kDecThreads), k12_lds(a), stream, a);
  return hipGetLastError();
}

hipError_t launch_decode_k3(const DecodeArgs& a, hipStream_t stream) {
  const int nblk = a.H / (16 * kDnTiles);
  const int n = a.max_seg * nblk + (a.Is > 0 ? nblk * kDecSdSplit : 0);
  hipLaunchKernelGGL(dec_k3, dim3(n), dim3(kDecThreads), k3_lds(a), stream, a);
  return hipGetLastError();
}

hipError_t launch_decode_k4(const DecodeArgs& a, hipStream_t stream) {
  const int n = a.T * (a.H / 8);
  hipLaunchKernelGGL(dec_k4, dim3((n + kDecThreads - 1) / kDecThreads), dim3(kDecThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace fmx
