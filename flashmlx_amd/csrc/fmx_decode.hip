// fmx_decode.hip -- the MoE block for decode batches (T <= 16 tokens) on
// packed expert weights, in three kernels:
//
//   K1  router: logits in column workgroups; the last of them to finish
//       derives softmax, top-k, the sort and the routed-expert tables
//       |  shared expert gate/up + SwiGLU (routing-independent, streams
//       meanwhile)
//   K2  routed experts' gate/up + SwiGLU tiles
//   K3  per 64 columns of H: the down projections of every routed expert and
//       of the shared expert; the last workgroup to finish a column block
//       does its top-k weighted combine and the gated shared add, written
//       straight to y
//
// Reference: server/src/model.cpp:750-807 (moe_block), :673-734 (switch_mlp:
// gather_qmm gate/up/down, SwiGLU), :736-748 (shared_expert_mlp), :14-25
// (compiled SwiGLU), :757-775 (router), :682-700 (sort).
//
// A whole forward runs K2 and K3 as one grid (K23): the gate/up tiles first,
// then the down workgroups, which start streaming their weights while the
// last gate/up tiles finish and wait (bounded) only for their own expert's
// h rows. A forward that stops after the gate/up stage runs K2 alone.
//
// Rows of every MFMA tile are indexed by token: a token selects an expert at
// most once, so expert e's tile rows are the tokens that routed to it and no
// gather or sort is needed for the products. Workgroups of one kernel hand
// data over in three places, K1's logits, K23's h rows and K3's column
// blocks, all the same way: device-scope stores, a wait for their
// completion, then a device-scope arrival counter. For the logits and the
// column blocks the last arrival does the consuming work; K23's down
// workgroups instead poll their expert's done flag. A down workgroup waits
// only on gate/up tiles with lower indices, and tiles never wait. Each XCD
// dispatches its workgroups in index order, so when the lowest-indexed
// waiting workgroup waits, every XCD has dispatched each tile it waits on
// (an XCD whose slots all hold waiting workgroups has dispatched everything
// below their indices): those tiles finish and the wait ends.
#include <algorithm>

#include "fmx_dev.hpp"

namespace fmx {

namespace {

constexpr int kDecK2Units = 4;  // units (of H / 128 <= 16) per wave of a gate/up tile pair
// Gate/up tile pairs per K2 workgroup (their loads in flight together, the
// routing tables and staged rows shared): two when the grid has at least
// kDecK2PairGrid tile pairs (about two resident grids of one-pair
// workgroups; the grid is sized for max_seg experts, of which fewer are
// usually routed), else one, so that a small batch still spreads over every
// CU. Measured (Qwen1.5): two pairs -6 % per layer at B=8, -11 % at B=16;
// +2 % at B=4, where one is kept.
constexpr int kDecK2MaxPairs = 2;
constexpr int kDecK2PairGrid = 2 * 4 * 256;
constexpr int kDecK1LpBytes = kDecWaves * kDecMaxT * 8;              // router partials per wave

constexpr int kDecK1LgBytes = kDecMaxT * (kDecMaxE + 1) * 2;         // every token's logits
// K1's LDS: the router's partials and logits, or the shared tiles' quarter
// reduction; then the staged rows
__host__ __device__ inline int k1_lds_main(int T, int H) {
  return (kDecQuadRedBytes > kDecK1LpBytes + kDecK1LgBytes ? kDecQuadRedBytes : kDecK1LpBytes + kDecK1LgBytes) +
         T * xstride(H) * 2;
}

// tile_units_lds for NP tile pairs at once: every pair's loads are issued
// before the one wait, then the pairs are multiplied in turn.
template <int NP, int NU, bool F16>
__device__ inline void pairs_units_lds(const uint8_t* const (&base)[NP], int u0, int u1, const uint16_t* xl,
                                       int lane, f32x4_t (&acc)[NP][2]) {
  PkUnit<true> L[NP][NU];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int d = 0; d < NU; ++d) L[p][d] = pk_load<true>(base[p] + min(u0 + d, u1 - 1) * kBlockPair, lane);
  __builtin_amdgcn_sched_barrier(0);
  wait_vmcnt<NP * NU * pk_load_insts<true>()>();
  lds_dma_barrier();
#pragma unroll
  for (int d = 0; d < NU; ++d) {
    if (u0 + d < u1) {
      act8_t<F16> A[4];
      lds_a<F16>(xl + (u0 + d) * 128, A);
#pragma unroll
      for (int p = 0; p < NP; ++p) pk_unit<true, F16>(L[p][d], A, acc[p][0], acc[p][1]);
    }
  }
}

// ---------------------------------------------------------------- K1: router

// Softmax (fp64, exp_det, fixed-order normaliser) and top-k of NT tokens by
// one wave, as model.cpp:764-775 with the renormalisation of
// moe-support-plan.md:319-322: the k largest bf16 probabilities, ties to the
// lower expert index, slots ordered (probability desc, index asc). The
// tokens' dependent fp64 chains are interleaved; tokens ts[n] >= T are
// computed on padding and not written. s_lg: every token's E (+1) logits.
// Lane l takes the experts e = r + 64 i, r the 6-bit reverse of l: lane l
// accumulates r's partial normaliser, and the DPP tree (adjacent lanes
// first) then adds the partials r and r xor 32 first, r xor 16 next, .., the
// association of the oracle's butterfly (w = 32, 16, .., 1). F16: logits,
// probabilities and scores in fp16 (nonnegative fp16 patterns order like
// their values too).
template <int NPER, int NT, bool F16>
__device__ void route_tokens(const DecodeArgs& a, const int (&ts)[NT], const uint16_t* s_lg, int lane,
                             uint32_t* s_inds) {
  const int E = a.E, ld = E + 1;
  const int r = static_cast<int>(__builtin_bitreverse32(static_cast<uint32_t>(lane)) >> 26);
  double ex[NT][NPER], m[NT], s[NT];
  float lf[NT][NPER];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int t = min(ts[n], a.T - 1);
    float mf = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
      const int e = r + 64 * i;
      lf[n][i] = e < E ? Act<F16>::ld(s_lg[t * ld + e]) : -__builtin_huge_valf();
      mf = fmaxf(mf, lf[n][i]);
    }
    // bf16 (fp16) logits are exact in fp32: the fp32 maximum is the fp64 one
    m[n] = static_cast<double>(wave_max_f32(mf));
  }
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    s[n] = 0.0;
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
      const int e = r + 64 * i;
      ex[n][i] = e < E ? exp_det(static_cast<double>(lf[n][i]) - m[n]) : 0.0;
      s[n] += ex[n][i];
    }
  }
#pragma unroll
  for (int n = 0; n < NT; ++n) s[n] = wave_sum_f64(s[n]);
  uint32_t key[NT][NPER];
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
      const int e = r + 64 * i;
      key[n][i] = 0u;
      if (e < E) {
        const uint16_t p = Act<F16>::from64(ex[n][i] / s[n]);
        if (a.probs && ts[n] < a.T) a.probs[static_cast<int64_t>(ts[n]) * E + e] = p;
        // probabilities are >= 0: their bf16 patterns order like their values
        key[n][i] = (static_cast<uint32_t>(p) << 16) | (0xffffu - static_cast<uint32_t>(e));
      }
    }
  float sc_sum[NT];
  uint32_t my_key[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    sc_sum[n] = 0.0f;
    my_key[n] = 0u;
  }
  for (int j = 0; j < a.k; ++j) {
    uint32_t best[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      best[n] = 0u;
#pragma unroll
      for (int i = 0; i < NPER; ++i) best[n] = max(best[n], key[n][i]);
    }
#pragma unroll
    for (int n = 0; n < NT; ++n) best[n] = wave_max_u32(best[n]);
#pragma unroll
    for (int n = 0; n < NT; ++n) {
#pragma unroll
      for (int i = 0; i < NPER; ++i)
        if (key[n][i] == best[n]) key[n][i] = 0u;
      sc_sum[n] += Act<F16>::ld(static_cast<uint16_t>(best[n] >> 16));  // fp32, slot order
      if (lane == j) my_key[n] = best[n];
    }
  }
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int t = ts[n];
    if (t >= a.T) continue;
    if (lane < a.k) {
      const uint32_t e = 0xffffu - (my_key[n] & 0xffffu);
      uint16_t sc = static_cast<uint16_t>(my_key[n] >> 16);
      if (a.norm) {
        const double den = static_cast<double>(Act<F16>::rnd(sc_sum[n]));
        sc = Act<F16>::st(static_cast<float>(static_cast<double>(Act<F16>::ld(sc)) / den));
      }
      s_inds[t * a.k + lane] = e;
      a.inds[t * a.k + lane] = e;
      a.scores[t * a.k + lane] = sc;
    }
  }
}

// Router column 0, once its own logit is out: the routing of every token,
// the ascending list of routed experts (seg) and each expert's token -> slot
// row (slots). Every column's logits come from the words of this epoch
// (device-scope loads, repeated until all are in: at most a.wait_polls
// rounds; a wait that runs out sets kStatusWaitTimeout and reads the missing
// logits as 0), then the epoch advances. Up to four tokens take a wave each,
// more two per wave; the tables are built by wave 0 alone (its LDS
// operations complete in order, so no workgroup barrier follows the
// routing's), the other waves form the shared gate's sigmoid and reset K23's
// counters meanwhile.
template <int NPER, bool F16>
__device__ void route_finish(const DecodeArgs& a, uint16_t* s_lg, uint32_t ep) {
  __shared__ uint32_t s_inds[kDecMaxT * kDecMaxK];
  __shared__ uint16_t s_segof[kDecMaxE];
  __shared__ uint8_t s_used[kDecMaxE];
  __shared__ uint8_t s_slot[kDecMaxE * kDecMaxT];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int T = a.T, E = a.E, k = a.k, n = T * k;
  const int ld = E + 1;
  const int ncols = E + (a.wsg.w ? 1 : 0);
  const int nw = ncols * T;
  for (int e = tid; e < E; e += kDecThreads) s_used[e] = 0;
  for (int i = tid; i < E * kDecMaxT / 4; i += kDecThreads) reinterpret_cast<uint32_t*>(s_slot)[i] = 0xffffffffu;
  for (int poll = 0;; ++poll) {
    int mine = 1;
    for (int i0 = tid; i0 < nw; i0 += 4 * kDecThreads) {
      uint64_t v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * kDecThreads;
        v[u] = i < nw ? __hip_atomic_load(a.lgx + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * kDecThreads;
        if (i < nw) {
          const int c = i / T, t = i - c * T;
          const bool in = static_cast<uint32_t>(v[u] >> 32) == ep;
          mine &= in ? 1 : 0;
          s_lg[t * ld + c] = in ? static_cast<uint16_t>(v[u]) : 0;
        }
      }
    }
    if (__syncthreads_and(mine)) break;
    if (poll + 1 >= a.wait_polls) {
      if (tid == 0) atomicOr(a.status, kStatusWaitTimeout);
      __syncthreads();
      break;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  if (tid == 0) *a.epoch = ep + 1;  // every column of this epoch has stored its logits
  if (T <= kDecWaves) {
    if (wave < T) {
      const int ts[1] = {wave};
      route_tokens<NPER, 1, F16>(a, ts, s_lg, lane, s_inds);
    }
  } else {
    // tokens wave, wave + 4 (, wave + 8, wave + 12) interleaved in one wave
    for (int t0 = wave; t0 < T; t0 += 2 * kDecWaves) {
      const int ts[2] = {t0, t0 + kDecWaves};
      route_tokens<NPER, 2, F16>(a, ts, s_lg, lane, s_inds);
    }
  }
  lds_barrier();
  if (wave != 0) {
    const int w = tid - kWave;
    if (a.wsg.w)
      for (int t = w; t < T; t += kDecThreads - kWave) a.sgate[t] = Act<F16>::sigmoid(Act<F16>::ld(s_lg[t * ld + E]));
    // K23's per-expert gate/up counters and done flags start the next grid
    // at zero (stores that drain with the kernel, off the chain)
    for (int i = w; i < a.max_seg * (1 + kDecGuFlags); i += kDecThreads - kWave)
      __hip_atomic_store(a.gu_counter + i * kDecCbStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  for (int i = lane; i < n; i += kWave) s_used[s_inds[i]] = 1;
  __builtin_amdgcn_wave_barrier();
  uint32_t U = 0;
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    const bool used = e < E && s_used[e];
    const uint64_t b = __ballot(used);
    if (used) {
      const uint32_t u = U + static_cast<uint32_t>(__popcll(b & lanes_below(lane)));
      a.seg[1 + u] = static_cast<uint32_t>(e);
      s_segof[e] = static_cast<uint16_t>(u);
    }
    U += static_cast<uint32_t>(__popcll(b));
  }
  if (lane == 0) a.seg[0] = U;
  __builtin_amdgcn_wave_barrier();
  // slot table, one byte per (expert u, token t): entry (t, j) marks its
  // expert's row, then the rows go out as whole words
  for (int i = lane; i < n; i += kWave) s_slot[s_segof[s_inds[i]] * kDecMaxT + i / k] = static_cast<uint8_t>(i % k);
  __builtin_amdgcn_wave_barrier();
  for (int i = lane; i < static_cast<int>(U) * (kDecMaxT / 4); i += kWave)
    reinterpret_cast<uint32_t*>(a.slots)[i] = reinterpret_cast<const uint32_t*>(s_slot)[i];
}

// Router column c (column E: the shared-expert gate row) for every token,
// one per workgroup: logits = x . w_c in fp64 (the products of bf16 x with
// bf16 or dequantised 4-bit weights are exact in fp64, and so is their sum up
// to far below the bf16 rounding step, independent of order), rounded once
// to bf16 (model.cpp:757-763, :787-799). Lane g of the workgroup takes
// 16-byte chunk g of H; each wave's partial sums meet in one reduce-scatter
// and the four waves' in LDS. The last router workgroup to finish derives
// the routing. NT: T rounded up to a power of two (the reduce-scatter's
// width).
template <int NPER, int NT, bool NIN, bool F16>
__device__ void dec_router(const DecodeArgs& a, int c, uint8_t* smem) {
  double* s_lp = reinterpret_cast<double*>(smem);
  uint16_t* s_lg = reinterpret_cast<uint16_t*>(smem + kDecK1LpBytes);
  uint16_t* s_x = reinterpret_cast<uint16_t*>(smem + kDecK1LpBytes + kDecK1LgBytes);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = a.H, T = a.T, E = a.E, xs = xstride(H);
  const int nch = H / 8;
  const uint32_t ep = __builtin_amdgcn_readfirstlane(*a.epoch);
  if (!NIN) dma_rows(a.x, H, T, H, s_x, xs, wave, kDecWaves, lane);
  const RChunk wv = c < E ? load_rchunk<F16>(a.wr, c, H, min(tid, nch - 1))
                          : load_rchunk<F16>(a.wsg, 0, H, min(tid, nch - 1));
  const bool biased = c < E && a.lbias;
  const uint16_t lb = biased ? a.lbias[c] : 0;
  if constexpr (NIN) {
    // the input norm, in flight with the router row's loads; column 0 hands
    // the rows on to K23
    __shared__ double s_nred[NT * (kNormThreads / kWave)];
    norm_rows_lds<NT>(a.nin, H, a.nin_w, a.nin_eps, T, H, s_x, xs, s_nred);
    if (c == 0)
      for (int i = tid; i < T * nch; i += kDecThreads) {
        const int t = i / nch, ch = i - t * nch;
        reinterpret_cast<u32x4_t*>(a.x_out + static_cast<int64_t>(t) * H)[ch] =
            *reinterpret_cast<const u32x4_t*>(s_x + t * xs + 8 * ch);
      }
  } else {
    wait_vmcnt0();
    lds_dma_barrier();
  }
  double wd[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) wd[q] = tid < nch ? wv.template get<F16>(q) : 0.0;
  double part[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    part[t] = 0.0;
    if (t < T) {
      const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(s_x + t * xs + min(tid, nch - 1) * 8);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        part[t] = __builtin_fma(static_cast<double>(Act<F16>::lo(xv[q])), wd[2 * q], part[t]);
        part[t] = __builtin_fma(static_cast<double>(Act<F16>::hi(xv[q])), wd[2 * q + 1], part[t]);
      }
    }
  }
  // the last lane of each block of 64 / NT then holds the wave's total of token l / (64 / NT)
  constexpr int kLanesPerToken = kWave / NT;
  const double r = reduce_scatter64<NT>(part, lane);
  if (rs64_holder<NT>(lane)) s_lp[wave * kDecMaxT + lane / kLanesPerToken] = r;
  __syncthreads();
  // The logits go out as device-scope stores (written through to the
  // device's coherence point), tagged with this forward's epoch; router
  // column 0 reads them with device-scope loads: no cache-wide write-back,
  // invalidation or arrival count on either side.
  if (wave == 0 && tid < T) {
    double v = 0.0;
#pragma unroll
    for (int q = 0; q < kDecWaves; ++q) v += s_lp[q * kDecMaxT + tid];
    uint16_t l = Act<F16>::from64(v);
    if (biased) l = Act<F16>::from64(static_cast<double>(Act<F16>::ld(l)) + static_cast<double>(Act<F16>::ld(lb)));
    __hip_atomic_store(a.lgx + c * T + tid, (static_cast<uint64_t>(ep) << 32) | l, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    a.logits[tid * (E + 1) + c] = l;  // the routing accessor's copy
  }
  if (c != 0) return;
  route_finish<NPER, F16>(a, s_lg, ep);
}

// Shared expert gate/up + SwiGLU for tile pair tp (model.cpp:741-747):
// hs[t, n] = swiglu(x_t . Wg[n], x_t . Wu[n]) for every token; wave q
// multiplies K quarter q.
template <int NT, bool NIN, bool F16>
__device__ void dec_shared_gu(const DecodeArgs& a, int tp, uint8_t* smem) {
  float* s_red = reinterpret_cast<float*>(smem);
  uint16_t* s_x = reinterpret_cast<uint16_t*>(smem + kDecQuadRedBytes);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = a.H, T = a.T, Is = a.Is, xs = xstride(H);
  const int nu = H / 128;
  const int u0 = (nu * wave) / kDecWaves, u1 = (nu * (wave + 1)) / kDecWaves;
  const int m = lane & 15, j = lane >> 4;
  const uint16_t* xl = s_x + min(m, T - 1) * xs + 8 * j;
  f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
  const uint8_t* tb = a.sgu + static_cast<int64_t>(tp) * nu * kBlockPair;
  // The router columns' loads go out first: from two tokens on, the tiles
  // hold theirs back about 0.85 us (up to 4 tokens) or 1.3 us (more), so
  // that the columns' rows and weights are not queued behind the shared
  // expert's (Qwen1.5 shape: batch 8 44.3 -> 43.0 us per layer, batch 16
  // 49.5 -> 47.8, batch 4 31.6 -> 30.9). The tiles still end before the
  // routing does; at one token (x and the weight rows land at about 1.9
  // us) the delay would only move their end past it. No last-level-cache
  // warming with the shared down weights either: that LDS DMA (6.5 MB at
  // the Qwen1.5 shape) delayed the columns' loads more than it saved K23.
  {
    const int naps = T <= 1 ? 0 : (T <= 4 ? 2 : 3);  // s_sleep 16 = 1024 clocks each
    for (int z = 0; z < naps; ++z) __builtin_amdgcn_s_sleep(16);
  }
  if constexpr (NIN) {
    // the tile's loads first, then the input norm (its barrier also waits
    // for them), then the products
    __shared__ double s_nred[NT * (kNormThreads / kWave)];
    PkUnit<true> L[kDecK2Units];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int d = 0; d < kDecK2Units; ++d) L[d] = pk_load<true>(tb + min(u0 + d, u1 - 1) * kBlockPair, lane);
    __builtin_amdgcn_sched_barrier(0);
    norm_rows_lds<NT>(a.nin, H, a.nin_w, a.nin_eps, T, H, s_x, xs, s_nred);
#pragma unroll
    for (int d = 0; d < kDecK2Units; ++d) {
      if (u0 + d < u1) {
        act8_t<F16> A[4];
        lds_a<F16>(xl + (u0 + d) * 128, A);
        pk_unit<true, F16>(L[d], A, acc0, acc1);
      }
    }
  } else {
    dma_rows(a.x, H, T, H, s_x, xs, wave, kDecWaves, lane);
    PkUnit<true> L[kDecK2Units];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int d = 0; d < kDecK2Units; ++d) L[d] = pk_load<true>(tb + min(u0 + d, u1 - 1) * kBlockPair, lane);
    __builtin_amdgcn_sched_barrier(0);
    // vector memory operations complete in order: the rows' DMA, issued
    // before the tile's loads, has landed at this count
    wait_vmcnt<kDecK2Units * pk_load_insts<true>()>();
    lds_dma_barrier();
#pragma unroll
    for (int d = 0; d < kDecK2Units; ++d) {
      if (u0 + d < u1) {
        act8_t<F16> A[4];
        lds_a<F16>(xl + (u0 + d) * 128, A);
        pk_unit<true, F16>(L[d], A, acc0, acc1);
      }
    }
  }
  quad_reduce(acc0, acc1, wave, lane, s_red);
  if (wave == 0) {
    const int n = tp * 16 + m;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 4 * j + i;
      if (t < T)
        a.hs[static_cast<int64_t>(t) * Is + n] = Act<F16>::swiglu(Act<F16>::rnd(acc0[i]), Act<F16>::rnd(acc1[i]));
    }
  }
}

// Workgroups [0, n_rt): router columns; [n_rt, n_rt + n_sgu): shared tile pairs.
// NIN: the input norm formed here (single-row forwards of the decoder stack)
// F16: the float16 block (no input norm)
template <int NPER, int NT, bool NIN, bool F16>
__global__ __launch_bounds__(kDecThreads) void dec_k1(DecodeArgs a) {
  static_assert(!(NIN && F16), "the input norm is formed in bf16");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int w = blockIdx.x;
  if (w < a.n_rt)
    dec_router<NPER, NT, NIN, F16>(a, w, smem);
  else
    dec_shared_gu<NT, NIN, F16>(a, w - a.n_rt, smem);
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

// Routed expert number u, gate/up tile pair tp (h columns 16 tp .. 16 tp + 15),
// one per workgroup: wave w multiplies K quarter w (model.cpp:703-715). Small
// equal workgroups keep the grid's last round nearly full. The last
// workgroup runs the sort for the routing accessors. SIGNAL (in K23): the h
// values go out as device-scope stores and, once they have completed, the
// tile is counted in on its expert's gate/up counter.
template <bool SIGNAL, int NP, bool F16>
__device__ void dec_gu_tile(const DecodeArgs& a, int b, uint8_t* smem) {
  float* s_red = reinterpret_cast<float*>(smem);
  uint16_t* s_x = reinterpret_cast<uint16_t*>(smem + NP * kDecQuadRedBytes);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int T = a.T, k = a.k, H = a.H, I = a.I, xs = xstride(H);
  if (b == a.max_seg * a.gu_wgs) {
    dec_sort(a);
    return;
  }
  const int u = b / a.gu_wgs, tp0 = (b - u * a.gu_wgs) * NP;
  // routing tables first: a workgroup without an expert leaves before it
  // starts any LDS DMA
  const int U = static_cast<int>(min(a.seg[0], static_cast<uint32_t>(a.max_seg)));
  if (u >= U) return;  // workgroup-uniform
  const int e = static_cast<int>(min(a.seg[1 + u], static_cast<uint32_t>(a.E - 1)));
  const uint32_t* srow = reinterpret_cast<const uint32_t*>(a.slots + u * kDecMaxT);
  const uint32_t slot4 = srow[lane & 3];  // slots of tokens 4*(lane&3) .. +3
  // the activation rows of the tokens that selected e -> LDS rows t (DMA), in
  // flight with the weight loads; the other rows stay unset, and their
  // products land in output rows that are never stored
  for (int t = wave; t < T; t += kDecWaves) {
    const uint32_t slot = (__shfl(slot4, t >> 2) >> (8 * (t & 3))) & 0xffu;
    if (slot < static_cast<uint32_t>(k)) dma_row(a.x + static_cast<int64_t>(t) * H, H, s_x + t * xs, lane);
  }
  const int nu = H / 128;
  const int u0 = (nu * wave) / kDecWaves, u1 = (nu * (wave + 1)) / kDecWaves;
  const int m = lane & 15, j = lane >> 4;
  const uint16_t* xl = s_x + min(m, T - 1) * xs + 8 * j;
  f32x4_t acc[NP][2];
  const uint8_t* base[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    acc[p][0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    acc[p][1] = acc[p][0];
    base[p] = a.gu + static_cast<int64_t>(e) * a.gu_es + static_cast<int64_t>(tp0 + p) * nu * kBlockPair;
  }
  pairs_units_lds<NP, kDecK2Units, F16>(base, u0, u1, xl, lane, acc);
#pragma unroll
  for (int p = 0; p < NP; ++p)
    quad_reduce(acc[p][0], acc[p][1], wave, lane, s_red + p * (kDecQuadRedBytes / 4));
  if (wave != 0) return;
  // lane 16j + c holds rows 4j..4j+3: their slots are the bytes of word j
  const uint32_t my_slots = __shfl(slot4, j);
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int n = (tp0 + p) * 16 + m;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 4 * j + i;
      const uint32_t slot = (my_slots >> (8 * i)) & 0xffu;
      if (t < T && slot < static_cast<uint32_t>(k)) {
        uint16_t* dst = a.h + static_cast<int64_t>(t * k + slot) * I + n;
        const uint16_t v = Act<F16>::swiglu(Act<F16>::rnd(acc[p][0][i]), Act<F16>::rnd(acc[p][1][i]));
        if (SIGNAL)
          __hip_atomic_store(dst, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
          *dst = v;
      }
    }
  }
  if (SIGNAL) {
    wait_vmcnt0();  // wave 0's device-scope stores have completed
    if (lane == 0) {
      uint32_t* g = a.gu_counter + u * kDecGuWords;
      const uint32_t prev = __hip_atomic_fetch_add(g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (prev == static_cast<uint32_t>(a.gu_wgs - 1)) {  // the expert's last workgroup: every h store is done
#pragma unroll
        for (int c = 1; c <= kDecGuFlags; ++c)
          __hip_atomic_store(g + c * kDecCbStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// K2 alone (forwards that stop after the gate/up stage)
template <int NP, bool F16>
__global__ __launch_bounds__(kDecThreads) void dec_k2(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  dec_gu_tile<false, NP, F16>(a, blockIdx.x, smem);
}

// ---------------------------------------------------------------- K3: down projections

constexpr int kDnTiles = 4;  // 16-row tiles of H per K3 workgroup (one per wave)
constexpr int kDnMaxUnits = 16;
constexpr int kDnSmallUnits = 12;  // a ring this short leaves room for four workgroups per CU

// The top-k weighted combine of column block cb (columns 64 cb .. 64 cb + 63)
// for every token (model.cpp:782-803): y = bf16(sum over slots, fp32 in slot
// order, of bf16(d * score)) + bf16(sigmoid(gate) * bf16(shared down, K
// slices added in order)) (F16: every rounding to fp16). d and the shared
// slices were written by other workgroups with device-scope stores; they are
// read with device-scope loads.
template <bool F16>
__device__ void dec_combine(const DecodeArgs& a, int cb) {
  const int T = a.T, k = a.k, H = a.H;
  for (int g = threadIdx.x; g < T * 32; g += kDecThreads) {
    const int t = g >> 5, c = cb * 64 + 2 * (g & 31);
    uint32_t dv[2 * kDecMaxK];
    uint16_t sv[kDecMaxK];
#pragma unroll
    for (int q = 0; q < kDecMaxK; ++q) {
      const int qq = min(q, k - 1);
      const uint32_t* p = a.dw + static_cast<int64_t>(t * k + qq) * H + c;
      dv[2 * q] = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      dv[2 * q + 1] = __hip_atomic_load(p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sv[q] = a.scores[t * k + qq];
    }
    uint32_t sp[2 * kDecSdSplit];
    if (a.Is > 0) {
#pragma unroll
      for (int ks = 0; ks < kDecSdSplit; ++ks) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(a.sd_part) + (static_cast<int64_t>(ks) * T + t) * H + c;
        sp[2 * ks] = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sp[2 * ks + 1] = __hip_atomic_load(p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    float acc[2] = {0.f, 0.f};
#pragma unroll
    for (int q = 0; q < kDecMaxK; ++q) {
      if (q < k) {
        const float sc = Act<F16>::ld(sv[q]);
#pragma unroll
        for (int i = 0; i < 2; ++i)
          acc[i] += Act<F16>::rnd(Act<F16>::ld(static_cast<uint16_t>(dv[2 * q + i])) * sc);
      }
    }
    float yv[2] = {Act<F16>::rnd(acc[0]), Act<F16>::rnd(acc[1])};
    if (a.Is > 0) {
      const float gt = a.sgate[t];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        float sd = 0.f;
#pragma unroll
        for (int ks = 0; ks < kDecSdSplit; ++ks) sd += __uint_as_float(sp[2 * ks + i]);
        yv[i] += Act<F16>::rnd(gt * Act<F16>::rnd(sd));
      }
    }
    *reinterpret_cast<uint32_t*>(a.y + static_cast<int64_t>(t) * H + c) =
        static_cast<uint32_t>(Act<F16>::st(yv[0])) | (static_cast<uint32_t>(Act<F16>::st(yv[1])) << 16);
  }
}

// Counts a K3 workgroup's outputs for column block cb in, once every wave's
// device-scope stores have completed; the last of the block's contributors
// (its U routed experts and the shared expert's K slices) combines the block
// and resets the count.
template <bool F16>
__device__ void dec_arrive(const DecodeArgs& a, int cb, int U) {
  __shared__ int s_last_cb;
  wait_vmcnt0();
  __syncthreads();  // also: every thread is done with the previous call's s_last_cb
  if (threadIdx.x == 0) {
    const uint32_t target = static_cast<uint32_t>(U + (a.Is > 0 ? kDecSdSplit : 0));
    s_last_cb = __hip_atomic_fetch_add(a.cb_counter + cb * kDecCbStride, 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT) == target - 1;
  }
  __syncthreads();
  if (!s_last_cb) return;
  dec_combine<F16>(a, cb);
  if (threadIdx.x == 0)
    __hip_atomic_store(a.cb_counter + cb * kDecCbStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Routed expert number u, columns 64*cb .. 64*cb + 63 of H for the TPW
// column blocks cb = TPW*cbp .. (model.cpp:718-721): d[t*k + slot, n] =
// h[t*k + slot] . Wd_e[n] for the tokens t that selected expert e. Wave w
// computes tile 4*cb + w of each block over the whole of I in one batch of
// loads (a short I, at most half the ring, leaves room for two blocks: half
// the workgroups, each with twice the bytes behind one preamble); the
// tokens' h rows are staged in LDS (rows indexed by token).
//
// h is written by gate/up workgroups of the same grid (K23). Wave 0 reads
// one copy of its expert's done flag, then every wave issues its weight
// loads (they do not depend on h); loads complete in order, so the flag's
// value is in while the weights are still in flight. Until the flag is set,
// wave 0 polls it (s_sleep between reads, at most a.wait_polls reads, by
// default kDecWaitPolls: far beyond any real wait, a guard against a hang)
// while the other waves wait at a barrier. Then every wave fetches its h rows
// with device-scope DMA. A wait that ran out stores NaN products, so that the
// failure shows in y instead of stale rows passing for results, and sets
// kStatusWaitTimeout in the workspace's status word.

template <int NU, int TPW, bool F16>
__device__ void dec_down_routed(const DecodeArgs& a, int u, int cbp, uint16_t* s_a) {
  // TPW column blocks of 64 (cb = TPW*cbp + c), one 16-row tile of each per wave
  static_assert(TPW == 1 || TPW == 2, "one or two column blocks per workgroup");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int T = a.T, k = a.k, H = a.H, I = a.I, xs = xstride(I);
  const int U = static_cast<int>(min(a.seg[0], static_cast<uint32_t>(a.max_seg)));
  if (u >= U) return;  // workgroup-uniform
  const int e = static_cast<int>(min(a.seg[1 + u], static_cast<uint32_t>(a.E - 1)));
  const uint32_t* srow = reinterpret_cast<const uint32_t*>(a.slots + u * kDecMaxT);
  const uint32_t slot4 = srow[lane & 3];
  const int nu = I / 128;  // TPW * nu <= NU (launch_decode_k23)
  const int m = lane & 15, j = lane >> 4;
  const uint16_t* xl = s_a + min(m, T - 1) * xs + 8 * j;
  const uint8_t* tb[TPW];
#pragma unroll
  for (int c = 0; c < TPW; ++c) {
    const int tile = kDnTiles * (TPW * cbp + c) + wave;
    tb[c] = a.dn + static_cast<int64_t>(e) * a.dn_es + static_cast<int64_t>(tile) * nu * kBlockSingle;
  }
  f32x4_t acc[TPW], unused = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < TPW; ++c) acc[c] = unused;
  __shared__ int s_timed_out;
  const uint32_t* flag = a.gu_counter + u * kDecGuWords + (1 + cbp % kDecGuFlags) * kDecCbStride;
  uint32_t done = 0;
  if (wave == 0) done = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // the ring's NU slots: tile c's units at c * (NU / TPW) ..
  constexpr int PER = NU / TPW;
  PkUnit<false> L[NU];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int c = 0; c < TPW; ++c)
#pragma unroll
    for (int d = 0; d < PER; ++d) L[c * PER + d] = pk_load<false>(tb[c] + min(d, nu - 1) * kBlockSingle, lane);
  __builtin_amdgcn_sched_barrier(0);
  if (wave == 0) {
    done = a.wait_polls > 0 ? __builtin_amdgcn_readfirstlane(done) : 0u;
    for (int poll = 1; done == 0 && poll < a.wait_polls; ++poll) {
      __builtin_amdgcn_s_sleep(16);
      done = __builtin_amdgcn_readfirstlane(__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    }
    if (lane == 0) {
      s_timed_out = done == 0;
      if (done == 0) atomicOr(a.status, kStatusWaitTimeout);
    }
    wait_lgkmcnt0();  // the LDS write lands before the barrier (the weights stay in flight)
  }
  lds_dma_barrier();  // wave 0 has seen the flag (no wait for the weights in flight)
  for (int t = wave; t < T; t += kDecWaves) {
    const uint32_t slot = (__shfl(slot4, t >> 2) >> (8 * (t & 3))) & 0xffu;
    if (slot < static_cast<uint32_t>(k))
      dma_row<kCpolDevice>(a.h + static_cast<int64_t>(t * k + slot) * I, I, s_a + t * xs, lane);
  }
  wait_vmcnt0();
  lds_dma_barrier();
#pragma unroll
  for (int d = 0; d < PER; ++d) {
    if (d < nu) {
      act8_t<F16> A[4];
      lds_a<F16>(xl + d * 128, A);
#pragma unroll
      for (int c = 0; c < TPW; ++c) pk_unit<false, F16>(L[c * PER + d], A, acc[c], unused);
    }
  }
  if (s_timed_out) {
#pragma unroll
    for (int c = 0; c < TPW; ++c) acc[c] = f32x4_t{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")};
  }
  const uint32_t my_slots = __shfl(slot4, j);
#pragma unroll
  for (int c = 0; c < TPW; ++c) {
    const int n = (kDnTiles * (TPW * cbp + c) + wave) * 16 + m;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 4 * j + i;
      const uint32_t slot = (my_slots >> (8 * i)) & 0xffu;
      if (t < T && slot < static_cast<uint32_t>(k))
        __hip_atomic_store(a.dw + static_cast<int64_t>(t * k + slot) * H + n, static_cast<uint32_t>(Act<F16>::st(acc[c][i])),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
#pragma unroll
  for (int c = 0; c < TPW; ++c) dec_arrive<F16>(a, TPW * cbp + c, U);
}

// Shared expert down projection, columns 64*cb .. +63, K slice ks of
// kDecSdSplit (model.cpp:746-747): fp32 partial sums sd_part[ks][t][n].
template <int NU, bool F16>
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
  tile_units_lds<false, NU, F16>(tb, 0, nu, xl, lane, acc, unused);
  const int n = tile * 16 + m;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 4 * j + i;
    if (t < T)
      __hip_atomic_store(reinterpret_cast<uint32_t*>(a.sd_part) + (static_cast<int64_t>(ks) * T + t) * H + n,
                         __float_as_uint(acc[i]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  dec_arrive<F16>(a, cb, static_cast<int>(min(a.seg[0], static_cast<uint32_t>(a.max_seg))));
}

// K23 in dispatch order: K2's workgroups (the gate/up tiles, expert-major,
// then the sort), the shared expert's down workgroups (they wait for
// nothing), then the routed down workgroups, expert-major, so that the
// experts whose tiles were dispatched first are the first waited on.
// (Dispatching an expert's down workgroups right behind its tiles, about one
// resident grid later, measured slower: their waits hold slots that the
// tiles still need.)
template <int NU, int NP, int TPW, bool F16>
__global__ __launch_bounds__(kDecThreads) void dec_k23(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint16_t* s_a = reinterpret_cast<uint16_t*>(smem);
  const int D = a.H / (16 * kDnTiles) / TPW;  // routed down workgroups per expert
  const int n_gu = a.max_seg * a.gu_wgs + 1;
  const int n_shared = a.Is > 0 ? (a.H / (16 * kDnTiles)) * kDecSdSplit : 0;
  const int b = blockIdx.x;
  if (b < n_gu)
    dec_gu_tile<true, NP, F16>(a, b, smem);
  else if (b - n_gu < n_shared)
    dec_down_shared<NU, F16>(a, (b - n_gu) / kDecSdSplit, (b - n_gu) % kDecSdSplit, s_a);
  else
    dec_down_routed<NU, TPW, F16>(a, (b - n_gu - n_shared) / D, (b - n_gu - n_shared) % D, s_a);
}

}  // namespace

// ---------------------------------------------------------------- host side

static size_t k1_lds(const DecodeArgs& a) { return k1_lds_main(a.T, a.H); }

// K2: the quarter reduction, then the staged rows
static size_t k2_lds(const DecodeArgs& a) {
  return static_cast<size_t>(a.k2_pairs) * kDecQuadRedBytes + static_cast<size_t>(a.T) * xstride(a.H) * 2;
}

static size_t k3_lds(const DecodeArgs& a) {
  const int nu_s = a.Is / 128;
  const int kk_s = ((nu_s + kDecSdSplit - 1) / kDecSdSplit) * 128;
  return static_cast<size_t>(a.T) * xstride(std::max(a.I, kk_s)) * 2;
}

bool decode_plan(DecodeArgs& a) {
  const int nu_i = a.I / 128, nu_s = a.Is / 128;
  if (a.nin && (a.T > kDecNinMaxT || !a.nin_w || !a.x_out || a.H / 8 > kNormThreads * kNormMaxChunks ||
                a.H / 128 > kDecK2Units * kDecWaves))
    return false;
  if (a.T < 1 || a.T > kDecMaxT || a.k < 1 || a.k > kDecMaxK || a.E < 1 || a.E > kDecMaxE ||
      a.H % 512 || a.I % 128 || a.Is % 128 || a.H / 8 > kDecThreads ||
      a.H / 128 > 16 || nu_i > kDnMaxUnits ||
      (nu_s + kDecSdSplit - 1) / kDecSdSplit > kDnMaxUnits || (a.Is > 0 && nu_s < kDecSdSplit) ||
      a.H % (16 * kDnTiles) || a.H / (16 * kDnTiles) > kDecMaxColBlocks)
    return false;
  a.n_rt = a.E + (a.Is > 0 ? 1 : 0);
  a.n_sgu = a.Is / 16;
  a.max_seg = std::min(a.E, a.T * a.k);
  a.gu_tiles = a.I / 16;
  a.k2_pairs = a.max_seg * a.gu_tiles >= kDecK2PairGrid ? kDecK2MaxPairs : 1;
  a.gu_wgs = a.gu_tiles / a.k2_pairs;  // I % 128 == 0: the pairs divide the tiles
  return k1_lds(a) <= 160 * 1024 && k2_lds(a) <= 160 * 1024 && k3_lds(a) <= 160 * 1024;
}

template <int NPER, bool F16>
static void launch_k1_nt(const DecodeArgs& a, hipStream_t stream) {
  const dim3 grid(a.n_rt + a.n_sgu), block(kDecThreads);
  static_assert(kDecNinMaxT == 1, "the input-norm K1 is instantiated for one row");
  if constexpr (!F16) {
    if (a.nin) {
      hipLaunchKernelGGL((dec_k1<NPER, 1, true, false>), grid, block, k1_lds(a), stream, a);
      return;
    }
  }
  if (a.T <= 1)
    hipLaunchKernelGGL((dec_k1<NPER, 1, false, F16>), grid, block, k1_lds(a), stream, a);
  else if (a.T <= 2)
    hipLaunchKernelGGL((dec_k1<NPER, 2, false, F16>), grid, block, k1_lds(a), stream, a);
  else if (a.T <= 4)
    hipLaunchKernelGGL((dec_k1<NPER, 4, false, F16>), grid, block, k1_lds(a), stream, a);
  else if (a.T <= 8)
    hipLaunchKernelGGL((dec_k1<NPER, 8, false, F16>), grid, block, k1_lds(a), stream, a);
  else
    hipLaunchKernelGGL((dec_k1<NPER, 16, false, F16>), grid, block, k1_lds(a), stream, a);
}

template <bool F16>
static void launch_k1_dt(const DecodeArgs& a, hipStream_t stream) {
  if (a.E <= 64)
    launch_k1_nt<1, F16>(a, stream);
  else if (a.E <= 128)
    launch_k1_nt<2, F16>(a, stream);
  else
    launch_k1_nt<4, F16>(a, stream);
}

hipError_t launch_decode_k1(const DecodeArgs& a, hipStream_t stream) {
  if (a.f16)
    launch_k1_dt<true>(a, stream);
  else
    launch_k1_dt<false>(a, stream);
  return hipGetLastError();
}

hipError_t launch_decode_k2(const DecodeArgs& a, hipStream_t stream) {
  const dim3 grid(a.max_seg * a.gu_wgs + 1);
  if (a.k2_pairs == 2)
    hipLaunchKernelGGL((a.f16 ? dec_k2<2, true> : dec_k2<2, false>), grid, dim3(kDecThreads), k2_lds(a), stream, a);
  else
    hipLaunchKernelGGL((a.f16 ? dec_k2<1, true> : dec_k2<1, false>), grid, dim3(kDecThreads), k2_lds(a), stream, a);
  return hipGetLastError();
}

static bool k3_small_ring(const DecodeArgs& a) {
  const int nu_s = a.Is / 128;
  return std::max(a.I / 128, (nu_s + kDecSdSplit - 1) / kDecSdSplit) <= kDnSmallUnits;
}

// Column blocks per routed down workgroup: two when a tile's units fill at
// most half the load ring (I <= 768 with the 12-unit ring) and the grid has
// at least kDecK3PairGrid routed down workgroups (about two resident grids),
// else one. Measured (Qwen3, I = 768): -3 % per layer at B=16, +14 % at B=1
// (half of 256 workgroups leaves CUs idle), where one is kept.
constexpr int kDecK3PairGrid = 2 * 4 * 256;

static int k3_blocks_per_wg(const DecodeArgs& a) {
  const int ring = k3_small_ring(a) ? kDnSmallUnits : kDnMaxUnits;
  const int nblk = a.H / (16 * kDnTiles);
  return (2 * (a.I / 128) <= ring && nblk % 2 == 0 && a.max_seg * nblk >= kDecK3PairGrid) ? 2 : 1;
}

static int k3_workgroups(const DecodeArgs& a) {
  const int nblk = a.H / (16 * kDnTiles);
  return a.max_seg * (nblk / k3_blocks_per_wg(a)) + (a.Is > 0 ? nblk * kDecSdSplit : 0);
}

template <int NU, int NP, int TPW>
static void launch_k23(const DecodeArgs& a, int n, size_t lds, hipStream_t stream) {
  if (a.f16)
    hipLaunchKernelGGL((dec_k23<NU, NP, TPW, true>), dim3(n), dim3(kDecThreads), lds, stream, a);
  else
    hipLaunchKernelGGL((dec_k23<NU, NP, TPW, false>), dim3(n), dim3(kDecThreads), lds, stream, a);
}

template <int NU, int NP>
static void launch_k23_tpw(const DecodeArgs& a, int n, size_t lds, hipStream_t stream) {
  if (k3_blocks_per_wg(a) == 2)
    launch_k23<NU, NP, 2>(a, n, lds, stream);
  else
    launch_k23<NU, NP, 1>(a, n, lds, stream);
}

hipError_t launch_decode_k23(const DecodeArgs& a, hipStream_t stream) {
  const int n = a.max_seg * a.gu_wgs + 1 + k3_workgroups(a);
  const size_t lds = std::max(k2_lds(a), k3_lds(a));
  const bool small = k3_small_ring(a);
  if (a.k2_pairs == 2) {
    if (small)
      launch_k23_tpw<kDnSmallUnits, 2>(a, n, lds, stream);
    else
      launch_k23_tpw<kDnMaxUnits, 2>(a, n, lds, stream);
  } else {
    if (small)
      launch_k23_tpw<kDnSmallUnits, 1>(a, n, lds, stream);
    else
      launch_k23_tpw<kDnMaxUnits, 1>(a, n, lds, stream);
  }
  return hipGetLastError();
}


}  // namespace fmx
