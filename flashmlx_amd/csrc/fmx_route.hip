// fmx_route.hip -- router (logits, softmax, top-k, scores) and the
// token->expert stable counting sort.
//
// Reference: server/src/model.cpp:757-775 (router, softmax, argpartition
// top-k, take_along_axis), :682-700 (switch_mlp's argsort-based sort), and
// the renormalisation of docs/superpowers/plans/2026-04-01-moe-support-plan.md:319-322.
#include "fmx_dev.hpp"

namespace fmx {

bool sort_fits(int64_t n, int64_t E) {
  const int64_t tiles = (n + 63) / 64;
  return n >= 0 && n <= kSortMaxN && E >= 1 && E * tiles <= kSortCntBytes;
}

__global__ __launch_bounds__(kSortThreads) void sort_kernel(const uint32_t* keys, int n, int k,
                                                            int E, SortOut o) {
  __shared__ uint8_t s_cnt[kSortCntBytes];
  __shared__ uint8_t s_rank[kSortMaxN];
  __shared__ uint32_t s_tmp[kSortThreads / kWave + 1];
  sort_block<kSortThreads>(keys, n, k, E, o, s_cnt, s_rank, s_tmp);
}

hipError_t launch_sort(const uint32_t* keys, int n, int k, int E, const SortOut& o,
                       hipStream_t stream) {
  hipLaunchKernelGGL(sort_kernel, dim3(1), dim3(kSortThreads), 0, stream, keys, n, k, E, o);
  return hipGetLastError();
}

// ------------------------------------------------------------------ router

bool router_sort_fits(int64_t n, int64_t E) {
  const int64_t tiles = (n + 63) / 64;
  return n <= kRouterSortMaxN && E * tiles <= kRouterSortCnt && E * 4 <= kRouterSortCnt;
}


// Release this workgroup's global writes and count it in; true in exactly
// one workgroup: the last of `expected` to arrive, which then sees all of
// their writes. Every thread fences its own stores before the barrier.
__device__ inline bool arrive_last(uint32_t* counter, uint32_t expected, int* s_flag) {
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = atomicAdd(counter, 1u);
    *s_flag = (prev == expected - 1) ? 1 : 0;
  }
  __syncthreads();
  const bool last = *s_flag != 0;
  if (last) __threadfence();
  return last;
}

constexpr int kMaxExpertsPerLane = 16;  // E <= 1024
constexpr int kRouterWaves = kRouterThreads / kWave;

// Phase 1 of the router: each wave forms the logits of TT tokens x CE
// consecutive columns. Lanes take interleaved 8-element chunks of H
// (coalesced 16-byte loads); products of bf16 values are exact in fp64.
template <int TT, int CE>
__device__ void router_logits(const RouterArgs& a, int ct, int tt, int wave, int lane) {
  const int H = a.H, E = a.E;
  const int ncols = E + (a.wsg ? 1 : 0);
  const int c0 = (ct * kRouterWaves + wave) * CE;
  if (c0 >= ncols) return;  // wave-uniform
  constexpr int NV = TT * CE;
  double acc[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) acc[i] = 0.0;
  const uint16_t* wrow[CE];
#pragma unroll
  for (int c = 0; c < CE; ++c) {
    const int col = min(c0 + c, ncols - 1);
    wrow[c] = col < E ? a.wr + static_cast<int64_t>(col) * H : a.wsg;
  }
  const uint16_t* xrow[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t)
    xrow[t] = a.x + static_cast<int64_t>(min(tt * kRouterTok + t, a.T - 1)) * H;
  const int nchunk = H / 8;
#pragma unroll 2
  for (int ch = lane; ch < nchunk; ch += kWave) {
    u32x4_t wv[CE], xv[TT];
#pragma unroll
    for (int c = 0; c < CE; ++c) wv[c] = *reinterpret_cast<const u32x4_t*>(wrow[c] + ch * 8);
#pragma unroll
    for (int t = 0; t < TT; ++t) xv[t] = *reinterpret_cast<const u32x4_t*>(xrow[t] + ch * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      double w0[CE], w1[CE];
#pragma unroll
      for (int c = 0; c < CE; ++c) {
        w0[c] = __uint_as_float(wv[c][i] << 16);
        w1[c] = __uint_as_float(wv[c][i] & 0xffff0000u);
      }
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        const double x0 = __uint_as_float(xv[t][i] << 16);
        const double x1 = __uint_as_float(xv[t][i] & 0xffff0000u);
#pragma unroll
        for (int c = 0; c < CE; ++c) {
          acc[t * CE + c] = __builtin_fma(x0, w0[c], acc[t * CE + c]);
          acc[t * CE + c] = __builtin_fma(x1, w1[c], acc[t * CE + c]);
        }
      }
    }
  }
  const double r = reduce_scatter64<NV>(acc, lane);
  constexpr int SH = NV == 1 ? 6 : NV == 2 ? 5 : NV == 4 ? 4 : NV == 8 ? 3 : NV == 16 ? 2 : NV == 32 ? 1 : 0;
  if ((lane & ((1 << SH) - 1)) == 0) {
    const int idx = lane >> SH;
    const int t = tt * kRouterTok + idx / CE, c = c0 + idx % CE;
    if (t < a.T && c < ncols) {
      uint16_t l = f64_to_bf16(r);
      if (c < E && a.lbias)
        l = f64_to_bf16(static_cast<double>(bf16_to_f32(l)) +
                        static_cast<double>(bf16_to_f32(a.lbias[c])));
      a.logits[static_cast<int64_t>(t) * (E + 1) + c] = l;
    }
  }
}

// Phase 2: softmax (fp64, exp_det) and top-k of one token, by one wave.
// The normaliser is summed in a fixed order: lane l adds e = l, l+64, ...
// in turn, then six butterfly steps s_l += s_{l^w} (w = 32..1) leave the
// same total in every lane.
__device__ void router_token(const RouterArgs& a, int t, int lane) {
  const int E = a.E;
  const uint16_t* lrow = a.logits + static_cast<int64_t>(t) * (E + 1);
  double lv[kMaxExpertsPerLane];
  double m = -__builtin_huge_val();
#pragma unroll
  for (int i = 0; i < kMaxExpertsPerLane; ++i) {
    const int e = lane + 64 * i;
    lv[i] = e < E ? static_cast<double>(bf16_to_f32(lrow[e])) : -__builtin_huge_val();
    m = fmax(m, lv[i]);
  }
  m = __ockl_wfred_max_f64(m);
  double ex[kMaxExpertsPerLane];
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < kMaxExpertsPerLane; ++i) {
    const int e = lane + 64 * i;
    ex[i] = e < E ? exp_det(lv[i] - m) : 0.0;
    s += ex[i];
  }
#pragma unroll
  for (int w = 32; w >= 1; w >>= 1) s += __shfl_xor(s, w);
  uint32_t key[kMaxExpertsPerLane];
#pragma unroll
  for (int i = 0; i < kMaxExpertsPerLane; ++i) {
    const int e = lane + 64 * i;
    if (e < E) {
      const uint16_t p = f64_to_bf16(ex[i] / s);
      if (a.probs) a.probs[static_cast<int64_t>(t) * E + e] = p;
      key[i] = (static_cast<uint32_t>(p) << 16) | (0xffffu - static_cast<uint32_t>(e));
    } else {
      key[i] = 0u;
    }
  }
  // top-k, (prob desc, expert asc): probabilities are >= 0, so their bf16
  // bit patterns order like their values. Slot j's winner stays in lane j.
  float sc_sum = 0.0f;
  uint16_t my_sc = 0;
  for (int j = 0; j < a.k; ++j) {
    uint32_t best = 0u;
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; ++i) best = max(best, key[i]);
    best = __ockl_wfred_max_u32(best);
    const uint32_t e = 0xffffu - (best & 0xffffu);
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; ++i)
      if (key[i] == best) key[i] = 0u;
    const uint16_t p = static_cast<uint16_t>(best >> 16);
    sc_sum += bf16_to_f32(p);  // fp32, slot order
    if (lane == j) {
      my_sc = p;
      a.inds[static_cast<int64_t>(t) * a.k + j] = e;
    }
  }
  if (lane < a.k) {
    uint16_t out = my_sc;
    if (a.norm) {
      const double den = static_cast<double>(round_bf16(sc_sum));
      out = f32_to_bf16(static_cast<float>(static_cast<double>(bf16_to_f32(my_sc)) / den));
    }
    a.scores[static_cast<int64_t>(t) * a.k + lane] = out;
  }
  if (lane == 0 && a.wsg && a.sgate) a.sgate[t] = sigmoid_bf16(bf16_to_f32(lrow[E]));
}

static_assert(kPassRows >= kWave, "a segment of at most 64 rows is one pass");

// Stable sort of n <= 64 keys by wave 0 of the workgroup (all threads call).
// s_hist: E words, s_idx: 64 words of LDS.
__device__ void sort_small(const uint32_t* keys, int n, int k, int E, const SortOut& o,
                           uint32_t* s_hist, uint32_t* s_idx) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e < E; e += kRouterThreads) s_hist[e] = 0u;
  __syncthreads();
  const bool valid = wave == 0 && lane < n;
  uint32_t key = valid ? keys[lane] : 0u;
  key = key < static_cast<uint32_t>(E) ? key : static_cast<uint32_t>(E - 1);
  int rank = 0;
  if (wave == 0) {
    const int nbits = E <= 1 ? 1 : 32 - __builtin_clz(static_cast<uint32_t>(E - 1));
    uint64_t eq = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (key >> b) & 1u;
      const uint64_t mb = __ballot(bit);
      eq &= bit ? mb : ~mb;
    }
    rank = __popcll(eq & lanes_below(lane));
    if (valid) atomicAdd(&s_hist[key], 1u);
  }
  __syncthreads();
  if (wave == 0) {
    const int per = (E + 63) / 64;
    const int eb = lane * per, ee = min(eb + per, E);
    uint32_t local = 0;
    for (int e = eb; e < ee; ++e) local += s_hist[e];
    uint32_t incl = local;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const uint32_t y = __shfl_up(incl, d);
      if (lane >= d) incl += y;
    }
    uint32_t run = incl - local;
    for (int e = eb; e < ee; ++e) {
      const uint32_t c = s_hist[e];
      o.offsets[e] = run;
      s_hist[e] = run;
      run += c;
    }
    if (lane == 0) o.offsets[E] = static_cast<uint32_t>(n);
  }
  __syncthreads();
  if (valid) {
    const uint32_t pos = s_hist[key] + rank;
    if (o.order) o.order[pos] = static_cast<uint32_t>(lane);
    if (o.inv) o.inv[lane] = pos;
    if (o.src) o.src[pos] = static_cast<uint32_t>(lane / k);
    if (o.idx) o.idx[pos] = key;
    s_idx[pos] = key;
  }
  __syncthreads();
  if (wave == 0 && o.seg_off) {
    const bool in = lane < n;
    const bool start = in && (lane == 0 || s_idx[lane] != s_idx[lane - 1]);
    const uint64_t b = __ballot(start);
    const int u = __popcll(b & lanes_below(lane));
    if (start) {
      if (o.seg_exp) o.seg_exp[u] = s_idx[lane];
      o.seg_off[u] = static_cast<uint32_t>(lane);
      if (o.pass_tab) {  // n <= 64 = kPassRows: one pass per segment
        const uint64_t above = b & ~((2ull << lane) - 1ull);
        const int next = above ? __ffsll(static_cast<unsigned long long>(above)) - 1 : n;
        o.pass_tab[2 * u] = static_cast<uint32_t>(lane);
        o.pass_tab[2 * u + 1] = s_idx[lane] | (static_cast<uint32_t>(next - lane) << 16);
      }
    }
    if (lane == 0) {
      const int U = __popcll(b);
      o.seg_off[U] = static_cast<uint32_t>(n);
      if (o.seg_n) *o.seg_n = static_cast<uint32_t>(U);
      if (o.pass_n) *o.pass_n = static_cast<uint32_t>(U);
    }
  }
}

__global__ __launch_bounds__(kRouterThreads) void router_kernel(RouterArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t s_cnt[kRouterSortCnt];
  __shared__ uint8_t s_rank[kRouterSortMaxN];
  __shared__ uint32_t s_tmp[kRouterThreads / kWave + 1];
  __shared__ uint32_t s_idx[kWave];
  __shared__ int s_flag;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ct = blockIdx.x, tt = blockIdx.y;
  const int H = a.H;

  // ---- phase 1: logits of this token tile x column tile
  if (a.cols_per_wave == 4)
    router_logits<kRouterTok, 4>(a, ct, tt, wave, lane);
  else if (a.T == 1)
    router_logits<1, 1>(a, ct, tt, wave, lane);
  else
    router_logits<kRouterTok, 1>(a, ct, tt, wave, lane);
  // P8 copy of the tile's x rows, once per token tile
  if (ct == 0 && a.xp) {
    const int oct = H / 8;
    for (int o = tid; o < kRouterTok * oct; o += kRouterThreads) {
      const int tl = o / oct, oc = o % oct;
      const int tok = tt * kRouterTok + tl;
      if (tok >= a.T) continue;
      const u32x4_t v =
          *reinterpret_cast<const u32x4_t*>(a.x + static_cast<int64_t>(tok) * H + oc * 8);
      // elements e0..e7 -> slots 0,2,4,6 (e0..e3) and 1,3,5,7 (e4..e7)
      u32x4_t p;
      p[0] = (v[0] & 0xffffu) | (v[2] << 16);
      p[1] = (v[0] >> 16) | (v[2] & 0xffff0000u);
      p[2] = (v[1] & 0xffffu) | (v[3] << 16);
      p[3] = (v[1] >> 16) | (v[3] & 0xffff0000u);
      *reinterpret_cast<u32x4_t*>(a.xp + static_cast<int64_t>(tok) * H + oc * 8) = p;
    }
  }
  if (!arrive_last(&a.counters[tt], static_cast<uint32_t>(a.n_ct), &s_flag)) return;

  // ---- phase 2 (last column tile of this token tile): softmax and top-k
  for (int tl = wave; tl < kRouterTok; tl += kRouterWaves) {
    const int t = tt * kRouterTok + tl;
    if (t < a.T) router_token(a, t, lane);
  }
  if (tid == 0) a.counters[tt] = 0u;  // every column tile of this token tile has arrived

  if (!a.fuse_sort) return;
  if (a.n_tt > 1) {
    if (!arrive_last(&a.counters[a.n_tt], static_cast<uint32_t>(a.n_tt), &s_flag)) return;
  } else {
    __syncthreads();  // this workgroup's own inds writes are visible after the barrier
  }

  // ---- phase 3 (last token tile): sort all tokens' expert indices
  const int n = a.T * a.k;
  if (n <= kWave)
    sort_small(a.inds, n, a.k, a.E, a.sort, reinterpret_cast<uint32_t*>(s_cnt), s_idx);
  else
    sort_block<kRouterThreads>(a.inds, n, a.k, a.E, a.sort, s_cnt, s_rank, s_tmp);
  if (tid == 0 && a.n_tt > 1) a.counters[a.n_tt] = 0u;
}

hipError_t launch_router(const RouterArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(router_kernel, dim3(a.n_ct, a.n_tt), dim3(kRouterThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace fmx
