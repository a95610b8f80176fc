// fmx_route.hip -- router (logits, softmax, top-k, scores) and the
// token->expert stable counting sort.
//
// Reference: server/src/model.cpp:757-775 (router, softmax, argpartition
// top-k, take_along_axis), :682-700 (switch_mlp's argsort-based sort), and
// the renormalisation of docs/superpowers/plans/2026-04-01-moe-support-plan.md:319-322.
#include "fmx_kernels.hpp"

namespace fmx {

// ------------------------------------------------------------------ helpers

__device__ inline uint64_t lanes_below(int lane) {
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

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

// Stable counting sort of n keys by value, by one workgroup of NT threads.
// Entries are cut into tiles of 64 (one per lane of a wave). Within a tile,
// the lanes holding an equal key are found with one ballot per key bit; a
// lane's rank among them is the popcount of the equal lanes below it. The
// per-(key, tile) counts, scanned in key-major order, give every (key, tile)
// its first output position, so position = base[key][tile] + rank.
// s_cnt: E * n_tiles bytes of LDS; s_rank: n bytes; s_tmp: NT/64 + 1 words.
template <int NT>
__device__ void sort_block(const uint32_t* __restrict__ keys, int n, int k, int E,
                           const SortOut& o, uint8_t* s_cnt, uint8_t* s_rank,
                           uint32_t* s_tmp) {
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

  // segment table of the non-empty keys, ascending
  if (o.seg_off) {
    const int eper = (E + NT - 1) / NT;
    const int eb = tid * eper, ee = min(eb + eper, E);
    uint32_t cnt = 0;
    for (int e = eb; e < ee; ++e) cnt += (o.offsets[e + 1] > o.offsets[e]) ? 1u : 0u;
    uint32_t U = 0;
    uint32_t u = block_exclusive_scan<NT>(cnt, s_tmp, &U);
    for (int e = eb; e < ee; ++e) {
      if (o.offsets[e + 1] > o.offsets[e]) {
        if (o.seg_exp) o.seg_exp[u] = static_cast<uint32_t>(e);
        o.seg_off[u] = o.offsets[e];
        ++u;
      }
    }
    if (tid == 0) {
      o.seg_off[U] = static_cast<uint32_t>(n);
      if (o.seg_n) *o.seg_n = U;
    }
  }
}

// Segment records for the decode GEMM (SortOut::recs): once the segment
// table and src are complete, record u = {src of the first min(count, 16)
// positions (the last one repeated), key, first position, count}.
__device__ void write_seg_recs(const SortOut& o, int nthreads) {
  if (!o.recs || !o.seg_n || !o.seg_exp || !o.seg_off || !o.src) return;
  __syncthreads();
  const uint32_t U = *o.seg_n;
  constexpr int F = 4 + 16;
  for (uint32_t i = threadIdx.x; i < U * F; i += nthreads) {
    const uint32_t u = i / F, f = i - u * F;
    const uint32_t r0 = o.seg_off[u], r1 = o.seg_off[u + 1];
    uint32_t v;
    if (f < 16)
      v = o.src[min(r0 + f, r1 - 1)];
    else if (f == 16)
      v = o.seg_exp[u];
    else if (f == 17)
      v = r0;
    else if (f == 18)
      v = r1 - r0;
    else
      v = 0u;
    o.recs[u * kSegRecWords + f] = v;
  }
}

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
  write_seg_recs(o, kSortThreads);
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

extern "C" __device__ __attribute__((const)) double __ockl_wfred_max_f64(double);

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

// Butterfly reduce-scatter of N = 2^P doubles over the 64 lanes of a wave:
// afterwards lane l holds the wave-wide total of value index l >> (6 - P).
// The router's partial sums are exact, so the association order is free.
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
  double r = v[0];
#pragma unroll
  for (int w = 32 >> P; w >= 1; w >>= 1) r += __shfl_xor(r, w);
  return r;
}

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
    }
    if (lane == 0) {
      const int U = __popcll(b);
      o.seg_off[U] = static_cast<uint32_t>(n);
      if (o.seg_n) *o.seg_n = static_cast<uint32_t>(U);
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
  write_seg_recs(a.sort, kRouterThreads);
  if (tid == 0 && a.n_tt > 1) a.counters[a.n_tt] = 0u;
}

hipError_t launch_router(const RouterArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(router_kernel, dim3(a.n_ct, a.n_tt), dim3(kRouterThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace fmx
