// fmx_route.hip -- router (logits, softmax, top-k, scores) and the
// token->expert stable counting sort.
//
// Reference: server/src/model.cpp:757-775 (router, softmax, argpartition
// top-k, take_along_axis), :682-700 (switch_mlp's argsort-based sort), and
// the renormalisation of docs/superpowers/plans/2026-04-01-moe-support-plan.md:319-322.
#include <algorithm>

#include "fmx_dev.hpp"

namespace fmx {

bool sort_fits(int64_t n, int64_t E) {
  return n >= 0 && n <= kSortMaxN && E >= 1 && E <= kSortMaxE;
}

namespace {

constexpr int kSortWaves = kSortThreads / kWave;

}  // namespace

// Stable counting sort of n keys (< E; larger ones count as E - 1), one
// workgroup per key value e. Every workgroup histograms all keys in LDS
// (LDS atomics; counts do not depend on order) and scans the histogram, so
// each knows every key's first sorted position; workgroup e then walks the
// entries in order, 1024 at a time, and gives each entry of key e its
// position: offset[e] + the number of earlier entries of key e (a ballot
// per wave, the waves' counts in order, a running total), which is the
// stable order. The outputs' scattered stores spread over E workgroups.
// Workgroup 0 writes offsets and the segment and pass counts; workgroup e
// its own segment and passes. Up to kSortLdsN keys stay in LDS between the
// two walks; more are read again from the key array (in the L2 by then).
__global__ __launch_bounds__(kSortThreads) void sort_kernel(const uint32_t* keys, int n, int k,
                                                            int E, SortOut o) {
  __shared__ uint16_t s_key[kSortLdsN];
  __shared__ uint32_t s_cnt[kSortMaxE];
  __shared__ uint32_t s_tmp[kSortWaves + 1];
  __shared__ uint32_t s_wcnt[kSortWaves];
  __shared__ uint32_t s_mine[4];  // offset, count, segment and first pass of key e
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int e = blockIdx.x;
  const uint32_t emax = static_cast<uint32_t>(E - 1);

  const bool in_lds = n <= kSortLdsN;
  for (int i = tid; i < E; i += kSortThreads) s_cnt[i] = 0u;
  __syncthreads();
#pragma unroll 8
  for (int i = tid; i < n; i += kSortThreads) {
    const uint32_t key = min(keys[i], emax);
    if (in_lds) s_key[i] = static_cast<uint16_t>(key);
    atomicAdd(&s_cnt[key], 1u);
  }
  __syncthreads();

  // offsets, segment numbers and first passes of every key (E <= kSortThreads)
  const uint32_t c = tid < E ? s_cnt[tid] : 0u;
  uint32_t U = 0, NP = 0;
  const uint32_t off = block_exclusive_scan<kSortThreads>(c, s_tmp, nullptr);
  const uint32_t u = block_exclusive_scan<kSortThreads>(c ? 1u : 0u, s_tmp, &U);
  const uint32_t p = block_exclusive_scan<kSortThreads>((c + kPassRows - 1) / kPassRows, s_tmp, &NP);
  if (tid == e) {
    s_mine[0] = off;
    s_mine[1] = c;
    s_mine[2] = u;
    s_mine[3] = p;
  }
  if (e == 0 && o.flag) {
    const int any = __syncthreads_or(tid < o.n_ovf ? static_cast<int>(o.ovf[tid] != 0u) : 0);
    if (tid == 0) *o.flag = any ? 1u : 0u;
  }
  if (e == 0) {
    if (tid < E) o.offsets[tid] = off;
    if (tid == 0) {
      o.offsets[E] = static_cast<uint32_t>(n);
      if (o.seg_off) o.seg_off[U] = static_cast<uint32_t>(n);
      if (o.seg_n) *o.seg_n = U;
      if (o.pass_n) *o.pass_n = NP;
    }
  }
  __syncthreads();
  const uint32_t my_off = s_mine[0], my_c = s_mine[1];
  if (my_c == 0) return;  // workgroup-uniform
  if (tid == 0 && o.seg_off) {
    const uint32_t su = s_mine[2];
    if (o.seg_exp) o.seg_exp[su] = static_cast<uint32_t>(e);
    o.seg_off[su] = my_off;
    if (o.pass_tab) {
      uint32_t pp = s_mine[3];
      for (uint32_t r = 0; r < my_c; r += kPassRows, ++pp) {
        o.pass_tab[2 * pp] = my_off + r;
        o.pass_tab[2 * pp + 1] = static_cast<uint32_t>(e) | (min(my_c - r, static_cast<uint32_t>(kPassRows)) << 16);
      }
    }
  }

  // the entries of key e, in order
  uint32_t run = my_off;
  for (int base = 0; base < n; base += kSortThreads) {
    const int i = base + tid;
    const bool match = i < n && (in_lds ? static_cast<uint32_t>(s_key[i]) : min(keys[i], emax)) ==
                                    static_cast<uint32_t>(e);
    const uint64_t b = __ballot(match);
    if (lane == 0) s_wcnt[wave] = static_cast<uint32_t>(__popcll(b));
    __syncthreads();
    uint32_t before = 0, all = 0;
    for (int w = 0; w < kSortWaves; ++w) {
      const uint32_t cw = s_wcnt[w];
      before += w < wave ? cw : 0u;
      all += cw;
    }
    if (match) {
      const uint32_t pos = run + before + static_cast<uint32_t>(__popcll(b & lanes_below(lane)));
      if (o.order) o.order[pos] = static_cast<uint32_t>(i);
      if (o.row_map) {
        const uint32_t m = static_cast<uint32_t>(o.row_m), ui = static_cast<uint32_t>(i);
        const uint32_t l = min(o.row_lhs[ui / m], static_cast<uint32_t>(o.x_rows / o.row_m - 1));
        o.row_map[pos] = l * m + ui % m;
      }
      if (o.inv) o.inv[i] = pos;
      if (o.src) o.src[pos] = static_cast<uint32_t>(i / k);
      if (o.idx) o.idx[pos] = static_cast<uint32_t>(e);
    }
    run += all;
    __syncthreads();  // s_wcnt is rewritten by the next chunk
  }
}

hipError_t launch_sort(const uint32_t* keys, int n, int k, int E, const SortOut& o,
                       hipStream_t stream) {
  if (o.row_map && (!o.row_lhs || o.row_m < 1 || o.x_rows < o.row_m)) return hipErrorInvalidValue;
  if (o.flag && (!o.ovf || o.n_ovf > kSortThreads)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(sort_kernel, dim3(E), dim3(kSortThreads), 0, stream, keys, n, k, E, o);
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
// (coalesced 16-byte loads); products of bf16 values are exact in fp64, and
// so are those of fp16 values (F16: a float16 block, logits rounded to fp16).
template <int TT, int CE, bool F16>
__device__ void router_logits(const RouterArgs& a, int ct, int tt, int wave, int lane) {
  const int H = a.H, E = a.E;
  const int ncols = E + (a.wsg.w ? 1 : 0);
  const int c0 = (ct * kRouterWaves + wave) * CE;
  if (c0 >= ncols) return;  // wave-uniform
  constexpr int NV = TT * CE;
  double acc[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) acc[i] = 0.0;
  int col[CE];
#pragma unroll
  for (int c = 0; c < CE; ++c) col[c] = min(c0 + c, ncols - 1);
  const uint16_t* xrow[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t)
    xrow[t] = a.x + static_cast<int64_t>(min(tt * kRouterTok + t, a.T - 1)) * H;
  const int nchunk = H / 8;
#pragma unroll 2
  for (int ch = lane; ch < nchunk; ch += kWave) {
    RChunk wv[CE];
    u32x4_t xv[TT];
#pragma unroll
    for (int c = 0; c < CE; ++c)
      wv[c] = col[c] < E ? load_rchunk<F16>(a.wr, col[c], H, ch) : load_rchunk<F16>(a.wsg, 0, H, ch);
#pragma unroll
    for (int t = 0; t < TT; ++t) xv[t] = *reinterpret_cast<const u32x4_t*>(xrow[t] + ch * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      double w0[CE], w1[CE];
#pragma unroll
      for (int c = 0; c < CE; ++c) {
        w0[c] = wv[c].template get<F16>(2 * i);
        w1[c] = wv[c].template get<F16>(2 * i + 1);
      }
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        const double x0 = Act<F16>::lo(xv[t][i]);
        const double x1 = Act<F16>::hi(xv[t][i]);
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
  if (rs64_holder<NV>(lane)) {
    const int idx = lane >> SH;
    const int t = tt * kRouterTok + idx / CE, c = c0 + idx % CE;
    if (t < a.T && c < ncols) {
      uint16_t l = Act<F16>::from64(r);
      if (c < E && a.lbias)
        l = Act<F16>::from64(static_cast<double>(Act<F16>::ld(l)) +
                             static_cast<double>(Act<F16>::ld(a.lbias[c])));
      a.logits[static_cast<int64_t>(t) * (E + 1) + c] = l;
    }
  }
}

// Phase 2: softmax (fp64, exp_det) and top-k of one token, by one wave.
// The normaliser is summed in a fixed order: lane l adds e = l, l+64, ...
// in turn, then six butterfly steps s_l += s_{l^w} (w = 32..1) leave the
// same total in every lane. F16: logits, probabilities and scores in fp16.
template <bool F16>
__device__ void router_token(const RouterArgs& a, int t, int lane) {
  const int E = a.E;
  const int nblk = (E + kWave - 1) / kWave;  // 64-expert blocks (wave-uniform)
  const uint16_t* lrow = a.logits + static_cast<int64_t>(t) * (E + 1);
  double lv[kMaxExpertsPerLane];
  double m = -__builtin_huge_val();
#pragma unroll
  for (int i = 0; i < kMaxExpertsPerLane; ++i) {
    const int e = lane + 64 * i;
    lv[i] = -__builtin_huge_val();
    if (i < nblk) {
      if (e < E) lv[i] = static_cast<double>(Act<F16>::ld(lrow[e]));
      m = fmax(m, lv[i]);
    }
  }
  m = __ockl_wfred_max_f64(m);
  double ex[kMaxExpertsPerLane];
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < kMaxExpertsPerLane; ++i) {
    const int e = lane + 64 * i;
    ex[i] = 0.0;
    if (i < nblk) {
      if (e < E) ex[i] = exp_det(lv[i] - m);
      s += ex[i];
    }
  }
#pragma unroll
  for (int w = 32; w >= 1; w >>= 1) s += __shfl_xor(s, w);
  uint32_t key[kMaxExpertsPerLane];
#pragma unroll
  for (int i = 0; i < kMaxExpertsPerLane; ++i) {
    const int e = lane + 64 * i;
    if (i < nblk && e < E) {
      const uint16_t p = Act<F16>::from64(ex[i] / s);
      if (a.probs) a.probs[static_cast<int64_t>(t) * E + e] = p;
      key[i] = (static_cast<uint32_t>(p) << 16) | (0xffffu - static_cast<uint32_t>(e));
    } else {
      key[i] = 0u;
    }
  }
  // top-k, (prob desc, expert asc): probabilities are >= 0, so their bf16
  // (fp16) bit patterns order like their values. Slot j's winner stays in lane j.
  float sc_sum = 0.0f;
  uint16_t my_sc = 0;
  for (int j = 0; j < a.k; ++j) {
    uint32_t best = 0u;
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; ++i)
      if (i < nblk) best = max(best, key[i]);
    best = __ockl_wfred_max_u32(best);
    const uint32_t e = 0xffffu - (best & 0xffffu);
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; ++i)
      if (i < nblk && key[i] == best) key[i] = 0u;
    const uint16_t p = static_cast<uint16_t>(best >> 16);
    sc_sum += Act<F16>::ld(p);  // fp32, slot order
    if (lane == j) {
      my_sc = p;
      a.inds[static_cast<int64_t>(t) * a.k + j] = e;
    }
  }
  if (lane < a.k) {
    uint16_t out = my_sc;
    if (a.norm) {
      const double den = static_cast<double>(Act<F16>::rnd(sc_sum));
      out = Act<F16>::st(static_cast<float>(static_cast<double>(Act<F16>::ld(my_sc)) / den));
    }
    a.scores[static_cast<int64_t>(t) * a.k + lane] = out;
  }
  if (lane == 0 && a.wsg.w && a.sgate) a.sgate[t] = Act<F16>::sigmoid(Act<F16>::ld(lrow[E]));
}

// The Nemotron-H selection of token t (nh_select_wave) from the logits row
// in global memory, into inds and scores32.
__device__ void router_token_nh(const RouterArgs& a, int t, int lane) {
  nh_select_wave<kMaxExpertsPerLane>(a.logits + static_cast<int64_t>(t) * (a.E + 1), a.E, a.k, a.norm,
                                     a.n_group, a.topk_group, a.scaling, a.cbias, lane,
                                     a.inds + static_cast<int64_t>(t) * a.k,
                                     a.scores32 + static_cast<int64_t>(t) * a.k, nullptr);
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

// ------------------------------------------------------------------ router, many tokens
//
// Forwards of more than a few token tiles route in two kernels with no
// cross-workgroup handoff inside either:
//   logits_kernel  16 tokens x 16 columns x one of lg_split slices of H per
//                  workgroup on v_mfma_f64_16x16x4f64: the bf16 operands
//                  are exact in fp64 and so are their products; 8 waves
//                  take interleaved 32-element pieces of the slice and their
//                  partial tiles are added in wave order. One slice: the sum
//                  is rounded once to bf16 (then the logit bias, as in
//                  phase 1 of router_kernel); more: the fp64 partial sums go
//                  to lg_part (about 1024 workgroups instead of 128 at 512
//                  tokens x 61 columns)
//   topk_kernel    the logits from the partial sums (added in slice order,
//                  then rounded and biased as above), softmax and top-k, one
//                  wave per token
// The sort follows as its own launch.

constexpr int kLgWaves = 8;
constexpr int kLgThreads = kLgWaves * kWave;
constexpr int kLgBatch = 8;  // 16-byte chunks of x and w in flight per lane

typedef double f64x4_t __attribute__((ext_vector_type(4)));

template <bool F16>
__global__ __launch_bounds__(kLgThreads) void logits_kernel(RouterArgs a) {
  __shared__ double s_red[(kLgWaves - 1) * 4 * kWave];
  // the forward's fp16-range flag starts clear (topk_kernel and the gate/up
  // GEMMs, which run after this grid, set its bits)
  if (a.f16_flag && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x == 0) *a.f16_flag = 0u;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i16 = lane & 15, kk = lane >> 4;
  const int H = a.H, E = a.E;
  const int ncols = E + (a.wsg.w ? 1 : 0);
  const int t0 = blockIdx.y * 16, c0 = blockIdx.x * 16;
  // MFMA operands: lane (i16, kk) feeds token row i16 (A) and column i16 (B)
  // at k = 8 * chunk + m for the m-th of 8 MFMAs per 16-byte chunk
  const uint16_t* xrow = a.x + static_cast<int64_t>(min(t0 + i16, a.T - 1)) * H;
  const int col = min(c0 + i16, ncols - 1);
  const RouterRows& wrows = col < E ? a.wr : a.wsg;
  const int64_t wrow = col < E ? col : 0;
  const int nch = H / 8;
  f64x4_t acc0 = {0.0, 0.0, 0.0, 0.0}, acc1 = {0.0, 0.0, 0.0, 0.0};
  // steps of kLgStep chunks (one per lane); this workgroup's slice is steps
  // [s0, s1). kLgBatch steps' chunks are loaded together (one memory
  // latency per batch, not per chunk), then multiplied in chunk order.
  constexpr int kLgStep = 4 * kLgWaves;
  const int kn = max(a.lg_split, 1), ks = blockIdx.z;
  const int steps = (nch + kLgStep - 1) / kLgStep;
  const int s0 = (steps * ks) / kn, s1 = (steps * (ks + 1)) / kn;
  for (int st = s0; st < s1; st += kLgBatch) {
    const int nb = min(kLgBatch, s1 - st);  // workgroup-uniform
    u32x4_t xv[kLgBatch];
    RChunk wv[kLgBatch];
#pragma unroll
    for (int b = 0; b < kLgBatch; ++b) {
      if (b < nb) {
        const int ch = min((st + b) * kLgStep + 4 * wave + kk, nch - 1);
        xv[b] = *reinterpret_cast<const u32x4_t*>(xrow + ch * 8);
        wv[b] = load_rchunk<F16>(wrows, wrow, H, ch);
      }
    }
#pragma unroll
    for (int b = 0; b < kLgBatch; ++b) {
      if (b < nb) {
        if ((st + b) * kLgStep + 4 * wave + kk >= nch)  // chunks past H contribute exact zeros
          xv[b] = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const double x0 = Act<F16>::lo(xv[b][i]), x1 = Act<F16>::hi(xv[b][i]);
          const double w0 = wv[b].template get<F16>(2 * i), w1 = wv[b].template get<F16>(2 * i + 1);
          acc0 = __builtin_amdgcn_mfma_f64_16x16x4f64(x0, w0, acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f64_16x16x4f64(x1, w1, acc1, 0, 0, 0);
        }
      }
    }
  }
  f64x4_t acc = acc0 + acc1;
  if (wave > 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) s_red[((wave - 1) * 4 + r) * kWave + lane] = acc[r];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < kLgWaves - 1; ++w)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] += s_red[(w * 4 + r) * kWave + lane];
  // the f64 MFMA's result layout: lane (i16, kk) holds rows kk + 4 r
  // (tokens t0 + kk + 4 r) of column i16 (column c0 + i16)
  const int c = c0 + i16;
  if (c >= ncols) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = t0 + kk + 4 * r;
    if (t >= a.T) continue;
    if (kn > 1) {
      a.lg_part[(static_cast<int64_t>(ks) * a.T + t) * (E + 1) + c] = acc[r];
      continue;
    }
    uint16_t l = Act<F16>::from64(acc[r]);
    if (c < E && a.lbias)
      l = Act<F16>::from64(static_cast<double>(Act<F16>::ld(l)) + static_cast<double>(Act<F16>::ld(a.lbias[c])));
    a.logits[static_cast<int64_t>(t) * (E + 1) + c] = l;
  }
}

// Logit column c of token t from logits_kernel's output: the slices' fp64
// partial sums added in slice order, rounded once, then the logit bias (as
// router_logits); the rounded logit is also stored for the routing
// accessors. One slice: the logit logits_kernel rounded.
template <bool F16>
__device__ inline uint16_t split_logit(const RouterArgs& a, int t, int c) {
  const int ld = a.E + 1;
  const int64_t at = static_cast<int64_t>(t) * ld + c;
  if (a.lg_split <= 1) return a.logits[at];
  double v = a.lg_part[at];
  for (int ks = 1; ks < a.lg_split; ++ks) v += a.lg_part[(static_cast<int64_t>(ks) * a.T + t) * ld + c];
  uint16_t l = Act<F16>::from64(v);
  if (c < a.E && a.lbias)
    l = Act<F16>::from64(static_cast<double>(Act<F16>::ld(l)) + static_cast<double>(Act<F16>::ld(a.lbias[c])));
  a.logits[at] = l;
  return l;
}

// Softmax (fp64, exp_det) and top-k of token t by one wave, for
// topk_kernel: the steps of router_token, with lane l on the experts e = r +
// 64 i (i < NPER), r the 6-bit reverse of l, and the wave reductions as DPP
// trees (adjacent lanes first: with lanes on bit-reversed expert classes the
// normaliser's tree adds the partials r and r xor 32 first, r xor 16 next,
// .., the association of router_token's butterfly, w = 32, 16, .., 1).
template <int NPER, bool F16>
__device__ void topk_token(const RouterArgs& a, int t, int lane) {
  const int E = a.E;
  const int r = static_cast<int>(__builtin_bitreverse32(static_cast<uint32_t>(lane)) >> 26);
  float lf[NPER];
  float mf = -__builtin_huge_valf();
#pragma unroll
  for (int i = 0; i < NPER; ++i) {
    const int e = r + 64 * i;
    lf[i] = e < E ? Act<F16>::ld(split_logit<F16>(a, t, e)) : -__builtin_huge_valf();
    mf = fmaxf(mf, lf[i]);
  }
  // the shared expert's gate logit (column E)
  if (lane == 0 && a.wsg.w) {
    const uint16_t g = split_logit<F16>(a, t, E);
    if (a.sgate) a.sgate[t] = Act<F16>::sigmoid(Act<F16>::ld(g));
  }
  // bf16 (fp16) logits are exact in fp32: the fp32 maximum is the fp64 one
  const double m = static_cast<double>(wave_max_f32(mf));
  double ex[NPER], s = 0.0;
#pragma unroll
  for (int i = 0; i < NPER; ++i) {
    const int e = r + 64 * i;
    ex[i] = e < E ? exp_det(static_cast<double>(lf[i]) - m) : 0.0;
    s += ex[i];
  }
  s = wave_sum_f64(s);
  uint32_t key[NPER];
#pragma unroll
  for (int i = 0; i < NPER; ++i) {
    const int e = r + 64 * i;
    key[i] = 0u;
    if (e < E) {
      const uint16_t p = Act<F16>::from64(ex[i] / s);
      if (a.probs) a.probs[static_cast<int64_t>(t) * E + e] = p;
      // probabilities are >= 0: their patterns order like their values
      key[i] = (static_cast<uint32_t>(p) << 16) | (0xffffu - static_cast<uint32_t>(e));
    }
  }
  // k rounds of the largest key (prob desc, expert asc); slot j's key stays in lane j
  float sc_sum = 0.0f;
  uint32_t my_key = 0u;
  for (int j = 0; j < a.k; ++j) {
    uint32_t best = 0u;
#pragma unroll
    for (int i = 0; i < NPER; ++i) best = max(best, key[i]);
    best = wave_max_u32(best);
#pragma unroll
    for (int i = 0; i < NPER; ++i)
      if (key[i] == best) key[i] = 0u;
    sc_sum += Act<F16>::ld(static_cast<uint16_t>(best >> 16));  // fp32, slot order
    if (lane == j) my_key = best;
  }
  if (lane < a.k) {
    uint16_t sc = static_cast<uint16_t>(my_key >> 16);
    if (a.norm) {
      const double den = static_cast<double>(Act<F16>::rnd(sc_sum));
      sc = Act<F16>::st(static_cast<float>(static_cast<double>(Act<F16>::ld(sc)) / den));
    }
    a.inds[static_cast<int64_t>(t) * a.k + lane] = 0xffffu - (my_key & 0xffffu);
    a.scores[static_cast<int64_t>(t) * a.k + lane] = sc;
  }
}

// elements e0..e7 of a 16-byte chunk -> P8 slots 0,2,4,6 (e0..e3) and
// 1,3,5,7 (e4..e7)
__device__ inline u32x4_t p8_chunk(const u32x4_t& v) {
  u32x4_t p;
  p[0] = (v[0] & 0xffffu) | (v[2] << 16);
  p[1] = (v[0] >> 16) | (v[2] & 0xffff0000u);
  p[2] = (v[1] & 0xffffu) | (v[3] << 16);
  p[3] = (v[1] >> 16) | (v[3] & 0xffff0000u);
  return p;
}

// The token's row of x in fp16 (P8 layout) for the prefill GEMMs; a
// value outside fp16's range sets kF16FlagX. F16: x is fp16 already (the
// copy only permutes it).
template <bool F16>
__device__ void f16_row(const RouterArgs& a, int t, int lane) {
  const u32x4_t* src = reinterpret_cast<const u32x4_t*>(a.x + static_cast<int64_t>(t) * a.H);
  u32x4_t* dst = reinterpret_cast<u32x4_t*>(a.xh + static_cast<int64_t>(t) * a.H);
  if constexpr (F16) {
    for (int ch = lane; ch < a.H / 8; ch += kWave) dst[ch] = p8_chunk(src[ch]);
  } else {
    bool ovf = false;
    for (int ch = lane; ch < a.H / 8; ch += kWave) dst[ch] = bf16_chunk_to_f16_p8(src[ch], ovf);
    if (__ballot(ovf) && lane == 0) atomicOr(a.f16_flag, kF16FlagX);
  }
}

// NPER: experts per lane (E <= 64 NPER); mode 1 (Nemotron-H) takes its own
// selection on rounded logits (no slices)
template <int NPER, bool F16>
__global__ __launch_bounds__(kRouterThreads) void topk_kernel(RouterArgs a) {
  const int t = blockIdx.x * kRouterWaves + (threadIdx.x >> 6);
  if (t >= a.T) return;
  if (a.mode == 1)
    router_token_nh(a, t, threadIdx.x & 63);
  else
    topk_token<NPER, F16>(a, t, threadIdx.x & 63);
  if (a.xh) f16_row<F16>(a, t, threadIdx.x & 63);
}

template <int NPER>
static void launch_topk(const RouterArgs& a, hipStream_t stream) {
  const dim3 grid((a.T + kRouterWaves - 1) / kRouterWaves), block(kRouterThreads);
  if (a.f16)
    hipLaunchKernelGGL((topk_kernel<NPER, true>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((topk_kernel<NPER, false>), grid, block, 0, stream, a);
}

int router_lg_split(int64_t T, int64_t E, int64_t cap) {
  const int64_t tiles = ((E + 1 + 15) / 16) * ((T + 15) / 16);
  int64_t s = std::min<int64_t>(4, std::max<int64_t>(1, 1024 / std::max<int64_t>(tiles, 1)));
  while (s > 1 && s * T * (E + 1) > std::min(kLgPartMax, cap)) --s;
  return static_cast<int>(s);
}

hipError_t launch_router_many(const RouterArgs& a, hipStream_t stream) {
  const int ncols = a.E + (a.wsg.w ? 1 : 0);
  const int kn = a.mode == 1 ? 1 : std::max(a.lg_split, 1);
  if (kn > 1 && (kn > 4 || !a.lg_part || static_cast<int64_t>(kn) * a.T * (a.E + 1) > kLgPartMax))
    return hipErrorInvalidValue;
  RouterArgs b = a;
  b.lg_split = kn;
  hipLaunchKernelGGL((a.f16 ? logits_kernel<true> : logits_kernel<false>),
                     dim3((ncols + 15) / 16, (a.T + 15) / 16, kn), dim3(kLgThreads), 0, stream, b);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  if (a.E <= 64)
    launch_topk<1>(b, stream);
  else if (a.E <= 128)
    launch_topk<2>(b, stream);
  else if (a.E <= 256)
    launch_topk<4>(b, stream);
  else if (a.E <= 512)
    launch_topk<8>(b, stream);
  else
    launch_topk<16>(b, stream);
  return hipGetLastError();
}

template <bool F16>
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
    router_logits<kRouterTok, 4, F16>(a, ct, tt, wave, lane);
  else if (a.T == 1)
    router_logits<1, 1, F16>(a, ct, tt, wave, lane);
  else
    router_logits<kRouterTok, 1, F16>(a, ct, tt, wave, lane);
  // P8 copy of the tile's x rows, once per token tile
  if (ct == 0 && a.xp) {
    const int oct = H / 8;
    for (int o = tid; o < kRouterTok * oct; o += kRouterThreads) {
      const int tl = o / oct, oc = o % oct;
      const int tok = tt * kRouterTok + tl;
      if (tok >= a.T) continue;
      const u32x4_t v =
          *reinterpret_cast<const u32x4_t*>(a.x + static_cast<int64_t>(tok) * H + oc * 8);
      *reinterpret_cast<u32x4_t*>(a.xp + static_cast<int64_t>(tok) * H + oc * 8) = p8_chunk(v);
    }
  }
  // fp16 copy (P8 layout) of the tile's x rows for the prefill GEMMs, once
  // per token tile; a value outside fp16's range sets kF16FlagX (the flag
  // is zero on entry: the caller's forward clears it after its GEMMs)
  if (ct == 0 && a.xh) {
    for (int tl = wave; tl < kRouterTok; tl += kRouterWaves) {
      const int tok = tt * kRouterTok + tl;
      if (tok < a.T) f16_row<F16>(a, tok, lane);
    }
  }
  if (!arrive_last(&a.counters[tt], static_cast<uint32_t>(a.n_ct), &s_flag)) return;

  // ---- phase 2 (last column tile of this token tile): softmax and top-k
  // (mode 1: the Nemotron-H selection)
  for (int tl = wave; tl < kRouterTok; tl += kRouterWaves) {
    const int t = tt * kRouterTok + tl;
    if (t >= a.T) continue;
    if (a.mode == 1)
      router_token_nh(a, t, lane);
    else
      router_token<F16>(a, t, lane);
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
  hipLaunchKernelGGL((a.f16 ? router_kernel<true> : router_kernel<false>), dim3(a.n_ct, a.n_tt), dim3(kRouterThreads),
                     0, stream, a);
  return hipGetLastError();
}

}  // namespace fmx
