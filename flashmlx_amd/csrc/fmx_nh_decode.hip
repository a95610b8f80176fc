// fmx_nh_decode.hip -- the Nemotron-H MoE block for decode batches (T <= 16
// tokens) on packed weights, in four launches:
//
//   D1  router columns, one workgroup per expert: fp64-exact logits; the
//       last column to finish selects (sigmoid, correction bias, group
//       limit, top-k, fp32 scores) and builds the routing tables
//       |  the shared expert's up tiles + relu^2 (routing-independent,
//       streaming meanwhile)
//   D2  the routed fc1 tiles + relu^2, one or two 16-row tiles per workgroup
//   D3  fc2 of every selected expert (64 columns and one K half per
//       workgroup) and the shared down projection in K slices, fp32
//       products; the last contributor of each 64-column block forms its
//       fp32 weighted sum and the shared add, rounded once to bf16
//
// Reference: server/src/nemotron_h.cpp:1010-1111 (moe_block), :54-63 (relu2).
//
// Each tile workgroup splits K over its four waves with every load of a
// wave's quarter in flight at once (decode is bound by the weight bytes);
// tile rows are indexed by token, so the tokens that selected an expert
// are multiplied in place and no gather or sort is needed. relu^2 of the
// bf16 fc1 output (at most 16 significant bits) is kept exactly as the sum
// of two bf16 values hi + lo, and fc2 multiplies both: the down products see
// the fp32 relu^2 of the reference (whose fp32 0 in relu2 promotes), with
// the weights dequantised exactly (s * P + (b - 128 s) * X per group).
#include <algorithm>

#include "fmx_dev.hpp"

namespace fmx {

namespace {

constexpr int kNhDnTiles = 4;     // 16-row tiles of H per D3 workgroup (one per wave)
constexpr int kNhDnSplit = 2;     // K halves of a routed fc2 tile (d, d2)
constexpr int kNhDnUnits = 8;     // D3's load ring: 128-k units per wave (a routed fc2 K half)
constexpr int kNhSdUnits = 8;     // the same for a shared down K slice
constexpr int kNhD2PairGrid = 2048;  // D2 runs two tiles per workgroup from this many tiles

// relu(bf16(acc))^2 as hi + lo bf16: v^2 of a bf16 v has at most 16
// significant bits, so hi = bf16(v^2) and lo = v^2 - hi are both exact
__device__ inline void relu2_split(float acc, uint16_t& hi, uint16_t& lo) {
  const float v = fmaxf(round_bf16(acc), 0.0f);
  const float sq = v * v;
  hi = f32_to_bf16(sq);
  lo = f32_to_bf16(sq - bf16_to_f32(hi));
}

// ---------------------------------------------------------------- D1

// The last router workgroup: every token's selection and the routing tables
// (seg: the selected experts ascending; slots: each expert's token -> slot
// byte row). s_lg reuses the x staging area: [T][E] logits.
template <int NPER>
__device__ void d1_finish(const NhDecArgs& a, uint16_t* s_lg) {
  __shared__ uint32_t s_inds[kDecMaxT * kDecMaxK];
  __shared__ uint32_t s_seg[kNhDecMaxE + 1];
  __shared__ uint16_t s_segof[kNhDecMaxE];
  __shared__ uint8_t s_used[kNhDecMaxE];
  __shared__ uint8_t s_slot[kNhDecMaxE * kDecMaxT];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int T = a.T, E = a.E, k = a.k, n = T * k;
  // the logits (device-scope loads: the other workgroups' device-scope
  // stores completed before their arrivals were counted)
  for (int i = tid; i < E * T; i += kDecThreads) {
    const int c = i / T, t = i - c * T;
    const uint16_t v = static_cast<uint16_t>(__hip_atomic_load(a.lgw + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    s_lg[t * E + c] = v;
    a.logits[static_cast<int64_t>(t) * (E + 1) + c] = v;
  }
  for (int e = tid; e < E; e += kDecThreads) s_used[e] = 0;
  __syncthreads();
  for (int t = wave; t < T; t += kDecWaves)
    nh_select_wave<NPER>(s_lg + t * E, E, k, a.norm, a.n_group, a.topk_group, a.scaling, a.cbias, lane,
                         a.inds + t * k, a.scores + t * k, s_inds + t * k);
  __syncthreads();
  for (int i = tid; i < n; i += kDecThreads) s_used[s_inds[i]] = 1;
  __syncthreads();
  if (wave == 0) {
    uint32_t U = 0;
    for (int e0 = 0; e0 < E; e0 += kWave) {
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
  for (int i = tid; i < E * kDecMaxT; i += kDecThreads) s_slot[i] = 0xff;
  __syncthreads();
  const int U = static_cast<int>(s_seg[0]);
  for (int i = tid; i <= U; i += kDecThreads) a.seg[i] = s_seg[i];
  for (int i = tid; i < n; i += kDecThreads)
    s_slot[s_segof[s_inds[i]] * kDecMaxT + i / k] = static_cast<uint8_t>(i % k);
  __syncthreads();
  for (int i = tid; i < U * (kDecMaxT / 4); i += kDecThreads)
    reinterpret_cast<uint32_t*>(a.slots)[i] = reinterpret_cast<const uint32_t*>(s_slot)[i];
}

// Router column c for every token (nemotron_h.cpp:1018): x . w_c in fp64
// (products of bf16 values are exact, and so is their sum far below the bf16
// step, in any order), rounded once to bf16. Thread i takes the 16-byte
// chunks i and i + 256 of H; the waves' partial sums meet in a
// reduce-scatter and then in LDS; wave 0 stores the column with device-scope
// stores and counts the workgroup in; the last one selects.
template <int NPER>
__device__ void d1_router(const NhDecArgs& a, int c, uint8_t* smem) {
  __shared__ int s_last;
  __shared__ double s_lp[kDecWaves * kDecMaxT];
  uint16_t* s_x = reinterpret_cast<uint16_t*>(smem);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = a.H, T = a.T, E = a.E, xs = xstride(H), nch = H / 8;
  dma_rows(a.x, H, T, H, s_x, xs, wave, kDecWaves, lane);
  const bool has0 = tid < nch, has1 = tid + kDecThreads < nch;
  const uint16_t* wrow = a.gate_w + static_cast<int64_t>(c) * H;
  const u32x4_t w0 = *reinterpret_cast<const u32x4_t*>(wrow + min(tid, nch - 1) * 8);
  const u32x4_t w1 = *reinterpret_cast<const u32x4_t*>(wrow + min(tid + kDecThreads, nch - 1) * 8);
  wait_vmcnt0();
  lds_dma_barrier();
  double part[kDecMaxT];
#pragma unroll
  for (int t = 0; t < kDecMaxT; ++t) {
    part[t] = 0.0;
    if (t < T) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (h == 0 ? has0 : has1) {
          const u32x4_t wv = h == 0 ? w0 : w1;
          const int ch = tid + h * kDecThreads;
          const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(s_x + t * xs + ch * 8);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            part[t] = __builtin_fma(static_cast<double>(__uint_as_float(xv[q] << 16)),
                                    static_cast<double>(__uint_as_float(wv[q] << 16)), part[t]);
            part[t] = __builtin_fma(static_cast<double>(__uint_as_float(xv[q] & 0xffff0000u)),
                                    static_cast<double>(__uint_as_float(wv[q] & 0xffff0000u)), part[t]);
          }
        }
      }
    }
  }
  // lane 4t + 3 then holds the wave's total of token t
  const double r = reduce_scatter64<kDecMaxT>(part, lane);
  if (rs64_holder<kDecMaxT>(lane)) s_lp[wave * kDecMaxT + (lane >> 2)] = r;
  __syncthreads();
  if (wave == 0) {
    if (tid < T) {
      double v = 0.0;
#pragma unroll
      for (int q = 0; q < kDecWaves; ++q) v += s_lp[q * kDecMaxT + tid];
      __hip_atomic_store(a.lgw + c * T + tid, static_cast<uint32_t>(f64_to_bf16(v)), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    wait_vmcnt0();
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               static_cast<uint32_t>(E - 1);
  }
  __syncthreads();
  if (!s_last) return;
  d1_finish<NPER>(a, s_x);
  if (tid == 0) *a.counter = 0u;  // every column has arrived
}

// The shared expert's up tile tp (nemotron_h.cpp:1102-1104): hs[t, n] =
// relu(bf16(x_t . Wsu[n]))^2 as hi + lo, every token; wave q multiplies K
// quarter q.
template <int NU>
__device__ void d1_shared_up(const NhDecArgs& a, int tp, uint8_t* smem) {
  float* s_red = reinterpret_cast<float*>(smem);
  uint16_t* s_x = reinterpret_cast<uint16_t*>(smem + kDecQuadRedBytes);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = a.H, T = a.T, xs = xstride(H), nu = H / 128;
  const int u0 = (nu * wave) / kDecWaves, u1 = (nu * (wave + 1)) / kDecWaves;
  const int m = lane & 15, j = lane >> 4;
  const uint16_t* xl = s_x + min(m, T - 1) * xs + 8 * j;
  f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
  dma_rows(a.x, H, T, H, s_x, xs, wave, kDecWaves, lane);
  tile_units_lds<false, NU>(a.sup + static_cast<int64_t>(tp) * nu * kBlockSingle, u0, u1, xl, lane, acc0, acc1);
  quad_reduce(acc0, acc1, wave, lane, s_red);
  if (wave != 0) return;
  const int n = tp * 16 + m;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 4 * j + i;
    if (t < T) {
      uint16_t hi, lo;
      relu2_split(acc0[i], hi, lo);
      a.hs_hi[static_cast<int64_t>(t) * a.Isp + n] = hi;
      a.hs_lo[static_cast<int64_t>(t) * a.Isp + n] = lo;
    }
  }
}

// Workgroups [0, E): router columns; [E, E + n_sup): shared up tiles.
template <int NPER, int NU>
__global__ __launch_bounds__(kDecThreads) void nh_d1(NhDecArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int w = blockIdx.x;
  if (w < a.E)
    d1_router<NPER>(a, w, smem);
  else
    d1_shared_up<NU>(a, w - a.E, smem);
}

// ---------------------------------------------------------------- D2

// Tiles NT tp .. NT tp + NT - 1 (fc1 rows 16 tp ..) of selected expert
// number u (nemotron_h.cpp:1086-1090): h[t*k + slot, n] = relu(bf16(x_t .
// W1_e[n]))^2 for the tokens t whose slot `slot` selected expert e. Two tiles
// per workgroup (large grids) share the routing-table reads and the staged
// rows and put both tiles' loads in flight together.
template <int NU, int NT>
__global__ __launch_bounds__(kDecThreads) void nh_d2(NhDecArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  float* s_red = reinterpret_cast<float*>(smem);
  uint16_t* s_x = reinterpret_cast<uint16_t*>(smem + kDecQuadRedBytes);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int T = a.T, k = a.k, H = a.H, Ip = a.Ip, xs = xstride(H);
  const int ntile = Ip / 16, ngrp = (ntile + NT - 1) / NT;
  const int u = static_cast<int>(blockIdx.x) / ngrp, tp = (static_cast<int>(blockIdx.x) - u * ngrp) * NT;
  const int U = static_cast<int>(min(a.seg[0], static_cast<uint32_t>(a.max_seg)));
  if (u >= U) return;  // workgroup-uniform
  const int e = static_cast<int>(min(a.seg[1 + u], static_cast<uint32_t>(a.E - 1)));
  const uint32_t* srow = reinterpret_cast<const uint32_t*>(a.slots + u * kDecMaxT);
  const uint32_t slot4 = srow[lane & 3];  // slots of tokens 4*(lane&3) .. +3
  // the activation rows of the tokens that selected e -> LDS rows t; the
  // other rows stay unset and their products land in rows never stored
  for (int t = wave; t < T; t += kDecWaves) {
    const uint32_t slot = (__shfl(slot4, t >> 2) >> (8 * (t & 3))) & 0xffu;
    if (slot < static_cast<uint32_t>(k)) dma_row(a.x + static_cast<int64_t>(t) * H, H, s_x + t * xs, lane);
  }
  const int nu = H / 128;
  const int u0 = (nu * wave) / kDecWaves, u1 = (nu * (wave + 1)) / kDecWaves;
  const int m = lane & 15, j = lane >> 4;
  const uint16_t* xl = s_x + min(m, T - 1) * xs + 8 * j;
  const uint8_t* eb = a.fc1 + static_cast<int64_t>(e) * a.fc1_es;
  f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;  // tile tp (and tp + 1)
  if constexpr (NT == 1) {
    tile_units_lds<false, NU>(eb + static_cast<int64_t>(tp) * nu * kBlockSingle, u0, u1, xl, lane, acc0, acc1);
  } else {
    // both tiles' units in flight, then the rows' DMA proven complete by
    // their count (the DMA was issued before them)
    PkUnit<false> L0[NU], L1[NU];
    const uint8_t* b0 = eb + static_cast<int64_t>(tp) * nu * kBlockSingle;
    const uint8_t* b1 = eb + static_cast<int64_t>(min(tp + 1, ntile - 1)) * nu * kBlockSingle;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int d = 0; d < NU; ++d) L0[d] = pk_load<false>(b0 + min(u0 + d, u1 - 1) * kBlockSingle, lane);
#pragma unroll
    for (int d = 0; d < NU; ++d) L1[d] = pk_load<false>(b1 + min(u0 + d, u1 - 1) * kBlockSingle, lane);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<2 * NU * pk_load_insts<false>()>();
    lds_dma_barrier();
    f32x4_t unused = acc0;
#pragma unroll
    for (int d = 0; d < NU; ++d) {
      if (u0 + d < u1) {
        bf16x8_t A[4];
        lds_a(xl + (u0 + d) * 128, A);
        pk_unit<false>(L0[d], A, acc0, unused);
        pk_unit<false>(L1[d], A, acc1, unused);
      }
    }
  }
  quad_reduce(acc0, acc1, wave, lane, s_red);
  if (wave != 0) return;
  const uint32_t my_slots = __shfl(slot4, j);  // rows 4j .. 4j + 3
#pragma unroll
  for (int q = 0; q < NT; ++q) {
    if (tp + q >= ntile) continue;
    const f32x4_t& acc = q ? acc1 : acc0;
    const int n = (tp + q) * 16 + m;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 4 * j + i;
      const uint32_t slot = (my_slots >> (8 * i)) & 0xffu;
      if (t < T && slot < static_cast<uint32_t>(k)) {
        uint16_t hi, lo;
        relu2_split(acc[i], hi, lo);
        const int64_t o = static_cast<int64_t>(t * k + slot) * Ip + n;
        a.h_hi[o] = hi;
        a.h_lo[o] = lo;
      }
    }
  }
}

// ---------------------------------------------------------------- D3

// nu units of one 16-row tile (blocks from tb) against hi and lo rows in LDS:
// every unit's loads are issued before the rows' DMA (issued by the caller
// in `stage`), then one wait.
template <int NU, typename Stage>
__device__ inline f32x4_t d3_tile(const uint8_t* tb, int nu, const uint16_t* xl_hi, const uint16_t* xl_lo,
                                  int lane, Stage stage) {
  PkUnit<false> L[NU];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int d = 0; d < NU; ++d) L[d] = pk_load<false>(tb + min(d, nu - 1) * kBlockSingle, lane);
  __builtin_amdgcn_sched_barrier(0);
  stage();
  wait_vmcnt0();
  lds_dma_barrier();
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f}, unused = acc;
#pragma unroll
  for (int d = 0; d < NU; ++d) {
    if (d < nu) {
      bf16x8_t A[4];
      lds_a(xl_hi + d * 128, A);
      pk_unit<false>(L[d], A, acc, unused);
      lds_a(xl_lo + d * 128, A);
      pk_unit<false>(L[d], A, acc, unused);
    }
  }
  return acc;
}

// The weighted sum of column block cb (columns 64 cb .. 64 cb + 63) for
// every token (nemotron_h.cpp:1096-1108): y = bf16(bf16(sum over slots of
// (d + d2) * score) + shared), products and sums fp32, each rounded on its
// own, slots in order, the shared expert's K slices added in order first.
// The products were stored device-scope by the block's contributors in this
// grid and are read with device-scope loads.
// a pair of fp32 values by one device-scope 8-byte load
__device__ inline void load2_dev(const float* p, float& lo, float& hi) {
  const uint64_t v = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  lo = __uint_as_float(static_cast<uint32_t>(v));
  hi = __uint_as_float(static_cast<uint32_t>(v >> 32));
}

__device__ void nh_combine_block(const NhDecArgs& a, int cb) {
  const int T = a.T, k = a.k, H = a.H;
  for (int g = threadIdx.x; g < T * 16; g += kDecThreads) {
    const int t = g >> 4, c = cb * 64 + 4 * (g & 15);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < k; ++j) {
      const float s = a.scores[t * k + j];
      const int64_t off = static_cast<int64_t>(t * k + j) * H + c;
      float v0[4], v1[4];
      load2_dev(a.d + off, v0[0], v0[1]);
      load2_dev(a.d + off + 2, v0[2], v0[3]);
      load2_dev(a.d2 + off, v1[0], v1[1]);
      load2_dev(a.d2 + off + 2, v1[2], v1[3]);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = __fadd_rn(acc[i], __fmul_rn(__fadd_rn(v0[i], v1[i]), s));
    }
    float out[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = round_bf16(acc[i]);
    if (a.Isp > 0) {
      float sd[4];
      load2_dev(a.sd_part + static_cast<int64_t>(t) * H + c, sd[0], sd[1]);
      load2_dev(a.sd_part + static_cast<int64_t>(t) * H + c + 2, sd[2], sd[3]);
      for (int ks = 1; ks < kNhDecSdSplit; ++ks) {
        float p[4];
        const float* src = a.sd_part + (static_cast<int64_t>(ks) * T + t) * H + c;
        load2_dev(src, p[0], p[1]);
        load2_dev(src + 2, p[2], p[3]);
#pragma unroll
        for (int i = 0; i < 4; ++i) sd[i] = __fadd_rn(sd[i], p[i]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) out[i] = __fadd_rn(out[i], sd[i]);
    }
    u32x2_t w;
    w[0] = static_cast<uint32_t>(f32_to_bf16(out[0])) | (static_cast<uint32_t>(f32_to_bf16(out[1])) << 16);
    w[1] = static_cast<uint32_t>(f32_to_bf16(out[2])) | (static_cast<uint32_t>(f32_to_bf16(out[3])) << 16);
    *reinterpret_cast<u32x2_t*>(a.y + static_cast<int64_t>(t) * H + c) = w;
  }
}

// Counts a D3 workgroup's outputs for column block cb in, once every wave's
// device-scope stores have completed; the last of the block's contributors
// (the K halves of its U selected experts and the shared expert's K
// slices) forms the block's sum and resets the count.
__device__ void nh_arrive(const NhDecArgs& a, int cb, int U) {
  __shared__ int s_last_cb;
  wait_vmcnt0();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t target = static_cast<uint32_t>(U * kNhDnSplit + (a.Isp > 0 ? kNhDecSdSplit : 0));
    s_last_cb = __hip_atomic_fetch_add(a.cb_counter + cb * kDecCbStride, 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT) == target - 1;
  }
  __syncthreads();
  if (!s_last_cb) return;
  nh_combine_block(a, cb);
  if (threadIdx.x == 0)
    __hip_atomic_store(a.cb_counter + cb * kDecCbStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Selected expert number u, columns 64 cb .. 64 cb + 63 of H, one 16-row
// tile per wave over K half ks of Ip (nemotron_h.cpp:1091-1094):
// d[t*k + slot, n] (ks 0) or d2[..] (ks 1) = h[t*k + slot] . W2_e[n] over
// the half, fp32. Halves keep a workgroup's staged rows (hi and lo) to half
// of Ip, so that more workgroups share a CU.
__device__ void d3_routed(const NhDecArgs& a, int u, int cb, int ks, uint8_t* smem) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int T = a.T, k = a.k, H = a.H, Ip = a.Ip;
  const int U = static_cast<int>(min(a.seg[0], static_cast<uint32_t>(a.max_seg)));
  if (u >= U) return;  // workgroup-uniform
  const int e = static_cast<int>(min(a.seg[1 + u], static_cast<uint32_t>(a.E - 1)));
  const uint32_t* srow = reinterpret_cast<const uint32_t*>(a.slots + u * kDecMaxT);
  const uint32_t slot4 = srow[lane & 3];
  const int nu_all = Ip / 128;
  const int ub = (nu_all * ks) / kNhDnSplit, ue = (nu_all * (ks + 1)) / kNhDnSplit, nu = ue - ub;
  const int kk = nu * 128, xs = xstride(kk);
  uint16_t* s_hi = reinterpret_cast<uint16_t*>(smem);
  uint16_t* s_lo = s_hi + T * xs;
  const int tile = kNhDnTiles * cb + wave;
  const uint8_t* tb =
      a.fc2 + static_cast<int64_t>(e) * a.fc2_es + (static_cast<int64_t>(tile) * nu_all + ub) * kBlockSingle;
  const int m = lane & 15, j = lane >> 4;
  const int r = min(m, T - 1);
  const f32x4_t acc = d3_tile<kNhDnUnits>(tb, nu, s_hi + r * xs + 8 * j, s_lo + r * xs + 8 * j, lane, [&]() {
    for (int t = wave; t < T; t += kDecWaves) {
      const uint32_t slot = (__shfl(slot4, t >> 2) >> (8 * (t & 3))) & 0xffu;
      if (slot < static_cast<uint32_t>(k)) {
        const int64_t o = static_cast<int64_t>(t * k + slot) * Ip + ub * 128;
        dma_row(a.h_hi + o, kk, s_hi + t * xs, lane);
        dma_row(a.h_lo + o, kk, s_lo + t * xs, lane);
      }
    }
  });
  uint32_t* const dst = reinterpret_cast<uint32_t*>(ks ? a.d2 : a.d);
  const uint32_t my_slots = __shfl(slot4, j);
  const int n = tile * 16 + m;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 4 * j + i;
    const uint32_t slot = (my_slots >> (8 * i)) & 0xffu;
    if (t < T && slot < static_cast<uint32_t>(k))
      __hip_atomic_store(dst + static_cast<int64_t>(t * k + slot) * H + n, __float_as_uint(acc[i]),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  nh_arrive(a, cb, U);
}

// The shared down projection, columns 64 cb .. +63, K slice ks of
// kNhDecSdSplit (nemotron_h.cpp:1105-1106): fp32 sums sd_part[ks][t][n].
__device__ void d3_shared(const NhDecArgs& a, int cb, int ks, uint8_t* smem) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int T = a.T, H = a.H, Isp = a.Isp;
  const int nu_all = Isp / 128;
  const int ub = (nu_all * ks) / kNhDecSdSplit, ue = (nu_all * (ks + 1)) / kNhDecSdSplit, nu = ue - ub;
  const int kk = nu * 128, xs = xstride(kk);
  uint16_t* s_hi = reinterpret_cast<uint16_t*>(smem);
  uint16_t* s_lo = s_hi + T * xs;
  const int tile = kNhDnTiles * cb + wave;
  const uint8_t* tb = a.sdn + (static_cast<int64_t>(tile) * nu_all + ub) * kBlockSingle;
  const int m = lane & 15, j = lane >> 4;
  const int r = min(m, T - 1);
  const f32x4_t acc = d3_tile<kNhSdUnits>(tb, nu, s_hi + r * xs + 8 * j, s_lo + r * xs + 8 * j, lane, [&]() {
    for (int t = wave; t < T; t += kDecWaves) {
      dma_row(a.hs_hi + static_cast<int64_t>(t) * Isp + ub * 128, kk, s_hi + t * xs, lane);
      dma_row(a.hs_lo + static_cast<int64_t>(t) * Isp + ub * 128, kk, s_lo + t * xs, lane);
    }
  });
  const int n = tile * 16 + m;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 4 * j + i;
    if (t < T)
      __hip_atomic_store(reinterpret_cast<uint32_t*>(a.sd_part) + (static_cast<int64_t>(ks) * T + t) * H + n,
                         __float_as_uint(acc[i]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  nh_arrive(a, cb, static_cast<int>(min(a.seg[0], static_cast<uint32_t>(a.max_seg))));
}

// Workgroups [0, max_seg * H/64 * 2): routed fc2 (the two K halves of a
// column block adjacent); then the shared down slices.
__global__ __launch_bounds__(kDecThreads) void nh_d3(NhDecArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int ncb = a.H / (16 * kNhDnTiles);
  const int b = blockIdx.x, nr = a.max_seg * ncb * kNhDnSplit;
  if (b < nr)
    d3_routed(a, b / (ncb * kNhDnSplit), (b / kNhDnSplit) % ncb, b % kNhDnSplit, smem);
  else
    d3_shared(a, (b - nr) / kNhDecSdSplit, (b - nr) % kNhDecSdSplit, smem);
}

// ---------------------------------------------------------------- host side

size_t d1_lds(const NhDecArgs& a) {
  return static_cast<size_t>(kDecQuadRedBytes) + static_cast<size_t>(a.T) * xstride(a.H) * 2;
}
size_t d2_lds(const NhDecArgs& a) { return d1_lds(a); }
size_t d3_lds(const NhDecArgs& a) {
  const int nu_r = a.Ip / 128, nu_s = a.Isp / 128;
  const int kk_r = ((nu_r + kNhDnSplit - 1) / kNhDnSplit) * 128;
  const int kk_s = ((nu_s + kNhDecSdSplit - 1) / kNhDecSdSplit) * 128;
  return static_cast<size_t>(2) * a.T * xstride(std::max(kk_r, kk_s)) * 2;
}
// units per wave of a D1 / D2 tile (K = H split in four)
int d12_units(const NhDecArgs& a) { return (a.H / 128 + kDecWaves - 1) / kDecWaves; }

template <int NPER>
void launch_d1(const NhDecArgs& a, hipStream_t stream) {
  const dim3 grid(a.E + a.n_sup), block(kDecThreads);
  const int nu = d12_units(a);
  if (nu <= 4)
    hipLaunchKernelGGL((nh_d1<NPER, 4>), grid, block, d1_lds(a), stream, a);
  else if (nu <= 6)
    hipLaunchKernelGGL((nh_d1<NPER, 6>), grid, block, d1_lds(a), stream, a);
  else
    hipLaunchKernelGGL((nh_d1<NPER, 8>), grid, block, d1_lds(a), stream, a);
}

}  // namespace

bool nh_decode_plan(NhDecArgs& a) {
  const int nu_s = a.Isp / 128;
  if (a.T < 1 || a.T > kDecMaxT || a.k < 1 || a.k > kDecMaxK || a.E < 1 || a.E > kNhDecMaxE || a.E > a.H ||
      a.H % 128 || a.H < 512 || a.H / 8 > 2 * kDecThreads || d12_units(a) > 8 || a.Ip % 128 ||
      a.Ip / 128 < kNhDnSplit || (a.Ip / 128 + kNhDnSplit - 1) / kNhDnSplit > kNhDnUnits ||
      a.H % (16 * kNhDnTiles) || a.Isp % 128 ||
      (a.Isp > 0 && (nu_s < kNhDecSdSplit || (nu_s + kNhDecSdSplit - 1) / kNhDecSdSplit > kNhSdUnits)) ||
      a.n_group > kWave || a.H / 64 > kNhDecMaxColBlocks)
    return false;
  a.max_seg = std::min(a.E, a.T * a.k);
  a.n_sup = a.Isp / 16;
  return d1_lds(a) + 16 * 1024 <= 160 * 1024 && d3_lds(a) <= 160 * 1024;
}

hipError_t launch_nh_decode(const NhDecArgs& a, hipStream_t stream, void* const* marks, int n_stages) {
  if (!a.cb_counter || !a.counter) return hipErrorInvalidValue;
  auto mark = [&](int i) -> hipError_t {
    return marks ? hipEventRecord(static_cast<hipEvent_t>(marks[i]), stream) : hipSuccess;
  };
  hipError_t err;
  if ((err = mark(0)) != hipSuccess) return err;
  if (a.E <= 64)
    launch_d1<1>(a, stream);
  else if (a.E <= 128)
    launch_d1<2>(a, stream);
  else if (a.E <= 256)
    launch_d1<4>(a, stream);
  else
    launch_d1<8>(a, stream);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  if ((err = mark(1)) != hipSuccess) return err;
  if (n_stages < 2) return hipSuccess;
  {
    const int ntile = a.Ip / 16;
    const bool two = a.max_seg * ntile >= kNhD2PairGrid;
    const dim3 grid(a.max_seg * (two ? (ntile + 1) / 2 : ntile)), block(kDecThreads);
    const int nu = d12_units(a);
    if (two) {
      if (nu <= 4)
        hipLaunchKernelGGL((nh_d2<4, 2>), grid, block, d2_lds(a), stream, a);
      else if (nu <= 6)
        hipLaunchKernelGGL((nh_d2<6, 2>), grid, block, d2_lds(a), stream, a);
      else
        hipLaunchKernelGGL((nh_d2<8, 2>), grid, block, d2_lds(a), stream, a);
    } else {
      if (nu <= 4)
        hipLaunchKernelGGL((nh_d2<4, 1>), grid, block, d2_lds(a), stream, a);
      else if (nu <= 6)
        hipLaunchKernelGGL((nh_d2<6, 1>), grid, block, d2_lds(a), stream, a);
      else
        hipLaunchKernelGGL((nh_d2<8, 1>), grid, block, d2_lds(a), stream, a);
    }
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  if ((err = mark(2)) != hipSuccess) return err;
  if (n_stages < 3) return hipSuccess;
  {
    const int ncb = a.H / (16 * kNhDnTiles);
    const int n = a.max_seg * ncb * kNhDnSplit + (a.Isp > 0 ? ncb * kNhDecSdSplit : 0);
    hipLaunchKernelGGL(nh_d3, dim3(n), dim3(kDecThreads), d3_lds(a), stream, a);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  // D3's last contributors have combined: the combine stage ends with it
  if ((err = mark(3)) != hipSuccess) return err;
  return mark(4);
}

}  // namespace fmx
