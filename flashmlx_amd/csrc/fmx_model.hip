// fmx_model.hip -- the decoder stack around the MoE block: embedding, RMSNorm
// (with the residual add), the attention projections for decode batches,
// RoPE with the KV-cache write, scaled dot-product attention and greedy
// token selection.
//
// Reference: server/src/model.cpp:486-497 (rms_norm, embed), :843-889
// (attention: q/k/v linears with biases, RoPE, cache concatenation, SDPA,
// o_proj), :891-911 (transformer_block), :1021-1033 (forward), :499-521
// (lm_head). The projections of more than 16 rows run on the prefill GEMM
// grid (fmx_prefill.hip); the MoE block is fmx_moe_block_forward.
#include <algorithm>

#include "fmx_dev.hpp"
#include "fmx_model_kernels.hpp"

namespace fmx {

namespace {

// ------------------------------------------------------------------ embedding

// Row ids[t] of the bf16 table (ids outside [0, V) take the nearest row);
// block 0 also clears the forward's fp16-range flag words.
__global__ __launch_bounds__(256) void embed_kernel(EmbedArgs a) {
  const int t = blockIdx.x;
  if (t == 0)
    for (int i = threadIdx.x; i < a.n_flags; i += blockDim.x) a.flags[i] = 0u;
  int64_t id = a.ids[t];
  id = id < 0 ? 0 : (id >= a.V ? a.V - 1 : id);
  const u32x4_t* src = reinterpret_cast<const u32x4_t*>(a.table + id * a.H);
  u32x4_t* dst = reinterpret_cast<u32x4_t*>(a.h + static_cast<int64_t>(t) * a.H);
  for (int c = threadIdx.x; c < a.H / 8; c += blockDim.x) dst[c] = src[c];
}

// ------------------------------------------------------------------ RMSNorm

// One workgroup per output row i (input row i * row_mul + row_add): optionally
// x = bf16(x + delta) first (written back: the residual stream), then the
// norm above. outh, when given, receives out in fp16 (P8 layout) for the
// prefill GEMMs, and a value outside fp16's range sets *flag.
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(NormArgs a) {
  __shared__ double s_red[kNormThreads / kWave];
  const int i = blockIdx.x, tid = threadIdx.x;
  const int64_t xr = static_cast<int64_t>(i) * a.row_mul + a.row_add;
  const int nch = a.H / 8;
  u32x4_t v[kNormMaxChunks], wv[kNormMaxChunks];
  // the weights' chunks are loaded with the row, not after the reduction
#pragma unroll
  for (int q = 0; q < kNormMaxChunks; ++q) {
    const int c = tid + q * kNormThreads;
    if (c < nch) wv[q] = reinterpret_cast<const u32x4_t*>(a.w)[c];
  }
  double ss = 0.0;
#pragma unroll
  for (int q = 0; q < kNormMaxChunks; ++q) {
    const int c = tid + q * kNormThreads;
    if (c >= nch) break;
    u32x4_t x = reinterpret_cast<const u32x4_t*>(a.x + xr * a.H)[c];
    if (a.delta) {
      x = norm_add(x, reinterpret_cast<const u32x4_t*>(a.delta + xr * a.H)[c]);
      reinterpret_cast<u32x4_t*>(a.x_out + xr * a.H)[c] = x;
    }
    v[q] = x;
    ss = norm_sq(x, ss);
  }
  ss = norm_wave_sum(ss);
  if ((tid & 63) == 0) s_red[tid >> 6] = ss;
  __syncthreads();
  const double r = norm_r(s_red, a.H, a.eps);
  bool ovf = false;
#pragma unroll
  for (int q = 0; q < kNormMaxChunks; ++q) {
    const int c = tid + q * kNormThreads;
    if (c >= nch) break;
    const u32x4_t o = norm_apply(v[q], wv[q], r);
    reinterpret_cast<u32x4_t*>(a.out + static_cast<int64_t>(i) * a.H)[c] = o;
    if (a.outh) reinterpret_cast<u32x4_t*>(a.outh + static_cast<int64_t>(i) * a.H)[c] = bf16_chunk_to_f16_p8(o, ovf);
  }
  if (a.outh && __ballot(ovf) && (tid & 63) == 0) atomicOr(a.flag, 1u);
}

// ------------------------------------------------------------------ decode projections

// out[t, :] for t < T <= 16 of a packed matrix (single blocks, fmx_dev.hpp):
// one workgroup per 16-column tile, its 4 waves taking every fourth 128-k
// unit, loads of kDnBatch units in flight per wave; exact dequantisation
// (pk_unit: the fp32 value of x.(s*q + b)); the waves' partial sums are
// added in wave order. Epilogue: bf16(acc), then + bias[col], then
// res[t] + (each step rounded to bf16, as MLX's separate ops).
constexpr int kDnBatch = 4;
static_assert(kNormThreads == 256, "the fused norms run on the projection's 256 threads");

// NIN: the row is formed in LDS by the input norm (every workgroup the
// same, rmsnorm_kernel's arithmetic), for single-row forwards: one kernel
// boundary fewer (a cache write-back and invalidation across the XCDs: the
// norm kernel took ~5 us at batch 1, the fused norm adds ~2.7 us to the
// projection; at 4 rows every workgroup's norms cost more than the kernel).
template <bool NIN>
__global__ __launch_bounds__(256) void dense_dec_kernel(DenseArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t s_dn[];  // NIN: the rows [T][K] bf16
  __shared__ f32x4_t s_acc[3][kWave];
  __shared__ double s_red[kDenseNormMaxT][kNormThreads / kWave];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i16 = lane & 15, j = lane >> 4;
  const int tile = blockIdx.x;
  const int K = a.nu * 128;
  const uint8_t* tb = a.w + static_cast<int64_t>(tile) * a.nu * kBlockSingle;
  const int col = tile * 16 + i16;
  // the epilogue's bias and residual values, loaded by wave 0 ahead of the
  // products (after them they would add a memory round trip)
  uint16_t bias_v = 0, res_v[4] = {0, 0, 0, 0}, res2_v[4] = {0, 0, 0, 0};
  if (wave == 0) {
    if (a.bias) bias_v = a.bias[col];
    if (a.res)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (4 * j + r < a.T) {
          res_v[r] = a.res[static_cast<int64_t>(4 * j + r) * a.ldr + col];
          if (a.res2) res2_v[r] = a.res2[static_cast<int64_t>(4 * j + r) * a.ldr + col];
        }
  }

  // the wave's first batch of weight units is issued before anything waits:
  // with the input norm, the raw rows' loads go out first and the norm is
  // formed while the weights are in flight (loads complete in order, so the
  // norm waits for the rows only)
  PkUnit<false> L[kDnBatch];
  auto load_batch = [&](int u0) {
#pragma unroll
    for (int d = 0; d < kDnBatch; ++d) {
      const int u = min(u0 + 4 * d, a.nu - 1);  // units past K repeat the last and are skipped
      L[d] = pk_load<false>(tb + static_cast<int64_t>(u) * kBlockSingle, lane);
    }
  };

  const uint16_t* xrow;
  if constexpr (NIN) {
    // the input norm of the T rows, into LDS
    const int nch = K / 8;
    u32x4_t xv[kDenseNormMaxT][kNormMaxChunks], dv[kDenseNormMaxT][kNormMaxChunks], wv[kNormMaxChunks];
    double ss[kDenseNormMaxT];
#pragma unroll
    for (int t = 0; t < kDenseNormMaxT; ++t) {
      if (t >= a.T) continue;
#pragma unroll
      for (int q = 0; q < kNormMaxChunks; ++q) {
        const int c = tid + q * kNormThreads;
        if (c >= nch) break;
        xv[t][q] = reinterpret_cast<const u32x4_t*>(a.nin + static_cast<int64_t>(t) * a.ldx)[c];
        if (a.ndelta) dv[t][q] = reinterpret_cast<const u32x4_t*>(a.ndelta + static_cast<int64_t>(t) * a.ldx)[c];
      }
    }
#pragma unroll
    for (int q = 0; q < kNormMaxChunks; ++q) {
      const int c = tid + q * kNormThreads;
      if (c < nch) wv[q] = reinterpret_cast<const u32x4_t*>(a.nin_w)[c];
    }
    load_batch(wave);
#pragma unroll
    for (int t = 0; t < kDenseNormMaxT; ++t) {
      ss[t] = 0.0;
      if (t >= a.T) continue;
#pragma unroll
      for (int q = 0; q < kNormMaxChunks; ++q) {
        const int c = tid + q * kNormThreads;
        if (c >= nch) break;
        if (a.ndelta) xv[t][q] = norm_add(xv[t][q], dv[t][q]);
        ss[t] = norm_sq(xv[t][q], ss[t]);
      }
    }
#pragma unroll
    for (int t = 0; t < kDenseNormMaxT; ++t) {
      if (t >= a.T) continue;
      const double sw = norm_wave_sum(ss[t]);
      if (lane == 0) s_red[t][wave] = sw;
    }
    __syncthreads();
    u32x4_t* s_x = reinterpret_cast<u32x4_t*>(s_dn);
#pragma unroll
    for (int t = 0; t < kDenseNormMaxT; ++t) {
      if (t >= a.T) continue;
      const double r = norm_r(s_red[t], K, a.eps);
#pragma unroll
      for (int q = 0; q < kNormMaxChunks; ++q) {
        const int c = tid + q * kNormThreads;
        if (c >= nch) break;
        s_x[t * nch + c] = norm_apply(xv[t][q], wv[q], r);
      }
    }
    __syncthreads();
    xrow = reinterpret_cast<const uint16_t*>(s_dn) + static_cast<int64_t>(min(i16, a.T - 1)) * K + 8 * j;
  } else {
    load_batch(wave);
    xrow = a.x + static_cast<int64_t>(min(i16, a.T - 1)) * a.ldx + 8 * j;
  }

  f32x4_t acc = {0.f, 0.f, 0.f, 0.f}, unused = {0.f, 0.f, 0.f, 0.f};
  for (int u0 = wave; u0 < a.nu; u0 += 4 * kDnBatch) {
    if (u0 != wave) load_batch(u0);
    bf16x8_t A[kDnBatch][4];
#pragma unroll
    for (int d = 0; d < kDnBatch; ++d) {
      const int u = min(u0 + 4 * d, a.nu - 1);
#pragma unroll
      for (int q = 0; q < 4; ++q) A[d][q] = *reinterpret_cast<const bf16x8_t*>(xrow + 128 * u + 32 * q);
    }
#pragma unroll
    for (int d = 0; d < kDnBatch; ++d)
      if (u0 + 4 * d < a.nu) pk_unit<false>(L[d], A[d], acc, unused);
  }
  if (wave > 0) s_acc[wave - 1][lane] = acc;
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int w = 0; w < 3; ++w) acc += s_acc[w][lane];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 4 * j + r;
      uint16_t v = f32_to_bf16(acc[r]);
      if (a.bias) v = f32_to_bf16(bf16_to_f32(v) + bf16_to_f32(bias_v));
      if (a.res) {
        const float rv = a.res2 ? bf16_to_f32(f32_to_bf16(bf16_to_f32(res_v[r]) + bf16_to_f32(res2_v[r])))
                                : bf16_to_f32(res_v[r]);
        v = f32_to_bf16(rv + bf16_to_f32(v));
      }
      if (t < a.T) a.out[static_cast<int64_t>(t) * a.ldo + col] = v;
    }
  }
}

// ------------------------------------------------------------------ RoPE + cache

__device__ inline int token_pos(const int32_t* offs, int off, int b, int l, int64_t max_seq) {
  int64_t p = static_cast<int64_t>(offs ? offs[b] : off) + l;
  return static_cast<int>(p < 0 ? 0 : (p >= max_seq ? max_seq - 1 : p));
}

// cache slot of sequence b: slots[b] (clamped to the cache) or b
__device__ inline int64_t cache_slot(const int32_t* slots, int n_slots, int b) {
  if (!slots) return b;
  const int s = slots[b];
  return s < 0 ? 0 : (s >= n_slots ? n_slots - 1 : s);
}

// One workgroup per token t = b * L + l at position p = offset(b) + l:
// q heads rotated into q_out, k heads rotated into the layer's key cache at
// p, v heads copied into the value cache at p. Rotation of pair (i, i + hd/2)
// by the table's (cos, sin) of p * base^(-2i/hd): each output is the exact
// fp64 value of x1 c - x2 s (or x1 s + x2 c) rounded once to bf16
// (mx::fast::rope, traditional = false, model.cpp:871-872).
__global__ __launch_bounds__(256) void rope_cache_kernel(RopeArgs a) {
  const int t = blockIdx.x;
  const int b = t / a.L, l = t - b * a.L;
  const int p = token_pos(a.offs, a.off, b, l, a.max_seq);
  const int64_t slot = cache_slot(a.slots, a.n_slots, b);
  const int half = a.hd / 2, nq = a.nh + 2 * a.nkv;
  const uint16_t* row = a.qkv + static_cast<int64_t>(t) * nq * a.hd;
  const float* cs = a.cs + static_cast<int64_t>(p) * half * 2;
  for (int it = threadIdx.x; it < (a.nh + a.nkv) * half; it += blockDim.x) {
    const int head = it / half, i = it - head * half;
    const uint16_t* src = row + head * a.hd;
    const double x1 = bf16_to_f32(src[i]), x2 = bf16_to_f32(src[i + half]);
    const double c = cs[2 * i], s = cs[2 * i + 1];
    const uint16_t o1 = f64_to_bf16(__builtin_fma(x1, c, -(x2 * s)));
    const uint16_t o2 = f64_to_bf16(__builtin_fma(x1, s, x2 * c));
    uint16_t* dst;
    if (head < a.nh) {
      dst = a.q_out + (static_cast<int64_t>(t) * a.nh + head) * a.hd;
    } else {
      const int g = head - a.nh;
      dst = a.kc + ((slot * a.nkv + g) * a.max_seq + p) * a.hd;
    }
    dst[i] = o1;
    dst[i + half] = o2;
  }
  for (int it = threadIdx.x; it < a.nkv * a.hd / 8; it += blockDim.x) {
    const int g = it / (a.hd / 8), c = it - g * (a.hd / 8);
    const u32x4_t v = reinterpret_cast<const u32x4_t*>(row + (a.nh + a.nkv + g) * a.hd)[c];
    reinterpret_cast<u32x4_t*>(a.vc + ((slot * a.nkv + g) * a.max_seq + p) * a.hd)[c] = v;
  }
}

// ------------------------------------------------------------------ attention

// One workgroup of kAttnThreads per (token t = b * L + l, q head h): keys
// 0 .. p of kv head g = h / (nh / nkv), p = offset(b) + l (causal).
//   s_j = scale * sum_d q_d k_jd   (fp32, d in order: exact bf16 products)
//   e_j = exp(s_j - max s)         (fp64, the deterministic exp)
//   out_d = sum_j e_j v_jd / sum_j e_j, both sums in fp64 over four
//           contiguous quarters of the keys (keys in order within a quarter,
//           fma), the quarter sums added in order; rounded once to bf16
// (mx::fast::scaled_dot_product_attention, model.cpp:879-882). Scores: a
// thread per key; the weighted sum: wave w takes quarter w, its lanes pairs
// of dimensions. Forwards of several tokens per sequence, after
// rope_cache_kernel (single-token forwards: attn_split_kernel).
constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / kWave;
constexpr int kAttnBatch = 32;  // keys whose value words are loaded together

template <int PAIRS>
__global__ __launch_bounds__(kAttnThreads) void attn_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t s_at[];
  __shared__ float s_q[kAttnMaxHd];
  __shared__ float s_max[kAttnWaves];
  __shared__ double s_num[kAttnWaves][kAttnMaxHd];
  __shared__ double s_den[kAttnWaves];
  double* s_e = reinterpret_cast<double*>(s_at);
  float* s_s = reinterpret_cast<float*>(s_at + static_cast<size_t>(a.max_seq) * 8);
  const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int b = t / a.L, l = t - b * a.L;
  const int p = token_pos(a.offs, a.off, b, l, a.max_seq);
  const int nk = p + 1;
  const int rep = a.nh / a.nkv, g = h / rep;
  const int64_t cbase = (cache_slot(a.slots, a.n_slots, b) * a.nkv + g) * a.max_seq * a.hd;
  uint16_t* kb = a.kc + cbase;
  uint16_t* vb = a.vc + cbase;
  const uint16_t* qrow = a.q + (static_cast<int64_t>(t) * a.nh + h) * a.hd;
  for (int d = tid; d < a.hd; d += kAttnThreads) s_q[d] = bf16_to_f32(qrow[d]);
  __syncthreads();

  // this wave's quarter of the keys for the weighted sum below; its first
  // kAttnBatch value words are loaded now, so that their latency overlaps
  // the scores
  const int quarter = (nk + kAttnWaves - 1) / kAttnWaves;
  const int j0 = min(wave * quarter, nk), j1 = min(j0 + quarter, nk);
  const int npair = a.hd / 2;
  const int jg = j1;
  // lanes past the head's pairs read pair 0 (in bounds) and discard it
  uint32_t vv[kAttnBatch][PAIRS];
  int prl[PAIRS];
#pragma unroll
  for (int i = 0; i < PAIRS; ++i) prl[i] = (lane + kWave * i) < npair ? lane + kWave * i : 0;
  auto load_values = [&](int jb) {
#pragma unroll
    for (int u = 0; u < kAttnBatch; ++u) {
      const uint32_t* vr = reinterpret_cast<const uint32_t*>(vb + static_cast<int64_t>(min(jb + u, jg - 1)) * a.hd);
#pragma unroll
      for (int i = 0; i < PAIRS; ++i) vv[u][i] = vr[prl[i]];
    }
  };
  if (j0 < jg) load_values(j0);

  // scores, a thread per key
  float m = -__builtin_huge_valf();
  for (int jk = tid; jk < nk; jk += kAttnThreads) {
    // the key row's chunks are loaded 16 at a time, then used in order
    float acc = 0.0f;
    const u32x4_t* kr = reinterpret_cast<const u32x4_t*>(kb + static_cast<int64_t>(jk) * a.hd);
    const int nch = a.hd / 8;
    for (int c0 = 0; c0 < nch; c0 += 16) {
      u32x4_t kv[16];
#pragma unroll
      for (int c = 0; c < 16; ++c) kv[c] = kr[min(c0 + c, nch - 1)];
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        if (c0 + c < nch) {
#pragma unroll
          for (int mm = 0; mm < 4; ++mm) {
            acc = __builtin_fmaf(s_q[8 * (c0 + c) + 2 * mm], bf16_to_f32(kv[c][mm] & 0xffffu), acc);
            acc = __builtin_fmaf(s_q[8 * (c0 + c) + 2 * mm + 1], bf16_to_f32(kv[c][mm] >> 16), acc);
          }
        }
      }
    }
    const float sc = acc * a.scale;
    s_s[jk] = sc;
    m = fmaxf(m, sc);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if (lane == 0) s_max[wave] = m;
  __syncthreads();
  m = s_max[0];
#pragma unroll
  for (int w = 1; w < kAttnWaves; ++w) m = fmaxf(m, s_max[w]);
  for (int jk = tid; jk < nk; jk += kAttnThreads)
    s_e[jk] = exp_det(static_cast<double>(s_s[jk]) - static_cast<double>(m));
  __syncthreads();

  // weighted sum: wave w over keys [j0, j1), lane over dimension pairs
  // (2 pr, 2 pr + 1), pr = lane + 64 i; the value words of kAttnBatch keys
  // are loaded together, then used in key order
  double num[PAIRS][2], den = 0.0;
#pragma unroll
  for (int i = 0; i < PAIRS; ++i) num[i][0] = num[i][1] = 0.0;
  for (int jb = j0; jb < jg; jb += kAttnBatch) {
    if (jb != j0) load_values(jb);
#pragma unroll
    for (int u = 0; u < kAttnBatch; ++u) {
      if (jb + u < jg) {
        const double e = s_e[jb + u];
        den += e;
#pragma unroll
        for (int i = 0; i < PAIRS; ++i) {
          num[i][0] = __builtin_fma(e, static_cast<double>(bf16_to_f32(vv[u][i] & 0xffffu)), num[i][0]);
          num[i][1] = __builtin_fma(e, static_cast<double>(bf16_to_f32(vv[u][i] >> 16)), num[i][1]);
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < PAIRS; ++i) {
    const int pr = lane + kWave * i;
    if (pr < npair) {
      s_num[wave][2 * pr] = num[i][0];
      s_num[wave][2 * pr + 1] = num[i][1];
    }
  }
  if (lane == 0) s_den[wave] = den;
  __syncthreads();

  bool ovf = false;
  for (int d = tid; d < a.hd; d += kAttnThreads) {
    double nsum = s_num[0][d], dsum = s_den[0];
#pragma unroll
    for (int w = 1; w < kAttnWaves; ++w) {
      nsum += s_num[w][d];
      dsum += s_den[w];
    }
    const uint16_t o = f64_to_bf16(nsum / dsum);
    const int64_t oc = static_cast<int64_t>(h) * a.hd + d;
    a.out[static_cast<int64_t>(t) * a.ldo + oc] = o;
    if (a.outh) {
      ovf = ovf || bf16_f16_overflow(o);
      a.outh[static_cast<int64_t>(t) * a.ldo + ((oc & ~7) | p8_slot(oc & 7))] =
          static_cast<uint16_t>(bf16_to_f16_bits(o));
    }
  }
  if (a.outh && __ballot(ovf) && lane == 0) atomicOr(a.flag, 1u);
}

// ------------------------------------------------------------------ split attention

// Single-token forwards (L == 1, head size at most kAttnSplitMaxHd): one
// workgroup per (token t, q head h), the keys 0 .. p in S = min(
// kAttnSplitMax, ceil((p + 1) / kAttnSplitKeys)) contiguous ranges
// [nk s / S, nk (s + 1) / S), wave s taking range s. At batch 1 the
// kernel's time is one workgroup's chain of memory round trips, so the
// ranges are short (up to 16 waves, 32 keys each up to 512 keys) and a wave
// issues everything its first 32 keys need at once, in the order it uses
// them (the rotation's inputs, then key rows and 16-byte value chunks: at
// most 21 loads), all as whole rows: one round trip before the arithmetic.
// In range s:
//   s_j = scale * (((P_0 + P_1) + ...) + P_{hd/8-1}), P_c = sum_{d in chunk
//         c} q_d k_jd (8 dimensions in order; exact bf16 products in fp32):
//         lane (key, c) forms P_c, an LDS transpose hands a key's P_c to one
//         lane, which adds them in order
//   m_s = max of the range's scores
//   e_j = exp(s_j - m_s) (fp64, the deterministic exp)
//   over the key classes c = (j - j0) mod 4, each in key order:
//   den_s = ((D_0 + D_1) + D_2) + D_3, D_c = sum_j e_j
//   num_s,d = ((N_0 + N_1) + N_2) + N_3, N_c = sum_j e_j v_jd (fma)
//   (lane (c, i) accumulates class c for dimensions 8i .. 8i + 7)
// and the ranges combine through LDS, in order:
//   M = max m_s, f_s = exp(m_s - M), den = sum_s f_s den_s,
//   num_d = sum_s f_s num_s,d (fma; the first term a product),
//   out_d = bf16(num_d / den)
// (one range: f_0 = 1, the range's own sums). q and the new key are
// rotated from the q/k/v row as rope_cache_kernel does; the new key and
// value (position p, the last key of the last range) are used from LDS, and
// the first q head of each kv group writes them into the caches (no
// workgroup reads position p from the cache in this launch).
constexpr int kAttnRound = 32;   // keys per score round and per value batch
constexpr int kAttnValKeys = kAttnRound / 4;  // keys per class in a value batch
constexpr int kAttnPcStride = 17;  // LDS floats per key of a round's chunk sums (16 + 1: no bank conflicts)
static_assert(kAttnSplitKeys == kAttnRound, "a range of the minimum length is one round");

__device__ inline int attn_splits(int nk) {
  return min(kAttnSplitMax, (nk + kAttnSplitKeys - 1) / kAttnSplitKeys);
}

__global__ __launch_bounds__(kWave * kAttnSplitMax) void attn_split_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t s_at[];
  __shared__ float s_q[kAttnSplitMaxHd];
  __shared__ uint16_t s_knew[kAttnSplitMaxHd], s_vnew[kAttnSplitMaxHd];
  __shared__ double s_part[kAttnSplitMax][kAttnSplitMaxHd + 2];  // per range: m, den, num
  __shared__ double s_f[kAttnSplitMax];
  const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int rep = a.nh / a.nkv, g = h / rep;
  const int half = a.hd / 2, nch = a.hd / 8;

  // 1. the position and the cache slot (token_pos, cache_slot): both words
  // are loaded together, ahead of every load whose address needs them (a
  // null pointer reads a word of the q/k/v row and discards it, so neither
  // load waits behind a branch): one memory round trip
  const uint16_t* row = a.qkv + static_cast<int64_t>(t) * (a.nh + 2 * a.nkv) * a.hd;
  const int32_t* po = a.offs ? a.offs + t : reinterpret_cast<const int32_t*>(row);
  const int32_t* ps = a.slots ? a.slots + t : reinterpret_cast<const int32_t*>(row);
  // both addresses formed before either load (scalar loads complete out of
  // order: a wait for one pointer argument would wait for the other word)
  asm volatile("" : "+s"(po), "+s"(ps));
  const int32_t ow = *po, sw = *ps;
  const int64_t p64 = a.offs ? static_cast<int64_t>(ow) : static_cast<int64_t>(a.off);
  const int p = static_cast<int>(p64 < 0 ? 0 : (p64 >= a.max_seq ? a.max_seq - 1 : p64));
  const int64_t slot = a.slots ? (sw < 0 ? 0 : (sw >= a.n_slots ? a.n_slots - 1 : sw)) : t;
  const int nk = p + 1, S = attn_splits(nk);
  const int64_t cbase = (slot * a.nkv + g) * a.max_seq * a.hd;
  uint16_t* kb = a.kc + cbase;
  uint16_t* vb = a.vc + cbase;
  // this wave's range; keys before jg come from the cache (p, the last key
  // of the last range, from LDS)
  const bool active = wave < S;
  const int j0 = active ? static_cast<int>(static_cast<int64_t>(nk) * wave / S) : 0;
  const int j1 = active ? static_cast<int>(static_cast<int64_t>(nk) * (wave + 1) / S) : 0;
  const bool last = wave == S - 1;
  const int jg = last ? j1 - 1 : j1;
  const int jclamp = max(jg - 1, 0);  // loads past the range re-read its last cached key
  // 2. the first key round (32 keys: instruction c brings keys c * kpi +
  // lane / nch, chunk lane mod nch) and value batch (lane (c, i): keys j0 +
  // c + 4u, chunk i)
  const int kc = lane >> 4, dc = lane & 15;
  const bool vlane = dc < nch;
  const int kpi = kWave / nch;                    // keys per load instruction
  const int kk = lane / nch, kch = lane % nch;   // this lane's key in it, its chunk
  const int nkin = max(1, kAttnRound / kpi);     // load instructions per round
  constexpr int kMaxKin = kAttnRound * kAttnSplitMaxHd / 8 / kWave;
  u32x4_t kv[kMaxKin], vv[kAttnValKeys];
  // the cache is read once per step: non-temporal loads keep it from
  // evicting the next kernels' code and data (decoder stack, batch 8: 1.855
  // -> 1.805 ms per step; batch 1 unchanged)
  auto load_keys = [&](int jb) {
#pragma unroll
    for (int c = 0; c < kMaxKin; ++c)
      if (c < nkin)
        kv[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(
            kb + static_cast<int64_t>(min(jb + c * kpi + kk, jclamp)) * a.hd + 8 * kch));
  };
  auto load_values = [&](int jb) {
#pragma unroll
    for (int u = 0; u < kAttnValKeys; ++u)
      vv[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(
          vb + static_cast<int64_t>(min(jb + kc + 4 * u, jclamp)) * a.hd + 8 * min(dc, nch - 1)));
  };
  if (active && j0 < jg) {
    load_keys(j0);
    load_values(j0);
  }
  // and, in the same round trip, the rotation's inputs: thread i < hd takes
  // pair i mod hd/2 of q (i < hd/2) or of the new key and the table's
  // (cos, sin) at p; thread d < hd the new value's element d
  const bool rot = tid < a.hd;
  const int hd_i = tid % half;
  uint16_t rx1 = 0, rx2 = 0, rv = 0;
  float rc = 0.0f, rsn = 0.0f;
  if (rot) {
    const uint16_t* src = row + (tid < half ? h : a.nh + g) * a.hd;
    const float* cs = a.cs + static_cast<int64_t>(p) * half * 2;
    rx1 = src[hd_i];
    rx2 = src[hd_i + half];
    rv = row[(a.nh + a.nkv + g) * a.hd + tid];
    rc = cs[2 * hd_i];
    rsn = cs[2 * hd_i + 1];
  }

  // 3. rotation (one rounding of the fp64 value), the new value
  if (rot) {
    const double x1 = bf16_to_f32(rx1), x2 = bf16_to_f32(rx2);
    const double c = rc, sn = rsn;
    const uint16_t o1 = f64_to_bf16(__builtin_fma(x1, c, -(x2 * sn)));
    const uint16_t o2 = f64_to_bf16(__builtin_fma(x1, sn, x2 * c));
    if (tid < half) {
      s_q[hd_i] = bf16_to_f32(o1);
      s_q[hd_i + half] = bf16_to_f32(o2);
    } else {
      s_knew[hd_i] = o1;
      s_knew[hd_i + half] = o2;
    }
    s_vnew[tid] = rv;
  }
  __syncthreads();

  // 4. scores (LDS per wave: the range's fp64 weights, its fp32 scores,
  // and the chunk sums of one 32-key round)
  const int kmax = attn_split_range_keys(a.max_seq);
  double* s_e = reinterpret_cast<double*>(s_at) + static_cast<size_t>(wave) * kmax;
  float* s_s = reinterpret_cast<float*>(s_at + static_cast<size_t>(kAttnSplitMax) * kmax * 8) +
               static_cast<size_t>(wave) * kmax;
  float* s_pc = reinterpret_cast<float*>(s_at + static_cast<size_t>(kAttnSplitMax) * kmax * 12) +
                static_cast<size_t>(wave) * kAttnRound * kAttnPcStride;
  float m = -__builtin_huge_valf();
  if (active) {
    // this lane's chunk of q, 8 dimensions
    float qc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) qc[e] = s_q[8 * kch + e];
    for (int jb = j0; jb < jg; jb += kAttnRound) {
      if (jb != j0) load_keys(jb);
#pragma unroll
      for (int c = 0; c < kMaxKin; ++c) {
        const int key = c * kpi + kk;
        if (c < nkin && key < kAttnRound) {
          float pc = 0.0f;
#pragma unroll
          for (int mm = 0; mm < 4; ++mm) {
            pc = __builtin_fmaf(qc[2 * mm], bf16_to_f32(kv[c][mm] & 0xffffu), pc);
            pc = __builtin_fmaf(qc[2 * mm + 1], bf16_to_f32(kv[c][mm] >> 16), pc);
          }
          s_pc[key * kAttnPcStride + kch] = pc;
        }
      }
      // the wave's LDS operations complete in order: each lane now sums its
      // key's chunks as the other lanes wrote them
      __builtin_amdgcn_wave_barrier();
      if (lane < kAttnRound && jb + lane < jg) {
        float acc = s_pc[lane * kAttnPcStride];
        for (int c = 1; c < nch; ++c) acc += s_pc[lane * kAttnPcStride + c];
        const float sc = acc * a.scale;
        s_s[jb + lane - j0] = sc;
        m = fmaxf(m, sc);
      }
      __builtin_amdgcn_wave_barrier();
    }
    if (last && lane == (p - j0) % kAttnRound) {  // the new key, from LDS (the lane that takes key p below)
      float acc = 0.0f;
      for (int c = 0; c < nch; ++c) {
        float pc = 0.0f;
        for (int e = 0; e < 8; ++e) pc = __builtin_fmaf(s_q[8 * c + e], bf16_to_f32(s_knew[8 * c + e]), pc);
        acc = c ? acc + pc : pc;
      }
      const float sc = acc * a.scale;
      s_s[p - j0] = sc;
      m = fmaxf(m, sc);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    // each lane reads back only the scores it wrote
    if (lane < kAttnRound)
      for (int jk = j0 + lane; jk < j1; jk += kAttnRound)
        s_e[jk - j0] = exp_det(static_cast<double>(s_s[jk - j0]) - static_cast<double>(m));
  }
  __syncthreads();

  // 5. the range's sums
  if (active) {
    double nv[8], dv = 0.0;
#pragma unroll
    for (int i = 0; i < 8; ++i) nv[i] = 0.0;
    for (int jb = j0; jb < jg; jb += kAttnRound) {
      if (jb != j0) load_values(jb);
#pragma unroll
      for (int u = 0; u < kAttnValKeys; ++u) {
        const int j = jb + kc + 4 * u;
        if (j < jg) {
          const double e = s_e[j - j0];
          dv += e;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            nv[2 * q] = __builtin_fma(e, static_cast<double>(bf16_to_f32(vv[u][q] & 0xffffu)), nv[2 * q]);
            nv[2 * q + 1] = __builtin_fma(e, static_cast<double>(bf16_to_f32(vv[u][q] >> 16)), nv[2 * q + 1]);
          }
        }
        // one key's fp64 conversions at a time (converting a batch ahead
        // would need more registers than the kernel has)
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (last && kc == (p - j0) % 4) {  // the new key's value, last of its class
      const double e = s_e[p - j0];
      dv += e;
      const u32x4_t w4 = reinterpret_cast<const u32x4_t*>(s_vnew)[min(dc, nch - 1)];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        nv[2 * q] = __builtin_fma(e, static_cast<double>(bf16_to_f32(w4[q] & 0xffffu)), nv[2 * q]);
        nv[2 * q + 1] = __builtin_fma(e, static_cast<double>(bf16_to_f32(w4[q] >> 16)), nv[2 * q + 1]);
      }
    }
    // the classes in order: ((X_0 + X_1) + X_2) + X_3 in the lanes of class 0
    const double d1 = __shfl(dv, lane + 16), d2 = __shfl(dv, lane + 32), d3 = __shfl(dv, lane + 48);
    const double den = ((dv + d1) + d2) + d3;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const double n1 = __shfl(nv[i], lane + 16), n2 = __shfl(nv[i], lane + 32), n3 = __shfl(nv[i], lane + 48);
      if (kc == 0 && vlane) s_part[wave][2 + 8 * dc + i] = ((nv[i] + n1) + n2) + n3;
    }
    if (lane == 0) {
      s_part[wave][0] = static_cast<double>(m);
      s_part[wave][1] = den;
    }
  }
  __syncthreads();

  // 6. the combine, ranges in order: thread d takes dimension d
  if (tid < S) {
    double M = s_part[0][0];
    for (int r = 1; r < S; ++r) M = fmax(M, s_part[r][0]);
    s_f[tid] = exp_det(s_part[tid][0] - M);
  }
  __syncthreads();
  bool ovf = false;
  if (tid < a.hd) {
    const int d = tid;
    double dn = 0.0, nm = 0.0;
    for (int r = 0; r < S; ++r) {
      const double f = s_f[r];
      dn = r ? __builtin_fma(s_part[r][1], f, dn) : s_part[r][1] * f;
      nm = r ? __builtin_fma(s_part[r][2 + d], f, nm) : s_part[r][2 + d] * f;
    }
    const uint16_t o = f64_to_bf16(nm / dn);
    const int64_t oc = static_cast<int64_t>(h) * a.hd + d;
    a.out[static_cast<int64_t>(t) * a.ldo + oc] = o;
    if (a.outh) {
      ovf = bf16_f16_overflow(o);
      a.outh[static_cast<int64_t>(t) * a.ldo + ((oc & ~7) | p8_slot(oc & 7))] =
          static_cast<uint16_t>(bf16_to_f16_bits(o));
    }
  }
  if (a.outh && __ballot(ovf) && lane == 0) atomicOr(a.flag, 1u);
  // the new key and value into the caches, last: nothing after them waits
  // for the stores
  if (h % rep == 0 && tid < a.hd) {
    kb[static_cast<int64_t>(p) * a.hd + tid] = s_knew[tid];
    vb[static_cast<int64_t>(p) * a.hd + tid] = s_vnew[tid];
  }
}

// ------------------------------------------------------------------ greedy

// ids[b] = argmax of logits row b (the first of equal maxima, as mx::argmax);
// offs[b] += inc when offs is given (the next decode position).
__global__ __launch_bounds__(1024) void greedy_kernel(GreedyArgs a) {
  __shared__ float s_v[1024 / kWave];
  __shared__ int64_t s_i[1024 / kWave];
  const int b = blockIdx.x, tid = threadIdx.x;
  const uint16_t* row = a.logits + static_cast<int64_t>(b) * a.ld;
  float best = -__builtin_huge_valf();
  int64_t bi = a.V;
  // a thread takes 16-byte chunks c = tid, tid + 1024, ... (index order, so
  // the first maximum it sees is its lowest), loads of 4 chunks in flight
  // (20 in flight measured no faster: one workgroup's row is bound by what
  // one CU draws from HBM, about 25 GB/s); rows that are not 16-byte aligned
  // or a multiple of 8 take the scalar loop
  const bool vec = (a.ld % 8 == 0) && (a.V % 8 == 0) && (reinterpret_cast<uintptr_t>(a.logits) % 16 == 0);
  if (vec) {
    const u32x4_t* rv = reinterpret_cast<const u32x4_t*>(row);
    const int64_t nch = a.V / 8;
    for (int64_t c0 = tid; c0 < nch; c0 += 4 * 1024) {
      u32x4_t ch[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) ch[u] = rv[min(c0 + 1024 * u, nch - 1)];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t c = c0 + 1024 * u;
        if (c >= nch) break;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = bf16_to_f32((ch[u][e >> 1] >> (16 * (e & 1))) & 0xffffu);
          if (x > best) {  // strict: within a thread indices ascend; NaN never wins
            best = x;
            bi = 8 * c + e;
          }
        }
      }
    }
  } else {
    for (int64_t v = tid; v < a.V; v += blockDim.x) {
      const float x = bf16_to_f32(row[v]);
      if (x > best) {
        best = x;
        bi = v;
      }
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ob = __shfl_xor(best, o);
    const int64_t oi = __shfl_xor(bi, o);
    if (ob > best || (ob == best && oi < bi)) {
      best = ob;
      bi = oi;
    }
  }
  if ((tid & 63) == 0) {
    s_v[tid >> 6] = best;
    s_i[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid != 0) return;
  for (int w = 1; w < static_cast<int>(blockDim.x) / kWave; ++w)
    if (s_v[w] > best || (s_v[w] == best && s_i[w] < bi)) {
      best = s_v[w];
      bi = s_i[w];
    }
  if (bi >= a.V) bi = 0;  // an all-NaN row
  a.ids[b] = static_cast<int32_t>(bi);
  if (a.offs) a.offs[b] += a.inc;
}

__global__ __launch_bounds__(256) void copy_u32_kernel(const uint32_t* src, uint32_t* dst, int64_t n) {
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
    dst[i] = src[i];
}

// one 16-byte chunk of one (layer, k/v, head, position) row per thread
__global__ __launch_bounds__(256) void kv_copy_kernel(KvCopyArgs a) {
  const int64_t per_row = a.hd / 8;
  const int64_t n = a.layers * 2 * a.nkv * a.n_pos * per_row;
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t c8 = i % per_row, r = i / per_row;
    const int64_t p = r % a.n_pos, lh = r / a.n_pos;  // lh = (layer * 2 + kv) * nkv + head
    const int64_t h = lh % a.nkv, lk = lh / a.nkv;
    const int64_t co = (((lk * a.cache_batch + a.slot) * a.nkv + h) * a.max_seq + p) * a.hd + c8 * 8;
    const int64_t eo = ((lk * a.nkv + h) * a.cap + p) * a.hd + c8 * 8;
    u32x4_t* dst = reinterpret_cast<u32x4_t*>(a.to_cache ? a.cache + co : a.entry + eo);
    const u32x4_t* src = reinterpret_cast<const u32x4_t*>(a.to_cache ? a.entry + eo : a.cache + co);
    *dst = *src;
  }
}

}  // namespace

hipError_t launch_kv_copy(const KvCopyArgs& a, hipStream_t stream) {
  const int64_t n = a.layers * 2 * a.nkv * a.n_pos * (a.hd / 8);
  if (n <= 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(kv_copy_kernel, dim3(static_cast<uint32_t>(blocks < 4096 ? blocks : 4096)), dim3(256), 0,
                     stream, a);
  return hipGetLastError();
}

hipError_t launch_copy_u32(const uint32_t* src, uint32_t* dst, int64_t n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(copy_u32_kernel, dim3(static_cast<uint32_t>(blocks < 1024 ? blocks : 1024)), dim3(256),
                     0, stream, src, dst, n);
  return hipGetLastError();
}

hipError_t launch_embed(const EmbedArgs& a, hipStream_t stream) {
  if (a.T == 0) return hipSuccess;
  hipLaunchKernelGGL(embed_kernel, dim3(a.T), dim3(256), 0, stream, a);
  return hipGetLastError();
}

bool rmsnorm_fits(int64_t H) { return H % 8 == 0 && H / 8 <= kNormThreads * kNormMaxChunks; }

hipError_t launch_rmsnorm(const NormArgs& a, int n_rows, hipStream_t stream) {
  if (n_rows == 0) return hipSuccess;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(n_rows), dim3(kNormThreads), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_dense_dec(const DenseArgs& a, hipStream_t stream) {
  if (a.T == 0 || a.nt == 0) return hipSuccess;
  const bool nin = a.nin != nullptr;
  if (nin && (a.T > kDenseNormMaxT || !a.nin_w || !rmsnorm_fits(a.nu * 128) || a.ldx % 8))
    return hipErrorInvalidValue;
  const size_t lds = nin ? static_cast<size_t>(a.T) * a.nu * 128 * 2 : 0;
  if (nin)
    hipLaunchKernelGGL(dense_dec_kernel<true>, dim3(a.nt), dim3(256), lds, stream, a);
  else
    hipLaunchKernelGGL(dense_dec_kernel<false>, dim3(a.nt), dim3(256), lds, stream, a);
  return hipGetLastError();
}

hipError_t launch_rope_cache(const RopeArgs& a, int T, hipStream_t stream) {
  if (T == 0) return hipSuccess;
  hipLaunchKernelGGL(rope_cache_kernel, dim3(T), dim3(256), 0, stream, a);
  return hipGetLastError();
}

size_t attn_lds_bytes(int64_t max_seq) { return static_cast<size_t>(max_seq) * 12; }

hipError_t launch_attn(const AttnArgs& a, int T, hipStream_t stream) {
  if (T == 0) return hipSuccess;
  if (a.qkv) {
    if (a.L != 1 || a.hd > kAttnSplitMaxHd || a.hd % 8 || kWave % (a.hd / 8)) return hipErrorInvalidValue;
    // LDS: per wave, a range's fp64 weights and fp32 scores, one round's chunk sums
    const int64_t keys = attn_split_range_keys(a.max_seq);
    hipLaunchKernelGGL(attn_split_kernel, dim3(T, a.nh), dim3(kWave * kAttnSplitMax),
                       static_cast<size_t>(kAttnSplitMax * (keys * 12 + kAttnRound * kAttnPcStride * 4)), stream, a);
    return hipGetLastError();
  }
  const dim3 grid(T, a.nh);
  const size_t lds = attn_lds_bytes(a.max_seq);
  if (a.hd <= 128)
    hipLaunchKernelGGL((attn_kernel<1>), grid, dim3(kAttnThreads), lds, stream, a);
  else
    hipLaunchKernelGGL((attn_kernel<2>), grid, dim3(kAttnThreads), lds, stream, a);
  return hipGetLastError();
}

hipError_t launch_greedy(const GreedyArgs& a, int B, hipStream_t stream) {
  if (B == 0) return hipSuccess;
  hipLaunchKernelGGL(greedy_kernel, dim3(B), dim3(1024), 0, stream, a);
  return hipGetLastError();
}

}  // namespace fmx
