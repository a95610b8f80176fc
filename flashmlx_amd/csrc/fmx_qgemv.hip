// fmx_qgemv.hip -- decode-shape grouped GEMM over packed 4-bit expert weights.
//
// Same product as fmx_qgemm.hip (mx::gather_qmm / quantized_matmul with
// transpose=true, group 64, bits 4: server/src/model.cpp:703-721, :741-747,
// fused gate/up SwiGLU of :14-25, :715), for segments of at most 16 rows
// (decode batches), on weights re-laid out once at load time by
// fmx_pack_expert_weights.
//
// Packed layout. A matrix [N, K] is cut into tiles of 16 rows and units of
// 128 k (two quantisation groups). Block (tile, unit) holds, for lane
// l = 16*j + c of a wave, the 16 bytes of row 16*tile + c that the lane feeds
// to four v_mfma_f32_16x16x32_bf16 as its B operand: words 4a + j (a = 0..3)
// of the unit, i.e. k = 32a + 8j .. 32a + 8j + 7. MFMAs a = 0, 1 then cover
// group 0 of the unit and a = 2, 3 group 1, so every group's partial sum is
// formed without masking. After the 1024 weight bytes come 16 x 8 bytes of
// (scale g0, scale g1, bias g0, bias g1) per row. A SwiGLU pair stores gate
// and up blocks side by side: [gate w | up w | gate sb | up sb], 2304 bytes.
// One wave's load of a unit is one contiguous 1 KB piece.
//
// Exact dequantisation as in fmx_qgemm.hip: nibbles become the bf16 values
// 128 + q; per group acc += s * x.(128+q) + (b - 128 s) * x.1.
//
// Schedule. One workgroup = one (segment, 16-row tile, K slice); its KS
// waves split the slice into runs of UPW units. Each wave first starts the
// copy of its share of the activation rows into LDS (LDS DMA, no registers),
// then issues the loads of all of its units at once, so a wave keeps its
// whole share of the weight stream in flight; the units are consumed in
// order as they arrive. Segment metadata (expert, rows, source rows) comes
// from one record per segment written by the router's sort, read with
// scalar loads.
#include <algorithm>

#include "fmx_kernels.hpp"

namespace fmx {

__device__ inline f32x4_t mfma_bf16(const bf16x8_t& a, const bf16x8_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 8 nibbles -> bf16 pairs (128 + q_i, 128 + q_{i+4}), i = 0..3
__device__ inline bf16x8_t nib8(uint32_t w) {
  u32x4_t d;
  d[0] = (w & 0x000f000fu) | 0x43004300u;
  d[1] = ((w >> 4) & 0x000f000fu) | 0x43004300u;
  d[2] = ((w >> 8) & 0x000f000fu) | 0x43004300u;
  d[3] = ((w >> 12) & 0x000f000fu) | 0x43004300u;
  return __builtin_bit_cast(bf16x8_t, d);
}

template <bool DUAL>
struct PkUnit {
  u32x4_t w0, w1;    // packed words (gate / up)
  u32x2_t sb0, sb1;  // (s g0 | s g1 << 16, b g0 | b g1 << 16)
};

template <bool DUAL>
__device__ inline PkUnit<DUAL> pk_load(const uint8_t* blk, int lane) {
  PkUnit<DUAL> L;
  const int col = lane & 15;
  L.w0 = *reinterpret_cast<const u32x4_t*>(blk + 16 * lane);
  if (DUAL) {
    L.w1 = *reinterpret_cast<const u32x4_t*>(blk + 1024 + 16 * lane);
    L.sb0 = *reinterpret_cast<const u32x2_t*>(blk + 2048 + 8 * col);
    L.sb1 = *reinterpret_cast<const u32x2_t*>(blk + 2048 + 128 + 8 * col);
  } else {
    L.sb0 = *reinterpret_cast<const u32x2_t*>(blk + 1024 + 8 * col);
  }
  return L;
}

// acc[i] += s0 P0 + (b0 - 128 s0) X0 + s1 P1 + (b1 - 128 s1) X1, rows i < MR
template <int MR>
__device__ inline void pk_epi(f32x4_t& acc, const u32x2_t& sb, const f32x4_t& P0, const f32x4_t& P1,
                              const f32x4_t& X0, const f32x4_t& X1) {
  const float s0 = __uint_as_float(sb[0] << 16), s1 = __uint_as_float(sb[0] & 0xffff0000u);
  const float c0 = __builtin_fmaf(-128.0f, s0, __uint_as_float(sb[1] << 16));
  const float c1 = __builtin_fmaf(-128.0f, s1, __uint_as_float(sb[1] & 0xffff0000u));
#pragma unroll
  for (int i = 0; i < MR; ++i) {
    acc[i] = __builtin_fmaf(s0, P0[i], acc[i]);
    acc[i] = __builtin_fmaf(c0, X0[i], acc[i]);
    acc[i] = __builtin_fmaf(s1, P1[i], acc[i]);
    acc[i] = __builtin_fmaf(c1, X1[i], acc[i]);
  }
}

template <bool DUAL, int MR>
__device__ inline void pk_unit(const PkUnit<DUAL>& L, const uint16_t* xu, f32x4_t& acc0,
                               f32x4_t& acc1) {
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
  const u32x4_t ones_u = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, ones_u);
  bf16x8_t A[4];
#pragma unroll
  for (int a = 0; a < 4; ++a) A[a] = *reinterpret_cast<const bf16x8_t*>(xu + 32 * a);
  f32x4_t X0 = mfma_bf16(A[1], ones, mfma_bf16(A[0], ones, zero));
  f32x4_t X1 = mfma_bf16(A[3], ones, mfma_bf16(A[2], ones, zero));
  {
    f32x4_t P0 = mfma_bf16(A[1], nib8(L.w0[1]), mfma_bf16(A[0], nib8(L.w0[0]), zero));
    f32x4_t P1 = mfma_bf16(A[3], nib8(L.w0[3]), mfma_bf16(A[2], nib8(L.w0[2]), zero));
    pk_epi<MR>(acc0, L.sb0, P0, P1, X0, X1);
  }
  if (DUAL) {
    f32x4_t P0 = mfma_bf16(A[1], nib8(L.w1[1]), mfma_bf16(A[0], nib8(L.w1[0]), zero));
    f32x4_t P1 = mfma_bf16(A[3], nib8(L.w1[3]), mfma_bf16(A[2], nib8(L.w1[2]), zero));
    pk_epi<MR>(acc1, L.sb1, P0, P1, X0, X1);
  }
}

struct GemvItem {
  int e, r0, rows, tile, kw;
  const uint32_t* rec;
};

template <bool DUAL, int UPW, int MR>
__device__ void gemv_finish(const GemvProblem& P, const GemvItem& it, const PkUnit<DUAL> (&L)[UPW],
                            int nu_w, const uint16_t* xl, float* s_red, int KS) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int j = lane >> 4, col = lane & 15;
  f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int d = 0; d < UPW; ++d)
    if (d < nu_w) pk_unit<DUAL, MR>(L[d], xl + d * 128, acc0, acc1);

  // the waves' partial sums meet in LDS; wave 0 adds them in wave order
  constexpr int NV = (DUAL ? 2 : 1) * MR;
  if (KS > 1) {
    if (wave > 0) {
      float* dst = s_red + (wave - 1) * NV * kWave;
#pragma unroll
      for (int i = 0; i < MR; ++i) {
        dst[i * kWave + lane] = acc0[i];
        if (DUAL) dst[(MR + i) * kWave + lane] = acc1[i];
      }
    }
    __syncthreads();
    if (wave != 0) return;
    for (int w = 1; w < KS; ++w) {
      const float* srcp = s_red + (w - 1) * NV * kWave;
#pragma unroll
      for (int i = 0; i < MR; ++i) {
        acc0[i] += srcp[i * kWave + lane];
        if (DUAL) acc1[i] += srcp[(MR + i) * kWave + lane];
      }
    }
  }
  const int n = it.tile * 16 + col;
  const int N = P.nt * 16;
#pragma unroll
  for (int i = 0; i < MR; ++i) {
    const int rl = 4 * j + i;
    if (rl >= it.rows) continue;
    const int64_t orow = it.r0 + rl;
    if (P.part) {
      P.part[(static_cast<int64_t>(it.kw) * P.out_rows + orow) * N + n] = acc0[i];
    } else {
      uint16_t v;
      if (DUAL)
        v = swiglu_bf16(round_bf16(acc0[i]), round_bf16(acc1[i]));
      else
        v = f32_to_bf16(acc0[i]);
      const int ncol = P.out_p8 ? ((n & ~7) | p8_slot(n & 7)) : n;
      P.out[orow * P.ldo + ncol] = v;
    }
  }
}

template <bool DUAL, int UPW>
__device__ void gemv_item(const GemvProblem& P, int b, int KS, uint16_t* s_x, float* s_red) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int per_seg = P.nt * P.ks_wg;
  const int seg = b / per_seg, rem = b - seg * per_seg;
  GemvItem it;
  it.tile = rem / P.ks_wg;
  it.kw = rem - it.tile * P.ks_wg;
  it.rec = nullptr;
  if (P.recs) {
    const uint32_t nseg = min(*P.seg_n, static_cast<uint32_t>(P.max_seg));
    if (static_cast<uint32_t>(seg) >= nseg) return;
    it.rec = P.recs + static_cast<int64_t>(seg) * kSegRecWords;
    it.e = static_cast<int>(min(it.rec[16], static_cast<uint32_t>(P.n_exp - 1)));
    it.r0 = static_cast<int>(min(it.rec[17], static_cast<uint32_t>(P.out_rows)));
    it.rows = static_cast<int>(min(min(it.rec[18], static_cast<uint32_t>(P.max_rows)),
                                   static_cast<uint32_t>(P.out_rows - it.r0)));
  } else {
    it.e = 0;
    it.r0 = 0;
    it.rows = min(P.rows_static, P.max_rows);
  }
  if (it.rows <= 0) return;

  // K range of this workgroup and of this wave (in units of 128)
  const int u_wg = UPW * KS;
  const int ub_wg = it.kw * u_wg;
  const int nu_wg = min(u_wg, P.nu - ub_wg);
  const int kw_len = nu_wg * 128;
  const int stride = static_cast<int>(align_up(kw_len, 512)) + 8;  // LDS row stride (elements)
  const int ub = ub_wg + wave * UPW;
  const int nu_w = max(0, min(UPW, P.nu - ub));

  // 1. activation rows -> LDS, 512 elements (one 16-byte piece per lane) per
  // copy. The source rows are read (scalar loads) before the first copy.
  // The copies are issued as inline assembly: they are older than every load
  // the compiler tracks, so its own vmcnt waits stay correct, and the wait
  // for the copies themselves is the explicit one in step 3.
  {
    typedef uint32_t u32x16_t __attribute__((ext_vector_type(16)));
    u32x16_t src;
    if (P.gather) {
      src = *reinterpret_cast<const u32x16_t*>(it.rec);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) src[i] = static_cast<uint32_t>(it.r0 + i);
    }
    const int cpr = (kw_len + 511) / 512;
    const int K = P.nu * 128;
    const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
        (__attribute__((address_space(3))) uint16_t*)s_x));
#pragma unroll
    for (int row = 0; row < 16; ++row) {
      if (row >= it.rows) break;
      const int64_t xrow = min(src[row], static_cast<uint32_t>(P.x_rows - 1));
      for (int pc = wave; pc < cpr; pc += KS) {
        const int k = min(ub_wg * 128 + pc * 512 + 8 * lane, K - 8);
        const uint16_t* g = P.x + xrow * P.ldx + k;
        const uint32_t l = lds0 + static_cast<uint32_t>(row * stride + pc * 512) * 2u;
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                     :
                     : "v"(g), "s"(l)
                     : "memory", "m0");
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. every unit of this wave: loads in flight together (unit indices are
  // clamped into the matrix; units past the slice are loaded but not used)
  constexpr int BB = DUAL ? 2304 : 1152;
  const uint8_t* base = P.wpk + static_cast<int64_t>(it.e) * P.estride +
                        static_cast<int64_t>(it.tile) * P.nu * BB;
  PkUnit<DUAL> L[UPW];
#pragma unroll
  for (int d = 0; d < UPW; ++d) L[d] = pk_load<DUAL>(base + min(ub + d, P.nu - 1) * BB, lane);
  __builtin_amdgcn_sched_barrier(0);

  // 3. wait for this wave's LDS copies, which were issued before its weight
  // loads (s_waitcnt vmcnt(NL), gfx9 encoding: vmcnt[3:0] | expcnt[6:4] |
  // lgkmcnt[11:8] | vmcnt[5:4] at [15:14]), then for every wave's
  {
    constexpr int NL = UPW * (DUAL ? 4 : 2);
    static_assert(NL <= 63, "vmcnt range");
    constexpr int imm = (NL & 15) | (7 << 4) | (15 << 8) | ((NL >> 4) << 14);
    __builtin_amdgcn_s_waitcnt(imm);
    __builtin_amdgcn_s_barrier();
  }

  const int m = lane & 15, j = lane >> 4;
  const uint16_t* xl = s_x + min(m, it.rows - 1) * stride + wave * UPW * 128 + 8 * j;
  if (it.rows == 1)
    gemv_finish<DUAL, UPW, 1>(P, it, L, nu_w, xl, s_red, KS);
  else if (it.rows == 2)
    gemv_finish<DUAL, UPW, 2>(P, it, L, nu_w, xl, s_red, KS);
  else
    gemv_finish<DUAL, UPW, 4>(P, it, L, nu_w, xl, s_red, KS);
}

template <bool DUAL, int UPW>
__global__ __launch_bounds__(kGemvMaxThreads) void qgemv_kernel(GemvProblem p0, GemvProblem p1,
                                                                int nblk0, int KS, int red_off) {
  extern __shared__ __attribute__((aligned(16))) uint16_t s_mem[];
  float* s_red = reinterpret_cast<float*>(reinterpret_cast<char*>(s_mem) + red_off);
  const int bid = blockIdx.x;
  if (bid < nblk0)
    gemv_item<DUAL, UPW>(p0, bid, KS, s_mem, s_red);
  else
    gemv_item<DUAL, UPW>(p1, bid - nblk0, KS, s_mem, s_red);
}

// LDS: staged rows (16 rows max) of the workgroup's K slice, then the
// cross-wave reduction buffer.
static size_t gemv_lds(const GemvProblem& p, int upw, int ks, int dual, size_t* red_off) {
  const int rows = p.max_rows;
  const int kw_len = std::min(upw * ks, p.nu) * 128;
  const size_t x_bytes = static_cast<size_t>(rows) * (align_up(kw_len, 512) + 8) * 2;
  *red_off = static_cast<size_t>(align_up(static_cast<int64_t>(x_bytes), 16));
  return *red_off + static_cast<size_t>(ks - 1) * (dual ? 8 : 4) * kWave * 4;
}

hipError_t launch_qgemv(const GemvProblem& p0_, const GemvProblem* p1_, int dual, int upw, int ks,
                        hipStream_t stream) {
  if (ks < 1 || ks * kWave > kGemvMaxThreads || (upw != 4 && upw != 8)) return hipErrorInvalidValue;
  if (p0_.max_rows < 1 || p0_.max_rows > 16 || (p1_ && (p1_->max_rows < 1 || p1_->max_rows > 16)))
    return hipErrorInvalidValue;
  GemvProblem p0 = p0_, p1 = p1_ ? *p1_ : p0_;
  for (GemvProblem* p : {&p0, &p1}) p->ks_wg = (p->nu + upw * ks - 1) / (upw * ks);
  size_t r0 = 0, r1 = 0;
  size_t lds = gemv_lds(p0, upw, ks, dual, &r0);
  if (p1_) lds = std::max(lds, gemv_lds(p1, upw, ks, dual, &r1));
  const size_t red_off = std::max(r0, r1);
  lds = std::max(lds, red_off + static_cast<size_t>(ks - 1) * (dual ? 8 : 4) * kWave * 4);
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  const int nblk0 = p0.max_seg * p0.nt * p0.ks_wg;
  const int nblk1 = p1_ ? p1.max_seg * p1.nt * p1.ks_wg : 0;
  if (nblk0 + nblk1 == 0) return hipSuccess;
  const dim3 grid(nblk0 + nblk1), block(ks * kWave);
  const int ro = static_cast<int>(red_off);
  if (dual && upw == 8)
    hipLaunchKernelGGL((qgemv_kernel<true, 8>), grid, block, lds, stream, p0, p1, nblk0, ks, ro);
  else if (dual)
    hipLaunchKernelGGL((qgemv_kernel<true, 4>), grid, block, lds, stream, p0, p1, nblk0, ks, ro);
  else if (upw == 8)
    hipLaunchKernelGGL((qgemv_kernel<false, 8>), grid, block, lds, stream, p0, p1, nblk0, ks, ro);
  else
    hipLaunchKernelGGL((qgemv_kernel<false, 4>), grid, block, lds, stream, p0, p1, nblk0, ks, ro);
  return hipGetLastError();
}

// ---------------------------------------------------------------- packing

// One thread per (expert, tile, unit, lane): the lane's 16 weight bytes of
// each matrix; lanes 0..15 also the (scale, bias) words of their row.
__global__ void pack_kernel(PackArgs a) {
  const int64_t blk = blockIdx.x;  // (expert, tile, unit)
  const int lane = threadIdx.x;
  const int64_t per_exp = static_cast<int64_t>(a.nt) * a.nu;
  const int64_t e = blk / per_exp;
  const int64_t r = blk - e * per_exp;
  const int tile = static_cast<int>(r / a.nu), u = static_cast<int>(r - static_cast<int64_t>(tile) * a.nu);
  const int col = lane & 15, j = lane >> 4;
  const int K = a.nu * 128, G = K / kGroup;
  const int64_t row = static_cast<int64_t>(tile) * 16 + col;
  const int nm = a.w1 ? 2 : 1;
  const int BB = nm == 2 ? 2304 : 1152;
  uint8_t* dst = a.dst + e * a.dst_estride + (static_cast<int64_t>(tile) * a.nu + u) * BB;
  for (int mtx = 0; mtx < nm; ++mtx) {
    const uint32_t* w = mtx ? a.w1 : a.w0;
    const uint16_t* s = mtx ? a.s1 : a.s0;
    const uint16_t* bb = mtx ? a.b1 : a.b0;
    const uint32_t* wr = w + (e * a.N + row) * (K / 8) + u * 16;
    u32x4_t v;
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = wr[4 * q + j];
    *reinterpret_cast<u32x4_t*>(dst + mtx * 1024 + 16 * lane) = v;
    if (lane < 16) {
      const int64_t g = (e * a.N + row) * G + 2 * u;
      u32x2_t sb;
      sb[0] = static_cast<uint32_t>(s[g]) | (static_cast<uint32_t>(s[g + 1]) << 16);
      sb[1] = static_cast<uint32_t>(bb[g]) | (static_cast<uint32_t>(bb[g + 1]) << 16);
      *reinterpret_cast<u32x2_t*>(dst + nm * 1024 + mtx * 128 + 8 * col) = sb;
    }
  }
}

hipError_t launch_pack(const PackArgs& a, hipStream_t stream) {
  const int64_t blocks = a.n_exp * a.nt * a.nu;
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(pack_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kWave), 0, stream, a);
  return hipGetLastError();
}

}  // namespace fmx
