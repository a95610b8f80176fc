// fmx_model_kernels.hpp -- argument blocks and launchers of the decoder-stack
// kernels (fmx_model.hip; library-internal).
#pragma once

#include "fmx_common.hpp"

namespace fmx {

struct EmbedArgs {
  const uint16_t* table;  // [V, H] bf16
  int64_t V;
  int H;
  const int32_t* ids;     // [T]
  int T;
  uint16_t* h;            // [T, H]
  uint32_t* flags;        // words cleared by block 0 (the forward's fp16-range flags)
  int n_flags;
};
hipError_t launch_embed(const EmbedArgs& a, hipStream_t stream);

struct NormArgs {
  const uint16_t* x;      // rows of H bf16; output row i reads row i * row_mul + row_add
  int64_t row_mul, row_add;
  const uint16_t* delta;  // null, or rows added first: x = bf16(x + delta), written to x_out
  uint16_t* x_out;
  const uint16_t* w;      // [H] bf16
  float eps;
  int H;
  uint16_t* out;          // [n, H] bf16
  uint16_t* outh;         // null, or [n, H] fp16 (P8 layout); values outside fp16 set *flag
  uint32_t* flag;
};
bool rmsnorm_fits(int64_t H);
hipError_t launch_rmsnorm(const NormArgs& a, int n_rows, hipStream_t stream);

// out[t, col] for t < T <= 16 of a packed single-block matrix [nt*16, nu*128]
struct DenseArgs {
  const uint16_t* x;      // [T, K] bf16, row stride ldx
  int64_t ldx;
  int T;
  const uint8_t* w;       // packed blocks
  int nt, nu;
  uint16_t* out;
  int64_t ldo;
  const uint16_t* bias;   // [nt*16] bf16 or null
  const uint16_t* res;    // rows added last (stride ldr) or null; may alias out
  const uint16_t* res2;   // or null: res = bf16(res + res2) first (same stride)
  int64_t ldr;
  // At most kDenseNormMaxT rows, K within rmsnorm_kernel's limit: input
  // norm (nin set): the rows are x = rmsnorm_kernel's output for the
  // rows bf16(nin + ndelta) (ndelta nullable, stride ldx) with weights
  // nin_w, formed by every workgroup in LDS (x unused; nothing written back)
  const uint16_t* nin;
  const uint16_t* ndelta;
  const uint16_t* nin_w;
  float eps;
};
constexpr int kDenseNormMaxT = 1;
hipError_t launch_dense_dec(const DenseArgs& a, hipStream_t stream);

// Positions: token t = b * L + l sits at offs[b] + l (device offsets) or
// off + l, clamped to [0, max_seq); its keys and values live in cache slot
// slots[b] (or b).
struct RopeArgs {
  const uint16_t* qkv;    // [T, (nh + 2 nkv) * hd]: q heads, k heads, v heads
  int L, nh, nkv, hd;
  const float* cs;        // [max_pos][hd/2][2] (cos, sin)
  const int32_t* offs;
  int off;
  int64_t max_seq;
  const int32_t* slots;   // cache slot of each sequence (null: slot b), clamped to n_slots
  int n_slots;
  uint16_t* q_out;        // [T, nh * hd] rotated q
  uint16_t* kc;           // this layer's caches [B_cache][nkv][max_seq][hd]
  uint16_t* vc;
};
hipError_t launch_rope_cache(const RopeArgs& a, int T, hipStream_t stream);

constexpr int kAttnMaxHd = 256;
constexpr int64_t kAttnMaxSeq = 4096;  // keys per query: 48 KB of LDS scores
struct AttnArgs {
  const uint16_t* q;      // [T, nh * hd] rotated (when qkv is null)
  const uint16_t* qkv;    // or: the q/k/v rows of a single-token-per-sequence forward
                          //   (L == 1), rotated and cached by the attention kernel itself
  const float* cs;        //   with this RoPE table
  int L, nh, nkv, hd;
  uint16_t* kc;           // [B_cache][nkv][max_seq][hd]
  uint16_t* vc;
  int64_t max_seq;
  const int32_t* offs;
  int off;
  const int32_t* slots;   // as RopeArgs
  int n_slots;
  float scale;
  uint16_t* out;          // [T, nh * hd] bf16 (row stride ldo)
  int64_t ldo;
  uint16_t* outh;         // null, or the same in fp16 (P8 layout); values outside fp16 set *flag
  uint32_t* flag;
};
// single-token forwards (qkv set; head size at most kAttnSplitMaxHd): a
// query's keys in min(kAttnSplitMax, ceil(keys / kAttnSplitKeys))
// contiguous ranges, one wave each
constexpr int kAttnSplitMax = 16;
constexpr int kAttnSplitKeys = 32;
constexpr int kAttnSplitMaxHd = 128;
// the longest range of a cache of max_seq positions
__host__ __device__ inline int attn_split_range_keys(int64_t max_seq) {
  const int64_t r = (max_seq + kAttnSplitMax - 1) / kAttnSplitMax;
  return static_cast<int>(r > kAttnSplitKeys ? r : kAttnSplitKeys);
}
size_t attn_lds_bytes(int64_t max_seq);
hipError_t launch_attn(const AttnArgs& a, int T, hipStream_t stream);

struct GreedyArgs {
  const uint16_t* logits; // [B][ld] bf16, V valid
  int64_t V, ld;
  int32_t* ids;           // [B]
  int32_t* offs;          // null, or offsets advanced by inc
  int32_t inc;
};
hipError_t launch_greedy(const GreedyArgs& a, int B, hipStream_t stream);

hipError_t launch_copy_u32(const uint32_t* src, uint32_t* dst, int64_t n, hipStream_t stream);

// Positions [0, n_pos) of one KV-cache slot ([layers][2][cache_batch][nkv]
// [max_seq][hd] bf16) to or from a compact copy [layers][2][nkv][cap][hd]
// (cap >= n_pos): the scheduler's prefix cache.
struct KvCopyArgs {
  uint16_t* cache;
  uint16_t* entry;
  int64_t layers, cache_batch, nkv, max_seq, hd, cap, n_pos;
  int64_t slot;
  int to_cache;          // 1: entry -> cache slot; 0: cache slot -> entry
};
hipError_t launch_kv_copy(const KvCopyArgs& a, hipStream_t stream);

}  // namespace fmx
