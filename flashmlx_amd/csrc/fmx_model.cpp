// fmx_model.cpp -- C-ABI of the decoder stack (include/fmx_model.h): the
// launch sequence of LlamaModel::forward (server/src/model.cpp:1021-1033)
// for all-MoE models, with the MoE block on fmx_moe_block_forward.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <vector>

#include "../../include/fmx_model.h"
#include "fmx_kernels.hpp"
#include "fmx_model_kernels.hpp"

namespace fmx {
int set_error(int status, const char* msg);
void clear_error();
}  // namespace fmx

using namespace fmx;

namespace {

int fail(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return set_error(status, buf);
}

int ok() {
  clear_error();
  return FMX_OK;
}

#define FMX_HIP(expr)                                                              \
  do {                                                                             \
    hipError_t e_ = (expr);                                                        \
    if (e_ != hipSuccess)                                                          \
      return fail(FMX_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_));            \
  } while (0)

#define FMX_RC(expr)        \
  do {                      \
    int rc_ = (expr);       \
    if (rc_) return rc_;    \
  } while (0)

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

constexpr int64_t kDenseDecMaxRows = 16;  // decode projections: at most 16 rows
constexpr int64_t kMaxPositions = 32768;  // RoPE table rows (the cache itself: kAttnMaxSeq)

struct Dims {
  int64_t H, L, nh, nkv, hd, V, P, nqkv;
};

Dims dims(const fmx_model_config& c) {
  Dims d{};
  d.H = c.hidden_size;
  d.L = c.num_hidden_layers;
  d.nh = c.num_attention_heads;
  d.nkv = c.num_key_value_heads;
  d.hd = c.head_dim > 0 ? c.head_dim : (c.num_attention_heads > 0 ? c.hidden_size / c.num_attention_heads : 0);
  d.V = c.vocab_size;
  d.P = c.max_position_embeddings;
  d.nqkv = (d.nh + 2 * d.nkv) * d.hd;
  return d;
}

int check_config(const fmx_model_config* c) {
  if (!c) return fail(FMX_ERR_ARG, "cfg is NULL");
  const Dims d = dims(*c);
  if (d.H <= 0 || d.H % 128 || !rmsnorm_fits(d.H))
    return fail(FMX_ERR_UNSUPPORTED, "hidden_size=%lld (a multiple of 128, <= 8192)", (long long)d.H);
  if (d.L < 1) return fail(FMX_ERR_SHAPE, "num_hidden_layers=%lld", (long long)d.L);
  if (d.nh < 1 || d.nkv < 1 || d.nh % d.nkv)
    return fail(FMX_ERR_SHAPE, "heads %lld / kv heads %lld", (long long)d.nh, (long long)d.nkv);
  if (d.hd < 8 || d.hd % 8 || d.hd > kAttnMaxHd)
    return fail(FMX_ERR_UNSUPPORTED, "head_dim=%lld (a multiple of 8, <= %d)", (long long)d.hd, kAttnMaxHd);
  if ((d.nh * d.hd) % 128 || d.nqkv % 16)
    return fail(FMX_ERR_UNSUPPORTED, "heads * head_dim=%lld (a multiple of 128)", (long long)(d.nh * d.hd));
  if (d.V < 16 || d.V % 16) return fail(FMX_ERR_UNSUPPORTED, "vocab_size=%lld (a multiple of 16)", (long long)d.V);
  if (d.P < 1 || d.P > kMaxPositions)
    return fail(FMX_ERR_UNSUPPORTED, "max_position_embeddings=%lld (1..%lld)", (long long)d.P,
                (long long)kMaxPositions);
  if (c->moe.hidden_size != d.H) return fail(FMX_ERR_SHAPE, "moe.hidden_size != hidden_size");
  if (c->moe.activation_dtype != FMX_BF16)
    return fail(FMX_ERR_UNSUPPORTED, "moe.activation_dtype=%d: the decoder stack runs in bf16",
                c->moe.activation_dtype);
  if (fmx_moe_workspace_size(&c->moe, 1) == 0) return fail(FMX_ERR_ARG, "invalid moe config");
  if (fmx_moe_packed_size(&c->moe) == 0)
    return fail(FMX_ERR_UNSUPPORTED, "the MoE block's shapes are outside the packed layout");
  return FMX_OK;
}

// ---------------------------------------------------------------- workspace

struct Arena {
  char* base;
  size_t used = 0;
  void* take(size_t bytes) {
    void* p = base ? base + used : nullptr;
    used = static_cast<size_t>(align_up(static_cast<int64_t>(used + bytes), 256));
    return p;
  }
};

// flags and the RoPE table first, then the MoE workspace (its counters at its
// start: both at offsets independent of the token count), then the
// activations
struct ModelLayout {
  uint32_t* flags;  // [2 L + 1]: per layer the q/k/v input and the o input, then the final norm
  float* rope;      // [P][hd/2][2]
  void* moe_ws;
  size_t moe_bytes;
  uint16_t *h, *normed, *normed_h, *qkv, *qrot, *attn, *attn_h, *moe_out;
  size_t total;
};

ModelLayout model_layout(const fmx_model_config& c, int64_t T, char* base) {
  const Dims d = dims(c);
  Arena ar{base};
  ModelLayout M{};
  M.flags = static_cast<uint32_t*>(ar.take((2 * d.L + 1) * 4));
  M.rope = static_cast<float*>(ar.take(d.P * (d.hd / 2) * 2 * 4));
  M.moe_bytes = fmx_moe_workspace_size(&c.moe, T);
  M.moe_ws = ar.take(M.moe_bytes);
  M.h = static_cast<uint16_t*>(ar.take(T * d.H * 2));
  M.normed = static_cast<uint16_t*>(ar.take(T * d.H * 2));
  M.normed_h = static_cast<uint16_t*>(ar.take(T * d.H * 2));
  M.qkv = static_cast<uint16_t*>(ar.take(T * d.nqkv * 2));
  M.qrot = static_cast<uint16_t*>(ar.take(T * d.nh * d.hd * 2));
  M.attn = static_cast<uint16_t*>(ar.take(T * d.nh * d.hd * 2));
  M.attn_h = static_cast<uint16_t*>(ar.take(T * d.nh * d.hd * 2));
  M.moe_out = static_cast<uint16_t*>(ar.take(T * d.H * 2));
  M.total = ar.used;
  return M;
}

// ---------------------------------------------------------------- linears

int64_t packed_linear_bytes(int64_t N, int64_t K) { return (N / 16) * (K / 128) * kPackedBlockSingle; }

// A decode projection's fused input norm (DenseArgs' nin fields; at most
// kDenseNormMaxT rows: the input rows formed from nin (+ ndelta)), and res2
// added to its residual first.
struct FusedNorms {
  const uint16_t* nin = nullptr;
  const uint16_t* ndelta = nullptr;
  const uint16_t* nin_w = nullptr;
  const uint16_t* res2 = nullptr;
  float eps = 0.0f;
};

// out = x . W^T (+ bias) (+ res) for T rows of a packed linear [N, K]: the
// decode kernel for at most 16 rows, else the prefill GEMM grid on the fp16
// copy of x (xh) with its range flag.
int linear(const uint16_t* x, const uint16_t* xh, uint32_t* flag, int64_t T, const void* w, int64_t N,
           int64_t K, const uint16_t* bias, const uint16_t* res, uint16_t* out, hipStream_t stream,
           const FusedNorms& fn = FusedNorms()) {
  if (T <= kDenseDecMaxRows) {
    DenseArgs a{};
    a.nin = fn.nin;
    a.ndelta = fn.ndelta;
    a.nin_w = fn.nin_w;
    a.res2 = fn.res2;
    a.eps = fn.eps;
    a.x = x;
    a.ldx = K;
    a.T = static_cast<int>(T);
    a.w = static_cast<const uint8_t*>(w);
    a.nt = static_cast<int>(N / 16);
    a.nu = static_cast<int>(K / 128);
    a.out = out;
    a.ldo = N;
    a.bias = bias;
    a.res = res;
    a.ldr = N;
    FMX_HIP(launch_dense_dec(a, stream));
    return FMX_OK;
  }
  PfSet s{};
  s.w = static_cast<const uint8_t*>(w);
  s.x = x;
  s.xh = xh;
  s.ldx = K;
  s.out = out;
  s.ldo = N;
  s.nt = static_cast<int>(N / 16);
  s.nu = static_cast<int>(K / 128);
  s.rows_static = s.rows_max = s.x_rows = static_cast<int>(T);
  s.n_exp = 1;
  s.bias = bias;
  s.res = res;
  s.ldr = N;
  PfArgs pa{};
  pa.s1 = s;
  pa.n_items1 = pf_items(pa.s1, false);
  pa.f16_flag = flag;
  pa.flag_in = 1u;
  pa.flag_out = 0u;
  FMX_HIP(launch_pf(pa, false, stream));
  return FMX_OK;
}

}  // namespace

extern "C" {

size_t fmx_packed_linear_size(int64_t n_rows, int64_t K) {
  if (n_rows <= 0 || K <= 0 || n_rows % 16 || K % 128) return 0;
  return static_cast<size_t>(packed_linear_bytes(n_rows, K));
}

int fmx_pack_linear(const fmx_qweight* parts, const int64_t* rows, int n_parts, int64_t K,
                    void* packed, size_t packed_bytes, fmx_stream stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (!parts || !rows || n_parts < 1 || !packed) return fail(FMX_ERR_ARG, "NULL argument");
  if (K <= 0 || K % 128) return fail(FMX_ERR_UNSUPPORTED, "K=%lld (a multiple of 128)", (long long)K);
  int64_t total = 0;
  for (int i = 0; i < n_parts; ++i) {
    if (rows[i] <= 0 || rows[i] % 16)
      return fail(FMX_ERR_UNSUPPORTED, "part %d: %lld rows (a multiple of 16)", i, (long long)rows[i]);
    if (!parts[i].w || !parts[i].scales || !parts[i].biases || !aligned(parts[i].w, 4))
      return fail(FMX_ERR_ARG, "part %d: NULL or misaligned arrays", i);
    total += rows[i];
  }
  if (packed_bytes < static_cast<size_t>(packed_linear_bytes(total, K)))
    return fail(FMX_ERR_WORKSPACE, "packed buffer %zu bytes, need %lld", packed_bytes,
                (long long)packed_linear_bytes(total, K));
  if (!aligned(packed, 256)) return fail(FMX_ERR_ARG, "packed not 256-byte aligned");
  int64_t row0 = 0;
  for (int i = 0; i < n_parts; ++i) {
    PackArgs a{};
    a.w0 = static_cast<const uint32_t*>(parts[i].w);
    a.s0 = static_cast<const uint16_t*>(parts[i].scales);
    a.b0 = static_cast<const uint16_t*>(parts[i].biases);
    a.n_exp = 1;
    a.N = static_cast<int>(rows[i]);
    a.nt = static_cast<int>(rows[i] / 16);
    a.nu = static_cast<int>(K / 128);
    a.dst = static_cast<uint8_t*>(packed) + packed_linear_bytes(row0, K);
    a.dst_estride = 0;
    FMX_HIP(launch_pack(a, stream));
    row0 += rows[i];
  }
  return ok();
}

size_t fmx_model_kv_cache_size(const fmx_model_config* cfg, int64_t cache_batch, int64_t cache_max_seq) {
  if (check_config(cfg) || cache_batch < 1 || cache_max_seq < 1 || cache_max_seq > kAttnMaxSeq) return 0;
  const Dims d = dims(*cfg);
  return static_cast<size_t>(d.L * 2 * cache_batch * d.nkv * cache_max_seq * d.hd * 2);
}

size_t fmx_model_workspace_size(const fmx_model_config* cfg, int64_t max_tokens) {
  if (check_config(cfg) || max_tokens < 1 || max_tokens > 65536) return 0;
  return model_layout(*cfg, max_tokens, nullptr).total;
}

int fmx_model_workspace_init(const fmx_model_config* cfg, void* workspace, size_t workspace_bytes,
                             fmx_stream stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  FMX_RC(check_config(cfg));
  if (!workspace || !aligned(workspace, 256)) return fail(FMX_ERR_ARG, "workspace NULL or misaligned");
  const ModelLayout M = model_layout(*cfg, 1, static_cast<char*>(workspace));
  if (workspace_bytes < M.total) return fail(FMX_ERR_WORKSPACE, "workspace smaller than one token's");
  const Dims d = dims(*cfg);
  FMX_RC(fmx_rope_table(M.rope, d.P, d.hd, cfg->rope_theta, stream_));
  FMX_RC(fmx_moe_workspace_init(M.moe_ws, workspace_bytes - (static_cast<char*>(M.moe_ws) -
                                                             static_cast<char*>(workspace)),
                                stream_));
  return ok();
}

int fmx_model_forward(const fmx_model_config* cfg, const fmx_model_weights* w, const int32_t* input_ids,
                      int64_t B, int64_t Lq, int64_t cache_offset, const int32_t* cache_offsets,
                      void* kv_cache, int64_t cache_batch, int64_t cache_max_seq, int last_only,
                      void* logits, void* workspace, size_t workspace_bytes, fmx_stream stream_) {
  return fmx_model_forward_traced(cfg, w, input_ids, B, Lq, cache_offset, cache_offsets, kv_cache,
                                  cache_batch, cache_max_seq, last_only, logits, workspace,
                                  workspace_bytes, stream_, nullptr);
}

int fmx_model_forward_traced(const fmx_model_config* cfg, const fmx_model_weights* w,
                             const int32_t* input_ids, int64_t B, int64_t Lq, int64_t cache_offset,
                             const int32_t* cache_offsets, void* kv_cache, int64_t cache_batch,
                             int64_t cache_max_seq, int last_only, void* logits, void* workspace,
                             size_t workspace_bytes, fmx_stream stream_, uint32_t* routing) {
  return fmx_model_forward_batched(cfg, w, input_ids, B, Lq, cache_offset, cache_offsets, nullptr, kv_cache,
                                   cache_batch, cache_max_seq, last_only, logits, workspace, workspace_bytes,
                                   stream_, routing);
}

int fmx_model_forward_batched(const fmx_model_config* cfg, const fmx_model_weights* w,
                              const int32_t* input_ids, int64_t B, int64_t Lq, int64_t cache_offset,
                              const int32_t* cache_offsets, const int32_t* cache_slots, void* kv_cache,
                              int64_t cache_batch, int64_t cache_max_seq, int last_only, void* logits,
                              void* workspace, size_t workspace_bytes, fmx_stream stream_,
                              uint32_t* routing) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  FMX_RC(check_config(cfg));
  if (!w || !w->embed || !w->norm_w || !w->lm_head || !w->layers)
    return fail(FMX_ERR_ARG, "weights incomplete");
  if (B < 0 || Lq < 0) return fail(FMX_ERR_SHAPE, "batch %lld, seq_len %lld", (long long)B, (long long)Lq);
  const int64_t T = B * Lq;
  if (T == 0) return ok();
  if (T > 65536) return fail(FMX_ERR_UNSUPPORTED, "%lld tokens (at most 65536)", (long long)T);
  if (!input_ids || !kv_cache || !logits || !workspace) return fail(FMX_ERR_ARG, "NULL buffer");
  if (!cache_slots && B > cache_batch)
    return fail(FMX_ERR_SHAPE, "batch %lld > cache_batch %lld", (long long)B, (long long)cache_batch);
  const Dims d = dims(*cfg);
  if (cache_max_seq < 1 || cache_max_seq > d.P || cache_max_seq > kAttnMaxSeq)
    return fail(FMX_ERR_SHAPE, "cache_max_seq=%lld (1..min(max_position_embeddings, %lld))",
                (long long)cache_max_seq, (long long)kAttnMaxSeq);
  if (!cache_offsets && (cache_offset < 0 || cache_offset + Lq > cache_max_seq))
    return fail(FMX_ERR_SHAPE, "positions %lld..%lld outside the cache (%lld)", (long long)cache_offset,
                (long long)(cache_offset + Lq - 1), (long long)cache_max_seq);
  const size_t need = model_layout(*cfg, T, nullptr).total;
  if (workspace_bytes < need) return fail(FMX_ERR_WORKSPACE, "workspace %zu bytes, need %zu", workspace_bytes, need);
  if (!aligned(workspace, 256) || !aligned(kv_cache, 16) || !aligned(logits, 16))
    return fail(FMX_ERR_ARG, "workspace (256), kv_cache or logits (16) misaligned");
  const ModelLayout M = model_layout(*cfg, T, static_cast<char*>(workspace));
  const bool many = T > kDenseDecMaxRows;
  const int64_t layer_cache = 2 * cache_batch * d.nkv * cache_max_seq * d.hd;  // elements
  const float scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(d.hd)));

  EmbedArgs ea{};
  ea.table = static_cast<const uint16_t*>(w->embed);
  ea.V = d.V;
  ea.H = static_cast<int>(d.H);
  ea.ids = input_ids;
  ea.T = static_cast<int>(T);
  ea.h = M.h;
  ea.flags = M.flags;
  ea.n_flags = static_cast<int>(2 * d.L + 1);
  FMX_HIP(launch_embed(ea, stream));

  for (int64_t l = 0; l < d.L; ++l) {
    const fmx_layer_weights& lw = w->layers[l];
    if (!lw.input_norm_w || !lw.post_norm_w || !lw.qkv || !lw.o)
      return fail(FMX_ERR_ARG, "layer %lld: weights incomplete", (long long)l);
    uint16_t* kc = static_cast<uint16_t*>(kv_cache) + l * layer_cache;
    uint16_t* vc = kc + layer_cache / 2;
    // single-row forwards: the input norm runs in the q/k/v projection and
    // the previous MoE output is added to the residual by the o projection
    // (one kernel, with its cache write-back at the boundary, fewer per
    // layer)
    const bool fuse = T <= kDenseNormMaxT && rmsnorm_fits(d.H);
    // input norm (with the previous layer's MoE residual)
    NormArgs na{};
    na.x = M.h;
    na.row_mul = 1;
    na.delta = l ? M.moe_out : nullptr;
    na.x_out = M.h;
    na.w = static_cast<const uint16_t*>(lw.input_norm_w);
    na.eps = cfg->rms_norm_eps;
    na.H = static_cast<int>(d.H);
    na.out = M.normed;
    na.outh = many ? M.normed_h : nullptr;
    na.flag = M.flags + 2 * l;
    FusedNorms fq, fo;
    if (fuse) {
      fq.nin = M.h;
      fq.ndelta = na.delta;
      fq.nin_w = na.w;
      fq.eps = na.eps;
      fo.res2 = na.delta;
    } else {
      FMX_HIP(launch_rmsnorm(na, static_cast<int>(T), stream));
    }
    // q, k, v (+ biases)
    FMX_RC(linear(M.normed, M.normed_h, M.flags + 2 * l, T, lw.qkv, d.nqkv, d.H,
                  static_cast<const uint16_t*>(lw.qkv_bias), nullptr, M.qkv, stream, fq));
    // RoPE, cache write, attention
    RopeArgs ra{};
    ra.qkv = M.qkv;
    ra.L = static_cast<int>(Lq);
    ra.nh = static_cast<int>(d.nh);
    ra.nkv = static_cast<int>(d.nkv);
    ra.hd = static_cast<int>(d.hd);
    ra.cs = M.rope;
    ra.offs = cache_offsets;
    ra.off = static_cast<int>(cache_offset);
    ra.max_seq = cache_max_seq;
    ra.slots = cache_slots;
    ra.n_slots = static_cast<int>(cache_batch);
    ra.q_out = M.qrot;
    ra.kc = kc;
    ra.vc = vc;
    // single-token forwards (head size up to kAttnSplitMaxHd, 64 / (hd / 8)
    // whole keys per load) rotate and cache inside the attention kernel
    const bool fused = Lq == 1 && d.hd <= kAttnSplitMaxHd && kWave % (d.hd / 8) == 0;
    if (!fused) FMX_HIP(launch_rope_cache(ra, static_cast<int>(T), stream));
    AttnArgs aa{};
    aa.q = M.qrot;
    aa.qkv = fused ? M.qkv : nullptr;
    aa.cs = M.rope;
    aa.L = ra.L;
    aa.nh = ra.nh;
    aa.nkv = ra.nkv;
    aa.hd = ra.hd;
    aa.kc = kc;
    aa.vc = vc;
    aa.max_seq = cache_max_seq;
    aa.offs = cache_offsets;
    aa.off = ra.off;
    aa.slots = cache_slots;
    aa.n_slots = ra.n_slots;
    aa.scale = scale;
    aa.out = M.attn;
    aa.ldo = d.nh * d.hd;
    aa.outh = many ? M.attn_h : nullptr;
    aa.flag = M.flags + 2 * l + 1;
    FMX_HIP(launch_attn(aa, static_cast<int>(T), stream));
    // o_proj with the residual: h = h + attn . Wo^T
    FMX_RC(linear(M.attn, M.attn_h, M.flags + 2 * l + 1, T, lw.o, d.H, d.nh * d.hd, nullptr, M.h, M.h,
                  stream, fo));
    // post-attention norm, MoE block: single-row decode forwards form the
    // norm inside the MoE block's first kernel (one kernel boundary fewer);
    // otherwise the norm kernel, then the block
    int mrc = FMX_ERR_UNSUPPORTED;
    if (T <= kDecNinMaxT && rmsnorm_fits(d.H)) {
      const MoEInputNorm mn{M.h, static_cast<const uint16_t*>(lw.post_norm_w), cfg->rms_norm_eps};
      mrc = moe_block_forward_nin(&cfg->moe, &lw.moe, mn, M.normed, T, M.moe_out, M.moe_ws, M.moe_bytes, stream);
      if (mrc != FMX_OK && mrc != FMX_ERR_UNSUPPORTED) return mrc;
    }
    if (mrc == FMX_ERR_UNSUPPORTED) {
      NormArgs nb = na;
      nb.delta = nullptr;
      nb.w = static_cast<const uint16_t*>(lw.post_norm_w);
      nb.outh = nullptr;
      FMX_HIP(launch_rmsnorm(nb, static_cast<int>(T), stream));
      FMX_RC(fmx_moe_block_forward(&cfg->moe, &lw.moe, M.normed, T, M.moe_out, M.moe_ws, M.moe_bytes,
                                   stream_));
    }
    if (routing) {
      const uint32_t* inds = nullptr;
      FMX_RC(fmx_moe_workspace_routing(&cfg->moe, T, M.moe_ws, &inds, nullptr, nullptr, nullptr, nullptr,
                                       nullptr, nullptr, nullptr));
      const int64_t n = T * cfg->moe.num_experts_per_tok;
      FMX_HIP(launch_copy_u32(inds, routing + l * n, n, stream));
    }
  }
  // final norm (with the last MoE residual) over the rows whose logits are
  // wanted, lm_head
  const int64_t rows = last_only ? B : T;
  NormArgs nf{};
  nf.x = M.h;
  nf.row_mul = last_only ? Lq : 1;
  nf.row_add = last_only ? Lq - 1 : 0;
  nf.delta = M.moe_out;
  nf.x_out = M.h;
  nf.w = static_cast<const uint16_t*>(w->norm_w);
  nf.eps = cfg->rms_norm_eps;
  nf.H = static_cast<int>(d.H);
  nf.out = M.normed;
  nf.outh = rows > kDenseDecMaxRows ? M.normed_h : nullptr;
  nf.flag = M.flags + 2 * d.L;
  FMX_HIP(launch_rmsnorm(nf, static_cast<int>(rows), stream));
  FMX_RC(linear(M.normed, M.normed_h, M.flags + 2 * d.L, rows, w->lm_head, d.V, d.H, nullptr, nullptr,
                static_cast<uint16_t*>(logits), stream));
  return ok();
}

int fmx_model_workspace_hidden(const fmx_model_config* cfg, int64_t n_tokens, const void* workspace,
                               const void** hidden) {
  FMX_RC(check_config(cfg));
  if (!workspace || !hidden) return fail(FMX_ERR_ARG, "NULL argument");
  if (n_tokens < 1 || n_tokens > 65536) return fail(FMX_ERR_SHAPE, "n_tokens=%lld", (long long)n_tokens);
  *hidden = model_layout(*cfg, n_tokens, static_cast<char*>(const_cast<void*>(workspace))).h;
  return ok();
}

int fmx_rope_table(float* rope_cs, int64_t n_pos, int64_t head_dim, float rope_theta, fmx_stream stream_) {
  if (n_pos < 1 || n_pos > kMaxPositions || head_dim < 2 || head_dim % 2 || head_dim > kAttnMaxHd)
    return fail(FMX_ERR_SHAPE, "n_pos must be in [1, %lld], head_dim even and at most %d",
                (long long)kMaxPositions, kAttnMaxHd);
  if (!rope_cs) return fail(FMX_ERR_ARG, "NULL table");
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  // (cos, sin) of p * theta^(-2i/hd) in fp64, rounded to fp32
  const int64_t half = head_dim / 2;
  std::vector<float> cs(static_cast<size_t>(n_pos * half * 2));
  for (int64_t i = 0; i < half; ++i) {
    const double inv = std::pow(static_cast<double>(rope_theta), -(2.0 * static_cast<double>(i)) /
                                                                     static_cast<double>(head_dim));
    for (int64_t p = 0; p < n_pos; ++p) {
      const double th = static_cast<double>(p) * inv;
      cs[(p * half + i) * 2] = static_cast<float>(std::cos(th));
      cs[(p * half + i) * 2 + 1] = static_cast<float>(std::sin(th));
    }
  }
  FMX_HIP(hipMemcpyAsync(rope_cs, cs.data(), cs.size() * 4, hipMemcpyHostToDevice, stream));
  FMX_HIP(hipStreamSynchronize(stream));  // the host table is released on return
  return ok();
}

int fmx_attention_decode(const void* qkv, int64_t batch, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                         const float* rope_cs, void* k_cache, void* v_cache, int64_t max_seq,
                         const int32_t* offsets, float scale, void* out, fmx_stream stream_) {
  if (batch < 0 || batch > 65535 || n_heads < 1 || n_kv_heads < 1 || n_heads % n_kv_heads || n_heads > 65535 ||
      head_dim < 8 || max_seq < 1)
    return fail(FMX_ERR_SHAPE, "batch, heads (n_heads a multiple of n_kv_heads), head_dim or max_seq");
  if (head_dim > kAttnSplitMaxHd || head_dim % 8 || kWave % (head_dim / 8) || max_seq > kAttnMaxSeq)
    return fail(FMX_ERR_UNSUPPORTED, "head_dim must be at most %d with 64 %% (head_dim / 8) == 0 and max_seq "
                "at most %lld", kAttnSplitMaxHd, (long long)kAttnMaxSeq);
  if (batch == 0) return ok();
  if (!qkv || !rope_cs || !k_cache || !v_cache || !offsets || !out) return fail(FMX_ERR_ARG, "NULL buffer");
  AttnArgs aa{};
  aa.qkv = static_cast<const uint16_t*>(qkv);
  aa.cs = rope_cs;
  aa.L = 1;
  aa.nh = static_cast<int>(n_heads);
  aa.nkv = static_cast<int>(n_kv_heads);
  aa.hd = static_cast<int>(head_dim);
  aa.kc = static_cast<uint16_t*>(k_cache);
  aa.vc = static_cast<uint16_t*>(v_cache);
  aa.max_seq = max_seq;
  aa.offs = offsets;
  aa.n_slots = static_cast<int>(batch);
  aa.scale = scale;
  aa.out = static_cast<uint16_t*>(out);
  aa.ldo = n_heads * head_dim;
  FMX_HIP(launch_attn(aa, static_cast<int>(batch), static_cast<hipStream_t>(stream_)));
  return ok();
}

int fmx_greedy_next(const void* logits, int64_t batch, int64_t vocab, int64_t row_stride, int32_t* ids,
                    int32_t* offsets, int32_t advance, fmx_stream stream_) {
  if (batch < 0 || vocab < 1 || row_stride < vocab) return fail(FMX_ERR_SHAPE, "batch/vocab/row_stride");
  if (batch == 0) return ok();
  if (!logits || !ids) return fail(FMX_ERR_ARG, "NULL buffer");
  GreedyArgs a{};
  a.logits = static_cast<const uint16_t*>(logits);
  a.V = vocab;
  a.ld = row_stride;
  a.ids = ids;
  a.offs = offsets;
  a.inc = advance;
  FMX_HIP(launch_greedy(a, static_cast<int>(batch), static_cast<hipStream_t>(stream_)));
  return ok();
}

}  // extern "C"
