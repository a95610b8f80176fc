// fmx_api.cpp -- the C-ABI of libfmx.so: argument checks with MLX's shape
// rules, workspace layout, and the launch sequence of each entry point.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/fmx.h"
#include "fmx_kernels.hpp"

using namespace fmx;

namespace {
thread_local std::string g_last_error;
}  // namespace

namespace fmx {
// the thread's last error message, shared with the decoder-stack entry points
int set_error(int status, const char* msg) {
  g_last_error = msg;
  return status;
}
void clear_error() { g_last_error.clear(); }
}  // namespace fmx

namespace {

int fail(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return status;
}

int ok() {
  g_last_error.clear();
  return FMX_OK;
}

#define FMX_HIP(expr)                                                              \
  do {                                                                             \
    hipError_t e_ = (expr);                                                        \
    if (e_ != hipSuccess)                                                          \
      return fail(FMX_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_));            \
  } while (0)

int64_t numel(const fmx_array& a) {
  int64_t n = 1;
  for (int i = 0; i < a.ndim; ++i) n *= a.shape[i];
  return n;
}

int64_t prod(const int64_t* s, int n) {
  int64_t p = 1;
  for (int i = 0; i < n; ++i) p *= s[i];
  return p;
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int check_array(const fmx_array* a, const char* name, int dtype, int min_ndim) {
  if (!a) return fail(FMX_ERR_ARG, "%s is NULL", name);
  if (a->ndim < min_ndim || a->ndim > FMX_MAX_NDIM)
    return fail(FMX_ERR_SHAPE, "%s: ndim %d (need %d..%d)", name, a->ndim, min_ndim, FMX_MAX_NDIM);
  for (int i = 0; i < a->ndim; ++i)
    if (a->shape[i] < 0) return fail(FMX_ERR_SHAPE, "%s: negative dim", name);
  if (dtype >= 0 && a->dtype != dtype)
    return fail(FMX_ERR_DTYPE, "%s: dtype %d, expected %d", name, a->dtype, dtype);
  if (!a->data && numel(*a) > 0) return fail(FMX_ERR_ARG, "%s: data is NULL", name);
  if (a->data && !aligned(a->data, 16)) return fail(FMX_ERR_ARG, "%s: data not 16-byte aligned", name);
  return FMX_OK;
}

int check_quant_args(int transpose, int group_size, int bits, const char* mode) {
  if (mode && std::strcmp(mode, "affine") != 0)
    return fail(FMX_ERR_UNSUPPORTED, "mode '%s' (only \"affine\")", mode);
  if (bits != 4) return fail(FMX_ERR_UNSUPPORTED, "bits=%d (only 4)", bits);
  if (group_size != 64) return fail(FMX_ERR_UNSUPPORTED, "group_size=%d (only 64)", group_size);
  if (!transpose) return fail(FMX_ERR_UNSUPPORTED, "transpose=false");
  return FMX_OK;
}

// Scratch arena over the caller's workspace (or a stream-ordered allocation).
struct Arena {
  char* base = nullptr;
  size_t cap = 0, used = 0;
  bool owned = false;
  hipStream_t stream = nullptr;
  void* take(size_t bytes) {
    void* p = base ? base + used : nullptr;
    used = static_cast<size_t>(align_up(static_cast<int64_t>(used + bytes), 256));
    return p;
  }
};

// Sizes a plan by running it against a null arena, then binds the real one.
struct WsGuard {
  Arena& a;
  explicit WsGuard(Arena& ar) : a(ar) {}
  ~WsGuard() {
    if (a.owned && a.base) (void)hipFreeAsync(a.base, a.stream);
  }
};

int bind_workspace(Arena& ar, void* ws, size_t ws_bytes, size_t need, hipStream_t stream) {
  ar.stream = stream;
  ar.used = 0;
  if (ws) {
    if (ws_bytes < need)
      return fail(FMX_ERR_WORKSPACE, "workspace %zu bytes, need %zu", ws_bytes, need);
    if (!aligned(ws, 256)) return fail(FMX_ERR_ARG, "workspace not 256-byte aligned");
    ar.base = static_cast<char*>(ws);
    ar.cap = ws_bytes;
    return FMX_OK;
  }
  if (need == 0) return FMX_OK;
  void* p = nullptr;
  FMX_HIP(hipMallocAsync(&p, need, stream));
  ar.base = static_cast<char*>(p);
  ar.cap = need;
  ar.owned = true;
  return FMX_OK;
}

// ---------------------------------------------------------------- MoE layout

constexpr int64_t kMoEMaxTokens = 65536;
// K slices of the shared expert's down projection (K = Is is long, N = H short)
constexpr int kSharedDownSplit = kDecSdSplit;
// the routers' arrival counters (1 + T / kRouterTok at most), then the
// decode combine's per-column-block counters
constexpr size_t kRouterCounterWords = kMoEMaxTokens / kRouterTok + 64;
constexpr size_t kCbCounterWords = static_cast<size_t>(kDecMaxColBlocks) * kDecCbStride;
constexpr size_t kGuCounterWords = static_cast<size_t>(kDecMaxE) * kDecGuWords;
// then the status word, on a line of its own
constexpr size_t kStatusWords = 64;
constexpr size_t kStatusOffsetWords = kRouterCounterWords + kCbCounterWords + kGuCounterWords;
// then the decode router's epoch word (a line of its own) and its logit
// words (64-bit: epoch and logit), which nothing else writes
constexpr size_t kEpochOffsetWords = kStatusOffsetWords + kStatusWords;
constexpr size_t kLgxOffsetWords = kEpochOffsetWords + 64;
constexpr size_t kLgxWords = 2 * static_cast<size_t>(kDecMaxT) * (kDecMaxE + 1);
constexpr size_t kCounterBytes = (kLgxOffsetWords + kLgxWords) * sizeof(uint32_t);

// Zeroes a workspace's counter block, then starts the decode router's epoch
// at 1: zeroed logit words carry epoch 0 and are never taken for a forward's.
hipError_t clear_counters(void* base, hipStream_t stream) {
  uint32_t* w = static_cast<uint32_t*>(base);
  const hipError_t e = launch_fill_u32(w, kCounterBytes / 4, 0u, stream);
  return e != hipSuccess ? e : launch_fill_u32(w + kEpochOffsetWords, 1, 1u, stream);
}

// bound of the decode down workgroups' wait (fmx_set_decode_wait_limit)
std::atomic<int> g_wait_polls{kDecWaitPolls};

struct MoELayout {
  uint32_t* counters;
  uint16_t* logits;
  double* lg_part;   // the prefill router's fp64 partial logits: aliases d (written later)
  int64_t lg_cap;    // doubles lg_part holds
  uint16_t* probs;
  uint32_t* inds;
  uint16_t* scores;
  uint32_t *order, *inv, *src, *idx, *offsets, *seg_n, *seg_exp, *seg_off, *sort_base, *seg;
  uint32_t *pass_n, *pass_tab;
  uint8_t* slots;
  float* sgate;
  uint16_t *xp, *h, *hs, *d;
  uint16_t *xh, *hh, *hsh;  // fp16 copies (P8 layout) of x, h, hs: prefill GEMM inputs
  uint32_t* f16_flag;
  uint32_t* dw;
  float* sd_part;
  size_t total;
};

MoELayout moe_layout(const fmx_moe_config& c, int64_t T, char* base) {
  Arena ar;
  ar.base = base;
  MoELayout L{};
  const int64_t E = c.num_experts, k = c.num_experts_per_tok, H = c.hidden_size;
  const int64_t I = c.moe_intermediate_size, Is = c.shared_expert_intermediate_size;
  const int64_t n = T * k;
  L.counters = static_cast<uint32_t*>(ar.take(kCounterBytes));
  L.logits = static_cast<uint16_t*>(ar.take(T * (E + 1) * 2));
  L.probs = static_cast<uint16_t*>(ar.take(T * E * 2));
  L.inds = static_cast<uint32_t*>(ar.take(n * 4));
  L.scores = static_cast<uint16_t*>(ar.take(n * 2));
  L.order = static_cast<uint32_t*>(ar.take(n * 4));
  L.inv = static_cast<uint32_t*>(ar.take(n * 4));
  L.src = static_cast<uint32_t*>(ar.take(n * 4));
  L.idx = static_cast<uint32_t*>(ar.take(n * 4));
  L.offsets = static_cast<uint32_t*>(ar.take((E + 1) * 4));
  L.seg_n = static_cast<uint32_t*>(ar.take(4));
  L.seg_exp = static_cast<uint32_t*>(ar.take(E * 4));
  L.seg_off = static_cast<uint32_t*>(ar.take((E + 1) * 4));
  L.sort_base = static_cast<uint32_t*>(ar.take(E * ((n + 63) / 64) * 4));
  L.seg = static_cast<uint32_t*>(ar.take((E + 1) * 4));
  L.pass_n = static_cast<uint32_t*>(ar.take(4));
  L.pass_tab = static_cast<uint32_t*>(ar.take(static_cast<int64_t>(max_passes(n, E)) * 8));
  L.slots = static_cast<uint8_t*>(ar.take(E * 16));
  L.sgate = static_cast<float*>(ar.take(T * 4));
  L.xp = static_cast<uint16_t*>(ar.take(T * H * 2));
  L.h = static_cast<uint16_t*>(ar.take(n * I * 2));
  L.hs = static_cast<uint16_t*>(ar.take(T * Is * 2));
  L.d = static_cast<uint16_t*>(ar.take(n * H * 2));
  L.lg_part = reinterpret_cast<double*>(L.d);  // consumed by the top-k kernel before d is written
  L.lg_cap = n * H * 2 / 8;
  L.sd_part = static_cast<float*>(ar.take(Is ? kSharedDownSplit * T * H * 4 : 0));
  L.f16_flag = static_cast<uint32_t*>(ar.take(4));
  L.xh = static_cast<uint16_t*>(ar.take(T * H * 2));
  L.hh = static_cast<uint16_t*>(ar.take(n * I * 2));
  L.hsh = static_cast<uint16_t*>(ar.take(T * Is * 2));
  // the decode kernels' down products (forwards of at most kDecMaxT tokens);
  // sized for min(T, kDecMaxT) at every T so that the layout only grows with T
  L.dw = static_cast<uint32_t*>(ar.take(std::min<int64_t>(T, kDecMaxT) * k * H * 4));
  L.total = ar.used;
  return L;
}

int check_moe_config(const fmx_moe_config* c) {
  if (!c) return fail(FMX_ERR_ARG, "cfg is NULL");
  if (c->quant_bits != 4) return fail(FMX_ERR_UNSUPPORTED, "quant_bits=%d (only 4)", c->quant_bits);
  if (c->quant_group_size != 64)
    return fail(FMX_ERR_UNSUPPORTED, "quant_group_size=%d (only 64)", c->quant_group_size);
  if (c->hidden_size <= 0 || c->hidden_size % 64)
    return fail(FMX_ERR_SHAPE, "hidden_size=%lld must be a positive multiple of 64",
                static_cast<long long>(c->hidden_size));
  if (c->moe_intermediate_size <= 0 || c->moe_intermediate_size % 64)
    return fail(FMX_ERR_SHAPE, "moe_intermediate_size=%lld must be a positive multiple of 64",
                static_cast<long long>(c->moe_intermediate_size));
  if (c->shared_expert_intermediate_size < 0 || c->shared_expert_intermediate_size % 64)
    return fail(FMX_ERR_SHAPE, "shared_expert_intermediate_size=%lld must be a multiple of 64",
                static_cast<long long>(c->shared_expert_intermediate_size));
  if (c->num_experts < 1 || c->num_experts > 1024)
    return fail(FMX_ERR_UNSUPPORTED, "num_experts=%lld (1..1024)", static_cast<long long>(c->num_experts));
  if (c->num_experts_per_tok < 1 || c->num_experts_per_tok > 16 ||
      c->num_experts_per_tok > c->num_experts)
    return fail(FMX_ERR_UNSUPPORTED, "num_experts_per_tok=%d (1..min(16, E))", c->num_experts_per_tok);
  if (c->activation_dtype != FMX_BF16 && c->activation_dtype != FMX_F16)
    return fail(FMX_ERR_DTYPE, "activation_dtype=%d (FMX_BF16 or FMX_F16)", c->activation_dtype);
  return FMX_OK;
}

bool qw_ok(const fmx_qweight& q) {
  return q.w && q.scales && q.biases && aligned(q.w, 16) && aligned(q.scales, 4) &&
         aligned(q.biases, 4);
}

// Offsets (bytes) of the parts of a packed layer (fmx_pack_expert_weights).
struct PackedLayout {
  int64_t gu_es, dn_es;           // bytes per routed expert: gate+up pair, down
  size_t gu, dn, sgu, sdn, total;
};

bool packable(const fmx_moe_config& c) {
  return c.hidden_size % 128 == 0 && c.moe_intermediate_size % 128 == 0 &&
         c.shared_expert_intermediate_size % 128 == 0;
}

PackedLayout packed_layout(const fmx_moe_config& c) {
  const int64_t H = c.hidden_size, E = c.num_experts, I = c.moe_intermediate_size;
  const int64_t Is = c.shared_expert_intermediate_size;
  PackedLayout P{};
  P.gu_es = (I / 16) * (H / 128) * kPackedBlockPair;
  P.dn_es = (H / 16) * (I / 128) * kPackedBlockSingle;
  P.gu = 0;
  P.dn = P.gu + static_cast<size_t>(align_up(E * P.gu_es, 256));
  P.sgu = P.dn + static_cast<size_t>(align_up(E * P.dn_es, 256));
  P.sdn = P.sgu + static_cast<size_t>(align_up((Is / 16) * (H / 128) * kPackedBlockPair, 256));
  P.total = P.sdn + static_cast<size_t>(align_up((H / 16) * (Is / 128) * kPackedBlockSingle, 256));
  return P;
}

// The router's rows and the shared-expert gate row (model.cpp:757-763,
// :787-799), bf16 or quantized; null rows when absent.
RouterRows router_rows(const fmx_moe_weights& w) {
  return RouterRows{w.router_w, static_cast<const uint16_t*>(w.router_scales),
                    static_cast<const uint16_t*>(w.router_biases)};
}
RouterRows sgate_rows(const fmx_moe_config& c, const fmx_moe_weights& w) {
  if (c.shared_expert_intermediate_size <= 0) return RouterRows{nullptr, nullptr, nullptr};
  return RouterRows{w.shared_expert_gate_w, static_cast<const uint16_t*>(w.shared_expert_gate_scales),
                    static_cast<const uint16_t*>(w.shared_expert_gate_biases)};
}

// A router row set is usable: bf16 rows 16-byte aligned, or 4-bit words
// 4-byte aligned with both scales and biases.
bool rows_ok(const RouterRows& r) {
  if (!r.w) return false;
  if (!r.s) return aligned(r.w, 16) && !r.b;
  return aligned(r.w, 4) && r.b && aligned(r.s, 2) && aligned(r.b, 2);
}

// Router launch shared by the block forward and fmx_moe_router_topk.
int run_router(const fmx_moe_config& c, const MoELayout& L, const void* x, int64_t T,
               const RouterRows& wr, const void* lbias, const RouterRows& wsg, uint32_t* inds,
               uint16_t* scores, uint16_t* probs, float* sgate, uint16_t* xp, bool want_sort,
               bool* sorted_in_router, hipStream_t stream, bool want_f16 = false) {
  RouterArgs a{};
  a.f16 = c.activation_dtype == FMX_F16 ? 1 : 0;
  a.x = static_cast<const uint16_t*>(x);
  a.wr = wr;
  a.lbias = static_cast<const uint16_t*>(lbias);
  a.wsg = wsg;
  a.T = static_cast<int>(T);
  a.H = static_cast<int>(c.hidden_size);
  a.E = static_cast<int>(c.num_experts);
  a.k = c.num_experts_per_tok;
  a.norm = c.norm_topk_prob ? 1 : 0;
  a.logits = L.logits;
  a.probs = probs;
  a.inds = inds;
  a.scores = scores;
  a.sgate = sgate;
  a.xp = xp;
  a.counters = L.counters;
  a.n_tt = static_cast<int>((T + kRouterTok - 1) / kRouterTok);
  // one token tile: a wave per column spreads the router weights over the
  // most CUs; many token tiles: 4 columns per wave re-read x 4x less
  a.cols_per_wave = a.n_tt > 1 ? 4 : 1;
  const int64_t cols_per_tile = 4 * a.cols_per_wave;
  a.n_ct = static_cast<int>((c.num_experts + (wsg.w ? 1 : 0) + cols_per_tile - 1) / cols_per_tile);
  const int64_t n = T * c.num_experts_per_tok;
  a.fuse_sort = want_sort && router_sort_fits(n, c.num_experts) ? 1 : 0;
  a.sort.order = L.order;
  a.sort.inv = L.inv;
  a.sort.src = L.src;
  a.sort.idx = L.idx;
  a.sort.offsets = L.offsets;
  a.sort.seg_n = L.seg_n;
  a.sort.seg_exp = L.seg_exp;
  a.sort.seg_off = L.seg_off;
  a.sort.base = L.sort_base;
  a.sort.pass_n = L.pass_n;
  a.sort.pass_tab = L.pass_tab;
  a.lg_part = L.lg_part;
  a.lg_split = router_lg_split(T, c.num_experts, L.lg_cap);
  if (want_f16) {  // the prefill GEMMs' fp16 copy of x and its range flag
    a.xh = L.xh;
    a.f16_flag = L.f16_flag;
  }
  if (T > kRouterManyMin || want_f16) {
    if (sorted_in_router) *sorted_in_router = false;
    FMX_HIP(launch_router_many(a, stream));
    if (xp) FMX_HIP(launch_permute_p8(static_cast<const uint16_t*>(x), T, c.hidden_size, xp, stream));
    return FMX_OK;
  }
  if (sorted_in_router) *sorted_in_router = a.fuse_sort != 0;
  FMX_HIP(launch_router(a, stream));
  return FMX_OK;
}

}  // namespace

namespace fmx {
// Byte offsets of a layer's packed parts (fmx_pack_expert_weights' layout),
// for the checkpoint loader, which packs expert by expert.
bool moe_packed_parts(const fmx_moe_config& c, size_t* gu, size_t* dn, size_t* sgu, size_t* sdn,
                      int64_t* gu_es, int64_t* dn_es) {
  if (check_moe_config(&c) || !packable(c)) return false;
  const PackedLayout P = packed_layout(c);
  *gu = P.gu;
  *dn = P.dn;
  *sgu = P.sgu;
  *sdn = P.sdn;
  *gu_es = P.gu_es;
  *dn_es = P.dn_es;
  return true;
}
}  // namespace fmx

extern "C" {

int fmx_abi_version(void) { return FMX_ABI_VERSION; }

const char* fmx_status_string(int s) {
  switch (s) {
    case FMX_OK: return "FMX_OK";
    case FMX_ERR_ARG: return "FMX_ERR_ARG";
    case FMX_ERR_SHAPE: return "FMX_ERR_SHAPE";
    case FMX_ERR_DTYPE: return "FMX_ERR_DTYPE";
    case FMX_ERR_UNSUPPORTED: return "FMX_ERR_UNSUPPORTED";
    case FMX_ERR_WORKSPACE: return "FMX_ERR_WORKSPACE";
    case FMX_ERR_HIP: return "FMX_ERR_HIP";
    default: return "FMX_ERR_UNKNOWN";
  }
}

const char* fmx_last_error(void) { return g_last_error.c_str(); }

// ---------------------------------------------------------------- quantized_matmul

int fmx_quantized_matmul_out_shape(const fmx_array* x, const fmx_array* w, int transpose,
                                   int group_size, int bits, fmx_array* out) {
  int rc;
  if ((rc = check_quant_args(transpose, group_size, bits, nullptr))) return rc;
  if (!x || !w || !out) return fail(FMX_ERR_ARG, "NULL argument");
  if (x->ndim < 2 || w->ndim != 2) return fail(FMX_ERR_SHAPE, "x.ndim >= 2 and w.ndim == 2 required");
  const int64_t K = x->shape[x->ndim - 1];
  if (w->shape[1] * 8 != K)
    return fail(FMX_ERR_SHAPE, "x K=%lld does not match w [%lld, %lld]", static_cast<long long>(K),
                static_cast<long long>(w->shape[0]), static_cast<long long>(w->shape[1]));
  out->ndim = x->ndim;
  for (int i = 0; i < x->ndim - 1; ++i) out->shape[i] = x->shape[i];
  out->shape[x->ndim - 1] = w->shape[0];
  out->dtype = x->dtype == FMX_F16 ? FMX_F16 : FMX_BF16;
  return ok();
}

namespace {

// Calls the standalone ops send to the prefill GEMM on the MLX-layout
// weights (fmx_prefill.hip): K in whole 128-k units, N in whole 16-row
// tiles, and at least min_rows rows; other calls go to the grouped GEMM
// (fmx_qgemm.hip), which reads x as it is. Measured at Qwen1.5-MoE shapes
// (K 2048): gather_qmm's passes are faster from 17 rows on (8 tokens x
// top-4: 28 against 40 us; 512 x 4: 65 against 360 us), quantized_matmul's
// from 32 rows (17-24 rows: 18.8 against 16.1-17.7 us).
constexpr int64_t kQmmPfMinRows = 32;
constexpr int64_t kGatherPfMinRows = 17;
bool op_uses_pf(int64_t rows, int64_t N, int64_t K, int64_t min_rows) {
  return rows >= min_rows && rows <= (1 << 20) && N % 16 == 0 && K % 128 == 0;
}

// The prefill GEMM's operand copies of x_rows rows (bf16 P8, fp16 Q8) and
// the copy blocks' overflow words.
struct PfRows {
  uint16_t* xp;
  uint16_t* xq;
  uint32_t* ovf;
  int n_ovf;
};
PfRows take_pf_rows(Arena& ar, int64_t x_rows, int64_t K) {
  PfRows r;
  r.xp = static_cast<uint16_t*>(ar.take(x_rows * K * 2));
  r.xq = static_cast<uint16_t*>(ar.take(x_rows * K * 2));
  r.n_ovf = ops_prologue_ovf_words(x_rows * (K / 8));
  r.ovf = static_cast<uint32_t*>(ar.take(static_cast<int64_t>(r.n_ovf) * 4));
  return r;
}

// One set of the prefill GEMM over MLX-layout weights [n_exp][N][K/8]
// (scales / biases [n_exp][N][K/64]), output rows of N bf16.
PfSet mlx_set(const fmx_array* w, const fmx_array* scales, const fmx_array* biases, const PfRows& xr,
              int64_t K, int64_t N, uint16_t* out) {
  PfSet s{};
  s.mw = static_cast<const uint32_t*>(w->data);
  s.ms = static_cast<const uint16_t*>(scales->data);
  s.mb = static_cast<const uint16_t*>(biases->data);
  s.x = xr.xp;
  s.xh = xr.xq;
  s.ldx = K;
  s.out = out;
  s.ldo = N;
  s.nt = static_cast<int>(N / 16);
  s.nu = static_cast<int>(K / 128);
  s.n_exp = 1;
  return s;
}

hipError_t launch_mlx_pf(const PfSet& s, const PfRows& xr, hipStream_t stream) {
  PfArgs pa{};
  pa.s1 = s;
  pa.n_items1 = pf_items(pa.s1, false);
  pa.f16_flag = xr.ovf;
  pa.n_flag = xr.n_ovf;
  pa.flag_in = 1u;
  pa.flag_out = 0u;
  return launch_pf(pa, false, stream);
}

}  // namespace

size_t fmx_quantized_matmul_workspace_size(const fmx_array* x, const fmx_array* w) {
  if (!x || x->ndim < 1) return 0;
  const int64_t K = x->shape[x->ndim - 1];
  const int64_t rows = K ? numel(*x) / K : 0;
  Arena ar;
  const int64_t min_rows = x->dtype == FMX_F16 ? 1 : kQmmPfMinRows;
  if (w && w->ndim == 2 && op_uses_pf(rows, w->shape[0], K, min_rows)) take_pf_rows(ar, rows, K);
  return ar.used;
}

int fmx_quantized_matmul(const fmx_array* x, const fmx_array* w, const fmx_array* scales,
                         const fmx_array* biases, int transpose, int group_size, int bits,
                         const char* mode, fmx_array* out, void* workspace,
                         size_t workspace_bytes, fmx_stream stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  int rc;
  if ((rc = check_quant_args(transpose, group_size, bits, mode))) return rc;
  if ((rc = check_array(x, "x", -1, 2))) return rc;
  if (x->dtype != FMX_BF16 && x->dtype != FMX_F16) return fail(FMX_ERR_DTYPE, "x must be bfloat16 or float16");
  const bool f16 = x->dtype == FMX_F16;
  if ((rc = check_array(w, "w", FMX_U32, 2))) return rc;
  if ((rc = check_array(scales, "scales", x->dtype, 2))) return rc;
  if (!biases) return fail(FMX_ERR_ARG, "affine mode requires biases");
  if ((rc = check_array(biases, "biases", x->dtype, 2))) return rc;
  if ((rc = check_array(out, "out", x->dtype, 2))) return rc;
  if (w->ndim != 2) return fail(FMX_ERR_UNSUPPORTED, "w with batch dims (use gather_qmm)");
  const int64_t K = x->shape[x->ndim - 1], N = w->shape[0];
  if (K % 64) return fail(FMX_ERR_SHAPE, "K=%lld not a multiple of 64", static_cast<long long>(K));
  if (w->shape[1] * 8 != K) return fail(FMX_ERR_SHAPE, "w.shape[1]*8 != K");
  if (scales->ndim != 2 || scales->shape[0] != N || scales->shape[1] != K / 64 ||
      biases->ndim != 2 || biases->shape[0] != N || biases->shape[1] != K / 64)
    return fail(FMX_ERR_SHAPE, "scales/biases must be [N, K/64]");
  fmx_array expect{};
  if ((rc = fmx_quantized_matmul_out_shape(x, w, transpose, group_size, bits, &expect))) return rc;
  if (out->ndim != expect.ndim || std::memcmp(out->shape, expect.shape, sizeof(int64_t) * out->ndim))
    return fail(FMX_ERR_SHAPE, "out shape mismatch");
  const int64_t rows = numel(*x) / K;
  if (rows == 0 || N == 0) return ok();
  if (rows > (1ll << 30)) return fail(FMX_ERR_UNSUPPORTED, "too many rows");

  Arena ar;
  WsGuard guard(ar);
  if ((rc = bind_workspace(ar, workspace, workspace_bytes,
                           fmx_quantized_matmul_workspace_size(x, w), stream)))
    return rc;
  // float16 rows run the prefill GEMM at every row count (its fp16 operands
  // are the values themselves); other shapes are not taken in float16
  if (f16 && !op_uses_pf(rows, N, K, 1))
    return fail(FMX_ERR_UNSUPPORTED, "float16 quantized_matmul needs K %% 128 == 0 and N %% 16 == 0");
  if (op_uses_pf(rows, N, K, f16 ? 1 : kQmmPfMinRows)) {
    const PfRows xr = take_pf_rows(ar, rows, K);
    OpsPrologue pro{};
    pro.x = static_cast<const uint16_t*>(x->data);
    pro.x_f16 = f16 ? 1 : 0;
    pro.n_oct = rows * (K / 8);
    pro.xp = xr.xp;
    pro.xq = xr.xq;
    pro.ovf = xr.ovf;
    FMX_HIP(launch_ops_prologue(pro, stream));
    PfSet s = mlx_set(w, scales, biases, xr, K, N, static_cast<uint16_t*>(out->data));
    s.io_f16 = f16 ? 1 : 0;
    s.rows_static = s.rows_max = s.x_rows = static_cast<int>(rows);
    // fewer work items than CUs: passes of 32 rows instead (twice the items,
    // each with half the rows; Qwen1.5 shared shape [5632, 2048]: 48-256 rows
    // 8-16 % faster, 512 rows, 352 items of 64, 9 % slower so)
    const int64_t groups = (N / 16 + 7) / 8;
    if (rows > 32 && ((rows + kPassRows - 1) / kPassRows) * groups < 256) s.pass_rows = 32;
    FMX_HIP(launch_mlx_pf(s, xr, stream));
    return ok();
  }
  QGemmProblem p{};
  p.x = static_cast<const uint16_t*>(x->data);
  p.x_natural = 1;
  p.ldx = K;
  p.rows_static = static_cast<int>(rows);
  p.max_seg = 1;
  p.w0 = static_cast<const uint32_t*>(w->data);
  p.s0 = static_cast<const uint16_t*>(scales->data);
  p.b0 = static_cast<const uint16_t*>(biases->data);
  p.N = static_cast<int>(N);
  p.K = static_cast<int>(K);
  p.out = static_cast<uint16_t*>(out->data);
  p.ldo = N;
  p.n_exp = 1;
  p.rows_max = p.x_rows = p.out_rows = static_cast<int>(rows);
  p.max_rows_per_seg = static_cast<int>(rows);
  FMX_HIP(launch_qgemm(p, nullptr, stream));
  return ok();
}

// ---------------------------------------------------------------- gather_qmm

namespace {

struct GatherPlan {
  int64_t K, N, M, E, n_x;
  int ndim;  // batch ndim
  int64_t batch[FMX_MAX_NDIM];
  int64_t nb;
};

// MLX: batch(x) = x.shape[:-2], batch(w) = w.shape[:-2]; default lhs/rhs are
// arange(prod(batch)).reshape(batch); out = broadcast(lhs, rhs) + [M, N].
int gather_plan(const fmx_array* x, const fmx_array* w, const fmx_array* lhs,
                const fmx_array* rhs, GatherPlan* p) {
  if (!x || !w) return fail(FMX_ERR_ARG, "NULL argument");
  if (x->ndim < 2 || w->ndim < 2) return fail(FMX_ERR_SHAPE, "x and w need ndim >= 2");
  p->K = x->shape[x->ndim - 1];
  p->M = x->shape[x->ndim - 2];
  p->N = w->shape[w->ndim - 2];
  if (w->shape[w->ndim - 1] * 8 != p->K) return fail(FMX_ERR_SHAPE, "w.shape[-1]*8 != K");
  p->E = prod(w->shape, w->ndim - 2);
  p->n_x = prod(x->shape, x->ndim - 2);
  const int64_t* ls = lhs ? lhs->shape : x->shape;
  const int ln = lhs ? lhs->ndim : x->ndim - 2;
  const int64_t* rs = rhs ? rhs->shape : w->shape;
  const int rn = rhs ? rhs->ndim : w->ndim - 2;
  const int nd = std::max(ln, rn);
  if (nd > FMX_MAX_NDIM - 2) return fail(FMX_ERR_SHAPE, "too many batch dims");
  for (int i = 0; i < nd; ++i) {
    const int li = i - (nd - ln), ri = i - (nd - rn);
    const int64_t a = li >= 0 ? ls[li] : 1, b = ri >= 0 ? rs[ri] : 1;
    if (a != b && a != 1 && b != 1)
      return fail(FMX_ERR_SHAPE, "lhs/rhs index shapes do not broadcast");
    p->batch[i] = (a == 1) ? b : a;
  }
  p->ndim = nd;
  p->nb = prod(p->batch, nd);
  return FMX_OK;
}

void fill_bcast(const GatherPlan& p, const fmx_array* idx, const int64_t* dflt_shape,
                int dflt_ndim, BcastArgs* b) {
  const int64_t* s = idx ? idx->shape : dflt_shape;
  const int n = idx ? idx->ndim : dflt_ndim;
  b->src = idx ? idx->data : nullptr;
  b->is_i32 = idx && idx->dtype == FMX_I32;
  b->ndim = p.ndim;
  b->n = p.nb;
  int64_t stride = 1;
  for (int i = p.ndim - 1; i >= 0; --i) {
    const int si = i - (p.ndim - n);
    b->out_shape[i] = p.batch[i];
    const int64_t dim = si >= 0 ? s[si] : 1;
    b->src_stride[i] = (dim == 1) ? 0 : stride;
    stride *= dim;
  }
}

// gather_qmm's workspace, in the order fmx_gather_qmm takes it
struct GatherWs {
  uint32_t *lhs_flat, *rhs_flat, *keys, *order, *offsets, *seg_n, *seg_exp, *seg_off, *sbase, *row_map;
  uint32_t *pass_n, *pass_tab, *flag;  // prefill GEMM only
  PfRows xr;                           // prefill GEMM only
};
GatherWs take_gather_ws(Arena& ar, const GatherPlan& p, bool pf) {
  const int64_t rows = p.nb * p.M;
  GatherWs g{};
  g.lhs_flat = static_cast<uint32_t*>(ar.take(p.nb * 4));
  g.rhs_flat = static_cast<uint32_t*>(ar.take(p.nb * 4));
  g.keys = static_cast<uint32_t*>(ar.take(rows * 4));
  g.order = static_cast<uint32_t*>(ar.take(rows * 4));
  g.offsets = static_cast<uint32_t*>(ar.take((p.E + 1) * 4));
  g.seg_n = static_cast<uint32_t*>(ar.take(4));
  g.seg_exp = static_cast<uint32_t*>(ar.take(p.E * 4));
  g.seg_off = static_cast<uint32_t*>(ar.take((p.E + 1) * 4));
  g.sbase = static_cast<uint32_t*>(ar.take(p.E * ((rows + 63) / 64) * 4));
  g.row_map = static_cast<uint32_t*>(ar.take(rows * 4));
  if (pf) {
    g.pass_n = static_cast<uint32_t*>(ar.take(4));
    g.pass_tab = static_cast<uint32_t*>(ar.take(static_cast<int64_t>(max_passes(rows, p.E)) * 8));
    g.xr = take_pf_rows(ar, p.n_x * p.M, p.K);
    g.flag = static_cast<uint32_t*>(ar.take(4));
  }
  return g;
}

bool gather_uses_pf(const GatherPlan& p, bool f16) {
  return op_uses_pf(p.nb * p.M, p.N, p.K, f16 ? 1 : kGatherPfMinRows);
}

size_t gather_ws(const GatherPlan& p, bool f16) {
  Arena ar;
  take_gather_ws(ar, p, gather_uses_pf(p, f16));
  return ar.used;
}

}  // namespace

int fmx_gather_qmm_out_shape(const fmx_array* x, const fmx_array* w, const fmx_array* lhs,
                             const fmx_array* rhs, int transpose, int group_size, int bits,
                             fmx_array* out) {
  int rc;
  if ((rc = check_quant_args(transpose, group_size, bits, nullptr))) return rc;
  if (!out) return fail(FMX_ERR_ARG, "out is NULL");
  GatherPlan p;
  if ((rc = gather_plan(x, w, lhs, rhs, &p))) return rc;
  out->ndim = p.ndim + 2;
  for (int i = 0; i < p.ndim; ++i) out->shape[i] = p.batch[i];
  out->shape[p.ndim] = p.M;
  out->shape[p.ndim + 1] = p.N;
  out->dtype = x->dtype == FMX_F16 ? FMX_F16 : FMX_BF16;
  return ok();
}

size_t fmx_gather_qmm_workspace_size(const fmx_array* x, const fmx_array* w,
                                     const fmx_array* lhs, const fmx_array* rhs) {
  GatherPlan p;
  if (gather_plan(x, w, lhs, rhs, &p)) return 0;
  return gather_ws(p, x && x->dtype == FMX_F16);
}

int fmx_gather_qmm(const fmx_array* x, const fmx_array* w, const fmx_array* scales,
                   const fmx_array* biases, const fmx_array* lhs, const fmx_array* rhs,
                   int transpose, int group_size, int bits, const char* mode,
                   int sorted_indices, fmx_array* out, void* workspace, size_t workspace_bytes,
                   fmx_stream stream_) {
  (void)sorted_indices;  // a hint; the rows are always grouped by expert
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  int rc;
  if ((rc = check_quant_args(transpose, group_size, bits, mode))) return rc;
  if ((rc = check_array(x, "x", -1, 2))) return rc;
  if (x->dtype != FMX_BF16 && x->dtype != FMX_F16) return fail(FMX_ERR_DTYPE, "x must be bfloat16 or float16");
  const bool f16 = x->dtype == FMX_F16;
  if ((rc = check_array(w, "w", FMX_U32, 2))) return rc;
  if ((rc = check_array(scales, "scales", x->dtype, 2))) return rc;
  if (!biases) return fail(FMX_ERR_ARG, "affine mode requires biases");
  if ((rc = check_array(biases, "biases", x->dtype, 2))) return rc;
  if ((rc = check_array(out, "out", x->dtype, 2))) return rc;
  if (lhs) {
    if ((rc = check_array(lhs, "lhs_indices", -1, 0))) return rc;
    if (lhs->dtype != FMX_U32 && lhs->dtype != FMX_I32)
      return fail(FMX_ERR_DTYPE, "lhs_indices must be uint32 or int32");
  }
  if (rhs) {
    if ((rc = check_array(rhs, "rhs_indices", -1, 0))) return rc;
    if (rhs->dtype != FMX_U32 && rhs->dtype != FMX_I32)
      return fail(FMX_ERR_DTYPE, "rhs_indices must be uint32 or int32");
  }
  GatherPlan p;
  if ((rc = gather_plan(x, w, lhs, rhs, &p))) return rc;
  if (p.K % 64) return fail(FMX_ERR_SHAPE, "K=%lld not a multiple of 64", static_cast<long long>(p.K));
  if (scales->ndim != w->ndim || biases->ndim != w->ndim)
    return fail(FMX_ERR_SHAPE, "scales/biases must have w's batch dims");
  for (int i = 0; i < w->ndim - 1; ++i)
    if (scales->shape[i] != w->shape[i] || biases->shape[i] != w->shape[i])
      return fail(FMX_ERR_SHAPE, "scales/biases batch dims differ from w");
  if (scales->shape[w->ndim - 1] != p.K / 64 || biases->shape[w->ndim - 1] != p.K / 64)
    return fail(FMX_ERR_SHAPE, "scales/biases last dim must be K/64");
  fmx_array expect{};
  if ((rc = fmx_gather_qmm_out_shape(x, w, lhs, rhs, transpose, group_size, bits, &expect)))
    return rc;
  if (out->ndim != expect.ndim || std::memcmp(out->shape, expect.shape, sizeof(int64_t) * out->ndim))
    return fail(FMX_ERR_SHAPE, "out shape mismatch");
  const int64_t rows = p.nb * p.M;
  if (rows == 0 || p.N == 0) return ok();
  if (p.E == 0 || p.n_x == 0) return fail(FMX_ERR_SHAPE, "empty w or x batch with non-empty output");
  if (!sort_fits(rows, p.E))
    return fail(FMX_ERR_UNSUPPORTED, "rows=%lld x experts=%lld exceed the sort's limits",
                static_cast<long long>(rows), static_cast<long long>(p.E));

  Arena ar;
  WsGuard guard(ar);
  if (f16 && !gather_uses_pf(p, true))
    return fail(FMX_ERR_UNSUPPORTED, "float16 gather_qmm needs K %% 128 == 0 and N %% 16 == 0");
  if ((rc = bind_workspace(ar, workspace, workspace_bytes, gather_ws(p, f16), stream))) return rc;
  const bool pf = gather_uses_pf(p, f16);
  const GatherWs g = take_gather_ws(ar, p, pf);

  // one launch: both index broadcasts (rhs also as per-row sort keys) and,
  // for the prefill GEMM, the operand copies of x
  OpsPrologue pro{};
  fill_bcast(p, lhs, x->shape, x->ndim - 2, &pro.lhs);
  pro.lhs.dst = g.lhs_flat;
  fill_bcast(p, rhs, w->shape, w->ndim - 2, &pro.rhs);
  pro.rhs.dst = g.rhs_flat;
  pro.rhs.M = static_cast<int>(p.M);
  pro.rhs.dst_rows = g.keys;
  if (pf) {
    pro.x = static_cast<const uint16_t*>(x->data);
    pro.x_f16 = f16 ? 1 : 0;
    pro.n_oct = p.n_x * p.M * (p.K / 8);
    pro.xp = g.xr.xp;
    pro.xq = g.xr.xq;
    pro.ovf = g.xr.ovf;
  }
  FMX_HIP(launch_ops_prologue(pro, stream));
  SortOut so{};
  so.order = g.order;
  so.offsets = g.offsets;
  so.seg_n = g.seg_n;
  so.seg_exp = g.seg_exp;
  so.seg_off = g.seg_off;
  so.base = g.sbase;
  so.pass_n = g.pass_n;
  so.pass_tab = g.pass_tab;
  // sorted row r is entry order[r] = b * M + m: it reads x row
  // row_map[r] = lhs[b] * M + m and writes output row order[r]
  so.row_map = g.row_map;
  so.row_lhs = g.lhs_flat;
  so.row_m = static_cast<int>(p.M);
  so.x_rows = static_cast<int>(p.n_x * p.M);
  if (pf) {  // one overflow word for the GEMM from the copy blocks' words
    so.ovf = g.xr.ovf;
    so.n_ovf = g.xr.n_ovf;
    so.flag = g.flag;
  }
  FMX_HIP(launch_sort(g.keys, static_cast<int>(rows), 1, static_cast<int>(p.E), so, stream));

  if (pf) {
    PfSet s = mlx_set(w, scales, biases, g.xr, p.K, p.N, static_cast<uint16_t*>(out->data));
    s.io_f16 = f16 ? 1 : 0;
    s.row_map = g.row_map;
    s.out_map = g.order;
    s.pass_n = g.pass_n;
    s.pass_tab = g.pass_tab;
    s.max_pass = max_passes(rows, p.E);
    s.n_exp = static_cast<int>(p.E);
    s.rows_max = static_cast<int>(rows);
    s.x_rows = static_cast<int>(p.n_x * p.M);
    PfRows one = g.xr;
    one.ovf = g.flag;
    one.n_ovf = 1;
    FMX_HIP(launch_mlx_pf(s, one, stream));
    return ok();
  }
  QGemmProblem q{};
  q.x = static_cast<const uint16_t*>(x->data);
  q.x_natural = 1;
  q.ldx = p.K;
  q.row_map = g.row_map;
  q.out_map = g.order;
  q.seg_n = g.seg_n;
  q.seg_exp = g.seg_exp;
  q.seg_off = g.seg_off;
  q.max_seg = static_cast<int>(std::min<int64_t>(p.E, rows));
  q.w0 = static_cast<const uint32_t*>(w->data);
  q.s0 = static_cast<const uint16_t*>(scales->data);
  q.b0 = static_cast<const uint16_t*>(biases->data);
  q.ew = p.N * (p.K / 8);
  q.es = p.N * (p.K / 64);
  q.N = static_cast<int>(p.N);
  q.K = static_cast<int>(p.K);
  q.out = static_cast<uint16_t*>(out->data);
  q.ldo = p.N;
  q.n_exp = static_cast<int>(p.E);
  q.rows_max = q.out_rows = static_cast<int>(rows);
  q.x_rows = static_cast<int>(p.n_x * p.M);
  q.max_rows_per_seg = static_cast<int>(rows);
  FMX_HIP(launch_qgemm(q, nullptr, stream));
  return ok();
}

// ---------------------------------------------------------------- quantize

int fmx_quantize(const fmx_array* w, int group_size, int bits, const char* mode, fmx_array* wq,
                 fmx_array* scales, fmx_array* biases, fmx_stream stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  int rc;
  if ((rc = check_quant_args(1, group_size, bits, mode))) return rc;
  if ((rc = check_array(w, "w", FMX_BF16, 1))) return rc;
  if ((rc = check_array(wq, "wq", FMX_U32, 1))) return rc;
  if ((rc = check_array(scales, "scales", FMX_BF16, 1))) return rc;
  if ((rc = check_array(biases, "biases", FMX_BF16, 1))) return rc;
  const int nd = w->ndim;
  const int64_t K = w->shape[nd - 1];
  if (K % 64) return fail(FMX_ERR_SHAPE, "last dim %lld not a multiple of 64", static_cast<long long>(K));
  if (wq->ndim != nd || scales->ndim != nd || biases->ndim != nd)
    return fail(FMX_ERR_SHAPE, "outputs must have w's ndim");
  for (int i = 0; i < nd - 1; ++i)
    if (wq->shape[i] != w->shape[i] || scales->shape[i] != w->shape[i] || biases->shape[i] != w->shape[i])
      return fail(FMX_ERR_SHAPE, "output leading dims differ from w");
  if (wq->shape[nd - 1] != K / 8 || scales->shape[nd - 1] != K / 64 || biases->shape[nd - 1] != K / 64)
    return fail(FMX_ERR_SHAPE, "wq last dim must be K/8, scales/biases K/64");
  FMX_HIP(launch_quantize(static_cast<const uint16_t*>(w->data), numel(*w) / 64,
                          static_cast<uint32_t*>(wq->data), static_cast<uint16_t*>(scales->data),
                          static_cast<uint16_t*>(biases->data), stream));
  return ok();
}

int fmx_dequantize(const fmx_array* wq, const fmx_array* scales, const fmx_array* biases,
                   int group_size, int bits, const char* mode, fmx_array* out, fmx_stream stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  int rc;
  if ((rc = check_quant_args(1, group_size, bits, mode))) return rc;
  if ((rc = check_array(wq, "wq", FMX_U32, 1))) return rc;
  if ((rc = check_array(scales, "scales", FMX_BF16, 1))) return rc;
  if (!biases) return fail(FMX_ERR_ARG, "affine mode requires biases");
  if ((rc = check_array(biases, "biases", FMX_BF16, 1))) return rc;
  if ((rc = check_array(out, "out", FMX_BF16, 1))) return rc;
  const int nd = wq->ndim;
  const int64_t K = wq->shape[nd - 1] * 8;
  if (out->ndim != nd || scales->ndim != nd || biases->ndim != nd)
    return fail(FMX_ERR_SHAPE, "ndim mismatch");
  for (int i = 0; i < nd - 1; ++i)
    if (out->shape[i] != wq->shape[i] || scales->shape[i] != wq->shape[i] || biases->shape[i] != wq->shape[i])
      return fail(FMX_ERR_SHAPE, "leading dims differ");
  if (out->shape[nd - 1] != K || scales->shape[nd - 1] != K / 64 || biases->shape[nd - 1] != K / 64)
    return fail(FMX_ERR_SHAPE, "last dims inconsistent");
  if (K % 64) return fail(FMX_ERR_SHAPE, "K not a multiple of 64");
  FMX_HIP(launch_dequantize(static_cast<const uint32_t*>(wq->data),
                            static_cast<const uint16_t*>(scales->data),
                            static_cast<const uint16_t*>(biases->data), numel(*out) / 64,
                            static_cast<uint16_t*>(out->data), stream));
  return ok();
}

int fmx_stack_experts(const void* const* src, int64_t n_experts, size_t bytes, void* dst,
                      fmx_stream stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (!src || !dst || n_experts < 0) return fail(FMX_ERR_ARG, "NULL argument");
  for (int64_t e = 0; e < n_experts; ++e) {
    if (!src[e]) return fail(FMX_ERR_ARG, "expert %lld source is NULL", static_cast<long long>(e));
    FMX_HIP(hipMemcpyAsync(static_cast<char*>(dst) + e * bytes, src[e], bytes,
                           hipMemcpyDeviceToDevice, stream));
  }
  return ok();
}

// ---------------------------------------------------------------- MoE block

size_t fmx_moe_workspace_size(const fmx_moe_config* cfg, int64_t max_tokens) {
  if (check_moe_config(cfg) || max_tokens < 0 || max_tokens > kMoEMaxTokens) return 0;
  return moe_layout(*cfg, max_tokens, nullptr).total;
}

size_t fmx_moe_packed_size(const fmx_moe_config* cfg) {
  if (check_moe_config(cfg) || !packable(*cfg)) return 0;
  return packed_layout(*cfg).total;
}

int fmx_pack_expert_weights(const fmx_moe_config* cfg, const fmx_moe_weights* src, void* packed,
                            size_t packed_bytes, fmx_stream stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  int rc;
  if ((rc = check_moe_config(cfg))) return rc;
  const fmx_moe_config& c = *cfg;
  if (!packable(c))
    return fail(FMX_ERR_UNSUPPORTED, "packing needs H, I and Is to be multiples of 128");
  if (!src || !packed) return fail(FMX_ERR_ARG, "NULL argument");
  if (!aligned(packed, 256)) return fail(FMX_ERR_ARG, "packed not 256-byte aligned");
  const PackedLayout PL = packed_layout(c);
  if (packed_bytes < PL.total)
    return fail(FMX_ERR_WORKSPACE, "packed buffer %zu bytes, need %zu", packed_bytes, PL.total);
  const bool has_sh = c.shared_expert_intermediate_size > 0;
  if (!qw_ok(src->gate) || !qw_ok(src->up) || !qw_ok(src->down))
    return fail(FMX_ERR_ARG, "expert weights NULL or misaligned");
  if (has_sh && (!qw_ok(src->shared_gate) || !qw_ok(src->shared_up) || !qw_ok(src->shared_down)))
    return fail(FMX_ERR_ARG, "shared expert weights NULL or misaligned");
  const int64_t H = c.hidden_size, E = c.num_experts, I = c.moe_intermediate_size;
  const int64_t Is = c.shared_expert_intermediate_size;
  uint8_t* dst = static_cast<uint8_t*>(packed);
  auto pack = [&](const fmx_qweight& a, const fmx_qweight* b, int64_t n_exp, int64_t N, int64_t K,
                  size_t off, int64_t es) -> hipError_t {
    PackArgs pa{};
    pa.w0 = static_cast<const uint32_t*>(a.w);
    pa.s0 = static_cast<const uint16_t*>(a.scales);
    pa.b0 = static_cast<const uint16_t*>(a.biases);
    if (b) {
      pa.w1 = static_cast<const uint32_t*>(b->w);
      pa.s1 = static_cast<const uint16_t*>(b->scales);
      pa.b1 = static_cast<const uint16_t*>(b->biases);
    }
    pa.n_exp = n_exp;
    pa.N = static_cast<int>(N);
    pa.nt = static_cast<int>(N / 16);
    pa.nu = static_cast<int>(K / 128);
    pa.dst = dst + off;
    pa.dst_estride = es;
    return launch_pack(pa, stream);
  };
  FMX_HIP(pack(src->gate, &src->up, E, I, H, PL.gu, PL.gu_es));
  FMX_HIP(pack(src->down, nullptr, E, H, I, PL.dn, PL.dn_es));
  if (has_sh) {
    FMX_HIP(pack(src->shared_gate, &src->shared_up, 1, Is, H, PL.sgu, 0));
    FMX_HIP(pack(src->shared_down, nullptr, 1, H, Is, PL.sdn, 0));
  }
  return ok();
}

int fmx_moe_workspace_init(void* workspace, size_t workspace_bytes, fmx_stream stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (!workspace) return fail(FMX_ERR_ARG, "workspace is NULL");
  if (workspace_bytes < kCounterBytes)
    return fail(FMX_ERR_WORKSPACE, "workspace %zu bytes < %zu", workspace_bytes, kCounterBytes);
  FMX_HIP(clear_counters(workspace, stream));
  return ok();
}

int fmx_moe_workspace_status(const void* workspace, size_t workspace_bytes, uint32_t* status,
                             int clear, fmx_stream stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (!workspace || !status) return fail(FMX_ERR_ARG, "workspace or status is NULL");
  if (workspace_bytes < kCounterBytes)
    return fail(FMX_ERR_WORKSPACE, "workspace %zu bytes < %zu", workspace_bytes, kCounterBytes);
  uint32_t* word = static_cast<uint32_t*>(const_cast<void*>(workspace)) + kStatusOffsetWords;
  FMX_HIP(hipStreamSynchronize(stream));
  FMX_HIP(hipMemcpy(status, word, 4, hipMemcpyDeviceToHost));
  if (clear) {
    // after a wait that ran out, late router columns may have tagged their
    // logit words with the next epoch, and late stores may have left counters
    // and flags set: the whole counter block back to its initial state (the
    // status word included) makes the next forward start clean
    FMX_HIP(clear_counters(const_cast<void*>(workspace), stream));
  }
  return ok();
}

int64_t fmx_set_decode_wait_limit(int64_t polls) {
  const int v = static_cast<int>(std::max<int64_t>(std::min<int64_t>(polls, INT32_MAX), 0));
  return g_wait_polls.exchange(polls < 0 ? kDecWaitPolls : v);
}

int fmx_moe_workspace_routing(const fmx_moe_config* cfg, int64_t n_tokens, const void* workspace,
                              const uint32_t** inds, const void** scores, const void** probs,
                              const uint32_t** order, const uint32_t** inv,
                              const uint32_t** src, const uint32_t** idx,
                              const uint32_t** expert_offsets) {
  int rc;
  if ((rc = check_moe_config(cfg))) return rc;
  if (!workspace) return fail(FMX_ERR_ARG, "workspace is NULL");
  if (n_tokens < 0 || n_tokens > kMoEMaxTokens) return fail(FMX_ERR_SHAPE, "n_tokens out of range");
  const MoELayout L = moe_layout(*cfg, n_tokens, static_cast<char*>(const_cast<void*>(workspace)));
  if (inds) *inds = L.inds;
  if (scores) *scores = L.scores;
  if (probs) *probs = L.probs;
  if (order) *order = L.order;
  if (inv) *inv = L.inv;
  if (src) *src = L.src;
  if (idx) *idx = L.idx;
  if (expert_offsets) *expert_offsets = L.offsets;
  return ok();
}

int fmx_moe_forward_path(const fmx_moe_config* cfg, int64_t T, int has_packed) {
  int rc;
  if ((rc = check_moe_config(cfg))) return -rc;
  if (T < 0 || T > kMoEMaxTokens) return -fail(FMX_ERR_SHAPE, "n_tokens out of range");
  if (cfg->activation_dtype == FMX_F16 && (!has_packed || !packable(*cfg)))
    return -fail(FMX_ERR_UNSUPPORTED, "float16 blocks run on packed weights");
  if (!has_packed || !packable(*cfg)) return 0;
  DecodeArgs da{};
  da.T = static_cast<int>(T);
  da.H = static_cast<int>(cfg->hidden_size);
  da.E = static_cast<int>(cfg->num_experts);
  da.k = cfg->num_experts_per_tok;
  da.I = static_cast<int>(cfg->moe_intermediate_size);
  da.Is = static_cast<int>(cfg->shared_expert_intermediate_size);
  return decode_plan(da) ? 1 : 2;
}

namespace {
int moe_forward(const fmx_moe_config* cfg, const fmx_moe_weights* w, const void* x, int64_t T,
                void* y, void* workspace, size_t workspace_bytes, fmx_stream stream_,
                void* const* stage_events, int n_stages, const MoEInputNorm* nin = nullptr);
}  // namespace



int fmx_moe_block_forward(const fmx_moe_config* cfg, const fmx_moe_weights* w, const void* x,
                          int64_t T, void* y, void* workspace, size_t workspace_bytes,
                          fmx_stream stream_) {
  return moe_forward(cfg, w, x, T, y, workspace, workspace_bytes, stream_, nullptr, 4);
}

int fmx_moe_block_forward_profiled(const fmx_moe_config* cfg, const fmx_moe_weights* w,
                                   const void* x, int64_t T, void* y, void* workspace,
                                   size_t workspace_bytes, fmx_stream stream_,
                                   void* const* stage_events) {
  return moe_forward(cfg, w, x, T, y, workspace, workspace_bytes, stream_, stage_events, 4);
}

int fmx_moe_block_forward_partial(const fmx_moe_config* cfg, const fmx_moe_weights* w,
                                  const void* x, int64_t T, void* y, void* workspace,
                                  size_t workspace_bytes, fmx_stream stream_, int n_stages) {
  if (n_stages < 1 || n_stages > 4) return fail(FMX_ERR_ARG, "n_stages=%d (1..4)", n_stages);
  return moe_forward(cfg, w, x, T, y, workspace, workspace_bytes, stream_, nullptr, n_stages);
}

}  // extern "C"

// ---------------------------------------------------------------- allocation-free forward
//
// A fixed device array serves as the workspace of fmx_moe_block_forward_noalloc.
// Each device the library runs on holds its own copy for the life of the
// process. Host code never passes the array's name to a kernel or a copy: the
// name is a host-side stand-in. The device address comes from
// hipGetSymbolAddress, taken once per device with that device current.
namespace {

static_assert(FMX_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size is a multiple of 256 bytes");
static __device__ __align__(256) uint8_t scratch[FMX_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`; on the first call for a device,
// also clears the completion counters at its start (on `stream`, by a fill
// kernel, so that a caller capturing a graph records no memset node).
int scratch_for_current_device(hipStream_t stream, void** out) {
  int dev = 0;
  FMX_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail(FMX_ERR_UNSUPPORTED, "device index %d", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    FMX_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(FMX_ERR_HIP, "hipGetSymbolAddress(scratch) gave NULL");
    FMX_HIP(clear_counters(p, stream));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FMX_OK;
}

}  // namespace

extern "C" int fmx_moe_block_forward_noalloc(const fmx_moe_config* cfg, const fmx_moe_weights* w,
                                             const void* x, int64_t T, void* y,
                                             fmx_stream stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  int rc;
  if ((rc = check_moe_config(cfg))) return rc;
  if (T < 0 || T > kMoEMaxTokens) return fail(FMX_ERR_SHAPE, "n_tokens=%lld out of range", static_cast<long long>(T));
  if (T == 0) return ok();
  const size_t need = moe_layout(*cfg, T, nullptr).total;
  if (need > static_cast<size_t>(FMX_NOALLOC_SCRATCH_BYTES))
    return fail(FMX_ERR_UNSUPPORTED,
                "a forward of %lld tokens needs %zu bytes of workspace, more than the %d-byte "
                "fixed scratch of the allocation-free forward",
                static_cast<long long>(T), need, FMX_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if ((rc = scratch_for_current_device(stream, &ws))) return rc;
  return moe_forward(cfg, w, x, T, y, ws, FMX_NOALLOC_SCRATCH_BYTES, stream_, nullptr, 4);
}

namespace {

int moe_forward(const fmx_moe_config* cfg, const fmx_moe_weights* w, const void* x, int64_t T,
                void* y, void* workspace, size_t workspace_bytes, fmx_stream stream_,
                void* const* stage_events, int n_stages, const MoEInputNorm* nin) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  auto mark = [&](int i) -> hipError_t {
    return stage_events ? hipEventRecord(static_cast<hipEvent_t>(stage_events[i]), stream)
                        : hipSuccess;
  };
  int rc;
  if ((rc = check_moe_config(cfg))) return rc;
  if (!w) return fail(FMX_ERR_ARG, "NULL argument");
  if (T < 0 || T > kMoEMaxTokens) return fail(FMX_ERR_SHAPE, "n_tokens=%lld out of range", static_cast<long long>(T));
  if (T == 0) return ok();  // nothing to run: x and y may be NULL (empty tensors)
  if (!x || !y) return fail(FMX_ERR_ARG, "NULL argument");
  const fmx_moe_config& c = *cfg;
  const bool has_sh = c.shared_expert_intermediate_size > 0;
  const RouterRows wr = router_rows(*w), wsg = sgate_rows(c, *w);
  if (!rows_ok(wr)) return fail(FMX_ERR_ARG, "router_w (or its scales/biases) NULL or misaligned");
  if (has_sh && !rows_ok(wsg))
    return fail(FMX_ERR_ARG, "shared_expert_gate_w (or its scales/biases) NULL or misaligned");
  // packed weights: the forward reads the experts from there only
  const bool use_packed = w->packed != nullptr;
  const bool f16 = c.activation_dtype == FMX_F16;
  if (f16 && !use_packed) return fail(FMX_ERR_UNSUPPORTED, "float16 blocks run on packed weights");
  if (f16 && nin) return fail(FMX_ERR_UNSUPPORTED, "the input norm in K1 is bf16 only");
  if (nin && (!use_packed || T > kDecNinMaxT || !nin->h || !nin->w || !aligned(nin->h, 16) || !aligned(nin->w, 16)))
    return fail(FMX_ERR_UNSUPPORTED, "input norm in K1: decode forwards of up to %d tokens on packed weights",
                kDecNinMaxT);
  if (use_packed) {
    if (!packable(c)) return fail(FMX_ERR_ARG, "packed weights given for a config that cannot be packed");
    if (!aligned(w->packed, 256)) return fail(FMX_ERR_ARG, "packed not 256-byte aligned");
    if (w->packed_bytes < packed_layout(c).total)
      return fail(FMX_ERR_WORKSPACE, "packed_bytes %zu, the config needs %zu", w->packed_bytes,
                  packed_layout(c).total);
  } else {
    if (!qw_ok(w->gate) || !qw_ok(w->up) || !qw_ok(w->down))
      return fail(FMX_ERR_ARG, "expert weights NULL or misaligned");
    if (has_sh && (!qw_ok(w->shared_gate) || !qw_ok(w->shared_up) || !qw_ok(w->shared_down)))
      return fail(FMX_ERR_ARG, "shared expert weights NULL or misaligned");
  }
  if (!aligned(x, 16) || !aligned(y, 16)) return fail(FMX_ERR_ARG, "x/y not 16-byte aligned");
  const int64_t H = c.hidden_size, E = c.num_experts, k = c.num_experts_per_tok;
  const int64_t I = c.moe_intermediate_size, Is = c.shared_expert_intermediate_size;
  const int64_t n = T * k;
  if (!sort_fits(n, E))
    return fail(FMX_ERR_UNSUPPORTED, "T*k=%lld with E=%lld exceeds the sort's limits",
                static_cast<long long>(n), static_cast<long long>(E));

  Arena ar;
  WsGuard guard(ar);
  const size_t need = moe_layout(c, T, nullptr).total;
  if ((rc = bind_workspace(ar, workspace, workspace_bytes, need, stream))) return rc;
  if (ar.owned) FMX_HIP(clear_counters(ar.base, stream));
  const MoELayout L = moe_layout(c, T, ar.base);

  // decode batches (T <= 16) on packed weights: two kernels, combine included
  if (use_packed) {
    const PackedLayout PL = packed_layout(c);
    const uint8_t* pk = static_cast<const uint8_t*>(w->packed);
    DecodeArgs da{};
    da.T = static_cast<int>(T);
    da.H = static_cast<int>(H);
    da.E = static_cast<int>(E);
    da.k = static_cast<int>(k);
    da.I = static_cast<int>(I);
    da.Is = static_cast<int>(Is);
    da.norm = c.norm_topk_prob ? 1 : 0;
    da.f16 = f16 ? 1 : 0;
    da.x = static_cast<const uint16_t*>(x);
    da.wr = wr;
    da.lbias = static_cast<const uint16_t*>(w->router_logit_bias);
    da.wsg = wsg;
    da.gu = pk + PL.gu;
    da.gu_es = PL.gu_es;
    da.dn = pk + PL.dn;
    da.dn_es = PL.dn_es;
    da.sgu = pk + PL.sgu;
    da.sdn = pk + PL.sdn;
    da.logits = L.logits;
    da.hs = L.hs;
    da.h = L.h;
    da.dw = L.dw;
    da.sd_part = L.sd_part;
    da.inds = L.inds;
    da.scores = L.scores;
    da.probs = L.probs;
    da.sgate = has_sh ? L.sgate : nullptr;
    da.sort = SortOut{L.order, L.inv, L.src, L.idx, L.offsets, nullptr, nullptr, nullptr, L.sort_base};
    da.seg = L.seg;
    da.slots = L.slots;
    da.counter = L.counters;
    da.cb_counter = L.counters + kRouterCounterWords;
    da.gu_counter = L.counters + kRouterCounterWords + kCbCounterWords;
    da.status = L.counters + kStatusOffsetWords;
    da.epoch = L.counters + kEpochOffsetWords;
    da.lgx = reinterpret_cast<uint64_t*>(L.counters + kLgxOffsetWords);
    da.wait_polls = g_wait_polls.load(std::memory_order_relaxed);
    da.y = static_cast<uint16_t*>(y);
    if (nin) {
      da.nin = nin->h;
      da.nin_w = nin->w;
      da.nin_eps = nin->eps;
      da.x_out = static_cast<uint16_t*>(const_cast<void*>(x));
    }
    const bool dec = decode_plan(da);
    if (nin && !dec) return fail(FMX_ERR_UNSUPPORTED, "input norm in K1: shapes outside the decode kernels");
    if (dec) {
      FMX_HIP(mark(0));
      FMX_HIP(launch_decode_k1(da, stream));
      FMX_HIP(mark(1));
      if (n_stages < 2) return ok();
      if (n_stages < 3) {  // gate/up alone
        FMX_HIP(launch_decode_k2(da, stream));
        FMX_HIP(mark(2));
        return ok();
      }
      // gate/up, down and combine in one grid
      FMX_HIP(launch_decode_k23(da, stream));
      FMX_HIP(mark(2));
      FMX_HIP(mark(3));
      FMX_HIP(mark(4));
      return ok();
    }

    // prefill batches: router (+ sort and pass table), gate/up grid, down
    // grid, combine
    FMX_HIP(mark(0));
    bool sorted = false;
    if ((rc = run_router(c, L, x, T, wr, w->router_logit_bias, wsg, L.inds, L.scores, L.probs,
                         has_sh ? L.sgate : nullptr, nullptr, true, &sorted, stream, true)))
      return rc;
    if (!sorted) {
      SortOut so{L.order, L.inv, L.src, L.idx, L.offsets, L.seg_n, L.seg_exp, L.seg_off,
                 L.sort_base, L.pass_n, L.pass_tab};
      FMX_HIP(launch_sort(L.inds, static_cast<int>(n), static_cast<int>(k), static_cast<int>(E), so, stream));
    }
    FMX_HIP(mark(1));
    if (n_stages < 2) return ok();

    const int mp = max_passes(n, E);
    auto routed = [&](const uint8_t* wp, int64_t es, const uint16_t* xr, const uint16_t* xrh,
                      int64_t ldx, const uint32_t* row_map, uint16_t* out, uint16_t* outh,
                      int64_t ldo, int64_t N, int64_t K) {
      PfSet s{};
      s.w = wp;
      s.es = es;
      s.x = xr;
      s.xh = xrh;
      s.ldx = ldx;
      s.row_map = row_map;
      s.out = out;
      s.outh = outh;
      s.ldo = ldo;
      s.nt = static_cast<int>(N / 16);
      s.nu = static_cast<int>(K / 128);
      s.pass_n = L.pass_n;
      s.pass_tab = L.pass_tab;
      s.max_pass = mp;
      s.n_exp = static_cast<int>(E);
      s.rows_max = static_cast<int>(n);
      s.x_rows = static_cast<int>(row_map ? T : n);
      s.io_f16 = f16 ? 1 : 0;
      return s;
    };
    auto shared = [&](const uint8_t* wp, const uint16_t* xr, const uint16_t* xrh, int64_t ldx,
                      uint16_t* out, uint16_t* outh, int64_t ldo, int64_t N, int64_t K) {
      PfSet s{};
      s.w = wp;
      s.x = xr;
      s.xh = xrh;
      s.ldx = ldx;
      s.out = out;
      s.outh = outh;
      s.ldo = ldo;
      s.nt = static_cast<int>(N / 16);
      s.nu = static_cast<int>(K / 128);
      s.rows_static = s.rows_max = s.x_rows = static_cast<int>(T);
      s.n_exp = 1;
      s.io_f16 = f16 ? 1 : 0;
      return s;
    };
    const uint16_t* xb = static_cast<const uint16_t*>(x);
    int sd_split = 0;
    {
      PfArgs pa{};
      pa.s1 = routed(pk + PL.gu, PL.gu_es, xb, L.xh, H, L.src, L.h, L.hh, I, I, H);
      pa.n_items1 = pf_items(pa.s1, true);
      if (has_sh) {
        pa.s0 = shared(pk + PL.sgu, xb, L.xh, H, L.hs, L.hsh, Is, Is, H);
        pa.n_items0 = pf_items(pa.s0, true);
      }
      // a float16 block's rows are fp16 already: no range flag, no exact path
      pa.f16_flag = L.f16_flag;
      pa.flag_in = f16 ? 0u : kF16FlagX;
      pa.flag_out = f16 ? 0u : kF16FlagH;
      FMX_HIP(launch_pf(pa, true, stream));
    }
    FMX_HIP(mark(2));
    if (n_stages < 3) return ok();
    {
      PfArgs pa{};
      pa.s1 = routed(pk + PL.dn, PL.dn_es, L.h, L.hh, I, nullptr, L.d, nullptr, H, H, I);
      pa.n_items1 = pf_items(pa.s1, false);
      if (has_sh) {
        // up to 256 tokens (four 64-token passes) the shared down
        // projection's K (Is) is cut into slices about as long as the routed
        // experts' (I), fp32 partial sums added by the combine: its few long
        // items otherwise outlast the routed ones (Qwen1.5 shape: 17 tokens
        // 77 -> 63 us per layer, 256 tokens 121 -> 113 us; at 512 tokens the
        // slices' extra items cost 4 %)
        pa.s0 = shared(pk + PL.sdn, L.hs, L.hsh, Is, nullptr, nullptr, H, H, Is);
        pa.s0.out32 = L.sd_part;
        pa.s0.ksplit = T > 4 * kPassRows
                           ? 1
                           : static_cast<int>(std::min<int64_t>(std::max<int64_t>((Is + I - 1) / I, 1),
                                                                std::min<int64_t>(kSharedDownSplit, Is / 128)));
        pa.s0.part_stride = T * H;
        pa.n_items0 = pf_items(pa.s0, false);
        sd_split = pa.s0.ksplit;
      }
      pa.f16_flag = L.f16_flag;
      pa.flag_in = f16 ? 0u : kF16FlagH;
      pa.flag_out = 0u;
      FMX_HIP(launch_pf(pa, false, stream));
    }
    FMX_HIP(mark(3));
    if (n_stages < 4) return ok();
    CombineArgs cb{};
    cb.d = L.d;
    cb.inv = L.inv;
    cb.scores = L.scores;
    cb.sd_part = has_sh ? L.sd_part : nullptr;
    cb.sd_ksplit = sd_split;
    cb.sgate = has_sh ? L.sgate : nullptr;
    cb.y = static_cast<uint16_t*>(y);
    cb.T = static_cast<int>(T);
    cb.k = static_cast<int>(k);
    cb.H = static_cast<int>(H);
    cb.f16 = f16 ? 1 : 0;
    FMX_HIP(launch_combine(cb, stream));
    FMX_HIP(mark(4));
    return ok();
  }

  // 1. router + top-k (+ sort when it fits in the router's last workgroup)
  FMX_HIP(mark(0));
  bool sorted = false;
  if ((rc = run_router(c, L, x, T, wr, w->router_logit_bias, wsg, L.inds, L.scores, L.probs,
                       has_sh ? L.sgate : nullptr, L.xp, true, &sorted, stream)))
    return rc;
  if (!sorted) {
    SortOut so{L.order, L.inv, L.src, L.idx, L.offsets, L.seg_n, L.seg_exp, L.seg_off, L.sort_base};
    FMX_HIP(launch_sort(L.inds, static_cast<int>(n), static_cast<int>(k), static_cast<int>(E), so, stream));
  }
  FMX_HIP(mark(1));
  if (n_stages < 2) return ok();

  {
  // 2. gate/up + SwiGLU: routed experts over the sorted rows, and the shared expert
  QGemmProblem gu{};
  gu.x = L.xp;
  gu.ldx = H;
  gu.row_map = L.src;
  gu.seg_n = L.seg_n;
  gu.seg_exp = L.seg_exp;
  gu.seg_off = L.seg_off;
  gu.max_seg = static_cast<int>(std::min(E, n));
  gu.w0 = static_cast<const uint32_t*>(w->gate.w);
  gu.s0 = static_cast<const uint16_t*>(w->gate.scales);
  gu.b0 = static_cast<const uint16_t*>(w->gate.biases);
  gu.w1 = static_cast<const uint32_t*>(w->up.w);
  gu.s1 = static_cast<const uint16_t*>(w->up.scales);
  gu.b1 = static_cast<const uint16_t*>(w->up.biases);
  gu.ew = I * (H / 8);
  gu.es = I * (H / 64);
  gu.N = static_cast<int>(I);
  gu.K = static_cast<int>(H);
  gu.out = L.h;
  gu.ldo = I;
  gu.dual = 1;
  gu.out_p8 = 1;
  gu.n_exp = static_cast<int>(E);
  gu.rows_max = gu.out_rows = static_cast<int>(n);
  gu.x_rows = static_cast<int>(T);
  gu.max_rows_per_seg = static_cast<int>(T);  // a token picks an expert at most once
  QGemmProblem sgu{};
  if (has_sh) {
    sgu.x = L.xp;
    sgu.ldx = H;
    sgu.rows_static = static_cast<int>(T);
    sgu.max_seg = 1;
    sgu.w0 = static_cast<const uint32_t*>(w->shared_gate.w);
    sgu.s0 = static_cast<const uint16_t*>(w->shared_gate.scales);
    sgu.b0 = static_cast<const uint16_t*>(w->shared_gate.biases);
    sgu.w1 = static_cast<const uint32_t*>(w->shared_up.w);
    sgu.s1 = static_cast<const uint16_t*>(w->shared_up.scales);
    sgu.b1 = static_cast<const uint16_t*>(w->shared_up.biases);
    sgu.N = static_cast<int>(Is);
    sgu.K = static_cast<int>(H);
    sgu.out = L.hs;
    sgu.ldo = Is;
    sgu.dual = 1;
    sgu.out_p8 = 1;
    sgu.n_exp = 1;
    sgu.rows_max = sgu.x_rows = sgu.out_rows = static_cast<int>(T);
    sgu.max_rows_per_seg = static_cast<int>(T);
  }
  FMX_HIP(launch_qgemm(gu, has_sh ? &sgu : nullptr, stream));
  FMX_HIP(mark(2));
  if (n_stages < 3) return ok();

  // 3. down: routed rows (sorted order) and the shared expert
  QGemmProblem dn{};
  dn.x = L.h;
  dn.ldx = I;
  dn.seg_n = L.seg_n;
  dn.seg_exp = L.seg_exp;
  dn.seg_off = L.seg_off;
  dn.max_seg = gu.max_seg;
  dn.w0 = static_cast<const uint32_t*>(w->down.w);
  dn.s0 = static_cast<const uint16_t*>(w->down.scales);
  dn.b0 = static_cast<const uint16_t*>(w->down.biases);
  dn.ew = H * (I / 8);
  dn.es = H * (I / 64);
  dn.N = static_cast<int>(H);
  dn.K = static_cast<int>(I);
  dn.out = L.d;
  dn.ldo = H;
  dn.n_exp = static_cast<int>(E);
  dn.rows_max = dn.x_rows = dn.out_rows = static_cast<int>(n);
  dn.max_rows_per_seg = static_cast<int>(T);
  QGemmProblem sdn{};
  if (has_sh) {
    sdn.x = L.hs;
    sdn.ldx = Is;
    sdn.rows_static = static_cast<int>(T);
    sdn.max_seg = 1;
    sdn.w0 = static_cast<const uint32_t*>(w->shared_down.w);
    sdn.s0 = static_cast<const uint16_t*>(w->shared_down.scales);
    sdn.b0 = static_cast<const uint16_t*>(w->shared_down.biases);
    sdn.N = static_cast<int>(H);
    sdn.K = static_cast<int>(Is);
    sdn.ldo = H;
    sdn.n_exp = 1;
    sdn.rows_max = sdn.x_rows = sdn.out_rows = static_cast<int>(T);
    sdn.max_rows_per_seg = static_cast<int>(T);
    sdn.ksplit = kSharedDownSplit;
    sdn.out_part = L.sd_part;
  }
  FMX_HIP(launch_qgemm(dn, has_sh ? &sdn : nullptr, stream));
  FMX_HIP(mark(3));
  if (n_stages < 4) return ok();
  }

  // 4. top-k weighted combine + gated shared expert
  CombineArgs cb{};
  cb.d = L.d;
  cb.inv = L.inv;
  cb.scores = L.scores;
  cb.sd = nullptr;
  cb.sd_part = has_sh ? L.sd_part : nullptr;
  cb.sd_ksplit = kSharedDownSplit;
  cb.sgate = has_sh ? L.sgate : nullptr;
  cb.y = static_cast<uint16_t*>(y);
  cb.T = static_cast<int>(T);
  cb.k = static_cast<int>(k);
  cb.H = static_cast<int>(H);
  FMX_HIP(launch_combine(cb, stream));
  FMX_HIP(mark(4));
  return ok();
}

}  // namespace

extern "C" {

int fmx_moe_router_topk(const fmx_moe_config* cfg, const void* x, int64_t T, const void* router_w,
                        const void* lbias, uint32_t* inds, void* scores, void* probs,
                        void* workspace, size_t workspace_bytes, fmx_stream stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  int rc;
  if ((rc = check_moe_config(cfg))) return rc;
  if (T < 0 || T > kMoEMaxTokens) return fail(FMX_ERR_SHAPE, "n_tokens out of range");
  if (T == 0) return ok();  // nothing to run: the buffers may be NULL (empty tensors)
  if (!x || !router_w || !inds || !scores) return fail(FMX_ERR_ARG, "NULL argument");
  if (!aligned(x, 16) || !aligned(router_w, 16)) return fail(FMX_ERR_ARG, "x/router_w not 16-byte aligned");
  Arena ar;
  WsGuard guard(ar);
  const size_t need = moe_layout(*cfg, T, nullptr).total;
  if ((rc = bind_workspace(ar, workspace, workspace_bytes, need, stream))) return rc;
  if (ar.owned) FMX_HIP(clear_counters(ar.base, stream));
  const MoELayout L = moe_layout(*cfg, T, ar.base);
  return run_router(*cfg, L, x, T, RouterRows{router_w, nullptr, nullptr}, lbias,
                    RouterRows{nullptr, nullptr, nullptr}, inds, static_cast<uint16_t*>(scores),
                    static_cast<uint16_t*>(probs), nullptr, nullptr, false, nullptr, stream);
}

int fmx_moe_router_topk_ex(const fmx_moe_config* cfg, const void* x, int64_t T, const fmx_moe_weights* w,
                           uint32_t* inds, void* scores, void* probs, void* shared_gate_out,
                           void* workspace, size_t workspace_bytes, fmx_stream stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  int rc;
  if ((rc = check_moe_config(cfg))) return rc;
  if (T < 0 || T > kMoEMaxTokens) return fail(FMX_ERR_SHAPE, "n_tokens out of range");
  if (T == 0) return ok();  // nothing to run: the buffers may be NULL (empty tensors)
  if (!x || !w || !inds || !scores) return fail(FMX_ERR_ARG, "NULL argument");
  if (!aligned(x, 16)) return fail(FMX_ERR_ARG, "x not 16-byte aligned");
  const RouterRows wr = router_rows(*w);
  if (!rows_ok(wr))
    return fail(FMX_ERR_ARG, "router_w: bf16 rows 16-byte aligned, or 4-bit words with both "
                             "router_scales and router_biases");
  RouterRows wsg{nullptr, nullptr, nullptr};
  if (shared_gate_out) {
    wsg = RouterRows{w->shared_expert_gate_w, static_cast<const uint16_t*>(w->shared_expert_gate_scales),
                     static_cast<const uint16_t*>(w->shared_expert_gate_biases)};
    if (!rows_ok(wsg))
      return fail(FMX_ERR_ARG, "shared_gate_out needs shared_expert_gate_w: a bf16 row 16-byte aligned, "
                               "or 4-bit words with both scales and biases");
  }
  Arena ar;
  WsGuard guard(ar);
  const size_t need = moe_layout(*cfg, T, nullptr).total;
  if ((rc = bind_workspace(ar, workspace, workspace_bytes, need, stream))) return rc;
  if (ar.owned) FMX_HIP(clear_counters(ar.base, stream));
  const MoELayout L = moe_layout(*cfg, T, ar.base);
  if ((rc = run_router(*cfg, L, x, T, wr, w->router_logit_bias, wsg, inds, static_cast<uint16_t*>(scores),
                       static_cast<uint16_t*>(probs), shared_gate_out ? L.sgate : nullptr, nullptr, false,
                       nullptr, stream)))
    return rc;
  if (shared_gate_out)
    FMX_HIP(launch_f32_bf16(L.sgate, T, static_cast<uint16_t*>(shared_gate_out), stream,
                            cfg->activation_dtype == FMX_F16));
  return FMX_OK;
}

size_t fmx_moe_sort_workspace_size(int64_t T, int32_t k, int64_t E) {
  if (T < 0 || k < 1 || E < 1) return 0;
  const int64_t n = T * k;
  Arena sizer;
  sizer.take((E + 1) * 4);
  sizer.take(E * ((n + 63) / 64) * 4);
  return sizer.used;
}

int fmx_moe_sort(const uint32_t* inds, int64_t T, int32_t k, int64_t E, uint32_t* order,
                 uint32_t* inv, uint32_t* src, uint32_t* idx, uint32_t* expert_offsets,
                 void* workspace, size_t workspace_bytes, fmx_stream stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (!inds && T > 0) return fail(FMX_ERR_ARG, "inds is NULL");
  if (T < 0 || k < 1 || E < 1) return fail(FMX_ERR_SHAPE, "bad sizes");
  const int64_t n = T * k;
  if (n == 0) return ok();
  if (!sort_fits(n, E)) return fail(FMX_ERR_UNSUPPORTED, "n=%lld, E=%lld exceed the sort's limits",
                                    static_cast<long long>(n), static_cast<long long>(E));
  Arena ar;
  WsGuard guard(ar);
  int rc;
  if ((rc = bind_workspace(ar, workspace, workspace_bytes, fmx_moe_sort_workspace_size(T, k, E),
                           stream)))
    return rc;
  uint32_t* off_scratch = static_cast<uint32_t*>(ar.take((E + 1) * 4));
  uint32_t* base = static_cast<uint32_t*>(ar.take(E * ((n + 63) / 64) * 4));
  SortOut so{order, inv, src, idx, expert_offsets ? expert_offsets : off_scratch,
             nullptr, nullptr, nullptr, base};
  FMX_HIP(launch_sort(inds, static_cast<int>(n), k, static_cast<int>(E), so, stream));
  return ok();
}

}  // extern "C"

int fmx::moe_block_forward_nin(const fmx_moe_config* cfg, const fmx_moe_weights* w, const MoEInputNorm& nin,
                               void* x_out, int64_t T, void* y, void* workspace, size_t workspace_bytes,
                               hipStream_t stream) {
  return moe_forward(cfg, w, x_out, T, y, workspace, workspace_bytes, stream, nullptr, 4, &nin);
}
