// fmx_nh.cpp -- the Nemotron-H MoE block (include/fmx_nemotron.h): the
// argument checks, the packed layout with I and Is padded to whole 128-k
// units, the workspace layout, and the launch sequence:
//
//   logits_kernel + topk_kernel (mode 1)  logits, sigmoid/group selection,
//                                         fp32 scores, the fp16 copy of x
//   sort_kernel                           expert-sorted rows and passes
//   pf_gemm<false> (act)                  fc1 + relu^2 of the routed passes
//                                         and the shared up projection
//   pf_gemm<false> (out32)                fc2 and the shared down, fp32
//   nh_combine_kernel                     weighted k-sum + shared, bf16
//
// Reference: server/src/nemotron_h.cpp:1010-1111 (moe_block), :54-63
// (relu2), :443-470 (the layer's cached weights).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>

#include "../../include/fmx_nemotron.h"
#include "fmx_kernels.hpp"

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

constexpr int64_t kNhMaxTokens = 65536;
constexpr int kNhMaxGroups = 64;  // the selection keeps one group score per lane

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int check_config(const fmx_nh_moe_config* c) {
  if (!c) return fail(FMX_ERR_ARG, "cfg is NULL");
  if (c->quant_bits != 4) return fail(FMX_ERR_UNSUPPORTED, "quant_bits=%d (only 4)", c->quant_bits);
  if (c->quant_group_size != 64)
    return fail(FMX_ERR_UNSUPPORTED, "quant_group_size=%d (only 64)", c->quant_group_size);
  if (c->hidden_size <= 0 || c->hidden_size % 128)
    return fail(FMX_ERR_SHAPE, "hidden_size=%lld must be a positive multiple of 128",
                static_cast<long long>(c->hidden_size));
  if (c->moe_intermediate_size <= 0 || c->moe_intermediate_size % 64)
    return fail(FMX_ERR_SHAPE, "moe_intermediate_size=%lld must be a positive multiple of 64",
                static_cast<long long>(c->moe_intermediate_size));
  if (c->moe_shared_expert_intermediate_size < 0 || c->moe_shared_expert_intermediate_size % 64)
    return fail(FMX_ERR_SHAPE, "moe_shared_expert_intermediate_size=%lld must be a multiple of 64",
                static_cast<long long>(c->moe_shared_expert_intermediate_size));
  const int64_t E = c->n_routed_experts;
  if (E < 1 || E > 1024) return fail(FMX_ERR_UNSUPPORTED, "n_routed_experts=%lld (1..1024)", static_cast<long long>(E));
  if (c->num_experts_per_tok < 1 || c->num_experts_per_tok > 16 || c->num_experts_per_tok > E)
    return fail(FMX_ERR_UNSUPPORTED, "num_experts_per_tok=%d (1..min(16, E))", c->num_experts_per_tok);
  if (c->n_group < 1 || c->n_group > kNhMaxGroups || E % c->n_group)
    return fail(FMX_ERR_UNSUPPORTED, "n_group=%d must divide n_routed_experts and be <= %d", c->n_group,
                kNhMaxGroups);
  if (c->n_group > 1 && (E / c->n_group < 2 || c->topk_group < 1 || c->topk_group > c->n_group))
    return fail(FMX_ERR_UNSUPPORTED, "n_group=%d, topk_group=%d: groups of at least 2 experts, "
                "1 <= topk_group <= n_group", c->n_group, c->topk_group);
  return FMX_OK;
}

// Packed layout: fc1 of every expert (Ip/16 tiles x H/128 units), fc2 of
// every expert (H/16 tiles x Ip/128 units), the shared up, the shared down.
struct NhPacked {
  int64_t Ip, Isp;
  int64_t fc1_es, fc2_es;
  size_t fc1, fc2, sup, sdn, total;
};

NhPacked nh_packed(const fmx_nh_moe_config& c) {
  NhPacked P{};
  const int64_t H = c.hidden_size, E = c.n_routed_experts;
  P.Ip = align_up(c.moe_intermediate_size, 128);
  P.Isp = align_up(c.moe_shared_expert_intermediate_size, 128);
  P.fc1_es = (P.Ip / 16) * (H / 128) * kPackedBlockSingle;
  P.fc2_es = (H / 16) * (P.Ip / 128) * kPackedBlockSingle;
  P.fc1 = 0;
  P.fc2 = P.fc1 + static_cast<size_t>(align_up(E * P.fc1_es, 256));
  P.sup = P.fc2 + static_cast<size_t>(align_up(E * P.fc2_es, 256));
  P.sdn = P.sup + static_cast<size_t>(align_up((P.Isp / 16) * (H / 128) * kPackedBlockSingle, 256));
  P.total = P.sdn + static_cast<size_t>(align_up((H / 16) * (P.Isp / 128) * kPackedBlockSingle, 256));
  return P;
}

// router arrival counters (the fused router of forwards of at most
// kRouterManyMin tokens: one per token tile and one more): zero on entry
// and exit
constexpr int64_t kNhCounterWords = 64;
// then the flag word (a 64-word slot of its own), then D3's per-column-block
// arrival counters: all cleared by the workspace's initialisation
constexpr int64_t kNhCbCounterWords = static_cast<int64_t>(kNhDecMaxColBlocks) * kDecCbStride;
constexpr int64_t kNhClearWords = kNhCounterWords + 64 + kNhCbCounterWords;

struct NhLayout {
  uint32_t* counters;  // [kNhCounterWords]
  uint32_t* cb_counter;  // [kNhDecMaxColBlocks][kDecCbStride]
  uint16_t* logits;    // [T, E + 1]
  uint32_t* inds;      // [n]
  float* scores;       // [n]
  uint32_t *order, *inv, *src, *idx, *offsets, *seg_n, *seg_exp, *seg_off, *sort_base;
  uint32_t *pass_n, *pass_tab;
  uint32_t* f16_flag;
  uint16_t* xh;        // [T, H] fp16 (P8)
  uint16_t *h, *hh;    // [n, Ip] relu^2 of fc1: bf16, fp16 (P8)
  uint16_t *hs, *hsh;  // [T, Isp] the shared expert's
  float* d;            // [n, H] fc2 products, sorted rows (decode: entry order, first K half)
  float* sd;           // [T, H] shared down
  // the decode kernels' (forwards of at most kDecMaxT tokens), sized for
  // min(T, kDecMaxT) at every T so that the layout only grows with T
  uint32_t* lgw;       // [E][Td] logits between the router workgroups
  uint32_t* seg;       // [1 + E]
  uint8_t* slots;      // [E][16]
  float* sd_part;      // [kNhDecSdSplit][Td][H]
  float* d2;           // [Td * k][H] decode fc2 products over the second K half
  size_t total;
};

NhLayout nh_layout(const fmx_nh_moe_config& c, int64_t T, char* base) {
  size_t used = 0;
  auto take = [&](int64_t bytes) -> void* {
    void* p = base ? base + used : nullptr;
    used = static_cast<size_t>(align_up(static_cast<int64_t>(used) + bytes, 256));
    return p;
  };
  const NhPacked P = nh_packed(c);
  const int64_t E = c.n_routed_experts, k = c.num_experts_per_tok, H = c.hidden_size, n = T * k;
  NhLayout L{};
  L.counters = static_cast<uint32_t*>(take(kNhCounterWords * 4));
  L.f16_flag = static_cast<uint32_t*>(take(4));
  L.cb_counter = static_cast<uint32_t*>(take(kNhCbCounterWords * 4));
  L.logits = static_cast<uint16_t*>(take(T * (E + 1) * 2));
  L.inds = static_cast<uint32_t*>(take(n * 4));
  L.scores = static_cast<float*>(take(n * 4));
  L.order = static_cast<uint32_t*>(take(n * 4));
  L.inv = static_cast<uint32_t*>(take(n * 4));
  L.src = static_cast<uint32_t*>(take(n * 4));
  L.idx = static_cast<uint32_t*>(take(n * 4));
  L.offsets = static_cast<uint32_t*>(take((E + 1) * 4));
  L.seg_n = static_cast<uint32_t*>(take(4));
  L.seg_exp = static_cast<uint32_t*>(take(E * 4));
  L.seg_off = static_cast<uint32_t*>(take((E + 1) * 4));
  L.sort_base = static_cast<uint32_t*>(take(E * ((n + 63) / 64) * 4));
  L.pass_n = static_cast<uint32_t*>(take(4));
  L.pass_tab = static_cast<uint32_t*>(take(static_cast<int64_t>(max_passes(n, E)) * 8));
  L.xh = static_cast<uint16_t*>(take(T * H * 2));
  L.h = static_cast<uint16_t*>(take(n * P.Ip * 2));
  L.hh = static_cast<uint16_t*>(take(n * P.Ip * 2));
  L.hs = static_cast<uint16_t*>(take(T * P.Isp * 2));
  L.hsh = static_cast<uint16_t*>(take(T * P.Isp * 2));
  L.d = static_cast<float*>(take(n * H * 4));
  L.sd = static_cast<float*>(take(P.Isp ? T * H * 4 : 0));
  const int64_t Td = std::min<int64_t>(T, kDecMaxT);
  L.lgw = static_cast<uint32_t*>(take(E * Td * 4));
  L.seg = static_cast<uint32_t*>(take((E + 1) * 4));
  L.slots = static_cast<uint8_t*>(take(E * kDecMaxT));
  L.sd_part = static_cast<float*>(take(P.Isp ? kNhDecSdSplit * Td * H * 4 : 0));
  L.d2 = static_cast<float*>(take(Td * k * H * 4));
  L.total = used;
  return L;
}

bool qw_ok(const fmx_qweight& q) {
  return q.w && q.scales && q.biases && aligned(q.w, 16) && aligned(q.scales, 4) && aligned(q.biases, 4);
}

}  // namespace

extern "C" {

size_t fmx_nh_moe_packed_size(const fmx_nh_moe_config* cfg) {
  if (check_config(cfg)) return 0;
  return nh_packed(*cfg).total;
}

int fmx_nh_pack_expert_weights(const fmx_nh_moe_config* cfg, const fmx_nh_moe_weights* src, void* packed,
                               size_t packed_bytes, fmx_stream stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  int rc;
  if ((rc = check_config(cfg))) return rc;
  if (!src || !packed) return fail(FMX_ERR_ARG, "NULL argument");
  const fmx_nh_moe_config& c = *cfg;
  const NhPacked P = nh_packed(c);
  if (!aligned(packed, 256)) return fail(FMX_ERR_ARG, "packed not 256-byte aligned");
  if (packed_bytes < P.total) return fail(FMX_ERR_WORKSPACE, "packed_bytes %zu, need %zu", packed_bytes, P.total);
  const int64_t H = c.hidden_size, E = c.n_routed_experts, I = c.moe_intermediate_size;
  const int64_t Is = c.moe_shared_expert_intermediate_size;
  if (!qw_ok(src->fc1) || !qw_ok(src->fc2)) return fail(FMX_ERR_ARG, "fc1/fc2 NULL or misaligned");
  if (Is > 0 && (!qw_ok(src->shared_up) || !qw_ok(src->shared_down)))
    return fail(FMX_ERR_ARG, "shared expert weights NULL or misaligned");
  uint8_t* dst = static_cast<uint8_t*>(packed);
  // n_exp matrices of N x K (source) into Np/16 tiles x Kp/128 units
  auto pack = [&](const fmx_qweight& a, int64_t n_exp, int64_t N, int64_t Np, int64_t K, int64_t Kp,
                  size_t off, int64_t es) -> hipError_t {
    PackArgs pa{};
    pa.w0 = static_cast<const uint32_t*>(a.w);
    pa.s0 = static_cast<const uint16_t*>(a.scales);
    pa.b0 = static_cast<const uint16_t*>(a.biases);
    pa.n_exp = n_exp;
    pa.N = static_cast<int>(N);
    pa.nt = static_cast<int>(Np / 16);
    pa.nu = static_cast<int>(Kp / 128);
    pa.k_src = static_cast<int>(K);
    pa.dst = dst + off;
    pa.dst_estride = es;
    return launch_pack(pa, stream);
  };
  FMX_HIP(pack(src->fc1, E, I, P.Ip, H, H, P.fc1, P.fc1_es));
  FMX_HIP(pack(src->fc2, E, H, H, I, P.Ip, P.fc2, P.fc2_es));
  if (Is > 0) {
    FMX_HIP(pack(src->shared_up, 1, Is, P.Isp, H, H, P.sup, 0));
    FMX_HIP(pack(src->shared_down, 1, H, H, Is, P.Isp, P.sdn, 0));
  }
  return ok();
}

int fmx_nh_moe_workspace_init(void* workspace, size_t workspace_bytes, fmx_stream stream) {
  if (!workspace) return fail(FMX_ERR_ARG, "workspace is NULL");
  if (!aligned(workspace, 256)) return fail(FMX_ERR_ARG, "workspace not 256-byte aligned");
  // the counters and the flag word that follows them (their own 256-byte slot)
  if (workspace_bytes < static_cast<size_t>(kNhClearWords * 4))
    return fail(FMX_ERR_WORKSPACE, "workspace %zu bytes is too small", workspace_bytes);
  FMX_HIP(launch_fill_u32(static_cast<uint32_t*>(workspace), kNhClearWords, 0u, static_cast<hipStream_t>(stream)));
  return ok();
}

size_t fmx_nh_moe_workspace_size(const fmx_nh_moe_config* cfg, int64_t max_tokens) {
  if (check_config(cfg) || max_tokens < 0 || max_tokens > kNhMaxTokens) return 0;
  return nh_layout(*cfg, std::max<int64_t>(max_tokens, 1), nullptr).total;
}

int fmx_nh_moe_workspace_routing(const fmx_nh_moe_config* cfg, int64_t T, const void* workspace,
                                 const uint32_t** inds, const float** scores, const void** logits) {
  int rc;
  if ((rc = check_config(cfg))) return rc;
  if (!workspace || T < 1 || T > kNhMaxTokens) return fail(FMX_ERR_ARG, "workspace NULL or n_tokens out of range");
  const NhLayout L = nh_layout(*cfg, T, static_cast<char*>(const_cast<void*>(workspace)));
  if (inds) *inds = L.inds;
  if (scores) *scores = L.scores;
  if (logits) *logits = L.logits;
  return ok();
}

}  // extern "C"

namespace {

// The forward's first n_stages kernel stages (1..4: router + sort, fc1,
// fc2, combine; the decode kernels D1, D2, D3 with D3 forming the combine),
// recording stage_events (when given) at the stage boundaries.
int nh_forward(const fmx_nh_moe_config* cfg, const fmx_nh_moe_weights* w, const void* x, int64_t T, void* y,
               void* workspace, size_t workspace_bytes, fmx_stream stream_, void* const* stage_events,
               int n_stages) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  auto mark = [&](int i) -> hipError_t {
    return stage_events ? hipEventRecord(static_cast<hipEvent_t>(stage_events[i]), stream) : hipSuccess;
  };
  int rc;
  if ((rc = check_config(cfg))) return rc;
  if (!w) return fail(FMX_ERR_ARG, "NULL weights");
  if (T < 0 || T > kNhMaxTokens) return fail(FMX_ERR_SHAPE, "n_tokens=%lld out of range", static_cast<long long>(T));
  if (T == 0) return ok();
  if (!x || !y) return fail(FMX_ERR_ARG, "NULL argument");
  if (!aligned(x, 16) || !aligned(y, 16)) return fail(FMX_ERR_ARG, "x/y not 16-byte aligned");
  const fmx_nh_moe_config& c = *cfg;
  const NhPacked P = nh_packed(c);
  if (!w->gate_w || !aligned(w->gate_w, 16)) return fail(FMX_ERR_ARG, "gate_w NULL or misaligned");
  if (w->correction_bias && !aligned(w->correction_bias, 4)) return fail(FMX_ERR_ARG, "correction_bias misaligned");
  if (!w->packed) return fail(FMX_ERR_ARG, "packed weights required (fmx_nh_pack_expert_weights)");
  if (!aligned(w->packed, 256)) return fail(FMX_ERR_ARG, "packed not 256-byte aligned");
  if (w->packed_bytes < P.total)
    return fail(FMX_ERR_WORKSPACE, "packed_bytes %zu, the config needs %zu", w->packed_bytes, P.total);
  const int64_t H = c.hidden_size, E = c.n_routed_experts, k = c.num_experts_per_tok, n = T * k;
  const bool has_sh = c.moe_shared_expert_intermediate_size > 0;
  if (!sort_fits(n, E))
    return fail(FMX_ERR_UNSUPPORTED, "T*k=%lld with E=%lld exceeds the sort's limits", static_cast<long long>(n),
                static_cast<long long>(E));
  const size_t need = nh_layout(c, T, nullptr).total;
  char* base = static_cast<char*>(workspace);
  bool owned = false;
  if (workspace) {
    if (workspace_bytes < need) return fail(FMX_ERR_WORKSPACE, "workspace %zu bytes, need %zu", workspace_bytes, need);
    if (!aligned(workspace, 256)) return fail(FMX_ERR_ARG, "workspace not 256-byte aligned");
  } else {
    void* p = nullptr;
    FMX_HIP(hipMallocAsync(&p, need, stream));
    base = static_cast<char*>(p);
    owned = true;
    const hipError_t e = launch_fill_u32(static_cast<uint32_t*>(p), kNhClearWords, 0u, stream);
    if (e != hipSuccess) {
      (void)hipFreeAsync(p, stream);
      return fail(FMX_ERR_HIP, "clearing the workspace: %s", hipGetErrorString(e));
    }
  }
  auto body = [&]() -> int {
    const NhLayout L = nh_layout(c, T, base);
    const uint8_t* pk = static_cast<const uint8_t*>(w->packed);
    const uint16_t* xb = static_cast<const uint16_t*>(x);

    // decode batches: the four decode kernels
    NhDecArgs da{};
    da.T = static_cast<int>(T);
    da.H = static_cast<int>(H);
    da.E = static_cast<int>(E);
    da.k = static_cast<int>(k);
    da.norm = c.norm_topk_prob ? 1 : 0;
    da.n_group = c.n_group;
    da.topk_group = c.topk_group;
    da.scaling = c.routed_scaling_factor;
    da.Ip = static_cast<int>(P.Ip);
    da.Isp = static_cast<int>(P.Isp);
    if (nh_decode_plan(da)) {
      da.x = xb;
      da.gate_w = static_cast<const uint16_t*>(w->gate_w);
      da.cbias = w->correction_bias;
      da.fc1 = pk + P.fc1;
      da.fc1_es = P.fc1_es;
      da.fc2 = pk + P.fc2;
      da.fc2_es = P.fc2_es;
      da.sup = pk + P.sup;
      da.sdn = pk + P.sdn;
      da.logits = L.logits;
      da.lgw = L.lgw;
      da.inds = L.inds;
      da.scores = L.scores;
      da.seg = L.seg;
      da.slots = L.slots;
      da.h_hi = L.h;
      da.h_lo = L.hh;
      da.hs_hi = L.hs;
      da.hs_lo = L.hsh;
      da.d = L.d;
      da.d2 = L.d2;
      da.sd_part = L.sd_part;
      da.y = static_cast<uint16_t*>(y);
      da.counter = L.counters;
      da.cb_counter = L.cb_counter;
      FMX_HIP(launch_nh_decode(da, stream, stage_events, n_stages));
      return FMX_OK;
    }

    // router: logits, selection, fp32 scores, the fp16 copy of x
    RouterArgs ra{};
    ra.x = xb;
    ra.wr = RouterRows{w->gate_w, nullptr, nullptr};
    ra.T = static_cast<int>(T);
    ra.H = static_cast<int>(H);
    ra.E = static_cast<int>(E);
    ra.k = static_cast<int>(k);
    ra.norm = c.norm_topk_prob ? 1 : 0;
    ra.logits = L.logits;
    ra.inds = L.inds;
    ra.xh = L.xh;
    ra.f16_flag = L.f16_flag;
    ra.mode = 1;
    ra.n_group = c.n_group;
    ra.topk_group = c.topk_group;
    ra.scaling = c.routed_scaling_factor;
    ra.cbias = w->correction_bias;
    ra.scores32 = L.scores;
    ra.counters = L.counters;
    SortOut so{L.order, L.inv, L.src, L.idx, L.offsets, L.seg_n, L.seg_exp, L.seg_off,
               L.sort_base, L.pass_n, L.pass_tab};
    ra.sort = so;
    FMX_HIP(mark(0));
    if (T <= kRouterManyMin && router_sort_fits(n, E)) {
      // one launch: logits in column workgroups, the last of each token
      // tile selects, the last tile sorts
      ra.n_tt = static_cast<int>((T + kRouterTok - 1) / kRouterTok);
      ra.cols_per_wave = ra.n_tt > 1 ? 4 : 1;
      ra.n_ct = static_cast<int>((E + 4 * ra.cols_per_wave - 1) / (4 * ra.cols_per_wave));
      ra.fuse_sort = 1;
      FMX_HIP(launch_router(ra, stream));
    } else {
      FMX_HIP(launch_router_many(ra, stream));
      FMX_HIP(launch_sort(L.inds, static_cast<int>(n), static_cast<int>(k), static_cast<int>(E), so, stream));
    }
    FMX_HIP(mark(1));
    if (n_stages < 2) return FMX_OK;

    const int mp = max_passes(n, E);
    auto routed = [&](const uint8_t* wp, int64_t es, const uint16_t* xr, const uint16_t* xrh, int64_t ldx,
                      const uint32_t* row_map, int64_t N, int64_t K) {
      PfSet s{};
      s.w = wp;
      s.es = es;
      s.x = xr;
      s.xh = xrh;
      s.ldx = ldx;
      s.row_map = row_map;
      s.nt = static_cast<int>(N / 16);
      s.nu = static_cast<int>(K / 128);
      s.pass_n = L.pass_n;
      s.pass_tab = L.pass_tab;
      s.max_pass = mp;
      s.n_exp = static_cast<int>(E);
      s.rows_max = static_cast<int>(n);
      s.x_rows = static_cast<int>(row_map ? T : n);
      return s;
    };
    auto shared = [&](const uint8_t* wp, const uint16_t* xr, const uint16_t* xrh, int64_t ldx, int64_t N,
                      int64_t K) {
      PfSet s{};
      s.w = wp;
      s.x = xr;
      s.xh = xrh;
      s.ldx = ldx;
      s.nt = static_cast<int>(N / 16);
      s.nu = static_cast<int>(K / 128);
      s.rows_static = s.rows_max = s.x_rows = static_cast<int>(T);
      s.n_exp = 1;
      return s;
    };
    {  // fc1 + relu^2 (routed passes) and the shared up projection
      PfArgs pa{};
      pa.s1 = routed(pk + P.fc1, P.fc1_es, xb, L.xh, H, L.src, P.Ip, H);
      pa.s1.act = 1;
      pa.s1.out = L.h;
      pa.s1.outh = L.hh;
      pa.s1.ldo = P.Ip;
      pa.n_items1 = pf_items(pa.s1, false);
      if (has_sh) {
        pa.s0 = shared(pk + P.sup, xb, L.xh, H, P.Isp, H);
        pa.s0.act = 1;
        pa.s0.out = L.hs;
        pa.s0.outh = L.hsh;
        pa.s0.ldo = P.Isp;
        pa.n_items0 = pf_items(pa.s0, false);
      }
      pa.f16_flag = L.f16_flag;
      pa.flag_in = kF16FlagX;
      pa.flag_out = kF16FlagH;
      FMX_HIP(launch_pf(pa, false, stream));
      FMX_HIP(mark(2));
    }
    if (n_stages < 3) return FMX_OK;
    {  // fc2 and the shared down projection, fp32 products
      PfArgs pa{};
      pa.s1 = routed(pk + P.fc2, P.fc2_es, L.h, L.hh, P.Ip, nullptr, H, P.Ip);
      pa.s1.out32 = L.d;
      pa.s1.ldo = H;
      pa.n_items1 = pf_items(pa.s1, false);
      if (has_sh) {
        pa.s0 = shared(pk + P.sdn, L.hs, L.hsh, P.Isp, H, P.Isp);
        pa.s0.out32 = L.sd;
        pa.s0.ldo = H;
        pa.n_items0 = pf_items(pa.s0, false);
      }
      pa.f16_flag = L.f16_flag;
      pa.flag_in = kF16FlagH;
      pa.flag_out = 0u;
      FMX_HIP(launch_pf(pa, false, stream));
      FMX_HIP(mark(3));
    }
    if (n_stages < 4) return FMX_OK;
    NhCombineArgs cb{};
    cb.d = L.d;
    cb.inv = L.inv;
    cb.scores = L.scores;
    cb.sd = has_sh ? L.sd : nullptr;
    cb.y = static_cast<uint16_t*>(y);
    cb.T = static_cast<int>(T);
    cb.k = static_cast<int>(k);
    cb.H = static_cast<int>(H);
    cb.clear = L.f16_flag;
    FMX_HIP(launch_nh_combine(cb, stream));
    FMX_HIP(mark(4));
    return FMX_OK;
  };
  rc = body();
  if (owned) (void)hipFreeAsync(base, stream);
  return rc ? rc : ok();
}

}  // namespace

extern "C" {

int fmx_nh_moe_block_forward(const fmx_nh_moe_config* cfg, const fmx_nh_moe_weights* w, const void* x,
                             int64_t T, void* y, void* workspace, size_t workspace_bytes, fmx_stream stream_) {
  return nh_forward(cfg, w, x, T, y, workspace, workspace_bytes, stream_, nullptr, 4);
}

int fmx_nh_moe_block_forward_profiled(const fmx_nh_moe_config* cfg, const fmx_nh_moe_weights* w,
                                      const void* x, int64_t T, void* y, void* workspace,
                                      size_t workspace_bytes, fmx_stream stream_, void* const* stage_events) {
  return nh_forward(cfg, w, x, T, y, workspace, workspace_bytes, stream_, stage_events, 4);
}

int fmx_nh_moe_block_forward_partial(const fmx_nh_moe_config* cfg, const fmx_nh_moe_weights* w,
                                     const void* x, int64_t T, void* y, void* workspace,
                                     size_t workspace_bytes, fmx_stream stream_, int n_stages) {
  if (n_stages < 1 || n_stages > 4) return fail(FMX_ERR_ARG, "n_stages=%d (1..4)", n_stages);
  return nh_forward(cfg, w, x, T, y, workspace, workspace_bytes, stream_, nullptr, n_stages);
}

}  // extern "C"
