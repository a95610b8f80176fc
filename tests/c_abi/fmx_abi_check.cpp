// fmx_abi_check.cpp -- a C++ program that uses libfmx only through
// include/fmx.h, the way the reference's C++ server would
// (server/src/model.cpp:368-470 at load time, :750-807 per forward):
// synthesise a small MoE layer, quantize it, stack and pack it, release the
// MLX-layout copies, then run one forward of 4 tokens. It writes y [T, H]
// (bf16) and the routing indices [T, k] (u32) to the files named on the
// command line; tests/test_c_abi.py compares them with the committed fixture.
//
// Shapes and seeds are those of the "small_dec_t4" workload: H 512, 8
// experts, top-2, I 256, shared expert 512, 4 tokens, seed 16; each tensor
// is its own stream of fmx_synth_normal_bf16 (x ~ N(0,1), weights ~
// N(0, 0.02)).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <vector>

#include "fmx.h"

#define FMX_CHECK(expr)                                                                    \
  do {                                                                                     \
    int s_ = (expr);                                                                       \
    if (s_ != FMX_OK)                                                                      \
      throw std::runtime_error(std::string(#expr) + ": " + fmx_status_string(s_) + ": " + \
                               fmx_last_error());                                          \
  } while (0)
#define HIP_CHECK(expr)                                                                              \
  do {                                                                                               \
    hipError_t e_ = (expr);                                                                          \
    if (e_ != hipSuccess) throw std::runtime_error(std::string(#expr) + ": " + hipGetErrorString(e_)); \
  } while (0)

namespace {

constexpr uint64_t kSeed = 16;
constexpr int64_t H = 512, E = 8, K = 2, I = 256, IS = 512, T = 4;

void* dev_alloc(size_t bytes, std::vector<void*>& owned) {
  void* p = nullptr;
  HIP_CHECK(hipMalloc(&p, bytes));
  owned.push_back(p);
  return p;
}

// bf16 synthetic tensor of n elements on the device
void* synth(int64_t n, uint64_t stream_id, double std_dev, std::vector<void*>& owned) {
  std::vector<uint16_t> h(n);
  FMX_CHECK(fmx_synth_normal_bf16(h.data(), n, kSeed, stream_id, 0.0, std_dev));
  void* d = dev_alloc(n * 2, owned);
  HIP_CHECK(hipMemcpy(d, h.data(), n * 2, hipMemcpyHostToDevice));
  return d;
}

fmx_array arr(void* data, fmx_dtype dt, std::initializer_list<int64_t> shape) {
  fmx_array a{};
  a.data = data;
  a.dtype = dt;
  a.ndim = static_cast<int32_t>(shape.size());
  int i = 0;
  for (int64_t s : shape) a.shape[i++] = s;
  return a;
}

// mx::quantize of an [n_exp, N, Kd] bf16 tensor, one expert at a time, then
// mx::stack of the per-expert parts (model.cpp:396-404)
fmx_qweight quantize_stacked(void* w, int64_t n_exp, int64_t N, int64_t Kd, hipStream_t s,
                             std::vector<void*>& owned) {
  std::vector<const void*> pw, ps, pb;
  std::vector<void*> parts;
  for (int64_t e = 0; e < n_exp; ++e) {
    void* wq = dev_alloc(N * Kd / 2, parts);
    void* sc = dev_alloc(N * Kd / 64 * 2, parts);
    void* bi = dev_alloc(N * Kd / 64 * 2, parts);
    fmx_array src = arr(static_cast<char*>(w) + e * N * Kd * 2, FMX_BF16, {N, Kd});
    fmx_array a_wq = arr(wq, FMX_U32, {N, Kd / 8});
    fmx_array a_sc = arr(sc, FMX_BF16, {N, Kd / 64});
    fmx_array a_bi = arr(bi, FMX_BF16, {N, Kd / 64});
    FMX_CHECK(fmx_quantize(&src, 64, 4, "affine", &a_wq, &a_sc, &a_bi, s));
    pw.push_back(wq);
    ps.push_back(sc);
    pb.push_back(bi);
  }
  fmx_qweight q{};
  void* dw = dev_alloc(n_exp * N * Kd / 2, owned);
  void* ds = dev_alloc(n_exp * N * Kd / 64 * 2, owned);
  void* db = dev_alloc(n_exp * N * Kd / 64 * 2, owned);
  FMX_CHECK(fmx_stack_experts(pw.data(), n_exp, N * Kd / 2, dw, s));
  FMX_CHECK(fmx_stack_experts(ps.data(), n_exp, N * Kd / 64 * 2, ds, s));
  FMX_CHECK(fmx_stack_experts(pb.data(), n_exp, N * Kd / 64 * 2, db, s));
  HIP_CHECK(hipStreamSynchronize(s));
  for (void* p : parts) HIP_CHECK(hipFree(p));  // the per-expert parts are not kept
  q.w = dw;
  q.scales = ds;
  q.biases = db;
  return q;
}

void write_file(const char* path, const void* data, size_t bytes) {
  FILE* f = std::fopen(path, "wb");
  if (!f || std::fwrite(data, 1, bytes, f) != bytes) throw std::runtime_error(std::string("write ") + path);
  std::fclose(f);
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 3) {
    std::fprintf(stderr, "usage: %s <y.bin> <inds.bin>\n", argv[0]);
    return 2;
  }
  try {
    if (fmx_abi_version() != FMX_ABI_VERSION) throw std::runtime_error("libfmx ABI version mismatch");
    hipStream_t s;
    HIP_CHECK(hipStreamCreate(&s));
    std::vector<void*> keep, mlx;  // device buffers: kept for the forward / MLX layout only

    // ---- load time (model.cpp:368-470)
    fmx_moe_config cfg{};
    cfg.hidden_size = H;
    cfg.num_experts = E;
    cfg.num_experts_per_tok = K;
    cfg.norm_topk_prob = 0;
    cfg.moe_intermediate_size = I;
    cfg.shared_expert_intermediate_size = IS;
    cfg.quant_bits = 4;
    cfg.quant_group_size = 64;

    fmx_moe_weights w{};
    w.router_w = synth(E * H, 2, 0.02, keep);
    std::vector<void*> raw;  // bf16 originals, freed after quantization
    w.gate = quantize_stacked(synth(E * I * H, 10, 0.02, raw), E, I, H, s, mlx);
    w.up = quantize_stacked(synth(E * I * H, 11, 0.02, raw), E, I, H, s, mlx);
    w.down = quantize_stacked(synth(E * H * I, 12, 0.02, raw), E, H, I, s, mlx);
    w.shared_gate = quantize_stacked(synth(IS * H, 20, 0.02, raw), 1, IS, H, s, mlx);
    w.shared_up = quantize_stacked(synth(IS * H, 21, 0.02, raw), 1, IS, H, s, mlx);
    w.shared_down = quantize_stacked(synth(H * IS, 22, 0.02, raw), 1, H, IS, s, mlx);
    w.shared_expert_gate_w = synth(H, 23, 0.02, keep);
    for (void* p : raw) HIP_CHECK(hipFree(p));

    const size_t pbytes = fmx_moe_packed_size(&cfg);
    if (pbytes == 0) throw std::runtime_error("config cannot be packed");
    void* packed = dev_alloc(pbytes, keep);
    FMX_CHECK(fmx_pack_expert_weights(&cfg, &w, packed, pbytes, s));
    HIP_CHECK(hipStreamSynchronize(s));
    // the layer now holds its expert weights once: drop the MLX layout
    for (void* p : mlx) HIP_CHECK(hipFree(p));
    w.gate = w.up = w.down = w.shared_gate = w.shared_up = w.shared_down = fmx_qweight{};
    w.packed = packed;
    w.packed_bytes = pbytes;

    const size_t ws_bytes = fmx_moe_workspace_size(&cfg, 16);
    if (ws_bytes == 0) throw std::runtime_error("workspace size query failed");
    void* ws = dev_alloc(ws_bytes, keep);
    FMX_CHECK(fmx_moe_workspace_init(ws, ws_bytes, s));

    // ---- forward (model.cpp:750-807)
    void* x = synth(T * H, 1, 1.0, keep);
    void* y = dev_alloc(T * H * 2, keep);
    if (fmx_moe_forward_path(&cfg, T, 1) != 1) throw std::runtime_error("expected the decode kernels");
    FMX_CHECK(fmx_moe_block_forward(&cfg, &w, x, T, y, ws, ws_bytes, s));
    const uint32_t* inds = nullptr;
    FMX_CHECK(fmx_moe_workspace_routing(&cfg, T, ws, &inds, nullptr, nullptr, nullptr, nullptr,
                                        nullptr, nullptr, nullptr));
    std::vector<uint16_t> hy(T * H);
    std::vector<uint32_t> hi(T * K);
    HIP_CHECK(hipMemcpyAsync(hy.data(), y, hy.size() * 2, hipMemcpyDeviceToHost, s));
    HIP_CHECK(hipMemcpyAsync(hi.data(), inds, hi.size() * 4, hipMemcpyDeviceToHost, s));
    HIP_CHECK(hipStreamSynchronize(s));
    write_file(argv[1], hy.data(), hy.size() * 2);
    write_file(argv[2], hi.data(), hi.size() * 4);
    for (void* p : keep) HIP_CHECK(hipFree(p));
    HIP_CHECK(hipStreamDestroy(s));
    std::printf("fmx_abi_check: forward of %lld tokens ok (packed layer %zu bytes, workspace %zu bytes)\n",
                static_cast<long long>(T), pbytes, ws_bytes);
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "fmx_abi_check: %s\n", e.what());
    return 1;
  }
}
