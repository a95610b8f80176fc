// fmx_loader.cpp -- the quantized-checkpoint loader (include/fmx_model.h):
// an MLX checkpoint directory (config.json + *.safetensors) read straight
// into the layout the decoder stack's kernels stream.
//
// Reference: server/src/model.cpp:100-146 (load_config), :148-184
// (load_weights: every *.safetensors file in name order, keys with a
// "model." prefix dropped), :186-224 (constructor: activation dtype, weight
// cache, pre-dequantized embedding), :246-340 (build_weight_cache),
// :368-470 (build_moe_weight_cache: per-expert arrays stacked into [E, ...]);
// key names docs/superpowers/specs/2026-04-01-moe-support-design.md:138-151.
//
// Unlike the reference, which keeps every per-expert array next to the
// stacked copy, each tensor is read once into a staging buffer and packed
// (experts one by one) into its final place: the layer holds its expert
// weights once, in the packed layout.
#include <hip/hip_runtime.h>

#include <dirent.h>
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/fmx_model.h"
#include "fmx_kernels.hpp"

namespace fmx {
int set_error(int status, const char* msg);
void clear_error();
bool moe_packed_parts(const fmx_moe_config& c, size_t* gu, size_t* dn, size_t* sgu, size_t* sdn,
                      int64_t* gu_es, int64_t* dn_es);
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

#define FMX_HIP(expr)                                                              \
  do {                                                                             \
    hipError_t e_ = (expr);                                                        \
    if (e_ != hipSuccess)                                                          \
      return fail(FMX_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_));            \
  } while (0)

#define FMX_RC(expr)     \
  do {                   \
    int rc_ = (expr);    \
    if (rc_) return rc_; \
  } while (0)

// ---------------------------------------------------------------- JSON

// The subset of JSON that config.json and safetensors headers use.
struct JVal {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  double num = 0.0;
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
  const JVal* get(const std::string& k) const {
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

struct JParser {
  const char* p;
  const char* e;
  bool ok = true;
  void ws() {
    while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool lit(const char* s) {
    const size_t n = strlen(s);
    if (static_cast<size_t>(e - p) < n || strncmp(p, s, n)) return false;
    p += n;
    return true;
  }
  std::string string() {
    std::string out;
    if (p >= e || *p != '"') {
      ok = false;
      return out;
    }
    ++p;
    while (p < e && *p != '"') {
      if (*p == '\\' && p + 1 < e) {
        ++p;
        switch (*p) {
          case 'n': out += '\n'; break;
          case 't': out += '\t'; break;
          case 'u':  // \uXXXX: kept as the escape (keys here are ASCII)
            out += "\\u";
            break;
          default: out += *p;
        }
        ++p;
      } else {
        out += *p++;
      }
    }
    if (p >= e) ok = false;
    ++p;
    return out;
  }
  JVal value(int depth = 0) {
    JVal v;
    ws();
    if (p >= e || depth > 64) {
      ok = false;
      return v;
    }
    if (*p == '{') {
      v.kind = JVal::OBJ;
      ++p;
      ws();
      if (p < e && *p == '}') {
        ++p;
        return v;
      }
      while (ok) {
        ws();
        std::string k = string();
        ws();
        if (p >= e || *p != ':') {
          ok = false;
          break;
        }
        ++p;
        v.obj.emplace_back(std::move(k), value(depth + 1));
        ws();
        if (p < e && *p == ',') {
          ++p;
          continue;
        }
        if (p < e && *p == '}') {
          ++p;
          break;
        }
        ok = false;
      }
    } else if (*p == '[') {
      v.kind = JVal::ARR;
      ++p;
      ws();
      if (p < e && *p == ']') {
        ++p;
        return v;
      }
      while (ok) {
        v.arr.push_back(value(depth + 1));
        ws();
        if (p < e && *p == ',') {
          ++p;
          continue;
        }
        if (p < e && *p == ']') {
          ++p;
          break;
        }
        ok = false;
      }
    } else if (*p == '"') {
      v.kind = JVal::STR;
      v.str = string();
    } else if (lit("true")) {
      v.kind = JVal::BOOL;
      v.b = true;
    } else if (lit("false")) {
      v.kind = JVal::BOOL;
    } else if (lit("null")) {
      v.kind = JVal::NUL;
    } else {
      char* end = nullptr;
      const std::string tok(p, std::min<size_t>(64, static_cast<size_t>(e - p)));
      v.num = strtod(tok.c_str(), &end);
      if (end == tok.c_str()) {
        ok = false;
        return v;
      }
      v.kind = JVal::NUM;
      p += end - tok.c_str();
    }
    return v;
  }
};

bool parse_json(const std::string& text, JVal& out) {
  JParser jp{text.data(), text.data() + text.size()};
  out = jp.value();
  return jp.ok;
}

bool read_file(const std::string& path, std::string& out) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) return false;
  char buf[1 << 16];
  size_t n;
  while ((n = fread(buf, 1, sizeof(buf), f)) > 0) out.append(buf, n);
  fclose(f);
  return true;
}

// ---------------------------------------------------------------- safetensors

struct Tensor {
  int file;
  std::string dtype;
  std::vector<int64_t> shape;
  uint64_t off, nbytes;  // absolute file offset of the data
  int64_t numel() const {
    int64_t n = 1;
    for (int64_t s : shape) n *= s;
    return n;
  }
};

struct Checkpoint {
  std::vector<std::string> files;
  std::vector<int> fds;
  std::map<std::string, Tensor> tensors;
  ~Checkpoint() {
    for (int fd : fds)
      if (fd >= 0) close(fd);
  }
  const Tensor* find(const std::string& k) const {
    auto it = tensors.find(k);
    return it == tensors.end() ? nullptr : &it->second;
  }
};

int64_t dtype_size(const std::string& d) {
  if (d == "BF16" || d == "F16" || d == "I16" || d == "U16") return 2;
  if (d == "F32" || d == "U32" || d == "I32") return 4;
  if (d == "F64" || d == "I64" || d == "U64") return 8;
  if (d == "U8" || d == "I8" || d == "BOOL") return 1;
  return 0;
}

// Every *.safetensors file of dir, in name order; a key's "model." prefix is
// dropped and a later file's key replaces an earlier one (model.cpp:148-184).
int open_checkpoint(const char* dir, Checkpoint& ck) {
  DIR* d = opendir(dir);
  if (!d) return fail(FMX_ERR_ARG, "cannot open checkpoint directory %s", dir);
  while (dirent* ent = readdir(d)) {
    const std::string n = ent->d_name;
    if (n.size() >= 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0)
      ck.files.push_back(std::string(dir) + "/" + n);
  }
  closedir(d);
  std::sort(ck.files.begin(), ck.files.end());
  if (ck.files.empty()) return fail(FMX_ERR_ARG, "no .safetensors files in %s", dir);
  for (size_t fi = 0; fi < ck.files.size(); ++fi) {
    const int fd = open(ck.files[fi].c_str(), O_RDONLY);
    ck.fds.push_back(fd);
    if (fd < 0) return fail(FMX_ERR_ARG, "cannot open %s", ck.files[fi].c_str());
    uint64_t hlen = 0;
    if (pread(fd, &hlen, 8, 0) != 8 || hlen > (1ull << 30))
      return fail(FMX_ERR_ARG, "%s: bad safetensors header", ck.files[fi].c_str());
    std::string hdr(hlen, '\0');
    if (pread(fd, &hdr[0], hlen, 8) != static_cast<ssize_t>(hlen))
      return fail(FMX_ERR_ARG, "%s: truncated header", ck.files[fi].c_str());
    JVal j;
    if (!parse_json(hdr, j) || j.kind != JVal::OBJ)
      return fail(FMX_ERR_ARG, "%s: header is not a JSON object", ck.files[fi].c_str());
    const off_t fsize = lseek(fd, 0, SEEK_END);
    for (const auto& kv : j.obj) {
      if (kv.first == "__metadata__") continue;
      const JVal& t = kv.second;
      const JVal *dt = t.get("dtype"), *sh = t.get("shape"), *of = t.get("data_offsets");
      if (!dt || !sh || !of || of->arr.size() != 2)
        return fail(FMX_ERR_ARG, "%s: tensor %s without dtype/shape/data_offsets", ck.files[fi].c_str(),
                    kv.first.c_str());
      Tensor tt;
      tt.file = static_cast<int>(fi);
      tt.dtype = dt->str;
      for (const JVal& s : sh->arr) tt.shape.push_back(static_cast<int64_t>(s.num));
      const uint64_t b = static_cast<uint64_t>(of->arr[0].num), en = static_cast<uint64_t>(of->arr[1].num);
      tt.off = 8 + hlen + b;
      tt.nbytes = en - b;
      if (en < b || tt.off + tt.nbytes > static_cast<uint64_t>(fsize) ||
          static_cast<int64_t>(tt.nbytes) != tt.numel() * dtype_size(tt.dtype))
        return fail(FMX_ERR_ARG, "%s: tensor %s has inconsistent offsets", ck.files[fi].c_str(),
                    kv.first.c_str());
      std::string key = kv.first;
      if (key.compare(0, 6, "model.") == 0) key = key.substr(6);
      ck.tensors[key] = tt;
    }
  }
  return FMX_OK;
}

// ---------------------------------------------------------------- device upload

}  // namespace

// The weights of a loaded model: device memory owned by this object.
struct fmx_loaded_model {
  fmx_model_config cfg{};
  std::vector<void*> allocs;
  std::vector<fmx_layer_weights> layers;
  fmx_model_weights w{};
  size_t bytes = 0;
  ~fmx_loaded_model() {
    for (void* p : allocs) (void)hipFree(p);
  }
};

namespace {

struct Uploader {
  const Checkpoint& ck;
  fmx_loaded_model& m;
  hipStream_t stream;
  void* host = nullptr;  // pinned staging
  size_t host_cap = 0;
  uint8_t* stage = nullptr;  // device staging for tensors that are re-laid out
  size_t stage_cap = 0, stage_used = 0;
  ~Uploader() {
    if (host) (void)hipHostFree(host);
    if (stage) (void)hipFree(stage);
  }

  int alloc(size_t bytes, void** p) {
    FMX_HIP(hipMalloc(p, std::max<size_t>(bytes, 256)));
    m.allocs.push_back(*p);
    m.bytes += bytes;
    return FMX_OK;
  }

  // tensor `key` (checked dtype and shape) into device memory at dst
  int read(const std::string& key, const char* dtype, std::vector<int64_t> shape, void* dst) {
    const Tensor* t = ck.find(key);
    if (!t) return fail(FMX_ERR_ARG, "checkpoint has no tensor %s", key.c_str());
    if (t->dtype != dtype)
      return fail(FMX_ERR_DTYPE, "%s: dtype %s, expected %s", key.c_str(), t->dtype.c_str(), dtype);
    if (t->shape != shape) {
      std::string got, want;
      for (int64_t s : t->shape) got += std::to_string(s) + " ";
      for (int64_t s : shape) want += std::to_string(s) + " ";
      return fail(FMX_ERR_SHAPE, "%s: shape [%s], expected [%s]", key.c_str(), got.c_str(), want.c_str());
    }
    if (t->nbytes > host_cap) {
      if (host) FMX_HIP(hipHostFree(host));
      host = nullptr;
      FMX_HIP(hipHostMalloc(&host, t->nbytes, hipHostMallocDefault));
      host_cap = t->nbytes;
    }
    FMX_HIP(hipStreamSynchronize(stream));  // the previous copy out of host is done
    uint64_t done = 0;
    while (done < t->nbytes) {
      const ssize_t r = pread(ck.fds[t->file], static_cast<char*>(host) + done, t->nbytes - done, t->off + done);
      if (r <= 0) return fail(FMX_ERR_ARG, "%s: read error", key.c_str());
      done += static_cast<uint64_t>(r);
    }
    FMX_HIP(hipMemcpyAsync(dst, host, t->nbytes, hipMemcpyHostToDevice, stream));
    return FMX_OK;
  }

  // a tensor into newly allocated device memory
  int own(const std::string& key, const char* dtype, std::vector<int64_t> shape, const void** out) {
    const Tensor* t = ck.find(key);
    void* p = nullptr;
    FMX_RC(alloc(t ? t->nbytes : 256, &p));
    FMX_RC(read(key, dtype, shape, p));
    *out = p;
    return FMX_OK;
  }

  // staging space for tensors packed right after (reset per group)
  int staged(size_t bytes, void** out) {
    bytes = static_cast<size_t>(align_up(static_cast<int64_t>(bytes), 256));
    if (stage_used + bytes > stage_cap) return fail(FMX_ERR_ARG, "staging overflow");
    *out = stage + stage_used;
    stage_used += bytes;
    return FMX_OK;
  }

  // quantized matrix prefix.{weight,scales,biases} [N, K] into staging
  int quant(const std::string& prefix, int64_t N, int64_t K, fmx_qweight* q) {
    void *w, *s, *b;
    FMX_RC(staged(static_cast<size_t>(N * K / 2), &w));
    FMX_RC(staged(static_cast<size_t>(N * K / 32), &s));
    FMX_RC(staged(static_cast<size_t>(N * K / 32), &b));
    FMX_RC(read(prefix + ".weight", "U32", {N, K / 8}, w));
    FMX_RC(read(prefix + ".scales", "BF16", {N, K / 64}, s));
    if (!ck.find(prefix + ".biases"))
      return fail(FMX_ERR_UNSUPPORTED, "%s: no biases (only affine quantization)", prefix.c_str());
    FMX_RC(read(prefix + ".biases", "BF16", {N, K / 64}, b));
    *q = fmx_qweight{w, s, b};
    return FMX_OK;
  }

  // a linear that is bf16 [N, K] or quantized: as-is into owned memory
  int router_rows(const std::string& prefix, int64_t N, int64_t K, const void** w, const void** s,
                  const void** b) {
    if (ck.find(prefix + ".scales")) {
      FMX_RC(own(prefix + ".weight", "U32", {N, K / 8}, w));
      FMX_RC(own(prefix + ".scales", "BF16", {N, K / 64}, s));
      FMX_RC(own(prefix + ".biases", "BF16", {N, K / 64}, b));
    } else {
      FMX_RC(own(prefix + ".weight", "BF16", {N, K}, w));
      *s = *b = nullptr;
    }
    return FMX_OK;
  }
};

hipError_t pack(const fmx_qweight& a, const fmx_qweight* b, int64_t N, int64_t K, uint8_t* dst,
                hipStream_t stream) {
  PackArgs pa{};
  pa.w0 = static_cast<const uint32_t*>(a.w);
  pa.s0 = static_cast<const uint16_t*>(a.scales);
  pa.b0 = static_cast<const uint16_t*>(a.biases);
  if (b) {
    pa.w1 = static_cast<const uint32_t*>(b->w);
    pa.s1 = static_cast<const uint16_t*>(b->scales);
    pa.b1 = static_cast<const uint16_t*>(b->biases);
  }
  pa.n_exp = 1;
  pa.N = static_cast<int>(N);
  pa.nt = static_cast<int>(N / 16);
  pa.nu = static_cast<int>(K / 128);
  pa.dst = dst;
  pa.dst_estride = 0;
  return launch_pack(pa, stream);
}

int64_t packed_linear(int64_t N, int64_t K) { return (N / 16) * (K / 128) * kPackedBlockSingle; }

int json_int(const JVal& j, const char* k, int64_t def) {
  const JVal* v = j.get(k);
  return v && v->kind == JVal::NUM ? static_cast<int>(v->num) : static_cast<int>(def);
}
double json_num(const JVal& j, const char* k, double def) {
  const JVal* v = j.get(k);
  return v && v->kind == JVal::NUM ? v->num : def;
}
bool json_bool(const JVal& j, const char* k, bool def) {
  const JVal* v = j.get(k);
  return v && v->kind == JVal::BOOL ? v->b : def;
}

}  // namespace

extern "C" {

int fmx_model_config_from_json(const char* path, fmx_model_config* cfg, int32_t* tie_word_embeddings) {
  if (!path || !cfg) return fail(FMX_ERR_ARG, "NULL argument");
  std::string text;
  if (!read_file(path, text)) return fail(FMX_ERR_ARG, "cannot read %s", path);
  JVal j;
  if (!parse_json(text, j) || j.kind != JVal::OBJ) return fail(FMX_ERR_ARG, "%s is not a JSON object", path);
  *cfg = fmx_model_config{};
  // the keys and defaults of LlamaModel::load_config (model.cpp:111-140)
  cfg->hidden_size = json_int(j, "hidden_size", 4096);
  cfg->num_hidden_layers = json_int(j, "num_hidden_layers", 32);
  cfg->num_attention_heads = json_int(j, "num_attention_heads", 32);
  cfg->num_key_value_heads = json_int(j, "num_key_value_heads", 8);
  cfg->head_dim = json_int(j, "head_dim", 0);
  cfg->vocab_size = json_int(j, "vocab_size", 128256);
  cfg->max_position_embeddings = json_int(j, "max_position_embeddings", 8192);
  cfg->rms_norm_eps = static_cast<float>(json_num(j, "rms_norm_eps", 1e-5));
  cfg->rope_theta = static_cast<float>(json_num(j, "rope_theta", 10000.0));
  if (tie_word_embeddings) *tie_word_embeddings = json_bool(j, "tie_word_embeddings", true) ? 1 : 0;
  cfg->moe.hidden_size = cfg->hidden_size;
  cfg->moe.num_experts = json_int(j, "num_experts", 0);
  cfg->moe.num_experts_per_tok = json_int(j, "num_experts_per_tok", 0);
  cfg->moe.moe_intermediate_size = json_int(j, "moe_intermediate_size", 0);
  cfg->moe.shared_expert_intermediate_size = json_int(j, "shared_expert_intermediate_size", 0);
  cfg->moe.norm_topk_prob = json_bool(j, "norm_topk_prob", false) ? 1 : 0;
  cfg->moe.quant_bits = 0;
  cfg->moe.quant_group_size = 64;
  if (const JVal* q = j.get("quantization")) {
    if (q->kind == JVal::OBJ) {
      cfg->moe.quant_bits = json_int(*q, "bits", 0);
      cfg->moe.quant_group_size = json_int(*q, "group_size", 64);
    }
  }
  clear_error();
  return FMX_OK;
}

int fmx_checkpoint_tensor(const char* dir, const char* name, char* dtype, int64_t* shape, int32_t* ndim) {
  if (!dir || !name) return fail(FMX_ERR_ARG, "NULL argument");
  Checkpoint ck;
  FMX_RC(open_checkpoint(dir, ck));
  const Tensor* t = ck.find(name);
  if (!t) return fail(FMX_ERR_ARG, "no tensor %s", name);
  if (dtype) snprintf(dtype, 8, "%s", t->dtype.c_str());
  if (ndim) *ndim = static_cast<int32_t>(t->shape.size());
  if (shape)
    for (size_t i = 0; i < t->shape.size() && i < 8; ++i) shape[i] = t->shape[i];
  clear_error();
  return FMX_OK;
}

int fmx_model_load(const char* dir, const fmx_model_config* cfg_in, fmx_loaded_model** out,
                   fmx_stream stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (!dir || !cfg_in || !out) return fail(FMX_ERR_ARG, "NULL argument");
  *out = nullptr;
  const fmx_model_config& c = *cfg_in;
  if (fmx_model_workspace_size(&c, 1) == 0) return FMX_ERR_UNSUPPORTED;  // the reason is set
  const int64_t H = c.hidden_size, L = c.num_hidden_layers, nh = c.num_attention_heads;
  const int64_t nkv = c.num_key_value_heads;
  const int64_t hd = c.head_dim > 0 ? c.head_dim : H / nh;
  const int64_t V = c.vocab_size, E = c.moe.num_experts, I = c.moe.moe_intermediate_size;
  const int64_t Is = c.moe.shared_expert_intermediate_size, nq = (nh + 2 * nkv) * hd;
  size_t gu, dn, sgu, sdn;
  int64_t gu_es, dn_es;
  if (!moe_packed_parts(c.moe, &gu, &dn, &sgu, &sdn, &gu_es, &dn_es))
    return fail(FMX_ERR_UNSUPPORTED, "MoE shapes outside the packed layout");
  Checkpoint ck;
  FMX_RC(open_checkpoint(dir, ck));
  auto m = new fmx_loaded_model();
  m->cfg = c;
  Uploader up{ck, *m, stream};
  auto body = [&]() -> int {
    // staging: the largest quantized matrix triple (embedding, lm_head, a
    // layer's q/k/v or an expert pair)
    const int64_t biggest = std::max({V * H, nq * H, 2 * I * H, 2 * Is * H, H * nh * hd});
    up.stage_cap = static_cast<size_t>(biggest / 2 + 2 * (biggest / 32) + 4096);
    FMX_HIP(hipMalloc(reinterpret_cast<void**>(&up.stage), up.stage_cap));
    const size_t moe_bytes = fmx_moe_packed_size(&c.moe);
    m->layers.resize(static_cast<size_t>(L));
    for (int64_t l = 0; l < L; ++l) {
      fmx_layer_weights& lw = m->layers[l];
      const std::string p = "layers." + std::to_string(l);
      FMX_RC(up.own(p + ".input_layernorm.weight", "BF16", {H}, &lw.input_norm_w));
      FMX_RC(up.own(p + ".post_attention_layernorm.weight", "BF16", {H}, &lw.post_norm_w));
      // q, k, v packed one after the other; their linear biases concatenated
      const std::string a = p + ".self_attn";
      void* qkv = nullptr;
      FMX_RC(up.alloc(static_cast<size_t>(packed_linear(nq, H)), &qkv));
      const char* names[3] = {"q_proj", "k_proj", "v_proj"};
      const int64_t rows[3] = {nh * hd, nkv * hd, nkv * hd};
      int64_t row0 = 0;
      const bool has_bias = ck.find(a + ".q_proj.bias") != nullptr;
      void* bias = nullptr;
      if (has_bias) FMX_RC(up.alloc(static_cast<size_t>(nq * 2), &bias));
      for (int i = 0; i < 3; ++i) {
        up.stage_used = 0;
        fmx_qweight q{};
        FMX_RC(up.quant(a + "." + names[i], rows[i], H, &q));
        FMX_HIP(pack(q, nullptr, rows[i], H, static_cast<uint8_t*>(qkv) + packed_linear(row0, H), stream));
        if (has_bias)
          FMX_RC(up.read(a + "." + names[i] + ".bias", "BF16", {rows[i]}, static_cast<uint16_t*>(bias) + row0));
        row0 += rows[i];
      }
      lw.qkv = qkv;
      lw.qkv_bias = bias;
      void* o = nullptr;
      FMX_RC(up.alloc(static_cast<size_t>(packed_linear(H, nh * hd)), &o));
      up.stage_used = 0;
      fmx_qweight oq{};
      FMX_RC(up.quant(a + ".o_proj", H, nh * hd, &oq));
      FMX_HIP(pack(oq, nullptr, H, nh * hd, static_cast<uint8_t*>(o), stream));
      lw.o = o;
      // the MoE block (model.cpp:368-470): router, experts packed one by one,
      // shared expert and its gate
      const std::string mp = p + ".mlp";
      if (!ck.find(mp + ".experts.0.gate_proj.weight"))
        return fail(FMX_ERR_UNSUPPORTED, "layer %lld is not an MoE layer", static_cast<long long>(l));
      fmx_moe_weights& mw = lw.moe;
      mw = fmx_moe_weights{};
      FMX_RC(up.router_rows(mp + ".gate", E, H, &mw.router_w, &mw.router_scales, &mw.router_biases));
      void* packed = nullptr;
      FMX_RC(up.alloc(moe_bytes, &packed));
      uint8_t* pk = static_cast<uint8_t*>(packed);
      for (int64_t e = 0; e < E; ++e) {
        const std::string ep = mp + ".experts." + std::to_string(e);
        up.stage_used = 0;
        fmx_qweight g{}, u{}, d{};
        FMX_RC(up.quant(ep + ".gate_proj", I, H, &g));
        FMX_RC(up.quant(ep + ".up_proj", I, H, &u));
        FMX_HIP(pack(g, &u, I, H, pk + gu + e * gu_es, stream));
        FMX_HIP(hipStreamSynchronize(stream));  // staging reused below
        up.stage_used = 0;
        FMX_RC(up.quant(ep + ".down_proj", H, I, &d));
        FMX_HIP(pack(d, nullptr, H, I, pk + dn + e * dn_es, stream));
        FMX_HIP(hipStreamSynchronize(stream));
      }
      if (Is > 0) {
        const std::string sp = mp + ".shared_expert";
        up.stage_used = 0;
        fmx_qweight g{}, u{}, d{};
        FMX_RC(up.quant(sp + ".gate_proj", Is, H, &g));
        FMX_RC(up.quant(sp + ".up_proj", Is, H, &u));
        FMX_HIP(pack(g, &u, Is, H, pk + sgu, stream));
        FMX_HIP(hipStreamSynchronize(stream));
        up.stage_used = 0;
        FMX_RC(up.quant(sp + ".down_proj", H, Is, &d));
        FMX_HIP(pack(d, nullptr, H, Is, pk + sdn, stream));
        FMX_HIP(hipStreamSynchronize(stream));
        FMX_RC(up.router_rows(mp + ".shared_expert_gate", 1, H, &mw.shared_expert_gate_w,
                              &mw.shared_expert_gate_scales, &mw.shared_expert_gate_biases));
      }
      mw.packed = packed;
      mw.packed_bytes = moe_bytes;
    }
    // embedding: dequantized once to a bf16 table (model.cpp:214-224), or
    // bf16 as stored; lm_head packed, or the embedding's quantized arrays
    // when the embeddings are tied (model.cpp:499-512)
    void* embed = nullptr;
    FMX_RC(up.alloc(static_cast<size_t>(V * H * 2), &embed));
    up.stage_used = 0;
    fmx_qweight eq{};
    const bool embed_q = ck.find("embed_tokens.scales") != nullptr;
    if (embed_q) {
      FMX_RC(up.quant("embed_tokens", V, H, &eq));
      FMX_HIP(launch_dequantize(static_cast<const uint32_t*>(eq.w), static_cast<const uint16_t*>(eq.scales),
                                static_cast<const uint16_t*>(eq.biases), V * H / 64, static_cast<uint16_t*>(embed),
                                stream));
    } else {
      FMX_RC(up.read("embed_tokens.weight", "BF16", {V, H}, embed));
    }
    void* head = nullptr;
    FMX_RC(up.alloc(static_cast<size_t>(packed_linear(V, H)), &head));
    if (ck.find("lm_head.weight")) {
      FMX_HIP(hipStreamSynchronize(stream));
      up.stage_used = 0;
      fmx_qweight hq{};
      FMX_RC(up.quant("lm_head", V, H, &hq));
      FMX_HIP(pack(hq, nullptr, V, H, static_cast<uint8_t*>(head), stream));
    } else if (embed_q) {
      FMX_HIP(pack(eq, nullptr, V, H, static_cast<uint8_t*>(head), stream));
    } else {
      return fail(FMX_ERR_UNSUPPORTED, "no lm_head and an unquantized embedding");
    }
    FMX_RC(up.own("norm.weight", "BF16", {H}, &m->w.norm_w));
    FMX_HIP(hipStreamSynchronize(stream));
    m->w.embed = embed;
    m->w.lm_head = head;
    m->w.layers = m->layers.data();
    return FMX_OK;
  };
  const int rc = body();
  if (rc) {
    (void)hipStreamSynchronize(stream);
    delete m;
    return rc;
  }
  *out = m;
  clear_error();
  return FMX_OK;
}

const fmx_model_weights* fmx_loaded_model_weights(const fmx_loaded_model* m) { return m ? &m->w : nullptr; }

size_t fmx_loaded_model_device_bytes(const fmx_loaded_model* m) { return m ? m->bytes : 0; }

void fmx_loaded_model_free(fmx_loaded_model* m) { delete m; }

}  // extern "C"
