// fmx_sched.cpp -- the server loop's batched decode (include/fmx_model.h):
// requests admitted into the slots of a KV pool, prefilled one at a time,
// and decoded together, one greedy token per live request per step.
//
// Reference: server/src/scheduler.cpp:19-101 (BatchScheduler submit / step /
// has_work / drain_completed / active_count), :103-232 (prefill_request:
// slot, batch-1 prefill at offset 0, first token from the last position),
// :527-680 (decode_batched: every live request's next token, one batched
// forward, argmax, per-request append and done check), kv_pool.cpp (slots of
// max_context positions). The pool here is the decoder stack's KV cache
// itself: a live request keeps its slot, and a decode step passes every
// request's slot and cache offset to fmx_model_forward_batched, so no cache
// is copied into a left-padded batch cache or flushed back
// (batch_kv_cache.cpp:10-91, scheduler.cpp:556-576, :658-678).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <deque>
#include <map>
#include <mutex>
#include <vector>

#include "../../include/fmx_model.h"
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

// A cached prompt: its tokens and the keys/values of its positions 0 .. n-2
// in a compact buffer [layers][2][nkv][max_prompt][hd].
struct PrefixEntry {
  std::vector<int32_t> tokens;
  void* kv = nullptr;
};

struct Request {
  std::vector<int32_t> prompt;
  int64_t max_tokens = 0;
  int slot = -1;          // KV pool slot while active
  int64_t offset = 0;     // cache positions filled
  int64_t generated = 0;
  int32_t next = 0;       // the latest token, the next step's input
};

}  // namespace

struct fmx_scheduler {
  fmx_model_config cfg{};
  const fmx_model_weights* w = nullptr;
  hipStream_t stream = nullptr;
  int64_t n_slots = 0, max_context = 0, max_prompt = 0, V = 0;
  void *kv = nullptr, *ws = nullptr, *logits = nullptr;
  size_t ws_bytes = 0;
  int32_t *d_ids = nullptr, *d_offs = nullptr, *d_slots = nullptr, *d_next = nullptr;
  int32_t* h_buf = nullptr;  // pinned: ids, offsets, slots going up; next tokens coming back
  // pending queue: written by submit (any thread), read by step
  std::mutex pending_mu;
  std::deque<std::pair<int64_t, Request>> pending;
  int64_t next_id = 0;
  // active requests by id (ids grow with submission, so this is also the
  // batch order of a decode step) and the free slots: touched by step only.
  // Other threads read the counts: n_live = requests submitted and not yet
  // completed (pending, being prefilled or active), n_active = active.size()
  std::map<int64_t, Request> active;
  std::vector<int> free_slots;
  std::atomic<int64_t> n_live{0}, n_active{0};
  std::mutex completed_mu;
  std::vector<int64_t> completed;
  // decode step of batch B (forward + argmax) as a HIP graph, captured on
  // the second step of that batch size; its inputs are the device ids,
  // offsets and slots, refilled before every launch
  std::vector<hipGraphExec_t> graphs;
  std::vector<int> uses;
  // prefix cache (oldest first) and its free entry buffers
  int64_t pc_max = 0, pc_hits = 0;
  std::deque<PrefixEntry> pc;
  std::vector<void*> pc_free;
  void free_prefix_cache() {
    for (auto& e : pc) pc_free.push_back(e.kv);
    pc.clear();
    for (void* p : pc_free) (void)hipFree(p);
    pc_free.clear();
    pc_max = 0;
  }
  ~fmx_scheduler() {
    free_prefix_cache();
    for (hipGraphExec_t g : graphs)
      if (g) (void)hipGraphExecDestroy(g);
    for (void* p : {kv, ws, logits, static_cast<void*>(d_ids), static_cast<void*>(d_offs),
                    static_cast<void*>(d_slots), static_cast<void*>(d_next)})
      if (p) (void)hipFree(p);
    if (h_buf) (void)hipHostFree(h_buf);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

namespace {

KvCopyArgs kv_copy_args(const fmx_scheduler& s, void* entry, int slot, int64_t n_pos, int to_cache) {
  const fmx_model_config& c = s.cfg;
  KvCopyArgs k{};
  k.cache = static_cast<uint16_t*>(s.kv);
  k.entry = static_cast<uint16_t*>(entry);
  k.layers = c.num_hidden_layers;
  k.cache_batch = s.n_slots;
  k.nkv = c.num_key_value_heads;
  k.max_seq = s.max_context;
  k.hd = c.head_dim ? c.head_dim : c.hidden_size / c.num_attention_heads;
  k.cap = s.max_prompt;
  k.n_pos = n_pos;
  k.slot = slot;
  k.to_cache = to_cache;
  return k;
}

// prefill_request with a prefix-cache hit (scheduler.cpp:121-168): the cached
// keys/values of positions 0 .. n-2 into the slot, then the last prompt
// token alone at offset n-1 (a decode step) gives the first token
int prefill_cached(fmx_scheduler& s, Request& r, const PrefixEntry& e) {
  const int64_t n = static_cast<int64_t>(r.prompt.size());
  int32_t* h = s.h_buf;
  h[0] = r.prompt.back();
  h[1] = r.slot;
  FMX_HIP(launch_kv_copy(kv_copy_args(s, e.kv, r.slot, n - 1, 1), s.stream));
  FMX_HIP(hipMemcpyAsync(s.d_ids, h, 4, hipMemcpyHostToDevice, s.stream));
  FMX_HIP(hipMemcpyAsync(s.d_slots, h + 1, 4, hipMemcpyHostToDevice, s.stream));
  FMX_RC(fmx_model_forward_batched(&s.cfg, s.w, s.d_ids, 1, 1, n - 1, nullptr, s.d_slots, s.kv, s.n_slots,
                                   s.max_context, 1, s.logits, s.ws, s.ws_bytes, s.stream, nullptr));
  FMX_RC(fmx_greedy_next(s.logits, 1, s.V, s.V, s.d_next, nullptr, 0, s.stream));
  FMX_HIP(hipMemcpyAsync(h, s.d_next, 4, hipMemcpyDeviceToHost, s.stream));
  FMX_HIP(hipStreamSynchronize(s.stream));
  r.offset = n;
  r.next = h[0];
  r.generated = 1;
  s.pc_hits += 1;
  return FMX_OK;
}

// prefill_request (scheduler.cpp:103-211): batch-1 prefill of the prompt into
// slot r.slot at offset 0, first token = argmax of the last position; with
// the prefix cache on, a prompt seen before takes prefill_cached, and a new
// one is cached afterwards (:213-231), the oldest entry making room
int prefill(fmx_scheduler& s, Request& r) {
  const int64_t n = static_cast<int64_t>(r.prompt.size());
  const bool cacheable = s.pc_max > 0 && n > 1;
  if (cacheable)
    for (const PrefixEntry& e : s.pc)
      if (e.tokens == r.prompt) return prefill_cached(s, r, e);
  int32_t* h = s.h_buf;
  for (int64_t i = 0; i < n; ++i) h[i] = r.prompt[static_cast<size_t>(i)];
  h[n] = r.slot;
  FMX_HIP(hipMemcpyAsync(s.d_ids, h, static_cast<size_t>(n * 4), hipMemcpyHostToDevice, s.stream));
  FMX_HIP(hipMemcpyAsync(s.d_slots, h + n, 4, hipMemcpyHostToDevice, s.stream));
  FMX_RC(fmx_model_forward_batched(&s.cfg, s.w, s.d_ids, 1, n, 0, nullptr, s.d_slots, s.kv, s.n_slots,
                                   s.max_context, 1, s.logits, s.ws, s.ws_bytes, s.stream, nullptr));
  FMX_RC(fmx_greedy_next(s.logits, 1, s.V, s.V, s.d_next, nullptr, 0, s.stream));
  FMX_HIP(hipMemcpyAsync(h, s.d_next, 4, hipMemcpyDeviceToHost, s.stream));
  if (cacheable) {
    PrefixEntry e;
    if (static_cast<int64_t>(s.pc.size()) >= s.pc_max) {
      e.kv = s.pc.front().kv;
      s.pc.pop_front();
    } else {
      e.kv = s.pc_free.back();
      s.pc_free.pop_back();
    }
    e.tokens = r.prompt;
    const hipError_t ce = launch_kv_copy(kv_copy_args(s, e.kv, r.slot, n - 1, 0), s.stream);
    if (ce != hipSuccess) {
      s.pc_free.push_back(e.kv);  // the evicted (or free) buffer stays the cache's
      return fail(FMX_ERR_HIP, "launch_kv_copy: %s", hipGetErrorString(ce));
    }
    s.pc.push_back(std::move(e));
  }
  FMX_HIP(hipStreamSynchronize(s.stream));
  r.offset = n;
  r.next = h[0];
  r.generated = 1;
  return FMX_OK;
}

// decode_batched (scheduler.cpp:527-627): one token for every request of live
int decode(fmx_scheduler& s, const std::vector<Request*>& live) {
  const int64_t B = static_cast<int64_t>(live.size());
  int32_t* h = s.h_buf;
  for (int64_t b = 0; b < B; ++b) {
    h[b] = live[static_cast<size_t>(b)]->next;
    h[B + b] = static_cast<int32_t>(live[static_cast<size_t>(b)]->offset);
    h[2 * B + b] = live[static_cast<size_t>(b)]->slot;
  }
  FMX_HIP(hipMemcpyAsync(s.d_ids, h, static_cast<size_t>(B * 4), hipMemcpyHostToDevice, s.stream));
  FMX_HIP(hipMemcpyAsync(s.d_offs, h + B, static_cast<size_t>(B * 4), hipMemcpyHostToDevice, s.stream));
  FMX_HIP(hipMemcpyAsync(s.d_slots, h + 2 * B, static_cast<size_t>(B * 4), hipMemcpyHostToDevice, s.stream));
  auto launch = [&]() -> int {
    FMX_RC(fmx_model_forward_batched(&s.cfg, s.w, s.d_ids, B, 1, 0, s.d_offs, s.d_slots, s.kv, s.n_slots,
                                     s.max_context, 1, s.logits, s.ws, s.ws_bytes, s.stream, nullptr));
    return fmx_greedy_next(s.logits, B, s.V, s.V, s.d_next, nullptr, 0, s.stream);
  };
  hipGraphExec_t& exec = s.graphs[static_cast<size_t>(B)];
  if (!exec && ++s.uses[static_cast<size_t>(B)] >= 2) {
    FMX_HIP(hipStreamBeginCapture(s.stream, hipStreamCaptureModeThreadLocal));
    const int rc = launch();
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(s.stream, &g);
    if (rc) {
      if (g) (void)hipGraphDestroy(g);
      return rc;
    }
    if (e != hipSuccess) return fail(FMX_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
    const hipError_t ei = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (ei != hipSuccess) {
      exec = nullptr;
      return fail(FMX_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(ei));
    }
  }
  if (exec)
    FMX_HIP(hipGraphLaunch(exec, s.stream));
  else
    FMX_RC(launch());
  int32_t* back = h + 3 * B;
  FMX_HIP(hipMemcpyAsync(back, s.d_next, static_cast<size_t>(B * 4), hipMemcpyDeviceToHost, s.stream));
  FMX_HIP(hipStreamSynchronize(s.stream));
  for (int64_t b = 0; b < B; ++b) {
    Request& r = *live[static_cast<size_t>(b)];
    r.next = back[b];
    r.generated += 1;
    r.offset += 1;
  }
  return FMX_OK;
}

}  // namespace

extern "C" {

int fmx_scheduler_create(const fmx_model_config* cfg, const fmx_model_weights* w, int64_t n_slots,
                         int64_t max_context, int64_t max_prompt, fmx_stream stream, fmx_scheduler** out) {
  if (!cfg || !w || !out) return fail(FMX_ERR_ARG, "NULL argument");
  *out = nullptr;
  if (n_slots < 1 || n_slots > FMX_SCHED_MAX_SLOTS || max_prompt < 1 || max_context < max_prompt + 1)
    return fail(FMX_ERR_SHAPE, "n_slots %lld (1..%d), max_context %lld, max_prompt %lld", (long long)n_slots,
                FMX_SCHED_MAX_SLOTS, (long long)max_context, (long long)max_prompt);
  const size_t kv = fmx_model_kv_cache_size(cfg, n_slots, max_context);
  const int64_t max_tokens = max_prompt > n_slots ? max_prompt : n_slots;
  const size_t wsb = fmx_model_workspace_size(cfg, max_tokens);
  if (!kv || !wsb)
    return fail(FMX_ERR_UNSUPPORTED, "config, max_context %lld or max_prompt %lld outside the decoder stack's limits",
                (long long)max_context, (long long)max_prompt);
  auto s = new fmx_scheduler();
  s->cfg = *cfg;
  s->w = w;
  s->graphs.assign(static_cast<size_t>(n_slots + 1), nullptr);
  s->uses.assign(static_cast<size_t>(n_slots + 1), 0);
  s->n_slots = n_slots;
  s->max_context = max_context;
  s->max_prompt = max_prompt;
  s->V = cfg->vocab_size;
  s->ws_bytes = wsb;
  auto body = [&]() -> int {
    // the weights are ready once the caller's stream is; the scheduler
    // works on a stream of its own (a capturable one)
    FMX_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    FMX_HIP(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking));
    FMX_HIP(hipMalloc(&s->kv, kv));
    FMX_HIP(hipMalloc(&s->ws, wsb));
    FMX_HIP(hipMalloc(&s->logits, static_cast<size_t>(n_slots * s->V * 2)));
    FMX_HIP(hipMalloc(reinterpret_cast<void**>(&s->d_ids), static_cast<size_t>(max_tokens * 4)));
    FMX_HIP(hipMalloc(reinterpret_cast<void**>(&s->d_offs), static_cast<size_t>(n_slots * 4)));
    FMX_HIP(hipMalloc(reinterpret_cast<void**>(&s->d_slots), static_cast<size_t>(n_slots * 4)));
    FMX_HIP(hipMalloc(reinterpret_cast<void**>(&s->d_next), static_cast<size_t>(n_slots * 4)));
    FMX_HIP(hipHostMalloc(reinterpret_cast<void**>(&s->h_buf),
                          static_cast<size_t>((max_tokens + 4 * n_slots + 4) * 4), hipHostMallocDefault));
    FMX_RC(fmx_model_workspace_init(cfg, s->ws, wsb, s->stream));
    FMX_HIP(hipStreamSynchronize(s->stream));
    for (int64_t i = n_slots - 1; i >= 0; --i) s->free_slots.push_back(static_cast<int>(i));
    return FMX_OK;
  };
  const int rc = body();
  if (rc) {
    delete s;
    return rc;
  }
  *out = s;
  clear_error();
  return FMX_OK;
}

int fmx_scheduler_submit(fmx_scheduler* s, const int32_t* prompt, int64_t n, int64_t max_tokens,
                         float temperature, int64_t* request_id) {
  if (!s || !prompt || !request_id) return fail(FMX_ERR_ARG, "NULL argument");
  if (temperature != 0.0f)
    return fail(FMX_ERR_UNSUPPORTED, "temperature %g: only greedy decoding (temperature 0)", (double)temperature);
  if (n < 1 || n > s->max_prompt)
    return fail(FMX_ERR_SHAPE, "prompt of %lld tokens (1..%lld)", (long long)n, (long long)s->max_prompt);
  if (max_tokens < 1 || n + max_tokens > s->max_context)
    return fail(FMX_ERR_SHAPE, "%lld prompt + %lld new tokens exceed the %lld positions of a slot", (long long)n,
                (long long)max_tokens, (long long)s->max_context);
  for (int64_t i = 0; i < n; ++i)
    if (prompt[i] < 0 || prompt[i] >= s->V)
      return fail(FMX_ERR_ARG, "prompt token %d outside the vocabulary of %lld", prompt[i], (long long)s->V);
  Request r;
  r.prompt.assign(prompt, prompt + n);
  r.max_tokens = max_tokens;
  {
    std::lock_guard<std::mutex> lock(s->pending_mu);
    const int64_t id = s->next_id++;
    s->pending.emplace_back(id, std::move(r));
    s->n_live.fetch_add(1);
    *request_id = id;
  }
  clear_error();
  return FMX_OK;
}

int fmx_scheduler_step(fmx_scheduler* s, int64_t* request_ids, int32_t* tokens, int64_t capacity,
                       int64_t* n_new) {
  if (!s || !n_new || !request_ids || !tokens) return fail(FMX_ERR_ARG, "NULL argument");
  if (capacity < 2 * s->n_slots)
    return fail(FMX_ERR_SHAPE, "capacity %lld < 2 * n_slots (%lld)", (long long)capacity, (long long)s->n_slots);
  int64_t n = 0;
  auto emit = [&](int64_t id, int32_t tok) {
    request_ids[n] = id;
    tokens[n] = tok;
    ++n;
  };
  std::vector<int64_t> done;
  // 1. admit pending requests while slots are free (scheduler.cpp:28-42):
  // each is taken off the queue under the lock and prefilled outside it, so
  // submit never waits for a prefill
  while (!s->free_slots.empty()) {
    int64_t id;
    Request r;
    {
      std::lock_guard<std::mutex> lock(s->pending_mu);
      if (s->pending.empty()) break;
      id = s->pending.front().first;
      r = std::move(s->pending.front().second);
      s->pending.pop_front();
    }
    r.slot = s->free_slots.back();
    s->free_slots.pop_back();
    const int rc = prefill(*s, r);
    if (rc) {
      // the request goes back to the head of the queue, its slot back to
      // the pool: a later step retries it, nothing is lost
      s->free_slots.push_back(r.slot);
      r.slot = -1;
      {
        std::lock_guard<std::mutex> lock(s->pending_mu);
        s->pending.emplace_front(id, std::move(r));
      }
      *n_new = n;
      return rc;
    }
    emit(id, r.next);
    // a request for one token is done after its prefill
    if (r.generated >= r.max_tokens) done.push_back(id);
    s->active.emplace(id, std::move(r));
    s->n_active.fetch_add(1);
  }
  // 2. one decode step of every request still decoding (scheduler.cpp:44-69)
  std::vector<Request*> live;
  std::vector<int64_t> live_ids;
  for (auto& kv : s->active)
    if (kv.second.generated < kv.second.max_tokens) {
      live.push_back(&kv.second);
      live_ids.push_back(kv.first);
    }
  if (!live.empty()) {
    const int rc = decode(*s, live);
    if (rc) {
      *n_new = n;
      return rc;
    }
    for (size_t b = 0; b < live.size(); ++b) {
      emit(live_ids[b], live[b]->next);
      if (live[b]->generated >= live[b]->max_tokens) done.push_back(live_ids[b]);
    }
  }
  // 3. free the slots of completed requests (scheduler.cpp:71-82)
  if (!done.empty()) {
    std::lock_guard<std::mutex> lock(s->completed_mu);
    for (int64_t id : done) {
      auto it = s->active.find(id);
      s->free_slots.push_back(it->second.slot);
      s->active.erase(it);
      s->n_active.fetch_sub(1);
      s->completed.push_back(id);
      s->n_live.fetch_sub(1);
    }
  }
  *n_new = n;
  clear_error();
  return FMX_OK;
}

int fmx_scheduler_has_work(fmx_scheduler* s) { return s && s->n_live.load() > 0; }

int64_t fmx_scheduler_active_count(const fmx_scheduler* s) { return s ? s->n_active.load() : 0; }

int fmx_scheduler_drain_completed(fmx_scheduler* s, int64_t* request_ids, int64_t capacity, int64_t* n) {
  if (!s || !n || (capacity > 0 && !request_ids)) return fail(FMX_ERR_ARG, "NULL argument");
  std::lock_guard<std::mutex> lock(s->completed_mu);
  const int64_t m = static_cast<int64_t>(s->completed.size());
  const int64_t take = m < capacity ? m : capacity;
  for (int64_t i = 0; i < take; ++i) request_ids[i] = s->completed[static_cast<size_t>(i)];
  s->completed.erase(s->completed.begin(), s->completed.begin() + take);
  *n = take;
  clear_error();
  return FMX_OK;
}

int fmx_scheduler_set_prefix_cache(fmx_scheduler* s, int64_t max_entries) {
  if (!s) return fail(FMX_ERR_ARG, "NULL scheduler");
  if (max_entries < 0 || max_entries > FMX_SCHED_MAX_PREFIX_ENTRIES)
    return fail(FMX_ERR_SHAPE, "max_entries %lld (0..%d)", (long long)max_entries, FMX_SCHED_MAX_PREFIX_ENTRIES);
  s->free_prefix_cache();
  const fmx_model_config& c = s->cfg;
  const int64_t hd = c.head_dim ? c.head_dim : c.hidden_size / c.num_attention_heads;
  const size_t bytes = static_cast<size_t>(c.num_hidden_layers * 2 * c.num_key_value_heads * s->max_prompt * hd * 2);
  for (int64_t i = 0; i < max_entries; ++i) {
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
      s->free_prefix_cache();
      return fail(FMX_ERR_HIP, "prefix cache entry %lld of %zu bytes: %s", (long long)i, bytes, hipGetErrorString(e));
    }
    s->pc_free.push_back(p);
  }
  s->pc_max = max_entries;
  clear_error();
  return FMX_OK;
}

int64_t fmx_scheduler_prefix_hits(const fmx_scheduler* s) { return s ? s->pc_hits : 0; }

void fmx_scheduler_free(fmx_scheduler* s) { delete s; }

}  // extern "C"
