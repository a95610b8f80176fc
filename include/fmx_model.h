/*
 * fmx_model.h -- C-ABI of the decoder stack around the MoE block (libfmx.so).
 *
 * Replaces LlamaModel's forward for MoE models (every layer MoE, as
 * Qwen1.5-MoE-A2.7B): embedding, per layer RMSNorm -> attention (q/k/v
 * linears with biases, RoPE, KV cache, scaled dot-product attention, o_proj)
 * -> residual -> RMSNorm -> MoE block (fmx_moe_block_forward) -> residual,
 * then the final RMSNorm and lm_head. Conventions as in fmx.h: device
 * pointers, asynchronous on `stream`, status codes, no allocation when a
 * workspace is given.
 *
 * Linear weights are read in the packed layout of fmx_pack_linear (the same
 * 0.5625 bytes per weight as MLX's affine 4-bit, group 64 arrays).
 */
#ifndef FMX_MODEL_H
#define FMX_MODEL_H

#include "fmx.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ModelConfig (server/include/flashmlx/model.h:20-54) for an all-MoE
 * decoder: head_dim = hidden_size / num_attention_heads when 0. Limits:
 * hidden_size and num_attention_heads * head_dim multiples of 128 (and
 * hidden_size <= 8192), head_dim a multiple of 8 and <= 256,
 * num_attention_heads a multiple of num_key_value_heads, vocab_size a
 * multiple of 16, max_position_embeddings <= 32768 (the RoPE table); a KV
 * cache holds at most 4096 positions per sequence. */
typedef struct fmx_model_config {
  int64_t hidden_size;
  int64_t num_hidden_layers;
  int64_t num_attention_heads;
  int64_t num_key_value_heads;
  int64_t head_dim;
  int64_t vocab_size;
  int64_t max_position_embeddings;
  float rms_norm_eps;
  float rope_theta;
  fmx_moe_config moe; /* every layer's MoE block */
} fmx_model_config;

/* One layer (LlamaModel::LayerWeights, model.h:242-254, and MoEWeights).
 * qkv: the q, k and v linears packed one after the other (fmx_pack_linear
 * with three parts); qkv_bias: the q, k and v linear biases
 * (model.cpp:864-866) concatenated, bf16 [(nh + 2 nkv) * hd], or NULL. */
typedef struct fmx_layer_weights {
  const void* input_norm_w; /* bf16 [H] */
  const void* post_norm_w;  /* bf16 [H] */
  const void* qkv;          /* packed [(nh + 2 nkv) * hd, H] */
  const void* qkv_bias;
  const void* o;            /* packed [H, nh * hd] */
  fmx_moe_weights moe;
} fmx_layer_weights;

/* embed: the embedding table as bf16 [V, H] (the reference dequantizes a
 * quantized table once at load, model.cpp:214-224, and gathers rows from it,
 * :490-497); lm_head: packed [V, H] (model.cpp:499-521); layers: a host
 * array of num_hidden_layers entries. */
typedef struct fmx_model_weights {
  const void* embed;
  const void* norm_w; /* bf16 [H] */
  const void* lm_head;
  const fmx_layer_weights* layers;
} fmx_model_weights;

/* Load-time packing of a quantized linear (replaces the per-call
 * quantized_matmul operands of LlamaModel::linear_fast, model.cpp:476-480):
 * n_parts MLX-layout matrices of rows[i] x K (w u32 [rows, K/8], scales and
 * biases bf16 [rows, K/64]) stacked into one packed matrix of sum(rows) rows.
 * K a multiple of 128, every rows[i] a multiple of 16. */
size_t fmx_packed_linear_size(int64_t n_rows, int64_t K);
int fmx_pack_linear(const fmx_qweight* parts, const int64_t* rows, int n_parts, int64_t K,
                    void* packed, size_t packed_bytes, fmx_stream stream);

/* KV cache of the stack: keys and values of every layer, bf16
 * [layers][2][cache_batch][nkv][cache_max_seq][hd]. */
size_t fmx_model_kv_cache_size(const fmx_model_config* cfg, int64_t cache_batch,
                               int64_t cache_max_seq);

/* Workspace for forwards of up to max_tokens = batch * seq_len tokens,
 * including the RoPE table; fmx_model_workspace_init fills the table and
 * prepares the MoE blocks' counters (once, before the first forward). */
size_t fmx_model_workspace_size(const fmx_model_config* cfg, int64_t max_tokens);
int fmx_model_workspace_init(const fmx_model_config* cfg, void* workspace,
                             size_t workspace_bytes, fmx_stream stream);

/* logits = forward(input_ids) (LlamaModel::forward, model.cpp:1021-1033):
 *   input_ids int32 [batch, seq_len] (device); sequence b's tokens sit at
 *   cache positions offset(b) .. offset(b) + seq_len - 1, where offset(b) =
 *   cache_offsets[b] (device int32 [batch], per-sequence offsets as in
 *   forward_heterogeneous, model.cpp:990-1019) or cache_offset when
 *   cache_offsets is NULL. Each layer writes the new keys/values into
 *   kv_cache (sequence b in cache slot b < cache_batch) and attends causally
 *   to positions 0 .. its own. Device offsets are clamped to the cache.
 *   logits bf16 [batch, seq_len, V], or [batch, V] (the last position of
 *   each sequence) when logits_last_only. */
int fmx_model_forward(const fmx_model_config* cfg, const fmx_model_weights* w,
                      const int32_t* input_ids, int64_t batch, int64_t seq_len,
                      int64_t cache_offset, const int32_t* cache_offsets, void* kv_cache,
                      int64_t cache_batch, int64_t cache_max_seq, int logits_last_only,
                      void* logits, void* workspace, size_t workspace_bytes, fmx_stream stream);

/* fmx_model_forward that also copies each layer's expert choice into
 * routing (device u32 [layers][batch * seq_len][k], the MoE block's inds in
 * token order, slots ordered as fmx_moe_block_forward orders them). A
 * debugging view, as LlamaModel's debug_forward (model.h:125): lets a
 * reference run take the same expert choice where a router is at a near-tie. */
int fmx_model_forward_traced(const fmx_model_config* cfg, const fmx_model_weights* w,
                             const int32_t* input_ids, int64_t batch, int64_t seq_len,
                             int64_t cache_offset, const int32_t* cache_offsets, void* kv_cache,
                             int64_t cache_batch, int64_t cache_max_seq, int logits_last_only,
                             void* logits, void* workspace, size_t workspace_bytes,
                             fmx_stream stream, uint32_t* routing);

/* fmx_model_forward_traced whose sequence b keeps its keys and values in
 * cache slot cache_slots[b] (device int32 [batch], each < cache_batch and
 * distinct; clamped to the cache) instead of slot b: the batched decode of
 * the scheduler (forward_batched_inplace, model.h:116-123, over the slots of
 * a KV pool) runs any subset of live sequences without copying caches into
 * a batch cache and back (scheduler.cpp:556-576, :658-678). NULL slots:
 * slot b; NULL routing: no record. */
int fmx_model_forward_batched(const fmx_model_config* cfg, const fmx_model_weights* w,
                              const int32_t* input_ids, int64_t batch, int64_t seq_len,
                              int64_t cache_offset, const int32_t* cache_offsets,
                              const int32_t* cache_slots, void* kv_cache, int64_t cache_batch,
                              int64_t cache_max_seq, int logits_last_only, void* logits,
                              void* workspace, size_t workspace_bytes, fmx_stream stream,
                              uint32_t* routing);

/* The residual stream after the last layer of the latest forward on this
 * workspace, bf16 [n_tokens, H] (every row when that forward returned the
 * logits of every position; the last position of each sequence otherwise).
 * Valid until the next call on the workspace. A debugging view, as
 * LlamaModel's debug_forward / debug_embed (model.h:125-126). */
int fmx_model_workspace_hidden(const fmx_model_config* cfg, int64_t n_tokens, const void* workspace,
                               const void** hidden);

/* ------------------------------------------------------------------------
 * Quantized-checkpoint loader (LlamaModel::load_config / load_weights /
 * build_weight_cache / build_moe_weight_cache, model.cpp:100-470)
 * --------------------------------------------------------------------- */

/* config.json of an MLX checkpoint -> fmx_model_config, with the keys and
 * defaults of load_config (model.cpp:111-140): quantization.bits /
 * group_size into cfg->moe.quant_bits / quant_group_size. The host-side
 * parse only; tie_word_embeddings (may be NULL) receives that key. */
int fmx_model_config_from_json(const char* config_json_path, fmx_model_config* cfg,
                               int32_t* tie_word_embeddings);

/* Metadata of one tensor of a checkpoint directory (every *.safetensors
 * file, in name order; a "model." key prefix dropped, model.cpp:160-170):
 * dtype ("BF16", "U32", ...; 8 bytes), shape (up to 8 dims), ndim. Host-side. */
int fmx_checkpoint_tensor(const char* dir, const char* name, char* dtype, int64_t* shape,
                          int32_t* ndim);

/* Loads an all-MoE checkpoint (MLX affine 4-bit, group 64; keys
 * layers.N.{input_layernorm, post_attention_layernorm}.weight,
 * layers.N.self_attn.{q,k,v,o}_proj.{weight,scales,biases} (+ q/k/v .bias),
 * layers.N.mlp.gate.*, layers.N.mlp.experts.E.{gate,up,down}_proj.*,
 * layers.N.mlp.shared_expert.* and .shared_expert_gate.*, embed_tokens.*,
 * norm.weight, lm_head.* (or the embedding's when tied)) into device memory
 * the returned object owns: each tensor is read once and packed in place
 * (experts one by one), so the expert weights exist once, in the packed
 * layout; the embedding is dequantized to bf16 as the reference does at
 * load. Synchronous on `stream`. Missing tensors, wrong dtypes or shapes
 * return an error naming the tensor. */
typedef struct fmx_loaded_model fmx_loaded_model;
int fmx_model_load(const char* dir, const fmx_model_config* cfg, fmx_loaded_model** out,
                   fmx_stream stream);
const fmx_model_weights* fmx_loaded_model_weights(const fmx_loaded_model* model);
size_t fmx_loaded_model_device_bytes(const fmx_loaded_model* model);
void fmx_loaded_model_free(fmx_loaded_model* model);

/* ------------------------------------------------------------------------
 * Batched decode of a server loop (BatchScheduler, scheduler.h:37-99,
 * scheduler.cpp:19-101, :103-232, :527-680)
 * --------------------------------------------------------------------- */

/* A KV pool of n_slots slots of max_context positions (KVCachePool,
 * kv_pool.cpp) with a request queue. Each step admits queued requests while
 * slots are free (a batch-1 prefill into the slot; the first token is the
 * argmax of the prompt's last position), then decodes every active request
 * one greedy token in one fmx_model_forward_batched over the requests' own
 * slots and offsets (no batch cache is built or flushed), then frees the
 * slots of requests that reached max_tokens. With at most 16 requests
 * decoding, every kernel computes a request's row on its own, so its tokens
 * equal those of the request decoded alone (fmx_model_forward + argmax).
 * All device memory is allocated at create; `weights` must outlive the
 * scheduler. create waits for `stream` (the one the weights were made on);
 * the scheduler then works on a stream of its own, and each step returns
 * with its work finished. The decode step of each batch size runs as a HIP
 * graph from the second time that size occurs. */
#define FMX_SCHED_MAX_SLOTS 256
typedef struct fmx_scheduler fmx_scheduler;
int fmx_scheduler_create(const fmx_model_config* cfg, const fmx_model_weights* weights,
                         int64_t n_slots, int64_t max_context, int64_t max_prompt,
                         fmx_stream stream, fmx_scheduler** out);

/* BatchScheduler::submit (scheduler.cpp:19-23): queues a request, safe to
 * call from another thread than the one that steps. prompt: host int32 [n],
 * 1 <= n <= max_prompt, each token < vocab; n + max_tokens <= max_context.
 * temperature other than 0 (sampling, sampling.cpp) returns
 * FMX_ERR_UNSUPPORTED. The request's id goes to *request_id. */
int fmx_scheduler_submit(fmx_scheduler* s, const int32_t* prompt, int64_t n, int64_t max_tokens,
                         float temperature, int64_t* request_id);

/* BatchScheduler::step (scheduler.cpp:25-85): admit, decode, clean up. The
 * tokens generated in this step go to (request_ids[i], tokens[i]) for
 * i < *n_new (a request admitted in this step gets its first token and its
 * second); capacity >= 2 * n_slots. A request finishes with exactly
 * max_tokens tokens (the reference decodes one more past its first token
 * when max_tokens is 1). One thread steps; a queued request is taken off
 * the queue under its lock and prefilled outside it, so submit does not wait
 * for prefills. A prefill that fails puts its request back at the head of
 * the queue (its slot freed) and step returns the error; the tokens emitted
 * before it in that step are in the outputs (*n_new). */
int fmx_scheduler_step(fmx_scheduler* s, int64_t* request_ids, int32_t* tokens, int64_t capacity,
                       int64_t* n_new);

/* BatchScheduler::has_work / active_count / drain_completed
 * (scheduler.cpp:87-101): requests submitted and not yet finished (1/0);
 * active requests; ids of requests finished since the last drain (up to
 * capacity, oldest first). Safe to call from any thread while another
 * steps. */
int fmx_scheduler_has_work(fmx_scheduler* s);
int64_t fmx_scheduler_active_count(const fmx_scheduler* s);
int fmx_scheduler_drain_completed(fmx_scheduler* s, int64_t* request_ids, int64_t capacity,
                                  int64_t* n);

/* The prefix cache of prefill_request (scheduler.cpp:121-168, :213-231; 32
 * entries at scheduler.h:78): the keys and values of up to max_entries
 * prompts of more than one token are kept (positions 0 .. n-2, device
 * memory allocated by this call: layers * 2 * nkv * max_prompt * hd bf16
 * per entry). A request whose prompt equals a cached one copies them into
 * its slot and forwards only its last prompt token (a decode step) for its
 * first token, as the reference does; its tokens may then differ from an
 * uncached prefill where the last position's logits are at a near-tie.
 * Entries match on the whole token sequence (the reference compares a
 * hash); the oldest is evicted first (the reference evicts an arbitrary
 * one). 0 (the default) turns the cache off and frees it. */
#define FMX_SCHED_MAX_PREFIX_ENTRIES 1024
int fmx_scheduler_set_prefix_cache(fmx_scheduler* s, int64_t max_entries);
int64_t fmx_scheduler_prefix_hits(const fmx_scheduler* s);
void fmx_scheduler_free(fmx_scheduler* s);

/* Greedy next token: ids[b] = argmax_v logits[b * row_stride + v] (the
 * first of equal maxima, as mx::argmax); when offsets is not NULL,
 * offsets[b] += advance (the next decode step's cache position). */
int fmx_greedy_next(const void* logits, int64_t batch, int64_t vocab, int64_t row_stride,
                    int32_t* ids, int32_t* offsets, int32_t advance, fmx_stream stream);

/* RoPE table of the decode attention: rope_cs [n_pos][head_dim / 2][2] fp32
 * on the device, (cos, sin) of p * theta^(-2i / head_dim) computed in fp64
 * and rounded to fp32 (the table fmx_model_workspace_init builds; the
 * frequencies of mx::fast::rope with base theta, model.cpp:875-876).
 * Synchronises the stream before it returns. */
int fmx_rope_table(float* rope_cs, int64_t n_pos, int64_t head_dim, float rope_theta, fmx_stream stream);

/* Single-token attention of a decode step, as the decoder stack runs it
 * (model.cpp:874-884: mx::fast::rope of q and k at the sequence's cache
 * offset, traditional = false; the KV-cache append; mx::fast::
 * scaled_dot_product_attention with no mask): for each sequence b at
 * position p = offsets[b], q and the new key are rotated, the new key and
 * value go to cache position p of slot b, and out[b] = softmax(q K^T scale) V
 * over positions 0 .. p for every query head (its kv head: head /
 * (n_heads / n_kv_heads)). qkv [batch, (n_heads + 2 n_kv_heads) head_dim]
 * bf16 (the q heads, then k, then v; unrotated); rope_cs from
 * fmx_rope_table with at least max_seq rows; k_cache, v_cache [batch]
 * [n_kv_heads][max_seq][head_dim] bf16; offsets [batch] int32 on the device
 * (clamped to [0, max_seq)); out [batch, n_heads head_dim] bf16.
 * head_dim <= 128 with 64 % (head_dim / 8) == 0, max_seq <= 4096; other
 * shapes: FMX_ERR_UNSUPPORTED. */
int fmx_attention_decode(const void* qkv, int64_t batch, int64_t n_heads, int64_t n_kv_heads,
                         int64_t head_dim, const float* rope_cs, void* k_cache, void* v_cache,
                         int64_t max_seq, const int32_t* offsets, float scale, void* out,
                         fmx_stream stream);

#ifdef __cplusplus
}
#endif
#endif /* FMX_MODEL_H */
