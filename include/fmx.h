/*
 * fmx.h -- C-ABI of the MI355X-native MoE hot path (libfmx.so).
 *
 * The reference (FlashMLX) runs its MoE block through MLX C++ ops on Apple
 * GPUs. This library replaces the ops on that path with HIP kernels for
 * gfx950 behind a plain C interface: device pointers and sizes in, status
 * codes out, no C++ or torch types in any signature.
 *
 * Conventions
 *   - Every pointer named `data`, `x`, `y`, weights, indices, outputs and
 *     `workspace` is DEVICE memory on the current HIP device. Arrays are
 *     row-major and contiguous.
 *   - Calls are asynchronous on `stream` (a hipStream_t; NULL = null
 *     stream). The caller synchronises.
 *   - Ownership: the library never frees caller memory and keeps no pointer
 *     past a call. Scratch memory comes from the caller's `workspace`; when
 *     `workspace` is NULL the call allocates it stream-ordered
 *     (hipMallocAsync) and frees it before returning.
 *   - Errors: every entry point returns an fmx_status. MLX raises C++
 *     exceptions (std::invalid_argument) for the same conditions; none
 *     crosses this boundary. fmx_last_error() gives the thread's last message.
 *   - Concurrency: calls are re-entrant for distinct (stream, workspace)
 *     pairs. Two calls sharing one workspace must be ordered on one stream.
 *   - Scope: affine mode, bits = 4, group_size = 64, transpose = true.
 *     Activations and scales/biases are bf16 or float16: fmx_quantized_matmul
 *     and fmx_gather_qmm take float16 ones (FMX_F16: x, scales, biases and
 *     out all float16), and so do the MoE block and router entry points when
 *     fmx_moe_config.activation_dtype is FMX_F16; the decoder stack and the
 *     Nemotron-H block are bf16. Any other valid MLX argument returns
 *     FMX_ERR_UNSUPPORTED and computes nothing.
 *
 * Packed weight layout (MLX's, unchanged): for a logical [N, K] matrix
 *   w       uint32 [..., N, K/8]   element k of a row is nibble k%8 (bits
 *                                   4*(k%8)..+3) of word k/8
 *   scales  bf16   [..., N, K/64]
 *   biases  bf16   [..., N, K/64]  dequantised value = scale * q + bias
 */
#ifndef FMX_H
#define FMX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FMX_ABI_VERSION 5

typedef enum fmx_status {
  FMX_OK = 0,
  FMX_ERR_ARG = 1,         /* null pointer or bad enum value                 */
  FMX_ERR_SHAPE = 2,       /* shapes/sizes inconsistent                      */
  FMX_ERR_DTYPE = 3,       /* dtype not the one the argument requires       */
  FMX_ERR_UNSUPPORTED = 4, /* valid MLX call outside this library's scope    */
  FMX_ERR_WORKSPACE = 5,   /* workspace smaller than the size query returned */
  FMX_ERR_HIP = 6          /* HIP runtime error (launch, allocation)         */
} fmx_status;

/* FMX_F16: float16 activations (a checkpoint whose norms are float16,
 * model.cpp:208-214), taken by fmx_quantized_matmul and fmx_gather_qmm with
 * float16 scales, biases and output, and by the MoE block
 * (fmx_moe_config.activation_dtype). */
typedef enum fmx_dtype { FMX_BF16 = 0, FMX_F32 = 1, FMX_U32 = 2, FMX_I32 = 3, FMX_F16 = 4 } fmx_dtype;

#define FMX_MAX_NDIM 8

/* Non-owning view of a contiguous device array. */
typedef struct fmx_array {
  void* data;
  int32_t dtype; /* fmx_dtype */
  int32_t ndim;
  int64_t shape[FMX_MAX_NDIM];
} fmx_array;

typedef void* fmx_stream; /* hipStream_t */

int fmx_abi_version(void);
const char* fmx_status_string(int status);
const char* fmx_last_error(void);

/* ------------------------------------------------------------------------
 * quantized_matmul
 * Replaces mx::quantized_matmul(x, w, scales, biases, transpose, group_size,
 * bits) as called by LlamaModel::linear_fast (server/src/model.cpp:476-480)
 * and LlamaModel::shared_expert_mlp (server/src/model.cpp:741-747).
 *   x [..., M, K] bf16, w [N, K/8] u32, scales/biases [N, K/64] bf16
 *   out [..., M, N] bf16 (caller-allocated; shape from the _out_shape query)
 * `mode` must be "affine" (or NULL, which means "affine").
 * --------------------------------------------------------------------- */
int fmx_quantized_matmul_out_shape(const fmx_array* x, const fmx_array* w, int transpose,
                                   int group_size, int bits, fmx_array* out);
size_t fmx_quantized_matmul_workspace_size(const fmx_array* x, const fmx_array* w);
int fmx_quantized_matmul(const fmx_array* x, const fmx_array* w, const fmx_array* scales,
                         const fmx_array* biases, int transpose, int group_size, int bits,
                         const char* mode, fmx_array* out, void* workspace,
                         size_t workspace_bytes, fmx_stream stream);

/* ------------------------------------------------------------------------
 * gather_qmm
 * Replaces mx::gather_qmm(x, w, scales, biases, lhs_indices, rhs_indices,
 * transpose, group_size, bits, mode, sorted_indices) as called by
 * LlamaModel::switch_mlp (server/src/model.cpp:703-721).
 *   x [..., M, K] bf16; w [E..., N, K/8] u32; scales/biases [E..., N, K/64]
 *   lhs_indices / rhs_indices: u32 or i32 arrays, or NULL for MLX's defaults
 *     (arange over the flattened batch dims of x / of w)
 *   out: broadcast(lhs.shape, rhs.shape) + [M, N], bf16
 * Out-of-range index values (undefined behaviour in MLX) are clamped to the
 * last valid row / expert on the device, so they never address memory
 * outside the arrays.
 * `sorted_indices` is a hint only: results never depend on it.
 * Up to 2^22 output rows (prod(broadcast batch) * M) and 1024 experts;
 * larger calls return FMX_ERR_UNSUPPORTED.
 * --------------------------------------------------------------------- */
int fmx_gather_qmm_out_shape(const fmx_array* x, const fmx_array* w,
                             const fmx_array* lhs_indices, const fmx_array* rhs_indices,
                             int transpose, int group_size, int bits, fmx_array* out);
size_t fmx_gather_qmm_workspace_size(const fmx_array* x, const fmx_array* w,
                                     const fmx_array* lhs_indices,
                                     const fmx_array* rhs_indices);
int fmx_gather_qmm(const fmx_array* x, const fmx_array* w, const fmx_array* scales,
                   const fmx_array* biases, const fmx_array* lhs_indices,
                   const fmx_array* rhs_indices, int transpose, int group_size, int bits,
                   const char* mode, int sorted_indices, fmx_array* out, void* workspace,
                   size_t workspace_bytes, fmx_stream stream);

/* ------------------------------------------------------------------------
 * quantize / dequantize
 * Replace mx::quantize / mx::dequantize (affine, bits 4, group 64): the
 * format the reference's checkpoints are stored in and that
 * LlamaModel::build_moe_weight_cache stacks (server/src/model.cpp:368-470).
 *   w [..., N, K] bf16 -> wq [..., N, K/8] u32, scales/biases [..., N, K/64] bf16
 * --------------------------------------------------------------------- */
int fmx_quantize(const fmx_array* w, int group_size, int bits, const char* mode,
                 fmx_array* wq, fmx_array* scales, fmx_array* biases, fmx_stream stream);
int fmx_dequantize(const fmx_array* wq, const fmx_array* scales, const fmx_array* biases,
                   int group_size, int bits, const char* mode, fmx_array* out,
                   fmx_stream stream);

/* ------------------------------------------------------------------------
 * Expert stacking: mx::stack of per-expert arrays into [E, ...]
 * (server/src/model.cpp:396-404). Copies n_experts device buffers of `bytes`
 * each into dst (device), expert e at dst + e*bytes.
 * --------------------------------------------------------------------- */
int fmx_stack_experts(const void* const* src_per_expert, int64_t n_experts, size_t bytes,
                      void* dst, fmx_stream stream);

/* ------------------------------------------------------------------------
 * MoE block
 * Replaces LlamaModel::moe_block (server/src/model.cpp:750-807) together with
 * switch_mlp (:673-734) and shared_expert_mlp (:736-748):
 *   gates  = softmax(x . router_w^T [+ logit_bias], precise)
 *   inds   = top-k of gates (ties: lower expert index; slots ordered by
 *            probability descending, then index ascending)
 *   scores = gates[inds]   (divided by their sum when norm_topk_prob)
 *   y      = sum_k scores_k * down_e(swiglu(gate_e(x), up_e(x)))
 *          + sigmoid(x . shared_expert_gate_w^T) * shared_expert(x)
 * --------------------------------------------------------------------- */

/* ModelConfig's MoE fields (server/include/flashmlx/model.h:20-54). */
typedef struct fmx_moe_config {
  int64_t hidden_size;                     /* H                          */
  int64_t num_experts;                     /* E  (<= 1024)               */
  int32_t num_experts_per_tok;             /* k  (<= 16, <= E)           */
  int32_t norm_topk_prob;                  /* 0 / 1                      */
  int64_t moe_intermediate_size;           /* I                          */
  int64_t shared_expert_intermediate_size; /* Is; 0 = no shared expert   */
  int32_t quant_bits;                      /* 4                          */
  int32_t quant_group_size;                /* 64                         */
  /* ModelConfig::activation_dtype (model.h:34, set at model.cpp:208-214):
   * FMX_BF16 (0) or FMX_F16. With FMX_F16, x, y, the router and shared-gate
   * rows (or their scales and biases), the logit bias and every expert scale
   * and bias are float16, and the block rounds in fp16 where the bf16 block
   * rounds in bf16 (logits, probabilities, scores, SwiGLU, expert outputs,
   * the combine). Float16 blocks run on packed weights (decode and prefill
   * kernels); without them the forward returns FMX_ERR_UNSUPPORTED, and so
   * does the input norm of the decoder stack. */
  int32_t activation_dtype;
} fmx_moe_config;

typedef struct fmx_qweight {
  const void* w;      /* u32  [.., N, K/8]  */
  const void* scales; /* bf16 [.., N, K/64] */
  const void* biases; /* bf16 [.., N, K/64] */
} fmx_qweight;

/* MoEWeights (server/include/flashmlx/model.h:58-72), stacked layout.
 * The router and the shared-expert gate come either unquantised (bf16 rows,
 * model.cpp:762, :797-799) or quantized like every other linear (affine,
 * 4 bits, group 64: model.cpp:758-760, :792-796; loaded at :389-392 and
 * :447-455); a non-NULL *_scales pointer selects the quantized form. Their
 * logits are formed exactly (fp64 sums of exact products, x times the
 * dequantised s*q + b) and rounded once to bf16, in either form.
 * When `packed` is given, the forward reads the expert weights from there
 * only: gate/up/down and shared_gate/up/down may then be NULL (the caller may
 * free the MLX-layout copies after fmx_pack_expert_weights). Every bf16
 * below is float16 in a float16 block (fmx_moe_config.activation_dtype). */
typedef struct fmx_moe_weights {
  const void* router_w;          /* bf16 [E, H], or u32 [E, H/8] when router_scales */
  const void* router_logit_bias; /* bf16 [E] added to the logits before softmax, or
                                    NULL. No counterpart in the reference: lets a
                                    caller skew expert loads (benchmarks).        */
  fmx_qweight gate;              /* [E, I, H/8] ...                                */
  fmx_qweight up;                /* [E, I, H/8] ...                                */
  fmx_qweight down;              /* [E, H, I/8] ...                                */
  fmx_qweight shared_gate;       /* [Is, H/8] ... (ignored when Is == 0)           */
  fmx_qweight shared_up;         /* [Is, H/8] ...                                  */
  fmx_qweight shared_down;       /* [H, Is/8] ...                                  */
  const void* shared_expert_gate_w; /* bf16 [1, H], or u32 [1, H/8] when
                                       shared_expert_gate_scales                  */
  const void* packed;            /* NULL, or the same expert weights re-laid out by
                                    fmx_pack_expert_weights (read by the decode
                                    kernels and the prefill GEMMs). No
                                    counterpart in the reference.                 */
  size_t packed_bytes;           /* bytes of `packed`: at least
                                    fmx_moe_packed_size(cfg), else FMX_ERR_WORKSPACE */
  const void* router_scales;     /* bf16 [E, H/64] or NULL (bf16 router)           */
  const void* router_biases;     /* bf16 [E, H/64]; required with router_scales   */
  const void* shared_expert_gate_scales; /* bf16 [1, H/64] or NULL                */
  const void* shared_expert_gate_biases; /* bf16 [1, H/64]                        */
} fmx_moe_weights;

/* Load-time re-layout of a layer's expert weights (replaces the stacking
 * step of model.cpp:368-470 as the last load-time transform). Packs gate+up
 * of every routed expert as interleaved pairs, down per expert, and the
 * shared expert the same way, into `packed` (device memory of
 * fmx_moe_packed_size(cfg) bytes, 256-byte aligned). Forwards then read only
 * the packed copy, so the MLX-layout expert arrays can be freed once the
 * stream has run this call: the layer holds its expert weights once (the
 * reference keeps the per-expert arrays next to the stacked ones). Returns 0
 * bytes / FMX_ERR_UNSUPPORTED when H, I or Is is not a multiple of 128. */
size_t fmx_moe_packed_size(const fmx_moe_config* cfg);
int fmx_pack_expert_weights(const fmx_moe_config* cfg, const fmx_moe_weights* src, void* packed,
                            size_t packed_bytes, fmx_stream stream);

/* Which kernels fmx_moe_block_forward runs for n_tokens tokens: 1 = the
 * decode kernels (packed weights given, at most 16 tokens, shapes within their
 * limits), 2 = the prefill GEMMs on packed weights (packed weights given, more
 * tokens or shapes outside the decode limits), 0 = the general ones on the
 * MLX layout, < 0 = an fmx_status error (negated). No counterpart in the
 * reference; for callers that size work per path. */
int fmx_moe_forward_path(const fmx_moe_config* cfg, int64_t n_tokens, int has_packed);

/* Bytes of workspace one forward of up to max_tokens tokens needs
 * (max_tokens <= 65536; 0 for an invalid config). Nondecreasing in
 * max_tokens: a workspace of this size serves every forward of 0..max_tokens
 * tokens. */
size_t fmx_moe_workspace_size(const fmx_moe_config* cfg, int64_t max_tokens);

/* Prepares a fresh workspace: clears the completion counters and the
 * status word kept in its first bytes. Call once after allocating; every
 * forward leaves the counters cleared again, so a workspace is reusable
 * across calls and sizes. */
int fmx_moe_workspace_init(void* workspace, size_t workspace_bytes, fmx_stream stream);

/* The workspace's status word, after the forwards queued on `stream` end
 * (synchronises the stream): 0, or FMX_STATUS_WAIT_TIMEOUT when a decode
 * forward's bounded wait ran out (a down workgroup waiting for its expert's
 * gate/up tiles: its products are written as NaN; or the router waiting for
 * the other router columns' logits: missing logits are read as 0). Bits
 * stay set until cleared (clear != 0 clears them after reading, in stream
 * order, and resets every counter, flag and logit word of the workspace,
 * which a forward whose wait ran out may leave set: clear before the next
 * forward). No counterpart in the reference: MLX's graph has no in-kernel
 * waits. */
#define FMX_STATUS_WAIT_TIMEOUT 1u
int fmx_moe_workspace_status(const void* workspace, size_t workspace_bytes, uint32_t* status,
                             int clear, fmx_stream stream);

/* Bound of those waits, in flag reads s_sleep(2) to s_sleep(16) apart
 * (default 2^21, far beyond any real wait): applies to forwards launched
 * after the call; polls = 0 gives up at once (a way to exercise the guard),
 * polls < 0 restores the default. Returns the previous bound. No
 * counterpart in the reference. */
int64_t fmx_set_decode_wait_limit(int64_t polls);

/* y [T, H] = moe_block(x [T, H]), T = B*L tokens, in the config's activation
 * dtype (bf16 or float16). The workspace
 * must hold fmx_moe_workspace_size(cfg, T) bytes and have been initialised
 * once with fmx_moe_workspace_init. T = 0 runs nothing and returns FMX_OK
 * (x and y may then be NULL, as for empty tensors). */
int fmx_moe_block_forward(const fmx_moe_config* cfg, const fmx_moe_weights* w,
                          const void* x, int64_t n_tokens, void* y, void* workspace,
                          size_t workspace_bytes, fmx_stream stream);

/* fmx_moe_block_forward without a workspace argument, for callers that
 * cannot allocate (code under HIP graph capture, serving loops that forbid
 * hipMalloc): no counterpart in the reference. It calls no allocating
 * routine; its workspace is a fixed device array of FMX_NOALLOC_SCRATCH_BYTES
 * bytes that the library holds on every device it runs on until the process
 * ends. Forwards whose fmx_moe_workspace_size(cfg, n_tokens) exceeds that
 * return FMX_ERR_UNSUPPORTED before launching anything (8 MiB: every decode
 * batch of up to 16 tokens, and forwards of up to 72 tokens of the
 * Qwen1.5-MoE-A2.7B shape or 104 of the Qwen3-30B-A3B shape). All calls on
 * one device share the array:
 * calls that overlap on one GPU (two streams, or two host threads) race and
 * must be ordered by the caller. Each forward leaves the array's completion
 * counters at zero for the next. */
#define FMX_NOALLOC_SCRATCH_BYTES (8 * 1024 * 1024)
int fmx_moe_block_forward_noalloc(const fmx_moe_config* cfg, const fmx_moe_weights* w,
                                  const void* x, int64_t n_tokens, void* y, fmx_stream stream);

/* fmx_moe_block_forward that also records caller-created HIP events
 * (hipEvent_t, as void*) on `stream` at its stage boundaries:
 *   stage_events[0] before the router, [1] after routing and sort,
 *   [2] after the gate/up GEMMs, [3] after the down GEMMs, [4] after the
 *   combine (for n_tokens <= 16 on packed weights gate/up, down and combine
 *   run as one grid and [2], [3], [4] are recorded together after it). Used
 *   to time each stage's kernels; no counterpart in the reference. */
#define FMX_MOE_STAGE_EVENTS 5
int fmx_moe_block_forward_profiled(const fmx_moe_config* cfg, const fmx_moe_weights* w,
                                   const void* x, int64_t n_tokens, void* y, void* workspace,
                                   size_t workspace_bytes, fmx_stream stream,
                                   void* const* stage_events);

/* fmx_moe_block_forward that launches only its first n_stages kernel stages
 * (1..4: router, gate/up, down, combine; 4 = the whole forward, y complete;
 * for n_tokens <= 16 on packed weights 2 runs the gate/up kernel alone and
 * 3 already runs the whole forward's gate/up + down + combine grid).
 * Timing graphs of 1, 2, 3 and 4 stages gives each stage's marginal time
 * inside the layer. No counterpart in the reference (a measurement aid). */
int fmx_moe_block_forward_partial(const fmx_moe_config* cfg, const fmx_moe_weights* w,
                                  const void* x, int64_t n_tokens, void* y, void* workspace,
                                  size_t workspace_bytes, fmx_stream stream, int n_stages);

/* Device views of the routing state a forward of n_tokens tokens left in
 * the workspace (valid until the next call on that workspace). Any out
 * pointer may be NULL.
 *   inds [T,k] u32, scores [T,k] bf16, probs [T,E] bf16,
 *   order/inv/src/idx [T*k] u32 (switch_mlp's sort, model.cpp:682-700),
 *   expert_offsets [E+1] u32 (rows of expert e are [off[e], off[e+1]) ). */
int fmx_moe_workspace_routing(const fmx_moe_config* cfg, int64_t n_tokens,
                              const void* workspace, const uint32_t** inds,
                              const void** scores, const void** probs,
                              const uint32_t** order, const uint32_t** inv,
                              const uint32_t** src, const uint32_t** idx,
                              const uint32_t** expert_offsets);

/* Router alone (model.cpp:757-775 + renorm): inds [T,k] u32, scores [T,k]
 * bf16, probs [T,E] bf16 (may be NULL). */
int fmx_moe_router_topk(const fmx_moe_config* cfg, const void* x, int64_t n_tokens,
                        const void* router_w, const void* router_logit_bias,
                        uint32_t* inds, void* scores, void* probs, void* workspace,
                        size_t workspace_bytes, fmx_stream stream);

/* Router alone, with the router and the shared-expert gate in either form
 * (model.cpp:757-775 + renorm, and the gate of :787-803). Reads from `w`
 * only: router_w with router_scales / router_biases (NULL scales = bf16 rows
 * [E, H], :762; given = 4-bit rows u32 [E, H/8] with bf16 scales and biases
 * [E, H/64], the quantized_matmul of :758-760), router_logit_bias, and,
 * when shared_gate_out is not NULL, shared_expert_gate_w with its scales and
 * biases (bf16 [1, H], or u32 [1, H/8] + [1, H/64]). Logits are formed as
 * fmx_moe_block_forward forms them (exact sums, one bf16 rounding), so inds,
 * scores and probs are bit-identical to the block's routing.
 *   inds [T,k] u32, scores [T,k] bf16, probs [T,E] bf16 (or NULL),
 *   shared_gate_out [T] bf16 = sigmoid(x . shared_expert_gate^T) (or NULL). */
int fmx_moe_router_topk_ex(const fmx_moe_config* cfg, const void* x, int64_t n_tokens,
                           const fmx_moe_weights* w, uint32_t* inds, void* scores, void* probs,
                           void* shared_gate_out, void* workspace, size_t workspace_bytes,
                           fmx_stream stream);

/* Sort / permutation alone (model.cpp:682-700): order = stable argsort of the
 * flattened inds, inv = argsort(order), src = order / k, idx = flat[order],
 * expert_offsets [E+1]. Any output may be NULL. Index values >= E are
 * treated as E-1. Up to 2^22 entries (T*k) and 1024 experts. Workspace:
 * fmx_moe_sort_workspace_size bytes (or NULL). */
size_t fmx_moe_sort_workspace_size(int64_t n_tokens, int32_t k, int64_t num_experts);
int fmx_moe_sort(const uint32_t* inds, int64_t n_tokens, int32_t k, int64_t num_experts,
                 uint32_t* order, uint32_t* inv, uint32_t* src, uint32_t* idx,
                 uint32_t* expert_offsets, void* workspace, size_t workspace_bytes,
                 fmx_stream stream);

/* ------------------------------------------------------------------------
 * Synthetic inputs (host memory; no counterpart in the reference, which
 * loads checkpoints). Counter-based: element i of (seed, stream) is a pure
 * function of (seed, stream, i), so any slice can be regenerated alone.
 *   out[i] = bf16(mean + std * N(0,1)), Box-Muller on splitmix64 counters.
 * --------------------------------------------------------------------- */
int fmx_synth_normal_bf16(uint16_t* host_out, int64_t n, uint64_t seed, uint64_t stream,
                          double mean, double std_dev);
/* The same values written to device memory by a kernel on `stream` (for
 * multi-GB weight sets). Its log and cos are the device library's: the bits
 * equal the host version's except where a last-ulp fp64 difference crosses a
 * bf16 rounding boundary (about one element in 2^44). */
int fmx_synth_normal_bf16_device(void* out, int64_t n, uint64_t seed, uint64_t stream,
                                 double mean, double std_dev, fmx_stream s);

#ifdef __cplusplus
}
#endif
#endif /* FMX_H */
