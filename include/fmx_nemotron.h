/*
 * fmx_nemotron.h -- C-ABI of the Nemotron-H MoE block (libfmx.so).
 *
 * Replaces NemotronHModel::moe_block (server/src/nemotron_h.cpp:1010-1111)
 * with the weights its loader caches (MoELayerWeights, nemotron_h.cpp:443-470):
 *   logits = x . gate_w^T                                   (bf16, :1018)
 *   orig   = sigmoid(fp32(logits)); sel = orig + correction_bias   (:1024-1028)
 *   groups (n_group > 1): sel of every expert outside the topk_group groups
 *          with the largest sum of their two best sel set to 0     (:1029-1041)
 *   inds   = top-k of sel                                   (:1042-1043)
 *   scores = orig[inds] (/ (sum + 1e-20) when norm_topk_prob and k > 1)
 *            * routed_scaling_factor                        (:1044-1049)
 *   y      = bf16(sum_k scores_k * fc2_e(relu(fc1_e(x))^2))  (:1052-1099)
 *          + shared_down(relu(shared_up(x))^2)              (:1101-1108)
 * Conventions as in fmx.h: device pointers, asynchronous on `stream`,
 * status codes, fmx_last_error().
 *
 * Arithmetic: logits are exact sums rounded once to bf16; orig is the fp64
 * sigmoid (a deterministic exp) rounded once to fp32; selection, scores and
 * the renormalisation are fp32 operations in slot order (slots ordered by
 * sel, ties to the lower expert index; lower group index on group ties).
 * relu^2 of the bf16 up projection is exact in fp32 (the reference's relu2
 * takes the maximum with an fp32 0, which promotes); the down projections
 * read it rounded to fp16 (2^-11 relative; bf16 when a value exceeds fp16's
 * range) and produce fp32, the weighted k-sum is fp32 in slot order, and
 * the shared expert's fp32 output is added before the one rounding to bf16.
 */
#ifndef FMX_NEMOTRON_H
#define FMX_NEMOTRON_H

#include "fmx.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ModelConfig's Nemotron-H MoE fields (nemotron_h.cpp:245-258). Limits:
 * hidden_size a multiple of 128; moe_intermediate_size and
 * moe_shared_expert_intermediate_size multiples of 64 (the packed layout pads
 * them to 128 with zero weights); n_routed_experts <= 1024; k <= 16;
 * n_group divides n_routed_experts, n_group <= 64, at least two experts per
 * group when n_group > 1, 1 <= topk_group <= n_group. */
typedef struct fmx_nh_moe_config {
  int64_t hidden_size;                         /* H                        */
  int64_t n_routed_experts;                    /* E                        */
  int32_t num_experts_per_tok;                 /* k                        */
  int32_t norm_topk_prob;                      /* 0 / 1                    */
  int64_t moe_intermediate_size;               /* I                        */
  int64_t moe_shared_expert_intermediate_size; /* Is; 0 = no shared expert */
  int32_t n_group;                             /* 1 = no group limit       */
  int32_t topk_group;
  float routed_scaling_factor;
  int32_t quant_bits;                          /* 4                        */
  int32_t quant_group_size;                    /* 64                       */
} fmx_nh_moe_config;

/* MoELayerWeights (nemotron_h.cpp:443-470), MLX affine 4-bit group 64
 * (fmx_qweight as in fmx.h). */
typedef struct fmx_nh_moe_weights {
  const void* gate_w;          /* bf16 [E, H]  mixer.gate.weight                    */
  const float* correction_bias; /* fp32 [E]   mixer.gate.e_score_correction_bias, or NULL */
  fmx_qweight fc1;             /* [E, I, H/8] ...  switch_mlp.fc1                   */
  fmx_qweight fc2;             /* [E, H, I/8] ...  switch_mlp.fc2                   */
  fmx_qweight shared_up;       /* [Is, H/8] ...    shared_experts.up_proj           */
  fmx_qweight shared_down;     /* [H, Is/8] ...    shared_experts.down_proj         */
  const void* packed;          /* fmx_nh_pack_expert_weights' output: the forward
                                  reads fc1/fc2/shared from there only (required) */
  size_t packed_bytes;
} fmx_nh_moe_weights;

/* Load-time re-layout of a layer's expert weights into 16-row x 128-k
 * blocks (the layout of fmx_pack_expert_weights, single matrices), I and Is
 * padded to multiples of 128 with zero weights (scale 0, bias 0). No
 * counterpart in the reference (its loader keeps the MLX arrays, :443-470).
 * The MLX-layout arrays may be freed once the stream has run the call. */
size_t fmx_nh_moe_packed_size(const fmx_nh_moe_config* cfg);
int fmx_nh_pack_expert_weights(const fmx_nh_moe_config* cfg, const fmx_nh_moe_weights* src,
                               void* packed, size_t packed_bytes, fmx_stream stream);

/* Bytes of workspace one forward of up to max_tokens tokens needs (0 for an
 * invalid config); nondecreasing in max_tokens. fmx_nh_moe_workspace_init
 * prepares a fresh workspace once (it clears the router's arrival counters
 * and a flag word in its first bytes, which every forward leaves cleared). */
size_t fmx_nh_moe_workspace_size(const fmx_nh_moe_config* cfg, int64_t max_tokens);
int fmx_nh_moe_workspace_init(void* workspace, size_t workspace_bytes, fmx_stream stream);

/* y [T, H] bf16 = moe_block(x [T, H] bf16) (NemotronHModel::moe_block),
 * T = B*L tokens, on the packed weights; T = 0 runs nothing. workspace NULL:
 * the call allocates (and initialises) its own, stream-ordered. */
int fmx_nh_moe_block_forward(const fmx_nh_moe_config* cfg, const fmx_nh_moe_weights* w,
                             const void* x, int64_t n_tokens, void* y, void* workspace,
                             size_t workspace_bytes, fmx_stream stream);

/* fmx_nh_moe_block_forward that records caller-created HIP events (as
 * void*) on `stream` at its stage boundaries: [0] before the router, [1]
 * after routing and the sort, [2] after the fc1 (+ shared up) grid, [3]
 * after the fc2 (+ shared down) grid, [4] after the combine. A measurement
 * aid with no counterpart in the reference. */
#define FMX_NH_STAGE_EVENTS 5
int fmx_nh_moe_block_forward_profiled(const fmx_nh_moe_config* cfg, const fmx_nh_moe_weights* w,
                                      const void* x, int64_t n_tokens, void* y, void* workspace,
                                      size_t workspace_bytes, fmx_stream stream,
                                      void* const* stage_events);

/* fmx_nh_moe_block_forward that launches only its first n_stages kernel
 * stages (1..4: router + sort, fc1 (+ shared up), fc2 (+ shared down),
 * combine; 4 = the whole forward, y complete; on the decode kernels 3
 * already forms the combine). Timing graphs of 1, 2, 3 and 4 stages gives
 * each stage's marginal time inside the layer. A measurement aid with no
 * counterpart in the reference. */
int fmx_nh_moe_block_forward_partial(const fmx_nh_moe_config* cfg, const fmx_nh_moe_weights* w,
                                     const void* x, int64_t n_tokens, void* y, void* workspace,
                                     size_t workspace_bytes, fmx_stream stream, int n_stages);

/* Device views of the routing the latest forward of n_tokens tokens left in
 * the workspace: inds [T, k] u32, scores [T, k] fp32, logits [T, E + 1] bf16
 * (row stride E + 1); any out pointer may be NULL. */
int fmx_nh_moe_workspace_routing(const fmx_nh_moe_config* cfg, int64_t n_tokens,
                                 const void* workspace, const uint32_t** inds,
                                 const float** scores, const void** logits);

#ifdef __cplusplus
}
#endif
#endif /* FMX_NEMOTRON_H */
