/*
 * fmx_oracle.h -- CPU restatement of FlashMLX's MoE hot path (TEST INFRASTRUCTURE).
 *
 * This library is the checker, never the product. Only tests/, the smoke
 * entry point and bench.py's CPU-baseline leg may load it. It restates, in
 * plain C, what the reference's MoE block computes through MLX ops:
 *
 *   server/src/model.cpp:750-807  LlamaModel::moe_block
 *   server/src/model.cpp:673-734  LlamaModel::switch_mlp   (sort / gather_qmm / unsort)
 *   server/src/model.cpp:736-748  LlamaModel::shared_expert_mlp
 *   server/src/model.cpp:14-25    compiled SwiGLU  g * sigmoid(g) * u
 *   server/src/model.cpp:476-480  linear_fast = quantized_matmul(transpose=true)
 *   server/include/flashmlx/model.h:20-72  ModelConfig / MoEWeights layout
 *
 * The arithmetic of those ops lives in MLX (third-party, pinned only as
 * mlx>=0.22.0 in pyproject.toml:7, not vendored, not installed here).
 * Each function below names which MLX op it restates and how it is pinned.
 *
 * Data conventions (all row-major, little-endian):
 *   bf16          uint16_t bit pattern
 *   packed weight w      uint32 [N, K/8]   nibble j of a word = element 8*word+j,
 *                                           stored at bits 4j..4j+3
 *                 scales bf16   [N, K/64]
 *                 biases bf16   [N, K/64]   dequant: s*q + b
 *   stacked experts: a leading [E] dimension on all three.
 *
 * Parity status per function (how each is pinned; see tests/test_oracle_*.py):
 *   orc_f32_to_bf16 / orc_f64_to_bf16   exact rational rounding (Python Fraction)
 *   orc_exp                              libm exp within 2 ulp + exact powers
 *   orc_quantize                         KAT grids, nearest-level property,
 *                                        nibble order, |deq-w| bound.  The MLX
 *                                        edge/q0 snap rule itself is recalled
 *                                        from MLX's CPU quantizer: parity of
 *                                        that rule against MLX is UNPINNED.
 *   orc_qmm_t / orc_gather_qmm (mode 0)  fp64 dequant + numpy matmul, one-hot
 *                                        reduction, brute force on tiny shapes
 *   orc_qmm_t modes A/B/C                recalled MLX CPU accumulators; which
 *                                        one MLX uses is UNPINNED (reported only)
 *   orc_router_topk(_q)                  numpy fp64 logits (of the bf16 rows or
 *                                        of numpy's own dequantisation of the
 *                                        4-bit rows), numpy softmax, full sort
 *                                        with (p desc, idx asc)
 *   orc_moe_sort                         numpy stable argsort + invariants
 *   orc_moe_block                        dense fp64 formula on tiny shapes
 *   orc_rms_norm                         scale invariance, constant rows, numpy fp64
 *   orc_rope_table / orc_rope            position 0 = identity, pair norms kept,
 *                                        composition of rotations, numpy complex
 *                                        rotation; MLX's rounding points inside
 *                                        rope (bf16 vs fp32 angles) are UNPINNED
 *   orc_nh_route                         top-k of the logits (sigmoid is monotone)
 *                                        against numpy; numpy sigmoid within 1 fp32
 *                                        ulp; group-limited and bias cases by
 *                                        constructed inputs with known answers;
 *                                        renormalised scores sum to the scaling
 *   orc_nh_moe_block                     dense numpy fp64 formula on tiny shapes;
 *                                        scaling 2 doubles y exactly; fc1 rows all
 *                                        negative leave y = shared expert alone.
 *                                        MLX's fp32 sigmoid (its own exp) and
 *                                        argpartition's tie order are UNPINNED
 *   orc_sdpa                             one key = v, equal keys = mean of values,
 *                                        causal prefix, numpy fp64 softmax(QK^T)V;
 *                                        MLX's intermediate roundings UNPINNED
 *   orc_sdpa_split                       the same checks; within one bf16 ulp of
 *                                        orc_sdpa at range boundaries and with
 *                                        one range's scores far above the rest
 */
#ifndef FMX_ORACLE_H
#define FMX_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* accumulation modes of the quantized products */
enum {
  ORC_ACC_F64 = 0,  /* fp64 dequant + fp64 accumulate: the mathematical value */
  ORC_ACC_A = 1,    /* fp32 dequant (s*q then +b) + sequential fp32 accumulate: parity gate */
  ORC_ACC_B = 2,    /* every op rounded to bf16 (MLX scalar `T sum` loop, recalled) */
  ORC_ACC_C = 3     /* 8 fp32 lanes over k mod 8 + lane sum (MLX simd loop, recalled) */
};

/* ---- numerics ---------------------------------------------------------- */
float    orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);   /* round to nearest even */
uint16_t orc_f64_to_bf16(double d);  /* single round to nearest even from fp64 */
double   orc_exp(double r);          /* deterministic exp used by the router softmax */
float    orc_sigmoid_bf16(uint16_t g); /* bf16(sigmoid(g)) as float */

/* ---- affine quantization (mx::quantize, bits=4, group_size=64) -------- */
int  orc_quantize(const uint16_t* w, int64_t N, int64_t K, int group_size, int bits,
                  uint32_t* wq, uint16_t* scales, uint16_t* biases);
int  orc_dequantize(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                    int64_t N, int64_t K, int group_size, int bits, float* out);

/* ---- quantized matmul, transpose=true --------------------------------- */
/* out[M,N] = x[M,K] . deq(w)[N,K]^T, output rounded to bf16. */
int orc_qmm_t(const uint16_t* x, int64_t M, int64_t K,
              const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
              int64_t N, int mode, uint16_t* out);

/* gather_qmm over already-broadcast index lists of length nb:
 *   out[b, M, N] = x[lhs[b], M, K] . deq(w[rhs[b]])^T                        */
int orc_gather_qmm(const uint16_t* x, int64_t n_x, int64_t M, int64_t K,
                   const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                   int64_t E, int64_t N,
                   const uint32_t* lhs, const uint32_t* rhs, int64_t nb,
                   int mode, uint16_t* out);

/* float16 forms (activation dtype float16, model.cpp:208-214): x, scales,
 * biases and out in IEEE binary16; modes ORC_ACC_F64 and ORC_ACC_A only. */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
uint16_t orc_f64_to_f16(double d);  /* one rounding to nearest even */
float orc_sigmoid_f16(uint16_t g);  /* fp16(sigmoid(g)) as float (fp64, one rounding) */
int orc_qmm_t_f16(const uint16_t* x, int64_t M, int64_t K,
                  const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                  int64_t N, int mode, uint16_t* out);
int orc_gather_qmm_f16(const uint16_t* x, int64_t n_x, int64_t M, int64_t K,
                       const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                       int64_t E, int64_t N,
                       const uint32_t* lhs, const uint32_t* rhs, int64_t nb,
                       int mode, uint16_t* out);

/* ---- router (model.cpp:757-775; renorm per moe-support-plan.md:319-322) -- */
/* logits/probs [T,E] may be NULL. logit_bias [E] may be NULL (harness-only
 * extension: a per-expert logit offset added before softmax). */
int orc_router_topk(const uint16_t* x, int64_t T, int64_t H,
                    const uint16_t* wr, int64_t E, const uint16_t* logit_bias,
                    int k, int norm_topk,
                    uint16_t* logits, uint16_t* probs, uint32_t* inds, uint16_t* scores);
/* The same with the router in either form (model.cpp:757-763): wr_s == NULL:
 * wr is bf16 [E, H]; else wr is u32 [E, H/8] (affine 4-bit, group 64) with
 * bf16 scales/biases wr_s, wr_b [E, H/64]. Logits are exact fp64 sums
 * rounded once to bf16 in both forms. */
int orc_router_topk_q(const uint16_t* x, int64_t T, int64_t H,
                      const void* wr, const uint16_t* wr_s, const uint16_t* wr_b, int64_t E,
                      const uint16_t* logit_bias, int k, int norm_topk,
                      uint16_t* logits, uint16_t* probs, uint32_t* inds, uint16_t* scores);
/* The same in the block's activation dtype: f16 = 1 takes x, the router
 * rows (or their scales and biases), logit_bias and every output in float16
 * (logits and probabilities rounded once to fp16, the top-k on fp16 values). */
int orc_router_topk_dt(const uint16_t* x, int64_t T, int64_t H,
                       const void* wr, const uint16_t* wr_s, const uint16_t* wr_b, int64_t E,
                       const uint16_t* logit_bias, int k, int norm_topk, int f16,
                       uint16_t* logits, uint16_t* probs, uint32_t* inds, uint16_t* scores);

/* ---- sort / permutation (model.cpp:682-700) ---------------------------- */
/* order = stable argsort(flat inds); inv = argsort(order); src = order / k;
 * idx = flat[order]; offsets[e] = #entries with expert < e (E+1 entries). */
int orc_moe_sort(const uint32_t* inds, int64_t T, int k, int64_t E,
                 uint32_t* order, uint32_t* inv, uint32_t* src, uint32_t* idx,
                 uint32_t* offsets);

/* ---- full MoE block (model.cpp:750-807) -------------------------------- */
typedef struct {
  int64_t hidden;        /* H */
  int64_t n_experts;     /* E */
  int     top_k;         /* k */
  int64_t inter;         /* I  (moe_intermediate_size) */
  int64_t shared_inter;  /* Is (shared_expert_intermediate_size), 0 = none */
  int     norm_topk;     /* renormalise the k scores */
  int     group_size;    /* 64 */
  int     bits;          /* 4 */
  int     act_f16;       /* 1: float16 activations, scales, biases and router (a float16
                            checkpoint, model.cpp:208-214); 0: bfloat16 */
} orc_moe_cfg;

typedef struct {
  const void* router_w;          /* [E, H] bf16, or [E, H/8] u32 when router_s */
  const uint16_t* router_bias;   /* [E] bf16 or NULL (harness extension) */
  const uint32_t* gate_w;  const uint16_t* gate_s;  const uint16_t* gate_b;   /* [E, I, ..] */
  const uint32_t* up_w;    const uint16_t* up_s;    const uint16_t* up_b;     /* [E, I, ..] */
  const uint32_t* down_w;  const uint16_t* down_s;  const uint16_t* down_b;   /* [E, H, ..] */
  const uint32_t* sh_gate_w; const uint16_t* sh_gate_s; const uint16_t* sh_gate_b; /* [Is, ..] */
  const uint32_t* sh_up_w;   const uint16_t* sh_up_s;   const uint16_t* sh_up_b;
  const uint32_t* sh_down_w; const uint16_t* sh_down_s; const uint16_t* sh_down_b; /* [H, ..] */
  const void* sh_expert_gate_w;  /* [1, H] bf16, or [1, H/8] u32 when sh_expert_gate_s */
  const uint16_t* router_s;      /* [E, H/64] bf16 or NULL: quantized router (model.cpp:758-760) */
  const uint16_t* router_b;
  const uint16_t* sh_expert_gate_s; /* [1, H/64] or NULL: quantized gate (model.cpp:792-796) */
  const uint16_t* sh_expert_gate_b;
} orc_moe_weights;

/* y [T, H] bf16. inds/scores [T,k] may be NULL. token_subset (may be NULL):
 * compute y only for these n_subset tokens (routing still uses all tokens;
 * rows of y for other tokens are left untouched). */
int orc_moe_block(const orc_moe_cfg* cfg, const orc_moe_weights* w,
                  const uint16_t* x, int64_t T, int mode,
                  const int64_t* token_subset, int64_t n_subset,
                  uint16_t* y, uint32_t* inds, uint16_t* scores);

/* ---- decoder stack pieces (model.cpp:486-488, :843-911) ---------------- */
/* out [T, H] = rms_norm(x [T, H], w [H], eps) (mx::fast::rms_norm) */
int orc_rms_norm(const uint16_t* x, int64_t T, int64_t H, const uint16_t* w, float eps,
                 uint16_t* out);
/* (cos, sin) of p * base^(-2i/hd), fp32, for p < n_pos, i < hd/2:
 * cs[(p * hd/2 + i) * 2 + {0, 1}] */
void orc_rope_table(int64_t n_pos, int64_t hd, double base, float* cs);
/* mx::fast::rope (traditional=false, scale 1) in place on x [T, n_heads, hd] */
int orc_rope(uint16_t* x, int64_t T, int64_t n_heads, int64_t hd, const int64_t* pos,
             const float* cs);
/* mx::fast::scaled_dot_product_attention of one sequence, causal from q_off:
 * q [L, nh, hd], kc/vc [nkv, max_seq, hd] -> out [L, nh, hd] */
int orc_sdpa(const uint16_t* q, int64_t L, int64_t nh, int64_t hd, const uint16_t* kc,
             const uint16_t* vc, int64_t nkv, int64_t max_seq, int64_t q_off, float scale,
             uint16_t* out);
/* the same attention with the keys in up to 8 ranges of at least 64 (the
 * single-token split kernel's order): per-range softmax sums rescaled by
 * exp(m_s - M) and added in range order */
int orc_sdpa_split(const uint16_t* q, int64_t L, int64_t nh, int64_t hd, const uint16_t* kc,
                   const uint16_t* vc, int64_t nkv, int64_t max_seq, int64_t q_off, float scale,
                   uint16_t* out);

/* orc_moe_block with the expert choice given (inds [T, k]); scores are the
 * router's probabilities of those experts (renormalised when norm_topk). */
int orc_moe_block_routed(const orc_moe_cfg* cfg, const orc_moe_weights* w,
                         const uint16_t* x, int64_t T, int mode, const uint32_t* inds,
                         uint16_t* y, uint16_t* scores_out);

/* ---- Nemotron-H MoE block (nemotron_h.cpp:1010-1111) ------------------- */
/* fp32(sigmoid(l)) of a bf16 logit: 1 / (1 + orc_exp(-l)) in fp64, rounded
 * once to fp32 (mx::sigmoid of the fp32 cast logits, nemotron_h.cpp:1024). */
float orc_sigmoid_f32(uint16_t logit);

typedef struct {
  int64_t hidden;        /* H */
  int64_t n_experts;     /* E (n_routed_experts) */
  int     top_k;         /* k */
  int     norm_topk;     /* s / (sum(s) + 1e-20) when k > 1 */
  int64_t inter;         /* I (moe_intermediate_size) */
  int64_t shared_inter;  /* Is (moe_shared_expert_intermediate_size), 0 = none */
  int     n_group;       /* expert groups (1: no group limit) */
  int     topk_group;    /* groups kept */
  float   scaling;       /* routed_scaling_factor */
  int     group_size;    /* 64 */
  int     bits;          /* 4 */
} orc_nh_cfg;

typedef struct {
  const uint16_t* gate_w;  /* [E, H] bf16 router (mixer.gate.weight) */
  const float* cbias;      /* [E] fp32 e_score_correction_bias or NULL */
  const uint32_t* fc1_w;   const uint16_t* fc1_s;   const uint16_t* fc1_b;   /* [E, I, ..] */
  const uint32_t* fc2_w;   const uint16_t* fc2_s;   const uint16_t* fc2_b;   /* [E, H, ..] */
  const uint32_t* sh_up_w; const uint16_t* sh_up_s; const uint16_t* sh_up_b; /* [Is, ..] */
  const uint32_t* sh_down_w; const uint16_t* sh_down_s; const uint16_t* sh_down_b; /* [H, ..] */
} orc_nh_weights;

/* The router (nemotron_h.cpp:1017-1050): logits = bf16(x . gate_w^T) (exact
 * sum, one rounding); orig = orc_sigmoid_f32(logit); sel = orig + cbias
 * (fp32); with n_group > 1 the groups (E / n_group consecutive experts) are
 * scored by the sum of their two largest sel and every expert outside the
 * topk_group best groups (ties: lower group index kept) gets sel = 0; the
 * k largest sel are selected (ties: lower expert index; slots ordered sel
 * desc, index asc); scores = orig of the selected, / (sum in slot order +
 * 1e-20) when norm_topk and k > 1, then * scaling, all fp32. logits [T, E]
 * may be NULL. */
int orc_nh_route(const orc_nh_cfg* cfg, const uint16_t* x, int64_t T, const uint16_t* gate_w,
                 const float* cbias, uint16_t* logits, uint32_t* inds, float* scores);

/* The block (nemotron_h.cpp:1052-1111): for each selected expert, h =
 * bf16(x . fc1^T) (a quantized product, `mode` as orc_qmm_t: ORC_ACC_F64
 * or ORC_ACC_A), a = relu(h)^2 in fp32 (compiled relu2, nemotron_h.cpp:54-63:
 * maximum with a fp32 0 promotes to fp32), d = a . fc2^T with fp32 input and
 * output; routed = bf16(sum over slots, fp32 in slot order, of d * score);
 * the shared expert the same way without routing, and y = bf16(routed +
 * shared) (fp32 add). inds: the expert choice to use instead of the
 * router's (NULL: the router's); scores are then recomputed for it.
 * inds_out / scores_out [T, k] may be NULL. */
int orc_nh_moe_block(const orc_nh_cfg* cfg, const orc_nh_weights* w, const uint16_t* x, int64_t T,
                     int mode, const uint32_t* inds, uint16_t* y, uint32_t* inds_out,
                     float* scores_out);

/* threads used by the OpenMP loops (0 = leave the runtime default) */
void orc_set_threads(int n);
int  orc_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
