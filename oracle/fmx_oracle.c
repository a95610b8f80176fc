/*
 * fmx_oracle.c -- CPU restatement of FlashMLX's MoE hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP library, and the CPU
 * baseline that bench.py times beside it. Nothing in the product links it.
 * Build: oracle/Makefile (gcc, -ffp-contract=off so that every a*b+c below is
 * two roundings exactly as written, never a contracted fma).
 *
 * Every function cites the reference line it restates; see fmx_oracle.h for
 * which MLX op each one stands for and how it is pinned by the tests.
 */
#include "fmx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* numerics                                                                  */
/* ------------------------------------------------------------------------ */

float orc_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t orc_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* One rounding from fp64 to bf16 (nearest even). Implemented as round-to-odd
 * into fp32 followed by nearest-even into bf16: with 16 spare bits the odd
 * sticky bit makes the second rounding equal to a single direct rounding. */
uint16_t orc_f64_to_bf16(double d) {
  if (d != d) return 0x7fc0u;
  float f = (float)d;
  if ((double)f != d && !isinf(f)) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if (fabs((double)f) > fabs(d)) u -= 1u; /* rounded away from zero: step back */
    u |= 1u;                                /* sticky */
    memcpy(&f, &u, 4);
  }
  return orc_f32_to_bf16(f);
}

/* exp for the router softmax, deterministic across machines: Cody-Waite
 * reduction by ln2 (fdlibm's split constants) and the degree-13 Taylor
 * polynomial of e^t on |t| <= ln2/2 evaluated by Horner with explicit fma.
 * Only IEEE basic operations are used, so any conforming machine computes
 * the same bits. Results below 2^-1000 are returned as 0 (they round to 0
 * in bf16 after normalisation anyway). */
double orc_exp(double r) {
  if (r != r) return r;
  if (r > 709.0) return INFINITY;
  if (r < -690.0) return 0.0;
  const double log2e = 1.4426950408889634074;
  const double ln2_hi = 6.93147180369123816490e-01;
  const double ln2_lo = 1.90821492927058770002e-10;
  double n = rint(r * log2e);
  double t = fma(-n, ln2_hi, r);
  t = fma(-n, ln2_lo, t);
  double p = 1.0 / 6227020800.0;         /* 1/13! */
  p = fma(p, t, 1.0 / 479001600.0);      /* 1/12! */
  p = fma(p, t, 1.0 / 39916800.0);       /* 1/11! */
  p = fma(p, t, 1.0 / 3628800.0);        /* 1/10! */
  p = fma(p, t, 1.0 / 362880.0);         /* 1/9!  */
  p = fma(p, t, 1.0 / 40320.0);          /* 1/8!  */
  p = fma(p, t, 1.0 / 5040.0);           /* 1/7!  */
  p = fma(p, t, 1.0 / 720.0);            /* 1/6!  */
  p = fma(p, t, 1.0 / 120.0);            /* 1/5!  */
  p = fma(p, t, 1.0 / 24.0);             /* 1/4!  */
  p = fma(p, t, 1.0 / 6.0);              /* 1/3!  */
  p = fma(p, t, 0.5);                    /* 1/2!  */
  p = fma(p, t, 1.0);
  p = fma(p, t, 1.0);
  return ldexp(p, (int)n);
}

/* bf16(sigmoid(g)): MLX's sigmoid on a bf16 array returns bf16
 * (model.cpp:17, :802). Computed in fp64 and rounded once. */
float orc_sigmoid_bf16(uint16_t g) {
  double v = (double)orc_bf16_to_f32(g);
  return orc_bf16_to_f32(orc_f64_to_bf16(1.0 / (1.0 + exp(-v))));
}

static inline float bf(uint16_t h) { return orc_bf16_to_f32(h); }
static inline uint16_t rb(float f) { return orc_f32_to_bf16(f); }

static int g_threads = 0;
void orc_set_threads(int n) {
  g_threads = n;
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#endif
}
int orc_get_threads(void) {
#ifdef _OPENMP
  return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* affine quantization                                                       */
/* ------------------------------------------------------------------------ */

/* Restates MLX's CPU affine quantizer (mx::quantize, mode "affine") as
 * recalled: per group, scale = max((max-min)/15, 1e-7), signed toward the
 * larger-magnitude edge; q0 = rint(edge/scale); if q0 != 0 the scale is
 * snapped to edge/q0 and the bias is the edge (so the edge is a level);
 * q = clamp(rint((w - bias)/scale), 0, 15); scale and bias stored as bf16.
 * The reference consumes checkpoints quantized this way
 * (docs/superpowers/specs/2026-04-01-moe-support-design.md:138-151). */
int orc_quantize(const uint16_t* w, int64_t N, int64_t K, int group_size, int bits,
                 uint32_t* wq, uint16_t* scales, uint16_t* biases) {
  if (bits != 4 || group_size != 64 || K % group_size != 0) return -1;
  const float n_bins = 15.0f;
  const float eps = 1e-7f;
  const int64_t groups = N * (K / group_size);
#pragma omp parallel for schedule(static)
  for (int64_t gi = 0; gi < groups; ++gi) {
    const uint16_t* src = w + gi * group_size;
    float w_min = INFINITY, w_max = -INFINITY;
    for (int j = 0; j < group_size; ++j) {
      float v = bf(src[j]);
      w_max = fmaxf(w_max, v);
      w_min = fminf(w_min, v);
    }
    int mask = fabsf(w_min) > fabsf(w_max);
    float scale = fmaxf((w_max - w_min) / n_bins, eps);
    scale = mask ? scale : -scale;
    float edge = mask ? w_min : w_max;
    float q0 = rintf(edge / scale);
    float bias = 0.0f;
    if (q0 != 0.0f) {
      scale = edge / q0;
      bias = edge;
    }
    uint32_t* dst = wq + gi * (group_size / 8);
    for (int p = 0; p < group_size / 8; ++p) {
      uint32_t word = 0;
      for (int j = 0; j < 8; ++j) {
        float v = bf(src[p * 8 + j]);
        float q = rintf((v - bias) / scale);
        q = fminf(fmaxf(q, 0.0f), n_bins);
        word |= (uint32_t)q << (4 * j);
      }
      dst[p] = word;
    }
    scales[gi] = rb(scale);
    biases[gi] = rb(bias);
  }
  return 0;
}

int orc_dequantize(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                   int64_t N, int64_t K, int group_size, int bits, float* out) {
  if (bits != 4 || group_size != 64 || K % group_size != 0) return -1;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) {
      uint32_t word = wq[n * (K / 8) + k / 8];
      float q = (float)((word >> (4 * (k % 8))) & 15u);
      int64_t g = n * (K / group_size) + k / group_size;
      out[n * K + k] = bf(scales[g]) * q + bf(biases[g]);
    }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* quantized products                                                        */
/* ------------------------------------------------------------------------ */

/* One output element: x[K] (bf16) . deq(w row)[K], returned as bf16.
 * This is the inner loop of MLX's CPU quantized matmul with transpose=true
 * (the `_qmm_t` family), in one of four accumulation modes. */
static uint16_t qdot_row(const uint16_t* x, const uint32_t* wrow, const uint16_t* srow,
                         const uint16_t* brow, int64_t K, int mode) {
  const int64_t G = K / 64;
  if (mode == ORC_ACC_F64) {
    double acc = 0.0;
    for (int64_t g = 0; g < G; ++g) {
      double s = bf(srow[g]), b = bf(brow[g]);
      for (int p = 0; p < 8; ++p) {
        uint32_t word = wrow[g * 8 + p];
        for (int j = 0; j < 8; ++j) {
          double q = (double)((word >> (4 * j)) & 15u);
          acc += (double)bf(x[g * 64 + p * 8 + j]) * (s * q + b);
        }
      }
    }
    return orc_f64_to_bf16(acc);
  }
  if (mode == ORC_ACC_A) {
    float acc = 0.0f;
    for (int64_t g = 0; g < G; ++g) {
      float s = bf(srow[g]), b = bf(brow[g]);
      for (int p = 0; p < 8; ++p) {
        uint32_t word = wrow[g * 8 + p];
        for (int j = 0; j < 8; ++j) {
          float q = (float)((word >> (4 * j)) & 15u);
          float wv = s * q + b;
          acc += bf(x[g * 64 + p * 8 + j]) * wv;
        }
      }
    }
    return rb(acc);
  }
  if (mode == ORC_ACC_B) {
    uint16_t sum = 0;
    for (int64_t g = 0; g < G; ++g) {
      uint16_t s = srow[g], b = brow[g];
      for (int p = 0; p < 8; ++p) {
        uint32_t word = wrow[g * 8 + p];
        for (int j = 0; j < 8; ++j) {
          uint16_t q = rb((float)((word >> (4 * j)) & 15u));
          uint16_t sq = rb(bf(s) * bf(q));
          uint16_t wv = rb(bf(sq) + bf(b));
          uint16_t pr = rb(bf(x[g * 64 + p * 8 + j]) * bf(wv));
          sum = rb(bf(sum) + bf(pr));
        }
      }
    }
    return sum;
  }
  /* ORC_ACC_C: 8 fp32 lanes over k mod 8, then a pairwise lane sum */
  float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t g = 0; g < G; ++g) {
    float s = bf(srow[g]), b = bf(brow[g]);
    for (int p = 0; p < 8; ++p) {
      uint32_t word = wrow[g * 8 + p];
      for (int j = 0; j < 8; ++j) {
        float q = (float)((word >> (4 * j)) & 15u);
        float wv = q * s;
        wv = wv + b;
        lane[j] = lane[j] + bf(x[g * 64 + p * 8 + j]) * wv;
      }
    }
  }
  float a0 = lane[0] + lane[4], a1 = lane[1] + lane[5], a2 = lane[2] + lane[6], a3 = lane[3] + lane[7];
  float b0 = a0 + a2, b1 = a1 + a3;
  return rb(b0 + b1);
}

/* IEEE binary16 <-> binary32: the activation dtype a float16 checkpoint
 * runs in (model.cpp:208-214 detects it). Decoding is exact; encoding
 * rounds to nearest even, with overflow to infinity. */
float orc_f16_to_f32(uint16_t h) {
  const uint32_t sgn = (uint32_t)(h >> 15), ex = (h >> 10) & 31u, man = h & 1023u;
  float v;
  if (ex == 0)
    v = ldexpf((float)man, -24);
  else if (ex == 31)
    v = man ? NAN : INFINITY;
  else
    v = ldexpf((float)(man | 1024u), (int)ex - 25);
  return sgn ? -v : v;
}

/* One rounding to nearest even from a double (every float converts to a
 * double exactly, so orc_f32_to_f16 is the same rounding of a float). */
uint16_t orc_f64_to_f16(double f) {
  const uint16_t sgn = signbit(f) ? 0x8000u : 0u;
  if (isnan(f)) return (uint16_t)(sgn | 0x7e00u);
  const double a = fabs(f);
  if (a >= 65520.0) return (uint16_t)(sgn | 0x7c00u); /* rounds past the largest finite */
  /* a = m * 2^e exactly in double; the spacing of fp16 values near a */
  int e;
  (void)frexp(a, &e);                  /* a in [2^(e-1), 2^e) */
  int step_exp = e - 11;               /* 10 fraction bits: spacing 2^(e-11) */
  if (step_exp < -24) step_exp = -24;  /* subnormals: spacing 2^-24 */
  const double q = a / ldexp(1.0, step_exp); /* exact: a power-of-two scale */
  double r = nearbyint(q);             /* round half to even (default mode) */
  double v = r * ldexp(1.0, step_exp);
  /* v is now an fp16 value (or 65536 for inputs that round up past 65504) */
  if (v >= 65536.0) return (uint16_t)(sgn | 0x7c00u);
  int ve;
  (void)frexp(v, &ve);
  uint16_t bits;
  if (v == 0.0)
    bits = 0;
  else if (ve - 1 < -14) /* subnormal */
    bits = (uint16_t)(v * ldexp(1.0, 24));
  else
    bits = (uint16_t)(((ve - 1 + 15) << 10) | ((uint32_t)(v * ldexp(1.0, 11 - ve)) & 1023u));
  return (uint16_t)(sgn | bits);
}

uint16_t orc_f32_to_f16(float f) { return orc_f64_to_f16((double)f); }

/* The block's activation dtype (a float16 checkpoint runs the whole block
 * in float16, model.cpp:208-214): loads, roundings from fp32 and fp64 */
static inline float ld_dt(int f16, uint16_t h) { return f16 ? orc_f16_to_f32(h) : orc_bf16_to_f32(h); }
static inline uint16_t rnd_dt(int f16, float f) { return f16 ? orc_f32_to_f16(f) : orc_f32_to_bf16(f); }
static inline uint16_t rnd64_dt(int f16, double d) { return f16 ? orc_f64_to_f16(d) : orc_f64_to_bf16(d); }

/* fp16(sigmoid(g)) of a float16 g: fp64, rounded once */
float orc_sigmoid_f16(uint16_t g) {
  const double v = (double)orc_f16_to_f32(g);
  return orc_f16_to_f32(orc_f64_to_f16(1.0 / (1.0 + exp(-v))));
}

/* One output element in float16: x, scales and biases fp16; modes
 * ORC_ACC_F64 (the mathematical value) and ORC_ACC_A (fp32 dequantisation
 * s*q + b and sequential fp32 accumulation, as the bf16 form); the result
 * rounded once to fp16. */
static uint16_t qdot_row_f16(const uint16_t* x, const uint32_t* wrow, const uint16_t* srow,
                             const uint16_t* brow, int64_t K, int mode) {
  const int64_t G = K / 64;
  double acc64 = 0.0;
  float acc = 0.0f;
  for (int64_t g = 0; g < G; ++g) {
    const float s = orc_f16_to_f32(srow[g]), b = orc_f16_to_f32(brow[g]);
    for (int p = 0; p < 8; ++p) {
      const uint32_t word = wrow[g * 8 + p];
      for (int j = 0; j < 8; ++j) {
        const uint32_t q = (word >> (4 * j)) & 15u;
        const float xv = orc_f16_to_f32(x[g * 64 + p * 8 + j]);
        if (mode == ORC_ACC_F64)
          acc64 += (double)xv * ((double)s * (double)q + (double)b);
        else
          acc += xv * (s * (float)q + b);
      }
    }
  }
  return orc_f32_to_f16(mode == ORC_ACC_F64 ? (float)acc64 : acc);
}

/* quantized_matmul(x, w, scales, biases, transpose=true, 64, 4):
 * model.cpp:476-480 (linear_fast), :741-747 (shared expert). */
int orc_qmm_t(const uint16_t* x, int64_t M, int64_t K,
              const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
              int64_t N, int mode, uint16_t* out) {
  if (K % 64 != 0 || mode < 0 || mode > 3) return -1;
#pragma omp parallel for schedule(static) collapse(2)
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n)
      out[m * N + n] = qdot_row(x + m * K, w + n * (K / 8), scales + n * (K / 64),
                                biases + n * (K / 64), K, mode);
  return 0;
}

/* quantized_matmul on float16 x, scales, biases and output. */
int orc_qmm_t_f16(const uint16_t* x, int64_t M, int64_t K,
                  const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                  int64_t N, int mode, uint16_t* out) {
  if (K % 64 != 0 || (mode != ORC_ACC_F64 && mode != ORC_ACC_A)) return -1;
#pragma omp parallel for schedule(static) collapse(2)
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n)
      out[m * N + n] = qdot_row_f16(x + m * K, w + n * (K / 8), scales + n * (K / 64),
                                    biases + n * (K / 64), K, mode);
  return 0;
}

/* gather_qmm(x, w, scales, biases, lhs, rhs, transpose=true, 64, 4, "affine"):
 * model.cpp:703-721. Index lists are already broadcast to a common length. */
int orc_gather_qmm(const uint16_t* x, int64_t n_x, int64_t M, int64_t K,
                   const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                   int64_t E, int64_t N,
                   const uint32_t* lhs, const uint32_t* rhs, int64_t nb,
                   int mode, uint16_t* out) {
  if (K % 64 != 0 || mode < 0 || mode > 3) return -1;
  for (int64_t b = 0; b < nb; ++b)
    if ((int64_t)lhs[b] >= n_x || (int64_t)rhs[b] >= E) return -2;
  const int64_t wstride = N * (K / 8), sstride = N * (K / 64);
#pragma omp parallel for schedule(static) collapse(3)
  for (int64_t b = 0; b < nb; ++b)
    for (int64_t m = 0; m < M; ++m)
      for (int64_t n = 0; n < N; ++n) {
        const uint32_t e = rhs[b];
        out[(b * M + m) * N + n] =
            qdot_row(x + ((int64_t)lhs[b] * M + m) * K, w + e * wstride + n * (K / 8),
                     scales + e * sstride + n * (K / 64), biases + e * sstride + n * (K / 64),
                     K, mode);
      }
  return 0;
}

/* gather_qmm on float16 x, scales, biases and output. */
int orc_gather_qmm_f16(const uint16_t* x, int64_t n_x, int64_t M, int64_t K,
                       const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                       int64_t E, int64_t N,
                       const uint32_t* lhs, const uint32_t* rhs, int64_t nb,
                       int mode, uint16_t* out) {
  if (K % 64 != 0 || (mode != ORC_ACC_F64 && mode != ORC_ACC_A)) return -1;
  for (int64_t b = 0; b < nb; ++b)
    if ((int64_t)lhs[b] >= n_x || (int64_t)rhs[b] >= E) return -2;
  const int64_t wstride = N * (K / 8), sstride = N * (K / 64);
#pragma omp parallel for schedule(static) collapse(3)
  for (int64_t b = 0; b < nb; ++b)
    for (int64_t m = 0; m < M; ++m)
      for (int64_t n = 0; n < N; ++n) {
        const uint32_t e = rhs[b];
        out[(b * M + m) * N + n] =
            qdot_row_f16(x + ((int64_t)lhs[b] * M + m) * K, w + e * wstride + n * (K / 8),
                         scales + e * sstride + n * (K / 64), biases + e * sstride + n * (K / 64),
                         K, mode);
      }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* router                                                                    */
/* ------------------------------------------------------------------------ */

/* x . w^T of bf16 vectors: the products of two bf16 values are exact in
 * fp64 and so, except in cases far below any bf16 rounding boundary, are
 * all partial sums; the result is therefore independent of summation order
 * and is rounded once to bf16 (MLX: bf16 matmul with fp32 accumulate,
 * model.cpp:762). */
static uint16_t bf16_dot_exact(const uint16_t* a, const uint16_t* b, int64_t n) {
  double acc = 0.0;
  for (int64_t i = 0; i < n; ++i) acc += (double)bf(a[i]) * (double)bf(b[i]);
  return orc_f64_to_bf16(acc);
}

/* x . deq(w)^T of a bf16 vector and one quantized row (affine 4-bit, group
 * 64): the dequantised weight s*q + b (bf16 s, b; q in 0..15) and its product
 * with a bf16 x are exact in fp64, so the sum is formed as for bf16_dot_exact
 * and rounded once (MLX: quantized_matmul of the router / shared-expert gate,
 * model.cpp:758-760, :792-796). */
static uint16_t q4_dot_exact(const uint16_t* x, const uint32_t* w, const uint16_t* s,
                             const uint16_t* b, int64_t n) {
  double acc = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const double q = (double)((w[i / 8] >> (4 * (i % 8))) & 15u);
    const double sv = bf(s[i / 64]), bv = bf(b[i / 64]);
    acc += (double)bf(x[i]) * (sv * q + bv);
  }
  return orc_f64_to_bf16(acc);
}

/* one router / gate row in either form: bf16 (s == NULL) or quantized */
static uint16_t row_dot_exact(const uint16_t* x, const void* w, const uint16_t* s,
                              const uint16_t* b, int64_t row, int64_t H) {
  if (!s) return bf16_dot_exact(x, (const uint16_t*)w + row * H, H);
  return q4_dot_exact(x, (const uint32_t*)w + row * (H / 8), s + row * (H / 64),
                      b + row * (H / 64), H);
}

/* row_dot_exact in the block's activation dtype: float16 x, row, scales
 * and biases (their products with x are exact in fp64 as well), one
 * rounding to float16 */
static uint16_t row_dot_exact_dt(int f16, const uint16_t* x, const void* w, const uint16_t* s,
                                 const uint16_t* b, int64_t row, int64_t H) {
  if (!f16) return row_dot_exact(x, w, s, b, row, H);
  double acc = 0.0;
  if (!s) {
    const uint16_t* wr = (const uint16_t*)w + row * H;
    for (int64_t i = 0; i < H; ++i) acc += (double)ld_dt(1, x[i]) * (double)ld_dt(1, wr[i]);
  } else {
    const uint32_t* wq = (const uint32_t*)w + row * (H / 8);
    const uint16_t *sr = s + row * (H / 64), *br = b + row * (H / 64);
    for (int64_t i = 0; i < H; ++i) {
      const double q = (double)((wq[i / 8] >> (4 * (i % 8))) & 15u);
      acc += (double)ld_dt(1, x[i]) * ((double)ld_dt(1, sr[i / 64]) * q + (double)ld_dt(1, br[i / 64]));
    }
  }
  return orc_f64_to_f16(acc);
}

/* Softmax normaliser in a fixed summation order (MLX's own order is an
 * implementation detail of its CPU kernel): 64 partial sums, partial l
 * taking ex[l], ex[l+64], ... in turn, then six butterfly rounds
 * s_l <- s_l + s_{l xor w} for w = 32, 16, ..., 1; the result is s_0. */
static double softmax_den(const double* ex, int64_t E) {
  double s[64], t[64];
  for (int l = 0; l < 64; ++l) {
    s[l] = 0.0;
    for (int64_t e = l; e < E; e += 64) s[l] += ex[e];
  }
  for (int w = 32; w >= 1; w >>= 1) {
    for (int l = 0; l < 64; ++l) t[l] = s[l] + s[l ^ w];
    memcpy(s, t, sizeof s);
  }
  return s[0];
}

/* model.cpp:757-775: gates = x.Wr^T; softmax(precise=true); top-k by
 * argpartition(-gates, k-1)[..., :k]; scores = take_along_axis.
 * The selected set is the k largest bf16 probabilities with ties going to
 * the lower expert index; slots are ordered (prob desc, index asc).
 * norm_topk: s / sum(s) (moe-support-plan.md:319-322; nemotron_h.cpp:1045). */
int orc_router_topk(const uint16_t* x, int64_t T, int64_t H,
                    const uint16_t* wr, int64_t E, const uint16_t* logit_bias,
                    int k, int norm_topk,
                    uint16_t* logits, uint16_t* probs, uint32_t* inds, uint16_t* scores) {
  return orc_router_topk_q(x, T, H, wr, NULL, NULL, E, logit_bias, k, norm_topk, logits, probs,
                           inds, scores);
}

int orc_router_topk_q(const uint16_t* x, int64_t T, int64_t H,
                      const void* wr, const uint16_t* wr_s, const uint16_t* wr_b, int64_t E,
                      const uint16_t* logit_bias, int k, int norm_topk,
                      uint16_t* logits, uint16_t* probs, uint32_t* inds, uint16_t* scores) {
  return orc_router_topk_dt(x, T, H, wr, wr_s, wr_b, E, logit_bias, k, norm_topk, 0, logits, probs,
                            inds, scores);
}

int orc_router_topk_dt(const uint16_t* x, int64_t T, int64_t H,
                       const void* wr, const uint16_t* wr_s, const uint16_t* wr_b, int64_t E,
                       const uint16_t* logit_bias, int k, int norm_topk, int f16,
                       uint16_t* logits, uint16_t* probs, uint32_t* inds, uint16_t* scores) {
  if (k <= 0 || k > E || E > 65535) return -1;
  if (wr_s && (!wr_b || H % 64)) return -1;
  int rc = 0;
#pragma omp parallel
  {
    uint16_t* lg = (uint16_t*)malloc(sizeof(uint16_t) * E);
    uint16_t* pb = (uint16_t*)malloc(sizeof(uint16_t) * E);
    double* ex = (double*)malloc(sizeof(double) * E);
    unsigned char* taken = (unsigned char*)malloc(E);
    if (!lg || !pb || !ex || !taken) {
#pragma omp atomic write
      rc = -3;
    } else {
#pragma omp for schedule(static)
      for (int64_t t = 0; t < T; ++t) {
        for (int64_t e = 0; e < E; ++e) {
          uint16_t l = row_dot_exact_dt(f16, x + t * H, wr, wr_s, wr_b, e, H);
          if (logit_bias) l = rnd64_dt(f16, (double)ld_dt(f16, l) + (double)ld_dt(f16, logit_bias[e]));
          lg[e] = l;
        }
        double m = -INFINITY;
        for (int64_t e = 0; e < E; ++e) m = fmax(m, (double)ld_dt(f16, lg[e]));
        for (int64_t e = 0; e < E; ++e) ex[e] = orc_exp((double)ld_dt(f16, lg[e]) - m);
        const double sum = softmax_den(ex, E);
        for (int64_t e = 0; e < E; ++e) pb[e] = rnd64_dt(f16, ex[e] / sum);
        memset(taken, 0, E);
        for (int j = 0; j < k; ++j) {
          int64_t best = -1;
          for (int64_t e = 0; e < E; ++e) {
            if (taken[e]) continue;
            /* strict: ties keep lower index */
            if (best < 0 || ld_dt(f16, pb[e]) > ld_dt(f16, pb[best])) best = e;
          }
          taken[best] = 1;
          inds[t * k + j] = (uint32_t)best;
          scores[t * k + j] = pb[best];
        }
        if (norm_topk) {
          float s = 0.0f;
          for (int j = 0; j < k; ++j) s += ld_dt(f16, scores[t * k + j]);
          uint16_t sb = rnd_dt(f16, s);
          for (int j = 0; j < k; ++j) {
            float q = (float)((double)ld_dt(f16, scores[t * k + j]) / (double)ld_dt(f16, sb));
            scores[t * k + j] = rnd_dt(f16, q);
          }
        }
        if (logits) memcpy(logits + t * E, lg, sizeof(uint16_t) * E);
        if (probs) memcpy(probs + t * E, pb, sizeof(uint16_t) * E);
      }
    }
    free(lg);
    free(pb);
    free(ex);
    free(taken);
  }
  return rc;
}

/* ------------------------------------------------------------------------ */
/* sort / permutation                                                        */
/* ------------------------------------------------------------------------ */

/* model.cpp:682-700: stable counting sort by expert, which equals MLX's
 * stable argsort of the flattened indices. */
int orc_moe_sort(const uint32_t* inds, int64_t T, int k, int64_t E,
                 uint32_t* order, uint32_t* inv, uint32_t* src, uint32_t* idx,
                 uint32_t* offsets) {
  const int64_t n = T * (int64_t)k;
  uint32_t* cursor = (uint32_t*)calloc((size_t)E + 1, sizeof(uint32_t));
  if (!cursor) return -3;
  for (int64_t i = 0; i < n; ++i) {
    if ((int64_t)inds[i] >= E) {
      free(cursor);
      return -2;
    }
    cursor[inds[i] + 1]++;
  }
  for (int64_t e = 0; e < E; ++e) cursor[e + 1] += cursor[e];
  if (offsets) memcpy(offsets, cursor, sizeof(uint32_t) * (E + 1));
  for (int64_t i = 0; i < n; ++i) {
    uint32_t e = inds[i];
    uint32_t pos = cursor[e]++;
    if (order) order[pos] = (uint32_t)i;
    if (inv) inv[i] = pos;
    if (src) src[pos] = (uint32_t)(i / k);
    if (idx) idx[pos] = e;
  }
  free(cursor);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* full block                                                                */
/* ------------------------------------------------------------------------ */

/* compiled SwiGLU (model.cpp:14-25): multiply(multiply(g, sigmoid(g)), u),
 * each op producing the activation dtype (bf16, or fp16 when f16). */
static uint16_t swiglu_dt(int f16, uint16_t g, uint16_t u) {
  float sg = f16 ? orc_sigmoid_f16(g) : orc_sigmoid_bf16(g);
  uint16_t t = rnd_dt(f16, ld_dt(f16, g) * sg);
  return rnd_dt(f16, ld_dt(f16, t) * ld_dt(f16, u));
}

/* dense out[n] = x . deq(W[n]) for n < N, in the activation dtype (fp16
 * supports modes ORC_ACC_A and ORC_ACC_F64) */
static void qmv(int f16, const uint16_t* x, int64_t K, const uint32_t* w, const uint16_t* s,
                const uint16_t* b, int64_t N, int mode, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n)
    out[n] = f16 ? qdot_row_f16(x, w + n * (K / 8), s + n * (K / 64), b + n * (K / 64), K, mode)
                 : qdot_row(x, w + n * (K / 8), s + n * (K / 64), b + n * (K / 64), K, mode);
}

static int moe_block_impl(const orc_moe_cfg* cfg, const orc_moe_weights* w,
                          const uint16_t* x, int64_t T, int mode,
                          const int64_t* token_subset, int64_t n_subset, const uint32_t* forced,
                          uint16_t* y, uint32_t* inds_out, uint16_t* scores_out) {
  const int64_t H = cfg->hidden, E = cfg->n_experts, I = cfg->inter, Is = cfg->shared_inter;
  const int k = cfg->top_k;
  const int f16 = cfg->act_f16;
  if (cfg->group_size != 64 || cfg->bits != 4 || H % 64 || I % 64 || (Is && Is % 64)) return -1;
  if (f16 && mode != ORC_ACC_A && mode != ORC_ACC_F64) return -1;
  uint32_t* inds = (uint32_t*)malloc(sizeof(uint32_t) * T * k);
  uint16_t* scores = (uint16_t*)malloc(sizeof(uint16_t) * T * k);
  int64_t Imax = I > Is ? I : Is;
  uint16_t* g = (uint16_t*)malloc(sizeof(uint16_t) * Imax);
  uint16_t* u = (uint16_t*)malloc(sizeof(uint16_t) * Imax);
  uint16_t* a = (uint16_t*)malloc(sizeof(uint16_t) * Imax);
  uint16_t* d = (uint16_t*)malloc(sizeof(uint16_t) * H);
  float* acc = (float*)malloc(sizeof(float) * H);
  if (!inds || !scores || !g || !u || !a || !d || !acc) return -3;

  uint16_t* probs = forced ? (uint16_t*)malloc(sizeof(uint16_t) * T * E) : NULL;
  if (forced && !probs) return -3;
  int rc = orc_router_topk_dt(x, T, H, w->router_w, w->router_s, w->router_b, E, w->router_bias, k,
                              cfg->norm_topk, f16, NULL, probs, inds, scores);
  if (rc) return rc;
  if (forced) {
    /* the given expert choice, with this router's probabilities as scores
     * (renormalised as the router does) */
    for (int64_t t = 0; t < T; ++t) {
      for (int j = 0; j < k; ++j) {
        uint32_t e = forced[t * k + j];
        if (e >= (uint32_t)E) e = (uint32_t)(E - 1);
        inds[t * k + j] = e;
        scores[t * k + j] = probs[t * E + e];
      }
      if (cfg->norm_topk) {
        float sum = 0.0f;
        for (int j = 0; j < k; ++j) sum += ld_dt(f16, scores[t * k + j]);
        const uint16_t sb = rnd_dt(f16, sum);
        for (int j = 0; j < k; ++j)
          scores[t * k + j] =
              rnd_dt(f16, (float)((double)ld_dt(f16, scores[t * k + j]) / (double)ld_dt(f16, sb)));
      }
    }
    free(probs);
  }

  const int64_t n_tok = token_subset ? n_subset : T;
  const int64_t wst_gu = I * (H / 8), sst_gu = I * (H / 64);
  const int64_t wst_d = H * (I / 8), sst_d = H * (I / 64);
  for (int64_t ti = 0; ti < n_tok; ++ti) {
    const int64_t t = token_subset ? token_subset[ti] : ti;
    const uint16_t* xt = x + t * H;
    for (int64_t h = 0; h < H; ++h) acc[h] = 0.0f;
    /* switch_mlp, one (token, slot) row at a time: gather_qmm gate/up,
     * SwiGLU, gather_qmm down (model.cpp:703-721) */
    for (int j = 0; j < k; ++j) {
      const int64_t e = inds[t * k + j];
      qmv(f16, xt, H, w->gate_w + e * wst_gu, w->gate_s + e * sst_gu, w->gate_b + e * sst_gu, I, mode, g);
      qmv(f16, xt, H, w->up_w + e * wst_gu, w->up_s + e * sst_gu, w->up_b + e * sst_gu, I, mode, u);
      for (int64_t i = 0; i < I; ++i) a[i] = swiglu_dt(f16, g[i], u[i]);
      qmv(f16, a, I, w->down_w + e * wst_d, w->down_s + e * sst_d, w->down_b + e * sst_d, H, mode, d);
      /* y = sum(y * scores[..., None], -2) (model.cpp:782-784): the product
       * is in the activation dtype, the k-sum accumulates in fp32 in slot
       * order */
      const float sc = ld_dt(f16, scores[t * k + j]);
      for (int64_t h = 0; h < H; ++h) acc[h] += ld_dt(f16, rnd_dt(f16, ld_dt(f16, d[h]) * sc));
    }
    for (int64_t h = 0; h < H; ++h) y[t * H + h] = rnd_dt(f16, acc[h]);
    if (Is > 0) {
      /* shared_expert_mlp (model.cpp:736-748) and its sigmoid gate (:787-803) */
      uint16_t gl = row_dot_exact_dt(f16, xt, w->sh_expert_gate_w, w->sh_expert_gate_s,
                                     w->sh_expert_gate_b, 0, H);
      float gv = f16 ? orc_sigmoid_f16(gl) : orc_sigmoid_bf16(gl);
      qmv(f16, xt, H, w->sh_gate_w, w->sh_gate_s, w->sh_gate_b, Is, mode, g);
      qmv(f16, xt, H, w->sh_up_w, w->sh_up_s, w->sh_up_b, Is, mode, u);
      for (int64_t i = 0; i < Is; ++i) a[i] = swiglu_dt(f16, g[i], u[i]);
      qmv(f16, a, Is, w->sh_down_w, w->sh_down_s, w->sh_down_b, H, mode, d);
      for (int64_t h = 0; h < H; ++h) {
        uint16_t sh = rnd_dt(f16, gv * ld_dt(f16, d[h]));
        y[t * H + h] = rnd_dt(f16, ld_dt(f16, y[t * H + h]) + ld_dt(f16, sh));
      }
    }
  }
  if (inds_out) memcpy(inds_out, inds, sizeof(uint32_t) * T * k);
  if (scores_out) memcpy(scores_out, scores, sizeof(uint16_t) * T * k);
  free(inds);
  free(scores);
  free(g);
  free(u);
  free(a);
  free(d);
  free(acc);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Nemotron-H MoE block                                                      */
/* ------------------------------------------------------------------------ */

float orc_sigmoid_f32(uint16_t logit) {
  return (float)(1.0 / (1.0 + orc_exp(-(double)bf(logit))));
}

/* nemotron_h.cpp:1022-1049 for one token: lg [E] bf16 logits in; inds, scores out */
static void nh_select(const orc_nh_cfg* c, const uint16_t* lg, const float* cbias, float* orig,
                      float* sel, unsigned char* taken, uint32_t* inds, float* scores) {
  const int64_t E = c->n_experts;
  const int k = c->top_k;
  for (int64_t e = 0; e < E; ++e) {
    orig[e] = orc_sigmoid_f32(lg[e]);
    sel[e] = cbias ? orig[e] + cbias[e] : orig[e];
  }
  if (c->n_group > 1) {
    /* group score: the two largest sel of the group, added (:1031) */
    const int64_t G = E / c->n_group;
    float gs[1024];
    for (int g = 0; g < c->n_group; ++g) {
      float m1 = -INFINITY, m2 = -INFINITY;
      for (int64_t e = g * G; e < (g + 1) * G; ++e) {
        if (sel[e] > m1) {
          m2 = m1;
          m1 = sel[e];
        } else if (sel[e] > m2) {
          m2 = sel[e];
        }
      }
      gs[g] = m1 + m2;
    }
    /* argpartition(group_scores, n_group - topk_group - 1) zeroes the
     * n_group - topk_group first groups in MLX's (value asc, index asc)
     * order (:1032-1039), the comparator behind the top-k tie rule below:
     * among equal group scores the lower index is zeroed first. So the
     * topk_group groups that stay are the last ones in that order: group
     * score desc, index desc. Their experts keep their selection scores;
     * the others' get 0. */
    unsigned char keep[1024];
    memset(keep, 0, sizeof keep);
    for (int r = 0; r < c->topk_group; ++r) {
      int best = -1;
      for (int g = 0; g < c->n_group; ++g)
        if (!keep[g] && (best < 0 || gs[g] >= gs[best])) best = g;
      keep[best] = 1;
    }
    for (int g = 0; g < c->n_group; ++g)
      if (!keep[g])
        for (int64_t e = g * G; e < (g + 1) * G; ++e) sel[e] = 0.0f;
  }
  /* top-k of sel (:1042-1043), ties to the lower index */
  memset(taken, 0, (size_t)E);
  for (int j = 0; j < k; ++j) {
    int64_t best = -1;
    for (int64_t e = 0; e < E; ++e)
      if (!taken[e] && (best < 0 || sel[e] > sel[best])) best = e;
    taken[best] = 1;
    inds[j] = (uint32_t)best;
  }
  /* scores from the unbiased sigmoid (:1044-1049) */
  float den = 0.0f;
  for (int j = 0; j < k; ++j) {
    scores[j] = orig[inds[j]];
    den += scores[j];
  }
  if (c->norm_topk && k > 1) {
    den += 1e-20f;
    for (int j = 0; j < k; ++j) scores[j] = scores[j] / den;
  }
  for (int j = 0; j < k; ++j) scores[j] = scores[j] * c->scaling;
}

static int nh_cfg_ok(const orc_nh_cfg* c) {
  if (c->group_size != 64 || c->bits != 4 || c->hidden % 64 || c->inter % 64 ||
      (c->shared_inter && c->shared_inter % 64))
    return 0;
  if (c->top_k < 1 || c->top_k > c->n_experts || c->n_experts > 1024) return 0;
  if (c->n_group < 1 || c->n_group > 1024 || c->n_experts % c->n_group) return 0;
  if (c->n_group > 1 && (c->n_experts / c->n_group < 2 || c->topk_group < 1 || c->topk_group > c->n_group))
    return 0;
  return 1;
}

int orc_nh_route(const orc_nh_cfg* c, const uint16_t* x, int64_t T, const uint16_t* gate_w,
                 const float* cbias, uint16_t* logits, uint32_t* inds, float* scores) {
  if (!nh_cfg_ok(c)) return -1;
  const int64_t E = c->n_experts, H = c->hidden;
  int rc = 0;
#pragma omp parallel
  {
    uint16_t* lg = (uint16_t*)malloc(sizeof(uint16_t) * E);
    float* orig = (float*)malloc(sizeof(float) * E);
    float* sel = (float*)malloc(sizeof(float) * E);
    unsigned char* taken = (unsigned char*)malloc(E);
    if (!lg || !orig || !sel || !taken) {
#pragma omp atomic write
      rc = -3;
    } else {
#pragma omp for schedule(static)
      for (int64_t t = 0; t < T; ++t) {
        for (int64_t e = 0; e < E; ++e) lg[e] = bf16_dot_exact(x + t * H, gate_w + e * H, H);
        nh_select(c, lg, cbias, orig, sel, taken, inds + t * c->top_k, scores + t * c->top_k);
        if (logits) memcpy(logits + t * E, lg, sizeof(uint16_t) * E);
      }
    }
    free(lg);
    free(orig);
    free(sel);
    free(taken);
  }
  return rc;
}

/* out[n] = a[K] (fp32) . deq(W[n]) for n < N, fp32 (gather_qmm / quantized_matmul
 * of an fp32 input: the dequantised weights and the accumulation in fp32) */
static void qmv_f32(const float* a, int64_t K, const uint32_t* w, const uint16_t* s,
                    const uint16_t* b, int64_t N, int mode, float* out) {
  const int64_t G = K / 64;
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    const uint32_t* wr = w + n * (K / 8);
    const uint16_t* sr = s + n * G;
    const uint16_t* br = b + n * G;
    if (mode == ORC_ACC_F64) {
      double acc = 0.0;
      for (int64_t i = 0; i < K; ++i) {
        const double q = (double)((wr[i / 8] >> (4 * (i % 8))) & 15u);
        acc += (double)a[i] * ((double)bf(sr[i / 64]) * q + (double)bf(br[i / 64]));
      }
      out[n] = (float)acc;
    } else {
      float acc = 0.0f;
      for (int64_t i = 0; i < K; ++i) {
        const float q = (float)((wr[i / 8] >> (4 * (i % 8))) & 15u);
        const float wv = bf(sr[i / 64]) * q + bf(br[i / 64]);
        acc += a[i] * wv;
      }
      out[n] = acc;
    }
  }
}

/* relu2 (nemotron_h.cpp:54-63) of a bf16 row: fp32, exact */
static void relu2_row(const uint16_t* h, int64_t n, float* a) {
  for (int64_t i = 0; i < n; ++i) {
    const float v = bf(h[i]) > 0.0f ? bf(h[i]) : 0.0f;
    a[i] = v * v;
  }
}

int orc_nh_moe_block(const orc_nh_cfg* c, const orc_nh_weights* w, const uint16_t* x, int64_t T,
                     int mode, const uint32_t* forced, uint16_t* y, uint32_t* inds_out,
                     float* scores_out) {
  if (!nh_cfg_ok(c) || (mode != ORC_ACC_F64 && mode != ORC_ACC_A)) return -1;
  const int64_t H = c->hidden, E = c->n_experts, I = c->inter, Is = c->shared_inter;
  const int k = c->top_k;
  uint32_t* inds = (uint32_t*)malloc(sizeof(uint32_t) * T * k);
  float* scores = (float*)malloc(sizeof(float) * T * k);
  uint16_t* lg = (uint16_t*)malloc(sizeof(uint16_t) * T * E);
  const int64_t Imax = I > Is ? I : Is;
  uint16_t* hb = (uint16_t*)malloc(sizeof(uint16_t) * Imax);
  float* a = (float*)malloc(sizeof(float) * Imax);
  float* d = (float*)malloc(sizeof(float) * H);
  float* acc = (float*)malloc(sizeof(float) * H);
  float* orig = (float*)malloc(sizeof(float) * E);
  float* sel = (float*)malloc(sizeof(float) * E);
  unsigned char* taken = (unsigned char*)malloc(E);
  if (!inds || !scores || !lg || !hb || !a || !d || !acc || !orig || !sel || !taken) return -3;
  int rc = orc_nh_route(c, x, T, w->gate_w, w->cbias, lg, inds, scores);
  if (rc) return rc;
  if (forced) {
    /* the given choice, scored as the router scores its own (:1044-1049) */
    orc_nh_cfg one = *c;
    for (int64_t t = 0; t < T; ++t) {
      float den = 0.0f;
      for (int j = 0; j < k; ++j) {
        uint32_t e = forced[t * k + j];
        if (e >= (uint32_t)E) e = (uint32_t)(E - 1);
        inds[t * k + j] = e;
        scores[t * k + j] = orc_sigmoid_f32(lg[t * E + e]);
        den += scores[t * k + j];
      }
      if (one.norm_topk && k > 1) {
        den += 1e-20f;
        for (int j = 0; j < k; ++j) scores[t * k + j] = scores[t * k + j] / den;
      }
      for (int j = 0; j < k; ++j) scores[t * k + j] = scores[t * k + j] * one.scaling;
    }
  }
  const int64_t wst1 = I * (H / 8), sst1 = I * (H / 64);
  const int64_t wst2 = H * (I / 8), sst2 = H * (I / 64);
  for (int64_t t = 0; t < T; ++t) {
    const uint16_t* xt = x + t * H;
    for (int64_t h = 0; h < H; ++h) acc[h] = 0.0f;
    /* switch_mlp: fc1 -> relu2 -> fc2 (:1086-1094), the weighted sum (:1098-1099) */
    for (int j = 0; j < k; ++j) {
      const int64_t e = inds[t * k + j];
      qmv(0, xt, H, w->fc1_w + e * wst1, w->fc1_s + e * sst1, w->fc1_b + e * sst1, I, mode, hb);
      relu2_row(hb, I, a);
      qmv_f32(a, I, w->fc2_w + e * wst2, w->fc2_s + e * sst2, w->fc2_b + e * sst2, H, mode, d);
      const float sc = scores[t * k + j];
      for (int64_t h = 0; h < H; ++h) {
        const float p = d[h] * sc;
        acc[h] = acc[h] + p;
      }
    }
    for (int64_t h = 0; h < H; ++h) y[t * H + h] = rb(acc[h]);
    if (Is > 0) {
      /* shared expert (:1102-1108): up -> relu2 -> down, added in fp32 */
      qmv(0, xt, H, w->sh_up_w, w->sh_up_s, w->sh_up_b, Is, mode, hb);
      relu2_row(hb, Is, a);
      qmv_f32(a, Is, w->sh_down_w, w->sh_down_s, w->sh_down_b, H, mode, d);
      for (int64_t h = 0; h < H; ++h) y[t * H + h] = rb(bf(y[t * H + h]) + d[h]);
    }
  }
  if (inds_out) memcpy(inds_out, inds, sizeof(uint32_t) * T * k);
  if (scores_out) memcpy(scores_out, scores, sizeof(float) * T * k);
  free(inds);
  free(scores);
  free(lg);
  free(hb);
  free(a);
  free(d);
  free(acc);
  free(orig);
  free(sel);
  free(taken);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* decoder stack pieces                                                      */
/* ------------------------------------------------------------------------ */

/* mx::fast::rms_norm (model.cpp:486-488) as MLX's fallback composes it
 * (recalled): x in fp32, x * rsqrt(mean(x^2) + eps) cast to bf16, then the
 * bf16 product with the weight. Restated with the sum of squares and the
 * normaliser in fp64, x * r rounded to bf16 and the product with w (two bf16
 * values, exact in fp64) rounded once. */
int orc_rms_norm(const uint16_t* x, int64_t T, int64_t H, const uint16_t* w, float eps,
                 uint16_t* out) {
  if (T < 0 || H <= 0) return -1;
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t) {
    const uint16_t* xr = x + t * H;
    double ss = 0.0;
    for (int64_t i = 0; i < H; ++i) {
      const double v = (double)bf(xr[i]);
      ss += v * v;
    }
    const double r = 1.0 / sqrt(ss / (double)H + (double)eps);
    for (int64_t i = 0; i < H; ++i) {
      const uint16_t n = orc_f64_to_bf16((double)bf(xr[i]) * r);
      out[t * H + i] = orc_f64_to_bf16((double)bf(n) * (double)bf(w[i]));
    }
  }
  return 0;
}

/* RoPE angles of mx::fast::rope (traditional = false, scale 1,
 * model.cpp:871-872): theta(p, i) = p * base^(-2i/hd) for i < hd/2, as
 * (cos, sin) pairs rounded to fp32: cs[(p * hd/2 + i) * 2 + {0, 1}]. */
void orc_rope_table(int64_t n_pos, int64_t hd, double base, float* cs) {
  const int64_t half = hd / 2;
  for (int64_t i = 0; i < half; ++i) {
    const double inv = pow(base, -(2.0 * (double)i) / (double)hd);
    for (int64_t p = 0; p < n_pos; ++p) {
      const double th = (double)p * inv;
      cs[(p * half + i) * 2] = (float)cos(th);
      cs[(p * half + i) * 2 + 1] = (float)sin(th);
    }
  }
}

/* Non-traditional RoPE in place on x [T, n_heads, hd] at positions pos[T]:
 * element pairs (i, i + hd/2) rotate by theta(pos, i):
 *   x1' = x1 cos - x2 sin,  x2' = x1 sin + x2 cos,
 * each from the exact products (bf16 x fp32 is exact in fp64), rounded once
 * to bf16. */
int orc_rope(uint16_t* x, int64_t T, int64_t n_heads, int64_t hd, const int64_t* pos,
             const float* cs) {
  if (hd % 2) return -1;
  const int64_t half = hd / 2;
  for (int64_t t = 0; t < T; ++t) {
    const float* c = cs + pos[t] * half * 2;
    for (int64_t h = 0; h < n_heads; ++h) {
      uint16_t* v = x + (t * n_heads + h) * hd;
      for (int64_t i = 0; i < half; ++i) {
        const double x1 = (double)bf(v[i]), x2 = (double)bf(v[i + half]);
        const double co = (double)c[2 * i], si = (double)c[2 * i + 1];
        v[i] = orc_f64_to_bf16(x1 * co - x2 * si);
        v[i + half] = orc_f64_to_bf16(x1 * si + x2 * co);
      }
    }
  }
  return 0;
}

/* mx::fast::scaled_dot_product_attention (model.cpp:879-882) for one
 * sequence: q [L, nh, hd] (roped), the cache of that sequence kc / vc
 * [nkv, max_seq, hd] holding keys 0 .. q_off + L - 1; query l (position
 * q_off + l) attends to keys 0 .. q_off + l (causal; for L = 1 that is every
 * key). q head h reads kv head h / (nh / nkv). Scores are fp32 dot products
 * (exact bf16 products, summed over d in order) times scale; the softmax is
 * formed in fp64 with the deterministic exp (e_j = exp(s_j - max)), the
 * output as sum_j e_j v_j / sum_j e_j in fp64, each sum over four contiguous
 * quarters of the keys (in order within a quarter, fma), the quarter sums
 * added in order, rounded once to bf16: out [L, nh, hd]. */
int orc_sdpa(const uint16_t* q, int64_t L, int64_t nh, int64_t hd, const uint16_t* kc,
             const uint16_t* vc, int64_t nkv, int64_t max_seq, int64_t q_off, float scale,
             uint16_t* out) {
  if (nkv <= 0 || nh % nkv || q_off + L > max_seq) return -1;
  const int64_t rep = nh / nkv;
#pragma omp parallel for schedule(static) collapse(2)
  for (int64_t l = 0; l < L; ++l) {
    for (int64_t h = 0; h < nh; ++h) {
      const int64_t g = h / rep, nk = q_off + l + 1;
      const uint16_t* qv = q + (l * nh + h) * hd;
      const uint16_t* kb = kc + g * max_seq * hd;
      const uint16_t* vb = vc + g * max_seq * hd;
      float* s = (float*)malloc(sizeof(float) * nk);
      double* e = (double*)malloc(sizeof(double) * nk);
      float m = -INFINITY;
      for (int64_t j = 0; j < nk; ++j) {
        float acc = 0.0f;
        for (int64_t d = 0; d < hd; ++d) acc += bf(qv[d]) * bf(kb[j * hd + d]);
        s[j] = acc * scale;
        if (s[j] > m) m = s[j];
      }
      for (int64_t j = 0; j < nk; ++j) e[j] = orc_exp((double)s[j] - (double)m);
      /* four contiguous quarters of the keys, each summed in order, the
       * quarter sums added in order */
      const int64_t qn = (nk + 3) / 4;
      double den = 0.0, dq[4];
      for (int qi = 0; qi < 4; ++qi) {
        const int64_t j0 = qi * qn < nk ? qi * qn : nk, j1 = j0 + qn < nk ? j0 + qn : nk;
        dq[qi] = 0.0;
        for (int64_t j = j0; j < j1; ++j) dq[qi] += e[j];
        den = qi ? den + dq[qi] : dq[qi];
      }
      for (int64_t d = 0; d < hd; ++d) {
        double num = 0.0;
        for (int qi = 0; qi < 4; ++qi) {
          const int64_t j0 = qi * qn < nk ? qi * qn : nk, j1 = j0 + qn < nk ? j0 + qn : nk;
          double part = 0.0;
          for (int64_t j = j0; j < j1; ++j) part = fma(e[j], (double)bf(vb[j * hd + d]), part);
          num = qi ? num + part : part;
        }
        out[(l * nh + h) * hd + d] = orc_f64_to_bf16(num / den);
      }
      free(s);
      free(e);
    }
  }
  return 0;
}

/* The single-token attention of libfmx's split kernel (attn_split_kernel):
 * query l's keys 0 .. nk - 1 (nk = q_off + l + 1) in S = min(16, ceil(nk /
 * 32)) contiguous ranges [nk s / S, nk (s + 1) / S); in range s, m_s = the
 * largest fp32 score, e_j = exp(s_j - m_s) in fp64 with the deterministic
 * exp, and over the key classes c = (j - j0) mod 4 (each in key order)
 * den_s = ((D_0 + D_1) + D_2) + D_3, D_c = sum e_j, and num_s likewise
 * from N_c = sum e_j v_j (fma); then M = max_s m_s, f_s = exp(m_s - M), den = sum_s f_s den_s and num =
 * sum_s f_s num_s (ranges in order, fma; the first term a product), out =
 * bf16(num / den). Scores: s_j = scale * (((P_0 + P_1) + ...) + P_{hd/8-1})
 * with P_c the fp32 sum over dimensions 8c .. 8c + 7 in order (exact bf16
 * products). */
int orc_sdpa_split(const uint16_t* q, int64_t L, int64_t nh, int64_t hd, const uint16_t* kc,
                   const uint16_t* vc, int64_t nkv, int64_t max_seq, int64_t q_off, float scale,
                   uint16_t* out) {
  if (nkv <= 0 || nh % nkv || q_off + L > max_seq) return -1;
  const int64_t rep = nh / nkv;
#pragma omp parallel for schedule(static) collapse(2)
  for (int64_t l = 0; l < L; ++l) {
    for (int64_t h = 0; h < nh; ++h) {
      const int64_t g = h / rep, nk = q_off + l + 1;
      const uint16_t* qv = q + (l * nh + h) * hd;
      const uint16_t* kb = kc + g * max_seq * hd;
      const uint16_t* vb = vc + g * max_seq * hd;
      int64_t S = (nk + 31) / 32;
      if (S > 16) S = 16;
      float* s = (float*)malloc(sizeof(float) * nk);
      double* ms = (double*)malloc(sizeof(double) * S);
      double* dens = (double*)malloc(sizeof(double) * S);
      double* nums = (double*)malloc(sizeof(double) * S * hd);
      for (int64_t j = 0; j < nk; ++j) {
        float acc = 0.0f;
        for (int64_t c = 0; c < hd / 8; ++c) {
          float pc = 0.0f;
          for (int64_t d = 8 * c; d < 8 * c + 8; ++d) pc += bf(qv[d]) * bf(kb[j * hd + d]);
          acc = c ? acc + pc : pc;
        }
        s[j] = acc * scale;
      }
      double M = -INFINITY;
      for (int64_t r = 0; r < S; ++r) {
        const int64_t j0 = nk * r / S, j1 = nk * (r + 1) / S;
        float m = -INFINITY;
        for (int64_t j = j0; j < j1; ++j)
          if (s[j] > m) m = s[j];
        ms[r] = (double)m;
        if (ms[r] > M) M = ms[r];
        double dc[4] = {0.0, 0.0, 0.0, 0.0};
        for (int64_t j = j0; j < j1; ++j) dc[(j - j0) % 4] += orc_exp((double)s[j] - ms[r]);
        dens[r] = ((dc[0] + dc[1]) + dc[2]) + dc[3];
        for (int64_t d = 0; d < hd; ++d) {
          double nc[4] = {0.0, 0.0, 0.0, 0.0};
          for (int64_t j = j0; j < j1; ++j)
            nc[(j - j0) % 4] = fma(orc_exp((double)s[j] - ms[r]), (double)bf(vb[j * hd + d]), nc[(j - j0) % 4]);
          nums[r * hd + d] = ((nc[0] + nc[1]) + nc[2]) + nc[3];
        }
      }
      double den = 0.0;
      for (int64_t r = 0; r < S; ++r) {
        const double f = orc_exp(ms[r] - M);
        den = r ? fma(dens[r], f, den) : dens[r] * f;
      }
      for (int64_t d = 0; d < hd; ++d) {
        double num = 0.0;
        for (int64_t r = 0; r < S; ++r) {
          const double f = orc_exp(ms[r] - M);
          num = r ? fma(nums[r * hd + d], f, num) : nums[r * hd + d] * f;
        }
        out[(l * nh + h) * hd + d] = orc_f64_to_bf16(num / den);
      }
      free(s);
      free(ms);
      free(dens);
      free(nums);
    }
  }
  return 0;
}

int orc_moe_block(const orc_moe_cfg* cfg, const orc_moe_weights* w,
                  const uint16_t* x, int64_t T, int mode,
                  const int64_t* token_subset, int64_t n_subset,
                  uint16_t* y, uint32_t* inds_out, uint16_t* scores_out) {
  return moe_block_impl(cfg, w, x, T, mode, token_subset, n_subset, NULL, y, inds_out, scores_out);
}

/* The MoE block with the expert choice given (inds [T, k]): the scores are
 * this router's probabilities of those experts (renormalised when
 * norm_topk), the rest as orc_moe_block. Lets a whole decoder stack be
 * compared with a GPU run that chose differently at a router near-tie. */
int orc_moe_block_routed(const orc_moe_cfg* cfg, const orc_moe_weights* w,
                         const uint16_t* x, int64_t T, int mode, const uint32_t* inds,
                         uint16_t* y, uint16_t* scores_out) {
  if (!inds) return -1;
  return moe_block_impl(cfg, w, x, T, mode, NULL, 0, inds, y, NULL, scores_out);
}
