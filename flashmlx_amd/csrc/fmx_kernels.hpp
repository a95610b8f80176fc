// fmx_kernels.hpp -- kernel argument blocks and launchers (library-internal).
#pragma once

#include "fmx_common.hpp"

struct fmx_moe_config;
struct fmx_moe_weights;

namespace fmx {

// ---------------------------------------------------------------- sorting
// Stable counting sort of n keys (< E) by key: the permutation MLX's
// argsort(flatten(inds)) produces in switch_mlp (server/src/model.cpp:686-699)
// plus the non-empty-expert segment table the grouped GEMMs walk.
struct SortOut {
  uint32_t* order;    // [n]   sorted position -> entry           (nullable)
  uint32_t* inv;      // [n]   entry -> sorted position           (nullable)
  uint32_t* src;      // [n]   sorted position -> entry / k       (nullable)
  uint32_t* idx;      // [n]   sorted position -> key             (nullable)
  uint32_t* offsets;  // [E+1] first sorted position of each key  (required)
  uint32_t* seg_n;    // [1]   number of non-empty keys U         (nullable)
  uint32_t* seg_exp;  // [E]   u -> key of the u-th non-empty key (nullable)
  uint32_t* seg_off;  // [E+1] u -> first sorted position         (nullable)
  uint32_t* base;     // [E * ceil(n/64)] scratch
  // pass table of the prefill GEMMs: each segment cut into passes of at
  // most kPassRows rows, in segment order (both nullable)
  uint32_t* pass_n;   // [1]   number of passes
  uint32_t* pass_tab; // [max_passes(n, E)][2]: first sorted row, key | rows << 16
  // gather_qmm (row_map nullable): sorted position -> x row of its entry
  // o = b * row_m + m, lhs[b] * row_m + m (lhs values clamped into the
  // x_rows / row_m batches of x)
  uint32_t* row_map;
  const uint32_t* row_lhs;
  int row_m, x_rows;
  // (flag nullable) workgroup 0 also writes *flag = the OR of the n_ovf
  // words at ovf (a copy kernel's per-block overflow words, n_ovf <= 1024)
  const uint32_t* ovf;
  int n_ovf;
  uint32_t* flag;
};

constexpr int kPassRows = 64;
// most passes n sorted rows over at most E keys can need
__host__ __device__ inline int max_passes(int64_t n, int64_t E) {
  return static_cast<int>((n < E ? n : E) + (n + kPassRows - 1) / kPassRows);
}

// Sort by one workgroup of 1024 threads per key value (separate launch),
// keys LDS-resident up to kSortLdsN of them, re-read from global memory
// (an L2-resident array) beyond.
constexpr int kSortThreads = 1024;
constexpr int kSortLdsN = 32 * 1024;       // keys held in LDS (16 bits each)
constexpr int64_t kSortMaxN = 1 << 22;     // keys of one sort
constexpr int kSortMaxE = 1024;            // per-wave key counters in LDS
bool sort_fits(int64_t n, int64_t E);
hipError_t launch_sort(const uint32_t* keys, int n, int k, int E, const SortOut& o,
                       hipStream_t stream);

// ---------------------------------------------------------------- router
// logits = x . [Wr; wsg]^T in fp64 (exact bf16 products), rounded once to
// bf16; per token: softmax in fp64 with exp_det, top-k, scores, renorm;
// optionally the sort of all tokens' indices in the last workgroup.
constexpr int kRouterTok = 8;      // tokens per tile
constexpr int kRouterThreads = 256;  // 4 waves; each wave forms 8 tokens x cols_per_wave logits
constexpr int kRouterSortCnt = 16 * 1024;  // LDS bytes for a fused sort's count table
constexpr int kRouterSortMaxN = 2048;

// Router rows come either as bf16 [rows, H] or as MLX affine 4-bit rows
// (u32 [rows, H/8] with bf16 scales/biases [rows, H/64]; `s` non-null).
struct RouterRows {
  const void* w;
  const uint16_t* s;
  const uint16_t* b;
};

struct RouterArgs {
  const uint16_t* x;       // [T, H] bf16
  RouterRows wr;           // [E, H] router
  const uint16_t* lbias;   // [E] bf16 or null
  RouterRows wsg;          // [1, H] shared-expert gate (wsg.w null: none)
  int T, H, E, k, norm;
  int f16;                 // 1: x, the rows, logits, probabilities and scores in float16
  uint16_t* logits;        // [T, E+1] bf16 scratch (column E: shared gate logit)
  uint16_t* probs;         // [T, E] bf16 or null
  uint32_t* inds;          // [T, k]
  uint16_t* scores;        // [T, k] bf16
  float* sgate;            // [T] sigmoid(shared gate logit) (bf16 value) or null
  uint16_t* xp;            // [T, H] P8 copy of x or null
  uint16_t* xh;            // [T, H] fp16 copy of x in P8 layout (topk_kernel) or null
  uint32_t* f16_flag;      // zeroed by logits_kernel; topk_kernel ORs in kF16FlagX (or null)
  // launch_router_many: logits_kernel splits H into lg_split slices (1..4)
  // and, with more than one, writes fp64 partial sums lg_part[slice][t][c]
  // that topk_kernel adds in slice order and rounds (router_lg_split)
  double* lg_part;
  int lg_split;
  uint32_t* counters;      // [n_tt + 1], zero on entry, zero on exit
  int n_tt, n_ct;          // token tiles, column tiles (4 * cols_per_wave columns each)
  int cols_per_wave;       // 1 (one token tile: decode) or 4 (prefill)
  int fuse_sort;           // last workgroup sorts inds (needs router_sort_fits)
  SortOut sort;
  // topk_kernel's selection: 0 = softmax (probs, scores bf16); 1 = the
  // Nemotron-H router: sigmoid, correction bias, group limit, fp32 scores
  int mode;
  int n_group, topk_group; // groups of E / n_group experts; groups kept
  float scaling;           // routed_scaling_factor
  const float* cbias;      // [E] correction bias or null
  float* scores32;         // [T, k] fp32 scores (mode 1)
};
bool router_sort_fits(int64_t n, int64_t E);
hipError_t launch_router(const RouterArgs& a, hipStream_t stream);
// Forwards of more than kRouterManyMin tokens: logits on fp64 MFMA tiles,
// then softmax/top-k per token, in two launches (no xp copy, no sort).
constexpr int kRouterManyMin = 16;
constexpr int64_t kLgPartMax = 262144;  // doubles of lg_part
// H slices of logits_kernel for T tokens and E experts: about 1024
// workgroups, at most 4, with lg_split * T * (E + 1) <= min(kLgPartMax, cap)
int router_lg_split(int64_t T, int64_t E, int64_t cap);
hipError_t launch_router_many(const RouterArgs& a, hipStream_t stream);

// ---------------------------------------------------------------- grouped GEMM
// One problem: rows grouped in segments that share one expert's packed
// weights. out[row] = x[row_map[row]] . deq(W[e])^T  (or SwiGLU of two).
struct QGemmProblem {
  const uint16_t* x;        // activation rows in P8 layout
  int64_t ldx;              // elements between x rows
  const uint32_t* row_map;  // sorted row -> x row (null: identity)
  const uint32_t* out_map;  // sorted row -> out row (null: identity)
  const uint32_t* seg_n;    // device segment count (null: 1 static segment)
  const uint32_t* seg_exp;  // device expert per segment (null: expert 0)
  const uint32_t* seg_off;  // device [n+1] row offsets (null: [0, rows_static))
  int rows_static;
  int max_seg;              // segments the grid covers
  const uint32_t* w0; const uint16_t* s0; const uint16_t* b0;  // gate (or the matrix)
  const uint32_t* w1; const uint16_t* s1; const uint16_t* b1;  // up (dual only)
  int64_t ew, es;           // per-expert strides: u32 words, bf16 elements
  int N, K;
  uint16_t* out;
  int64_t ldo;
  int dual;                 // out = swiglu(x.W0^T, x.W1^T)
  int out_p8;               // write out rows in P8 layout (needs N % 8 == 0)
  int n_tiles;              // output tiles of 32 rows (set by launch_qgemm)
  // bounds the device-side tables are clamped to, so that stale or invalid
  // routing state can never address memory outside the arrays
  int n_exp;                // experts in w (seg_exp values clamp to n_exp-1)
  int rows_max;             // sorted rows (seg_off values clamp to it)
  int x_rows;               // rows of x (row_map values clamp to x_rows-1)
  int out_rows;             // rows of out (out_map values clamp to out_rows-1)
  // split-K over workgroups: ksplit > 1 writes fp32 partial sums of each K
  // slice to out_part[ks][out_rows][N] (not with dual) instead of `out`
  int ksplit;
  float* out_part;
  // activation rows are staged in LDS in passes of rows_per_pass rows (set
  // by launch_qgemm from max_rows_per_seg, the most rows a segment can hold)
  int max_rows_per_seg;
  int rows_per_pass;
  // x rows in natural order (permuted to P8 while staged)
  int x_natural;
};
// Launch one or two independent problems in one grid (p1 may be null).
hipError_t launch_qgemm(const QGemmProblem& p0, const QGemmProblem* p1, hipStream_t stream);

// ---------------------------------------------------------------- decode (T <= 16)
// The MoE block for decode batches on packed weights (fmx_decode.hip):
// K1 router + shared gate/up, K2 routed gate/up, K3 down projections and
// the combine; a whole forward runs K2 and K3 as one grid (K23).
constexpr int kDecMaxT = 16;            // tokens
constexpr int kDecMaxK = 16;            // top-k
constexpr int kDecMaxE = 256;           // experts
constexpr int kDecThreads = 256;        // K1, K2 workgroups
constexpr int kDecSdSplit = 4;          // K slices of the shared expert's down projection
constexpr int kDecMaxColBlocks = 32;    // 64-column blocks of H (K3 arrival counters)
// K3 arrival counters sit kDecCbStride words (256 bytes) apart: device-scope
// atomics on one line are served one at a time
constexpr int kDecCbStride = 64;
// K23 per routed expert: the gate/up tiles' arrival counter, then
// kDecGuFlags copies of a done flag that the last tile sets (the down
// workgroups poll the copies, spread over separate lines, and never the line
// the tiles count on); each on its own kDecCbStride-word line
constexpr int kDecGuFlags = 4;
constexpr int kDecGuWords = (1 + kDecGuFlags) * kDecCbStride;
constexpr int kPackedBlockSingle = 1152;  // bytes of one (16-row tile, 128-k unit) block
constexpr int kPackedBlockPair = 2304;    // gate + up

struct DecodeArgs {
  int T, H, E, k, I, Is, norm;
  int f16;                  // 1: x, y, the router rows and every scale and bias are
                            //   float16, and the block rounds in fp16 throughout
  const uint16_t* x;        // [T, H] bf16
  RouterRows wr;            // [E, H] router
  const uint16_t* lbias;    // [E] bf16 router logit bias or null
  RouterRows wsg;           // [1, H] shared-expert gate row (wsg.w null when Is == 0)
  const uint8_t* gu;        // packed gate/up pairs of the routed experts
  int64_t gu_es;            //   bytes per expert
  const uint8_t* dn;        // packed down projections of the routed experts
  int64_t dn_es;
  const uint8_t* sgu;       // packed shared gate/up pair
  const uint8_t* sdn;       // packed shared down
  uint16_t* logits;         // [T, E+1] bf16 (column E: shared gate logit)
  uint16_t* hs;             // [T, Is] shared SwiGLU output
  uint16_t* h;              // [T*k, I] routed SwiGLU output, entry order
  uint32_t* dw;             // [T*k, H] routed down projections, entry order, bf16 in the
                            //   low halves (written and read with device-scope accesses)
  float* sd_part;           // [kDecSdSplit, T, H] shared down projection, fp32 K-slice sums
  uint32_t* inds;           // [T, k]
  uint16_t* scores;         // [T, k] bf16
  uint16_t* probs;          // [T, E] bf16 or null
  float* sgate;             // [T] bf16-valued sigmoid of the shared gate logit, or null
  SortOut sort;             // order/inv/src/idx/offsets (+ base scratch)
  uint32_t* seg;            // [1 + max_seg]: U, then the routed experts ascending
  uint8_t* slots;           // [max_seg][16]: slot of token t for routed expert u, or 0xff
  uint32_t* counter;        // router arrival counter: zero on entry, zero on exit
  // K1's logit handoff: column c stores (epoch << 32) | logit of token t in
  // lgx[c * T + t]; router column 0 accepts words of the current epoch only
  // and advances the epoch once it has them all
  uint64_t* lgx;            // [kDecMaxT * (kDecMaxE + 1)]
  uint32_t* epoch;
  uint32_t* cb_counter;     // [H / 64, stride kDecCbStride] K3 arrivals per column block: zero on entry and exit
  uint32_t* gu_counter;     // [max_seg][kDecGuWords] K23: gate/up tiles finished per routed expert
                            //   and their done flags; K1 zeroes them for every forward
  uint16_t* y;              // [T, H] bf16
  // status word (sticky: set bits stay until the caller clears them):
  // kStatusWaitTimeout when a down workgroup's bounded wait for its expert's
  // gate/up tiles ran out (its products are then NaN), or router column 0's
  // wait for the other columns' logits (missing logits then read as 0)
  uint32_t* status;
  int wait_polls;           // the waits' bound in flag reads; <= 0 gives up at once
  // launch shape (decode_plan)
  int n_rt, n_sgu;          // K1: router columns, shared gate/up tile pairs (one each per workgroup)
  int max_seg, gu_tiles;    // K2: expert slots x gate/up tile pairs
  int k2_pairs, gu_wgs;     // K2: tile pairs per workgroup, workgroups per expert slot
  // input norm in K1 (nin non-null, T <= kDecNinMaxT): every K1 workgroup
  // forms x = rmsnorm(nin) * nin_w in LDS itself (rmsnorm_kernel's bits),
  // and router column 0 writes it to x_out (= x, read by K23)
  const uint16_t* nin;
  const uint16_t* nin_w;
  float nin_eps;
  uint16_t* x_out;
};
constexpr uint32_t kStatusWaitTimeout = 1u;
// rows K1 normalises itself: every workgroup forms every row's norm, which
// at 4 and 8 rows costs more than the norm kernel (stack decode step 1678 ->
// 1825 us at batch 4, 1970 -> 2402 us at batch 8)
constexpr int kDecNinMaxT = 1;
// default bound of the down workgroups' wait (flag reads, s_sleep 16 apart):
// far beyond any real wait, a guard against a hang
constexpr int kDecWaitPolls = 1 << 21;
// Fills the launch shape; false when the shapes are outside the decode path.
bool decode_plan(DecodeArgs& a);
hipError_t launch_decode_k1(const DecodeArgs& a, hipStream_t stream);
hipError_t launch_decode_k2(const DecodeArgs& a, hipStream_t stream);
hipError_t launch_decode_k23(const DecodeArgs& a, hipStream_t stream);

// ---------------------------------------------------------------- prefill (T > 16)
// The expert GEMMs of the MoE block for prefill on packed weights
// (fmx_prefill.hip): one grid for gate/up + SwiGLU, one for down, each over
// the routed experts' passes and the shared expert's.
struct PfSet {
  const uint8_t* w;          // packed blocks of expert 0 (pairs for gate/up)
  int64_t es;                // bytes per expert
  const uint16_t* x;         // activation rows, bf16
  const uint16_t* xh;        // the same rows in fp16, P8 layout
  int64_t ldx;               // elements between rows (both copies)
  const uint32_t* row_map;   // pass row -> x row (null: identity)
  uint16_t* out;             // output rows (indexed like the pass rows), bf16
  uint16_t* outh;            // gate/up: the same rows in fp16, P8 layout
  int64_t ldo;
  // single-matrix sets only (both nullable): out = bf16(bf16(x.W^T) + bias[col]),
  // then out = bf16(res[row] + out) (a residual add; res may alias out)
  const uint16_t* bias;
  const uint16_t* res;
  int64_t ldr;
  // single-matrix sets: act = 1 writes relu(bf16(x.W^T))^2 (fp32, exact)
  // rounded to bf16 into out and to fp16 (P8 layout) into outh, and ORs
  // flag_out into the flag when a value is outside fp16's range; out32
  // (non-null) takes the fp32 products unrounded instead of out
  int act;
  float* out32;
  // static sets with out32 only: ksplit > 1 cuts K into that many slices of
  // whole units, one work item each; slice ks writes its fp32 sums to
  // out32 + ks * part_stride
  int ksplit;
  int64_t part_stride;
  // single matrices in the MLX layout instead of w (mw set): mw [n_exp][nt*16]
  // [K/8] u32, ms / mb [n_exp][nt*16][K/64] bf16 scales / biases; then x is
  // the rows in the P8 layout (bf16) and xh in the Q8 layout (fp16), the
  // orders in which an MLX word's nibbles convert. out_map (nullable): pass
  // row r is written to output row out_map[r]
  const uint32_t* mw;
  const uint16_t* ms;
  const uint16_t* mb;
  const uint32_t* out_map;
  int io_f16;                // scales, biases and out in float16 (not bf16): MLX sets of
                             //   an fp16 x, and every set of a float16 MoE block (gate/up
                             //   then writes fp16 SwiGLU rows, the exact path is never taken)
  int nt;                    // 16-row tiles of the weight matrix (pairs: of gate)
  int nu;                    // 128-k units of K
  int ng;                    // column groups (kPfWaves * blocks per wave tiles each)
  const uint32_t* pass_n;    // device pass count (null: static passes over rows_static)
  const uint32_t* pass_tab;  // [max_pass][2] (see SortOut)
  int max_pass;              // passes the grid covers
  int rows_static;           // rows of the static passes
  int pass_rows;             // static passes: rows per pass (0: kPassRows; at most kPassRows)
  int n_exp;                 // experts in w (table values clamp to n_exp - 1)
  int rows_max;              // pass rows (table rows clamp to it)
  int x_rows;                // rows of x (row_map values clamp to x_rows - 1)
};
struct PfArgs {
  PfSet s0, s1;              // work items [0, n_items0) serve s0, the rest s1
  int n_items0, n_items1;
  // f16_flag & flag_in set: an input row holds a value outside fp16's range,
  // so the grid multiplies the bf16 rows exactly; gate/up ORs flag_out into
  // it when one of its outputs does. n_flag > 1: the input test ORs the
  // n_flag (at most 256, 16-byte aligned) words at f16_flag (per-block
  // words of a copy kernel; each wave reads them all, which costs a grid
  // of many work items more than one word does)
  uint32_t* f16_flag;
  uint32_t flag_in, flag_out;
  int n_flag;
};
constexpr uint32_t kF16FlagX = 1u;  // x (gate/up input)
constexpr uint32_t kF16FlagH = 2u;  // h (down input)
// Fills ng / max_pass of a set; items of it.
int pf_items(PfSet& s, bool dual);
size_t pf_lds_bytes(bool dual);
hipError_t launch_pf(const PfArgs& a, bool dual, hipStream_t stream);

struct PackArgs {
  const uint32_t* w0; const uint16_t* s0; const uint16_t* b0;  // MLX layout [n_exp][N][..]
  const uint32_t* w1; const uint16_t* s1; const uint16_t* b1;  // second matrix of a pair or null
  int64_t n_exp;
  int N, nt, nu;            // N: source rows per expert; nt * 16 >= N packed rows
  int k_src;                // source K (0: nu * 128); groups past it pack as zeros
  uint8_t* dst;
  int64_t dst_estride;      // bytes per expert in dst
};
hipError_t launch_pack(const PackArgs& a, hipStream_t stream);

// ---------------------------------------------------------------- elementwise
struct CombineArgs {
  const uint16_t* d;       // [T*k, H] bf16, sorted rows
  const uint32_t* inv;     // [T*k] entry -> sorted row
  const uint16_t* scores;  // [T, k] bf16
  const uint16_t* sd;      // [T, H] bf16 shared-expert output or null
  const float* sd_part;    // or [sd_ksplit, T, H] fp32 partial sums of it (added in order)
  int sd_ksplit;
  const float* sgate;      // [T] or null
  uint16_t* y;             // [T, H] bf16
  int T, k, H;
  int f16;                 // d, scores, sd and y float16, every rounding to fp16
};
hipError_t launch_combine(const CombineArgs& a, hipStream_t stream);

// The Nemotron-H block for decode batches (T <= 16) on packed weights
// (fmx_nh_decode.hip): D1 router columns (+ the shared up tiles), D2 the
// routed fc1 tiles, D3 fc2 and the shared down, D4 the combine.
constexpr int kNhDecMaxE = 512;       // experts (the router tables in LDS)
constexpr int kNhDecSdSplit = 4;      // K slices of the shared down projection
struct NhDecArgs {
  int T, H, E, k, norm, n_group, topk_group;
  float scaling;
  int Ip, Isp;                 // I and Is padded to whole 128-k units
  const uint16_t* x;           // [T, H] bf16
  const uint16_t* gate_w;      // [E, H] bf16 router
  const float* cbias;          // [E] or null
  const uint8_t* fc1;          // packed [E][Ip/16 tiles][H/128 units]
  int64_t fc1_es;
  const uint8_t* fc2;          // packed [E][H/16 tiles][Ip/128 units]
  int64_t fc2_es;
  const uint8_t* sup;          // packed [Isp/16][H/128]
  const uint8_t* sdn;          // packed [H/16][Isp/128]
  uint16_t* logits;            // [T, E + 1] bf16 (the routing accessor's view)
  uint32_t* lgw;               // [E][T] the logits between D1 workgroups (low halves)
  uint32_t* inds;              // [T, k]
  float* scores;               // [T, k] fp32
  uint32_t* seg;               // [1 + max_seg]: U, then the selected experts ascending
  uint8_t* slots;              // [max_seg][16]: token t's slot for expert u, or 0xff
  uint16_t *h_hi, *h_lo;       // [T*k, Ip] relu^2 of fc1 as hi + lo bf16 (exact sum)
  uint16_t *hs_hi, *hs_lo;     // [T, Isp] the shared expert's
  float* d;                    // [T*k, H] fc2 products, entry order (first K half)
  float* d2;                   // [T*k, H] the same over the second K half
  float* sd_part;              // [kNhDecSdSplit][T][H] shared down, K-slice sums
  uint16_t* y;                 // [T, H]
  uint32_t* counter;           // D1 arrival counter: zero on entry and exit
  uint32_t* cb_counter;        // [H / 64, stride kDecCbStride] D3 arrivals per column block: zero on entry and exit
  int max_seg, n_sup;          // launch shape: expert slots, shared up tiles
};
constexpr int kNhDecMaxColBlocks = 64;  // 64-column blocks of H (D3 arrival counters)
bool nh_decode_plan(NhDecArgs& a);
hipError_t launch_nh_decode(const NhDecArgs& a, hipStream_t stream, void* const* marks, int n_stages = 4);

// The Nemotron-H combine: y = bf16(bf16(sum over slots, fp32 in slot order,
// of d * score) + sd) (the add in fp32; sd null: no shared expert).
struct NhCombineArgs {
  const float* d;          // [T*k, H] fp32, sorted rows
  const uint32_t* inv;     // [T*k] entry -> sorted row
  const float* scores;     // [T, k] fp32
  const float* sd;         // [T, H] fp32 shared-expert output or null
  uint16_t* y;             // [T, H] bf16
  int T, k, H;
  uint32_t* clear;         // a word set to zero (the forward's fp16-range flag) or null
};
hipError_t launch_nh_combine(const NhCombineArgs& a, hipStream_t stream);

hipError_t launch_permute_p8(const uint16_t* x, int64_t rows, int64_t K, uint16_t* xp,
                             hipStream_t stream);
hipError_t launch_fill_u32(uint32_t* p, int64_t n, uint32_t v, hipStream_t stream);
// dst[i] = bf16 bits of src[i], a value that is exactly a bf16 (f16: fp16
// bits of an fp16 value)
hipError_t launch_f32_bf16(const float* src, int64_t n, uint16_t* dst, hipStream_t stream, bool f16 = false);

// MLX broadcasting of index arrays to the common batch shape (up to 8 dims).
struct BcastArgs {
  const void* src; int is_i32;  // null: arange over the flattened batch
  int ndim;
  int64_t out_shape[8];
  int64_t src_stride[8];        // 0 on broadcast dims
  int64_t n;
  uint32_t* dst;
  // M > 1: also emit the per-row key expansion: dst_rows[b*M + m] = dst[b]
  int M;
  uint32_t* dst_rows;           // nullable
};

// The standalone ops' first launch: gather_qmm's index broadcasts (lhs, and
// rhs with its per-row key expansion; n == 0: none) and the two operand
// copies of the rows for the prefill GEMM on MLX-layout weights (xp: bf16 in
// the P8 layout, xq: fp16 in the Q8 layout, fmx_dev.hpp; n_oct == 0: none).
// Copy block c writes ovf[c] = 1 when its rows hold a value outside fp16's
// range, else 0: every word is written on every call, none needs clearing.
struct OpsPrologue {
  BcastArgs lhs, rhs;
  const uint16_t* x;
  int x_f16;      // x in float16: xq is x in the Q8 order, xp unused, ovf words 0
  int64_t n_oct;  // 8-element chunks of x
  uint16_t* xp;
  uint16_t* xq;
  uint32_t* ovf;  // [ops_prologue_ovf_words(n_oct)]
};
constexpr int kOvfBlocks = 256;  // most copy blocks (ovf words)
int ops_prologue_ovf_words(int64_t n_oct);
hipError_t launch_ops_prologue(const OpsPrologue& a, hipStream_t stream);

// ---------------------------------------------------------------- quantization
hipError_t launch_quantize(const uint16_t* w, int64_t n_groups, uint32_t* wq, uint16_t* s,
                           uint16_t* b, hipStream_t stream);
hipError_t launch_dequantize(const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                             int64_t n_groups, uint16_t* out, hipStream_t stream);

// ---------------------------------------------------------------- stack hook
// The MoE block forward on the rows x = rmsnorm(h) * w (the decoder stack's
// post-attention norm), for forwards the decode kernels take with at most
// kDecNinMaxT tokens: K1 forms the rows itself and writes them to x_out.
// Other forwards return FMX_ERR_UNSUPPORTED before launching anything (the
// caller then runs the norm kernel and fmx_moe_block_forward).
struct MoEInputNorm {
  const uint16_t* h;
  const uint16_t* w;
  float eps;
};

}  // namespace fmx

namespace fmx {
int moe_block_forward_nin(const ::fmx_moe_config* cfg, const ::fmx_moe_weights* w, const MoEInputNorm& nin,
                          void* x_out, int64_t T, void* y, void* workspace, size_t workspace_bytes,
                          hipStream_t stream);
}  // namespace fmx
