// Internal launch interface between the C-ABI entry points (uocr_moe.cpp) and
// the kernel translation units.  Not part of the public header.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace uocr {

// Kernel timing for benchmarks: while uocr_moe_timing_begin() is in effect,
// timing_slot() hands out a start/stop event pair per launch (until the
// capacity runs out) and the launch records them around the kernel.
bool timing_slot(const char* name, hipEvent_t* start, hipEvent_t* stop);

#define UOCR_LAUNCH(name, kernel, grid, block, shmem, stream, ...)                                   \
  do {                                                                                               \
    hipEvent_t uocr_t0_ = nullptr, uocr_t1_ = nullptr;                                               \
    if (::uocr::timing_slot(name, &uocr_t0_, &uocr_t1_))                                             \
      hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, uocr_t0_, uocr_t1_, 0, __VA_ARGS__); \
    else                                                                                             \
      hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                           \
  } while (0)

// Elements per chunk of the bf16 chains (the int8 chains use the quant group).
constexpr int kChunk = 128;

enum WKind : int {
  kInt8Rows = 0,      // routed int8 stack [E, N, K] + fp32 scales [E, N, K/G]
  kBf16Rows = 1,      // routed bf16 stack [E, N, K]
  kBf16KBlocked = 2,  // dense bf16 weight K-blocked [K/16, N, 16]
};

struct Proj {
  const void* w;
  const float* s;
};

// Rows grouped by the expert they read.  n_groups == nullptr means one group
// of `identity` rows 0..identity-1 reading expert 0 (a dense weight).
struct Rows {
  const int32_t* n_groups;
  const int32_t* group_expert;
  const int32_t* group_start;
  const int32_t* group_rows;
  int identity;
};

struct GemvArgs {
  float* out;
  int64_t ldo;
  const float* x;
  int64_t ldx;
  int x_div;  // activation row of output row r is r / x_div
  Proj p[2];
  WKind kind;
  int E, N, K;
  int gsize;    // int8: quant group size; bf16: 128
  int nchunks;  // K / gsize (int8) or ceil(K / 128) (bf16)
  int vec;      // 16-byte weight loads allowed
  int batch;    // chunks per LDS batch (<= kGemvMaxBatch / nproj * 2)
  Rows rows;
};

// Waves per GEMV workgroup are at most 10 (640 threads: 168 VGPRs a lane);
// an LDS batch holds up to 16 chunks x 2 projections x 8 rows of partials.
constexpr int kGemvMaxWaves = 10;
constexpr int kGemvMaxThreads = kGemvMaxWaves * 64;
constexpr int kGemvMaxBatch = 16;

// dense_bf16_qmv: below kDenseNarrowMaxN output columns and for at most
// kDenseNarrowMaxRows rows, a (column, chunk) lane mapping (8 columns a
// workgroup, the same bits); else launch_gemv.
constexpr int kDenseNarrowMaxN = 16384;
constexpr int kDenseNarrowMaxRows = 2;
hipError_t launch_dense(const GemvArgs& a, int waves, hipStream_t s);
// The same narrow projection of rmsnorm(x + residual) * gamma (x + residual
// written to x_out when residual is given), normed in LDS with the order of
// the standalone RMSNorm kernel: at most kDenseNarrowMaxRows rows, K <= 2048.
hipError_t launch_norm_dense(const GemvArgs& a, const float* residual, float* x_out, const float* gamma, float eps,
                             hipStream_t s);
int gemv_workgroups(const GemvArgs& a, int max_groups);
size_t gemv_lds_bytes(int batch, int nproj);
hipError_t launch_gemv(const GemvArgs& a, int max_groups, int nproj, int waves, hipStream_t s);
hipError_t launch_gemv_pair(const GemvArgs& routed, int max_groups, const GemvArgs& shared, int nproj,
                            int waves, hipStream_t s);

// ---- routing (route.hip) ----

// logits[t*E + e] = dot(x[t], router[e]) in the 64-lane tree order; xb (may
// be null) receives x rounded to bf16, [T][H] (needs H % 64 == 0, H <= 2048).
// zero (may be null): nzero words the launch clears for a later kernel.
hipError_t launch_logits(float* logits, const float* x, int64_t ldx, const float* router, int T, int E,
                         int H, uint16_t* xb, hipStream_t s, int32_t* zero = nullptr, int nzero = 0);
// Softmax + top-k per token (one wave per token).  ids32/ids64/wts may be null.
hipError_t launch_softmax_topk(const float* logits, int T, int E, int topk, int renorm, int32_t* ids32,
                               int64_t* ids64, float* wts, hipStream_t s);

struct GroupTables {
  int32_t* n_groups;      // [1]
  int32_t* group_expert;  // [E]
  int32_t* group_start;   // [E + 1]
  int32_t* group_rows;    // [R]
  int32_t* tile_start;    // [E + 1] prefix of ceil(count / bm), may be null
  int32_t* inv;           // [R] position of row r in group_rows, may be null
};
// Groups R rows by their clamped expert id (ascending expert).
hipError_t launch_group(const int32_t* ids, int R, int E, int bm, const GroupTables& g, hipStream_t s);
// Prefill routing over many workgroups (E <= 64): softmax + top-k of T
// tokens and their rows per expert in 16-token blocks, then the grouping of
// their T*topk rows.  `hist` holds route_count_blocks(T) * E ints of scratch.
constexpr int kRouteMaxExperts = 64;  // a lane per expert in the top-k
int route_count_blocks(int T);
hipError_t launch_topk_group(const float* logits, int T, int E, int topk, int renorm, int32_t* ids32, float* wts,
                             int bm, const GroupTables& g, int32_t* hist, hipStream_t s);
// Prefill routing for T < 2048 (E <= 64): logits, softmax + top-k and
// per-workgroup counts in one launch (xb as launch_logits), then the
// grouping.  hist holds fused_route_blocks(T) * E ints of scratch.
int fused_route_blocks(int T);
hipError_t launch_logits_topk_group(float* logits, uint16_t* xb, const float* x, int64_t ldx, const float* router,
                                    int T, int E, int H, int topk, int renorm, int32_t* ids32, float* wts, int bm,
                                    const GroupTables& g, int32_t* hist, hipStream_t s);
// Decode-size routing in one workgroup: softmax + top-k of T <= 64 tokens, then
// the grouping of their T*topk rows.
hipError_t launch_route_small(const float* logits, int T, int E, int topk, int renorm, int32_t* ids32,
                              float* wts, const GroupTables& g, hipStream_t s);

// out[t, n] = fma-chain over j of wts[t*k+j] * y[row(t*k+j), n] from 0, then
// + shared[r][t, n] for r < shared_parts in turn (parts T x H floats apart).
// row(i) = inv ? inv[i] : i.  shared may be null.
hipError_t launch_combine(float* out, const float* y, int64_t ldy, const float* wts, const int32_t* inv,
                          const float* shared, int T, int H, int topk, hipStream_t s, int shared_parts = 1);

// ---- int8 dequantisation and the prefill grouped GEMM (gemm.hip) ----

// q int8 [groups_total * group], scales fp32 [groups_total] from w fp32 or bf16 bits.
hipError_t launch_quantize(int8_t* q, float* scales, const void* w, int w_bf16, int64_t groups_total, int group,
                           hipStream_t s);
hipError_t launch_dequant(void* out, int out_f32, const int8_t* w, const float* scales, const int32_t* idx,
                          int E, int N, int K, int groups, int vec, hipStream_t s);

struct GemmProblem {
  // A operand: bf16 rows [.., K] at a + row * lda; with grouped rows and
  // a_by_token, row = group_rows[position] / x_div (gate/up: x rows), else
  // row = position (down: h, already in group order; dense: the token).
  const uint16_t* a;
  int64_t lda;
  int a_by_token;
  int x_div;
  // B operand(s)
  Proj p[2];
  WKind kind;
  int N, K, groups;
  // rows
  Rows rows;
  const int32_t* tile_start;  // [max_groups + 1] m-tile prefix (routed), null for dense
  int max_groups;
  int M;                      // dense rows (identity); routed: the rows of all groups (bounds the tiles)
  // output
  int swiglu;                 // 1: out is bf16 silu(g)*u, row = position; 0: fp32
  uint16_t* outb;
  float* outf;
  int64_t ldo;
  int out_by_position;        // 1: output row = position in group order, 0: row id
  // A dense K-blocked problem (the shared one) in kparts > 1 K ranges of
  // K / kparts: each range's sums are computed from zero and stored at
  // outf + r * part_stride, the caller adds them (both kernels cut K the
  // same way, so they give the same bits)
  int kparts;
  int64_t part_stride;
};
// bm: rows per tile, 64 or 128.  vec: every weight pointer is 16-byte
// aligned; else the weights are read at any alignment (bm must be 64), with
// the same bits.  N must be a multiple of 32 and K of 128 (and of the int8
// group, itself a multiple of 64); a routed problem has at most 64 groups.
hipError_t launch_gemm_pair(const GemmProblem& routed, const GemmProblem& shared, int bm, hipStream_t s,
                            bool vec = true);
// The K ranges to cut the shared problem into for this pair (1 or 2).
int gemm_shared_parts(const GemmProblem& routed, const GemmProblem& shared);

// ---- the n-gram logit guard (ngram.hip) ----

constexpr int kNgramMaxHistory = 8192;
// result [rows, vocab] = logits with every banned id set to BLOCKED; history
// [rows, hist_len] int32, ngram int32 [1] (device).  result may alias logits.
hipError_t launch_ngram_block(float* result, const float* logits, int64_t rows, int64_t vocab,
                              const int32_t* history, int hist_len, const int32_t* ngram, hipStream_t s);

// ---- the decoder layer's per-row steps (decoder.hip) ----

// out = rmsnorm(x + delta) * gamma per row of `dim`; x + delta is written to
// x_out (may be x).  delta null: out = rmsnorm(x) * gamma, x_out unused.
hipError_t launch_add_rmsnorm(float* out, float* x_out, const float* x, const float* delta, const float* gamma,
                              int64_t rows, int dim, float eps, hipStream_t s);
// rotate_half RoPE of q and k [rows, heads, head_dim] (k may be null) at each
// row's position, and a copy of v (may be null); input rows are in_stride
// floats apart, outputs packed; an output may alias its input when packed.
hipError_t launch_rope(float* q_out, float* k_out, float* v_out, const float* q, const float* k, const float* v,
                       int64_t rows, int heads, int head_dim, int64_t in_stride, const int32_t* positions,
                       const float* cos_t, const float* sin_t, int table_rows, hipStream_t s);
// out [rows, ffn] = silu(gate_up[:, :ffn]) * gate_up[:, ffn:].
hipError_t launch_swiglu(float* out, const float* gate_up, int64_t rows, int ffn, hipStream_t s);

// ---- paged decode attention (attention.hip) ----

constexpr int kAttnSplitRows = 128;  // logical rows per partial workgroup (the page size is a multiple)
struct PagedAttention {
  float* out;            // [rows, heads, D]
  const float* q;        // [rows, heads, D] post-RoPE
  const float* k_new;    // [rows, heads, D] post-RoPE
  const float* v_new;    // [rows, heads, D]
  float* kv_blocks;      // [pages, 2, layers, page_size, heads, D]
  int pages, layers, page_size, heads, head_dim, layer;
  const uint32_t* lookup;       // [rows, lookup_cols]
  int lookup_cols;
  const uint32_t* write_index;     // [rows]
  const uint32_t* attend_lengths;  // [rows], attend_len - 1 (the new row is one of attend_len)
  int max_attend;                  // the largest attend_len (host)
  int64_t rows;
  float scale;
  float* workspace;             // attn_workspace_bytes(rows, heads, max_attend)
  uint32_t* counters;           // rows * heads words, zero between calls, or null (a second launch merges)
  int64_t in_stride;            // floats between rows of q / k_new / v_new (0: heads * head_dim, packed)
  const int32_t* positions;     // null: q, k_new are post-RoPE; else rotated here at these positions
  const float* cos_table;       // [table_rows, head_dim]
  const float* sin_table;
  int table_rows;
};
size_t attn_workspace_bytes(int64_t rows, int heads, int max_attend);
hipError_t launch_paged_attention(const PagedAttention& p, hipStream_t s);

// ---- the persistent decode layer (decode.hip) ----

constexpr int kFusedWaves = 12;  // waves per workgroup, one workgroup per CU (168 VGPRs a lane)
constexpr int kFusedXPad = 132;  // floats per 128-element chunk of an LDS activation row
constexpr int kFusedCtlWords = 2368;      // control words per slot: error word, epoch copies, counters
constexpr int kFusedXcds = 8;              // XCDs of the device (workgroup b runs on XCD b % 8)
constexpr int kFusedLogitCopies = kFusedXcds;  // copies of the tagged logits, one per XCD
constexpr int kFusedRouterWaves = 4;       // router tasks per workgroup
#ifndef UOCR_EARLY_SHARED_ROWS
#define UOCR_EARLY_SHARED_ROWS 1
#endif
constexpr int kFusedEarlySharedRows = UOCR_EARLY_SHARED_ROWS;  // batches up to this size use early_shared, defer_down
constexpr int kFusedLogitCopyWords = 576;  // 64-bit words per copy (8 tokens x 64 experts, padded)

// Task layout, LDS and tagged-buffer sizes of one layer shape.
struct FusedLayout {
  int gh, gf, gfs;          // 128-element chunks of H, F, Fs
  int sub;                  // column blocks per routed task (int8 weights at larger batches: 2)
  int c_gu, c_dn;           // columns per routed gate/up and down block
  int per_e_gu, per_e_dn;   // routed tasks per selected expert
  int cb_fs, cb_h;          // 64-column blocks of Fs and H
  int n_sgu, n_sdn;         // shared chunk tasks
  int n_sfold, n_comb;      // per-token fold and combine tasks
  int lds_x, lds_act;       // LDS bytes: x rows, per-wave activation stage
  size_t lds_bytes;
  int max_tasks;
  // offsets (in 64-bit words) of the tagged buffers, sized for 8 tokens
  int64_t off_logits, off_h, off_y, off_hs, off_psgu, off_psdn, data_words;
};
// Routed int8 tasks take two column blocks from this many tokens on: a wave
// then waits for its weights once per two blocks (the int8 stage is half the
// bf16 one, so two fit the registers).
constexpr int kFusedSubRows = 4;
int fused_sub(bool int8, int B);
FusedLayout fused_layout(int B, int E, int H, int F, int Fs, int topk, int sub = 1);

// One layer's weights (the stacked layouts of uocr_moe_layer).
struct FusedLayerW {
  const float* router;
  const void* gate_w;
  const void* up_w;
  const void* down_w;
  const float* gate_s;
  const float* up_s;
  const float* down_s;
  const uint16_t* sh_gate;
  const uint16_t* sh_up;
  const uint16_t* sh_down;
};
constexpr int kFusedMaxLayers = 12;  // layers of one stacked launch

struct FusedArgs {
  int B, E, H, F, Fs, topk;
  int int8, renorm;
  // residual = 0: one layer, out = MoE(x) (n_layers = 1).  residual = 1: a
  // stack of n_layers chained through the residual stream, x_{l+1} = x_l +
  // MoE_l(x_l), out = x_n; layer l's tagged buffers at l * layer_words from
  // those below, x_{l+1} (l < n - 1) as tagged pairs [B][H] at xs_pairs + l * B * H.
  int residual;
  int n_layers;
  int64_t layer_words;
  uint64_t* xs_pairs;
  FusedLayerW w[kFusedMaxLayers];
  const float* x;
  float* out;
  int32_t* ids_out;  // optional routing outputs [B*topk]
  float* wts_out;
  // library-owned, zeroed when allocated: control words and tagged pairs
  uint32_t* ctl;
  uint64_t* logits;  // [kFusedLogitCopies][kFusedLogitCopyWords]: copy c, token t, expert e at c*576 + t*64 + e
  uint64_t* h;       // [B*topk][F]
  uint64_t* y;       // [B*topk][H]
  uint64_t* hs;      // [B][Fs]
  uint64_t* p_sgu;   // [Fs/64][2][H/128][B][64]
  uint64_t* p_sdn;   // [H/64][Fs/128][B][64]
  // layout (FusedLayout)
  int gh, gf, gfs, sub, c_gu, c_dn, per_e_gu, per_e_dn, cb_fs, cb_h, n_sgu, n_sdn, n_sfold, n_comb, lds_x, lds_act;
  float inv_gh, inv_gf;
  // the kernel's divisors d as m = ceil(2^32 / d) (0 for d = 1): x / d =
  // mulhi(x, m) exactly while x * d < 2^32 (task indices stay below 2^20,
  // element indices below 2^14, divisors below 2^12)
  uint32_t m_2gh, m_gh, m_gu, m_b, m_gfs, m_dn, m_h;
  // polls a wait may take before it fails (sets the error word, takes NaN)
  uint32_t spin_limit;
  int r_tok;  // tokens per router task
  int x_vec;  // x is 16-byte aligned
  // small batches: the shared fold and down tasks come before the routed
  // ones (their weights stream while the routing is computed), and a routed
  // down task issues its weights once its workgroup's routed gate/up weights
  // have landed (the gate/up weights, which the next step waits for, then
  // have the memory to themselves)
  int early_shared;
  int defer_down;
  // optional per-task phase timestamps (8 words per task), null when off;
  // per-workgroup words start at trace_wg; a stack's layer l has its records
  // trace_layer records (of 8 words) after layer 0's
  int64_t* trace;
  int64_t trace_wg;
  int64_t trace_layer;
};
hipError_t fused_grid(size_t lds_bytes, int* grid);
bool fused_trace_built();  // the kernel was compiled with its phase trace (UOCR_DECODE_TRACE=1)
hipError_t launch_decode_fused(const FusedArgs& a, int grid, size_t lds_bytes, hipStream_t s);
hipError_t launch_zero_words(uint32_t* p, int64_t n, hipStream_t s);
// flag[0] = 1 if the error word of the control words at ctl_a or ctl_b (either
// may be null) is set, else 0; stream-ordered, one tiny kernel.
hipError_t launch_error_status(uint32_t* flag, const uint32_t* ctl_a, const uint32_t* ctl_b, hipStream_t s);

}  // namespace uocr
