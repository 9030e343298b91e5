/*
 * uocr_moe -- the DeepSeek-V2 routed-expert MoE block of unlimited-ocr-max on
 * AMD Instinct MI355X (gfx950), behind a plain C ABI.
 *
 * Every entry point takes device pointers (HIP memory), the shapes of each
 * tensor as the reference's ops see them, a HIP stream (NULL = the null
 * stream) and an optional error buffer.  The work is enqueued on the stream
 * and the call returns without waiting.  Return value: 0 on success, nonzero
 * on a refused call, with the reference's message text ("<op>: <reason>")
 * copied into err (NUL-terminated, truncated to errlen).  Shape checks run on
 * the host before anything is enqueued; device-side the ops never fail:
 * out-of-range expert ids are clamped to [0, E).
 *
 * Tensors are row-major and packed.  bf16 tensors are passed as uint16_t bit
 * patterns.  The library keeps no pointer past the call.  Scratch memory for
 * the grouping tables and the layer intermediates comes from the `workspace`
 * argument when one is given (size: uocr_moe_workspace_bytes), else from a
 * buffer the library keeps per device and stream (grown on demand, so a call
 * under stream capture passes its own workspace).  A superseded library
 * buffer is kept until uocr_moe_release, so graphs captured with it stay valid.
 */
#ifndef UOCR_MOE_H
#define UOCR_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UOCR_MOE_ABI_VERSION 1

int uocr_moe_abi_version(void);

/* ---------------------------------------------------------------------------
 * The reference's custom ops (the MAX @register ops of the Mojo files in
 * unlimited_ocr_max/kernels/), one entry point each.
 * ------------------------------------------------------------------------- */

/* moe_int8_qmv -- replaces MoeInt8Qmv.execute
 * (unlimited_ocr_max/kernels/moe_int8.mojo:181-258; staged by
 * StackedExperts._qmv, unlimited_ocr_max/decoder.py:355-366).
 *   result fp32 [k, N], x fp32 [k, K], expert_ids int32 [k],
 *   w int8 [E, N, K], scales fp32 [E, N, K/G]
 *   result[s,n] = sum_g scales[e,n,g] * sum_{kk in g} f32(w[e,n,kk]) * x[s,kk],
 *   e = clamp(expert_ids[s]); bitwise the reference's operation order
 *   (a per-group fma chain in kk order, then fma(scale, gsum, acc) per group). */
int uocr_moe_int8_qmv(float* result, int64_t result_k, int64_t result_n,
                      const float* x, int64_t x_k, int64_t x_kdim,
                      const int32_t* expert_ids, int64_t ids_k,
                      const int8_t* w, int64_t w_e, int64_t w_n, int64_t w_kdim,
                      const float* scales, int64_t s_e, int64_t s_n, int64_t s_groups,
                      void* stream, char* err, size_t errlen);

/* moe_bf16_qmv -- replaces MoeBf16Qmv.execute
 * (unlimited_ocr_max/kernels/moe_bf16.mojo:264-345).
 *   result fp32 [k, N], x fp32 [k, K], expert_ids int32 [k], w bf16 [E, N, K]
 *   result[s,n] = sum_kk f32(w[e,n,kk]) * x[s,kk], fp32 accumulation in
 *   128-element chunks (fma chain per chunk, chunk sums added in order). */
int uocr_moe_bf16_qmv(float* result, int64_t result_k, int64_t result_n,
                      const float* x, int64_t x_k, int64_t x_kdim,
                      const int32_t* expert_ids, int64_t ids_k,
                      const uint16_t* w, int64_t w_e, int64_t w_n, int64_t w_kdim,
                      void* stream, char* err, size_t errlen);

/* int8_dequant_expert -- replaces Int8DequantExpert.execute
 * (unlimited_ocr_max/kernels/moe_int8.mojo:261-342; staged by
 * StackedExperts._dequant, unlimited_ocr_max/decoder.py:325-330).
 *   result [N, K] bf16 (result_f32 = 0) or fp32 (result_f32 = 1),
 *   w int8 [E, N, K], scales fp32 [E, N, K/G], expert_idx int32 [1] (device)
 *   result[n,kk] = round(f32(w[e,n,kk]) * scales[e,n,kk/G]), e = clamp(idx),
 *   bf16 by round-to-nearest-even. */
int uocr_int8_dequant_expert(void* result, int64_t result_n, int64_t result_kdim, int result_f32,
                             const int8_t* w, int64_t w_e, int64_t w_n, int64_t w_kdim,
                             const float* scales, int64_t s_e, int64_t s_n, int64_t s_groups,
                             const int32_t* expert_idx, int64_t idx_len,
                             void* stream, char* err, size_t errlen);

/* quantize_per_group -- replaces quantize_per_group (tools/quantize_int8.py:298-329;
 * the format of tools/quantize_int8.py:54-70), on the device.
 *   w fp32 (w_bf16 = 0) or bf16 bits (w_bf16 = 1) [rows, K] -> q int8 [rows, K],
 *   scales fp32 [rows, K/group]: per group of `group` elements along K,
 *   amax = max |w|, scale = amax / 127 (1.0 when amax == 0),
 *   q = clip(rint(w / scale), -127, 127), fp32 divisions correctly rounded and
 *   rint half to even (bitwise the reference's numpy arithmetic).  NaN or Inf
 *   in w is not detected here (the Python wrapper refuses it, as the
 *   reference's tool does). */
int uocr_quantize_per_group(int8_t* q, float* scales, const void* w, int w_bf16, int64_t rows, int64_t kdim,
                            int64_t group, void* stream, char* err, size_t errlen);

/* ngram_block -- replaces NgramBlock.execute
 * (unlimited_ocr_max/kernels/ngram_block.mojo:60-151; staged by apply_ngram_guard,
 * unlimited_ocr_max/ngram.py:33-53).
 *   result fp32 [rows, vocab], logits fp32 [rows, vocab], history int32 [rows, hist_len]
 *   (each row's last `window` ids, newest last), ngram int32 [1] (device).  A rank-1
 *   call is rows = 1.  Row b's id v is set to -3.0e38 when some n-gram of history
 *   row b ends in v and its first n-1 ids equal the row's last n-1 ids (n == 1: every
 *   id of the history); n < 1 or hist_len < n leaves the row unchanged.  result may
 *   be logits (in place).  hist_len <= 8192. */
int uocr_ngram_block(float* result, int64_t result_rows, int64_t result_vocab, const float* logits,
                     int64_t logits_rows, int64_t logits_vocab, const int32_t* history, int64_t hist_rows,
                     int64_t hist_len, const int32_t* ngram, int64_t ngram_len, void* stream, char* err,
                     size_t errlen);

/* paged_decode_attention -- replaces paged_decode_attention
 * (unlimited_ocr_max/decoder.py:425-437: store_k/v_cache_ragged at the write
 * index, then flash_attention_ragged under the causal mask; the pool and its
 * step metadata of unlimited_ocr_max/kv_cache.py:1-36 and :305-329).
 *   out, q, k_new, v_new fp32 [rows, heads, head_dim] (post-RoPE), head_dim 128;
 *   kv_blocks fp32 [pages, 2, layers, page_size, heads, head_dim], page_size a
 *   multiple of 128; lookup uint32 [rows, lookup_cols]; attend_lengths uint32
 *   [rows] = attend_len - 1; write_index uint32 [rows] (all device);
 *   attend_max (host) = the largest attend_len.  Logical row r of batch row b is
 *   slot r % page_size of page lookup[b, r / page_size].  Stores k_new / v_new
 *   at row write_index[b] of layer `layer`, then
 *   out[b,h] = sum_{r < attend_len} softmax_r(scale * q[b,h] . k_r) v_r,
 *   fp32 throughout.  Device metadata past what the lookup row addresses is
 *   clamped there (a write index past it stores nothing).  workspace may be
 *   NULL (the library's own) or at least
 *   uocr_paged_attention_workspace_bytes(rows, heads, attend_max) bytes,
 *   16-byte aligned.  Up to 65536 (row, head) pairs merge their splits inside
 *   the one launch, with per-device counters that the first call outside
 *   stream capture allocates; each stream takes one of 16 slots of them, and
 *   launches on streams that share a slot must not overlap in time. */
size_t uocr_paged_attention_workspace_bytes(int64_t rows, int64_t heads, int64_t attend_max);
int uocr_paged_decode_attention(float* out, const float* q, const float* k_new, const float* v_new,
                                int64_t rows, int64_t heads, int64_t head_dim,
                                float* kv_blocks, int64_t pages, int64_t layers, int64_t page_size,
                                int64_t layer, const uint32_t* lookup, int64_t lookup_cols,
                                const uint32_t* attend_lengths, int64_t attend_max,
                                const uint32_t* write_index, float scale, void* workspace,
                                size_t workspace_bytes, void* stream, char* err, size_t errlen);

/* paged_decode_attention_qkv -- Attention.decode's RoPE and paged_decode_attention
 * in one launch (unlimited_ocr_max/decoder.py:487-492 with :425-437): the same op
 * as uocr_paged_decode_attention, whose q / k_new / v_new are here the thirds of
 * one fused projection's output, qkv [rows, 3, heads, head_dim] with rows
 * row_stride floats apart, q and k_new before RoPE.  q and the new k row are
 * rotated in the kernel exactly as uocr_rope does (the stored k row and the
 * output have the bits of uocr_rope followed by uocr_paged_decode_attention);
 * positions int32 [rows], cos_table / sin_table fp32 [table_rows, head_dim]. */
int uocr_paged_decode_attention_qkv(float* out, const float* qkv, int64_t rows, int64_t heads, int64_t head_dim,
                                    int64_t row_stride, const int32_t* positions, const float* cos_table,
                                    const float* sin_table, int64_t table_rows, int64_t table_dim,
                                    float* kv_blocks, int64_t pages, int64_t layers, int64_t page_size,
                                    int64_t layer, const uint32_t* lookup, int64_t lookup_cols,
                                    const uint32_t* attend_lengths, int64_t attend_max,
                                    const uint32_t* write_index, float scale, void* workspace,
                                    size_t workspace_bytes, void* stream, char* err, size_t errlen);

/* rms_norm -- replaces RmsNorm.__call__ (unlimited_ocr_max/decoder.py:252-261,
 * ops.rms_norm with gamma cast to fp32) and, given `residual`, the residual add
 * before it (DecoderLayer.decode, decoder.py:702-709).
 *   x, residual, x_out, out fp32 [rows, dim]; gamma fp32 [dim].
 *   v = x + residual (written to x_out, which may be x) or v = x;
 *   out = (v * r) * gamma, r = 1 / sqrt(mean(v^2) + eps), fp32. */
int uocr_rms_norm(float* out, float* x_out, const float* x, const float* residual, const float* gamma,
                  int64_t rows, int64_t dim, float eps, void* stream, char* err, size_t errlen);

/* rms_norm_dense_bf16_qmv -- RmsNorm (with the residual add before it) and the
 * dense_bf16_qmv that consumes it in one launch, for decode rows
 * (DecoderLayer.decode's input_layernorm and q/k/v projections,
 * decoder.py:702-709 with :487-491; the ops of uocr_rms_norm and
 * uocr_dense_bf16_qmv, with their bits).
 *   x fp32 [M, K] (M <= 2, K <= 2048), residual fp32 [M, K] or NULL, x_out fp32
 *   [M, K] (x + residual; must not overlap x or residual), gamma fp32 [K],
 *   w bf16 K-blocked [K/16, N, 16] (N < 16384), result fp32 [M, N] =
 *   rmsnorm(x + residual) * gamma @ W^T. */
int uocr_rms_norm_dense_bf16_qmv(float* result, int64_t result_m, int64_t result_n, const float* x, int64_t x_m,
                                 int64_t x_kdim, const float* residual, float* x_out, const float* gamma, float eps,
                                 const uint16_t* w, int64_t w_blocks, int64_t w_n, int64_t w_kblock, void* stream,
                                 char* err, size_t errlen);

/* rope -- replaces Attention._rope over the decode rows (decoder.py:459-462,
 * 487-491) with rope_rows' gather (decoder.py:766-775).
 *   q, k, v: [rows, heads, head_dim] fp32 views whose rows are in_row_stride
 *   floats apart (e.g. the thirds of one fused q/k/v projection's output);
 *   k and v may be NULL.  q_out, k_out, v_out fp32 [rows, heads, head_dim],
 *   packed (an output may be its input when in_row_stride = heads * head_dim).
 *   positions int32 [rows]; cos_table, sin_table fp32 [table_rows, head_dim]
 *   (rope_tables, decoder.py:115-123), all device.
 *   q_out, k_out = x * cos[pos] + rotate_half(x) * sin[pos], rotate_half(x) =
 *   concat(-x[D/2:], x[:D/2]), both products and the sum rounded to fp32;
 *   v_out = v.  A position outside [0, table_rows) is clamped into it. */
int uocr_rope(float* q_out, float* k_out, float* v_out, const float* q, const float* k, const float* v,
              int64_t rows, int64_t heads, int64_t head_dim, int64_t in_row_stride, const int32_t* positions,
              const float* cos_table, const float* sin_table, int64_t table_rows, int64_t table_dim,
              void* stream, char* err, size_t errlen);

/* swiglu -- replaces ops.silu(gate) * up of GatedMlp.decode_rows
 * (decoder.py:274-276) over one gate+up projection's output.
 *   gate_up fp32 [rows, 2 * ffn] (gate columns, then up); out fp32 [rows, ffn];
 *   out = silu(gate) * up, silu(g) = g / (1 + exp(-g)), each step rounded to
 *   fp32 (the MoE kernels' silu). */
int uocr_swiglu(float* out, const float* gate_up, int64_t rows, int64_t ffn, void* stream, char* err,
                size_t errlen);

/* dense_bf16_qmv -- replaces DenseBf16Qmv.execute[tile]
 * (unlimited_ocr_max/kernels/dense_bf16.mojo:119-158; staged by
 * dense_bf16_qmv, unlimited_ocr_max/decoder.py:166-184).
 *   result fp32 [M, N], x fp32 [M, K], w bf16 K-blocked [K/16, N, 16]
 *   result[m,n] = sum_kk f32(W[n,kk]) * x[m,kk], W[n,kk] = w[kk/16, n, kk%16].
 *   `tile` (>= 1) is the reference's rows-per-read parameter; a row's bits
 *   do not depend on it. */
int uocr_dense_bf16_qmv(float* result, int64_t result_m, int64_t result_n,
                        const float* x, int64_t x_m, int64_t x_kdim,
                        const uint16_t* w, int64_t w_blocks, int64_t w_n, int64_t w_kblock,
                        int64_t tile, void* stream, char* err, size_t errlen);

/* ---------------------------------------------------------------------------
 * The MoE block.
 * ------------------------------------------------------------------------- */

/* One MoE layer's weights (unlimited_ocr_max/decoder.py:517-554, declared
 * names in StackedExperts.__init__, decoder.py:297-313):
 *   router             fp32 [E, H]                 gate.gate_score.weight
 *   gate_proj/up_proj  [E, F, H], down_proj [E, H, F]   experts.*
 *                      int8 (int8 = 1) or bf16 bits (int8 = 0)
 *   *_scales           fp32 [E, F, H/G], [E, F, H/G], [E, H, F/G] (int8 only)
 *   shared_*           bf16 bits, K-blocked: gate/up [H/16, Fs, 16],
 *                      down [Fs/16, H, 16]          shared_experts.*
 * E <= 64.  renormalize = 0 is the reference's gate (model_config.py:149-150);
 * 1 divides the top-k weights by their sum. */
typedef struct uocr_moe_layer {
  int64_t num_experts; /* E */
  int64_t hidden;      /* H */
  int64_t ffn;         /* F, moe_intermediate_size */
  int64_t shared_ffn;  /* Fs = n_shared_experts * F */
  int64_t top_k;
  int64_t group;       /* int8 group size along K (128) */
  int32_t int8;
  int32_t renormalize;
  const float* router;
  const void* gate_proj;
  const void* up_proj;
  const void* down_proj;
  const float* gate_proj_scales;
  const float* up_proj_scales;
  const float* down_proj_scales;
  const uint16_t* shared_gate;
  const uint16_t* shared_up;
  const uint16_t* shared_down;
} uocr_moe_layer;

/* Bytes of workspace the layer entries need for `rows` tokens
 * (prefill = 0: uocr_moe_decode_rows, 1: uocr_moe_forward). */
size_t uocr_moe_workspace_bytes(const uocr_moe_layer* layer, int64_t rows, int prefill);

/* MoEGate.__call__ -- replaces the gate of unlimited_ocr_max/decoder.py:509-514
 * (router matmul + ops.softmax + ops.top_k).
 *   indices int64 [T, k], weights fp32 [T, k] in score order, ties to the
 *   lower id; x fp32 [T, H], router fp32 [E, H], E <= 64. */
int uocr_moe_gate(int64_t* indices, float* weights, const float* x, int64_t seq, int64_t hidden,
                  const float* router, int64_t num_experts, int64_t top_k, int renormalize,
                  void* workspace, size_t workspace_bytes, void* stream, char* err, size_t errlen);

/* MoE.decode_rows -- replaces unlimited_ocr_max/decoder.py:641-655 (gate,
 * _routed_qmv through moe_int8_qmv / moe_bf16_qmv, SwiGLU, _mix, shared
 * experts through dense_bf16_qmv).  x fp32 [B, H] -> out fp32 [B, H], B <= 64.
 * Bitwise the CPU oracle's or_moe_decode_exact.  expert_ids / expert_weights
 * (device, [B, k], may be NULL) receive the routing. */
int uocr_moe_decode_rows(float* out, const float* x, int64_t rows, int64_t hidden,
                         const uocr_moe_layer* layer, int32_t* expert_ids, float* expert_weights,
                         void* workspace, size_t workspace_bytes, void* stream, char* err, size_t errlen);

/* uocr_moe_decode_rows_static -- uocr_moe_decode_rows without any allocation.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments, bits and routing outputs as
 * uocr_moe_decode_rows, minus the workspace: its scratch is one static 16 MiB
 * device array per GPU (9 MiB for the persistent kernel's control words and
 * tagged arena, 7 MiB of multi-kernel workspace), resolved and cleared by the
 * first call on each device and held until the process ends.  It calls no
 * hipMalloc or hipFree.  A call whose layer and row count need more than the
 * 7 MiB (only the multi-kernel path can: rows > 8, or a layer the persistent
 * kernel does not take) is refused before anything is enqueued.  Every call on
 * a GPU shares that GPU's array: calls that overlap in time on one GPU (other
 * streams, other threads) race and must not be made.  A persistent launch whose
 * bounded waits ran out poisons the array's arena (NaN outputs) until
 * uocr_moe_fused_errors on any stream of that device reports it and clears its
 * error word; uocr_moe_fused_status reports it in stream order. */
int uocr_moe_decode_rows_static(float* out, const float* x, int64_t rows, int64_t hidden,
                                const uocr_moe_layer* layer, int32_t* expert_ids, float* expert_weights,
                                void* stream, char* err, size_t errlen);

/* uocr_moe_decode_stack -- the MoE blocks of consecutive decoder layers chained
 * through the residual stream in one persistent launch: x_{l+1} = x_l +
 * MoE_l(x_l) for l < n_layers, out = x_{n_layers}; each MoE_l is exactly
 * uocr_moe_decode_rows of layers[l] (the same bits), and the adds are the
 * residual adds of unlimited_ocr_max/decoder.py:709 (`x + self.mlp.decode_rows(...)`)
 * with nothing between them.  No single call of the reference matches it: it
 * serves the MoE stack of a decode step (the 11 MoE layers of
 * decoder.py:790-791 with their attention taken out), where one launch replaces
 * n_layers launches and n_layers adds.  rows <= 8; 1 <= n_layers <= 12 layers
 * of one shape and kind, each of which uocr_moe_decode_rows would run on the
 * persistent kernel (other layers are refused: chain uocr_moe_decode_rows for
 * them).  Each stream that makes such calls holds a zeroed arena of tagged
 * words (about 100 MB) until uocr_moe_release(); a call outside stream capture
 * makes the first and keeps one spare for a stream first seen under capture, so
 * a stacked call is made outside capture before one is captured. */
int uocr_moe_decode_stack(float* out, const float* x, int64_t rows, int64_t hidden,
                          const uocr_moe_layer* const* layers, int64_t n_layers, void* stream, char* err,
                          size_t errlen);

/* MoE.__call__ (prefill) -- replaces unlimited_ocr_max/decoder.py:657-667
 * (the dense 64-expert chain of the int8 path, _routed_native of the bf16
 * path).  x fp32 [T, H] -> out fp32 [T, H].  The top-k experts of every token
 * run as a grouped GEMM on the bf16 matrix cores: int8 weights dequantised to
 * bf16_rne(f32(q)*scale) (the reference's prefill values), activations
 * rounded to bf16, fp32 accumulation.  H, F, Fs multiples of 128. */
int uocr_moe_forward(float* out, const float* x, int64_t seq, int64_t hidden,
                     const uocr_moe_layer* layer, int32_t* expert_ids, float* expert_weights,
                     void* workspace, size_t workspace_bytes, void* stream, char* err, size_t errlen);

/* Frees the library's own workspaces (those used when workspace == NULL) and
 * control words.  No call may be in flight. */
void uocr_moe_release(void);

/* Waits for `stream` and reports whether a persistent decode launch on it (or
 * on the device's static scratch) ran out of its bounded waits: errors = 1.
 * Such a launch wrote NaN where its outputs depended on what it waited for,
 * and every later launch on the same slot writes NaN until this call, which
 * then clears the slot's error word (the launch epoch keeps counting, so no
 * value the failed launch left behind can satisfy a later launch's waits).
 * The waits run out only when the persistent kernel's workgroups cannot all
 * be resident, i.e. another kernel holds CUs for tens of milliseconds.  No
 * counterpart in the reference; the error path of this build's decode kernel. */
int uocr_moe_fused_errors(void* stream, uint32_t* errors, char* err, size_t errlen);

/* The same report without a synchronisation: enqueues on `stream` one tiny
 * kernel that writes flag[0] (device memory, one uint32) = 1 if the error word
 * of `stream`'s slot or of the device's static scratch is set, else 0.  Stream
 * ordered after the decode launches before it, so a serving loop reads the
 * flag with its outputs (or tests it on the device); capturable in a graph.
 * It clears nothing: after a 1, uocr_moe_fused_errors resets the slot.  No
 * counterpart in the reference (its ops fail on the host only,
 * kernels/moe_int8.mojo:194-210); the error path of this build's decode kernel. */
int uocr_moe_fused_status(uint32_t* flag, void* stream, char* err, size_t errlen);

/* Arms a phase trace for the next persistent decode launch (one layer, or a
 * stack): for task i of layer l it writes 8 int64 words at buffer[8 (i + l R)]
 * (device memory, `words` long; R = the layout's task capacity + the grid's
 * workgroups): 100 MHz wall-clock stamps of its phases (0 start, 1 weights
 * landed, 3 inputs polled, 4 chain done, 2 end, 5 when its wave learnt the
 * routing), word 6 its kind and word 7 the wave that ran it; each workgroup's
 * 8 words follow the layer's tasks (its entry, epoch read or x landed, and the
 * routing's steps).  grid_waves receives the waves of the last traced launch.
 * A diagnostic of this build's decode kernel; tracing waits for each task's
 * loads, so a traced launch runs slower.  The trace is compiled in only when
 * the library is built with UOCR_DECODE_TRACE=1; other builds refuse the
 * call. */
int uocr_moe_fused_trace(void* buffer, int64_t words, int* grid_waves, char* err, size_t errlen);

/* ---------------------------------------------------------------------------
 * Kernel timing (no counterpart in the reference; for benchmarks).  After
 * uocr_moe_timing_begin(capacity), each of the next `capacity` kernel
 * launches of this library records a start/stop event pair around the kernel
 * (hipExtLaunchKernelGGL).  uocr_moe_timing_end waits for them and writes, per
 * launch in order, the duration in ms and the kernel's name (NUL-terminated,
 * name_stride bytes apart); it ends the timing.  Not for use under stream
 * capture; not thread-safe against concurrent callers.
 * ------------------------------------------------------------------------- */
int uocr_moe_timing_begin(int capacity, char* err, size_t errlen);
int uocr_moe_timing_end(int capacity, float* ms, char* names, size_t name_stride, int* count,
                        char* err, size_t errlen);

#ifdef __cplusplus
}
#endif
#endif
