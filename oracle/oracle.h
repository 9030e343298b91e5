/*
 * CPU oracle for the DeepSeek-V2 routed-expert MoE block of unlimited-ocr-max.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load this library, and only as the checker or
 * as the timed CPU baseline.  The product (the HIP library) never links it,
 * and never falls back to it.
 *
 * Every function restates one piece of the reference's arithmetic and cites
 * the reference file:line it follows (paths relative to the reference root).
 * Where the reference leaves an order to a third-party library (MAX's matmul,
 * softmax, top_k, silu), the function defines one order and says so; those
 * functions are pinned by float64 closed forms and by the reference's own
 * known-answer tests, not bit for bit against the reference.
 *
 * Pinning (what checks each function; see tests/test_oracle_*.py):
 *   or_quantize_per_group     the reference's hand-derived golden micro-tensor
 *                             (tools/quantize_int8.py:787-870) and its scalar
 *                             twin's contract (tools/quantize_int8.py:332-361)
 *   or_bf16_rne               exhaustive tie sweep + torch's bf16 cast
 *   or_int8_dequant_expert    closed form bf16_rne(f32(q)*scale)
 *                             (tests/test_kernels_int8.py:200-208)
 *   or_moe_int8_qmv           float64 closed form at 1e-6 and a float64-emulated
 *                             fma chain (tests/test_kernels_int8.py:150-197)
 *   or_moe_bf16_qmv_*         float64 closed form at 1e-5, one-hot exact answers
 *                             (tests/test_kernels_bf16.py:118-122,199-211)
 *   or_dense_bf16_qmv_*       float64 closed form at 1e-5, one-hot exact answers
 *                             (tests/test_kernels_dense_bf16.py:86-87,136-147)
 *   or_uexp / or_silu         libm expf within 2 ulp over a dense sweep
 *   or_moe_gate               float64 softmax + stable argsort top-k
 *                             (tests/test_decoder_int8.py:720-727)
 *   or_moe_decode_*           float64 layer closed form, cosine >= 0.99999 and
 *                             rel <= 1e-4 (tests/test_decoder_int8.py:701-769)
 */
#ifndef UOCR_ORACLE_H
#define UOCR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar helpers ---------------------------------------------------- */

/* fp32 -> bf16 bits, round-to-nearest-even, NaN canonicalised to 0x7FC0
 * (unlimited_ocr_max/bf16.py:122-136). */
uint16_t or_bf16_rne(float f);
float or_bf16_to_f32(uint16_t b);

/* exp(x) by Cody-Waite reduction (ln2 split in a 16-bit head and a tail) and
 * the degree-7 Taylor polynomial of e^r on |r| <= ln2/2 in Horner form, then
 * two exact power-of-two scalings.  The decode layer's softmax and SiLU use it
 * so that the GPU (which evaluates the same steps) agrees bit for bit. */
float or_uexp(float x);
/* silu(g) = g / (1 + uexp(-g)), each step rounded to fp32. */
float or_silu(float g);
void or_uexp_array(float* out, const float* x, int64_t n);
void or_silu_array(float* out, const float* x, int64_t n);

/* ---- thread pool ------------------------------------------------------- */

/* Worker threads used by the functions that take `threads` (0 = every online
 * core).  Returns the number actually used. */
int or_threads(int threads);

/* ---- quantiser --------------------------------------------------------- */

/* tools/quantize_int8.py:298-329: per group of `group` along K,
 * amax = max|w|, scale = amax == 0 ? 1 : amax/127 (fp32),
 * q = clip(rint(w/scale), -127, 127).  Returns 0, or -1 if k % group. */
int or_quantize_per_group(const float* w, int64_t n, int64_t k, int64_t group,
                          int8_t* q, float* scales);

/* ---- the reference's custom ops --------------------------------------- */

/* moe_int8_qmv (unlimited_ocr_max/kernels/moe_int8.mojo:181-258, sums at
 * :126-148): out[s,n] = fma-chain over groups of fma-chain over kk, in the
 * reference's work decomposition (one item per (s,n), leader rows serve tiles
 * of up to 4 rows; moe_routing.mojo:26-92).  Returns 0 or a negative code. */
int or_moe_int8_qmv(float* out, const float* x, const int32_t* ids,
                    const int8_t* w, const float* scales, int64_t k,
                    int64_t E, int64_t N, int64_t K, int64_t groups,
                    int threads);

/* moe_bf16_qmv, CPU path (unlimited_ocr_max/kernels/moe_bf16.mojo:119-148,
 * 310-345): VEC=16 lane partial sums (product rounded, then added), reduced by
 * a halving tree at the end; K % 16 != 0 runs one scalar sum.  The reference
 * leaves the product/add contraction to its compiler, so this is a tolerance
 * pin only.  w holds bf16 bit patterns. */
int or_moe_bf16_qmv_ref(float* out, const float* x, const int32_t* ids,
                        const uint16_t* w, int64_t k, int64_t E, int64_t N,
                        int64_t K, int threads);

/* moe_bf16_qmv in the chunked order the HIP kernels define: K cut into
 * chunks of 128, each an fma chain in k order from 0, the chunk sums added in
 * chunk order.  Ids clamp to [0, E). */
int or_moe_bf16_qmv_chunked(float* out, const float* x, const int32_t* ids,
                            const uint16_t* w, int64_t k, int64_t E,
                            int64_t N, int64_t K, int threads);

/* dense_bf16_qmv (unlimited_ocr_max/kernels/dense_bf16.mojo:85-116,119-158)
 * on a K-blocked weight w[K/16][N][16]: per block, the 16 products folded to
 * 4 lanes by a halving tree and accumulated, then the 4 lanes reduced by a
 * halving tree.  Tolerance pin only (contraction is compiler-defined). */
int or_dense_bf16_qmv_ref(float* out, const float* x, const uint16_t* w_kb,
                          int64_t M, int64_t N, int64_t K, int64_t tile,
                          int threads);

/* dense_bf16_qmv in the chunked order of the HIP kernels (as
 * or_moe_bf16_qmv_chunked, chunks of 128 = 8 K-blocks). */
int or_dense_bf16_qmv_chunked(float* out, const float* x, const uint16_t* w_kb,
                              int64_t M, int64_t N, int64_t K, int threads);

/* int8_dequant_expert (unlimited_ocr_max/kernels/moe_int8.mojo:261-342):
 * out[n,kk] = bf16_rne(f32(w[e,n,kk]) * scales[e,n,kk/G]), e = clamp(idx). */
int or_int8_dequant_expert(uint16_t* out, const int8_t* w, const float* scales,
                           int32_t idx, int64_t E, int64_t N, int64_t K,
                           int64_t groups);

/* ---- the MoE block ----------------------------------------------------- */

/* fp32 dot product in the order the HIP gate kernel defines: 64 lane partial
 * fma chains (lane l takes k = l, l+64, ...), then a halving tree
 * p[l] += p[l+off] for off = 32, 16, ..., 1. */
float or_dot_tree64(const float* a, const float* b, int64_t K);

/* MoEGate.__call__ (unlimited_ocr_max/decoder.py:509-514): logits = x Wr^T,
 * softmax over E, top-k in score order, ties to the lower id (the stable
 * argsort of tests/test_decoder_int8.py:727), no renormalisation
 * (model_config.py:149-150) unless `renorm`.  Softmax: m = max, ex = uexp(l-m),
 * S = halving-tree sum of ex over 64 slots, p = ex / S.  E <= 64. */
int or_moe_gate(int32_t* ids, float* weights, const float* x, const float* wr,
                int64_t T, int64_t E, int64_t H, int64_t topk, int renorm);

/* Weights of one MoE layer.  Routed stacks are int8 + fp32 scales
 * ([E,F,H]/[E,F,H]/[E,H,F], scales [E,F,H/G]/[E,F,H/G]/[E,H,F/G]) when
 * int8 != 0, else bf16 bit patterns.  Shared experts are bf16, K-blocked:
 * gate/up [H/16][Fs][16], down [Fs/16][H][16] (decoder.py:264-278,
 * weight_adapters.py:222-233).  Router fp32 [E,H]. */
typedef struct {
  int64_t E, H, F, Fs, topk, group;
  int int8;
  int renorm;
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
} or_moe_layer;

/* MoE.decode_rows (unlimited_ocr_max/decoder.py:641-655) in the exact orders
 * the HIP decode path defines: gate as or_moe_gate; routed rows b*k+j through
 * the int8 chain of or_moe_int8_qmv (or the chunked bf16 chain); h = silu(g)*u;
 * shared experts through the chunked bf16 chain; out = fma chain over j of
 * w[b,j]*y[b*k+j] from 0, plus the shared output.  Optional outputs ids/wts
 * (may be NULL). */
int or_moe_decode_exact(float* out, int32_t* ids, float* wts, const float* x,
                        int64_t B, const or_moe_layer* L, int threads);

/* The same layer in the reference's own CPU decomposition, for timing: the
 * qmv ops as or_moe_int8_qmv / or_moe_bf16_qmv_ref over the B*k repeated rows
 * (decoder.py:616-639), silu*mul as its own pass, the mix as a [1,k]@[k,H]
 * product per token (decoder.py:599-604), the shared experts through
 * or_dense_bf16_qmv_ref at the tile decoder._rows_per_read picks
 * (decoder.py:144-163). */
int or_moe_decode_refdecomp(float* out, const float* x, int64_t B,
                            const or_moe_layer* L, int threads);

#ifdef __cplusplus
}
#endif
#endif
