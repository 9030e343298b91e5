// The elementwise and per-row steps of the decoder layer's decode path that
// sit around the MoE block and the attention (unlimited_ocr_max/decoder.py):
//
//   add_rmsnorm  RmsNorm (decoder.py:252-261, ops.rms_norm with the gamma in
//                the activation dtype) over rows of x, optionally after the
//                residual add that precedes it (DecoderLayer.decode,
//                decoder.py:702-709): v = x + delta is written back, then
//                y = (v * r) * gamma with r = 1 / sqrt(mean(v^2) + eps).
//   rope         the rotate_half RoPE of Attention._rope (decoder.py:459-462)
//                on q and k [rows, heads, D] (v copied alongside, so that one
//                fused q/k/v projection feeds it) with each row's cos / sin row
//                gathered at its position (rope_rows, decoder.py:766-775):
//                out = x * cos + rotate_half(x) * sin, each product and the sum
//                rounded to fp32 (no contraction), as the reference's
//                elementwise graph computes it.
//   swiglu       silu(gate) * up of GatedMlp.decode_rows (decoder.py:274-276)
//                over the [rows, 2F] output of one gate+up projection.
//
// All three are HBM-bound and tiny at decode shapes (a few KB per row).
#include "uocr_device.h"
#include "uocr_kernels.h"

namespace uocr {

namespace {

constexpr int kNormThreads = 256;

// One workgroup per row.  Sum of squares: thread t chains fma(v, v, s) over
// elements t, t + 256, ...; the 64 lanes of a wave add by a halving tree; the
// 4 wave sums add as (w0 + w1) + (w2 + w3).  A thread keeps its elements (and
// their gamma) in registers between the two passes when the row has at most
// kNormRegs * 256 of them, so the second pass reads nothing from memory.
constexpr int kNormRegs = 8;

template <bool RESID>
__global__ void __launch_bounds__(kNormThreads) k_add_rmsnorm(float* __restrict__ out, float* x_out, const float* x,
                                                              const float* __restrict__ delta,
                                                              const float* __restrict__ gamma, int dim, float eps) {
  __shared__ float red[kNormThreads / kWave];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * dim;
  const float* dr = RESID ? delta + row * dim : nullptr;
  float* xo = RESID ? x_out + row * dim : nullptr;
  const int tid = (int)threadIdx.x;
  const bool regs = dim <= kNormRegs * kNormThreads;
  float vk[kNormRegs], gk[kNormRegs];
  float ss = 0.0f;
  if (regs) {
#pragma unroll
    for (int j = 0; j < kNormRegs; ++j) {
      const int i = tid + j * kNormThreads;
      vk[j] = 0.0f;
      gk[j] = 0.0f;
      if (i < dim) {
        vk[j] = xr[i];
        if constexpr (RESID) vk[j] = vk[j] + dr[i];
        gk[j] = ldg(gamma + i);
      }
    }
#pragma unroll
    for (int j = 0; j < kNormRegs; ++j) {
      const int i = tid + j * kNormThreads;
      if (i < dim) {
        if constexpr (RESID) xo[i] = vk[j];  // x_out may be x: each element is read then written by the same thread
        ss = __builtin_fmaf(vk[j], vk[j], ss);
      }
    }
  } else {
    for (int i = tid; i < dim; i += kNormThreads) {
      float v = xr[i];
      if constexpr (RESID) {
        v = v + dr[i];
        xo[i] = v;
      }
      ss = __builtin_fmaf(v, v, ss);
    }
  }
  ss = tree_sum(ss);
  if (lane_id() == 0) red[tid / kWave] = ss;
  __syncthreads();
  ss = (red[0] + red[1]) + (red[2] + red[3]);
  const float r = 1.0f / sqrtf(ss / (float)dim + eps);
  float* yr = out + row * dim;
  if (regs) {
#pragma unroll
    for (int j = 0; j < kNormRegs; ++j) {
      const int i = tid + j * kNormThreads;
      if (i < dim) yr[i] = (vk[j] * r) * gk[j];
    }
  } else {
    for (int i = tid; i < dim; i += kNormThreads) {
      float v = xr[i];
      if constexpr (RESID) v = xo[i];
      yr[i] = (v * r) * ldg(gamma + i);
    }
  }
}

// Thread (tensor, row, head, d < D/2) writes elements d and d + D/2 of one
// head: tensor 0 is q, 1 is k (rotated), 2 is v (copied, when given).  Inputs
// are rows `in_stride` floats apart (views of one fused projection's output);
// outputs are packed [rows, heads, D].
__global__ void k_rope(float* q_out, float* k_out, float* v_out, const float* q, const float* k, const float* v,
                       int64_t rows, int heads, int half, int64_t in_stride, const int32_t* __restrict__ positions,
                       const float* __restrict__ cos_t, const float* __restrict__ sin_t, int table_rows) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_tensor = rows * heads * half;
  if (i >= 3 * per_tensor) return;
  const int which = (int)(i / per_tensor);
  const int64_t j = i - which * per_tensor;
  const int d = (int)(j % half);
  const int64_t rh = j / half;  // row * heads + head
  const int64_t row = rh / heads;
  const int h = (int)(rh - row * heads);
  const float* src = which == 0 ? q : which == 1 ? k : v;
  float* dst = which == 0 ? q_out : which == 1 ? k_out : v_out;
  if (src == nullptr) return;
  const float* x = src + row * in_stride + (int64_t)h * 2 * half;
  float* y = dst + rh * 2 * half;
  const float lo = x[d], hi = x[d + half];
  if (which == 2) {
    y[d] = lo;
    y[d + half] = hi;
    return;
  }
  const int pos = min(max(ldg(positions + row), 0), table_rows - 1);  // device data: clamped into the table
  const float* c = cos_t + (int64_t)pos * 2 * half;
  const float* s = sin_t + (int64_t)pos * 2 * half;
  const float out_lo = lo * ldg(c + d) + (-hi) * ldg(s + d);
  const float out_hi = hi * ldg(c + d + half) + lo * ldg(s + d + half);
  y[d] = out_lo;
  y[d + half] = out_hi;
}

__global__ void k_swiglu(float* __restrict__ out, const float* __restrict__ gate_up, int64_t rows, int ffn) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * ffn) return;
  const int64_t r = i / ffn;
  const int c = (int)(i - r * ffn);
  const float* gu = gate_up + r * 2 * ffn;
  out[i] = silu(gu[c]) * gu[ffn + c];
}

}  // namespace

hipError_t launch_add_rmsnorm(float* out, float* x_out, const float* x, const float* delta, const float* gamma,
                              int64_t rows, int dim, float eps, hipStream_t s) {
  if (rows == 0 || dim == 0) return hipSuccess;
  if (delta != nullptr)
    UOCR_LAUNCH("add_rmsnorm", k_add_rmsnorm<true>, dim3((unsigned)rows), dim3(kNormThreads), 0, s, out, x_out, x,
                delta, gamma, dim, eps);
  else
    UOCR_LAUNCH("rmsnorm", k_add_rmsnorm<false>, dim3((unsigned)rows), dim3(kNormThreads), 0, s, out, x_out, x,
                delta, gamma, dim, eps);
  return hipGetLastError();
}

hipError_t launch_rope(float* q_out, float* k_out, float* v_out, const float* q, const float* k, const float* v,
                       int64_t rows, int heads, int head_dim, int64_t in_stride, const int32_t* positions,
                       const float* cos_t, const float* sin_t, int table_rows, hipStream_t s) {
  const int64_t n = 3 * rows * heads * (head_dim / 2);
  if (n == 0) return hipSuccess;
  UOCR_LAUNCH("rope", k_rope, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, q_out, k_out, v_out, q, k, v, rows,
              heads, head_dim / 2, in_stride, positions, cos_t, sin_t, table_rows);
  return hipGetLastError();
}

hipError_t launch_swiglu(float* out, const float* gate_up, int64_t rows, int ffn, hipStream_t s) {
  const int64_t n = rows * ffn;
  if (n == 0) return hipSuccess;
  UOCR_LAUNCH("swiglu", k_swiglu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, out, gate_up, rows, ffn);
  return hipGetLastError();
}

}  // namespace uocr
