// Decode-shape expert GEMVs: the routed int8 / bf16 stacks and the K-blocked
// bf16 shared experts, one output column per lane.
//
// Arithmetic (the contract the CPU oracle restates):
//   int8  out[r,n] = fma-chain over groups g of  fma(scale[e,n,g], gsum_g, acc)
//         gsum_g   = fma-chain over kk in group g of fma(f32(w[e,n,kk]), x[r,kk], .)
//         -- the order of unlimited_ocr_max/kernels/moe_int8.mojo:126-148;
//   bf16  out[r,n] = sum over 128-element chunks c, in order, of
//         csum_c   = fma-chain over kk in chunk c of fma(f32(w[n,kk]), x[r,kk], .)
// A row's result depends only on its own activation row and expert, never on
// which rows share the call (the reference's batch invariance).
//
// Work decomposition (MI355X): a workgroup owns one expert, a tile of up to 8
// rows routed to it, and 64 consecutive output columns (lane = column).  Its
// waves take one chunk each (wave w -> chunk w, w+NW, ...): a lane streams the
// chunk's bytes of its weight row with 16-byte loads -- every weight byte is
// read once per tile -- while the wave-uniform activations come in through
// scalar loads.  The per-chunk partials meet in LDS, where wave 0 folds them
// in chunk order.  Gate and up run in the same workgroup so SwiGLU is fused
// into the fold.
#include "uocr_device.h"
#include "uocr_kernels.h"

namespace uocr {

namespace {

template <WKind W, int NPROJ, int R>
__device__ __attribute__((always_inline)) void chunk_chain(const GemvArgs& a, int e, int n, int c,
                                            const float* const (&xr)[R],
                                            float (&part)[NPROJ][R]) {
  if constexpr (W == kInt8Rows) {
    const int64_t kbase = (int64_t)c * a.gsize;
    for (int s0 = 0; s0 < a.gsize; s0 += 128) {
      const int len = min(128, a.gsize - s0);
      const int64_t k0 = kbase + s0;
      if (a.vec && len == 128) {
        int4 buf[NPROJ][8];
#pragma unroll
        for (int p = 0; p < NPROJ; ++p) {
          const int8_t* wrow = (const int8_t*)a.p[p].w + ((int64_t)e * a.N + n) * a.K + k0;
#pragma unroll
          for (int i = 0; i < 8; ++i) buf[p][i] = load_nt16((const int4*)wrow + i);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int kk = i * 16 + q * 4 + j;
              float wv[NPROJ];
#pragma unroll
              for (int p = 0; p < NPROJ; ++p) {
                const int word = q == 0 ? buf[p][i].x : q == 1 ? buf[p][i].y : q == 2 ? buf[p][i].z : buf[p][i].w;
                wv[p] = (float)(int8_t)(word >> (8 * j));
              }
#pragma unroll
              for (int r = 0; r < R; ++r) {
                const float xv = ldc(xr[r] + k0 + kk);
#pragma unroll
                for (int p = 0; p < NPROJ; ++p) part[p][r] = __builtin_fmaf(wv[p], xv, part[p][r]);
              }
            }
          }
        }
      } else {
        for (int i = 0; i < len; ++i) {
          float wv[NPROJ];
#pragma unroll
          for (int p = 0; p < NPROJ; ++p)
            wv[p] = (float)ldg((const int8_t*)a.p[p].w + ((int64_t)e * a.N + n) * a.K + k0 + i);
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const float xv = ldc(xr[r] + k0 + i);
#pragma unroll
            for (int p = 0; p < NPROJ; ++p) part[p][r] = __builtin_fmaf(wv[p], xv, part[p][r]);
          }
        }
      }
    }
  } else {
    // bf16: chunk c covers k in [c*128, min(K, c*128 + 128)).
    const int64_t k0 = (int64_t)c * kChunk;
    const int len = (int)min((int64_t)kChunk, (int64_t)a.K - k0);
    if (a.vec && len == kChunk) {
      // Two halves of 64 elements: 8 loads of 8 bf16 per projection each.
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        int4 buf[NPROJ][8];
#pragma unroll
        for (int p = 0; p < NPROJ; ++p) {
          const uint16_t* w = (const uint16_t*)a.p[p].w;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int64_t kk = k0 + half * 64 + i * 8;
            const uint16_t* src;
            if constexpr (W == kBf16Rows)
              src = w + ((int64_t)e * a.N + n) * a.K + kk;
            else
              src = w + ((kk >> 4) * a.N + n) * 16 + (kk & 15);
            buf[p][i] = load_nt16(src);
          }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int kk = half * 64 + i * 8 + q * 2 + h;
              float wv[NPROJ];
#pragma unroll
              for (int p = 0; p < NPROJ; ++p) {
                const uint32_t word = (uint32_t)(q == 0 ? buf[p][i].x : q == 1 ? buf[p][i].y : q == 2 ? buf[p][i].z : buf[p][i].w);
                wv[p] = h == 0 ? bf16_lo(word) : bf16_hi(word);
              }
#pragma unroll
              for (int r = 0; r < R; ++r) {
                const float xv = ldc(xr[r] + k0 + kk);
#pragma unroll
                for (int p = 0; p < NPROJ; ++p) part[p][r] = __builtin_fmaf(wv[p], xv, part[p][r]);
              }
            }
          }
        }
      }
    } else {
      for (int i = 0; i < len; ++i) {
        const int64_t kk = k0 + i;
        float wv[NPROJ];
#pragma unroll
        for (int p = 0; p < NPROJ; ++p) {
          const uint16_t* w = (const uint16_t*)a.p[p].w;
          uint16_t b;
          if constexpr (W == kBf16Rows)
            b = ldg(w + ((int64_t)e * a.N + n) * a.K + kk);
          else
            b = ldg(w + ((kk >> 4) * a.N + n) * 16 + (kk & 15));
          wv[p] = bf16_bits_to_f32(b);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float xv = ldc(xr[r] + kk);
#pragma unroll
          for (int p = 0; p < NPROJ; ++p) part[p][r] = __builtin_fmaf(wv[p], xv, part[p][r]);
        }
      }
    }
  }
}

// Rows t .. t+R-1 of a group: group_rows[t + r], or t + r for the identity
// grouping of a dense weight.
template <WKind W, int NPROJ, int R>
__device__ __attribute__((always_inline)) void gemv_tile(const GemvArgs& a, int e, const int32_t* rows, int t, int cnt,
                                                         int n, bool valid, float* lds) {
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int NW = (int)(blockDim.x >> 6);
  const int lane = lane_id();
  int rowv[R];
  const float* xr[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    // padded rows (r >= cnt) repeat the last real row and are not stored
    const int rr = min(r, cnt - 1);
    rowv[r] = __builtin_amdgcn_readfirstlane(rows ? ldc(rows + t + rr) : t + rr);
    xr[r] = a.x + (int64_t)(rowv[r] / a.x_div) * a.ldx;
  }
  float acc[NPROJ][R];
#pragma unroll
  for (int p = 0; p < NPROJ; ++p)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[p][r] = 0.0f;

  // Chunks go to LDS in batches of `batch`; wave w takes chunks w, w+NW, ...
  // of the batch, then wave 0 folds the batch in chunk order.
  for (int cb = 0; cb < a.nchunks; cb += a.batch) {
    const int nb = min(a.batch, a.nchunks - cb);
    for (int cc = w; cc < nb; cc += NW) {
      float part[NPROJ][R];
#pragma unroll
      for (int p = 0; p < NPROJ; ++p)
#pragma unroll
        for (int r = 0; r < R; ++r) part[p][r] = 0.0f;
      chunk_chain<W, NPROJ, R>(a, e, n, cb + cc, xr, part);
#pragma unroll
      for (int p = 0; p < NPROJ; ++p)
#pragma unroll
        for (int r = 0; r < R; ++r) lds[((cc * NPROJ + p) * R + r) * kWave + lane] = part[p][r];
    }
    __syncthreads();
    if (w == 0) {
      for (int cc = 0; cc < nb; ++cc) {
#pragma unroll
        for (int p = 0; p < NPROJ; ++p) {
          float s = 1.0f;
          if constexpr (W == kInt8Rows) s = ldg(a.p[p].s + ((int64_t)e * a.N + n) * a.nchunks + cb + cc);
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const float v = lds[((cc * NPROJ + p) * R + r) * kWave + lane];
            if constexpr (W == kInt8Rows)
              acc[p][r] = __builtin_fmaf(s, v, acc[p][r]);
            else
              acc[p][r] = acc[p][r] + v;
          }
        }
      }
    }
    __syncthreads();
  }
  if (w == 0 && valid) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r >= cnt) break;
      float v;
      if constexpr (NPROJ == 2)
        v = silu(acc[0][r]) * acc[1][r];
      else
        v = acc[0][r];
      stg(a.out + (int64_t)rowv[r] * a.ldo + n, v);
    }
  }
}

template <WKind W, int NPROJ>
__device__ __attribute__((always_inline)) void gemv_part(const GemvArgs& a, int wg, float* lds) {
  const int cols = (a.N + kWave - 1) / kWave;
  const int g = wg / cols;
  const int cb = wg - g * cols;
  int e, r0, r1;
  const int32_t* rows;
  if (a.rows.n_groups == nullptr) {
    if (g > 0) return;
    e = 0;
    r0 = 0;
    r1 = a.rows.identity;
    rows = nullptr;
  } else {
    if (g >= ldc(a.rows.n_groups)) return;
    e = ldc(a.rows.group_expert + g);
    r0 = ldc(a.rows.group_start + g);
    r1 = ldc(a.rows.group_start + g + 1);
    rows = a.rows.group_rows;
  }
  const int nraw = cb * kWave + lane_id();
  const bool valid = nraw < a.N;
  const int n = valid ? nraw : a.N - 1;
  for (int t = r0; t < r1; t += 8) {
    const int cnt = min(8, r1 - t);
    if (cnt == 1)
      gemv_tile<W, NPROJ, 1>(a, e, rows, t, cnt, n, valid, lds);
    else if (cnt == 2)
      gemv_tile<W, NPROJ, 2>(a, e, rows, t, cnt, n, valid, lds);
    else if (cnt <= 4)
      gemv_tile<W, NPROJ, 4>(a, e, rows, t, cnt, n, valid, lds);
    else
      gemv_tile<W, NPROJ, 8>(a, e, rows, t, cnt, n, valid, lds);
  }
}

// One launch, up to two parts (e.g. routed experts + shared experts): the
// first `split` workgroups run part 0, the rest part 1.
template <WKind W0, int NP0, WKind W1, int NP1>
__global__ void __launch_bounds__(kGemvMaxThreads) k_gemv2(GemvArgs a0, GemvArgs a1, int split) {
  extern __shared__ float lds[];
  const int wg = (int)blockIdx.x;
  if (wg < split)
    gemv_part<W0, NP0>(a0, wg, lds);
  else
    gemv_part<W1, NP1>(a1, wg - split, lds);
}

template <WKind W, int NPROJ>
__global__ void __launch_bounds__(kGemvMaxThreads) k_gemv1(GemvArgs a) {
  extern __shared__ float lds[];
  gemv_part<W, NPROJ>(a, (int)blockIdx.x, lds);
}

// ---------------------------------------------------------------------------
// dense_bf16_qmv for narrow outputs (N < kDenseNarrowMaxN) and at most
// kDenseNarrowMaxRows rows (past 2 rows the activation reads from LDS, 32 per
// row and chunk, cost more than k_gemv1's scalar loads).  k_gemv1 gives a
// workgroup 64 output columns (lane = column, wave = chunk), so a 1280-wide
// projection runs on 20 workgroups.  Here a lane is a (column, chunk) pair: a
// workgroup holds kNarrowCols columns x kNarrowSlots chunks (256 lanes), so
// N = 1280 gets 160 workgroups.  Each lane runs the same chain as chunk_chain
// (fma over the chunk's k in ascending order, from 0), the partials meet in
// LDS, and thread (row, column) adds them in chunk order from 0 -- the bits of
// k_gemv1.  The activations of a batch of chunks are staged in LDS (a chunk's
// 128 floats, padded to 132 so that the 4 chunks a wave reads at once sit in
// different banks), since a wave now spans 4 chunks.
constexpr int kNarrowCols = 8;  // 8 rather than 16: twice the workgroups, the decode step 1 % faster at B=1
constexpr int kNarrowThreads = 256;
constexpr int kNarrowSlots = kNarrowThreads / kNarrowCols;  // chunks per batch
constexpr int kNarrowPitch = kChunk + 4;

// The RMSNorm prologue of a fused call (rows of x replaced by rmsnorm(x + residual) * gamma before the
// projection): the order of k_add_rmsnorm, so the normed rows have its bits.
struct NormPrologue {
  const float* residual;  // null: no residual add
  float* x_out;           // x + residual, written by workgroup 0 (with a residual)
  const float* gamma;
  float eps;
};

template <int R>
__device__ __attribute__((always_inline)) void norm_staged(const GemvArgs& a, const NormPrologue& np, int t,
                                                           int cnt, float* xs, float* red) {
  const int tid = (int)threadIdx.x;
  for (int r = 0; r < R; ++r) {
    if (r >= cnt) break;  // padded rows are never stored
    float* xr = xs + r * kNarrowSlots * kNarrowPitch;
    float ss = 0.0f;
    for (int k = tid; k < a.K; k += kNarrowThreads) {
      const int idx = (k / kChunk) * kNarrowPitch + k % kChunk;
      float v = xr[idx];
      if (np.residual != nullptr) {
        v = v + ldg(np.residual + (int64_t)(t + r) * a.ldx + k);
        xr[idx] = v;
        if (blockIdx.x == 0) np.x_out[(int64_t)(t + r) * a.ldx + k] = v;
      }
      ss = __builtin_fmaf(v, v, ss);
    }
    ss = tree_sum(ss);
    if (lane_id() == 0) red[tid / kWave] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();  // red is reused by the next row
    const float rn = 1.0f / sqrtf(ss / (float)a.K + np.eps);
    for (int k = tid; k < a.K; k += kNarrowThreads) {
      const int idx = (k / kChunk) * kNarrowPitch + k % kChunk;
      xr[idx] = (xr[idx] * rn) * ldg(np.gamma + k);
    }
  }
  __syncthreads();
}

template <int R, bool NORM>
__device__ __attribute__((always_inline)) void dense_narrow_tile(const GemvArgs& a, const NormPrologue& np, int t,
                                                                 int cnt, int n0, float* xs, float* fold,
                                                                 float* red) {
  const int tid = (int)threadIdx.x;
  const int c = tid % kNarrowCols, j = tid / kNarrowCols;
  const int n = min(n0 + c, a.N - 1);
  const uint16_t* w = (const uint16_t*)a.p[0].w;
  // the fold thread (row fr, column fc) keeps its sum across batches
  const int fr = tid / kNarrowCols, fc = tid % kNarrowCols;
  float acc = 0.0f;
  for (int cb = 0; cb < a.nchunks; cb += kNarrowSlots) {
    const int nb = min(kNarrowSlots, a.nchunks - cb);
    // stage x rows t .. t+R-1 (padded rows repeat the last real row) for chunks cb .. cb+nb-1
    for (int i = tid; i < R * nb * kChunk; i += kNarrowThreads) {
      const int r = i / (nb * kChunk);
      const int rem = i - r * nb * kChunk;
      const int ch = rem / kChunk, kk = rem - ch * kChunk;
      const int64_t k = (int64_t)(cb + ch) * kChunk + kk;
      const int row = t + min(r, cnt - 1);
      xs[(r * kNarrowSlots + ch) * kNarrowPitch + kk] = k < a.K ? ldg(a.x + (int64_t)row * a.ldx + k) : 0.0f;
    }
    __syncthreads();
    if constexpr (NORM) norm_staged<R>(a, np, t, cnt, xs, red);  // the whole row is in this one batch
    float part[R];
#pragma unroll
    for (int r = 0; r < R; ++r) part[r] = 0.0f;
    if (j < nb) {
      const int64_t k0 = (int64_t)(cb + j) * kChunk;
      const int len = (int)min((int64_t)kChunk, (int64_t)a.K - k0);
      const float* xj = xs + j * kNarrowPitch;
      if (a.vec && len == kChunk) {
        int4 buf[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int64_t kk = k0 + i * 8;
          buf[i] = load_nt16(w + ((kk >> 4) * a.N + n) * 16 + (kk & 15));
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const f32x4 x0 = *(const f32x4*)(xj + r * kNarrowSlots * kNarrowPitch + i * 8);
            const f32x4 x1 = *(const f32x4*)(xj + r * kNarrowSlots * kNarrowPitch + i * 8 + 4);
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const uint32_t word =
                  (uint32_t)(q == 0 ? buf[i].x : q == 1 ? buf[i].y : q == 2 ? buf[i].z : buf[i].w);
              part[r] = __builtin_fmaf(bf16_lo(word), xv[2 * q], part[r]);
              part[r] = __builtin_fmaf(bf16_hi(word), xv[2 * q + 1], part[r]);
            }
          }
        }
      } else {
        for (int i = 0; i < len; ++i) {
          const int64_t kk = k0 + i;
          const float wv = bf16_bits_to_f32(ldg(w + ((kk >> 4) * a.N + n) * 16 + (kk & 15)));
#pragma unroll
          for (int r = 0; r < R; ++r)
            part[r] = __builtin_fmaf(wv, xj[r * kNarrowSlots * kNarrowPitch + i], part[r]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) fold[(r * kNarrowSlots + j) * kNarrowCols + c] = part[r];
    __syncthreads();
    if (fr < R) {
      for (int jj = 0; jj < nb; ++jj) acc = acc + fold[(fr * kNarrowSlots + jj) * kNarrowCols + fc];
    }
    __syncthreads();  // xs and fold are rewritten by the next batch
  }
  if (fr < cnt && n0 + fc < a.N) stg(a.out + (int64_t)(t + fr) * a.ldo + n0 + fc, acc);
}

template <bool NORM>
__global__ void __launch_bounds__(kNarrowThreads) k_dense_narrow(GemvArgs a, NormPrologue np) {
  extern __shared__ float lds[];
  __shared__ float red[kNarrowThreads / kWave];
  float* fold = lds;                                           // [8][slots][cols]
  float* xs = lds + 8 * kNarrowSlots * kNarrowCols;            // [R][slots][pitch]
  const int n0 = (int)blockIdx.x * kNarrowCols;
  const int rows = a.rows.identity;
  for (int t = 0; t < rows; t += 8) {
    const int cnt = min(8, rows - t);
    if (cnt == 1)
      dense_narrow_tile<1, NORM>(a, np, t, cnt, n0, xs, fold, red);
    else if (cnt == 2)
      dense_narrow_tile<2, NORM>(a, np, t, cnt, n0, xs, fold, red);
    else if (cnt <= 4)
      dense_narrow_tile<4, NORM>(a, np, t, cnt, n0, xs, fold, red);
    else
      dense_narrow_tile<8, NORM>(a, np, t, cnt, n0, xs, fold, red);
  }
}

}  // namespace

static size_t dense_narrow_lds(int rows) {
  const int rmax = rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8;
  return (size_t)(8 * kNarrowSlots * kNarrowCols + rmax * kNarrowSlots * kNarrowPitch) * sizeof(float);
}

hipError_t launch_dense(const GemvArgs& a, int waves, hipStream_t s) {
  if (a.N >= kDenseNarrowMaxN || a.rows.identity > kDenseNarrowMaxRows || a.kind != kBf16KBlocked ||
      a.rows.n_groups != nullptr)
    return launch_gemv(a, 1, 1, waves, s);
  if (a.N == 0 || a.rows.identity == 0) return hipSuccess;
  // 8 rows need 74 KB of LDS, past the default limit of a launch
  static const hipError_t attr = hipFuncSetAttribute((const void*)k_dense_narrow<false>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024);
  if (attr != hipSuccess) return attr;
  UOCR_LAUNCH("dense_narrow", k_dense_narrow<false>, dim3((unsigned)((a.N + kNarrowCols - 1) / kNarrowCols)),
              dim3(kNarrowThreads), dense_narrow_lds(a.rows.identity), s, a, NormPrologue{});
  return hipGetLastError();
}

hipError_t launch_norm_dense(const GemvArgs& a, const float* residual, float* x_out, const float* gamma, float eps,
                             hipStream_t s) {
  if (a.N >= kDenseNarrowMaxN || a.rows.identity > kDenseNarrowMaxRows || a.kind != kBf16KBlocked ||
      a.K > kNarrowSlots * kChunk || a.rows.n_groups != nullptr)
    return hipErrorInvalidValue;
  if (a.N == 0 || a.rows.identity == 0) return hipSuccess;
  static const hipError_t attr = hipFuncSetAttribute((const void*)k_dense_narrow<true>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024);
  if (attr != hipSuccess) return attr;
  UOCR_LAUNCH("norm_dense", k_dense_narrow<true>, dim3((unsigned)((a.N + kNarrowCols - 1) / kNarrowCols)),
              dim3(kNarrowThreads), dense_narrow_lds(a.rows.identity), s, a, NormPrologue{residual, x_out, gamma, eps});
  return hipGetLastError();
}

int gemv_workgroups(const GemvArgs& a, int max_groups) {
  const int cols = (a.N + kWave - 1) / kWave;
  return (a.rows.n_groups == nullptr ? 1 : max_groups) * cols;
}

size_t gemv_lds_bytes(int batch, int nproj) { return (size_t)batch * nproj * 8 * kWave * sizeof(float); }

hipError_t launch_gemv(const GemvArgs& a, int max_groups, int nproj, int waves, hipStream_t s) {
  const int wgs = gemv_workgroups(a, max_groups);
  if (wgs == 0) return hipSuccess;
  const size_t lds = gemv_lds_bytes(a.batch, nproj);
  const dim3 grid(wgs), block(waves * kWave);
  if (nproj == 1) {
    switch (a.kind) {
      case kInt8Rows: UOCR_LAUNCH("gemv_op", (k_gemv1<kInt8Rows, 1>), grid, block, lds, s, a); break;
      case kBf16Rows: UOCR_LAUNCH("gemv_op", (k_gemv1<kBf16Rows, 1>), grid, block, lds, s, a); break;
      case kBf16KBlocked: UOCR_LAUNCH("gemv_op", (k_gemv1<kBf16KBlocked, 1>), grid, block, lds, s, a); break;
    }
  } else {
    return hipErrorInvalidValue;  // the fused gate/up pair runs through launch_gemv_pair
  }
  return hipGetLastError();
}

hipError_t launch_gemv_pair(const GemvArgs& routed, int max_groups, const GemvArgs& shared, int nproj,
                            int waves, hipStream_t s) {
  const int split = gemv_workgroups(routed, max_groups);
  const int wgs = split + gemv_workgroups(shared, 1);
  const size_t lds = gemv_lds_bytes(routed.batch > shared.batch ? routed.batch : shared.batch, nproj);
  const dim3 grid(wgs), block(waves * kWave);
  if (routed.kind == kInt8Rows) {
    if (nproj == 2)
      UOCR_LAUNCH("gemv_gateup", (k_gemv2<kInt8Rows, 2, kBf16KBlocked, 2>), grid, block, lds, s, routed, shared, split);
    else
      UOCR_LAUNCH("gemv_down", (k_gemv2<kInt8Rows, 1, kBf16KBlocked, 1>), grid, block, lds, s, routed, shared, split);
  } else {
    if (nproj == 2)
      UOCR_LAUNCH("gemv_gateup", (k_gemv2<kBf16Rows, 2, kBf16KBlocked, 2>), grid, block, lds, s, routed, shared, split);
    else
      UOCR_LAUNCH("gemv_down", (k_gemv2<kBf16Rows, 1, kBf16KBlocked, 1>), grid, block, lds, s, routed, shared, split);
  }
  return hipGetLastError();
}

}  // namespace uocr
