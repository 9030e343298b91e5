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

}  // namespace

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
