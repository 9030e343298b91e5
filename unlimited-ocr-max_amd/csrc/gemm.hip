// Prefill-shape expert contractions on the bf16 matrix cores, and the
// standalone int8 dequantisation op.
//
// Grouped GEMM: the routed rows are grouped by expert (route.hip); a
// workgroup owns a 64-row tile of one expert's rows and a 128-column tile of
// its weights.  Per 64-wide K step it dequantises the int8 weight tile with the
// reference's prefill numerics, w = bf16_rne(f32(q) * scale)
// (unlimited_ocr_max/kernels/moe_int8.mojo:340, the int8_dequant_expert values),
// into LDS, rounds the activations to bf16, and runs
// v_mfma_f32_32x32x16_bf16 with fp32 accumulation.  The gate/up launch fuses
// SwiGLU into its epilogue and writes h in bf16, already packed in group order,
// which is the down launch's A operand.  The shared experts (K-blocked bf16)
// ride in the same launches as extra tiles with every token as a row.
#include "uocr_device.h"
#include "uocr_kernels.h"

namespace uocr {

namespace {

constexpr int BM = 64;
constexpr int BN = 128;
constexpr int BK = 64;
constexpr int LDA = BK + 8;  // bf16 elements per LDS row (16-byte pad)
constexpr int kGemmThreads = 256;

// ------------------------------------------------------------- dequant op

__global__ void __launch_bounds__(256) k_dequant(void* __restrict__ out, int out_f32, const int8_t* __restrict__ w,
                                                 const float* __restrict__ scales, const int32_t* __restrict__ idx,
                                                 int E, int N, int K, int groups, int vec) {
  const int e = clamp_expert(idx[0], E);
  const int gsize = K / groups;
  const int64_t total = (int64_t)N * K;
  const int64_t base = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (base >= total) return;
  const int8_t* src = w + (int64_t)e * total;
  const float* sc = scales + (int64_t)e * N * groups;
  if (vec && base + 8 <= total) {
    const int2 q = *(const int2*)(src + base);
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t i = base + j;
      const int64_t n = i / K;
      const int kk = (int)(i - n * K);
      const int word = j < 4 ? q.x : q.y;
      v[j] = (float)(int8_t)(word >> (8 * (j & 3))) * sc[n * groups + kk / gsize];
    }
    if (out_f32) {
      float4* o = (float4*)((float*)out + base);
      o[0] = make_float4(v[0], v[1], v[2], v[3]);
      o[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
      uint4 o;
      o.x = pack_bf16x2(v[0], v[1]);
      o.y = pack_bf16x2(v[2], v[3]);
      o.z = pack_bf16x2(v[4], v[5]);
      o.w = pack_bf16x2(v[6], v[7]);
      *(uint4*)((uint16_t*)out + base) = o;
    }
    return;
  }
  for (int j = 0; j < 8 && base + j < total; ++j) {
    const int64_t i = base + j;
    const int64_t n = i / K;
    const int kk = (int)(i - n * K);
    const float v = (float)src[i] * sc[n * groups + kk / gsize];
    if (out_f32)
      ((float*)out)[i] = v;
    else
      ((uint16_t*)out)[i] = f32_to_bf16_rne(v);
  }
}

// ------------------------------------------------------------- grouped GEMM

struct TileRef {
  int valid;
  int e;        // expert (routed) or 0
  int pos0;     // first row position of the tile (group order) or first token
  int rows;     // valid rows in the tile
  int n0;       // first output column
};

// Decodes workgroup `wg` of a problem into its tile.
__device__ TileRef locate(const GemmProblem& P, int wg) {
  TileRef t{0, 0, 0, 0, 0};
  const int ntiles = P.N / BN;
  const int mt = wg / ntiles;
  t.n0 = (wg - mt * ntiles) * BN;
  if (P.rows.n_groups == nullptr) {
    t.pos0 = mt * BM;
    if (t.pos0 >= P.M) return t;
    t.rows = min(BM, P.M - t.pos0);
    t.valid = 1;
    return t;
  }
  const int ng = ldc(P.rows.n_groups);
  if (mt >= ldc(P.tile_start + ng)) return t;
  int g = 0;
  while (g + 1 < ng && ldc(P.tile_start + g + 1) <= mt) ++g;
  const int start = ldc(P.rows.group_start + g);
  const int count = ldc(P.rows.group_start + g + 1) - start;
  const int local = mt - ldc(P.tile_start + g);
  t.e = ldc(P.rows.group_expert + g);
  t.pos0 = start + local * BM;
  t.rows = min(BM, count - local * BM);
  t.valid = 1;
  return t;
}

template <WKind W, int NPROJ>
__device__ void gemm_tile(const GemmProblem& P, const TileRef& t, uint16_t* lds) {
  uint16_t* As = lds;                         // [BM][LDA]
  uint16_t* Bs = lds + BM * LDA;              // [NPROJ][BN][LDA]
  const int tid = (int)threadIdx.x;
  const int lane = lane_id();
  const int w = tid >> 6;
  const int wm = w & 1;   // 32-row half of the tile
  const int wn = w >> 1;  // 64-column half of the tile

  // ---- A-loader coordinates: 64 rows x 64 k, 4 threads per row, 16 k each
  const int a_row = tid >> 2;
  const int a_k = (tid & 3) * 16;
  const int a_rc = min(a_row, t.rows - 1);  // padded rows repeat the last real row
  const float* a_src_f = nullptr;
  const uint16_t* a_src_b = nullptr;
  if (P.x != nullptr) {
    int token;
    if (P.rows.n_groups == nullptr)
      token = t.pos0 + a_rc;
    else
      token = ldg(P.rows.group_rows + t.pos0 + a_rc) / P.x_div;
    a_src_f = P.x + (int64_t)token * P.ldx + a_k;
  } else {
    a_src_b = P.hb + (int64_t)(t.pos0 + a_rc) * P.ldh + a_k;
  }

  // ---- B-loader coordinates
  // int8 rows: 128 rows x 64 k bytes, 2 threads per row, 32 k each
  // bf16 rows: 128 rows x 64 k, 2 threads per row, 32 k (64 bytes) each
  // bf16 K-blocked: 4 blocks of 16 k; thread -> (block tid/64, rows 2*(tid%64), +1)
  const int b_row = tid >> 1;
  const int b_k = (tid & 1) * 32;

  f32x16 acc[NPROJ][2];
#pragma unroll
  for (int p = 0; p < NPROJ; ++p)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[p][c][i] = 0.0f;

  const int ksteps = P.K / BK;
  for (int ks = 0; ks < ksteps; ++ks) {
    const int k0 = ks * BK;
    // ---------------- global -> LDS: A
    {
      uint4 packed[2];
      if (a_src_f != nullptr) {
        const float4* src = (const float4*)(a_src_f + k0);
        const float4 v0 = ldg_f4(src), v1 = ldg_f4(src + 1), v2 = ldg_f4(src + 2), v3 = ldg_f4(src + 3);
        packed[0] = make_uint4(pack_bf16x2(v0.x, v0.y), pack_bf16x2(v0.z, v0.w), pack_bf16x2(v1.x, v1.y),
                               pack_bf16x2(v1.z, v1.w));
        packed[1] = make_uint4(pack_bf16x2(v2.x, v2.y), pack_bf16x2(v2.z, v2.w), pack_bf16x2(v3.x, v3.y),
                               pack_bf16x2(v3.z, v3.w));
      } else {
        const uint4* src = (const uint4*)(a_src_b + k0);
        packed[0] = ldg_u4(src);
        packed[1] = ldg_u4(src + 1);
      }
      uint4* dst = (uint4*)(As + a_row * LDA + a_k);
      dst[0] = packed[0];
      dst[1] = packed[1];
    }
    // ---------------- global -> LDS: B (dequantised)
#pragma unroll
    for (int p = 0; p < NPROJ; ++p) {
      uint16_t* Bp = Bs + p * BN * LDA;
      if constexpr (W == kInt8Rows) {
        const int n = t.n0 + b_row;
        const int8_t* src = (const int8_t*)P.p[p].w + ((int64_t)t.e * P.N + n) * P.K + k0 + b_k;
        const float s = ldg(P.p[p].s + ((int64_t)t.e * P.N + n) * P.groups + k0 / (P.K / P.groups));
        const int4 q0 = load_nt16(src);
        const int4 q1 = load_nt16(src + 16);
        const int qs[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        uint32_t o[16];
#pragma unroll
        for (int d = 0; d < 8; ++d) {
          const int v = qs[d];
          o[2 * d] = pack_bf16x2((float)(int8_t)v * s, (float)(int8_t)(v >> 8) * s);
          o[2 * d + 1] = pack_bf16x2((float)(int8_t)(v >> 16) * s, (float)(int8_t)(v >> 24) * s);
        }
        uint4* dst = (uint4*)(Bp + b_row * LDA + b_k);
#pragma unroll
        for (int d = 0; d < 4; ++d) dst[d] = make_uint4(o[4 * d], o[4 * d + 1], o[4 * d + 2], o[4 * d + 3]);
      } else if constexpr (W == kBf16Rows) {
        const int n = t.n0 + b_row;
        const uint4* src =
            (const uint4*)((const uint16_t*)P.p[p].w + ((int64_t)t.e * P.N + n) * P.K + k0 + b_k);
        uint4* dst = (uint4*)(Bp + b_row * LDA + b_k);
#pragma unroll
        for (int d = 0; d < 4; ++d) dst[d] = load_nt16u(src + d);
      } else {
        const int kb = tid >> 6;            // which 16-wide K block of the step
        const int nr = (tid & 63) * 2;      // two adjacent rows
        const uint4* src = (const uint4*)((const uint16_t*)P.p[p].w +
                                          ((int64_t)(k0 / 16 + kb) * P.N + t.n0 + nr) * 16);
        const uint4 r0 = load_nt16u(src), r1 = load_nt16u(src + 1);
        const uint4 r2 = load_nt16u(src + 2), r3 = load_nt16u(src + 3);
        uint4* d0 = (uint4*)(Bp + nr * LDA + kb * 16);
        uint4* d1 = (uint4*)(Bp + (nr + 1) * LDA + kb * 16);
        d0[0] = r0;
        d0[1] = r1;
        d1[0] = r2;
        d1[1] = r3;
      }
    }
    __syncthreads();
    // ---------------- MFMA over the step: 4 x k16
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      const int kofs = kk + (lane >> 5) * 8;
      const bf16x8 a = *(const bf16x8*)(As + (wm * 32 + (lane & 31)) * LDA + kofs);
#pragma unroll
      for (int p = 0; p < NPROJ; ++p) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const bf16x8 b = *(const bf16x8*)(Bs + p * BN * LDA + (wn * 64 + c * 32 + (lane & 31)) * LDA + kofs);
          acc[p][c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[p][c], 0, 0, 0);
        }
      }
    }
    __syncthreads();
  }

  // ---------------- epilogue: C[i][j], lane = j + 32*(i/4 % 2), reg = 4*(i/8) + i%4
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int col = t.n0 + wn * 64 + c * 32 + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      const int row = wm * 32 + i;
      if (row >= t.rows) continue;
      const int64_t orow = (int64_t)(t.pos0 + row);
      if constexpr (NPROJ == 2) {
        const float h = silu(acc[0][c][r]) * acc[1][c][r];
        stg(P.outb + orow * P.ldo + col, f32_to_bf16_rne(h));
      } else {
        stg(P.outf + orow * P.ldo + col, acc[0][c][r]);
      }
    }
  }
}

template <WKind W0, int NP, WKind W1>
__global__ void __launch_bounds__(kGemmThreads) k_gemm_pair(GemmProblem a, GemmProblem b, int split) {
  extern __shared__ uint16_t lds[];
  const int wg = (int)blockIdx.x;
  if (wg < split) {
    const TileRef t = locate(a, wg);
    if (!t.valid) return;
    gemm_tile<W0, NP>(a, t, lds);
  } else {
    const TileRef t = locate(b, wg - split);
    if (!t.valid) return;
    gemm_tile<W1, NP>(b, t, lds);
  }
}

}  // namespace

hipError_t launch_dequant(void* out, int out_f32, const int8_t* w, const float* scales, const int32_t* idx, int E,
                          int N, int K, int groups, int vec, hipStream_t s) {
  const int64_t total = (int64_t)N * K;
  if (total == 0) return hipSuccess;
  const int64_t blocks = (total + 8 * 256 - 1) / (8 * 256);
  UOCR_LAUNCH("dequant", k_dequant, dim3((unsigned)blocks), dim3(256), 0, s, out, out_f32, w, scales, idx, E, N, K,
                     groups, vec);
  return hipGetLastError();
}

int gemm_bm() { return BM; }
int gemm_bn() { return BN; }
int gemm_bk() { return BK; }

hipError_t launch_gemm_pair(const GemmProblem& routed, const GemmProblem& shared, int max_mtiles, hipStream_t s) {
  const int nproj = routed.swiglu ? 2 : 1;
  const int split = max_mtiles * (routed.N / BN);
  const int shared_wgs = ((shared.M + BM - 1) / BM) * (shared.N / BN);
  const int wgs = split + shared_wgs;
  if (wgs == 0) return hipSuccess;
  const size_t lds = (size_t)(BM + nproj * BN) * LDA * sizeof(uint16_t);
  const dim3 grid(wgs), block(kGemmThreads);
  if (routed.kind == kInt8Rows) {
    if (nproj == 2)
      UOCR_LAUNCH("gemm_gateup", (k_gemm_pair<kInt8Rows, 2, kBf16KBlocked>), grid, block, lds, s, routed, shared, split);
    else
      UOCR_LAUNCH("gemm_down", (k_gemm_pair<kInt8Rows, 1, kBf16KBlocked>), grid, block, lds, s, routed, shared, split);
  } else {
    if (nproj == 2)
      UOCR_LAUNCH("gemm_gateup", (k_gemm_pair<kBf16Rows, 2, kBf16KBlocked>), grid, block, lds, s, routed, shared, split);
    else
      UOCR_LAUNCH("gemm_down", (k_gemm_pair<kBf16Rows, 1, kBf16KBlocked>), grid, block, lds, s, routed, shared, split);
  }
  return hipGetLastError();
}

}  // namespace uocr
