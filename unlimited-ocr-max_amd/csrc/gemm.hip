// Prefill-shape expert contractions on the bf16 matrix cores, and the
// standalone int8 dequantisation op.
//
// Grouped GEMM: the routed rows are grouped by expert (route.hip).  Weights
// are dequantised with the reference's prefill numerics, w = bf16_rne(f32(q) *
// scale) (unlimited_ocr_max/kernels/moe_int8.mojo:340, the int8_dequant_expert
// values), activations rounded to bf16, and v_mfma_f32_32x32x16_bf16
// accumulates in fp32.  The gate/up launch fuses SwiGLU into its epilogue and
// writes h in bf16, already packed in group order, which is the down launch's
// A operand.  The shared experts (K-blocked bf16) ride in the same launches as
// extra tiles with every token as a row.
#include "uocr_device.h"
#include "uocr_kernels.h"

namespace uocr {

namespace {


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

// ------------------------------------------------------------- quantiser
//
// Symmetric per-group int8 along K (tools/quantize_int8.py:54-70,298-329): one
// wave per (row, group): amax = max |w| over the group (exact in any order),
// scale = amax / 127 (1.0 for an all-zero group), q = clip(rint(w / scale),
// +-127), every division correctly rounded fp32 and rint half to even -- the
// reference's numpy arithmetic, bit for bit.

__global__ void __launch_bounds__(256) k_quantize(int8_t* __restrict__ q, float* __restrict__ scales,
                                                  const void* __restrict__ w, int w_bf16, int64_t groups_total,
                                                  int group) {
  const int64_t gi = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (gi >= groups_total) return;
  const int l = lane_id();
  const int64_t base = gi * group;
  auto value = [&](int64_t i) -> float {
    return w_bf16 ? __uint_as_float((uint32_t)((const uint16_t*)w)[i] << 16) : ((const float*)w)[i];
  };
  float amax = 0.0f;
  for (int i = l; i < group; i += kWave) amax = fmaxf(amax, fabsf(value(base + i)));
  amax = tree_max(amax);
  const float s = amax == 0.0f ? 1.0f : amax / 127.0f;
  for (int i = l; i < group; i += kWave) {
    const float r = __builtin_rintf(value(base + i) / s);
    q[base + i] = (int8_t)(int)fminf(fmaxf(r, -127.0f), 127.0f);
  }
  if (l == 0) scales[gi] = s;
}

// ------------------------------------------------------------- grouped GEMM
//
// A workgroup owns a BM-row tile of one expert's rows (or of the tokens, for
// the shared experts) and 128 weight rows: 64 columns of both gate and up
// (SwiGLU launch) or 128 columns of down.  Its waves form a (BM/32) x 2 grid,
// each computing 32 rows x 32 columns of both projections (or 32 x 64 of
// down) with v_mfma_f32_32x32x16_bf16.  K advances in steps of BK = 128 (one
// int8 quantisation group of 128, or half of one of 256, ...): the raw global
// data of step k+1 (bf16 activations, int8 or bf16 weights and the step's
// scales) is loaded into registers while the matrix cores work on step k,
// then converted (weights to bf16_rne(f32(q) * scale)) into the single LDS
// tile.  Workgroups are dealt to XCDs so that all column tiles of one row
// tile run on the same XCD: the activation tile they share stays in its L2.

constexpr int BK = 128;
constexpr int kRow = BK + 8;   // bf16 per LDS row (272 bytes: rows 4 banks apart)
constexpr int kBRows = 128;    // weight rows per workgroup
constexpr int kWN = kBRows / 64;  // waves along the columns
constexpr int kXcds = 8;

template <int BM>
struct Geo {
  static constexpr int kWaves = BM / 32 * kWN;
  static constexpr int kThreads = kWaves * 64;
};

struct TileRef {
  int valid;
  int e;     // expert (routed) or 0
  int pos0;  // first row position of the tile (group order) or first token
  int rows;  // valid rows in the tile
  int n0;    // first output column
};

// The tile of workgroup `wg` of a problem with `mtiles` row tiles and `ntiles`
// column tiles of width bn: workgroup w runs on XCD w % 8, and XCD x takes
// the row tiles x, x+8, ... with all their column tiles in turn.
template <int BM>
__device__ TileRef locate(const GemmProblem& P, int wg, int bn) {
  TileRef t{0, 0, 0, 0, 0};
  const int ntiles = P.N / bn;
  const int x = wg % kXcds;
  const int j = wg / kXcds;  // the j-th workgroup of XCD x
  const int mt = x + kXcds * (j / ntiles);
  t.n0 = (j % ntiles) * bn;
  if (P.rows.n_groups == nullptr) {
    t.pos0 = mt * BM;
    if (t.pos0 >= P.M) return t;
    t.rows = min(BM, P.M - t.pos0);
    t.valid = 1;
    return t;
  }
  const int ng = ldc(P.rows.n_groups);
  if (mt >= ldc(P.tile_start + ng)) return t;
  int lo = 0, hi = ng - 1;  // the group g with tile_start[g] <= mt < tile_start[g + 1]
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (ldc(P.tile_start + mid) <= mt)
      lo = mid;
    else
      hi = mid - 1;
  }
  const int g = lo;
  const int start = ldc(P.rows.group_start + g);
  const int count = ldc(P.rows.group_start + g + 1) - start;
  const int local = mt - ldc(P.tile_start + g);
  t.e = ldc(P.rows.group_expert + g);
  t.pos0 = start + local * BM;
  t.rows = min(BM, count - local * BM);
  t.valid = 1;
  return t;
}

// Workgroups of a problem: row tiles rounded up to whole XCD rounds.
__host__ __device__ inline int grid_of(int mtiles, int ntiles) {
  return ((mtiles + kXcds - 1) / kXcds) * kXcds * ntiles;
}

// Raw global data of one K step, per thread.
template <int BM, WKind W>
struct StepRegs {
  static constexpr int kThreads = Geo<BM>::kThreads;
  static constexpr int kAParts = kThreads / BM;                     // threads per activation row (8)
  static constexpr int kABytes = BK * 2 / kAParts;                  // 32
  static constexpr int kBBytes = kBRows * BK * (W == kInt8Rows ? 1 : 2) / kThreads;
  i32x4 a[kABytes / 16];
  i32x4 b[kBBytes / 16];
  float scale;
};

// Per-thread global cursors of a tile, set up once: the activation row, the
// weight row (or K-blocked column run) and, for int8, the scale of the
// thread's piece together with its position inside the quantisation group.
struct Cursor {
  const uint16_t* a;
  const char* b;
  const float* s;
  int grem;   // K offset of the piece inside its group (groups wider than a step)
  int gwrap;  // group width when wider than a step, else never reached
  int sinc;   // scales per step when a step spans whole groups
};

template <int BM, WKind W, int NPROJ>
__device__ __forceinline__ Cursor make_cursor(const GemmProblem& P, const TileRef& t, const uint16_t* a_src) {
  using S = StepRegs<BM, W>;
  constexpr int T = S::kThreads;
  const int tid = (int)threadIdx.x;
  Cursor c;
  c.a = a_src;
  c.s = nullptr;
  c.grem = 0;
  c.gwrap = 0x7fffffff;
  c.sinc = 0;
  // the projection's pointers, selected without indexing the argument block
  const void* w0 = P.p[0].w;
  const void* w1 = NPROJ == 2 ? P.p[1].w : w0;
  if constexpr (W == kBf16KBlocked) {
    // K-blocked [K/16][N][16]: 8 blocks x kBRows rows x 32 bytes per step;
    // thread -> block, consecutive rows (contiguous in memory)
    constexpr int kRowsPer = kBRows * 8 / T;
    constexpr int kPerBlock = kBRows / kRowsPer;
    const int kb = tid / kPerBlock;
    const int r0 = (tid % kPerBlock) * kRowsPer;
    const int half = kBRows / NPROJ;
    const bool second = NPROJ == 2 && r0 >= half;
    const int n = t.n0 + (NPROJ == 2 ? r0 % half : r0);
    c.b = (const char*)(second ? w1 : w0) + ((int64_t)kb * P.N + n) * 32;
  } else {
    constexpr int kParts = T / kBRows;  // threads per weight row
    const int row = tid / kParts;
    const int part = tid % kParts;
    const int half = kBRows / NPROJ;
    const bool second = NPROJ == 2 && row >= half;
    const int n = t.n0 + (NPROJ == 2 ? row % half : row);
    constexpr int kEsz = W == kInt8Rows ? 1 : 2;
    c.b = (const char*)(second ? w1 : w0) + ((int64_t)t.e * P.N + n) * P.K * kEsz + part * S::kBBytes;
    if constexpr (W == kInt8Rows) {
      const float* s0 = P.p[0].s;
      const float* s1 = NPROJ == 2 ? P.p[1].s : s0;
      // group widths are multiples of 64 that divide or are multiples of BK
      const int gsize = P.K / P.groups;
      const int kk = part * S::kBBytes;
      c.s = (second ? s1 : s0) + ((int64_t)t.e * P.N + n) * P.groups + kk / gsize;
      if (gsize <= BK) {
        c.sinc = BK / gsize;
      } else {
        c.gwrap = gsize;
        c.grem = kk % gsize;
      }
    }
  }
  return c;
}

// 16 weight bytes at any alignment (the caller's stack may start anywhere):
// the compiler splits the copy into loads the pointer's alignment allows.
__device__ __forceinline__ i32x4 ld16_any(const char* p) {
  i32x4 v;
  __builtin_memcpy(&v, (const UOCR_GLOBAL char*)p, 16);
  return v;
}

// Loads one K step at the cursor into registers.  VEC: the weights are
// 16-byte aligned (one 16-byte load per piece); else each piece is read at
// whatever alignment it has -- the same bytes either way.
template <int BM, WKind W, int NPROJ, bool VEC>
__device__ __forceinline__ void load_step(const Cursor& c, StepRegs<BM, W>& R) {
  using S = StepRegs<BM, W>;
#pragma unroll
  for (int i = 0; i < S::kABytes / 16; ++i) R.a[i] = *(const UOCR_GLOBAL i32x4*)(c.a + 8 * i);
  constexpr int NB = S::kBBytes / 16;
#pragma unroll
  for (int i = 0; i < NB; ++i)
    R.b[i] = VEC ? *(const UOCR_GLOBAL i32x4*)(c.b + 16 * i) : ld16_any(c.b + 16 * i);
  if constexpr (W == kInt8Rows) R.scale = ldg(c.s);
}

// Moves the cursor one K step on when `more` (else it stays on the last step,
// whose data a repeated load finds in cache).
template <WKind W>
__device__ __forceinline__ void advance(const GemmProblem& P, Cursor& c, bool more) {
  c.a += more ? BK : 0;
  if constexpr (W == kBf16KBlocked) {
    c.b += more ? (int64_t)8 * P.N * 32 : 0;  // the thread's K-block, 8 blocks on
  } else {
    c.b += more ? BK * (W == kInt8Rows ? 1 : 2) : 0;
    if constexpr (W == kInt8Rows) {
      const int grem = c.grem + (more ? BK : 0);
      const bool wrap = grem >= c.gwrap;
      c.s += (more ? c.sinc : 0) + (wrap ? 1 : 0);
      c.grem = wrap ? grem - c.gwrap : grem;
    }
  }
}

template <int BM, WKind W>
__device__ __forceinline__ void store_step(const StepRegs<BM, W>& R, uint16_t* As, uint16_t* Bs) {
  using S = StepRegs<BM, W>;
  constexpr int T = S::kThreads;
  const int tid = (int)threadIdx.x;
  {
    i32x4* dst = (i32x4*)(As + (tid / S::kAParts) * kRow + (tid % S::kAParts) * (S::kABytes / 2));
#pragma unroll
    for (int i = 0; i < S::kABytes / 16; ++i) dst[i] = R.a[i];
  }
  constexpr int NB = S::kBBytes / 16;
  if constexpr (W == kBf16KBlocked) {
    constexpr int kRowsPer = kBRows * 8 / T;
    constexpr int kPerBlock = kBRows / kRowsPer;
    const int kb = tid / kPerBlock;
    const int r0 = (tid % kPerBlock) * kRowsPer;
#pragma unroll
    for (int i = 0; i < NB; ++i) *(i32x4*)(Bs + (r0 + i / 2) * kRow + kb * 16 + (i & 1) * 8) = R.b[i];
  } else if constexpr (W == kBf16Rows) {
    constexpr int kParts = T / kBRows;
    const int row = tid / kParts, part = tid % kParts;
    i32x4* dst = (i32x4*)(Bs + row * kRow + part * (BK / kParts));
#pragma unroll
    for (int i = 0; i < NB; ++i) dst[i] = R.b[i];
  } else {
    // int8: 16 weights per piece -> 2 x 16 bytes of bf16
    constexpr int kParts = T / kBRows;
    const int row = tid / kParts, part = tid % kParts;
    i32x4* dst = (i32x4*)(Bs + row * kRow + part * (BK / kParts));
    const float s = R.scale;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      uint32_t o[8];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int v = R.b[i][d];
        o[2 * d] = pack_bf16x2(i8_to_f32<0>(v) * s, i8_to_f32<1>(v) * s);
        o[2 * d + 1] = pack_bf16x2(i8_to_f32<2>(v) * s, i8_to_f32<3>(v) * s);
      }
      dst[2 * i] = i32x4{(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
      dst[2 * i + 1] = i32x4{(int)o[4], (int)o[5], (int)o[6], (int)o[7]};
    }
  }
}

// silu(g) * u for the prefill epilogue: v_exp_f32 and v_rcp_f32 (within a
// couple of ulp of the correctly rounded value, far below the bf16 rounding
// of h that follows; the prefill is held to a tolerance, the decode path
// keeps its exactly specified silu).
__device__ __forceinline__ float swiglu_fast(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(-g * 1.44269504088896341f);
  return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

template <int BM, WKind W, int NPROJ, bool VEC>
__device__ void gemm_tile(const GemmProblem& P, const TileRef& t, uint16_t* lds) {
  using S = StepRegs<BM, W>;
  uint16_t* As = lds;               // [BM][kRow]
  uint16_t* Bs = lds + BM * kRow;   // [kBRows][kRow]
  const int tid = (int)threadIdx.x;
  const int lane = lane_id();
  const int w = tid >> 6;
  const int wm = w / kWN;  // 32-row slice
  const int wn = w % kWN;  // column slice

  // this thread's activation row (padded rows repeat the last real one)
  const int a_pos = t.pos0 + min(tid / S::kAParts, t.rows - 1);
  const int a_row =
      (P.a_by_token && P.rows.n_groups != nullptr) ? ldg(P.rows.group_rows + a_pos) / P.x_div : a_pos;
  const uint16_t* a_src = P.a + (int64_t)a_row * P.lda + (tid % S::kAParts) * (S::kABytes / 2);
  Cursor cur = make_cursor<BM, W, NPROJ>(P, t, a_src);

  f32x16 acc[2];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[c][i] = 0.0f;
  // LDS rows of this wave's two 32-column B tiles
  const int brow0 = NPROJ == 2 ? wn * 32 : wn * 64;
  const int brow1 = NPROJ == 2 ? kBRows / 2 + wn * 32 : wn * 64 + 32;

  // One K step of raw global data in flight: step ks + 1 is loaded into
  // registers right after step ks has been stored from them, and lands while
  // the matrix cores work on step ks (the barriers order LDS only, so they
  // do not wait for it).
  S R;
  const int ksteps = P.K / BK;
  load_step<BM, W, NPROJ, VEC>(cur, R);
  advance<W>(P, cur, ksteps > 1);
  for (int ks = 0; ks < ksteps; ++ks) {
    if (ks > 0) lds_barrier();
    store_step<BM, W>(R, As, Bs);
    if (ks + 1 < ksteps) {
      load_step<BM, W, NPROJ, VEC>(cur, R);
      advance<W>(P, cur, ks + 2 < ksteps);
    }
    lds_barrier();
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      const int kofs = kk + (lane >> 5) * 8;
      const bf16x8 a = *(const bf16x8*)(As + (wm * 32 + (lane & 31)) * kRow + kofs);
      const bf16x8 b0 = *(const bf16x8*)(Bs + (brow0 + (lane & 31)) * kRow + kofs);
      const bf16x8 b1 = *(const bf16x8*)(Bs + (brow1 + (lane & 31)) * kRow + kofs);
      acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b0, acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b1, acc[1], 0, 0, 0);
    }
  }

  // ---------------- epilogue: C[i][j], lane = j + 32*(i/4 % 2), reg = 4*(i/8) + i%4
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int i = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    const int row = wm * 32 + i;
    if (row >= t.rows) continue;
    const int64_t orow = (int64_t)(t.pos0 + row);
    if constexpr (NPROJ == 2) {
      const int col = t.n0 + wn * 32 + (lane & 31);
      stg(P.outb + orow * P.ldo + col, f32_to_bf16_rne(swiglu_fast(acc[0][r], acc[1][r])));
    } else {
      const int col = t.n0 + wn * 64 + (lane & 31);
      stg(P.outf + orow * P.ldo + col, acc[0][r]);
      stg(P.outf + orow * P.ldo + col + 32, acc[1][r]);
    }
  }
}

template <int BM, WKind W0, int NP, WKind W1, bool VEC>
__global__ void __launch_bounds__(Geo<BM>::kThreads) k_gemm_pair(GemmProblem a, GemmProblem b, int split) {
  extern __shared__ uint16_t lds[];
  constexpr int bn = kBRows / NP;
  const int wg = (int)blockIdx.x;
  if (wg < split) {
    const TileRef t = locate<BM>(a, wg, bn);
    if (!t.valid) return;
    gemm_tile<BM, W0, NP, VEC>(a, t, lds);
  } else {
    const TileRef t = locate<BM>(b, wg - split, bn);
    if (!t.valid) return;
    gemm_tile<BM, W1, NP, VEC>(b, t, lds);
  }
}

template <int BM, WKind W0, int NP, bool VEC = true>
hipError_t launch_pair_bm(const GemmProblem& routed, const GemmProblem& shared, int max_mtiles, hipStream_t s,
                          const char* name) {
  constexpr int bn = kBRows / NP;
  const int split = grid_of(max_mtiles, routed.N / bn);
  const int shared_wgs = grid_of((shared.M + BM - 1) / BM, shared.N / bn);
  const int wgs = split + shared_wgs;
  if (wgs == 0) return hipSuccess;
  const size_t lds = (size_t)(BM + kBRows) * kRow * sizeof(uint16_t);
  UOCR_LAUNCH(name, (k_gemm_pair<BM, W0, NP, kBf16KBlocked, VEC>), dim3(wgs), dim3(Geo<BM>::kThreads), lds, s, routed,
              shared, split);
  return hipGetLastError();
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

hipError_t launch_quantize(int8_t* q, float* scales, const void* w, int w_bf16, int64_t groups_total, int group,
                           hipStream_t s) {
  if (groups_total == 0) return hipSuccess;
  UOCR_LAUNCH("quantize", k_quantize, dim3((unsigned)((groups_total + 3) / 4)), dim3(256), 0, s, q, scales, w, w_bf16,
              groups_total, group);
  return hipGetLastError();
}

int gemm_bk() { return BK; }

hipError_t launch_gemm_pair(const GemmProblem& routed, const GemmProblem& shared, int bm, int max_mtiles,
                            hipStream_t s, bool vec) {
  const bool gu = routed.swiglu != 0;
  const char* name = gu ? "gemm_gateup" : "gemm_down";
  if (!vec) {  // weights at any alignment: 64-row tiles only
    if (bm != 64) return hipErrorInvalidValue;
    if (routed.kind == kInt8Rows)
      return gu ? launch_pair_bm<64, kInt8Rows, 2, false>(routed, shared, max_mtiles, s, name)
                : launch_pair_bm<64, kInt8Rows, 1, false>(routed, shared, max_mtiles, s, name);
    return gu ? launch_pair_bm<64, kBf16Rows, 2, false>(routed, shared, max_mtiles, s, name)
              : launch_pair_bm<64, kBf16Rows, 1, false>(routed, shared, max_mtiles, s, name);
  }
  if (bm == 128) {
    if (routed.kind == kInt8Rows)
      return gu ? launch_pair_bm<128, kInt8Rows, 2>(routed, shared, max_mtiles, s, name)
                : launch_pair_bm<128, kInt8Rows, 1>(routed, shared, max_mtiles, s, name);
    return gu ? launch_pair_bm<128, kBf16Rows, 2>(routed, shared, max_mtiles, s, name)
              : launch_pair_bm<128, kBf16Rows, 1>(routed, shared, max_mtiles, s, name);
  }
  if (routed.kind == kInt8Rows)
    return gu ? launch_pair_bm<64, kInt8Rows, 2>(routed, shared, max_mtiles, s, name)
              : launch_pair_bm<64, kInt8Rows, 1>(routed, shared, max_mtiles, s, name);
  return gu ? launch_pair_bm<64, kBf16Rows, 2>(routed, shared, max_mtiles, s, name)
            : launch_pair_bm<64, kBf16Rows, 1>(routed, shared, max_mtiles, s, name);
}

}  // namespace uocr
