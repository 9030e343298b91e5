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
//
// Two kernels share the tiling: the LDS-staged one (16-byte aligned weights,
// the product path) and the fragment-load one (weights at any alignment);
// both run the same MFMA sequence on the same values, so they give the same
// bits.  On gfx950 the int8 dequantisation (a conversion, a multiply and half
// a pack per weight, once per row tile) issues in turn with the MFMAs on a
// SIMD -- a second wave does not overlap them -- so the int8 kernels are
// bounded by that issue time; the tiles are sized to spread each dequantised
// weight over as many rows as the expert has (up to 128).
#include <atomic>

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
// C[rows, cols] = A[rows, K] . W[cols, K]^T with v_mfma_f32_32x32x16_bf16
// (fp32 accumulation): A is bf16 (the gathered x rows for gate/up, h in group
// order for down, the tokens for the shared experts), W one expert's weight
// rows (int8 + per-group scales, bf16, or the shared experts' K-blocked bf16).
//
// Tile.  A workgroup of 4 waves owns BM rows x 256 weight rows.  Wave w owns
// weight rows [64w, 64w + 64) as two 32-row MFMA blocks, against all BM rows:
// every weight is loaded and dequantised by exactly one wave, once per row
// tile, and each dequantised fragment feeds BM/32 x 2 MFMAs.  The
// fragment-load kernel (below) reads the weights straight into B-operand
// registers; the LDS-staged kernel (further below) streams them through LDS.  In the gate/up launch block 0
// holds gate columns n0 + 32w .. +32 and block 1 the same up columns, so
// SwiGLU pairs the registers of one lane.  K advances in steps of 64: the A
// step (BM x 64 bf16) goes global -> registers -> LDS (two buffers, one
// barrier per step; 16-byte chunks XOR-swizzled by row so that the fragment
// reads are free of bank conflicts); the weight and A steps are both loaded
// kWStages steps ahead.  Inside a step, lane half h covers
// k = 32h .. 32h + 31 in both operands: the MFMA's k order is a permutation of
// the step's 64, the same for A and W.
//
// Placement.  A problem's tiles are (group, column tile, row tile).  Each
// group's column tiles are cut into ranges (two per routed expert, up to
// eight for the shared experts); range r of the problem goes to XCD r % 8,
// whose workgroups walk their XCD's tiles range by range, row tile major and
// column tile minor.  A range's weight tiles are fetched into one L2 and serve
// all of its row tiles there, and an A row tile serves the range's column
// tiles back to back.  The grid is persistent (a fixed number of workgroups
// per XCD strides through that XCD's list), so no bound on the routing is
// needed at launch.

constexpr int BK = 64;                    // K per step
constexpr int kGThreads = 256;            // 4 waves
constexpr int kXcds = 8;
constexpr int kWRowsWave = 64;            // weight rows per wave
constexpr int kWRowsWg = 4 * kWRowsWave;  // weight rows per workgroup

template <WKind W>
constexpr int kWStages = W == kInt8Rows ? 4 : 2;  // weight steps in flight

struct TileRef {
  int e;     // expert (routed), or the K range of a dense problem in K ranges (else 0)
  int pos0;  // first row position (group order) or first token
  int rows;  // valid rows
  int n0;    // first output column
};

// K ranges of a problem (a dense K-blocked one may be cut into kparts).
__host__ __device__ __forceinline__ int parts_of(const GemmProblem& P) {
  return P.kind == kBf16KBlocked && P.kparts > 1 ? P.kparts : 1;
}

// K range r of a K-blocked problem ([K / 16][N][16] bf16 weights) as a
// problem of its own: K / parts, the operands from the range's first k, the
// sums at outf + r * part_stride.
__device__ __forceinline__ GemmProblem part_problem(const GemmProblem& P, int r) {
  GemmProblem Q = P;
  const int kr = P.K / parts_of(P);
  Q.K = kr;
  Q.kparts = 1;
  Q.a = P.a + (int64_t)r * kr;
  Q.p[0].w = (const char*)P.p[0].w + (int64_t)r * (kr / 16) * P.N * 32;
  Q.outf = P.outf + r * P.part_stride;
  return Q;
}

// The cut of a problem's column tiles into ranges.
struct Plan {
  int nt;   // column tiles
  int per;  // column tiles per range
  int nr;   // ranges per group
  int ng;   // groups
};

__device__ __forceinline__ Plan plan_of(const GemmProblem& P, int bn) {
  Plan p;
  const bool routed = P.rows.n_groups != nullptr;
  p.nt = (P.N + bn - 1) / bn;
  p.per = routed ? (p.nt + 1) / 2 : (p.nt + kXcds - 1) / kXcds;
  p.nr = (p.nt + p.per - 1) / p.per;
  p.ng = routed ? ldc(P.rows.n_groups) : (P.M > 0 ? 1 : 0);
  return p;
}

template <int BM>
__device__ __forceinline__ int row_tiles(const GemmProblem& P, int g) {
  if (P.rows.n_groups == nullptr) return (P.M + BM - 1) / BM;
  return (ldg(P.rows.group_start + g + 1) - ldg(P.rows.group_start + g) + BM - 1) / BM;
}

// Lane q: the inclusive prefix of the tile counts of XCD x's ranges x, x + 8,
// ... (range r: group r / nr, column tiles from (r % nr) * per); the host
// keeps ng * nr <= 8 * 64.
template <int BM>
__device__ int xcd_prefix(const GemmProblem& P, const Plan& p, int x) {
  const int q = lane_id();
  const int r = x + kXcds * q;
  int n = 0;
  if (r < p.ng * p.nr) {
    const int g = r / p.nr;
    const int c = r - g * p.nr;
    n = row_tiles<BM>(P, g) * min(p.per, p.nt - c * p.per);
  }
  return wave_scan_i(n);
}

// Tile `it` of XCD x's list (prefix from xcd_prefix).
template <int BM>
__device__ TileRef tile_at(const GemmProblem& P, const Plan& p, int x, int prefix, int it, int bn) {
  const int q = (int)__popcll(__ballot(prefix <= it));
  const int before = q > 0 ? __builtin_amdgcn_readlane(prefix, q - 1) : 0;
  const int r = x + kXcds * q;
  const int g = r / p.nr;
  const int c = r - g * p.nr;
  const int cols = min(p.per, p.nt - c * p.per);
  const int local = it - before;
  const int mt = local / cols;
  TileRef t;
  t.n0 = (c * p.per + local - mt * cols) * bn;
  if (P.rows.n_groups == nullptr) {
    t.e = 0;
    t.pos0 = mt * BM;
    t.rows = min(BM, P.M - t.pos0);
  } else {
    const int start = ldg(P.rows.group_start + g);
    const int count = ldg(P.rows.group_start + g + 1) - start;
    t.e = ldg(P.rows.group_expert + g);
    t.pos0 = start + mt * BM;
    t.rows = min(BM, count - mt * BM);
  }
  return t;
}

// 16 weight bytes at any alignment (the caller's stack may start anywhere):
// the compiler splits the copy into loads the pointer's alignment allows.
__device__ __forceinline__ i32x4 ld16_any(const char* p) {
  i32x4 v;
  __builtin_memcpy(&v, (const UOCR_GLOBAL char*)p, 16);
  return v;
}
template <bool VEC>
__device__ __forceinline__ i32x4 ld16w(const char* p) {
  if constexpr (VEC) return *(const UOCR_GLOBAL i32x4*)p;
  else return ld16_any(p);
}

// One K step of one wave's weights, per lane: the 32 k of the lane's column
// in each block (16-byte pieces), and for int8 the step's scale of each.
template <WKind W>
struct WStep {
  static constexpr int kPieces = W == kInt8Rows ? 2 : 4;
  i32x4 v[2][kPieces];
  float s[2];
};

// The lane's weight addresses at step 0.
struct WCursor {
  const char* p[2];
  const float* s[2];
  int64_t step;     // bytes per K step
  int64_t kblock;   // K-blocked: bytes from one 16-k block to the next
  float spg_inv;    // int8: BK / group width (steps per group, inverted)
};

template <WKind W, int NPROJ>
__device__ __forceinline__ WCursor wcursor(const GemmProblem& P, const TileRef& t, int w, int l) {
  const int m = l & 31, h = l >> 5;
  WCursor c;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    // a block past the last column reads the last row; its results are not stored
    const int row = min(NPROJ == 2 ? t.n0 + 32 * w + m : t.n0 + 64 * w + 32 * b + m, P.N - 1);
    const char* base = (const char*)(NPROJ == 2 && b == 1 ? P.p[1].w : P.p[0].w);
    const int64_t wrow = (int64_t)t.e * P.N + row;
    if constexpr (W == kInt8Rows) {
      c.p[b] = base + wrow * P.K + 32 * h;
      c.s[b] = (NPROJ == 2 && b == 1 ? P.p[1].s : P.p[0].s) + wrow * P.groups;
    } else if constexpr (W == kBf16Rows) {
      c.p[b] = base + (wrow * P.K + 32 * h) * 2;
      c.s[b] = nullptr;
    } else {
      c.p[b] = base + ((int64_t)(2 * h) * P.N + row) * 32;  // [K/16][N][16]: k-block 2h of step 0
      c.s[b] = nullptr;
    }
  }
  c.kblock = (int64_t)P.N * 32;
  c.step = W == kInt8Rows ? BK : W == kBf16Rows ? 2 * BK : (BK / 16) * c.kblock;
  c.spg_inv = W == kInt8Rows ? (float)BK * (float)P.groups / (float)P.K : 0.0f;
  return c;
}

template <WKind W, bool VEC>
__device__ __forceinline__ void load_w(const WCursor& c, int k, WStep<W>& o) {
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const char* q = c.p[b] + (int64_t)k * c.step;
    if constexpr (W == kBf16KBlocked) {
      o.v[b][0] = ld16w<VEC>(q);
      o.v[b][1] = ld16w<VEC>(q + 16);
      o.v[b][2] = ld16w<VEC>(q + c.kblock);
      o.v[b][3] = ld16w<VEC>(q + c.kblock + 16);
    } else {
#pragma unroll
      for (int i = 0; i < WStep<W>::kPieces; ++i) o.v[b][i] = ld16w<VEC>(q + 16 * i);
    }
    if constexpr (W == kInt8Rows) {
      // the step lies in group k / (steps per group); k < 2^16, so the float
      // quotient of k + 1/2 truncates to it exactly
      o.s[b] = ldg(c.s[b] + (int)(((float)k + 0.5f) * c.spg_inv));
    }
  }
}

// The B fragment of block b for k sub-step `sub` (8 k per lane): int8 weights
// become bf16_rne(f32(q) * scale), the reference's dequantised values.
template <WKind W>
__device__ __forceinline__ bf16x8 wfrag(const WStep<W>& S, int b, int sub) {
  if constexpr (W == kInt8Rows) {
    const i32x4 piece = S.v[b][sub >> 1];
    const int d0 = piece[(sub & 1) * 2], d1 = piece[(sub & 1) * 2 + 1];
    const float s = S.s[b];
    i32x4 o;
    o[0] = (int)pack_bf16x2(i8_to_f32<0>(d0) * s, i8_to_f32<1>(d0) * s);
    o[1] = (int)pack_bf16x2(i8_to_f32<2>(d0) * s, i8_to_f32<3>(d0) * s);
    o[2] = (int)pack_bf16x2(i8_to_f32<0>(d1) * s, i8_to_f32<1>(d1) * s);
    o[3] = (int)pack_bf16x2(i8_to_f32<2>(d1) * s, i8_to_f32<3>(d1) * s);
    return __builtin_bit_cast(bf16x8, o);
  } else {
    return __builtin_bit_cast(bf16x8, S.v[b][sub]);
  }
}

// The thread's share of one A step: chunk (tid & 7) of rows (tid >> 3) + 32j.
template <int BM>
struct AStep {
  i32x4 v[BM / 32];
};

template <int BM>
__device__ __forceinline__ void load_a(const uint16_t* a, const int (&off)[BM / 32], int k, AStep<BM>& o) {
#pragma unroll
  for (int j = 0; j < BM / 32; ++j) o.v[j] = *(const UOCR_GLOBAL i32x4*)(a + off[j] + k * BK);
}

// The stored position of a row's 16-byte chunk c is c ^ swz(row): any 8
// consecutive rows, and any 16 (their two 128-byte halves fill a 256-byte
// bank cycle), put the chunk in different banks.
__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

template <int BM>
__device__ __forceinline__ void store_a(const AStep<BM>& o, uint16_t* buf) {
  const int tid = (int)threadIdx.x;
  const int r = tid >> 3, c = tid & 7;
#pragma unroll
  for (int j = 0; j < BM / 32; ++j) *(i32x4*)(buf + (r + 32 * j) * BK + 8 * (c ^ swz(r))) = o.v[j];
}

// One K step: 4 sub-steps of 16 k, each BM/32 x 2 MFMAs.  The A fragments
// of sub-step k + 1 are read from LDS before the MFMAs of sub-step k issue.
template <int BM, WKind W>
__device__ __forceinline__ void mfma_step(f32x16 (&acc)[BM / 32][2], const uint16_t* As, const WStep<W>& ws, int m,
                                          int h) {
  constexpr int MB = BM / 32;
  const uint16_t* row = As + m * BK;  // row 32i + m has the swizzle of m
  const int sw = swz(m);
  bf16x8 a[2][MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) a[0][i] = *(const bf16x8*)(row + 32 * i * BK + 8 * ((4 * h) ^ sw));
#pragma unroll
  for (int sub = 0; sub < 4; ++sub) {
    if (sub < 3) {
#pragma unroll
      for (int i = 0; i < MB; ++i)
        a[(sub + 1) & 1][i] = *(const bf16x8*)(row + 32 * i * BK + 8 * ((4 * h + sub + 1) ^ sw));
    }
    const bf16x8 b0 = wfrag<W>(ws, 0, sub);
    const bf16x8 b1 = wfrag<W>(ws, 1, sub);
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[sub & 1][i], b0, acc[i][0], 0, 0, 0);
      acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[sub & 1][i], b1, acc[i][1], 0, 0, 0);
    }
  }
}

// The per-tile pipeline state: NS steps of weights and of A in flight in
// registers, the accumulators.
template <int BM, WKind W>
struct Pipe {
  static constexpr int MB = BM / 32;
  static constexpr int NS = kWStages<W>;
  WStep<W> ws[NS];
  AStep<BM> as[NS];
  f32x16 acc[MB][2];
};

// Step s = round start + u of the main loop.  Vector loads complete in issue
// order, so waiting for one load waits for every earlier one: the weights
// and A of step s + NS are both issued during step s, and every wait targets
// loads issued NS - 1 or more steps earlier.  The loads' step index is
// clamped to the last step (re-reading it is harmless), so the loop body has
// no branches and the compiler's waits stay exact.
template <int u, int BM, WKind W, bool VEC>
__device__ __forceinline__ void pipe_step(Pipe<BM, W>& p, const GemmProblem& P, const int (&aoff)[BM / 32],
                                          const WCursor& cur, uint16_t* lds, int s, int S, int m, int h) {
  constexpr int NS = Pipe<BM, W>::NS;
  load_a<BM>(P.a, aoff, min(s + NS, S - 1), p.as[u % NS]);  // as[u % NS] held step s, already in LDS
  mfma_step<BM, W>(p.acc, lds + (u & 1) * BM * BK, p.ws[u % NS], m, h);
  load_w<W, VEC>(cur, min(s + NS, S - 1), p.ws[u % NS]);
  // the other buffer was last read in step s - 1, before the barrier that ended it
  store_a<BM>(p.as[(u + 1) % NS], lds + ((u + 1) & 1) * BM * BK);
  lds_barrier();
}

// silu(g) * u for the prefill epilogue: v_exp_f32 and v_rcp_f32 (within a
// couple of ulp of the correctly rounded value, far below the bf16 rounding
// of h that follows; the prefill is held to a tolerance, the decode path
// keeps its exactly specified silu).
__device__ __forceinline__ float swiglu_fast(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(-g * 1.44269504088896341f);
  return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// v[0..3] of the 4 lanes of a quad (qd = lane & 3) as a 4 x 4 matrix, lane
// qd holding row qd, transposed in place: afterwards lane qd holds column qd
// (v[j] = what lane j held in v[qd]).  Two rounds of DPP exchanges (lanes
// qd ^ 2, then qd ^ 1); moves only, the values are not altered.
__device__ __forceinline__ void quad_transpose(float (&v)[4], int qd) {
  const bool lo = (qd & 2) == 0;
  const float s0 = lo ? v[2] : v[0], s1 = lo ? v[3] : v[1];
  const float r0 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s0), 0x4E, 0xf, 0xf, false));
  const float r1 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s1), 0x4E, 0xf, 0xf, false));
  if (lo) {
    v[2] = r0;
    v[3] = r1;
  } else {
    v[0] = r0;
    v[1] = r1;
  }
  const bool ev = (qd & 1) == 0;
  const float t0 = ev ? v[1] : v[0], t1 = ev ? v[3] : v[2];
  const float u0 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t0), 0xB1, 0xf, 0xf, false));
  const float u1 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t1), 0xB1, 0xf, 0xf, false));
  if (ev) {
    v[1] = u0;
    v[3] = u1;
  } else {
    v[0] = u0;
    v[2] = u1;
  }
}

// The tile's outputs.  C[i][j] of a 32 x 32 MFMA block sits in lane
// j + 32 * (i / 4 % 2), register 4 * (i / 8) + i % 4: lane (m, h) holds column
// m, rows 8 k + 4 h + q in registers 4 k + q.  A 4 x 4 transpose inside each
// quad of lanes (m = 4 c + q') gives lane q' of the quad row 8 k + 4 h + q',
// columns 4 c .. 4 c + 3: one 8-byte (bf16) or 16-byte (fp32) store where the
// MFMA layout needs four (scattered 2- and 4-byte stores took 20-30 k cycles a
// 256 x 256 tile and slowed the loads queued behind them).  Gate/up: h rows in
// bf16, silu(gate) * up of the two blocks; down: fp32 rows.
template <int BM, int NPROJ>
__device__ __forceinline__ void store_tile(const GemmProblem& P, const TileRef& t, const f32x16 (&acc)[BM / 32][2],
                                           int w, int m, int h) {
  const int qd = m & 3;
#pragma unroll
  for (int ib = 0; ib < BM / 32; ++ib) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int row = 32 * ib + 8 * k + 4 * h + qd;
      const bool live = row < t.rows;
      const int64_t orow = (int64_t)(t.pos0 + row);
      if constexpr (NPROJ == 2) {
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = swiglu_fast(acc[ib][0][4 * k + q], acc[ib][1][4 * k + q]);
        quad_transpose(v, qd);
        const int col = t.n0 + 32 * w + (m & ~3);
        if (live && col < P.N) {
          const uint64_t o = (uint64_t)pack_bf16x2(v[0], v[1]) | ((uint64_t)pack_bf16x2(v[2], v[3]) << 32);
          *(UOCR_GLOBAL uint64_t*)(P.outb + orow * P.ldo + col) = o;
        }
      } else {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = acc[ib][b][4 * k + q];
          quad_transpose(v, qd);
          const int col = t.n0 + 64 * w + 32 * b + (m & ~3);
          if (live && col < P.N) *(UOCR_GLOBAL f32x4*)(P.outf + orow * P.ldo + col) = f32x4{v[0], v[1], v[2], v[3]};
        }
      }
    }
  }
}

template <int BM, WKind W, int NPROJ, bool VEC>
__device__ void gemm_tile(const GemmProblem& P, const TileRef& t, uint16_t* lds) {
  constexpr int MB = BM / 32;
  constexpr int NS = kWStages<W>;
  const int tid = (int)threadIdx.x;
  const int l = lane_id();
  const int w = tid >> 6;
  const int m = l & 31, h = l >> 5;
  const int S = P.K / BK;

  // this thread's A rows (padded rows repeat the last real one)
  int aoff[MB];
#pragma unroll
  for (int j = 0; j < MB; ++j) {
    const int pos = t.pos0 + min((tid >> 3) + 32 * j, t.rows - 1);
    const int row = (P.a_by_token && P.rows.n_groups != nullptr) ? ldg(P.rows.group_rows + pos) / P.x_div : pos;
    aoff[j] = (int)((int64_t)row * P.lda) + 8 * (tid & 7);
  }
  const WCursor cur = wcursor<W, NPROJ>(P, t, w, l);

  Pipe<BM, W> p;
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) p.acc[i][0][r] = p.acc[i][1][r] = 0.0f;
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    load_a<BM>(P.a, aoff, min(i, S - 1), p.as[i]);
    load_w<W, VEC>(cur, min(i, S - 1), p.ws[i]);
  }
  store_a<BM>(p.as[0], lds);
  lds_barrier();
  // S is even (K is a multiple of 2 * BK): full rounds of NS steps, then the
  // remaining S % NS (0 or 2) steps, whose data the last round loaded
  const int rounds = S / NS;
  for (int rd = 0; rd < rounds; ++rd) {
    const int s = rd * NS;
    pipe_step<0, BM, W, VEC>(p, P, aoff, cur, lds, s, S, m, h);
    pipe_step<1, BM, W, VEC>(p, P, aoff, cur, lds, s + 1, S, m, h);
    if constexpr (NS == 4) {
      pipe_step<2, BM, W, VEC>(p, P, aoff, cur, lds, s + 2, S, m, h);
      pipe_step<3, BM, W, VEC>(p, P, aoff, cur, lds, s + 3, S, m, h);
    }
  }
  if (NS == 4 && rounds * NS < S) {
    // the tail's steps are rounds * 4 + {0, 1}: weights in ws[0], ws[1]; A in buffer 0 and in as[1]
    mfma_step<BM, W>(p.acc, lds, p.ws[0], m, h);
    store_a<BM>(p.as[1], lds + BM * BK);
    lds_barrier();
    mfma_step<BM, W>(p.acc, lds + BM * BK, p.ws[1], m, h);
    lds_barrier();
  }
  store_tile<BM, NPROJ>(P, t, p.acc, w, m, h);
}

// The routed problem `a` (weights W0) and the shared experts' `b` (K-blocked
// bf16) in one persistent launch: each XCD's workgroups walk that XCD's tiles
// of a, then of b.
template <int BM, WKind W0, int NP, bool VEC>
__global__ void __launch_bounds__(kGThreads) k_moe_gemm(GemmProblem a, GemmProblem b) {
  extern __shared__ uint16_t lds[];
  constexpr int bn = kWRowsWg / NP;
  const int x = (int)blockIdx.x % kXcds;
  const int j = (int)blockIdx.x / kXcds;
  const int J = (int)gridDim.x / kXcds;
  const Plan pa = plan_of(a, bn);
  const Plan pb = plan_of(b, bn);
  const int fa = xcd_prefix<BM>(a, pa, x);
  const int fb = xcd_prefix<BM>(b, pb, x);
  const int na = __builtin_amdgcn_readlane(fa, kWave - 1);
  const int nb = __builtin_amdgcn_readlane(fb, kWave - 1);
  for (int it = j; it < na + nb; it += J) {
    if (it < na) {
      gemm_tile<BM, W0, NP, VEC>(a, tile_at<BM>(a, pa, x, fa, it, bn), lds);
    } else {
      const TileRef t = tile_at<BM>(b, pb, x, fb, it - na, bn);
      for (int r = 0; r < parts_of(b); ++r) gemm_tile<BM, kBf16KBlocked, NP, VEC>(part_problem(b, r), t, lds);
    }
  }
}

// Workgroups of the persistent grid: every CU's resident share, a whole
// number per XCD.
template <int BM, WKind W0, int NP, bool VEC>
hipError_t moe_gemm_grid(int* grid) {
  static std::atomic<int> cached{0};
  int g = cached.load(std::memory_order_relaxed);
  if (g == 0) {
    int dev = 0, cus = 0, per_cu = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess)
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_moe_gemm<BM, W0, NP, VEC>, kGThreads,
                                                       (size_t)2 * BM * BK * sizeof(uint16_t));
    if (e != hipSuccess) return e;
    g = (cus / kXcds > 0 ? cus / kXcds : 1) * (per_cu > 0 ? per_cu : 1) * kXcds;
    cached.store(g, std::memory_order_relaxed);
  }
  *grid = g;
  return hipSuccess;
}

template <int BM, WKind W0, int NP, bool VEC = true>
hipError_t launch_moe_gemm(const GemmProblem& routed, const GemmProblem& shared, hipStream_t s, const char* name) {
  int grid = 0;
  const hipError_t e = moe_gemm_grid<BM, W0, NP, VEC>(&grid);
  if (e != hipSuccess) return e;
  UOCR_LAUNCH(name, (k_moe_gemm<BM, W0, NP, VEC>), dim3(grid), dim3(kGThreads), (size_t)2 * BM * BK * sizeof(uint16_t),
              s, routed, shared);
  return hipGetLastError();
}

// ------------------------------------------------------------- LDS-staged path
//
// The same tiles and placement for 16-byte aligned operands, with every
// operand streamed into LDS by global_load_lds_dwordx4 (lane l of a wave
// writes its 16 bytes at the instruction's LDS address + 16 l), so no
// registers hold data in flight: with 64-row tiles two workgroups share a CU
// and one's MFMAs overlap the other's dequantisation (the int8 path's VALU
// work, about ten VALU instructions per MFMA, bounds a lone wave).  A step is
// 64 k: every weight row contributes 64 (int8) or 128 (bf16) contiguous bytes,
// 4 or 8 lanes to a row, where the fragment-layout loads touch 32 rows per
// instruction.  A stage holds the workgroup's 256 weight rows and the A step;
// kCount stages form a ring, each loaded kCount - 1 steps ahead.  The int8
// scales of the tile's weight rows (one contiguous block of rows x groups
// floats per projection) are loaded into LDS once, at the tile's start: read
// step by step they would touch a cache line per few rows every step.  The
// waits are explicit (s_waitcnt vmcnt(n) before the barrier, n the loads
// issued since the step's own): every thread issues the same number of loads
// per step, the loads past the last step re-read it, and no other vector
// memory access happens inside the K loop.  Lane half h covers k = 32h ..
// 32h + 31 of a step, as in the fragment-load path, so both give the same bits.

// Rows per tile of the LDS-staged path: 128 for int8 weights (each
// dequantised weight feeds up to four 32-row MFMA blocks; blocks past a
// tile's rows are skipped), 64 for bf16 weights, whose 128-byte weight rows
// leave room for two stages of 64-row A steps only.
template <WKind W>
constexpr int kLdsBM = W == kInt8Rows ? 128 : 64;
constexpr int kWgPerCu = 2;  // two workgroups share a CU: one's barrier waits overlap the other's work

// LDS for an int8 tile's scales: 256 weight rows x up to 16 groups (K / 16
// or coarser groups; finer ones go to the fragment-load kernel).
constexpr int kMaxScaleGroups = 16;
constexpr int kScaleLds = kWRowsWg * kMaxScaleGroups * 4;

template <int BM, WKind W>
struct Stage {
  static constexpr int kBRowBytes = W == kInt8Rows ? BK : 2 * BK;  // one step of a weight row
  static constexpr int kBBytes = kWRowsWg * kBRowBytes;
  static constexpr int kABytes = BM * 2 * BK;
  static constexpr int kBytes = kBBytes + kABytes;
  static constexpr int kBudget = 160 * 1024 / kWgPerCu - (W == kInt8Rows ? kScaleLds : 0);
  static constexpr int kCount = kBudget / kBytes < 4 ? kBudget / kBytes : 4;
  static constexpr int kBLoads = kBBytes / 1024 / 4;  // weight loads per thread per step
  // loads per thread per step of a tile with NACT active 32-row blocks: the
  // weights and one 1 KB A load per block (32 rows x 128 bytes over 256 threads)
  template <int NACT>
  static constexpr int loads() {
    return kBLoads + NACT;
  }
  static_assert(kCount >= 2, "two stages");
  static_assert(kABytes == (BM / 32) * 16 * kGThreads, "one A load per thread per 32-row block");
};

template <WKind W>
constexpr int kRing = Stage<kLdsBM<W>, W>::kBytes * Stage<kLdsBM<W>, W>::kCount;
template <WKind W>
constexpr int kTileLds = kRing<W> + (W == kInt8Rows ? kScaleLds : 0);  // the scales follow the ring
template <WKind W0>
constexpr int kLdsBytes = kTileLds<W0> > kTileLds<kBf16KBlocked> ? kTileLds<W0> : kTileLds<kBf16KBlocked>;

typedef __attribute__((address_space(3))) void* lds_ptr;
__device__ __forceinline__ void dma16(const void* g, void* l) {
  __builtin_amdgcn_global_load_lds((const UOCR_GLOBAL void*)g, (lds_ptr)l, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* g, void* l) {
  __builtin_amdgcn_global_load_lds((const UOCR_GLOBAL void*)g, (lds_ptr)l, 4, 0, 0);
}

// This thread's loads of the step N loads back have landed, then the barrier:
// after it every wave's loads of that step are in LDS and every wave has
// finished reading the previous step.
template <int N>
__device__ __forceinline__ void step_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Stored position of chunk c of a 64-byte int8 weight row r: c ^ swz64(r).
// Any 8 consecutive rows (128-byte bank cycle) and any 16 (256-byte cycle)
// put a chunk in different banks.
__device__ __forceinline__ int swz64(int r) { return ((r >> 1) & 3) ^ ((r >> 3) & 1); }

// One step from a stage: 4 MFMA sub-steps, lane half h at k = 32h + 8 sub,
// over the tile's NACT active 32-row blocks (the rows past them are not
// computed).  The wave's weight bytes of the step are read first, and the A
// fragments of sub-step k + 1 before the MFMAs of sub-step k.
template <int BM, WKind W, int NACT>
__device__ __forceinline__ void lds_step(f32x16 (&acc)[NACT][2], const char* st, const float (&sc)[2], int w, int m,
                                         int h) {
  using St = Stage<BM, W>;
  constexpr int MB = NACT;
  constexpr int RB = St::kBRowBytes;
  constexpr int NQ = W == kInt8Rows ? 2 : 4;  // the lane's 16-byte weight chunks per block
  const char* Bw = st + 64 * w * RB;          // the wave's 64 weight rows
  const char* A = st + St::kBBytes;
  const int sw = swz(m);  // 128-byte rows 32i + m (A, bf16 weights)
  i32x4 raw[2][NQ];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int c = NQ * h + q;
      if constexpr (W == kBf16KBlocked) {
        // [4 k-blocks][256 rows][32 bytes], the two 16-byte halves of rows 8..15 of
        // every 16 swapped: k-block c / 2 of the step, half c % 2
        raw[b][q] = *(const i32x4*)(st + ((c >> 1) * kWRowsWg + 64 * w + 32 * b + m) * 32 +
                                    16 * ((c & 1) ^ ((m >> 3) & 1)));
      } else {
        raw[b][q] = *(const i32x4*)(Bw + (32 * b + m) * RB + 16 * (c ^ (W == kInt8Rows ? swz64(m) : sw)));
      }
    }
  // The A fragments of sub-step k + 1 are read during sub-step k.
  constexpr int AB = 2;
  bf16x8 a[AB][MB];
  auto read_a = [&](bf16x8(&dst)[MB], int sub) {
#pragma unroll
    for (int i = 0; i < MB; ++i) dst[i] = *(const bf16x8*)(A + (32 * i + m) * 2 * BK + 16 * ((4 * h + sub) ^ sw));
  };
  if constexpr (AB == 2) read_a(a[0], 0);
#pragma unroll
  for (int sub = 0; sub < 4; ++sub) {
    if constexpr (AB == 2) {
      if (sub < 3) read_a(a[(sub + 1) & 1], sub + 1);
    } else {
      read_a(a[0], sub);
    }
    bf16x8 bf[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      if constexpr (W == kInt8Rows) {
        const int d0 = raw[b][sub >> 1][(sub & 1) * 2], d1 = raw[b][sub >> 1][(sub & 1) * 2 + 1];
        i32x4 o;
        o[0] = (int)pack_bf16x2(i8_to_f32<0>(d0) * sc[b], i8_to_f32<1>(d0) * sc[b]);
        o[1] = (int)pack_bf16x2(i8_to_f32<2>(d0) * sc[b], i8_to_f32<3>(d0) * sc[b]);
        o[2] = (int)pack_bf16x2(i8_to_f32<0>(d1) * sc[b], i8_to_f32<1>(d1) * sc[b]);
        o[3] = (int)pack_bf16x2(i8_to_f32<2>(d1) * sc[b], i8_to_f32<3>(d1) * sc[b]);
        bf[b] = __builtin_bit_cast(bf16x8, o);
      } else {
        bf[b] = __builtin_bit_cast(bf16x8, raw[b][sub]);
      }
    }
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[sub % AB][i], bf[0], acc[i][0], 0, 0, 0);
      acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[sub % AB][i], bf[1], acc[i][1], 0, 0, 0);
    }
  }
}

// One tile whose rows fill NACT 32-row blocks: only those blocks' A rows are
// loaded and computed.
template <int BM, WKind W, int NPROJ, int NACT>
__device__ __forceinline__ void lds_tile(const GemmProblem& P, const TileRef& t, char* lds) {
  using St = Stage<BM, W>;
  constexpr int NS = St::kCount, NB = St::kBLoads, NA = NACT;
  constexpr int NL = St::template loads<NACT>();
  constexpr int RB = St::kBRowBytes;
  constexpr int RPL = 1024 / RB;  // weight rows per load
  // The thread index passes through an empty asm per tile, so that what is
  // derived from it (addresses, swizzles) is computed in the tile and not
  // hoisted out of the tile loop, where it held about 40 VGPRs across every
  // K loop (with 256 VGPRs at two waves a SIMD, the 3-4-block loops then read
  // their A fragments one at a time, each behind its own LDS wait).
  int tid = (int)threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int j = tid & (kWave - 1);
  const int w = tid >> 6;
  const int m = j & 31, h = j >> 5;
  // the tile's K range: all of K, or range t.e of a problem in K ranges
  const int parts = parts_of(P);
  const int S = P.K / BK / parts;
  const int k0 = parts > 1 ? t.e * S : 0;

  // weight rows: load i of the step fills stage rows 64w + RPL i + j / (RB / 16),
  // stored chunk j % (RB / 16) holding chunk (stored) ^ swizzle(row)
  const char* bsrc[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    if constexpr (W == kBf16KBlocked) {
      // load i: k-block i / 2 of the step for rows 32 (i % 2) .. + 31 of the wave's 64,
      // 1 KB contiguous in [K/16][N][16]; lane j holds half (j % 2) ^ (row bit 3) of row j / 2
      const int b = i & 1;
      const int lr = j >> 1;
      const int row = min(NPROJ == 2 ? t.n0 + 32 * w + lr : t.n0 + 64 * w + 32 * b + lr, P.N - 1);
      const int hf = (j & 1) ^ ((lr >> 3) & 1);
      const char* base = (const char*)(NPROJ == 2 && b == 1 ? P.p[1].w : P.p[0].w);
      bsrc[i] = base + ((int64_t)(i >> 1) * P.N + row) * 32 + 16 * hf;
      continue;
    }
    const int rr = RPL * i + j / (RB / 16);  // row within the wave's 64
    const int b = rr >> 5;
    const int mm = rr & 31;
    const int row = min(NPROJ == 2 ? t.n0 + 32 * w + mm : t.n0 + 64 * w + rr, P.N - 1);
    const int c = (j % (RB / 16)) ^ (W == kInt8Rows ? swz64(rr) : swz(rr));
    const char* base = (const char*)(NPROJ == 2 && b == 1 ? P.p[1].w : P.p[0].w);
    const int64_t wrow = (int64_t)t.e * P.N + row;
    if constexpr (W == kInt8Rows)
      bsrc[i] = base + wrow * P.K + 16 * c;
    else
      bsrc[i] = base + wrow * P.K * 2 + 16 * c;
  }
  const int64_t bstep = W == kBf16KBlocked ? (int64_t)(BK / 16) * P.N * 32 : RB;

  // A: load i of the step fills 1 KB unit 4i + w of the A stage, chunk j % 8 of
  // stage row 8 (4i + w) + j / 8
  int aoff[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int r = 8 * (4 * i + w) + (j >> 3);
    const int c = (j & 7) ^ swz(r);
    const int pos = t.pos0 + min(r, t.rows - 1);
    const int row = (P.a_by_token && P.rows.n_groups != nullptr) ? ldg(P.rows.group_rows + pos) / P.x_div : pos;
    aoff[i] = (int)((int64_t)row * P.lda) + 8 * c;
  }

  // int8 scales, loaded once for the tile after the ring: NPROJ 1, [256 rows
  // from n0][G]; NPROJ 2, [128 gate rows from n0][G] then the up rows'.  Each
  // projection's block is contiguous in [E][N][G]; rows past N re-read the
  // last real scale.  64-float units, G of them per wave; these loads precede
  // the stages', so the first step's wait covers them.
  float* sl = (float*)(lds + kRing<W>);
  int srow[2] = {0, 0};  // this lane's rows of blocks 0 and 1, times G
  if constexpr (W == kInt8Rows) {
    const int G = P.groups;
    constexpr int PR = NPROJ == 2 ? 128 : 256;  // rows per projection block
    const int64_t base = ((int64_t)t.e * P.N + t.n0) * G;
    const int lim = min(PR, P.N - t.n0) * G - 1;
    for (int u = w; u < 4 * G; u += 4) {
      const bool up = NPROJ == 2 && u >= 2 * G;
      const int f = 64 * (up ? u - 2 * G : u) + j;
      dma4((up ? P.p[1].s : P.p[0].s) + base + min(f, lim), sl + 64 * u);
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) srow[b] = (NPROJ == 2 ? PR * b + 32 * w + m : 64 * w + 32 * b + m) * G;
  }
  const int spg = W == kInt8Rows ? P.K / P.groups / BK : 1;  // steps per scale group

  // the loads of step s (clamped to the last step) into stage s % NS
  auto issue = [&](int s) {
    const int sc = k0 + min(s, S - 1);
    char* st = lds + (s % NS) * St::kBytes;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      if constexpr (W == kBf16KBlocked)
        dma16(bsrc[i] + sc * bstep, st + ((i >> 1) * kWRowsWg + 64 * w + 32 * (i & 1)) * 32);
      else
        dma16(bsrc[i] + sc * bstep, st + (64 * w + RPL * i) * RB);
    }
#pragma unroll
    for (int i = 0; i < NA; ++i) dma16(P.a + aoff[i] + sc * BK, st + St::kBBytes + (4 * i + w) * 1024);
  };

  f32x16 acc[NACT][2];
#pragma unroll
  for (int i = 0; i < NACT; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][0][r] = acc[i][1][r] = 0.0f;
  int g = 0, gs = 0;  // the step's scale group, and steps into it
  auto compute = [&](int s) {
    float sc[2] = {1.0f, 1.0f};
    if constexpr (W == kInt8Rows) {
      sc[0] = sl[srow[0] + g];
      sc[1] = sl[srow[1] + g];
      const bool next = ++gs == spg;
      g += next;
      gs = next ? 0 : gs;
    }
    lds_step<BM, W, NACT>(acc, lds + (s % NS) * St::kBytes, sc, w, m, h);
  };
  // S is even and at least 2, so the NS - 1 <= 2 prologue steps exist; the
  // last NS - 1 steps load nothing, and no load is in flight when the tile ends
  static_assert(NS >= 2 && NS <= 3, "ring depth");
#pragma unroll
  for (int i = 0; i < NS - 1; ++i) issue(i);
  for (int s = 0; s < S - (NS - 1); ++s) {
    step_barrier<(NS - 2) * NL>();
    issue(s + NS - 1);  // into the stage read in step s - 1, which every wave has finished
    compute(s);
  }
#pragma unroll
  for (int u = 0; u < NS - 1; ++u) {
    // tail step S - (NS - 1) + u: its loads and the NS - 2 - u stages after it are the ones outstanding
    if constexpr (NS == 3) {
      if (u == 0)
        step_barrier<NL>();
      else
        step_barrier<0>();
    } else {
      step_barrier<0>();
    }
    compute(S - (NS - 1) + u);
  }
  // every wave has finished reading the stages (and the scales) before the next tile's loads
  step_barrier<0>();
  if (parts > 1) {
    GemmProblem Q = P;  // range t.e's sums
    Q.outf += t.e * P.part_stride;
    store_tile<32 * NACT, NPROJ>(Q, t, acc, w, m, h);
  } else {
    store_tile<32 * NACT, NPROJ>(P, t, acc, w, m, h);
  }
}

// Placement for the LDS-staged path, two ways, chosen per launch from the
// rows (the tile count it bounds).
//
// Balanced (BAL, launches of several rounds: T = 4096).  The routed tiles
// form a sequence: the groups from the most rows to the fewest (ties in
// group order), each row tile by row tile and, within a row tile, column
// tile by column tile.  The sequence is cut into 8 contiguous ranges of equal
// estimated cost (a tile belongs to the range its cost midpoint falls in),
// range x going to XCD x; the shared experts' row tiles are cut into 8 runs
// of equal length (all their column tiles), run x going to XCD x ahead of
// its routed range.  Workgroup j of an XCD walks tiles j, j + J, ... of that
// list.  So every XCD gets the same work whatever the routing (dealing whole
// (group, column tile) units round robin left the XCDs up to 2x apart with
// skewed routing: T = 4096 down 144 -> 127 us, adversarial routing 400 ->
// 358 us a layer), and a group stays on one XCD (two where a range ends
// inside it): its weight tiles and its gathered A rows are fetched into that
// XCD's L2 and serve all of the group's row and column tiles there, the row
// tiles running in order so that the XCD's workgroups share a few row tiles'
// A at a time.
//
// By class (launches of at most two rounds: T = 512, about one tile a
// workgroup, where the balance of single tiles matters more).  A unit is one
// column tile of one group and a run of its row tiles (a routed expert's
// unit has all of them, so each expert weight tile is fetched into one L2
// and serves all of its rows there; the shared experts' many row tiles are
// cut into at most 8 runs).  Units are dealt round robin to the XCDs (routed
// first, the shared ones numbered on).  An XCD's tiles are listed class by
// class in decreasing estimated cost (class: problem and active blocks;
// within a class, unit order), and its workgroup j walks tiles j, j + J, ...
// of the list: the costly tiles start first and the second round is made of
// the cheapest ones.  (The balanced placement made T = 512 131 -> 151 us: its
// contiguous ranges put a range's costly tiles in one XCD's second round.)
//
// (A work queue -- atomic per-XCD counters, tiles taken as workgroups finish
// them -- measured slower on this GPU: the counter round trips and their
// broadcast cost more than the balance gained.)
//
// Cost.  A tile's cost grows with its active 32-row blocks, and an int8
// tile's more than a bf16 one's (the dequantisation is paid per tile).
// Estimated cost per 64-k step: 100 + 35 per block for int8 weights, 65 + 36
// per block for bf16, plus 600 a tile for its start and its stores
// (per-XCD busy times at T = 4096 fit these within about 10 %).
__device__ __forceinline__ int tile_cost(const GemmProblem& P, int nact) {
  return (P.K / BK / parts_of(P)) * (P.kind == kInt8Rows ? 100 + 35 * nact : 65 + 36 * nact) + 600;
}

// One problem's row tiles: rt in all, the last one partial with `apart`
// active blocks when part is set.
struct RowTiles {
  int rt, part, apart;
};
template <int BM>
__device__ __forceinline__ RowTiles row_tiles_of(int count) {
  RowTiles r;
  r.rt = (count + BM - 1) / BM;
  const int rem = count - (r.rt - 1) * BM;
  r.part = count > 0 && rem < BM ? 1 : 0;
  r.apart = r.part ? (rem + 31) >> 5 : 0;
  return r;
}

// The routed tile sequence.  Lane p holds the group of rank p (most rows
// first): the tiles and cost before it, its first row position, rows and
// expert (ranks past the last group hold no rows).
struct Seq {
  int tp, cp, start, count, e;
  int ta, ca;    // routed tiles and cost
  int nta, ntb;  // column tiles of each problem
};

template <int BMA, int BMB>
__device__ __forceinline__ Seq make_seq(const GemmProblem& a, const GemmProblem& b, int bn) {
  Seq q;
  q.nta = (a.N + bn - 1) / bn;
  q.ntb = (b.N + bn - 1) / bn * parts_of(b);  // column tiles of every K range
  const bool routed = a.rows.n_groups != nullptr;
  const int l = lane_id();
  // the group tables for every lane at once, clamped to their size, before
  // the group count is known (one memory latency at the kernel's start)
  int g0 = 0, g1 = 0, ge = 0;
  if (routed && a.max_groups > 0) {
    const int g = min(l, a.max_groups - 1);
    g0 = ldg(a.rows.group_start + g);
    g1 = ldg(a.rows.group_start + g + 1);
    ge = ldg(a.rows.group_expert + g);
  }
  const int ng = routed ? ldc(a.rows.n_groups) : (a.M > 0 ? 1 : 0);
  int start = 0, count = 0, e = 0;
  if (l < ng) {
    start = routed ? g0 : 0;
    count = routed ? g1 - g0 : a.M;
    e = routed ? ge : 0;
  }
  // the group's rank, most rows first (ties in group order; no rows last),
  // and its values moved to the lane of that rank
  int rank = 0;
#pragma unroll 8
  for (int k = 0; k < kWave; ++k) {
    const int ck = __builtin_amdgcn_readlane(count, k);
    rank += (ck > count || (ck == count && k < l)) ? 1 : 0;
  }
  q.start = __builtin_amdgcn_ds_permute(rank << 2, start);
  q.count = __builtin_amdgcn_ds_permute(rank << 2, count);
  q.e = __builtin_amdgcn_ds_permute(rank << 2, e);
  const RowTiles r = row_tiles_of<BMA>(q.count);
  const int tiles = q.nta * r.rt;
  const int cost = q.nta * ((r.rt - r.part) * tile_cost(a, BMA / 32) + (r.part ? tile_cost(a, r.apart) : 0));
  const int ti = wave_scan_i(tiles), ci = wave_scan_i(cost);
  q.tp = ti - tiles;
  q.cp = ci - cost;
  q.ta = __builtin_amdgcn_readlane(ti, kWave - 1);
  q.ca = __builtin_amdgcn_readlane(ci, kWave - 1);
  return q;
}

// Tiles of cost c each whose midpoints lie below t (t >= 0): (2i + 1) c < 2t.
__device__ __forceinline__ int below(int64_t t, int c) {
  return 2 * t > c ? (int)((2 * t - c + 2 * (int64_t)c - 1) / (2 * (int64_t)c)) : 0;
}
// Tiles of one problem's group (its row tiles r, nt columns) whose cost
// midpoints lie below t (0 <= t <= the group's cost).
template <int BM>
__device__ __forceinline__ int group_below(const GemmProblem& P, const RowTiles& r, int nt, int64_t t) {
  const int cf = tile_cost(P, BM / 32);
  const int64_t full = (int64_t)nt * (r.rt - r.part) * cf;
  if (t <= full) return below(t, cf);
  return nt * (r.rt - r.part) + (r.part ? min(nt, below(t - full, tile_cost(P, r.apart))) : 0);
}
// Index of the first routed tile whose cost midpoint is at least t.
template <int BMA>
__device__ __forceinline__ int seq_below(const GemmProblem& a, const Seq& q, int64_t t) {
  if (t <= 0) return 0;
  if (t >= q.ca) return q.ta;
  // the last group whose cost starts at or below t (the ranked groups with rows come first)
  const int g = (int)__popcll(__ballot(q.count > 0 && q.cp <= t)) - 1;
  const int cp = __builtin_amdgcn_readlane(q.cp, g), tp = __builtin_amdgcn_readlane(q.tp, g);
  const int count = __builtin_amdgcn_readlane(q.count, g);
  return tp + group_below<BMA>(a, row_tiles_of<BMA>(count), q.nta, t - cp);
}

constexpr int kMaxUnits = 1024;  // per problem: 128 per XCD, two a lane

struct Units {  // lane v holds the XCD's units v and v + 64 of its problem (hh = 0, 1)
  int nfull[2];  // tiles in full row tiles (BM rows)
  int npart[2];  // 1 if the unit has the group's last row tile and that one is partial
  int apart[2];  // the active 32-row blocks of that row tile
  int mt0[2];    // first row tile of the unit
  int c[2];      // column tile
  int start[2];  // the group's first row position
  int count[2];  // the group's rows
  int e[2];      // the group's expert (routed)
  int n;         // units of the problem (all XCDs)
};

// Problem P's units on XCD x, unit u going to XCD (u0 + u) % 8 (at most 1024
// units).  Routed: unit u = group u / nt, column u % nt, every row tile.
// Dense: run u / nt of ceil(row tiles / 8) row tiles, column u % nt.
template <int BM>
__device__ __forceinline__ Units plan_units(const GemmProblem& P, int nt, int ng, int x, int u0) {
  const bool routed = P.rows.n_groups != nullptr;
  const int rt_dense = (P.M + BM - 1) / BM;
  const int run = routed ? 1 << 30 : max(1, (rt_dense + kXcds - 1) / kXcds);
  const int nrun = routed ? 1 : (rt_dense + run - 1) / run;
  Units q;
  q.n = routed ? ng * nt : (P.M > 0 ? nrun * nt : 0);
  const int xs = ((x - u0) % kXcds + kXcds) % kXcds;
  // The group tables are read for every lane's unit at once, with the group
  // clamped to the tables' size, before the group count is known (one memory
  // latency at the kernel's start instead of two).
  int gs[2][2], ge[2];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int u = xs + kXcds * (lane_id() + 64 * hh);
    gs[hh][0] = gs[hh][1] = ge[hh] = 0;
    if (routed && P.max_groups > 0) {
      const int g = min(u / nt, P.max_groups - 1);
      gs[hh][0] = ldg(P.rows.group_start + g);
      gs[hh][1] = ldg(P.rows.group_start + g + 1);
      ge[hh] = ldg(P.rows.group_expert + g);
    }
  }
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int u = xs + kXcds * (lane_id() + 64 * hh);
    q.nfull[hh] = q.npart[hh] = q.apart[hh] = q.mt0[hh] = q.c[hh] = q.start[hh] = q.count[hh] = q.e[hh] = 0;
    if (u < q.n) {
      const int ri = routed ? 0 : u / nt;  // row run (dense)
      int start = 0, count = P.M, e = 0;
      if (routed) {
        start = gs[hh][0];
        count = gs[hh][1] - start;
        e = ge[hh];
      }
      const int rt = (count + BM - 1) / BM;
      const int mt0 = routed ? 0 : ri * run;
      const int mt1 = min(rt, mt0 + run);
      const int rem = count - (rt - 1) * BM;  // rows of the group's last row tile
      const bool part = count > 0 && rem < BM && mt1 == rt;
      q.nfull[hh] = mt1 - mt0 - (part ? 1 : 0);
      q.npart[hh] = part ? 1 : 0;
      q.apart[hh] = part ? (rem + 31) >> 5 : 0;
      q.mt0[hh] = mt0;
      q.c[hh] = u % nt;
      q.start[hh] = start;
      q.count[hh] = count;
      q.e[hh] = e;
    }
  }
  return q;
}

// A unit's tiles with nact active blocks: its full row tiles (nact = BM / 32),
// then its partial row tile if that has nact blocks.
template <int BM>
__device__ __forceinline__ int class_count(const Units& q, int hh, int nact) {
  return (nact == BM / 32 ? q.nfull[hh] : 0) + (q.apart[hh] == nact ? q.npart[hh] : 0);
}

// Tile `it` of class (nact active blocks) in the XCD's units (lanes' hh = 0
// units, then hh = 1).
template <int BM>
__device__ __forceinline__ TileRef class_tile(const GemmProblem& P, const Units& q, int nact, int it, int bn) {
  const int inc0 = wave_scan_i(class_count<BM>(q, 0, nact));
  const int tot0 = __builtin_amdgcn_readlane(inc0, kWave - 1);
  const int hh = it >= tot0 ? 1 : 0;
  const int inc = hh ? wave_scan_i(class_count<BM>(q, 1, nact)) + tot0 : inc0;
  const int lane = (int)__popcll(__ballot(inc <= it));
  const int before = lane > 0 ? __builtin_amdgcn_readlane(inc, lane - 1) : (hh ? tot0 : 0);
  const int local = it - before;
  const int nfull = nact == BM / 32 ? __builtin_amdgcn_readlane(hh ? q.nfull[1] : q.nfull[0], lane) : 0;
  const int count = __builtin_amdgcn_readlane(hh ? q.count[1] : q.count[0], lane);
  const int mt = local < nfull ? __builtin_amdgcn_readlane(hh ? q.mt0[1] : q.mt0[0], lane) + local : (count - 1) / BM;
  TileRef t;
  t.n0 = __builtin_amdgcn_readlane(hh ? q.c[1] : q.c[0], lane) * bn;
  t.pos0 = __builtin_amdgcn_readlane(hh ? q.start[1] : q.start[0], lane) + mt * BM;
  t.rows = min(BM, count - mt * BM);
  t.e = __builtin_amdgcn_readlane(hh ? q.e[1] : q.e[0], lane);
  return t;
}

// The classes of a launch in decreasing estimated cost, and an XCD's tiles
// of each.  Class k: problem cls[k] >> 8 (0 routed, 1 shared), cls[k] & 255
// active blocks, ordered by tile_cost.
constexpr int kMaxClasses = 6;
struct Sched {
  int n;
  int cls[kMaxClasses];
  int cnt[kMaxClasses];
  int total;
};

template <int BMA, int BMB>
__device__ __forceinline__ Sched make_sched(const GemmProblem& a, const GemmProblem& b, const Units& qa,
                                            const Units& qb) {
  constexpr int MA = BMA / 32, MB = BMB / 32;
  static_assert(MA + MB <= kMaxClasses, "classes");
  Sched sd;
  int key[kMaxClasses];
  sd.n = MA + MB;
#pragma unroll
  for (int k = 0; k < kMaxClasses; ++k) {
    const bool isa = k < MA;
    const int nact = isa ? MA - k : MA + MB - k;
    sd.cls[k] = k < MA + MB ? ((isa ? 0 : 1) << 8) | nact : 0;
    key[k] = k < MA + MB ? tile_cost(isa ? a : b, nact) : -1;
  }
  // stable sort by decreasing cost (a fixed exchange network on uniform values)
#pragma unroll
  for (int i = 0; i < kMaxClasses; ++i)
#pragma unroll
    for (int k = kMaxClasses - 1; k > i; --k)
      if (key[k] > key[k - 1]) {
        const int tk = key[k], tc = sd.cls[k];
        key[k] = key[k - 1];
        sd.cls[k] = sd.cls[k - 1];
        key[k - 1] = tk;
        sd.cls[k - 1] = tc;
      }
  sd.total = 0;
#pragma unroll
  for (int k = 0; k < kMaxClasses; ++k) {
    const int prob = sd.cls[k] >> 8, nact = sd.cls[k] & 255;
    const int v = k >= sd.n ? 0
                  : prob ? class_count<BMB>(qb, 0, nact) + class_count<BMB>(qb, 1, nact)
                         : class_count<BMA>(qa, 0, nact) + class_count<BMA>(qa, 1, nact);
    sd.cnt[k] = __builtin_amdgcn_readfirstlane(wave_sum_i(v));
    sd.total += sd.cnt[k];
  }
  return sd;
}

// The balanced placement's walk of the XCD's list.
template <WKind W0, int NP>
__device__ __forceinline__ void walk_balanced(const GemmProblem& a, const GemmProblem& b, char* lds_stages) {
  constexpr int bn = kWRowsWg / NP;
  constexpr int BMA = kLdsBM<W0>, BMB = kLdsBM<kBf16KBlocked>;
  const int x = (int)blockIdx.x % kXcds;
  const int j = (int)blockIdx.x / kXcds;
  const int J = (int)gridDim.x / kXcds;
  const Seq q = make_seq<BMA, BMB>(a, b, bn);
  // the XCD's shared row tiles [b0, b1) and routed tiles [s0, s1)
  const int rtb = (b.M + BMB - 1) / BMB;
  const int b0 = rtb * x / kXcds, b1 = rtb * (x + 1) / kXcds;
  const int nsh = (b1 - b0) * q.ntb;
  const int s0 = seq_below<BMA>(a, q, (int64_t)q.ca * x / kXcds);
  const int s1 = seq_below<BMA>(a, q, (int64_t)q.ca * (x + 1) / kXcds);
  // tile i of the XCD's list: its problem, row tile and column tile
  auto run = [&](int i) __attribute__((always_inline)) {
    if (i >= nsh) {
      i += s0 - nsh;
      // the last ranked group whose tiles start at or below i
      const int g = (int)__popcll(__ballot(q.count > 0 && q.tp <= i)) - 1;
      const int local = i - __builtin_amdgcn_readlane(q.tp, g);
      const int mt = local / q.nta;
      const int count = __builtin_amdgcn_readlane(q.count, g);
      TileRef t;
      t.n0 = (local - mt * q.nta) * bn;
      t.pos0 = __builtin_amdgcn_readlane(q.start, g) + mt * BMA;
      t.rows = min(BMA, count - mt * BMA);
      t.e = __builtin_amdgcn_readlane(q.e, g);
      const int nact = (t.rows + 31) >> 5;
      if constexpr (BMA == 128) {
        if (nact == 4)
          lds_tile<BMA, W0, NP, 4>(a, t, lds_stages);
        else if (nact == 3)
          lds_tile<BMA, W0, NP, 3>(a, t, lds_stages);
        else if (nact == 2)
          lds_tile<BMA, W0, NP, 2>(a, t, lds_stages);
        else
          lds_tile<BMA, W0, NP, 1>(a, t, lds_stages);
      } else {
        static_assert(BMA == 64, "64- or 128-row tiles");
        if (nact == 2)
          lds_tile<BMA, W0, NP, 2>(a, t, lds_stages);
        else
          lds_tile<BMA, W0, NP, 1>(a, t, lds_stages);
      }
    } else {
      static_assert(BMB == 64, "64-row shared tiles");
      const int mt = b0 + i / q.ntb;
      const int cr = i - (mt - b0) * q.ntb;  // K range cr / ntr, column tile cr % ntr
      const int ntr = q.ntb / parts_of(b);
      TileRef t;
      t.e = cr / ntr;
      t.n0 = (cr - t.e * ntr) * bn;
      t.pos0 = mt * BMB;
      t.rows = min(BMB, b.M - mt * BMB);
      if (t.rows > 32)
        lds_tile<BMB, kBf16KBlocked, NP, 2>(b, t, lds_stages);
      else
        lds_tile<BMB, kBf16KBlocked, NP, 1>(b, t, lds_stages);
    }
  };
  // Two rounds at most (small batches): the second round runs in reverse, so
  // that the workgroups with the list's costliest first tiles take none and
  // those with its cheapest take the rest.  More rounds walk in order.
  const int n = nsh + s1 - s0;
  const bool two = n <= 2 * J;
  const int rounds = two ? 2 : (n - j + J - 1) / J;
  for (int k = 0; k < rounds; ++k) {
    const int it = two && k == 1 ? 2 * J - 1 - j : j + k * J;
    if (it < n) run(it);
  }
}

// The by-class placement's walk of the XCD's list.
template <WKind W0, int NP>
__device__ __forceinline__ void walk_classes(const GemmProblem& a, const GemmProblem& b, char* lds_stages) {
  constexpr int bn = kWRowsWg / NP;
  constexpr int BMA = kLdsBM<W0>, BMB = kLdsBM<kBf16KBlocked>;
  const int x = (int)blockIdx.x % kXcds;
  const int ntr = (b.N + bn - 1) / bn;  // the shared problem's column tiles, in every K range
  const int nta = (a.N + bn - 1) / bn, ntb = ntr * parts_of(b);
  const int nga = a.rows.n_groups != nullptr ? ldc(a.rows.n_groups) : 1;
  const int j = (int)blockIdx.x / kXcds;
  const int J = (int)gridDim.x / kXcds;
  const Units qa = plan_units<BMA>(a, nta, nga, x, 0);
  const Units qb = plan_units<BMB>(b, ntb, 1, x, qa.n);  // dealt on from where the routed units ended
  const Sched sd = make_sched<BMA, BMB>(a, b, qa, qb);
  // tile `it` of the XCD's list: its class, then the class's tile
  auto run = [&](int it) __attribute__((always_inline)) {
    int cls = sd.cls[0];
    bool found = false;
#pragma unroll
    for (int k = 0; k < kMaxClasses; ++k) {
      if (!found && k < sd.n) {
        if (it < sd.cnt[k]) {
          cls = sd.cls[k];
          found = true;
        } else {
          it -= sd.cnt[k];
        }
      }
    }
    const int nact = cls & 255;
    if ((cls >> 8) == 0) {
      if constexpr (BMA == 128) {
        if (nact == 4)
          lds_tile<BMA, W0, NP, 4>(a, class_tile<BMA>(a, qa, 4, it, bn), lds_stages);
        else if (nact == 3)
          lds_tile<BMA, W0, NP, 3>(a, class_tile<BMA>(a, qa, 3, it, bn), lds_stages);
        else if (nact == 2)
          lds_tile<BMA, W0, NP, 2>(a, class_tile<BMA>(a, qa, 2, it, bn), lds_stages);
        else
          lds_tile<BMA, W0, NP, 1>(a, class_tile<BMA>(a, qa, 1, it, bn), lds_stages);
      } else {
        static_assert(BMA == 64, "64- or 128-row tiles");
        if (nact == 2)
          lds_tile<BMA, W0, NP, 2>(a, class_tile<BMA>(a, qa, 2, it, bn), lds_stages);
        else
          lds_tile<BMA, W0, NP, 1>(a, class_tile<BMA>(a, qa, 1, it, bn), lds_stages);
      }
    } else {
      static_assert(BMB == 64, "64-row shared tiles");
      TileRef t = class_tile<BMB>(b, qb, nact, it, bn);
      const int cr = t.n0 / bn;  // K range cr / ntr, column tile cr % ntr
      t.e = cr / ntr;
      t.n0 = (cr - t.e * ntr) * bn;
      if (nact == 2)
        lds_tile<BMB, kBf16KBlocked, NP, 2>(b, t, lds_stages);
      else
        lds_tile<BMB, kBf16KBlocked, NP, 1>(b, t, lds_stages);
    }
  };
  // Two rounds at most (small batches): the second round runs in reverse, so
  // that the workgroups with the costliest first tiles take the cheapest
  // second ones (at T = 512, gate/up 70 -> 66 us).  More rounds walk in
  // order (reversing every other round made T = 4096 slower).
  const bool two = sd.total <= 2 * J;
  const int rounds = two ? 2 : (sd.total - j + J - 1) / J;
  for (int k = 0; k < rounds; ++k) {
    const int it = two && k == 1 ? 2 * J - 1 - j : j + k * J;
    if (it < sd.total) run(it);
  }
}

template <WKind W0, int NP, bool BAL>
__global__ void __launch_bounds__(kGThreads, kWgPerCu) k_moe_gemm_lds(GemmProblem a, GemmProblem b) {
  extern __shared__ __attribute__((aligned(16))) char lds_stages[];
  if constexpr (BAL)
    walk_balanced<W0, NP>(a, b, lds_stages);
  else
    walk_classes<W0, NP>(a, b, lds_stages);
}

// Workgroups of the LDS-staged grid: every CU's resident share, a whole
// number per XCD (the same for both placements).
template <WKind W0, int NP>
hipError_t moe_gemm_lds_grid(int* grid) {
  constexpr size_t lds = kLdsBytes<W0>;
  static std::atomic<int> cached{0};
  int g = cached.load(std::memory_order_relaxed);
  if (g == 0) {
    int dev = 0, cus = 0, per_cu = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    for (const void* f : {(const void*)k_moe_gemm_lds<W0, NP, false>, (const void*)k_moe_gemm_lds<W0, NP, true>})
      if (e == hipSuccess) e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e == hipSuccess)
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_moe_gemm_lds<W0, NP, false>, kGThreads, lds);
    if (e != hipSuccess) return e;
    g = (cus / kXcds > 0 ? cus / kXcds : 1) * (per_cu > 0 ? per_cu : 1) * kXcds;
    cached.store(g, std::memory_order_relaxed);
  }
  *grid = g;
  return hipSuccess;
}

// The balanced placement once the launch's tiles (bounded from the rows)
// exceed two rounds of the grid.
template <WKind W0, int NP>
hipError_t launch_moe_gemm_lds(const GemmProblem& routed, const GemmProblem& shared, hipStream_t s,
                               const char* name) {
  constexpr size_t lds = kLdsBytes<W0>;
  int grid = 0;
  const hipError_t e = moe_gemm_lds_grid<W0, NP>(&grid);
  if (e != hipSuccess) return e;
  constexpr int bn = kWRowsWg / NP;
  constexpr int BMA = kLdsBM<W0>, BMB = kLdsBM<kBf16KBlocked>;
  const int64_t tiles = (int64_t)((routed.N + bn - 1) / bn) * ((routed.M + BMA - 1) / BMA + routed.max_groups) +
                        (int64_t)((shared.N + bn - 1) / bn) * parts_of(shared) * ((shared.M + BMB - 1) / BMB);
  if (tiles > 2 * (int64_t)grid)
    UOCR_LAUNCH(name, (k_moe_gemm_lds<W0, NP, true>), dim3(grid), dim3(kGThreads), lds, s, routed, shared);
  else
    UOCR_LAUNCH(name, (k_moe_gemm_lds<W0, NP, false>), dim3(grid), dim3(kGThreads), lds, s, routed, shared);
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

// K granularity of the grouped GEMM: two steps.
int gemm_bk() { return 2 * BK; }

// Two K ranges for the shared problem where the launch has at most two
// rounds of tiles (the by-class placement, T = 512: about a tile a
// workgroup), so that its tiles, twice a routed down tile's K when the shared
// width is twice the routed one, are not the launch's longest.  With more
// rounds the extra tiles and the combine's second read cost more (T = 4096:
// down 123 -> 129 us, the combine 25 -> 29 us).  Both kernels cut the same
// way; the bound on the tiles is the LDS-staged launch's.
int gemm_shared_parts(const GemmProblem& routed, const GemmProblem& shared) {
  if (shared.kind != kBf16KBlocked || shared.swiglu || shared.K % (2 * 2 * BK)) return 1;
  int grid = 0;
  const bool int8 = routed.kind == kInt8Rows;
  const hipError_t e = routed.swiglu ? (int8 ? moe_gemm_lds_grid<kInt8Rows, 2>(&grid) : moe_gemm_lds_grid<kBf16Rows, 2>(&grid))
                                     : (int8 ? moe_gemm_lds_grid<kInt8Rows, 1>(&grid) : moe_gemm_lds_grid<kBf16Rows, 1>(&grid));
  if (e != hipSuccess || grid <= 0) return 1;
  const int bn = kWRowsWg / (routed.swiglu ? 2 : 1);
  const int BMA = int8 ? kLdsBM<kInt8Rows> : kLdsBM<kBf16Rows>, BMB = kLdsBM<kBf16KBlocked>;
  const int64_t tiles = (int64_t)((routed.N + bn - 1) / bn) * ((routed.M + BMA - 1) / BMA + routed.max_groups) +
                        (int64_t)((shared.N + bn - 1) / bn) * 2 * ((shared.M + BMB - 1) / BMB);
  return tiles <= 2 * (int64_t)grid ? 2 : 1;
}

hipError_t launch_gemm_pair(const GemmProblem& routed, const GemmProblem& shared, int bm, hipStream_t s, bool vec) {
  const bool gu = routed.swiglu != 0;
  const char* name = gu ? "gemm_gateup" : "gemm_down";
  if (routed.N % 32 || shared.N % 32 || routed.K % (2 * BK) || shared.K % (2 * BK)) return hipErrorInvalidValue;
  // K ranges: the shared problem only, each an even number of K steps, fp32 sums
  if (parts_of(shared) > 1 && (shared.K % (parts_of(shared) * 2 * BK) || shared.swiglu || shared.outf == nullptr))
    return hipErrorInvalidValue;
  if (routed.kind == kInt8Rows && (routed.K % routed.groups || (routed.K / routed.groups) % BK))
    return hipErrorInvalidValue;
  if ((routed.kind == kInt8Rows && routed.groups > kMaxScaleGroups) || routed.max_groups > kWave) {
    // groups finer than K / 16 (the fragment-load kernel reads each step's scale itself), or more
    // routed groups than the LDS-staged kernel's placement holds (one a lane)
    if (routed.kind == kInt8Rows)
      return gu ? launch_moe_gemm<64, kInt8Rows, 2, false>(routed, shared, s, name)
                : launch_moe_gemm<64, kInt8Rows, 1, false>(routed, shared, s, name);
    return gu ? launch_moe_gemm<64, kBf16Rows, 2, false>(routed, shared, s, name)
              : launch_moe_gemm<64, kBf16Rows, 1, false>(routed, shared, s, name);
  }
  if (!vec) {  // weights at any alignment: 64-row tiles only
    if (bm != 64) return hipErrorInvalidValue;
    if (routed.kind == kInt8Rows)
      return gu ? launch_moe_gemm<64, kInt8Rows, 2, false>(routed, shared, s, name)
                : launch_moe_gemm<64, kInt8Rows, 1, false>(routed, shared, s, name);
    return gu ? launch_moe_gemm<64, kBf16Rows, 2, false>(routed, shared, s, name)
              : launch_moe_gemm<64, kBf16Rows, 1, false>(routed, shared, s, name);
  }
  // 16-byte aligned operands: the LDS-staged kernel (its tile heights are its own)
  if (routed.kind == kInt8Rows)
    return gu ? launch_moe_gemm_lds<kInt8Rows, 2>(routed, shared, s, name)
              : launch_moe_gemm_lds<kInt8Rows, 1>(routed, shared, s, name);
  return gu ? launch_moe_gemm_lds<kBf16Rows, 2>(routed, shared, s, name)
            : launch_moe_gemm_lds<kBf16Rows, 1>(routed, shared, s, name);
}

}  // namespace uocr
