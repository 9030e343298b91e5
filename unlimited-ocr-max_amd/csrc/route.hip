// Routing: router logits, softmax + top-k, grouping of routed rows by expert,
// and the routing-weighted combine.
//
// Arithmetic (restated by the CPU oracle):
//   logit[t,e] = 64 lane fma chains over k = lane, lane+64, ... of x[t,k]*Wr[e,k],
//                then a halving tree over the lanes (v[l] += v[l+off], off 32..1);
//   p = uexp(l - max) / S, S the same halving tree over the 64 expert slots;
//   top-k in score order, ties to the lower id (unlimited_ocr_max/decoder.py:509-514,
//   no renormalisation unless asked: model_config.py:149-150);
//   combine: fma chain over the k slots from 0, then + shared
//   (decoder.py:599-604,655).
#include "uocr_device.h"
#include "uocr_kernels.h"

namespace uocr {

namespace {

// ---------------------------------------------------------------- logits

// logits[t][e] for 4 tokens x 4 experts per wave (grid: 16 experts per
// workgroup in x, 4 tokens in y), H <= kLogitsMaxH: the lane's x and router
// values (k = lane + 64 j) are all loaded before the fmas, then each (t, e)
// is the 64-lane tree (the order of wave_tree_sum, batched by
// tree_sum_quads).  The waves of the first expert group also write the
// tokens' x rows rounded to bf16 (xb), when asked: the prefill GEMM's A
// operand.
constexpr int kLogitsMaxH = 2048;
constexpr int kXcds = kFusedXcds;  // XCDs; workgroup b runs on XCD b % kXcds

// The first workgroup of a launch clears `n` words for a later kernel of the
// same stream (the routing's counters).
__device__ __forceinline__ void zero_words_once(int32_t* p, int n) {
  if (p != nullptr && blockIdx.x == 0 && blockIdx.y == 0)
    for (int i = (int)threadIdx.x; i < n; i += (int)blockDim.x) p[i] = 0;
}

template <int kJ>  // >= H / 64
__global__ void __launch_bounds__(256) k_logits_wide(float* __restrict__ logits, uint16_t* __restrict__ xb,
                                                     const float* __restrict__ x, int64_t ldx,
                                                     const float* __restrict__ router, int T, int E, int H,
                                                     int32_t* __restrict__ zero, int nzero) {
  zero_words_once(zero, nzero);
  const int w = (int)(threadIdx.x >> 6);
  const int l = lane_id();
  const int e0 = (int)blockIdx.x * 16 + w * 4;
  const int t0 = (int)blockIdx.y * 4;
  if (e0 >= E) return;
  const int nj = H / kWave;
  float xv[4][kJ], wv[4][kJ];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float* xr = x + (int64_t)min(t0 + i, T - 1) * ldx + l;
    const float* wr = router + (int64_t)min(e0 + i, E - 1) * H + l;
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
      if (j < nj) {
        xv[i][j] = ldg(xr + kWave * j);
        wv[i][j] = ldg(wr + kWave * j);
      }
    }
  }
  if (xb != nullptr && blockIdx.x == 0 && w == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (t0 + i < T) {
        uint16_t* dst = xb + (int64_t)(t0 + i) * H + l;
#pragma unroll
        for (int j = 0; j < kJ; ++j)
          if (j < nj) dst[kWave * j] = f32_to_bf16_rne(xv[i][j]);
      }
    }
  }
  float p[16], sums[4];  // p[4 ti + ei]
#pragma unroll
  for (int ti = 0; ti < 4; ++ti) {
#pragma unroll
    for (int ei = 0; ei < 4; ++ei) {
      float a = 0.0f;
#pragma unroll
      for (int j = 0; j < kJ; ++j)
        if (j < nj) a = __builtin_fmaf(xv[ti][j], wv[ei][j], a);
      p[4 * ti + ei] = a;
    }
  }
  // lane 16 r of sums[ti] holds token ti's logit of expert e0 + tree_row_value(r)
  tree_sum_quads(p, sums);
  const int ei = tree_row_value(l >> 4);
#pragma unroll
  for (int ti = 0; ti < 4; ++ti)
    if ((l & 15) == 0 && t0 + ti < T && e0 + ei < E) logits[(int64_t)(t0 + ti) * E + e0 + ei] = sums[ti];
}

// logits[t][e] for TW tokens x EW experts per wave (grid: x = blocks of EW
// experts, y = blocks of 4 TW tokens; the 4 waves of a workgroup share the
// expert block, so its router rows come from L1 after the first wave), for
// prefill sizes: every x row and router row is read T / TW + E / EW times
// instead of once per (token, expert) quad.  Per lane the same fma chains over
// k = lane + 64 j as k_logits_wide, the operands of step j + 1 loaded while
// step j is computed, then the same 64-lane tree; the waves of the first
// expert block also write the tokens' x rows rounded to bf16 (xb).
// One wave's TW tokens x EW experts from token t0 and expert e0 (wave-uniform;
// nothing to do past the ends).  xb rows are written when write_xb.
template <int TW, int EW>
__device__ __forceinline__ void logits_tile(float* __restrict__ logits, uint16_t* __restrict__ xb,
                                            const float* __restrict__ x, int64_t ldx,
                                            const float* __restrict__ router, int T, int E, int H, int t0, int e0,
                                            bool write_xb) {
  if (t0 >= T || e0 >= E) return;
  const int l = lane_id();
  const int nj = H / kWave;
  const float* xl = x + (int64_t)t0 * ldx + l;
  const float* wl = router + (int64_t)e0 * H + l;
  int64_t xo[TW], wo[EW];  // wave-uniform row offsets (rows past the end repeat the last one)
#pragma unroll
  for (int t = 0; t < TW; ++t) xo[t] = (int64_t)min(t, T - 1 - t0) * ldx;
#pragma unroll
  for (int e = 0; e < EW; ++e) wo[e] = (int64_t)min(e, E - 1 - e0) * H;

  float p[TW][EW];
#pragma unroll
  for (int t = 0; t < TW; ++t)
#pragma unroll
    for (int e = 0; e < EW; ++e) p[t][e] = 0.0f;
  // JB steps of x and router values are requested at once (one memory
  // latency per JB steps); each lane's chain still runs over j in order
  constexpr int JB = TW * EW >= 128 ? 2 : 5;
  for (int j0 = 0; j0 < nj; j0 += JB) {
    float xa[JB][TW], wa[JB][EW];
#pragma unroll
    for (int jj = 0; jj < JB; ++jj) {
      const int jo = min(j0 + jj, nj - 1) * kWave;
#pragma unroll
      for (int t = 0; t < TW; ++t) xa[jj][t] = ldg(xl + xo[t] + jo);
#pragma unroll
      for (int e = 0; e < EW; ++e) wa[jj][e] = ldg(wl + wo[e] + jo);
    }
#pragma unroll
    for (int jj = 0; jj < JB; ++jj) {
      if (j0 + jj < nj) {
        if (write_xb) {
#pragma unroll
          for (int t = 0; t < TW; ++t)
            if (t0 + t < T) xb[(int64_t)(t0 + t) * H + l + (j0 + jj) * kWave] = f32_to_bf16_rne(xa[jj][t]);
        }
#pragma unroll
        for (int t = 0; t < TW; ++t)
#pragma unroll
          for (int e = 0; e < EW; ++e) p[t][e] = __builtin_fmaf(xa[jj][t], wa[jj][e], p[t][e]);
      }
    }
  }
  // the trees of all TW x EW values at once: lane 16 r of sums[j] holds
  // value 4 j + tree_row_value(r) of p (row-major), one store per 4 values
  static_assert(EW % 4 == 0, "a quad of values shares its token");
  float flat[TW * EW], sums[TW * EW / 4];
#pragma unroll
  for (int t = 0; t < TW; ++t)
#pragma unroll
    for (int e = 0; e < EW; ++e) flat[t * EW + e] = p[t][e];
  tree_sum_quads(flat, sums);
  const int e_row = tree_row_value(l >> 4);
#pragma unroll
  for (int j = 0; j < TW * EW / 4; ++j) {
    const int t = 4 * j / EW;
    const int e = 4 * j % EW + e_row;
    if ((l & 15) == 0 && t0 + t < T && e0 + e < E) logits[(int64_t)(t0 + t) * E + e0 + e] = sums[j];
  }
}

// logits_tile for H = 64 NJ (NJ compile-time): the same chains and trees,
// the operands in a ring of D register slots, so that the loads of step
// j + D are issued as step j's fmas are done and D steps are in flight at
// once (logits_tile waits for each batch of JB steps before its fmas).
// Slot t holds token t0 + (t + rot) % TW (every slot's chains are its own, so
// the order of the slots changes no bits); the xb rows of slots 0 .. XK-1 are
// written.
template <int TW, int EW, int NJ, int XK>
__device__ __forceinline__ void logits_ring(float* __restrict__ logits, uint16_t* __restrict__ xb,
                                            const float* __restrict__ x, int64_t ldx,
                                            const float* __restrict__ router, int T, int E, int t0, int e0,
                                            int rot) {
  constexpr int D = 2;
  constexpr int H = NJ * kWave;
  if (t0 >= T || e0 >= E) return;
  const int l = lane_id();
  // wave-uniform row bases (rows past the end repeat the last one), the lane's
  // element k = l + 64 j at byte 4 l + 256 j of a row
  const UOCR_GLOBAL char* xr[TW];
  const UOCR_GLOBAL char* wr[EW];
  uint16_t* br[TW];
#pragma unroll
  for (int t = 0; t < TW; ++t) {
    const int64_t row = min(t0 + (t + rot) % TW, T - 1);
    xr[t] = (const UOCR_GLOBAL char*)(x + row * ldx);
    br[t] = xb + row * H;
  }
#pragma unroll
  for (int e = 0; e < EW; ++e) wr[e] = (const UOCR_GLOBAL char*)(router + (int64_t)min(e0 + e, E - 1) * H);
  // (the instruction's offset field holds below 4 KiB: 16 steps from each of
  // these lane offsets, kept opaque so that none is folded back into it)
  uint32_t lo[(NJ + 15) / 16];
#pragma unroll
  for (int i = 0; i < (NJ + 15) / 16; ++i) {
    lo[i] = 4u * (uint32_t)l + 4096u * i;
    asm volatile("" : "+v"(lo[i]));
  }
  float p[TW][EW];
#pragma unroll
  for (int t = 0; t < TW; ++t)
#pragma unroll
    for (int e = 0; e < EW; ++e) p[t][e] = 0.0f;
  float xa[D][TW], wa[D][EW];
#pragma unroll
  for (int s = 0; s < D; ++s) {
#pragma unroll
    for (int t = 0; t < TW; ++t) xa[s][t] = *(const UOCR_GLOBAL float*)(xr[t] + (lo[0] + 256u * s));
#pragma unroll
    for (int e = 0; e < EW; ++e) wa[s][e] = *(const UOCR_GLOBAL float*)(wr[e] + (lo[0] + 256u * s));
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int s = j % D;
    // (a row past the end stores the last row's value again, to its place)
#pragma unroll
    for (int t = 0; t < XK; ++t) br[t][l + j * kWave] = f32_to_bf16_rne(xa[s][t]);
#pragma unroll
    for (int t = 0; t < TW; ++t)
#pragma unroll
      for (int e = 0; e < EW; ++e) p[t][e] = __builtin_fmaf(xa[s][t], wa[s][e], p[t][e]);
    if (j + D < NJ) {
      const uint32_t o = lo[(j + D) / 16] + 256u * ((j + D) % 16);
#pragma unroll
      for (int t = 0; t < TW; ++t) xa[s][t] = *(const UOCR_GLOBAL float*)(xr[t] + o);
#pragma unroll
      for (int e = 0; e < EW; ++e) wa[s][e] = *(const UOCR_GLOBAL float*)(wr[e] + o);
    }
    // each step's loads stay after its fmas (hoisted higher, they would hold
    // more slots than the ring's)
    __builtin_amdgcn_sched_barrier(0);
  }
  static_assert(EW % 4 == 0, "a quad of values shares its token");
  float flat[TW * EW], sums[TW * EW / 4];
#pragma unroll
  for (int t = 0; t < TW; ++t)
#pragma unroll
    for (int e = 0; e < EW; ++e) flat[t * EW + e] = p[t][e];
  tree_sum_quads(flat, sums);
  const int e_row = tree_row_value(l >> 4);
#pragma unroll
  for (int j = 0; j < TW * EW / 4; ++j) {
    const int t = t0 + (4 * j / EW + rot) % TW;
    const int e = 4 * j % EW + e_row;
    if ((l & 15) == 0 && t < T && e0 + e < E) logits[(int64_t)t * E + e0 + e] = sums[j];
  }
}

template <int TW, int EW, int NJ>
__global__ void __launch_bounds__(256) k_logits_ring(float* __restrict__ logits, uint16_t* __restrict__ xb,
                                                     const float* __restrict__ x, int64_t ldx,
                                                     const float* __restrict__ router, int T, int E,
                                                     int32_t* __restrict__ zero, int nzero) {
  zero_words_once(zero, nzero);
  // Workgroup b runs on XCD b % 8: the E / EW expert blocks of one block of
  // 4 TW tokens run on the same XCD, whose L2 then fetches those x rows once.
  const int b = (int)blockIdx.x;
  const int neb = (E + EW - 1) / EW;
  const int slot = b / kXcds;
  const int tb = (slot / neb) * kXcds + b % kXcds;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int t0 = (tb * 4 + w) * TW;
  const int eb = slot % neb;
  const int e0 = eb * EW;
  // The xb rows: each of the 4 expert blocks (E = 4 EW, which the launch
  // checks) writes 2 of a wave's 8 tokens, its slots 0 and 1 (tokens 2 eb and
  // 2 eb + 1), so that no block's waves take longer than the others'.  (One
  // copy of the loop with the stores and one without: a branch in each step
  // would split it into blocks that the scheduler cannot order.)
  static_assert(TW == 8, "2 of 8 tokens per expert block");
  if (xb != nullptr)
    logits_ring<TW, EW, NJ, 2>(logits, xb, x, ldx, router, T, E, t0, e0, 2 * eb);
  else
    logits_ring<TW, EW, NJ, 0>(logits, xb, x, ldx, router, T, E, t0, e0, 0);
}

template <int TW, int EW>
__global__ void __launch_bounds__(256) k_logits_tile(float* __restrict__ logits, uint16_t* __restrict__ xb,
                                                     const float* __restrict__ x, int64_t ldx,
                                                     const float* __restrict__ router, int T, int E, int H,
                                                     int32_t* __restrict__ zero, int nzero) {
  zero_words_once(zero, nzero);
  const int w = (int)(threadIdx.x >> 6);
  logits_tile<TW, EW>(logits, xb, x, ldx, router, T, E, H, ((int)blockIdx.y * 4 + w) * TW, (int)blockIdx.x * EW,
                      xb != nullptr && blockIdx.x == 0);
}

template <int TT, int EE>
__global__ void __launch_bounds__(256) k_logits(float* __restrict__ logits, const float* __restrict__ x,
                                                int64_t ldx, const float* __restrict__ router, int T, int E,
                                                int H) {
  const int w = (int)(threadIdx.x >> 6);
  const int lane = lane_id();
  const int e0 = ((int)blockIdx.x * 4 + w) * EE;
  const int t0 = (int)blockIdx.y * TT;
  if (e0 >= E) return;
  const float* xr[TT];
  const float* wr[EE];
#pragma unroll
  for (int t = 0; t < TT; ++t) xr[t] = x + (int64_t)min(t0 + t, T - 1) * ldx;
#pragma unroll
  for (int e = 0; e < EE; ++e) wr[e] = router + (int64_t)min(e0 + e, E - 1) * H;
  float p[TT][EE];
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int e = 0; e < EE; ++e) p[t][e] = 0.0f;
  // k = lane + 64 j; U steps of loads are issued before their fmas
  constexpr int U = TT * EE > 16 ? 2 : 4;
  for (int k0 = lane; k0 < H; k0 += U * kWave) {
    float xv[U][TT], wv[U][EE];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = k0 + u * kWave;
#pragma unroll
      for (int t = 0; t < TT; ++t) xv[u][t] = k < H ? xr[t][k] : 0.0f;
#pragma unroll
      for (int e = 0; e < EE; ++e) wv[u][e] = k < H ? wr[e][k] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (k0 + u * kWave >= H) break;
#pragma unroll
      for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int e = 0; e < EE; ++e) p[t][e] = __builtin_fmaf(xv[u][t], wv[u][e], p[t][e]);
    }
  }
  // lane 16 r of sums[j] holds value 4 j + tree_row_value(r) of p (row-major)
  static_assert(TT * EE % 4 == 0, "values come in quads");
  float flat[TT * EE], sums[TT * EE / 4];
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int e = 0; e < EE; ++e) flat[t * EE + e] = p[t][e];
  tree_sum_quads(flat, sums);
  const int rv = tree_row_value(lane >> 4);
#pragma unroll
  for (int j = 0; j < TT * EE / 4; ++j) {
    const int t = (4 * j + rv) / EE;
    const int e = (4 * j + rv) % EE;
    if ((lane & 15) == 0 && t0 + t < T && e0 + e < E) logits[(int64_t)(t0 + t) * E + e0 + e] = sums[j];
  }
}

// ---------------------------------------------------------------- softmax + top-k

// LDS words a wave's token_topk needs: 64 keys, then up to 64 selected
// probabilities (as floats, 32 words).
constexpr int kTopkScratch = 96;

// One wave: softmax over the E <= 64 logits of one token and its top-k.  The
// max and the sum are the halving trees (the sum's additions in the order of
// wave_tree_sum); the k largest probabilities in turn, ties to the lower id,
// as ranks: lane l's key (bits of p) << 32 | (64 - l) is distinct and orders
// the lanes by probability then lower id, so the j-th selection is the lane
// with j larger keys, counted over the 64 keys in `scratch` (kTopkScratch
// words of this wave's LDS).  The chosen lanes write their slot; with renorm
// the weights are divided by their sum taken in selection order.
__device__ void token_topk(const float* __restrict__ lrow, int E, int topk, int renorm, int32_t* ids32,
                           int64_t* ids64, float* wts, int32_t* lds_ids, uint64_t* scratch) {
  const int l = lane_id();
  const float v = l < E ? lrow[l] : -__builtin_huge_valf();
  const float m = tree_max(v);
  const float ex = l < E ? uexp(v - m) : 0.0f;
  const float S = tree_sum(ex);
  const float p = l < E ? ex / S : 0.0f;
  const uint64_t key = l < E ? (((uint64_t)__float_as_uint(p) << 32) | (uint64_t)(kWave - l)) : 0ull;
  scratch[l] = key;
  int rank = 0;
#pragma unroll
  for (int j = 0; j < kWave; j += 2) {
    const u64x2 kk = *(const u64x2*)(scratch + j);
    rank += (kk[0] > key ? 1 : 0) + (kk[1] > key ? 1 : 0);
  }
  const bool chosen = l < E && rank < topk;
  float w = p;
  if (renorm) {
    float* sel = (float*)(scratch + kWave);
    if (chosen) sel[rank] = p;
    float d = 0.0f;  // the renormaliser, summed in selection order
    for (int j0 = 0; j0 < topk; j0 += 8) {
      float sv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) sv[i] = sel[min(j0 + i, topk - 1)];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (j0 + i < topk) d = d + sv[i];
    }
    w = p / d;
  }
  if (chosen) {
    if (ids32) ids32[rank] = l;
    if (ids64) ids64[rank] = l;
    if (wts) wts[rank] = w;
    if (lds_ids) lds_ids[rank] = l;
  }
}

__global__ void __launch_bounds__(256) k_softmax_topk(const float* __restrict__ logits, int T, int E, int topk,
                                                      int renorm, int32_t* ids32, int64_t* ids64, float* wts) {
  __shared__ uint64_t scratch[4][kTopkScratch];
  const int w = (int)(threadIdx.x >> 6);
  const int t = (int)blockIdx.x * 4 + w;
  if (t >= T) return;
  const int64_t o = (int64_t)t * topk;
  token_topk(logits + (int64_t)t * E, E, topk, renorm, ids32 ? ids32 + o : nullptr, ids64 ? ids64 + o : nullptr,
             wts ? wts + o : nullptr, nullptr, scratch[w]);
}

// ---------------------------------------------------------------- grouping

constexpr int kMaxGroupExperts = 1024;

// Lanes of the wave whose key equals this lane's (keys < 2^bits): one ballot
// per key bit.
__device__ __forceinline__ uint64_t same_key_lanes(int key, int bits) {
  uint64_t m = ~0ull;
  for (int b = 0; b < bits; ++b) {
    const int bit = (key >> b) & 1;
    const uint64_t on = __ballot(bit);
    m &= bit ? on : ~on;
  }
  return m;
}

// Set bits of m below this lane.
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}


// Groups R rows by clamped expert id, stably: a group holds its rows in row
// order.  `idof(r)` returns row r's raw id.  One workgroup of up to 16 waves
// and E <= blockDim.x; `hist` is LDS of (waves x E) ints, `part` of 3 x 16.
//
// Wave w owns the rows [w * chunk, (w + 1) * chunk).  Pass 1 counts its rows
// per expert, 64 rows at a time: the lanes holding one expert find each other
// with one ballot per key bit, and the lowest of them adds their number.  The
// counts are turned into each wave's first position per expert (experts in
// order, waves in order inside an expert), and pass 2 walks the same rows
// again, placing each at its wave's cursor plus its rank among the batch's
// lanes of the same expert.  No atomics, and the order is fixed.
template <typename IdOf>
__device__ void group_rows(IdOf idof, int R, int E, int bm, const GroupTables& g, int* hist, int* part) {
  const int tid = (int)threadIdx.x;
  const int nt = (int)blockDim.x;
  const int nw = nt / kWave;
  const int w = tid / kWave;
  const int bits = 32 - __builtin_clz((unsigned)E);  // key E (no row) fits too
  for (int i = tid; i < nw * E; i += nt) hist[i] = 0;
  __syncthreads();
  const int chunk = ((R + nw - 1) / nw + kWave - 1) / kWave * kWave;
  const int r0 = w * chunk;
  const int r1 = min(R, r0 + chunk);
  int* my = hist + w * E;
  for (int b = r0; b < r1; b += kWave) {
    const int r = b + lane_id();
    const int e = r < r1 ? clamp_expert(idof(r), E) : E;
    const uint64_t m = same_key_lanes(e, bits);
    if (e < E && lanes_below(m) == 0) my[e] += __popcll(m);
  }
  __syncthreads();

  // per expert: rows, row tiles and whether it is a group; exclusive prefix
  // sums over the experts (per wave, then across the waves' totals)
  int c = 0;
  if (tid < E) {
    for (int v = 0; v < nw; ++v) {
      const int h = hist[v * E + tid];
      hist[v * E + tid] = c;
      c += h;
    }
  }
  const int tiles = c > 0 ? (c + bm - 1) / bm : 0;
  const int nz = c > 0 ? 1 : 0;
  const int ic = wave_scan_i(c), it = wave_scan_i(tiles), in = wave_scan_i(nz);
  if (lane_id() == kWave - 1) {
    part[w] = ic;
    part[16 + w] = it;
    part[32 + w] = in;
  }
  __syncthreads();
  int pc = 0, pt = 0, pn = 0;
  for (int v = 0; v < w; ++v) {
    pc += part[v];
    pt += part[16 + v];
    pn += part[32 + v];
  }
  const int start = pc + ic - c, tile0 = pt + it - tiles, grp = pn + in - nz;
  if (tid < E) {
    if (c > 0) {
      stg(g.group_expert + grp, tid);
      stg(g.group_start + grp, start);
      if (g.tile_start) stg(g.tile_start + grp, tile0);
    }
    for (int v = 0; v < nw; ++v) hist[v * E + tid] += start;
    if (tid == E - 1) {
      stg(g.group_start + grp + nz, start + c);
      if (g.tile_start) stg(g.tile_start + grp + nz, tile0 + tiles);
      stg(g.n_groups, grp + nz);
    }
  }
  __syncthreads();

  for (int b = r0; b < r1; b += kWave) {
    const int r = b + lane_id();
    const int e = r < r1 ? clamp_expert(idof(r), E) : E;
    const uint64_t m = same_key_lanes(e, bits);
    const int rank = lanes_below(m);
    const int base = e < E ? my[e] : 0;
    if (e < E) {
      const int pos = base + rank;
      stg(g.group_rows + pos, r);
      if (g.inv) stg(g.inv + r, pos);
      if (rank == 0) my[e] = base + __popcll(m);
    }
  }
}

// LDS of group_rows for a workgroup of `threads` threads.
__host__ __device__ constexpr size_t group_lds_bytes(int threads, int E) {
  return ((size_t)(threads / 64) * E + 48) * sizeof(int);
}

__global__ void __launch_bounds__(1024) k_group(const int32_t* __restrict__ ids, int R, int E, int bm, GroupTables g) {
  extern __shared__ int lds_group[];
  group_rows([&](int r) { return ids[r]; }, R, E, bm, g, lds_group + 48, lds_group);
}

// ---------------------------------------------------------------- prefill routing over many workgroups
//
// k_topk_count: a wave per token (softmax + top-k), 16 tokens per workgroup;
// the workgroup's rows per expert go to hist[b] (every expert, zeros
// included), and k_group_scatter_hist places them as for the fused routing
// (16-token blocks).  A reservation by one atomic add per (workgroup, expert)
// on the experts' row totals took about half the launch at T=4096 (256
// workgroups on 64 addresses) and made the order inside a group the atomics'.

constexpr int kCountThreads = 1024;
constexpr int kCountTokens = kCountThreads / 64;

__global__ void __launch_bounds__(kCountThreads) k_topk_count(const float* __restrict__ logits, int T, int E, int topk,
                                                              int renorm, int32_t* __restrict__ ids32,
                                                              float* __restrict__ wts, int32_t* __restrict__ hist) {
  __shared__ int cnt[kRouteMaxExperts];
  __shared__ uint64_t scratch[kCountTokens][kTopkScratch];
  const int b = (int)blockIdx.x;
  const int tid = (int)threadIdx.x;
  const int t0 = b * kCountTokens;
  const int t1 = min(T, t0 + kCountTokens);
  for (int e = tid; e < E; e += kCountThreads) cnt[e] = 0;
  const int t = t0 + tid / kWave;
  if (t < t1) {
    const int64_t o = (int64_t)t * topk;
    token_topk(logits + (int64_t)t * E, E, topk, renorm, ids32 + o, nullptr, wts + o, nullptr, scratch[tid / kWave]);
  }
  __syncthreads();  // the block's ids (global) are visible to the whole workgroup
  for (int64_t r = (int64_t)t0 * topk + tid; r < (int64_t)t1 * topk; r += kCountThreads)
    atomicAdd(&cnt[clamp_expert(ids32[r], E)], 1);
  __syncthreads();
  for (int e = tid; e < E; e += kCountThreads) stg(hist + (int64_t)b * E + e, cnt[e]);
}

// ---------------------------------------------------------------- prefill routing, T below 2048
//
// k_logits_topk: a workgroup of 16 waves owns 4 tokens and every expert
// (E <= 64).  Its x rows go to LDS (and to xb, rounded to bf16, when asked)
// while each wave loads the router rows of its 4 experts (4w .. 4w+3) for
// every k step at once: one memory latency for both.  Wave w then computes
// the 4 tokens' logits of its experts (the tile kernel's chains over
// k = lane + 64 j and its trees: the same bits) into LDS and the logits
// buffer; after a barrier waves 0-3 run one token's softmax + top-k each, and
// the workgroup's rows per expert go to hist[b] (every expert, zeros
// included).  k_group_scatter_hist: workgroup b sums hist over all counting
// workgroups and over those before it, derives the tables (workgroup 0
// writes them) and places its rows.  No counters to clear.

constexpr int kFusedTokens = 4;
constexpr int kRouteWaves = 16;
constexpr int kFusedSteps = 20;  // router k steps per batch (H <= 1280 in one batch)

__global__ void __launch_bounds__(kRouteWaves * 64) k_logits_topk(
    float* __restrict__ logits, uint16_t* __restrict__ xb, const float* __restrict__ x, int64_t ldx,
    const float* __restrict__ router, int T, int E, int H, int topk, int renorm, int32_t* __restrict__ ids32,
    float* __restrict__ wts, int32_t* __restrict__ hist) {
  __shared__ float xs[kFusedTokens * kLogitsMaxH];
  __shared__ float lg[kFusedTokens][64];
  __shared__ int cnt[64];
  __shared__ int ids_lds[kFusedTokens * 64];
  __shared__ uint64_t scratch[kFusedTokens][kTopkScratch];
  const int b = (int)blockIdx.x;
  const int w = (int)(threadIdx.x >> 6);
  const int l = lane_id();
  const int tid = (int)threadIdx.x;
  const int t0 = b * kFusedTokens;
  const int nt = min(kFusedTokens, T - t0);
  const int nj = H / kWave;
  // wave w's 4 experts, rotated by the workgroup (the workgroups of an XCD then
  // ask for different router rows at the same moment, not all for the same
  // rows in the same order)
  const int e0 = 4 * ((w + b) % kRouteWaves);
  const bool active = e0 < E;
  if (tid < 64) cnt[tid] = 0;
  // The x rows' loads are issued first, then every router value: the x rows
  // land first, and once they are in LDS the fmas of step j wait only for
  // step j's router values (with the router loads first, staging x waited for
  // all of them).
  const bool xvec = (((uintptr_t)x | (uintptr_t)(ldx * 4) | (uintptr_t)(H * 4)) & 15) == 0;
  constexpr int kXv = kFusedTokens * kLogitsMaxH / 4 / (kRouteWaves * kWave);
  const int h4 = H / 4;
  f32x4 xv[kXv];
  if (xvec) {
    // 16-byte pieces, every thread's loads issued before the first is stored
    // (a loop of single loads waited out one memory latency per element)
#pragma unroll
    for (int j = 0; j < kXv; ++j) {
      const int i = tid + j * kRouteWaves * kWave;
      const int t = min(i / h4, nt - 1);
      xv[j] = *(const UOCR_GLOBAL f32x4*)(x + (int64_t)(t0 + t) * ldx + 4 * (i - (i / h4) * h4));
    }
  }
  const float* wl = router + (int64_t)min(e0, E - 1) * H + l;
  int64_t wo[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) wo[e] = (int64_t)min(e, E - 1 - min(e0, E - 1)) * H;
  float wa[kFusedSteps][4];
  if (active) {
#pragma unroll
    for (int jj = 0; jj < kFusedSteps; ++jj)
#pragma unroll
      for (int e = 0; e < 4; ++e) wa[jj][e] = ldg(wl + wo[e] + min(jj, nj - 1) * kWave);
  }
  if (xvec) {
#pragma unroll
    for (int j = 0; j < kXv; ++j) {
      const int i = tid + j * kRouteWaves * kWave;
      const int t = i / h4;
      const int k = 4 * (i - t * h4);
      if (t < nt) {
        *(f32x4*)(xs + t * H + k) = xv[j];
        if (xb != nullptr) {
          const uint32_t lo = (uint32_t)f32_to_bf16_rne(xv[j].x) | ((uint32_t)f32_to_bf16_rne(xv[j].y) << 16);
          const uint32_t hi = (uint32_t)f32_to_bf16_rne(xv[j].z) | ((uint32_t)f32_to_bf16_rne(xv[j].w) << 16);
          *(uint2*)(xb + (int64_t)(t0 + t) * H + k) = make_uint2(lo, hi);
        }
      }
    }
  } else {
    for (int i = tid; i < nt * H; i += kRouteWaves * kWave) {
      const int t = i / H;
      const int k = i - t * H;
      const float v = ldg(x + (int64_t)(t0 + t) * ldx + k);
      xs[t * H + k] = v;
      if (xb != nullptr) xb[(int64_t)(t0 + t) * H + k] = f32_to_bf16_rne(v);
    }
  }
  __syncthreads();
  if (active) {
    float p[kFusedTokens][4];
#pragma unroll
    for (int t = 0; t < kFusedTokens; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) p[t][e] = 0.0f;
    const float* xl = xs + l;
    for (int j0 = 0; j0 < nj; j0 += kFusedSteps) {
      if (j0 > 0) {
#pragma unroll
        for (int jj = 0; jj < kFusedSteps; ++jj)
#pragma unroll
          for (int e = 0; e < 4; ++e) wa[jj][e] = ldg(wl + wo[e] + min(j0 + jj, nj - 1) * kWave);
      }
#pragma unroll
      for (int jj = 0; jj < kFusedSteps; ++jj) {
        if (j0 + jj < nj) {
#pragma unroll
          for (int t = 0; t < kFusedTokens; ++t) {
            const float xv = xl[min(t, nt - 1) * H + (j0 + jj) * kWave];
#pragma unroll
            for (int e = 0; e < 4; ++e) p[t][e] = __builtin_fmaf(xv, wa[jj][e], p[t][e]);
          }
        }
      }
    }
    // lane 16 r of sums[t] holds token t's logit of expert e0 + tree_row_value(r)
    float flat[kFusedTokens * 4], sums[kFusedTokens];
#pragma unroll
    for (int t = 0; t < kFusedTokens; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) flat[t * 4 + e] = p[t][e];
    tree_sum_quads(flat, sums);
    const int e = e0 + tree_row_value(l >> 4);
#pragma unroll
    for (int t = 0; t < kFusedTokens; ++t) {
      if ((l & 15) == 0 && t < nt && e < E) {
        lg[t][e] = sums[t];
        logits[(int64_t)(t0 + t) * E + e] = sums[t];
      }
    }
  }
  __syncthreads();
  if (w < nt) {
    const int64_t o = (int64_t)(t0 + w) * topk;
    token_topk(lg[w], E, topk, renorm, ids32 + o, nullptr, wts + o, ids_lds + w * topk, scratch[w]);
  }
  __syncthreads();
  const int rows = nt * topk;
  for (int r = tid; r < rows; r += kRouteWaves * kWave) atomicAdd(&cnt[clamp_expert(ids_lds[r], E)], 1);
  __syncthreads();
  if (tid < E) stg(hist + (int64_t)b * E + tid, cnt[tid]);
}

constexpr int kScatterRows = 256;  // rows ranked at once (a pass per 256 rows of a block)

__global__ void __launch_bounds__(256) k_group_scatter_hist(const int32_t* __restrict__ ids, int T, int E, int topk,
                                                            int bm, int blocks, int block_tokens,
                                                            const int32_t* __restrict__ hist, GroupTables g) {
  __shared__ int part_before[4][64];
  __shared__ int wcnt[4][64];  // a pass's rows per (wave, expert)
  __shared__ int part_tot[4][64];
  __shared__ int cursor[64];
  const int b = (int)blockIdx.x;
  const int tid = (int)threadIdx.x;
  const int e = tid & 63;
  const int c = tid >> 6;
  // four threads per expert, each over every fourth counting workgroup, 16
  // loads in flight at a time (indices past the last block re-read it and
  // are not counted)
  constexpr int kBatch = 16;
  int before = 0, tot = 0;
  if (e < E) {
    for (int v0 = c; v0 < blocks; v0 += 4 * kBatch) {
      int h[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) h[i] = ldg(hist + (int64_t)min(v0 + 4 * i, blocks - 1) * E + e);
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int v = v0 + 4 * i;
        before += v < b ? h[i] : 0;
        tot += v < blocks ? h[i] : 0;
      }
    }
  }
  part_before[c][e] = before;
  part_tot[c][e] = tot;
  __syncthreads();
  if (tid < 64) {
    // per-expert sums (in a fixed order), then the scans over the experts in one wave
    before = part_before[0][e] + part_before[1][e] + part_before[2][e] + part_before[3][e];
    tot = e < E ? part_tot[0][e] + part_tot[1][e] + part_tot[2][e] + part_tot[3][e] : 0;
    const int tiles = tot > 0 ? (tot + bm - 1) / bm : 0;
    const int nz = tot > 0 ? 1 : 0;
    const int ic = wave_scan_i(tot), it = wave_scan_i(tiles), in = wave_scan_i(nz);
    const int start = ic - tot, tile0 = it - tiles, grp = in - nz;
    if (e < E) {
      cursor[e] = start + before;
      if (b == 0) {
        if (tot > 0) {
          stg(g.group_expert + grp, e);
          stg(g.group_start + grp, start);
          if (g.tile_start) stg(g.tile_start + grp, tile0);
        }
        if (e == E - 1) {
          stg(g.group_start + grp + nz, start + tot);
          if (g.tile_start) stg(g.tile_start + grp + nz, tile0 + tiles);
          stg(g.n_groups, grp + nz);
        }
      }
    }
  }
  // The block's rows in row order within each group: row r goes after the
  // rows of the same expert before it in the block (a rank, not an atomic, so
  // the order does not depend on the schedule), 256 rows a pass: the rank
  // inside the wave from ballots over the expert id's bits, plus the rows of
  // that expert in the pass's earlier waves.
  const int64_t r0 = (int64_t)b * block_tokens * topk;
  const int nr = (int)min((int64_t)T * topk - r0, (int64_t)block_tokens * topk);
  const int w = tid >> 6;
  for (int c0 = 0; c0 < nr; c0 += kScatterRows) {
    const bool live = tid < nr - c0;
    __syncthreads();  // the cursors are final for the rows before this pass
    wcnt[w][tid & 63] = 0;
    // (lanes past the rows take key 64, which no row has)
    const int ex = live ? clamp_expert(ldg(ids + r0 + c0 + tid), E) : 64;
    const uint64_t same = same_key_lanes(ex, 7);
    const int below = lanes_below(same);
    __syncthreads();
    if (live && below == 0) wcnt[w][ex] = __builtin_popcountll(same);
    __syncthreads();
    if (live) {
      int pos = cursor[ex] + below;
      for (int v = 0; v < w; ++v) pos += wcnt[v][ex];
      stg(g.group_rows + pos, (int32_t)(r0 + c0 + tid));
      if (g.inv) stg(g.inv + r0 + c0 + tid, pos);
    }
    __syncthreads();  // every position read the cursors
    if (tid < E) cursor[tid] += wcnt[0][tid] + wcnt[1][tid] + wcnt[2][tid] + wcnt[3][tid];
  }
}

constexpr int kSmallTokens = 64;

__global__ void __launch_bounds__(1024) k_route_small(const float* __restrict__ logits, int T, int E, int topk,
                                                      int renorm, int32_t* ids32, float* wts, GroupTables g) {
  extern __shared__ int lds_group[];
  __shared__ int ids_lds[kSmallTokens * 64];
  __shared__ uint64_t scratch[16][kTopkScratch];  // blockDim.x <= 1024
  const int nw = (int)(blockDim.x >> 6);
  for (int t = (int)(threadIdx.x >> 6); t < T; t += nw) {
    const int64_t o = (int64_t)t * topk;
    token_topk(logits + (int64_t)t * E, E, topk, renorm, ids32 + o, nullptr, wts + o, ids_lds + o,
               scratch[threadIdx.x >> 6]);
  }
  __syncthreads();
  group_rows([&](int r) { return ids_lds[r]; }, T * topk, E, 1, g, lds_group + 48, lds_group);
}

// ---------------------------------------------------------------- combine

constexpr int kCombineThreads = 320;  // 1280 columns as float4
constexpr int kCombineMaxK = 8;  // rows loaded per round

// A workgroup per token; a thread takes W = 4 consecutive columns (16-byte
// loads, when every row and `out` are 16-byte aligned) or W = 1.
template <int W>
__global__ void __launch_bounds__(kCombineThreads) k_combine(float* __restrict__ out, const float* __restrict__ y,
                                                             int64_t ldy, const float* __restrict__ wts,
                                                             const int32_t* __restrict__ inv,
                                                             const float* __restrict__ shared, int T, int H, int topk,
                                                             int parts) {
  typedef float vec __attribute__((ext_vector_type(W)));
  const int t = (int)blockIdx.x;
  for (int n = W * (int)threadIdx.x; n < H; n += W * kCombineThreads) {
    vec acc = {};
    // up to kCombineMaxK rows in flight; the fma chain stays in slot order
    for (int j0 = 0; j0 < topk; j0 += kCombineMaxK) {
      vec v[kCombineMaxK];
#pragma unroll
      for (int j = 0; j < kCombineMaxK; ++j) {
        if (j0 + j < topk) {
          const int i = t * topk + j0 + j;
          const int row = inv ? ldc(inv + i) : i;
          v[j] = *(const UOCR_GLOBAL vec*)(y + (int64_t)row * ldy + n);
        }
      }
#pragma unroll
      for (int j = 0; j < kCombineMaxK; ++j) {
        if (j0 + j < topk) {
          const float wj = ldc(wts + t * topk + j0 + j);
#pragma unroll
          for (int c = 0; c < W; ++c) acc[c] = __builtin_fmaf(wj, v[j][c], acc[c]);
        }
      }
    }
    // the shared experts' sums, one K range after another (T x H floats apart)
    for (int r = 0; shared && r < parts; ++r) {
      const vec sh = *(const UOCR_GLOBAL vec*)(shared + ((int64_t)r * T + t) * H + n);
#pragma unroll
      for (int c = 0; c < W; ++c) acc[c] = acc[c] + sh[c];
    }
    *(UOCR_GLOBAL vec*)(out + (int64_t)t * H + n) = acc;
  }
}

}  // namespace

hipError_t launch_logits(float* logits, const float* x, int64_t ldx, const float* router, int T, int E, int H,
                         uint16_t* xb, hipStream_t s, int32_t* zero, int nzero) {
  if (T <= 0) return hipSuccess;
  if (H == 20 * kWave && E == 64 && T >= 2048) {
    // every XCD an equal share of the token blocks (those past T return at once)
    const int ntb = (T + 31) / 32;
    const dim3 grid((unsigned)(kXcds * ((ntb + kXcds - 1) / kXcds) * ((E + 15) / 16)));
    UOCR_LAUNCH("logits", (k_logits_ring<8, 16, 20>), grid, dim3(256), 0, s, logits, xb, x, ldx, router, T, E, zero,
                nzero);
    return hipGetLastError();
  }
  if (H % kWave == 0 && T >= 2048) {
    const dim3 grid((unsigned)((E + 15) / 16), (unsigned)((T + 31) / 32));
    UOCR_LAUNCH("logits", (k_logits_tile<8, 16>), grid, dim3(256), 0, s, logits, xb, x, ldx, router, T, E, H, zero, nzero);
    return hipGetLastError();
  }
  if (H % kWave == 0 && T >= 256) {
    const dim3 grid((unsigned)((E + 7) / 8), (unsigned)((T + 15) / 16));
    UOCR_LAUNCH("logits", (k_logits_tile<4, 8>), grid, dim3(256), 0, s, logits, xb, x, ldx, router, T, E, H, zero, nzero);
    return hipGetLastError();
  }
  if (H % kWave == 0 && H <= kLogitsMaxH && (xb != nullptr || T > 8)) {
    // every wave: 4 tokens x 4 experts, all loads issued at once
    const dim3 grid((unsigned)((E + 15) / 16), (unsigned)((T + 3) / 4));
    const int nj = H / kWave;
    if (nj <= 16)
      UOCR_LAUNCH("logits", k_logits_wide<16>, grid, dim3(256), 0, s, logits, xb, x, ldx, router, T, E, H, zero, nzero);
    else if (nj <= 20)
      UOCR_LAUNCH("logits", k_logits_wide<20>, grid, dim3(256), 0, s, logits, xb, x, ldx, router, T, E, H, zero, nzero);
    else
      UOCR_LAUNCH("logits", k_logits_wide<32>, grid, dim3(256), 0, s, logits, xb, x, ldx, router, T, E, H, zero, nzero);
    return hipGetLastError();
  }
  if (xb != nullptr || zero != nullptr) return hipErrorInvalidValue;
  if (T <= 8) {
    // decode: one wave per expert, every token of the step against it
    const dim3 grid((unsigned)((E + 3) / 4), 1);
    UOCR_LAUNCH("logits", (k_logits<8, 1>), grid, dim3(256), 0, s, logits, x, ldx, router, T, E, H);
  } else {
    const dim3 grid((unsigned)((E + 15) / 16), (unsigned)((T + 15) / 16));
    UOCR_LAUNCH("logits", (k_logits<16, 4>), grid, dim3(256), 0, s, logits, x, ldx, router, T, E, H);
  }
  return hipGetLastError();
}

hipError_t launch_softmax_topk(const float* logits, int T, int E, int topk, int renorm, int32_t* ids32,
                               int64_t* ids64, float* wts, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  UOCR_LAUNCH("softmax_topk", k_softmax_topk, dim3((T + 3) / 4), dim3(256), 0, s, logits, T, E, topk, renorm, ids32, ids64,
                     wts);
  return hipGetLastError();
}

hipError_t launch_group(const int32_t* ids, int R, int E, int bm, const GroupTables& g, hipStream_t s) {
  if (E > kMaxGroupExperts) return hipErrorInvalidValue;
  UOCR_LAUNCH("group", k_group, dim3(1), dim3(1024), group_lds_bytes(1024, E), s, ids, R, E, bm, g);
  return hipGetLastError();
}

int route_count_blocks(int T) { return (T + kCountTokens - 1) / kCountTokens; }

hipError_t launch_topk_group(const float* logits, int T, int E, int topk, int renorm, int32_t* ids32, float* wts,
                             int bm, const GroupTables& g, int32_t* hist, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  if (E > kRouteMaxExperts) return hipErrorInvalidValue;
  const int blocks = route_count_blocks(T);
  UOCR_LAUNCH("topk_count", k_topk_count, dim3(blocks), dim3(kCountThreads), 0, s, logits, T, E, topk, renorm, ids32,
              wts, hist);
  UOCR_LAUNCH("group_scatter", k_group_scatter_hist, dim3(blocks), dim3(256), 0, s, ids32, T, E, topk, bm, blocks,
              kCountTokens, hist, g);
  return hipGetLastError();
}

int fused_route_blocks(int T) { return (T + kFusedTokens - 1) / kFusedTokens; }

hipError_t launch_logits_topk_group(float* logits, uint16_t* xb, const float* x, int64_t ldx, const float* router,
                                    int T, int E, int H, int topk, int renorm, int32_t* ids32, float* wts, int bm,
                                    const GroupTables& g, int32_t* hist, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  if (E > 64 || H % kWave != 0 || H > kLogitsMaxH || topk > 64) return hipErrorInvalidValue;
  const int blocks = fused_route_blocks(T);
  UOCR_LAUNCH("logits_topk", k_logits_topk, dim3(blocks), dim3(kRouteWaves * kWave), 0, s, logits, xb, x, ldx,
              router, T, E, H, topk, renorm, ids32, wts, hist);
  UOCR_LAUNCH("group_scatter", k_group_scatter_hist, dim3(blocks), dim3(256), 0, s, ids32, T, E, topk, bm, blocks,
              kFusedTokens, hist, g);
  return hipGetLastError();
}

hipError_t launch_route_small(const float* logits, int T, int E, int topk, int renorm, int32_t* ids32, float* wts,
                              const GroupTables& g, hipStream_t s) {
  if (T > kSmallTokens || E > 64 || topk > 64) return hipErrorInvalidValue;
  UOCR_LAUNCH("route_small", k_route_small, dim3(1), dim3(1024), group_lds_bytes(1024, E), s, logits, T, E, topk,
              renorm, ids32, wts, g);
  return hipGetLastError();
}

hipError_t launch_combine(float* out, const float* y, int64_t ldy, const float* wts, const int32_t* inv,
                          const float* shared, int T, int H, int topk, hipStream_t s, int shared_parts) {
  if (T <= 0) return hipSuccess;
  if (shared_parts < 1) return hipErrorInvalidValue;
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if (H % 4 == 0 && ldy % 4 == 0 && a16(out) && a16(y) && (shared == nullptr || a16(shared)))
    UOCR_LAUNCH("combine", k_combine<4>, dim3(T), dim3(kCombineThreads), 0, s, out, y, ldy, wts, inv, shared, T, H,
                topk, shared_parts);
  else
    UOCR_LAUNCH("combine", k_combine<1>, dim3(T), dim3(kCombineThreads), 0, s, out, y, ldy, wts, inv, shared, T, H,
                topk, shared_parts);
  return hipGetLastError();
}

}  // namespace uocr
