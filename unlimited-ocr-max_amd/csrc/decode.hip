// The decode-step MoE layer (MoE.decode_rows, unlimited_ocr_max/decoder.py:641-655)
// as ONE persistent kernel for batch <= 8 tokens.
//
// Arithmetic: bitwise the multi-kernel path (gemv.hip, route.hip) and so the CPU
// oracle: router logits in the 64-lane tree order; softmax + top-k; per (row,
// column) int8 chains per 128-group folded by fma(scale, gsum, acc) in group
// order (unlimited_ocr_max/kernels/moe_int8.mojo:126-148) or bf16 chains per
// 128-element chunk added in chunk order; SwiGLU; the routing-weighted fma
// combine plus the shared experts.
//
// Work decomposition.  The layer is a list of tasks; task i belongs to wave
// i mod (number of waves), and every wave walks its tasks in order:
//   router     one expert's logits for every token          (E tasks)
//   sgu        shared gate or up, 64 columns x one chunk     (Fs/64 x 2 x H/128)
//   rgu        routed gate or up of one selected expert,
//              64 columns x one chunk                        (slots x F/64 x 2 x H/G)
//   sdn        shared down, 64 columns x one chunk           (H/64 x Fs/128)
//   rdn        routed down, 64 columns x one chunk           (slots x H/64 x F/G)
// A chunk task streams a 64-row x 128-byte weight tile with coalesced 16-byte
// loads (8 lanes per 128-byte line), transposes it through LDS so each lane
// holds one weight row, runs the bit-exact chain for every token row of its
// expert, and stores the chain results (plus the group scale) as partials.
// The task that completes a unit's last chunk (an atomic counter) folds the
// partials in chunk order: SwiGLU for gate/up, the combine for the last down
// unit of a column block.  The last router task computes the softmax, top-k
// and expert grouping.  A task only ever waits on tasks with smaller indices,
// and every wave of the grid is resident (the grid is sized to the occupancy),
// so the waits end; each wait is also bounded and records an error if it
// ever runs out.  The next task's weight tile is loaded into registers while
// the current one is computed.
//
// Cross-workgroup data (partials, h, y, routing tables) is written and read
// with device-coherent (agent-scope) accesses, and every counter update waits
// for the wave's earlier stores first.  The control counters live in a
// library-owned buffer that the last wave of a launch resets to zero.
#include "uocr_device.h"
#include "uocr_kernels.h"

namespace uocr {

namespace {

constexpr int kWavesPerWg = 4;
constexpr int kTileRow = 144;   // LDS bytes per weight row of a tile (128 + 16 pad)
constexpr int kTileBytes = 64 * kTileRow;
constexpr uint32_t kSpinLimit = 1u << 21;

// ctl word indices
constexpr int C_DONE = 0, C_ROUTER = 1, C_READY = 2, C_HS = 3, C_ERR = 4, C_BASE = 8;

__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ld_dev(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits for this wave's earlier stores, then adds 1 to a counter; returns the
// old value in every lane.
__device__ __forceinline__ uint32_t signal(uint32_t* c) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  uint32_t old = 0;
  if (lane_id() == 0) old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return __shfl(old, 0, kWave);
}

// Spins until *c >= target; on running out of spins, records an error and
// returns (the results of such a launch are wrong, but it ends).
__device__ void wait_ge(uint32_t* ctl, int idx, uint32_t target) {
  for (uint32_t spin = 0;; ++spin) {
    if (ld_dev(ctl + idx) >= target) return;
    if (spin > kSpinLimit) {
      if (lane_id() == 0) st_dev(ctl + C_ERR, 1u);
      return;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

// The same pointer, asserted wave-uniform (both halves through readfirstlane).
__device__ __forceinline__ const float* uniform_ptr(const float* p) {
  const uint64_t u = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return (const float*)(((uint64_t)hi << 32) | lo);
}

// Rows a chain template covers for B rows (1, 2, 4 or 8): the activation stage
// holds that many rows so padded rows read inside it.
__host__ __device__ constexpr int padded_rows(int B) { return B <= 1 ? 1 : B <= 2 ? 2 : B <= 4 ? 4 : 8; }

// Phase timestamps of a task (the constant-rate wall clock), when tracing.
#define UOCR_TRACE(a, task, slot)                                                    \
  do {                                                                               \
    if ((a).trace != nullptr && lane_id() == 0) (a).trace[(int64_t)(task) * 8 + (slot)] = (int64_t)wall_clock64(); \
  } while (0)

enum TaskKind : int { T_ROUTER = 0, T_SGU = 1, T_RGU = 2, T_SDN = 3, T_RDN = 4, T_NONE = 5 };

struct Task {
  int kind;
  int slot;   // routed expert slot (group index)
  int cb;     // 64-column block
  int p;      // 0 gate, 1 up (gate/up tasks)
  int c;      // chunk
  int e;      // router: expert
};

__device__ __forceinline__ Task decode_task(const FusedArgs& a, int t) {
  Task k{T_NONE, 0, 0, 0, 0, 0};
  if (t < a.n_router) {
    k.kind = T_ROUTER;
    k.e = t;
    return k;
  }
  t -= a.n_router;
  if (t < a.n_sgu) {
    k.kind = T_SGU;
    const int per_unit = 2 * a.ch_h;
    k.cb = t / per_unit;
    const int r = t - k.cb * per_unit;
    k.p = r / a.ch_h;
    k.c = r - k.p * a.ch_h;
    return k;
  }
  t -= a.n_sgu;
  if (t < a.n_rgu) {
    k.kind = T_RGU;
    const int per_unit = 2 * a.ch_h;
    const int unit = t / per_unit;
    const int r = t - unit * per_unit;
    k.slot = unit / a.cb_f;
    k.cb = unit - k.slot * a.cb_f;
    k.p = r / a.ch_h;
    k.c = r - k.p * a.ch_h;
    return k;
  }
  t -= a.n_rgu;
  if (t < a.n_sdn) {
    k.kind = T_SDN;
    k.cb = t / a.ch_fs;
    k.c = t - k.cb * a.ch_fs;
    return k;
  }
  t -= a.n_sdn;
  if (t < a.n_rdn) {
    k.kind = T_RDN;
    const int unit = t / a.ch_f;
    k.c = t - unit * a.ch_f;
    k.slot = unit / a.cb_h;
    k.cb = unit - k.slot * a.cb_h;
    return k;
  }
  return k;
}

// --------------------------------------------------------------------------- weight tiles

// Registers holding one task's weight tile(s) in flight: up to 2 sub-tiles
// of 64 rows x 128 bytes, 8 x 16 bytes per lane each.
struct Stage {
  i32x4 v[2][8];
};

// Issues the loads of one 64x128-byte sub-tile of a row-major [N, Kbytes]
// matrix (rows n0.., bytes kb0..kb0+127): instruction i, lane l -> row
// n0 + 8i + l/8, bytes (l%8)*16.  Rows past N repeat row N-1.
__device__ __forceinline__ void issue_rows(i32x4 (&v)[8], const char* base, int64_t row_bytes, int n0, int N,
                                           int64_t kb0) {
  const int l = lane_id();
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int n = min(n0 + 8 * i + (l >> 3), N - 1);
    v[i] = *(const UOCR_GLOBAL i32x4*)(base + (int64_t)n * row_bytes + kb0 + (l & 7) * 16);
  }
}

// The same for a K-blocked bf16 [K/16, N, 16] matrix: the sub-tile is 64 rows
// x 64 elements (K blocks kb0..kb0+3); instruction i, lane l -> block
// kb0 + i/2, row n0 + 32*(i%2) + l/2, half l%2.
__device__ __forceinline__ void issue_kblocked(i32x4 (&v)[8], const uint16_t* w, int N, int n0, int kb0) {
  const int l = lane_id();
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int kb = kb0 + (i >> 1);
    const int n = min(n0 + 32 * (i & 1) + (l >> 1), N - 1);
    v[i] = *(const UOCR_GLOBAL i32x4*)(w + ((int64_t)kb * N + n) * 16 + (l & 1) * 8);
  }
}

// Writes a staged sub-tile to the wave's LDS tile in row order (row r at
// r*kTileRow, 16-byte piece q at q*16).
__device__ __forceinline__ void tile_store(char* tile, const i32x4 (&v)[8], bool kblocked) {
  const int l = lane_id();
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int r, q;
    if (kblocked) {
      r = 32 * (i & 1) + (l >> 1);
      q = (i >> 1) * 2 + (l & 1);
    } else {
      r = 8 * i + (l >> 3);
      q = l & 7;
    }
    *(i32x4*)(tile + r * kTileRow + q * 16) = v[i];
  }
}

// ---------------------------------------------------------------------------- chains

// Activation access: scalar loads of the kernel input x, or LDS broadcast of
// an activation staged by the wave (h, hs: produced inside the kernel).
struct XSrc {
  const float* row[8];   // x rows (global) when from_lds == false
  const float* lds;      // staged rows, row r at lds + r * 128, when from_lds
  bool from_lds;
};


// Elements of the chunk handled per step: 16, or 8 for 8 rows (the x values
// of a step live in scalar registers).
template <int R, bool LDSX>
constexpr int kStep = LDSX ? 4 : (R > 4 ? 8 : 16);

// x[r][k..k+S-1] of every row r < R into registers: scalar loads of the kernel
// input, or LDS broadcasts of a staged activation.
template <int R, int S, bool LDSX>
__device__ __forceinline__ void load_x(const XSrc& xs, int k, float (&xv)[8][16]) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if constexpr (LDSX) {
#pragma unroll
      for (int v = 0; v < S / 4; ++v) {
        const f32x4 q = *(const f32x4*)(xs.lds + r * 128 + k + 4 * v);
        xv[r][4 * v] = q.x;
        xv[r][4 * v + 1] = q.y;
        xv[r][4 * v + 2] = q.z;
        xv[r][4 * v + 3] = q.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < S; ++j) xv[r][j] = ldc(xs.row[r] + k + j);
    }
  }
}

// One int8 sub-tile: the lane's 128 weights of its row, chained per token row
// into part[] in k order.
template <int R, bool LDSX>
__device__ __forceinline__ void chain_int8(const char* tile, const XSrc& xs, float (&part)[8]) {
  constexpr int S = kStep<R, LDSX>;
  const int l = lane_id();
#pragma unroll 1
  for (int k0 = 0; k0 < 128; k0 += S) {
    const i32x4 wq = *(const i32x4*)(tile + l * kTileRow + (k0 & ~15));
    float xv[8][16];
    load_x<R, S, LDSX>(xs, k0, xv);
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const int kk = (k0 & 15) + j;  // byte of the 16-byte piece
      const float wv = (float)(int8_t)(wq[kk >> 2] >> (8 * (kk & 3)));
#pragma unroll
      for (int r = 0; r < R; ++r) part[r] = __builtin_fmaf(wv, xv[r][j], part[r]);
    }
  }
}

// One bf16 sub-tile: the lane's 64 weights of its row (k = koff..koff+63).
template <int R, bool LDSX>
__device__ __forceinline__ void chain_bf16(const char* tile, const XSrc& xs, int koff, float (&part)[8]) {
  constexpr int S = kStep<R, LDSX>;
  const int l = lane_id();
#pragma unroll 1
  for (int k0 = 0; k0 < 64; k0 += S) {
    float xv[8][16];
    load_x<R, S, LDSX>(xs, koff + k0, xv);
    // 16-byte pieces of 8 bf16 covering the step
    constexpr int NP = S >= 8 ? S / 8 : 1;
    i32x4 wq[NP];
#pragma unroll
    for (int pc = 0; pc < NP; ++pc) wq[pc] = *(const i32x4*)(tile + l * kTileRow + ((k0 & ~7) + 8 * pc) * 2);
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const int kk = (k0 & 7) + j;  // element counted from the first piece
      const uint32_t word = (uint32_t)wq[kk >> 3][(kk & 7) >> 1];
      const float wv = (kk & 1) == 0 ? bf16_lo(word) : bf16_hi(word);
#pragma unroll
      for (int r = 0; r < R; ++r) part[r] = __builtin_fmaf(wv, xv[r][j], part[r]);
    }
  }
}

template <int R, bool LDSX>
__device__ __forceinline__ void run_chain(bool int8, int subtiles, char* tile, const Stage& st, bool kblocked,
                                          const XSrc& xs, float (&part)[8]) {
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    if (s >= subtiles) break;
    tile_store(tile, st.v[s], kblocked);
    __builtin_amdgcn_wave_barrier();
    if (int8)
      chain_int8<R, LDSX>(tile, xs, part);
    else
      chain_bf16<R, LDSX>(tile, xs, s * 64, part);
    __builtin_amdgcn_wave_barrier();
  }
}

template <bool LDSX>
__device__ __forceinline__ void run_chain_rows(int R, bool int8, int subtiles, char* tile, const Stage& st,
                                               bool kblocked, const XSrc& xs, float (&part)[8]) {
  if (R <= 1)
    run_chain<1, LDSX>(int8, subtiles, tile, st, kblocked, xs, part);
  else if (R <= 2)
    run_chain<2, LDSX>(int8, subtiles, tile, st, kblocked, xs, part);
  else if (R <= 4)
    run_chain<4, LDSX>(int8, subtiles, tile, st, kblocked, xs, part);
  else
    run_chain<8, LDSX>(int8, subtiles, tile, st, kblocked, xs, part);
}

// ---------------------------------------------------------------------------- the kernel

struct Wave {
  char* tile;     // kTileBytes
  float* xstage;  // B * 128 floats
};

__device__ __forceinline__ uint32_t* ctl_sgu(const FusedArgs& a) { return a.ctl + C_BASE; }
__device__ __forceinline__ uint32_t* ctl_hready(const FusedArgs& a) { return a.ctl + C_BASE + a.cb_fs; }
__device__ __forceinline__ uint32_t* ctl_sdn(const FusedArgs& a) { return ctl_hready(a) + 64; }
__device__ __forceinline__ uint32_t* ctl_out(const FusedArgs& a) { return ctl_sdn(a) + a.cb_h; }
__device__ __forceinline__ uint32_t* ctl_rgu(const FusedArgs& a) { return ctl_out(a) + a.cb_h; }
__device__ __forceinline__ uint32_t* ctl_rdn(const FusedArgs& a) { return ctl_rgu(a) + a.max_slots * a.cb_f; }

__device__ __forceinline__ bool routing_ready(const FusedArgs& a) { return ld_dev(a.ctl + C_READY) != 0u; }

// Loads the weight tile(s) of a chunk task into registers.  Routed tasks need
// the routing; returns false for a routed slot beyond the selected experts.
__device__ __attribute__((always_inline)) bool issue_task(const FusedArgs& a, const Task& k, Stage& st) {
  if (k.kind == T_SGU) {
    const uint16_t* w = k.p == 0 ? a.sh_gate : a.sh_up;
    issue_kblocked(st.v[0], w, a.Fs, k.cb * 64, k.c * 8);
    issue_kblocked(st.v[1], w, a.Fs, k.cb * 64, k.c * 8 + 4);
    return true;
  }
  if (k.kind == T_SDN) {
    issue_kblocked(st.v[0], a.sh_down, a.H, k.cb * 64, k.c * 8);
    issue_kblocked(st.v[1], a.sh_down, a.H, k.cb * 64, k.c * 8 + 4);
    return true;
  }
  if (k.kind == T_RGU || k.kind == T_RDN) {
    if (k.slot >= ld_dev(a.n_groups)) return false;
    const int e = ld_dev(a.group_expert + k.slot);
    const bool gu = k.kind == T_RGU;
    const char* w = (const char*)(gu ? (k.p == 0 ? a.gate_w : a.up_w) : a.down_w);
    const int N = gu ? a.F : a.H;
    const int K = gu ? a.H : a.F;
    if (a.int8) {
      issue_rows(st.v[0], w + (int64_t)e * N * K, K, k.cb * 64, N, (int64_t)k.c * 128);
    } else {
      const int64_t rb = (int64_t)K * 2;
      issue_rows(st.v[0], w + (int64_t)e * N * rb, rb, k.cb * 64, N, (int64_t)k.c * 256);
      issue_rows(st.v[1], w + (int64_t)e * N * rb, rb, k.cb * 64, N, (int64_t)k.c * 256 + 128);
    }
    return true;
  }
  return false;
}

// router task: logits[t][e] for every token t of the step (H <= 2048): the
// lane's router values and each token's x values are loaded in one batch.
constexpr int kMaxHPerLane = 32;

__device__ __attribute__((always_inline)) void router_task(const FusedArgs& a, int e) {
  const int l = lane_id();
  const float* wr = a.router + (int64_t)e * a.H;
  const int nk = (a.H - l + kWave - 1) / kWave;  // k = l + 64j, j < nk
  float w[kMaxHPerLane];
#pragma unroll
  for (int j = 0; j < kMaxHPerLane; ++j) w[j] = j < nk ? ldg(wr + l + kWave * j) : 0.0f;
  for (int t = 0; t < a.B; ++t) {
    const float* xr = a.x + (int64_t)t * a.H + l;
    float xv[kMaxHPerLane];
#pragma unroll
    for (int j = 0; j < kMaxHPerLane; ++j) xv[j] = j < nk ? ldg(xr + kWave * j) : 0.0f;
    float p = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxHPerLane; ++j)
      if (j < nk) p = __builtin_fmaf(xv[j], w[j], p);
    const float v = wave_tree_sum(p);
    if (l == 0) st_dev(a.logits + t * 64 + e, v);
  }
}

// The routing (by the last router task): softmax + top-k per token, then the
// selected (token, slot) rows grouped by expert in ascending expert id, rows
// ascending within a group.
__device__ __attribute__((always_inline)) void routing(const FusedArgs& a) {
  const int l = lane_id();
  const int R = a.B * a.topk;
  for (int t = 0; t < a.B; ++t) {
    const float v = l < a.E ? ld_dev(a.logits + t * 64 + l) : -__builtin_huge_valf();
    float m = v;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
    const float ex = l < a.E ? uexp(v - m) : 0.0f;
    const float S = __shfl(wave_tree_sum(ex), 0, kWave);
    const float pr = l < a.E ? ex / S : 0.0f;
    uint64_t key = l < a.E ? (((uint64_t)__float_as_uint(pr) << 32) | (uint64_t)(kWave - l)) : 0ull;
    float d = 0.0f;
    for (int j = 0; j < a.topk; ++j) {
      uint64_t best = key;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        const uint64_t o = __shfl_xor(best, off, kWave);
        best = o > best ? o : best;
      }
      const int sel = kWave - (int)(best & 0xFFFFFFFFu);
      const float ws = __shfl(pr, sel, kWave);
      d = d + ws;
      if (l == sel) key = 0ull;
      if (l == 0) {
        st_dev(a.ids + t * a.topk + j, sel);
        st_dev(a.wts + t * a.topk + j, ws);
      }
    }
    if (a.renorm && l == 0)
      for (int j = 0; j < a.topk; ++j) st_dev(a.wts + t * a.topk + j, ld_dev(a.wts + t * a.topk + j) / d);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // grouping: lane r holds row r's expert (R <= 64)
  const int my = l < R ? ld_dev(a.ids + l) : -1;
  int ng = 0, off = 0;
  for (int e = 0; e < a.E; ++e) {
    const uint64_t mask = __ballot(my == e);
    if (mask == 0ull) continue;
    if (my == e) {
      const int rank = __builtin_popcountll(mask & ((1ull << l) - 1ull));
      st_dev(a.group_rows + off + rank, l);
    }
    if (l == 0) {
      st_dev(a.group_expert + ng, e);
      st_dev(a.group_start + ng, off);
    }
    off += __builtin_popcountll(mask);
    ++ng;
  }
  if (l == 0) {
    st_dev(a.group_start + ng, off);
    st_dev(a.n_groups, ng);
  }
}

// Rows of a unit: tokens (shared) or the routed rows of a group.
struct Rows8 {
  int cnt;
  int row[8];
};

__device__ __attribute__((always_inline)) Rows8 unit_rows(const FusedArgs& a, const Task& k) {
  Rows8 r;
  if (k.kind == T_SGU || k.kind == T_SDN) {
    r.cnt = a.B;
#pragma unroll
    for (int i = 0; i < 8; ++i) r.row[i] = min(i, a.B - 1);
  } else {
    const int s0 = ld_dev(a.group_start + k.slot);
    r.cnt = ld_dev(a.group_start + k.slot + 1) - s0;
#pragma unroll
    for (int i = 0; i < 8; ++i) r.row[i] = __builtin_amdgcn_readfirstlane(ld_dev(a.group_rows + s0 + min(i, r.cnt - 1)));
  }
  return r;
}

// Stages activation rows (produced in this kernel) for a chunk: rows
// src[row*ld + k0 .. +128), every load issued before the first LDS write.
__device__ __attribute__((always_inline)) void stage_rows(float* xstage, const float* src, int64_t ld, int64_t k0,
                                                         const Rows8& rows) {
  const int l = lane_id();
  float v[16];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const float* srow = src + (int64_t)rows.row[r] * ld + k0;
    v[2 * r] = r < rows.cnt ? ld_dev(srow + l) : 0.0f;
    v[2 * r + 1] = r < rows.cnt ? ld_dev(srow + 64 + l) : 0.0f;
  }
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    if (r < rows.cnt) {
      xstage[r * 128 + l] = v[2 * r];
      xstage[r * 128 + 64 + l] = v[2 * r + 1];
    }
  }
  __builtin_amdgcn_wave_barrier();
}

// Folds the partials of a unit in chunk order; returns acc[r] for the lane's
// column.  Per row, the chunk partials (and the scales, once) are loaded in
// one batch, then chained.
constexpr int kMaxChunks = 16;

__device__ __attribute__((always_inline)) void fold(const float* part, const float* scl, int chunks, int rm, int cnt,
                                                   bool int8, float (&acc)[8]) {
  const int l = lane_id();
  float s[kMaxChunks];
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) s[c] = (int8 && c < chunks) ? ld_dev(scl + c * 64 + l) : 1.0f;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    acc[r] = 0.0f;
    if (r < cnt) {
      float v[kMaxChunks];
#pragma unroll
      for (int c = 0; c < kMaxChunks; ++c) v[c] = c < chunks ? ld_dev(part + (c * rm + r) * 64 + l) : 0.0f;
      float x = 0.0f;
#pragma unroll
      for (int c = 0; c < kMaxChunks; ++c)
        if (c < chunks) x = int8 ? __builtin_fmaf(s[c], v[c], x) : x + v[c];
      acc[r] = x;
    }
  }
}

__device__ __attribute__((always_inline)) void combine_block(const FusedArgs& a, int cb) {
  const int l = lane_id();
  const int n = cb * 64 + l;
  if (n >= a.H) return;
  constexpr int kMaxK = 8;
  for (int t = 0; t < a.B; ++t) {
    float w[kMaxK], y[kMaxK];
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
      const int i = t * a.topk + j;
      w[j] = j < a.topk ? ld_dev(a.wts + i) : 0.0f;
      y[j] = j < a.topk ? ld_dev(a.y + (int64_t)i * a.H + n) : 0.0f;
    }
    const float shv = ld_dev(a.sh + (int64_t)t * a.H + n);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxK; ++j)
      if (j < a.topk) acc = __builtin_fmaf(w[j], y[j], acc);
    a.out[(int64_t)t * a.H + n] = acc + shv;
  }
}

__device__ __attribute__((always_inline)) void after_down_fold(const FusedArgs& a, int cb) {
  const uint32_t target = (uint32_t)ld_dev(a.n_groups) + 1u;
  if (signal(ctl_out(a) + cb) + 1u == target) combine_block(a, cb);
}

__device__ __attribute__((always_inline)) void chunk_task(const FusedArgs& a, const Wave& W, const Task& k, int tid) {
  const int l = lane_id();
  UOCR_TRACE(a, tid, 0);
  if (k.kind == T_RGU || k.kind == T_RDN) {
    wait_ge(a.ctl, C_READY, 1u);
    if (k.slot >= ld_dev(a.n_groups)) return;
  }
  UOCR_TRACE(a, tid, 1);
  Stage st;
  issue_task(a, k, st);
  if (a.trace != nullptr) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    UOCR_TRACE(a, tid, 2);
  }
  const Rows8 rows = unit_rows(a, k);
  const bool routed = k.kind == T_RGU || k.kind == T_RDN;
  const bool int8 = routed && a.int8;
  const int subtiles = int8 ? 1 : 2;
  const bool kblocked = !routed;
  int e = 0;
  if (routed) e = ld_dev(a.group_expert + k.slot);

  XSrc xs;
  xs.from_lds = false;
  xs.lds = W.xstage;
  int64_t kx0;  // first activation element of the chunk
  if (k.kind == T_SGU || k.kind == T_RGU) {
    kx0 = (int64_t)k.c * 128;
    const int div = k.kind == T_RGU ? a.topk : 1;
#pragma unroll
    for (int r = 0; r < 8; ++r) xs.row[r] = uniform_ptr(a.x + (int64_t)(rows.row[r] / div) * a.H + kx0);
  } else if (k.kind == T_SDN) {
    wait_ge(a.ctl, C_HS, (uint32_t)a.cb_fs);
    stage_rows(W.xstage, a.hs, a.Fs, (int64_t)k.c * 128, rows);
    xs.from_lds = true;
  } else {
    wait_ge(a.ctl, C_BASE + a.cb_fs + k.slot, (uint32_t)a.cb_f);
    stage_rows(W.xstage, a.h, a.F, (int64_t)k.c * 128, rows);
    xs.from_lds = true;
  }

  UOCR_TRACE(a, tid, 3);
  float part[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) part[r] = 0.0f;
  if (xs.from_lds)
    run_chain_rows<true>(rows.cnt, int8, subtiles, W.tile, st, kblocked, xs, part);
  else
    run_chain_rows<false>(rows.cnt, int8, subtiles, W.tile, st, kblocked, xs, part);

  // partials (and, for int8, the chunk's scale per column)
  const int rm = a.B;
  float* pbase;
  float* sbase = nullptr;
  int unit_chunks, pc;
  uint32_t* counter;
  if (k.kind == T_SGU) {
    unit_chunks = 2 * a.ch_h;
    pc = k.p * a.ch_h + k.c;
    pbase = a.p_sgu + (int64_t)k.cb * unit_chunks * rm * 64;
    counter = ctl_sgu(a) + k.cb;
  } else if (k.kind == T_RGU) {
    unit_chunks = 2 * a.ch_h;
    pc = k.p * a.ch_h + k.c;
    const int unit = k.slot * a.cb_f + k.cb;
    pbase = a.p_rgu + (int64_t)unit * unit_chunks * rm * 64;
    sbase = a.s_rgu + (int64_t)unit * unit_chunks * 64;
    counter = ctl_rgu(a) + unit;
  } else if (k.kind == T_SDN) {
    unit_chunks = a.ch_fs;
    pc = k.c;
    pbase = a.p_sdn + (int64_t)k.cb * unit_chunks * rm * 64;
    counter = ctl_sdn(a) + k.cb;
  } else {
    unit_chunks = a.ch_f;
    pc = k.c;
    const int unit = k.slot * a.cb_h + k.cb;
    pbase = a.p_rdn + (int64_t)unit * unit_chunks * rm * 64;
    sbase = a.s_rdn + (int64_t)unit * unit_chunks * 64;
    counter = ctl_rdn(a) + unit;
  }
#pragma unroll
  for (int r = 0; r < 8; ++r)
    if (r < rows.cnt) st_dev(pbase + (pc * rm + r) * 64 + l, part[r]);
  const int N = (k.kind == T_SGU) ? a.Fs : (k.kind == T_RGU ? a.F : a.H);
  const int n = min(k.cb * 64 + l, N - 1);
  if (int8) {
    const float* scales = k.kind == T_RGU ? (k.p == 0 ? a.gate_s : a.up_s) : a.down_s;
    const int groups = k.kind == T_RGU ? a.ch_h : a.ch_f;
    st_dev(sbase + pc * 64 + l, ldg(scales + ((int64_t)e * N + n) * groups + k.c));
  }
  UOCR_TRACE(a, tid, 4);
  const bool last = signal(counter) + 1u == (uint32_t)unit_chunks;
  UOCR_TRACE(a, tid, 5);
  if (!last) return;

  // ---- the last chunk of the unit: fold
  const bool valid = k.cb * 64 + l < N;
  float acc[8];
  if (k.kind == T_SGU || k.kind == T_RGU) {
    float accu[8];
    const int half = a.ch_h;
    fold(pbase, sbase, half, rm, rows.cnt, int8, acc);
    fold(pbase + (int64_t)half * rm * 64, sbase ? sbase + half * 64 : nullptr, half, rm, rows.cnt, int8, accu);
    float* dst = k.kind == T_SGU ? a.hs : a.h;
    const int ldd = k.kind == T_SGU ? a.Fs : a.F;
    if (valid) {
#pragma unroll
      for (int r = 0; r < 8; ++r)
        if (r < rows.cnt) st_dev(dst + (int64_t)rows.row[r] * ldd + n, silu(acc[r]) * accu[r]);
    }
    if (k.kind == T_SGU)
      signal(a.ctl + C_HS);
    else
      signal(ctl_hready(a) + k.slot);
  } else {
    fold(pbase, sbase, unit_chunks, rm, rows.cnt, int8, acc);
    float* dst = k.kind == T_SDN ? a.sh : a.y;
    if (valid) {
#pragma unroll
      for (int r = 0; r < 8; ++r)
        if (r < rows.cnt) st_dev(dst + (int64_t)rows.row[r] * a.H + n, acc[r]);
    }
    after_down_fold(a, k.cb);
  }
  UOCR_TRACE(a, tid, 6);
}

__global__ void __launch_bounds__(kWavesPerWg * 64) k_decode_fused(FusedArgs a) {
  extern __shared__ char lds[];
  const int wv = (int)(threadIdx.x >> 6);
  Wave W;
  W.tile = lds + wv * (kTileBytes + padded_rows(a.B) * 128 * 4);
  W.xstage = (float*)(W.tile + kTileBytes);
  const int nwaves = (int)gridDim.x * kWavesPerWg;
  int t = (int)blockIdx.x * kWavesPerWg + wv;

  for (; t < a.n_tasks; t += nwaves) {
    const Task k = decode_task(a, t);
    if (k.kind == T_ROUTER) {
      UOCR_TRACE(a, t, 0);
      router_task(a, k.e);
      UOCR_TRACE(a, t, 3);
      if (signal(a.ctl + C_ROUTER) + 1u == (uint32_t)a.n_router) {
        UOCR_TRACE(a, t, 5);
        routing(a);
        signal(a.ctl + C_READY);
        UOCR_TRACE(a, t, 6);
      }
    } else if (k.kind != T_NONE) {
      chunk_task(a, W, k, t);
    }
    if (a.trace != nullptr && lane_id() == 0) a.trace[(int64_t)t * 8 + 7] = (int64_t)((int)blockIdx.x * kWavesPerWg + wv);
  }

  // the last wave of the launch resets the control words for the next one
  if (signal(a.ctl + C_DONE) + 1u == (uint32_t)nwaves) {
    const int words = a.ctl_words;
    for (int i = lane_id(); i < words; i += kWave)
      if (i != C_DONE && i != C_ERR) st_dev(a.ctl + i, 0u);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (lane_id() == 0) st_dev(a.ctl + C_DONE, 0u);
  }
}

}  // namespace

int fused_ctl_words(int cb_fs, int cb_h, int cb_f, int max_slots) {
  return C_BASE + cb_fs + 64 + cb_h + cb_h + max_slots * cb_f + max_slots * cb_h;
}

size_t fused_lds_bytes(int B) { return (size_t)kWavesPerWg * (kTileBytes + padded_rows(B) * 128 * 4); }

hipError_t fused_grid(int B, int* grid) {
  int dev = 0, cus = 0, per_cu = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess)
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_decode_fused, kWavesPerWg * 64, fused_lds_bytes(B));
  if (e != hipSuccess) return e;
  *grid = cus * (per_cu < 1 ? 1 : per_cu);
  return hipSuccess;
}

hipError_t launch_decode_fused(const FusedArgs& a, int grid, hipStream_t s) {
  UOCR_LAUNCH("decode_fused", k_decode_fused, dim3(grid), dim3(kWavesPerWg * 64), fused_lds_bytes(a.B), s, a);
  return hipGetLastError();
}

__global__ void k_zero_words(uint32_t* p, int n) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i < n) p[i] = 0u;
}

hipError_t launch_zero_words(uint32_t* p, int n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  UOCR_LAUNCH("zero_words", k_zero_words, dim3((n + 255) / 256), dim3(256), 0, s, p, n);
  return hipGetLastError();
}

}  // namespace uocr
