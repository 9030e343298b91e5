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
// Work decomposition.  One workgroup of 12 waves per CU; the layer is a list of
// tasks dealt round robin to the waves (task t to the wave of rank t mod
// waves, ranks interleaved across workgroups so neighbouring tasks land on
// different CUs and XCDs), every wave walking its tasks in increasing order:
//   router  one expert's logits for a few tokens (on every XCD)      (E x tokens / r_tok)
//   sgu     shared gate or up: 64 columns x one 128-chunk of H         (Fs/64 x 2 x H/128)
//   rgu     routed gate+up of one selected expert: a few columns,
//           every chunk of H (lane = column, projection, chunk)        (experts x F/c_gu)
//   rdn     routed down of one selected expert: a few columns, every
//           chunk of F (lane = column, chunk)                          (experts x H/c_dn)
//   sfold   shared gate/up partials of 64 columns, one token -> SwiGLU
//           -> hs                                                      (Fs/64 x B)
//   sdn     shared down: 64 columns x one 128-chunk of Fs              (H/64 x Fs/128)
//   comb    64 columns, one token: shared-down partials -> sh, then the
//           weighted combine of the token's routed rows plus sh        (H/64 x B)
// The sgu tasks need no routing: a wave runs those while the routing is
// computed.  The shared folds and down partials, which wait for the sgu
// partials, come after the routed gate/up tasks, so that no routed gate/up
// task is queued behind such a wait, but before the routed down tasks: their
// inputs are long ready when a wave reaches them, and the combine, which waits
// for them, is not kept waiting at the end.  A routed task holds every chunk of its columns, so
// its per-group fold runs
// inside the wave (lane shuffles); only the shared experts, whose chunks are
// spread over tasks, fold partials written by other waves.  Each lane loads
// the weights of its own row and chunk (128 int8 or 256 bf16 bytes, 16 bytes
// per load) straight into registers; 12 waves per CU keep enough loads in
// flight without a software pipeline.
//
// Synchronisation.  Every value one wave hands to another (logits, partials,
// h, hs, y) is stored as a 64-bit pair (fp32 bits, launch tag) with one
// device-coherent store, and the consumer polls the pairs it needs until all
// carry the tag of the current launch: no counters and no fences on the data
// path.  Each workgroup computes the routing itself from the tagged logits.
// A task waits only on tasks with smaller indices and every workgroup of the
// grid is resident (the grid is sized to the occupancy), so the waits end.
// Each wait is also bounded: one that runs out (another kernel holding CUs
// for tens of milliseconds) sets the error word and takes NaN for what it
// waited for, so the launch still ends with NaN in the outputs that depend on
// it; while the word stays set, every later launch on the slot writes NaN,
// until the host reads and clears it (uocr_moe_fused_errors).  The
// launch tag is the control word EPOCH + 1: every workgroup reads EPOCH at its
// start and then adds one to its ARRIVED counter; the workgroup whose
// addition completes the grid's count (known once its control wave has
// finished its tasks, so the atomics' round trips stay off the other waves'
// work) clears the counters and advances EPOCH.  Every workgroup has read
// EPOCH by then, and the next launch on the stream starts after this one
// ends, so no wave ever takes another launch's tag.
// The tagged buffers and control words are library-owned and zeroed when
// allocated; tags start at 1, so no zeroed word is ever taken for data.
#include "uocr_device.h"
#include "uocr_kernels.h"

namespace uocr {

namespace {

constexpr int kWaves = kFusedWaves;
constexpr int kThreads = kWaves * kWave;
constexpr int kXPad = kFusedXPad;

// control words
// Words every workgroup touches are spread over 128-byte lines (kLine words
// apart): agent-scope loads and atomics skip the L2, and those on one line
// queue one after another at the memory (256 workgroups on one word cost
// microseconds, and on this architecture a wave's later waits for its loads
// also wait for its earlier atomics).
//   C_EPOCH   + k * kLine, k < kSpread: the epoch, one copy per line;
//             workgroup b reads copy b % kSpread at its start
//   C_ARRIVED + k * kLine, k < kSpread: workgroups arrived, workgroup b adds
//             to counter b % kSpread; the workgroup that completes a
//             counter adds to C_ARRIVED2, and the one that completes that
//             is the launch's last
constexpr int kLine = 32, kSpread = 32;
constexpr int C_ERR = 4, C_ARRIVED2 = kLine, C_EPOCH = 2 * kLine, C_ARRIVED = C_EPOCH + kSpread * kLine;
static_assert(C_ARRIVED + kSpread * kLine <= kFusedCtlWords, "control words");

// Workgroup b runs on XCD b % kXcds (the dispatcher deals workgroups to the
// XCDs round robin).  Every XCD computes all the logits itself into its own
// copy, with workgroup-scope stores that stay in that XCD's L2, where its
// workgroups' polls find them: the hand-off never waits in the memory's
// queues behind the weight streams.
constexpr int kXcds = kFusedXcds;
constexpr int kLogitCopies = kFusedLogitCopies;
constexpr int kLogitCopyWords = kFusedLogitCopyWords;

// Kernel arguments are read through a constant-address-space reference
// (scalar loads); the task loop re-derives the pointer every iteration so
// that the compiler reloads fields where they are used instead of keeping
// every field in scalar registers across the loop.
#define KA __attribute__((address_space(4)))

// Lane index through a volatile asm: recomputed where it is used, so that the
// compiler does not hoist lane-derived values (shuffle addresses, masks) out
// of the task loop and keep them live across every task.
__device__ __forceinline__ int lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// v of lane src (0..63).
__device__ __forceinline__ float shfl(float v, int src) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(v)));
}
__device__ __forceinline__ uint32_t shfl(uint32_t v, int src) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)v);
}
__device__ __forceinline__ uint64_t shfl(uint64_t v, int src) {
  return ((uint64_t)shfl((uint32_t)(v >> 32), src) << 32) | shfl((uint32_t)v, src);
}

__device__ __forceinline__ uint32_t ld_word(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_word(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_pair(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_pair(uint64_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A pair for waves of the same XCD only: the workgroup-scope store stays in the
// XCD's L2, where their (agent-scope) polls find it without a memory round trip.
__device__ __forceinline__ void st_pair_xcd(uint64_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ float pair_value(uint64_t q) { return __uint_as_float((uint32_t)q); }
__device__ __forceinline__ bool pair_has(uint64_t q, uint32_t tag) { return (uint32_t)(q >> 32) == tag; }

// One round of a bounded poll: true once every lane is ready.  `spin` starts
// at the wait's limit (FusedArgs::spin_limit rounds, tens of milliseconds by
// default: real waits take microseconds; 0 makes every wait fail at once) and
// counts down.  When it runs out,
// or once another wait has failed (the error word, read every 8192 rounds), it
// records an error and lets the wave go on with spin = 0 (expired()): the
// waiter then takes NaN for the values it waited for, so every output that
// depends on them is NaN, and the launch still ends.
__device__ __forceinline__ bool poll_done(bool ready, uint32_t& spin, uint32_t* ctl) {
  if (spin != 0u && __all(ready)) return true;  // a limit of 0 fails every wait (the host's test of this path)
  if (spin != 0u) --spin;
  if (spin == 0u || ((spin & 8191u) == 0u && ld_word(ctl + C_ERR) != 0u)) {
    if (lane() == 0) st_word(ctl + C_ERR, 1u);
    spin = 0u;
    return true;
  }
  __builtin_amdgcn_s_sleep(2);
  return false;
}
__device__ __forceinline__ bool expired(uint32_t spin) { return spin == 0u; }

// Polls n tagged pairs p[i * stride] (i < n <= N, per lane) until all carry
// `tag`; their values land in v[0..n).  A round trip is about a microsecond
// under the weight streams.  kPollProbe: each lane probes a single pair
// (`probe`, else the first) until it arrives, then loads the set until it is
// complete: the many waves of a long wait keep their reads light, which the
// weight streams they share the memory with need.  kPollEager: when `eager`,
// a first round loads the whole set (one round trip when it is there
// already), then as kPollProbe.  kPollFull: every round loads the set (one
// round trip after the last pair lands; for the few waves of the combine).
// The addresses advance from p (no per-index offsets for the compiler to
// hoist out of the task loop).
enum : int { kPollProbe = 0, kPollEager = 1, kPollFull = 2 };
template <int N>
__device__ __forceinline__ bool load_pairs(const uint64_t* p, int64_t stride, int n, uint32_t tag, float (&v)[N]) {
  uint64_t q[N];
  const uint64_t* a = p;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    q[i] = ld_pair(a);
    if (i + 1 < n) a += stride;
  }
  bool ok = true;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    v[i] = pair_value(q[i]);
    ok = ok && pair_has(q[i], tag);
  }
  return ok;
}
template <int N, int MODE = kPollProbe>
__device__ __forceinline__ void poll_pairs(const uint64_t* p, int64_t stride, int n, uint32_t tag, uint32_t* ctl,
                                           uint32_t limit, float (&v)[N], const uint64_t* probe = nullptr,
                                           bool eager = true) {
  uint32_t spin = limit;
  if (MODE == kPollEager && eager && __all(load_pairs<N>(p, stride, n, tag, v))) return;
  if (MODE != kPollFull) {
    if (probe == nullptr) probe = p;
    while (!poll_done(pair_has(ld_pair(probe), tag), spin, ctl)) {
    }
  }
  while (!poll_done(load_pairs<N>(p, stride, n, tag, v), spin, ctl)) {
  }
  if (expired(spin)) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = __builtin_nanf("");
  }
}

// x / d for 0 <= x < 2^16 and 1 <= d <= 64, from inv = 1/d: (x + 1/2)/d stays
// at least 1/(2d) away from the next integer, far beyond the rounding error.
__device__ __forceinline__ int small_div(int x, float inv) { return (int)(((float)x + 0.5f) * inv); }

// The phase trace (uocr_moe_fused_trace) is compiled in only with
// UOCR_DECODE_TRACE=1: every launch starts with cold instruction caches, so
// code on the paths each workgroup runs once costs a fetch per cache line.
#ifndef UOCR_DECODE_TRACE
#define UOCR_DECODE_TRACE 0
#endif
constexpr bool kTrace = UOCR_DECODE_TRACE != 0;

// Phase timestamps of a task (the constant-rate wall clock), when tracing:
// 0 start, 1 weights landed (waited for only when tracing), 3 inputs polled,
// 4 chains done, 2 end, 5 when the wave learnt the routing, 6 the task kind, 7 the wave.
#define UOCR_TRACE(a, task, slot)                                                                          \
  do {                                                                                                     \
    if (kTrace && (a).trace != nullptr && lane() == 0) (a).trace[(int64_t)(task) * 8 + (slot)] = (int64_t)wall_clock64(); \
  } while (0)
#define UOCR_TRACE_LOADS(a, task)                       \
  do {                                                  \
    if (kTrace && (a).trace != nullptr) {                         \
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); \
      UOCR_TRACE(a, task, 1);                           \
    }                                                   \
  } while (0)

// --------------------------------------------------------------------------- tasks

enum Kind : int { K_ROUTER, K_SGU, K_RGU, K_SFOLD, K_SDN, K_RDN, K_COMB, K_NONE };

struct Task {
  int kind;
  int a;  // router: expert; sgu/sfold: column block of Fs; rgu/rdn: expert slot; sdn/comb: column block of H
  int b;  // sgu: projection; rgu/rdn: column group; sdn: chunk of Fs; sfold/comb: token
  int c;  // sgu: chunk of H
};

__device__ __forceinline__ int task_count(const KA FusedArgs& A, int ng) {
  return A.E + A.n_sgu + A.n_sfold + A.n_sdn + ng * A.per_e_gu + ng * A.per_e_dn + A.n_comb;
}

// Tasks before the routed ones: the router, and the shared gate/up partials
// (which wait for nothing); at small batches (early_shared) also the shared
// folds and down partials, which wait for the sgu partials.  Otherwise these
// follow the routed gate/up tasks (at B=8 their waves are better spent on
// routed tasks: 49.8 against 55.0 us a layer).
__device__ __forceinline__ int unrouted_count(const KA FusedArgs& A) {
  return A.E + A.n_sgu + (A.early_shared ? A.n_sfold + A.n_sdn : 0);
}

// x / d from m = ceil(2^32 / d) (0 for d = 1), exact while x * d < 2^32: a
// multiply-high in place of an integer division's ~40 dependent instructions,
// in the task list's decoding and the stacked kernel's x polls (11-layer
// step B=1 202 -> 191 us, B=8 595 -> 568 us; the single layer's x staging
// kept its division, which measured faster there).
__device__ __forceinline__ int task_div(int x, uint32_t m) { return m ? (int)__umulhi((uint32_t)x, m) : x; }

// Task order: router, sgu, rgu, sfold, sdn, rdn, comb, or at small batches
// (early_shared) router, sgu, sfold, sdn, rgu, rdn, comb (either way every
// task waits only for tasks before it).
__device__ __forceinline__ Task task_at(const KA FusedArgs& A, int ng, int t) {
  if (t < A.E) return {K_ROUTER, t, 0, 0};
  t -= A.E;
  if (t < A.n_sgu) {
    const int u = task_div(t, A.m_2gh);
    const int r = t - u * 2 * A.gh;
    const int p = task_div(r, A.m_gh);
    return {K_SGU, u, p, r - p * A.gh};
  }
  t -= A.n_sgu;
  // the routed gate/up tasks' place: first, or after the shared folds and downs
  const int n_gu = ng * A.per_e_gu;
  const int gu0 = A.early_shared ? A.n_sfold + A.n_sdn : 0;
  if (t >= gu0 && t < gu0 + n_gu) {
    const int s = task_div(t - gu0, A.m_gu);
    return {K_RGU, s, t - gu0 - s * A.per_e_gu, 0};
  }
  if (t >= gu0) t -= n_gu;
  if (t < A.n_sfold) {
    const int u = task_div(t, A.m_b);
    return {K_SFOLD, u, t - u * A.B, 0};
  }
  t -= A.n_sfold;
  if (t < A.n_sdn) {
    const int cb = task_div(t, A.m_gfs);
    return {K_SDN, cb, t - cb * A.gfs, 0};
  }
  t -= A.n_sdn;
  if (t < ng * A.per_e_dn) {
    const int s = task_div(t, A.m_dn);
    return {K_RDN, s, t - s * A.per_e_dn, 0};
  }
  t -= ng * A.per_e_dn;
  if (t < A.n_comb) {
    const int cb = task_div(t, A.m_b);
    return {K_COMB, cb, t - cb * A.B, 0};
  }
  return {K_NONE, 0, 0, 0};
}

// --------------------------------------------------------------------------- routing

// The routing as every wave holds it: `mask` the selected experts, ng their
// number, ids the workgroup's table of routed rows' experts (LDS, row r at
// ids[r], B*topk rows).  Slot s is the s-th selected expert in ascending id.
struct Route {
  uint64_t mask;
  int ng;
  const int* ids;
  int rows;
};

__device__ __forceinline__ int slot_expert(const Route& rt, int s) {
  const int l = lane();
  const bool bit = ((rt.mask >> l) & 1ull) != 0ull;
  const int prefix = __builtin_popcountll(rt.mask & ((1ull << l) - 1ull));
  const uint64_t b = __ballot(bit && prefix == s);
  return (int)__builtin_ctzll(b);
}

// Routed rows of expert e, ascending (a bit per row).
__device__ __forceinline__ uint64_t slot_rows(const Route& rt, int e) {
  const int l = lane();
  const int id = l < rt.rows ? rt.ids[l] : -1;
  return __ballot(id == e);
}

// Softmax + top-k of token t from its tagged logits into the workgroup's
// tables (same steps as route.hip's k_softmax_topk: max, exp, halving-tree
// sum, divide; the k largest probabilities in turn, ties to the lower id),
// then one more on the workgroup's count of routed tokens.
__device__ __attribute__((always_inline)) void route_token(const KA FusedArgs& A, int64_t boff, int64_t twg, int t,
                                                           uint32_t tag,
                                                           int* r_ids,
                                                           float* r_wts, int* r_done, uint64_t* keys) {
  const int l = lane();
  const uint64_t* src = A.logits + boff + (blockIdx.x % kXcds) * kLogitCopyWords + t * 64 + (l < A.E ? l : A.E - 1);
  uint64_t q;
  uint32_t spin = A.spin_limit;
  const bool wtrace = kTrace && A.trace != nullptr && t == 0 && l == 0;
  if (wtrace) A.trace[twg + blockIdx.x * 8 + 0] = (int64_t)wall_clock64();
  do {
    q = ld_pair(src);
  } while (!poll_done(pair_has(q, tag), spin, A.ctl));
  if (wtrace) A.trace[twg + blockIdx.x * 8 + 1] = (int64_t)wall_clock64();
  const bool real = l < A.E;
  const float v = real ? (expired(spin) ? __builtin_nanf("") : pair_value(q)) : -__builtin_huge_valf();
  const float m = tree_max(v);
  if (wtrace) A.trace[twg + blockIdx.x * 8 + 3] = (int64_t)wall_clock64();
  const float ex = real ? uexp(v - m) : 0.0f;
  const float S = tree_sum(ex);
  if (wtrace) A.trace[twg + blockIdx.x * 8 + 4] = (int64_t)wall_clock64();
  const float pr = real ? ex / S : 0.0f;
  // The k largest probabilities in turn, ties to the lower id, as ranks: lane
  // l's key ((bits of pr) << 6 | 63 - l) + 1 (0 past the experts) is distinct
  // and orders lanes exactly that way, so the j-th selection is the lane with
  // j larger keys.  Every lane counts them over the 64 keys in LDS (independent
  // compares, where selecting in turn is six dependent wave reductions).
  const uint64_t key = real ? ((((uint64_t)__float_as_uint(pr)) << 6) | (uint64_t)(63 - l)) + 1ull : 0ull;
  keys[l] = key;
  // (each half's 16 reads issued before its compares: left to the scheduler,
  // the reads went out one or two at a time, each waited for in turn)
  int rank = 0;
#pragma unroll
  for (int h = 0; h < kWave; h += 32) {
    u64x2 kk[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) kk[j] = *(const u64x2*)(keys + h + 2 * j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 16; ++j) rank += (kk[j][0] > key ? 1 : 0) + (kk[j][1] > key ? 1 : 0);
  }
  const bool chosen = real && rank < A.topk;
  float my_w = pr;
  if (A.renorm) {
    // the selected probabilities summed in selection order, then divided
    float* ws = (float*)(keys + kWave);
    if (chosen) ws[rank] = pr;
    float wv[8];  // topk <= 8
#pragma unroll
    for (int j = 0; j < 8; ++j) wv[j] = ws[min(j, A.topk - 1)];
    float d = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < A.topk) d = d + wv[j];
    my_w = pr / d;
  }
  if (wtrace) A.trace[twg + blockIdx.x * 8 + 5] = (int64_t)wall_clock64();
  if (chosen) {
    const int i = t * A.topk + rank;
    r_ids[i] = l;
    r_wts[i] = my_w;
    if (blockIdx.x == 0) {
      if (A.ids_out != nullptr) A.ids_out[i] = l;
      if (A.wts_out != nullptr) A.wts_out[i] = my_w;
    }
  }
  // the tables are in LDS before the count says so
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  if (l == 0) {
    __hip_atomic_fetch_add(r_done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (wtrace) A.trace[twg + blockIdx.x * 8 + 2] = (int64_t)wall_clock64();
  }
}

__device__ __forceinline__ Route make_route(const KA FusedArgs& A, const int* r_ids) {
  const int l = lane();
  Route rt;
  rt.ids = r_ids;
  rt.rows = A.B * A.topk;
  const int id = l < rt.rows ? r_ids[l] : -1;
  const uint32_t lo = tree_or(id >= 0 && id < 32 ? (1u << id) : 0u);
  const uint32_t hi = tree_or(id >= 32 ? (1u << (id - 32)) : 0u);
  rt.mask = ((uint64_t)hi << 32) | lo;
  rt.ng = __builtin_popcountll(rt.mask);
  return rt;
}

// --------------------------------------------------------------------------- weights

// The lane's weights of one task: its row's chunk as 16-byte pieces in k
// order, 8 pieces of 16 int8 or 16 pieces of 8 bf16.
template <bool INT8>
struct Stage {
  i32x4 v[INT8 ? 8 : 16];
};

__device__ __forceinline__ i32x4 ld16(const void* p) { return *(const UOCR_GLOBAL i32x4*)p; }

// A routed expert task: lane l is (column c, projection p, chunk g) =
// ((2c + p) * gh + g) for gate/up, (c * gf + g) for down, and loads its 128
// (int8) or 256 (bf16) contiguous bytes; lanes past the task repeat its last
// lane's row.
template <bool INT8>
__device__ __attribute__((always_inline)) void issue_routed(const KA FusedArgs& A, const KA FusedLayerW& W, bool gu,
                                                            int e, int n0, int ncols, Stage<INT8>& st) {
  const int l = lane();
  const int G = gu ? A.gh : A.gf;
  const int N = gu ? A.F : A.H;
  constexpr int64_t esz = INT8 ? 1 : 2;
  const int lam = min(l, (gu ? 2 : 1) * ncols * G - 1);
  const int cp = small_div(lam, gu ? A.inv_gh : A.inv_gf);
  const int g = lam - cp * G;
  const int c = gu ? cp >> 1 : cp;
  const char* w = (const char*)(gu ? ((cp & 1) ? W.up_w : W.gate_w) : W.down_w);
  const char* p = w + (((int64_t)e * N + n0 + c) * (gu ? A.H : A.F) + (int64_t)g * 128) * esz;
#pragma unroll
  for (int i = 0; i < (INT8 ? 8 : 16); ++i) st.v[i] = ld16(p + 16 * i);
}

// A shared task (K-blocked bf16 [K/16, N, 16]): lane l is column n0 + l and
// loads chunk g, K-blocks 8g..8g+7, 32 bytes each.
__device__ __forceinline__ void issue_kblocked(const uint16_t* w, int N, int n0, int g, Stage<false>& st) {
  const uint16_t* p = w + ((int64_t)(8 * g) * N + n0 + lane()) * 16;
  const int64_t block = (int64_t)N * 16;
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    st.v[i] = ld16(p);
    st.v[i + 1] = ld16(p + 8);
    p += block;
  }
}

// ---------------------------------------------------------------------------- chains

// Makes the weight registers opaque (an empty asm that "modifies" them in
// place): whatever is computed from them cannot be hoisted out of the loop
// the call sits in.
__device__ __forceinline__ void launder(Stage<true>& st) {
  asm volatile("" : "+v"(st.v[0]), "+v"(st.v[1]), "+v"(st.v[2]), "+v"(st.v[3]), "+v"(st.v[4]), "+v"(st.v[5]),
               "+v"(st.v[6]), "+v"(st.v[7]));
}
__device__ __forceinline__ void launder(Stage<false>& st) {
  asm volatile("" : "+v"(st.v[0]), "+v"(st.v[1]), "+v"(st.v[2]), "+v"(st.v[3]), "+v"(st.v[4]), "+v"(st.v[5]),
               "+v"(st.v[6]), "+v"(st.v[7]));
  asm volatile("" : "+v"(st.v[8]), "+v"(st.v[9]), "+v"(st.v[10]), "+v"(st.v[11]), "+v"(st.v[12]), "+v"(st.v[13]),
               "+v"(st.v[14]), "+v"(st.v[15]));
}

// The fp32 chain of one row over the lane's chunk, in k order: acc =
// fma(w_k, x_k, acc) from 0, x_k at xp[k] (LDS).  The activations of piece
// q+1 are read while piece q is computed; their offset passes through an
// empty asm that takes the accumulator, so the read cannot be issued before
// piece q-1 is done and the scheduler cannot hoist every read (128 floats)
// to the top.  Callers run it once per row: a second empty asm makes each
// piece's weights opaque so that the compiler widens them inside the row loop
// instead of hoisting all of them out of it.
template <bool INT8>
__device__ __forceinline__ float chain(const Stage<INT8>& st, const float* xp) {
  constexpr int NP = INT8 ? 8 : 16;  // pieces
  constexpr int EP = INT8 ? 16 : 8;  // elements per piece
  constexpr int NV = EP / 4;         // 4-float LDS reads per piece
  float acc = 0.0f;
  f32x4 cur[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) cur[v] = *(const f32x4*)(xp + 4 * v);
#pragma unroll
  for (int q = 0; q < NP; ++q) {
    f32x4 nxt[NV];
    if (q + 1 < NP) {
      int off = (q + 1) * EP;
      asm volatile("" : "+v"(off) : "v"(acc));
#pragma unroll
      for (int v = 0; v < NV; ++v) nxt[v] = *(const f32x4*)(xp + off + 4 * v);
    }
    const i32x4 wq = st.v[q];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      float w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = 4 * v + j;
        if constexpr (INT8)
          w[j] = (float)(int8_t)((uint32_t)wq[e >> 2] >> (8 * (e & 3)));
        else
          w[j] = (e & 1) ? bf16_hi((uint32_t)wq[e >> 1]) : bf16_lo((uint32_t)wq[e >> 1]);
      }
      acc = __builtin_fmaf(w[0], cur[v].x, acc);
      acc = __builtin_fmaf(w[1], cur[v].y, acc);
      acc = __builtin_fmaf(w[2], cur[v].z, acc);
      acc = __builtin_fmaf(w[3], cur[v].w, acc);
    }
    if (q + 1 < NP) {
#pragma unroll
      for (int v = 0; v < NV; ++v) cur[v] = nxt[v];
    }
  }
  return acc;
}

// Two rows' chains over the same weights: each weight converted once, the
// two fma chains interleaved (each row's chain is chain()'s, in k order from
// 0: the same bits).  Piece q's activations of both rows are read while the
// previous piece is computed, as in chain().
template <bool INT8>
__device__ __forceinline__ void chain2(const Stage<INT8>& st, const float* xp0, const float* xp1, float& out0,
                                       float& out1) {
  constexpr int NP = INT8 ? 8 : 16;
  constexpr int EP = INT8 ? 16 : 8;
  constexpr int NV = EP / 4;
  float a0 = 0.0f, a1 = 0.0f;
  f32x4 c0[NV], c1[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    c0[v] = *(const f32x4*)(xp0 + 4 * v);
    c1[v] = *(const f32x4*)(xp1 + 4 * v);
  }
#pragma unroll
  for (int q = 0; q < NP; ++q) {
    f32x4 n0[NV], n1[NV];
    if (q + 1 < NP) {
      int off = (q + 1) * EP;
      asm volatile("" : "+v"(off) : "v"(a0), "v"(a1));
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        n0[v] = *(const f32x4*)(xp0 + off + 4 * v);
        n1[v] = *(const f32x4*)(xp1 + off + 4 * v);
      }
    }
    const i32x4 wq = st.v[q];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      float w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = 4 * v + j;
        if constexpr (INT8)
          w[j] = (float)(int8_t)((uint32_t)wq[e >> 2] >> (8 * (e & 3)));
        else
          w[j] = (e & 1) ? bf16_hi((uint32_t)wq[e >> 1]) : bf16_lo((uint32_t)wq[e >> 1]);
      }
      a0 = __builtin_fmaf(w[0], c0[v].x, a0);
      a1 = __builtin_fmaf(w[0], c1[v].x, a1);
      a0 = __builtin_fmaf(w[1], c0[v].y, a0);
      a1 = __builtin_fmaf(w[1], c1[v].y, a1);
      a0 = __builtin_fmaf(w[2], c0[v].z, a0);
      a1 = __builtin_fmaf(w[2], c1[v].z, a1);
      a0 = __builtin_fmaf(w[3], c0[v].w, a0);
      a1 = __builtin_fmaf(w[3], c1[v].w, a1);
    }
    if (q + 1 < NP) {
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        c0[v] = n0[v];
        c1[v] = n1[v];
      }
    }
  }
  out0 = a0;
  out1 = a1;
}

// ----------------------------------------------------------------------------- tasks

struct Ctx {
  const float* xs;  // x rows in LDS, row t at t * gh * kXPad, chunk g at + g * kXPad
  const int* r_ids;
  const float* r_wts;
  float* act;       // the wave's activation stage
  uint32_t tag;
  int* landed;      // the workgroup's routed gate/up tasks whose weights have landed (LDS; defer_down)
  int t;            // the running task
  int tr;           // its trace record: t, plus the layer's offset in a stack
  int layer;        // the layer of a stack (0 for one layer)
  int64_t boff;     // the layer's tagged buffers, in words from the first layer's
  const KA FusedLayerW* W;  // the layer's weights
};

// Router task of expert e: the lane's router weights (k = l + 64 j), loaded
// before the x rows are staged, then every token's logit in the 64-lane tree
// order, stored into each copy of the logits.
constexpr int kMaxJ = 32;  // H <= 2048
constexpr int kRouterWaves = kFusedRouterWaves;  // router tasks per workgroup

__device__ __attribute__((always_inline)) void router_load(const KA FusedArgs& A, const KA FusedLayerW& W, int e,
                                                           float (&w)[kMaxJ]) {
  const int l = lane();
  const float* wr = W.router + (int64_t)e * A.H + l;
  const int nk = A.H / kWave;
#pragma unroll
  for (int j = 0; j < kMaxJ; ++j) w[j] = ldg(wr + (j < nk ? j : nk - 1) * kWave);
}

// Logits of expert e for tokens t0 .. t1-1.
template <bool STACK>
__device__ __attribute__((always_inline)) void router_task(const KA FusedArgs& A, const Ctx& C, int e, int t0, int t1,
                                                           const float (&w)[kMaxJ]) {
  const int l = lane();
  const int nk = A.H / kWave;
  uint64_t* dst = A.logits + C.boff + (blockIdx.x % kXcds) * kLogitCopyWords + e;
  if (t1 - t0 == 1) {
    const float* xr = C.xs + t0 * A.gh * kXPad + l;
    // In the stack (router weights loaded during the previous layer, so the
    // chain starts as x lands) the 20 x reads of H = 1280 go out before the
    // chain, without the loop bound's branch between them (179.2 -> 176.5 us
    // for 11 layers at one token); in one layer, whose chain waits for the
    // router rows' first load anyway, the same made the launch slower.
    float p = 0.0f;
    if (STACK && nk == 20) {
      float xv[20];
#pragma unroll
      for (int j = 0; j < 20; ++j) xv[j] = xr[(j >> 1) * kXPad + kWave * (j & 1)];
#pragma unroll
      for (int j = 0; j < 20; ++j) p = __builtin_fmaf(xv[j], w[j], p);
    } else {
#pragma unroll
      for (int j = 0; j < kMaxJ; ++j)
        if (j < nk) p = __builtin_fmaf(xr[(j >> 1) * kXPad + kWave * (j & 1)], w[j], p);
    }
    const float v = tree_sum(p);
    if (l == 0) st_pair_xcd(dst + t0 * 64, v, C.tag);
  } else {
    // four tokens' chains side by side (each in its own order), their lane
    // sums in one quad tree: lane 16 r holds token t + tree_row_value(r)'s
    for (int t = t0; t < t1; t += 4) {
      const float* xr[4];
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xr[i] = C.xs + min(t + i, t1 - 1) * A.gh * kXPad + l;
        p[i] = 0.0f;
      }
#pragma unroll
      for (int j = 0; j < kMaxJ; ++j)
        if (j < nk) {
#pragma unroll
          for (int i = 0; i < 4; ++i) p[i] = __builtin_fmaf(xr[i][(j >> 1) * kXPad + kWave * (j & 1)], w[j], p[i]);
        }
      float v[1];
      tree_sum_quads<4>(p, v);
      const int tt = t + tree_row_value(l >> 4);
      if ((l & 15) == 0 && tt < t1) st_pair_xcd(dst + tt * 64, v[0], C.tag);
    }
  }
  if (t0 == 0) UOCR_TRACE(A, C.tr, 4);
}

// Shared gate or up, 64 columns x chunk g of H, every token: partials.
__device__ __attribute__((always_inline)) void sgu_rows(const KA FusedArgs& A, const Ctx& C, const Task& k,
                                                        Stage<false>& st) {
  uint64_t* dst = A.p_sgu + C.boff + ((int64_t)(k.a * 2 + k.b) * A.gh + k.c) * A.B * 64 + lane();
  // rows two at a time (each weight converted once for both)
  int r = 0;
  for (; r + 1 < A.B; r += 2) {
    launder(st);
    float v0, v1;
    chain2<false>(st, C.xs + (r * A.gh + k.c) * kXPad, C.xs + ((r + 1) * A.gh + k.c) * kXPad, v0, v1);
    st_pair(dst + r * 64, v0, C.tag);
    st_pair(dst + (r + 1) * 64, v1, C.tag);
  }
  if (r < A.B) {
    launder(st);
    st_pair(dst + r * 64, chain<false>(st, C.xs + (r * A.gh + k.c) * kXPad), C.tag);
  }
}

__device__ __attribute__((always_inline)) void task_sgu(const KA FusedArgs& A, const Ctx& C, const Task& k) {
  Stage<false> st;
  issue_kblocked(k.b ? C.W->sh_up : C.W->sh_gate, A.Fs, k.a * 64, k.c, st);
  UOCR_TRACE_LOADS(A, C.tr);
  sgu_rows(A, C, k, st);
}

// Shared gate/up fold of 64 columns for token r: hs = silu(sum_g gate) *
// (sum_g up), chunk sums added in order.
__device__ __attribute__((always_inline)) void task_sfold(const KA FusedArgs& A, const Ctx& C, const Task& k) {
  constexpr int kMaxG = 16;
  const int l = lane();
  const int r = k.b;
  float acc[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    float v[kMaxG];
    poll_pairs<kMaxG>(A.p_sgu + C.boff + ((int64_t)(k.a * 2 + p) * A.gh * A.B + r) * 64 + l, (int64_t)A.B * 64, A.gh,
                      C.tag,
                      A.ctl, A.spin_limit, v);
    float sum = 0.0f;
#pragma unroll
    for (int g = 0; g < kMaxG; ++g)
      if (g < A.gh) sum = sum + v[g];
    acc[p] = sum;
  }
  UOCR_TRACE(A, C.tr, 3);
  st_pair(A.hs + C.boff + (int64_t)r * A.Fs + k.a * 64 + l, silu(acc[0]) * acc[1], C.tag);
}

// Shared down, 64 columns x chunk g of Fs, every token: partials.
__device__ __attribute__((always_inline)) void task_sdn(const KA FusedArgs& A, const Ctx& C, const Task& k) {
  const int l = lane();
  const int g = k.b;
  Stage<false> st;
  issue_kblocked(C.W->sh_down, A.H, k.a * 64, g, st);
  UOCR_TRACE_LOADS(A, C.tr);
  // hs[r][g*128 .. +128) of every token into the activation stage (row r at r*128)
  {
    // pair i is row i/2, element (i%2)*64 + l; the first pair is probed first
    constexpr int kMaxP = 16;
    const int np = 2 * A.B;
    const uint64_t* src = A.hs + C.boff + (int64_t)g * 128 + l;
    float v[kMaxP];
    uint32_t spin = A.spin_limit;
    while (!poll_done(pair_has(ld_pair(src), C.tag), spin, A.ctl)) {
    }
    for (;;) {
      uint64_t q[kMaxP];
      const uint64_t* a = src;
#pragma unroll
      for (int i = 0; i < kMaxP; i += 2) {
        q[i] = ld_pair(a);
        q[i + 1] = ld_pair(a + 64);
        if (i + 2 < np) a += A.Fs;
      }
      bool ok = true;
#pragma unroll
      for (int i = 0; i < kMaxP; ++i) {
        v[i] = pair_value(q[i]);
        ok = ok && pair_has(q[i], C.tag);
      }
      if (poll_done(ok, spin, A.ctl)) break;
    }
    if (expired(spin)) {
#pragma unroll
      for (int i = 0; i < kMaxP; ++i) v[i] = __builtin_nanf("");
    }
#pragma unroll
    for (int i = 0; i < kMaxP; ++i)
      if (i < np) C.act[(i >> 1) * 128 + (i & 1) * 64 + l] = v[i];
    __builtin_amdgcn_wave_barrier();
  }
  UOCR_TRACE(A, C.tr, 3);
  uint64_t* dst = A.p_sdn + C.boff + ((int64_t)k.a * A.gfs + g) * A.B * 64 + l;
  int r = 0;
  for (; r + 1 < A.B; r += 2) {
    launder(st);
    float v0, v1;
    chain2<false>(st, C.act + r * 128, C.act + (r + 1) * 128, v0, v1);
    st_pair(dst + r * 64, v0, C.tag);
    st_pair(dst + (r + 1) * 64, v1, C.tag);
  }
  if (r < A.B) {
    launder(st);
    st_pair(dst + r * 64, chain<false>(st, C.act + r * 128), C.tag);
  }
}

// The fold of a column's G group partials (lanes base .. base+G-1) in group
// order: acc = fma(scale_g, partial_g, acc) from 0 (int8, scale_g in the same
// lane as partial_g), or the plain sum (bf16).  Every shuffle of a batch is
// issued before its first add (a shuffle under the loop's bound would wait for
// each one in turn).
template <bool INT8, int MAXG, bool STACK>
__device__ __forceinline__ float fold_groups(float part, float scale, int base, int G) {
  constexpr int kBatch = 8;  // shuffles in flight (registers)
  // In the stacked kernel, G through an empty asm: the group bounds below are
  // compared where they are used, not hoisted out of the layer loop as masks
  // live (and spilled) across every layer
  if constexpr (STACK) asm volatile("" : "+s"(G));
  float acc = 0.0f;
#pragma unroll
  for (int g0 = 0; g0 < MAXG; g0 += kBatch) {
    if (g0 < G) {
      float pv[kBatch], sv[INT8 ? kBatch : 1];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int src = base + min(g0 + i, G - 1);
        pv[i] = shfl(part, src);
        if constexpr (INT8) sv[i] = shfl(scale, src);
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        if (g0 + i < G) {
          if constexpr (INT8)
            acc = __builtin_fmaf(sv[i], pv[i], acc);
          else
            acc = acc + pv[i];
        }
      }
    }
  }
  return acc;
}

// Column blocks of a routed task: SUB blocks of c columns from column
// (task index) * SUB * c; a block past the last column is empty (ncols <= 0)
// and neither loads nor computes.  Every block's weights are loaded before
// the first is computed, so a wave waits for its weights once per SUB blocks.
template <bool INT8, int SUB>
struct Blocks {
  Stage<INT8> st[SUB];
  float scale[SUB];
  int n0[SUB], ncols[SUB];
};

// Routed gate+up of one expert for SUB blocks of c_gu columns, every chunk of
// H, the expert's routed rows: h = silu(fold(gate)) * fold(up), fold over the
// 128-groups in order.  Lane l of a block is (column, projection, group) =
// ((2c + p) * gh + g).
template <bool INT8, int SUB, bool STACK>
__device__ __attribute__((always_inline)) void task_rgu(const KA FusedArgs& A, const Ctx& C, const Route& rt,
                                                        const Task& k) {
  constexpr int kMaxG = 16;
  const int l = lane();
  const int e = slot_expert(rt, k.a);
  const uint64_t rows0 = slot_rows(rt, e);
  Blocks<INT8, SUB> bk;
#pragma unroll
  for (int j = 0; j < SUB; ++j) {
    bk.n0[j] = (k.b * SUB + j) * A.c_gu;
    bk.ncols[j] = min(A.c_gu, A.F - bk.n0[j]);
    bk.scale[j] = 0.0f;
    if (bk.ncols[j] > 0) {
      issue_routed<INT8>(A, *C.W, true, e, bk.n0[j], bk.ncols[j], bk.st[j]);
      if constexpr (INT8) {
        const int lam = min(l, 2 * bk.ncols[j] * A.gh - 1);
        const int cp = small_div(lam, A.inv_gh);
        bk.scale[j] = ldg(((cp & 1) ? C.W->up_s : C.W->gate_s) + ((int64_t)e * A.F + bk.n0[j] + (cp >> 1)) * A.gh +
                          (lam - cp * A.gh));
      }
    }
  }
  UOCR_TRACE_LOADS(A, C.tr);
  if (A.defer_down) {
    // the weights and scales have landed: the workgroup's down tasks may issue theirs
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (lane() == 0) __hip_atomic_fetch_add(C.landed, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
#pragma unroll
  for (int j = 0; j < SUB; ++j) {
    if (bk.ncols[j] <= 0) break;
    const int n0 = bk.n0[j];
    const int lanes = 2 * bk.ncols[j] * A.gh;
    const int lam = min(l, lanes - 1);
    const int cp = small_div(lam, A.inv_gh);
    const int g = lam - cp * A.gh;
    const int c = cp >> 1;
    const int base = cp * A.gh;  // first lane of the lane's (column, projection)
    const bool writer = (cp & 1) == 0 && g == 0 && l < lanes;
    uint64_t rows = rows0;
    while (rows != 0ull) {
      const int r = (int)__builtin_ctzll(rows);
      rows &= rows - 1ull;
      launder(bk.st[j]);
      // the row's token r / topk: in the single layer, small_div with a
      // hardware reciprocal (r < 64, topk <= 8: the error stays far below
      // 1 / (2 topk); B=8 50.1 -> 49.8 us), in the stack the division (the
      // reciprocal made its B=1 step 4 us slower)
      const int tok = STACK ? r / A.topk : small_div(r, __builtin_amdgcn_rcpf((float)A.topk));
      const float part = chain<INT8>(bk.st[j], C.xs + (tok * A.gh + g) * kXPad);
      const float acc = fold_groups<INT8, kMaxG, STACK>(part, bk.scale[j], base, A.gh);
      UOCR_TRACE(A, C.tr, 4);
      const float up = shfl(acc, min(l + A.gh, kWave - 1));
      if (writer) st_pair(A.h + C.boff + (int64_t)r * A.F + n0 + c, silu(acc) * up, C.tag);
    }
  }
}

// defer_down: waits until the routed gate/up tasks that the workgroup's waves
// took first have their weights landed (they wait only for the routing, so
// the count is reached), for at most kDeferTicks of the wall clock.
constexpr int64_t kDeferTicks = 1000;  // 10 us at 100 MHz
__device__ __forceinline__ void defer_for_gate_up(const KA FusedArgs& A, const Ctx& C, const Route& rt) {
  const int gu0 = unrouted_count(A);
  const int gu1 = gu0 + rt.ng * A.per_e_gu;
  int want = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int t = A.E + w * (int)gridDim.x + (int)blockIdx.x;
    want += (t >= gu0 && t < gu1) ? 1 : 0;
  }
  const int64_t end = (int64_t)wall_clock64() + kDeferTicks;
  while (__hip_atomic_load(C.landed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < want &&
         (int64_t)wall_clock64() < end)
    __builtin_amdgcn_s_sleep(1);
}

// Routed down of one expert for SUB blocks of c_dn columns, every chunk of F,
// row by row: y = fold over the 128-groups in order.  Lane l of a block is
// (column, group of F) = (c * gf + g).  A row of h is polled once for all
// blocks.
template <bool INT8, int SUB, bool STACK>
__device__ __attribute__((always_inline)) void task_rdn(const KA FusedArgs& A, const Ctx& C, const Route& rt,
                                                        const Task& k) {
  constexpr int kMaxG = 16;
  constexpr int kMaxP = 16;  // pairs per lane per poll round (F <= 1024 in one round)
  const int l = lane();
  const int e = slot_expert(rt, k.a);
  uint64_t rows = slot_rows(rt, e);
  if (A.defer_down) defer_for_gate_up(A, C, rt);
  Blocks<INT8, SUB> bk;
#pragma unroll
  for (int j = 0; j < SUB; ++j) {
    bk.n0[j] = (k.b * SUB + j) * A.c_dn;
    bk.ncols[j] = min(A.c_dn, A.H - bk.n0[j]);
    bk.scale[j] = 0.0f;
    if (bk.ncols[j] > 0) {
      issue_routed<INT8>(A, *C.W, false, e, bk.n0[j], bk.ncols[j], bk.st[j]);
      if constexpr (INT8) {
        const int lam = min(l, bk.ncols[j] * A.gf - 1);
        const int c = small_div(lam, A.inv_gf);
        bk.scale[j] = ldg(C.W->down_s + ((int64_t)e * A.H + bk.n0[j] + c) * A.gf + (lam - c * A.gf));
      }
    }
  }
  UOCR_TRACE_LOADS(A, C.tr);
  const int npairs = A.F / kWave;  // pairs of one h row per lane: element l + 64 i
  while (rows != 0ull) {
    const int r = (int)__builtin_ctzll(rows);
    rows &= rows - 1ull;
    const uint64_t* src = A.h + C.boff + (int64_t)r * A.F + l;
    for (int i0 = 0; i0 < npairs; i0 += kMaxP) {
      float v[kMaxP];
      // The probe is the row's last pair (its columns come from the expert's
      // last gate/up tasks).  The whole set is tried first only when the
      // wave's previous task (this one's index less the wave count) came
      // after every routed gate/up task: all of them have then been running
      // for at least a task's time, and h is likely there.  Otherwise (every
      // down task at one token) the eager round would only add traffic.
      poll_pairs<kMaxP, kPollEager>(src + (int64_t)i0 * kWave, kWave, min(kMaxP, npairs - i0), C.tag, A.ctl,
                                    A.spin_limit, v, src + (int64_t)(npairs - 1) * kWave,
                                    C.t - (int)gridDim.x * kWaves >= unrouted_count(A) + rt.ng * A.per_e_gu);
#pragma unroll
      for (int i = 0; i < kMaxP; ++i) {
        if (i0 + i < npairs) {
          const int kk = (i0 + i) * kWave + l;
          C.act[(kk >> 7) * kXPad + (kk & 127)] = v[i];
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
    UOCR_TRACE(A, C.tr, 3);
#pragma unroll
    for (int j = 0; j < SUB; ++j) {
      if (bk.ncols[j] <= 0) break;
      const int lanes = bk.ncols[j] * A.gf;
      const int lam = min(l, lanes - 1);
      const int c = small_div(lam, A.inv_gf);
      const int g = lam - c * A.gf;
      launder(bk.st[j]);
      const float part = chain<INT8>(bk.st[j], C.act + g * kXPad);
      const float acc = fold_groups<INT8, kMaxG, STACK>(part, bk.scale[j], c * A.gf, A.gf);
      UOCR_TRACE(A, C.tr, 4);
      if (g == 0 && l < lanes) st_pair(A.y + C.boff + (int64_t)r * A.H + bk.n0[j] + c, acc, C.tag);
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// 64 columns of token t's output: sh = shared-down chunk partials added in
// order; out = fma chain over j of w_j * y_j from 0, plus sh.
__device__ __attribute__((always_inline)) void task_comb(const KA FusedArgs& A, const Ctx& C, const Task& k) {
  constexpr int kMaxG = 16;
  constexpr int kMaxK = 8;
  const int l = lane();
  const int n = k.a * 64 + l;
  const int t = k.b;
  // a failed earlier launch leaves the error word set: every output is then NaN until the host clears it
  const uint32_t failed = ld_word(A.ctl + C_ERR);
  float v[kMaxG];
  poll_pairs<kMaxG>(A.p_sdn + C.boff + ((int64_t)k.a * A.gfs * A.B + t) * 64 + l, (int64_t)A.B * 64, A.gfs, C.tag,
                    A.ctl, A.spin_limit, v);
  float shv = 0.0f;
#pragma unroll
  for (int g = 0; g < kMaxG; ++g)
    if (g < A.gfs) shv = shv + v[g];
  float y[kMaxK];
  poll_pairs<kMaxK, kPollFull>(A.y + C.boff + (int64_t)t * A.topk * A.H + n, A.H, A.topk, C.tag, A.ctl,
                               A.spin_limit, y);
  UOCR_TRACE(A, C.tr, 3);
  float wj[kMaxK];
#pragma unroll
  for (int j = 0; j < kMaxK; ++j) wj[j] = C.r_wts[t * A.topk + min(j, A.topk - 1)];
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < kMaxK; ++j)
    if (j < A.topk) acc = __builtin_fmaf(wj[j], y[j], acc);
  const float res = acc + shv;
  if (!A.residual) {
    A.out[(int64_t)t * A.H + n] = failed != 0u ? __builtin_nanf("") : res;
  } else {
    // the residual stream: x_{l+1} = x_l + MoE_l(x_l), x_l from the LDS rows
    const float xn = C.xs[t * A.gh * kXPad + (n >> 7) * kXPad + (n & 127)] + res;
    if (C.layer + 1 < A.n_layers)
      st_pair(A.xs_pairs + ((int64_t)C.layer * A.B + t) * A.H + n, failed != 0u ? __builtin_nanf("") : xn, C.tag);
    else
      A.out[(int64_t)t * A.H + n] = failed != 0u ? __builtin_nanf("") : xn;
  }
}

// Runs task t (INT8: the routed experts' weights are int8 with scales;
// STACK: in the stacked kernel).
template <bool INT8, bool STACK>
__device__ __attribute__((always_inline)) void run_task(const KA FusedArgs& A, const Ctx& C0, const Route& rt, int t,
                                                        const Task& k, int64_t troute) {
  Ctx C = C0;
  C.t = t;
  C.tr = kTrace ? t + C.layer * (int)A.trace_layer : t;
  UOCR_TRACE(A, C.tr, 0);
  if (kTrace && A.trace != nullptr && lane() == 0) {
    A.trace[(int64_t)C.tr * 8 + 5] = troute;
    A.trace[(int64_t)C.tr * 8 + 6] = k.kind;
  }
  switch (k.kind) {
    case K_SGU: task_sgu(A, C, k); break;
    case K_RGU:
      if (INT8 && A.sub == 2)
        task_rgu<INT8, 2, STACK>(A, C, rt, k);
      else
        task_rgu<INT8, 1, STACK>(A, C, rt, k);
      break;
    case K_SFOLD: task_sfold(A, C, k); break;
    case K_SDN: task_sdn(A, C, k); break;
    case K_RDN: task_rdn<INT8, 1, STACK>(A, C, rt, k); break;
    case K_COMB: task_comb(A, C, k); break;
    default: break;
  }
  UOCR_TRACE(A, C.tr, 2);
  if (kTrace && A.trace != nullptr && lane() == 0)
    A.trace[(int64_t)C.tr * 8 + 7] = (int64_t)(threadIdx.x >> 6) * gridDim.x + blockIdx.x;
}

// One instantiation per routed weight type, each with its own register
// allocation (the bf16 stage is twice the int8 one), and per kind of launch:
// one layer (STACK = false, no layer loop), or a stack of layers.
template <bool INT8, bool STACK>
__global__ void __launch_bounds__(kThreads) k_decode_fused(FusedArgs args) {
  (void)args;  // read in place, through the kernel-argument segment
  const KA FusedArgs* Ap = (const KA FusedArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  const KA FusedArgs& A = *Ap;
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int wave = (int)(threadIdx.x >> 6);
  Ctx C;
  float* xs = (float*)lds;
  int* r_ids = (int*)(lds + A.lds_x);
  float* r_wts = (float*)(lds + A.lds_x + 256);
  int* r_done = (int*)(lds + A.lds_x + 512);  // tokens routed so far
  C.landed = (int*)(lds + A.lds_x + 520);
  C.xs = xs;
  C.r_ids = r_ids;
  C.r_wts = r_wts;
  C.act = (float*)(lds + A.lds_x + 528 + wave * A.lds_act);
  const int nwaves = (int)gridDim.x * kWaves;
  const int rank = wave * (int)gridDim.x + (int)blockIdx.x;
  if (kTrace && A.trace != nullptr && threadIdx.x == kThreads - kWave)
    A.trace[A.trace_wg + blockIdx.x * 8 + 6] = (int64_t)wall_clock64();
  // Every XCD computes all the logits: its router task i (expert i % E,
  // tokens r_tok * (i / E) onwards) runs on wave i % kRouterWaves of its
  // (i / kRouterWaves)-th workgroup, the XCD's first workgroups (the grid's
  // start is spread over about a microsecond, and every routing waits for the
  // last logit).  Every wave then takes the rest of the task list from
  // E + rank on.
  const int re = ((int)blockIdx.x / kXcds) * kRouterWaves + wave;
  const int n_router = A.E * ((A.B + A.r_tok - 1) / A.r_tok);
  const bool router = wave < kRouterWaves && re < n_router;
  const int r_e = re % A.E;
  const int r_t0 = (re / A.E) * A.r_tok;
  constexpr int kCtlThread = kThreads - kWave;
  uint32_t* lds_epoch = (uint32_t*)(lds + A.lds_x + 516);
  uint32_t arrived = 0u, epoch = 0u;

  // One layer, or a stack of layers chained through the residual stream: a
  // workgroup starts layer l + 1 once every one of its waves is done with
  // layer l (its LDS tables are then free) and the layer's input, x_{l+1} as
  // tagged pairs from every combine task of layer l, has arrived.  Each layer
  // has buffers of its own, so no wait of layer l can see layer l + 1's data.
  const int n_layers = STACK ? Ap->n_layers : 1;
  for (int layer = 0; layer < n_layers; ++layer) {
    // In the stacked kernel the arguments and the thread index pass through
    // empty asms each layer: nothing derived from them is hoisted out of the
    // loop, where it would stay live (and spill) across every layer.
    const KA FusedArgs* Al = Ap;
    int tid = (int)threadIdx.x;
    if constexpr (STACK) {
      asm volatile("" : "+s"(Al));
      asm volatile("" : "+v"(tid));
    }
    const KA FusedArgs& A = *Al;
    C.layer = layer;
    C.boff = (int64_t)layer * A.layer_words;
    // this layer's per-workgroup trace records
    const int64_t twg = kTrace ? A.trace_wg + (int64_t)layer * A.trace_layer * 8 : 0;
    C.W = &A.w[layer];
    int t = A.E + rank;

    // a router task's weights do not depend on x: they load while x is staged
    // (defined for every wave, so that no value is carried from the previous layer)
    float w[kMaxJ];
    // The launch's epoch word (first layer): loaded before x so that its round
    // trip overlaps x's; after x it added a round trip to every routing.
    uint32_t epoch_word = 0u;
    if (layer == 0 && threadIdx.x == kCtlThread) epoch_word = ld_word(A.ctl + C_EPOCH + (blockIdx.x % kSpread) * kLine);
    if constexpr (STACK) {
#pragma unroll
      for (int j = 0; j < kMaxJ; ++j) w[j] = 0.0f;
    }
    if (router) router_load(A, *C.W, r_e, w);
    if (STACK && layer > 0) __syncthreads();  // every wave is done with the previous layer

    // x rows into LDS, each 128-element chunk padded to kXPad floats
    if (STACK && layer > 0) {
      // x_l as tagged pairs: every thread's pairs loaded and their values
      // written to the LDS rows, until all of the wave's carry the tag
      constexpr int kPPasses = (8 * 2048 + kThreads - 1) / kThreads;  // B <= 8, H <= 2048
      const int n = A.B * A.H;
      const uint64_t* src = A.xs_pairs + (int64_t)(layer - 1) * n;
      uint32_t spin = A.spin_limit;
      // (traced: the layer's start, every wave done with the previous one, as the epoch-read record)
      if (kTrace && A.trace != nullptr && threadIdx.x == kCtlThread)
        A.trace[twg + blockIdx.x * 8 + 7] = (int64_t)wall_clock64();
      for (;;) {
        bool ok = true;
#pragma unroll
        for (int j = 0; j < kPPasses; ++j) {
          const int i = tid + j * kThreads;
          if (i < n) {
            const uint64_t q = ld_pair(src + i);
            const int r = task_div(i, A.m_h);
            const int kk = i - r * A.H;
            xs[r * A.gh * kXPad + (kk >> 7) * kXPad + (kk & 127)] = pair_value(q);
            ok = ok && pair_has(q, C.tag);
          }
        }
        if (poll_done(ok, spin, A.ctl)) break;
      }
      // (traced: the control wave's x landed, as the entry record)
      if (kTrace && A.trace != nullptr && threadIdx.x == kCtlThread)
        A.trace[twg + blockIdx.x * 8 + 6] = (int64_t)wall_clock64();
      if (expired(spin)) {
        for (int i = tid; i < n; i += kThreads) {
          const int r = task_div(i, A.m_h);
          const int kk = i - r * A.H;
          xs[r * A.gh * kXPad + (kk >> 7) * kXPad + (kk & 127)] = __builtin_nanf("");
        }
      }
    } else if (A.x_vec) {
      // 16-byte pieces (a chunk is 32 of them), every thread's loads issued
      // before the first is used, in little code (each launch runs it with
      // cold caches)
      constexpr int kXPasses = (8 * 2048 / 4 + kThreads - 1) / kThreads;  // B <= 8, H <= 2048
      const int n4 = A.B * A.H / 4;
      f32x4 xv[kXPasses];
#pragma unroll
      for (int j = 0; j < kXPasses; ++j) {
        const int i = tid + j * kThreads;
        if constexpr (STACK) xv[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};  // (no value carried from another layer)
        if (i < n4) xv[j] = *(const UOCR_GLOBAL f32x4*)(A.x + 4 * i);
      }
#pragma unroll
      for (int j = 0; j < kXPasses; ++j) {
        const int i = tid + j * kThreads;
        if (i < n4) {
          const int r = (4 * i) / A.H;
          const int kk = 4 * i - r * A.H;
          *(f32x4*)(xs + r * A.gh * kXPad + (kk >> 7) * kXPad + (kk & 127)) = xv[j];
        }
      }
    } else {
      for (int i = tid; i < A.B * A.H; i += kThreads) {
        const int r = task_div(i, A.m_h);
        const int kk = i - r * A.H;
        xs[r * A.gh * kXPad + (kk >> 7) * kXPad + (kk & 127)] = ldg(A.x + i);
      }
    }
    // One load of the epoch per workgroup and launch (3 072 waves loading the
    // one word at once would queue every workgroup's start behind it), shared
    // through LDS.  The last wave loads it (before x, above) and makes the
    // arrival count below: its
    // first work is to wait for the logits, while the router tasks run on the
    // first waves.
    if (threadIdx.x == kCtlThread) {
      *r_done = 0;
      *C.landed = 0;
      if (layer == 0) {
        *lds_epoch = epoch_word;
        if (kTrace && A.trace != nullptr) {
          asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
          A.trace[twg + blockIdx.x * 8 + 7] = (int64_t)wall_clock64();
        }
      }
    }
    __syncthreads();
    if (layer == 0) {
      epoch = __builtin_amdgcn_readfirstlane(*lds_epoch);
      C.tag = epoch + 1u;
      // the arrival count; its returned value is read after the control wave's tasks
      if (threadIdx.x == kCtlThread)
        arrived = __hip_atomic_fetch_add(A.ctl + C_ARRIVED + (blockIdx.x % kSpread) * kLine, 1u, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    }

    if (router) {
      // the trace keeps one record per expert: XCD 0's task of its first tokens
      const bool traced = r_t0 == 0 && blockIdx.x % kXcds == 0;
      C.t = r_e;
      C.tr = kTrace ? r_e + layer * (int)A.trace_layer : r_e;
      if (traced) UOCR_TRACE(A, C.tr, 0);
      if (traced) UOCR_TRACE_LOADS(A, C.tr);
      router_task<STACK>(A, C, r_e, r_t0, min(A.B, r_t0 + A.r_tok), w);
      if (traced) UOCR_TRACE(A, C.tr, 2);
      if (traced && kTrace && A.trace != nullptr && lane() == 0) A.trace[(int64_t)C.tr * 8 + 7] = rank;
    }
    // The routing of token i is computed by wave kWaves-1-i (high waves, whose
    // tasks come late in the list); the other waves meanwhile run their tasks
    // that do not need the routing (the shared experts).
    const int rwave = kWaves - 1 - wave;
    // (the routing wave's activation stage, idle until its first task, holds the keys)
    if (rwave < A.B) route_token(A, C.boff, twg, rwave, C.tag, r_ids, r_wts, r_done, (uint64_t*)C.act);
    // One task loop (one copy of the task code): the first routed task waits
    // for the workgroup's routing.
    Route rt{0ull, 0, r_ids, 0};
    int n_tasks = unrouted_count(A);
    bool routed = false;
    int64_t troute = 0;
    for (;; t += nwaves) {
      if (!routed && t >= n_tasks) {
        uint32_t spin = A.spin_limit;
        while (!poll_done(__hip_atomic_load(r_done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= A.B, spin,
                          A.ctl)) {
        }
        asm volatile("" ::: "memory");
        if (kTrace && A.trace != nullptr) troute = (int64_t)wall_clock64();
        // without the routing (a failed wait), no routed task runs: the combine's waits for them fail too
        rt = expired(spin) ? Route{0ull, 0, r_ids, 0} : make_route(A, r_ids);
        n_tasks = task_count(A, rt.ng);
        routed = true;
      }
      if (t >= n_tasks) break;
      const KA FusedArgs* Ai = Ap;
      asm volatile("" : "+s"(Ai));
      run_task<INT8, STACK>(*Ai, C, rt, t, task_at(*Ai, rt.ng, t), troute);
    }
  }
  // Two-level arrival count: the workgroup that completes its counter (of the
  // workgroups b with the same b % kSpread) adds to C_ARRIVED2, and the one that
  // completes that is the launch's last: it clears the counters and advances
  // the epoch for the next launch.
  if (wave == kWaves - 1) {
    const int l = lane();
    const uint32_t grp = blockIdx.x % kSpread;
    const uint32_t in_grp = (gridDim.x - grp + kSpread - 1) / kSpread;
    const uint32_t groups = gridDim.x < (uint32_t)kSpread ? gridDim.x : (uint32_t)kSpread;
    if (shfl(arrived, 0) + 1u == in_grp) {
      uint32_t old = 0u;
      if (l == 0) old = __hip_atomic_fetch_add(A.ctl + C_ARRIVED2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (shfl(old, 0) + 1u == groups && l < kSpread) {
        st_word(A.ctl + C_ARRIVED + l * kLine, 0u);
        if (l == 0) st_word(A.ctl + C_ARRIVED2, 0u);
        st_word(A.ctl + C_EPOCH + l * kLine, epoch + 1u);
      }
    }
  }
}

}  // namespace

int fused_sub(bool int8, int B) { return int8 && B >= kFusedSubRows ? 2 : 1; }

FusedLayout fused_layout(int B, int E, int H, int F, int Fs, int topk, int sub) {
  FusedLayout L{};
  L.gh = H / 128;
  L.gf = F / 128;
  L.gfs = Fs / 128;
  L.sub = sub;
  L.c_gu = L.gh > 0 ? 64 / (2 * L.gh) : 0;
  L.c_dn = L.gf > 0 ? 64 / L.gf : 0;
  L.per_e_gu = L.c_gu > 0 ? (F + L.c_gu * sub - 1) / (L.c_gu * sub) : 0;
  L.per_e_dn = L.c_dn > 0 ? (H + L.c_dn - 1) / L.c_dn : 0;
  L.cb_fs = Fs / 64;
  L.cb_h = H / 64;
  L.n_sgu = L.cb_fs * 2 * L.gh;
  L.n_sdn = L.cb_h * L.gfs;
  L.n_sfold = L.cb_fs * B;
  L.n_comb = L.cb_h * B;
  L.lds_x = B * L.gh * kXPad * 4;
  const int act_rows = B * 128 * 4;
  const int act_h = L.gf * kXPad * 4;
  L.lds_act = act_rows > act_h ? act_rows : act_h;
  // a routing wave's stage first holds its 64 top-k keys and the selected weights
  const int act_route = kWave * 8 + 8 * 4;
  L.lds_act = L.lds_act > act_route ? L.lds_act : act_route;
  L.lds_act = (L.lds_act + 15) & ~15;
  L.lds_bytes = (size_t)L.lds_x + 528 + (size_t)kWaves * L.lds_act;
  const int R = B * topk;
  const int slots = E < R ? E : R;
  L.max_tasks = E + L.n_sgu + L.n_sfold + L.n_sdn + slots * (L.per_e_gu + L.per_e_dn) + L.n_comb;
  // tagged words for the largest batch (8 tokens) of this layer
  const int64_t rmax = 8 * (int64_t)topk;
  L.off_logits = 0;
  L.off_h = L.off_logits + (int64_t)kLogitCopies * kLogitCopyWords;
  L.off_y = L.off_h + rmax * F;
  L.off_hs = L.off_y + rmax * H;
  L.off_psgu = L.off_hs + 8 * (int64_t)Fs;
  L.off_psdn = L.off_psgu + (int64_t)L.cb_fs * 2 * L.gh * 8 * 64;
  L.data_words = L.off_psdn + (int64_t)L.cb_h * L.gfs * 8 * 64;
  return L;
}

bool fused_trace_built() { return kTrace; }

// The resident capacity of every instantiation (the smallest, so that one
// grid suits any).
hipError_t fused_grid(size_t lds_bytes, int* grid) {
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const void* kernels[4] = {(const void*)k_decode_fused<true, false>, (const void*)k_decode_fused<false, false>,
                            (const void*)k_decode_fused<true, true>, (const void*)k_decode_fused<false, true>};
  int per_cu[4] = {0, 0, 0, 0};
  for (int i = 0; i < 4 && e == hipSuccess; ++i) {
    e = hipFuncSetAttribute(kernels[i], hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu[i], kernels[i], kThreads, lds_bytes);
  }
  if (e != hipSuccess) return e;
  int least = per_cu[0];
  for (int i = 1; i < 4; ++i) least = per_cu[i] < least ? per_cu[i] : least;
  *grid = cus * least;
  return hipSuccess;
}

hipError_t launch_decode_fused(const FusedArgs& a, int grid, size_t lds_bytes, hipStream_t s) {
  // every XCD runs all router tasks on its own workgroups (the routing waits for all logits)
  if (grid % kXcds != 0 || a.r_tok < 1 ||
      (int64_t)(grid / kXcds) * kRouterWaves < (int64_t)a.E * ((a.B + a.r_tok - 1) / a.r_tok))
    return hipErrorInvalidConfiguration;
  if (a.residual) {
    if (a.int8)
      UOCR_LAUNCH("decode_stack", (k_decode_fused<true, true>), dim3(grid), dim3(kThreads), lds_bytes, s, a);
    else
      UOCR_LAUNCH("decode_stack", (k_decode_fused<false, true>), dim3(grid), dim3(kThreads), lds_bytes, s, a);
  } else {
    if (a.int8)
      UOCR_LAUNCH("decode_fused", (k_decode_fused<true, false>), dim3(grid), dim3(kThreads), lds_bytes, s, a);
    else
      UOCR_LAUNCH("decode_fused", (k_decode_fused<false, false>), dim3(grid), dim3(kThreads), lds_bytes, s, a);
  }
  return hipGetLastError();
}

__global__ void k_zero_words(uint32_t* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

hipError_t launch_zero_words(uint32_t* p, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  UOCR_LAUNCH("zero_words", k_zero_words, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, n);
  return hipGetLastError();
}

// flag[0] = the OR of the error words at a and b (either may be null), read
// with the agent-scope loads the persistent kernel writes them with.
__global__ void k_error_status(uint32_t* flag, const uint32_t* a, const uint32_t* b) {
  if (threadIdx.x != 0) return;
  uint32_t v = 0u;
  if (a != nullptr) v |= ld_word(a + C_ERR);
  if (b != nullptr) v |= ld_word(b + C_ERR);
  flag[0] = v != 0u ? 1u : 0u;
}

hipError_t launch_error_status(uint32_t* flag, const uint32_t* ctl_a, const uint32_t* ctl_b, hipStream_t s) {
  UOCR_LAUNCH("error_status", k_error_status, dim3(1), dim3(64), 0, s, flag, ctl_a, ctl_b);
  return hipGetLastError();
}

}  // namespace uocr
