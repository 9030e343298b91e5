// Host side of the C ABI (include/uocr_moe.h): the reference's host-side shape
// checks with its messages, workspace carving, and the launch sequences of the
// ops and of the MoE layer (decode and prefill).
#include "../../include/uocr_moe.h"

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "uocr_kernels.h"

namespace uocr {
int gemm_bk();
}  // namespace uocr

// Scratch of the allocation-free decode entry (uocr_moe_decode_rows_static): one
// array per GPU, held until the process ends.  The first kScratchFusedBytes
// hold the persistent kernel's control words and tagged arena (room for any
// layer the persistent path accepts); the rest is the multi-kernel decode's
// workspace.  Host code never passes `scratch` itself to a kernel: it passes
// the device address hipGetSymbolAddress returns for the current device.
constexpr size_t kScratchBytes = (size_t)16 << 20;
constexpr size_t kScratchFusedBytes = (size_t)9 << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

using namespace uocr;

// ------------------------------------------------------------------ kernel timing

namespace {

struct Timing {
  std::mutex mu;
  bool on = false;
  size_t used = 0;
  std::vector<hipEvent_t> start, stop;
  std::vector<std::string> names;
};
Timing g_timing;

}  // namespace

bool uocr::timing_slot(const char* name, hipEvent_t* start, hipEvent_t* stop) {
  std::lock_guard<std::mutex> lock(g_timing.mu);
  if (!g_timing.on || g_timing.used >= g_timing.start.size()) return false;
  *start = g_timing.start[g_timing.used];
  *stop = g_timing.stop[g_timing.used];
  g_timing.names[g_timing.used] = name;
  ++g_timing.used;
  return true;
}

namespace {

int fail(char* err, size_t errlen, const char* fmt, ...) {
  if (err != nullptr && errlen > 0) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
  }
  return 1;
}

int hip_fail(char* err, size_t errlen, const char* op, hipError_t e) {
  return fail(err, errlen, "%s: HIP error %d (%s)", op, (int)e, hipGetErrorString(e));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ------------------------------------------------------------------ workspace

struct Carve {
  char* base;
  size_t off = 0;
  explicit Carve(void* b) : base(static_cast<char*>(b)) {}
  template <typename T>
  T* take(size_t count) {
    off = (off + 255) & ~size_t(255);
    T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
    off += count * sizeof(T);
    return p;
  }
};

struct CachedBuffer {
  void* ptr = nullptr;
  size_t bytes = 0;
};

std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, CachedBuffer> g_ws;
std::vector<void*> g_retired;  // superseded library workspaces (freed by uocr_moe_release)

// The library's own workspace for (current device, stream), at least `bytes`.
hipError_t own_workspace(hipStream_t stream, size_t bytes, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(g_ws_mu);
  CachedBuffer& b = g_ws[{dev, stream}];
  if (b.bytes < bytes) {
    if (b.ptr != nullptr) {
      // queued work or a captured graph may still use the old buffer: it lives until uocr_moe_release
      g_retired.push_back(b.ptr);
      b.ptr = nullptr;
      b.bytes = 0;
    }
    // the next power of two (at least 1 MiB): a rising series of sizes retires
    // less than the live buffer in all, however long it runs
    size_t grow = size_t(1) << 20;
    while (grow < bytes) grow <<= 1;
    e = hipMalloc(&b.ptr, grow);
    if (e != hipSuccess) return e;
    b.bytes = grow;
  }
  *out = b.ptr;
  return hipSuccess;
}

// State of the persistent decode kernel.  Each (device, stream) owns one slot:
// kFusedCtlWords control words and a tagged-data arena sized for the largest
// layer the persistent path accepts (fused_max_words), zeroed when allocated.
// Slots come in chunks of kFusedChunk, allocated by calls outside stream
// capture; a stream first seen under capture takes a spare slot, or the call is
// refused.  No slot is shared by two streams, and nothing is freed before
// uocr_moe_release(), so graphs captured earlier keep valid pointers.
constexpr int kFusedChunk = 4;
constexpr int C_ERR_WORD = 4;  // the kernel's error word (decode.hip)
struct FusedSlot {
  uint32_t* ctl = nullptr;
  uint64_t* data = nullptr;
};
struct FusedDevice {
  std::vector<void*> chunks;
  std::vector<FusedSlot> spare;
  std::map<hipStream_t, FusedSlot> slot;
  std::map<hipStream_t, uint64_t*> stack;  // tagged arenas of stacked launches (fused_stack_words)
  std::vector<uint64_t*> stack_spare;      // one kept for a stream first seen under capture
  hipStream_t last_stream = nullptr;  // stream of the last eager persistent launch
  hipEvent_t handoff = nullptr;       // orders eager launches on different streams
};
std::map<int, FusedDevice> g_fused;
std::map<std::pair<int, size_t>, int> g_fused_grid;  // (device, LDS bytes) -> workgroups
std::map<int, char*> g_scratch;  // device -> the address of `scratch` on it

// Optional phase trace of the next persistent decode launch (diagnostics).
int64_t* g_trace = nullptr;
int64_t g_trace_words = 0;
int g_trace_grid = 0;

bool capturing(hipStream_t stream) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

// Tagged words of the largest layer the persistent path takes (8 tokens, top-8,
// 64 experts, every width 2048): every slot has room for any eligible layer.
int64_t fused_max_words() { return fused_layout(8, 64, 2048, 2048, 2048, 8).data_words; }
size_t fused_slot_bytes() { return ((size_t)kFusedCtlWords * 4 + (size_t)fused_max_words() * 8 + 255) & ~size_t(255); }

// A new chunk of zeroed slots (g_ws_mu held, not under capture).
hipError_t fused_grow(FusedDevice& d, hipStream_t stream) {
  const size_t bytes = kFusedChunk * fused_slot_bytes();
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) return e;
  e = launch_zero_words(static_cast<uint32_t*>(p), (int64_t)(bytes / 4), stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);  // zero before any stream uses a slot
  if (e != hipSuccess) {
    (void)hipFree(p);
    return e;
  }
  d.chunks.push_back(p);
  for (int i = kFusedChunk - 1; i >= 0; --i) {
    char* base = static_cast<char*>(p) + (size_t)i * fused_slot_bytes();
    d.spare.push_back(FusedSlot{reinterpret_cast<uint32_t*>(base),
                                reinterpret_cast<uint64_t*>(base + (size_t)kFusedCtlWords * 4)});
  }
  return hipSuccess;
}

// The slot of (current device, stream); *need_alloc is set when the stream is
// new and no spare slot is left under capture.
hipError_t fused_slot(hipStream_t stream, FusedSlot* out, bool* need_alloc) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(g_ws_mu);
  FusedDevice& d = g_fused[dev];
  *need_alloc = false;
  auto it = d.slot.find(stream);
  if (it != d.slot.end()) {
    *out = it->second;
    return hipSuccess;
  }
  const bool cap = capturing(stream);
  if (d.spare.empty()) {
    if (cap) {
      *need_alloc = true;
      return hipSuccess;
    }
    e = fused_grow(d, stream);
    if (e != hipSuccess) return e;
  }
  *out = d.spare.back();
  d.spare.pop_back();
  d.slot[stream] = *out;
  // keep a spare for a stream that first appears under capture
  if (d.spare.empty() && !cap) e = fused_grow(d, stream);
  return e;
}

// Tagged words of a stacked launch's arena: kFusedMaxLayers layers of the
// largest eligible layer's buffers, then the residual stream x_{l+1} of every
// layer but the last as tagged pairs [8][2048].
int64_t fused_stack_words() { return (int64_t)kFusedMaxLayers * (fused_max_words() + 8 * 2048); }

// A new zeroed stacked-launch arena (g_ws_mu held, not under capture).
hipError_t fused_stack_grow(FusedDevice& d, hipStream_t stream) {
  const size_t bytes = (size_t)fused_stack_words() * 8;
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) return e;
  e = launch_zero_words(static_cast<uint32_t*>(p), (int64_t)(bytes / 4), stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);  // zero before any stream uses it
  if (e != hipSuccess) {
    (void)hipFree(p);
    return e;
  }
  d.chunks.push_back(p);  // freed with the slots
  d.stack_spare.push_back(static_cast<uint64_t*>(p));
  return hipSuccess;
}

// The stacked-launch arena of (current device, stream), as fused_slot hands
// out slots: a stream seen for the first time takes the spare arena (made by
// an earlier call outside capture) or, outside capture, a new one; a spare is
// then made again outside capture.  *need_alloc is set when a stream first
// seen under capture finds no spare.  Kept until uocr_moe_release().
hipError_t fused_stack_arena(hipStream_t stream, uint64_t** out, bool* need_alloc) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(g_ws_mu);
  FusedDevice& d = g_fused[dev];
  *need_alloc = false;
  auto it = d.stack.find(stream);
  if (it != d.stack.end()) {
    *out = it->second;
    return hipSuccess;
  }
  const bool cap = capturing(stream);
  if (d.stack_spare.empty()) {
    if (cap) {
      *need_alloc = true;
      return hipSuccess;
    }
    e = fused_stack_grow(d, stream);
    if (e != hipSuccess) return e;
  }
  *out = d.stack_spare.back();
  d.stack_spare.pop_back();
  d.stack[stream] = *out;
  if (d.stack_spare.empty() && !cap) e = fused_stack_grow(d, stream);
  return e;
}

// Eager persistent launches need the whole device: one on another stream than
// the previous one first waits for everything queued on that stream.  The
// wait and the launch are enqueued under one lock, so that the next launch's
// wait (made by any thread) is recorded after this launch.
template <typename Launch>
hipError_t fused_ordered_launch(hipStream_t stream, Launch&& launch) {
  if (capturing(stream)) return launch();
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(g_ws_mu);
  FusedDevice& d = g_fused[dev];
  if (d.last_stream != nullptr && d.last_stream != stream) {
    if (d.handoff == nullptr) e = hipEventCreateWithFlags(&d.handoff, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(d.handoff, d.last_stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(stream, d.handoff, 0);
    if (e != hipSuccess) return e;
  }
  e = launch();
  if (e == hipSuccess) d.last_stream = stream;
  return e;
}

hipError_t fused_grid_cached(size_t lds_bytes, int* grid) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(g_ws_mu);
  auto it = g_fused_grid.find({dev, lds_bytes});
  if (it != g_fused_grid.end()) {
    *grid = it->second;
    return hipSuccess;
  }
  e = fused_grid(lds_bytes, grid);
  if (e == hipSuccess) g_fused_grid[{dev, lds_bytes}] = *grid;
  return e;
}

// Resolves the workspace of a call: the caller's (checked for size) or ours.
int resolve_workspace(const char* op, void* workspace, size_t workspace_bytes, size_t need, hipStream_t stream,
                      void** out, char* err, size_t errlen) {
  if (workspace != nullptr) {
    if (workspace_bytes < need)
      return fail(err, errlen, "%s: workspace of %zu bytes is smaller than the %zu needed", op, workspace_bytes,
                  need);
    *out = workspace;
    return 0;
  }
  const hipError_t e = own_workspace(stream, need, out);
  return e == hipSuccess ? 0 : hip_fail(err, errlen, op, e);
}

// Waves of a GEMV workgroup: every chunk of the batch in flight at once when
// it fits, else the fewest waves that split the chunks evenly.
int waves_for(int nchunks) {
  if (nchunks < 1) return 1;
  const int rounds = (nchunks + kGemvMaxWaves - 1) / kGemvMaxWaves;
  return (nchunks + rounds - 1) / rounds;
}

int batch_for(int nchunks) { return nchunks < kGemvMaxBatch ? (nchunks < 1 ? 1 : nchunks) : kGemvMaxBatch; }

GroupTables carve_tables(Carve& c, int E, int R, bool tiles, bool inv) {
  GroupTables g{};
  g.n_groups = c.take<int32_t>(1);
  g.group_expert = c.take<int32_t>(E);
  g.group_start = c.take<int32_t>(E + 1);
  g.group_rows = c.take<int32_t>(R > 0 ? R : 1);
  g.tile_start = tiles ? c.take<int32_t>(E + 1) : nullptr;
  g.inv = inv ? c.take<int32_t>(R > 0 ? R : 1) : nullptr;
  return g;
}

Rows rows_of(const GroupTables& g) { return Rows{g.n_groups, g.group_expert, g.group_start, g.group_rows, 0}; }

// ------------------------------------------------------------------ the routed qmv ops

int routed_qmv(const char* op, WKind kind, float* result, const float* x, const int32_t* ids, const void* w,
               const float* scales, int64_t k, int64_t E, int64_t N, int64_t K, int64_t groups, hipStream_t s,
               char* err, size_t errlen) {
  if (k == 0 || N == 0) return 0;
  if (E > 1024) return fail(err, errlen, "%s: more than 1024 experts are not supported", op);
  if (k > (int64_t)1 << 30 || N > (int64_t)1 << 30 || K > (int64_t)1 << 30)
    return fail(err, errlen, "%s: dimensions beyond 2^30 are not supported", op);
  const int max_groups = (int)(E < k ? E : k);
  Carve dry(nullptr);
  carve_tables(dry, (int)E, (int)k, false, false);
  void* ws = nullptr;
  if (resolve_workspace(op, nullptr, 0, dry.off, s, &ws, err, errlen)) return 1;
  Carve c(ws);
  const GroupTables g = carve_tables(c, (int)E, (int)k, false, false);
  hipError_t e = launch_group(ids, (int)k, (int)E, 1, g, s);
  if (e != hipSuccess) return hip_fail(err, errlen, op, e);

  GemvArgs a{};
  a.out = result;
  a.ldo = N;
  a.x = x;
  a.ldx = K;
  a.x_div = 1;
  a.p[0] = Proj{w, scales};
  a.kind = kind;
  a.E = (int)E;
  a.N = (int)N;
  a.K = (int)K;
  if (kind == kInt8Rows) {
    a.gsize = (int)(K / groups);
    a.nchunks = (int)groups;
    a.vec = (K % 16 == 0) && (a.gsize % 16 == 0) && aligned16(w);
  } else {
    a.gsize = kChunk;
    a.nchunks = (int)((K + kChunk - 1) / kChunk);
    a.vec = (K % 8 == 0) && aligned16(w);
  }
  a.batch = batch_for(a.nchunks);
  a.rows = rows_of(g);
  e = launch_gemv(a, max_groups, 1, waves_for(a.batch), s);
  return e == hipSuccess ? 0 : hip_fail(err, errlen, op, e);
}

}  // namespace

extern "C" {

int uocr_moe_abi_version(void) { return UOCR_MOE_ABI_VERSION; }

int uocr_moe_int8_qmv(float* result, int64_t result_k, int64_t result_n, const float* x, int64_t x_k,
                      int64_t x_kdim, const int32_t* expert_ids, int64_t ids_k, const int8_t* w, int64_t w_e,
                      int64_t w_n, int64_t w_kdim, const float* scales, int64_t s_e, int64_t s_n, int64_t s_groups,
                      void* stream, char* err, size_t errlen) {
  // unlimited_ocr_max/kernels/moe_int8.mojo:194-210
  if (x_k != result_k) return fail(err, errlen, "moe_int8_qmv: x and output disagree on k");
  if (ids_k != result_k) return fail(err, errlen, "moe_int8_qmv: expert_ids and output disagree on k");
  if (w_n != result_n) return fail(err, errlen, "moe_int8_qmv: w and output disagree on N");
  if (w_kdim != x_kdim) return fail(err, errlen, "moe_int8_qmv: w and x disagree on K");
  if (w_e < 1) return fail(err, errlen, "moe_int8_qmv: the expert stack is empty");
  if (s_e != w_e) return fail(err, errlen, "moe_int8_qmv: scales and w disagree on E");
  if (s_n != w_n) return fail(err, errlen, "moe_int8_qmv: scales and w disagree on N");
  if (s_groups < 1 || w_kdim % s_groups != 0)
    return fail(err, errlen, "moe_int8_qmv: K must be a multiple of the group count");
  return routed_qmv("moe_int8_qmv", kInt8Rows, result, x, expert_ids, w, scales, result_k, w_e, w_n, w_kdim,
                    s_groups, (hipStream_t)stream, err, errlen);
}

int uocr_moe_bf16_qmv(float* result, int64_t result_k, int64_t result_n, const float* x, int64_t x_k,
                      int64_t x_kdim, const int32_t* expert_ids, int64_t ids_k, const uint16_t* w, int64_t w_e,
                      int64_t w_n, int64_t w_kdim, void* stream, char* err, size_t errlen) {
  // unlimited_ocr_max/kernels/moe_bf16.mojo:276-285
  if (x_k != result_k) return fail(err, errlen, "moe_bf16_qmv: x and output disagree on k");
  if (ids_k != result_k) return fail(err, errlen, "moe_bf16_qmv: expert_ids and output disagree on k");
  if (w_n != result_n) return fail(err, errlen, "moe_bf16_qmv: w and output disagree on N");
  if (w_kdim != x_kdim) return fail(err, errlen, "moe_bf16_qmv: w and x disagree on K");
  if (w_e < 1) return fail(err, errlen, "moe_bf16_qmv: the expert stack is empty");
  return routed_qmv("moe_bf16_qmv", kBf16Rows, result, x, expert_ids, w, nullptr, result_k, w_e, w_n, w_kdim, 1,
                    (hipStream_t)stream, err, errlen);
}

int uocr_int8_dequant_expert(void* result, int64_t result_n, int64_t result_kdim, int result_f32, const int8_t* w,
                             int64_t w_e, int64_t w_n, int64_t w_kdim, const float* scales, int64_t s_e,
                             int64_t s_n, int64_t s_groups, const int32_t* expert_idx, int64_t idx_len,
                             void* stream, char* err, size_t errlen) {
  // unlimited_ocr_max/kernels/moe_int8.mojo:280-296
  if (w_n != result_n) return fail(err, errlen, "int8_dequant_expert: w and output disagree on N");
  if (w_kdim != result_kdim) return fail(err, errlen, "int8_dequant_expert: w and output disagree on K");
  if (w_e < 1) return fail(err, errlen, "int8_dequant_expert: the expert stack is empty");
  if (s_e != w_e) return fail(err, errlen, "int8_dequant_expert: scales and w disagree on E");
  if (s_n != w_n) return fail(err, errlen, "int8_dequant_expert: scales and w disagree on N");
  if (idx_len != 1) return fail(err, errlen, "int8_dequant_expert: `expert_idx` must be a single int32");
  if (s_groups < 1 || w_kdim % s_groups != 0)
    return fail(err, errlen, "int8_dequant_expert: K must be a multiple of the group count");
  if (w_n * w_kdim > ((int64_t)1 << 40)) return fail(err, errlen, "int8_dequant_expert: the expert is too large");
  const int vec = (w_kdim % 8 == 0) && aligned16(w) && aligned16(result);
  const hipError_t e = launch_dequant(result, result_f32, w, scales, expert_idx, (int)w_e, (int)w_n, (int)w_kdim,
                                      (int)s_groups, vec, (hipStream_t)stream);
  return e == hipSuccess ? 0 : hip_fail(err, errlen, "int8_dequant_expert", e);
}

int uocr_quantize_per_group(int8_t* q, float* scales, const void* w, int w_bf16, int64_t rows, int64_t kdim,
                            int64_t group, void* stream, char* err, size_t errlen) {
  // tools/quantize_int8.py:306-310
  if (group < 1 || group > (1 << 20)) return fail(err, errlen, "quantize_per_group: bad group size %lld", (long long)group);
  if (rows < 0 || kdim < 0) return fail(err, errlen, "quantize_per_group: bad shape [%lld, %lld]", (long long)rows,
                                        (long long)kdim);
  if (kdim % group)
    return fail(err, errlen, "quantize_per_group: K=%lld is not divisible by the group size %lld", (long long)kdim,
                (long long)group);
  if (rows == 0 || kdim == 0) return 0;
  if (!q || !scales || !w) return fail(err, errlen, "quantize_per_group: a tensor is missing");
  const hipError_t e = launch_quantize(q, scales, w, w_bf16 != 0, rows * (kdim / group), (int)group, (hipStream_t)stream);
  return e == hipSuccess ? 0 : hip_fail(err, errlen, "quantize_per_group", e);
}

int uocr_dense_bf16_qmv(float* result, int64_t result_m, int64_t result_n, const float* x, int64_t x_m,
                        int64_t x_kdim, const uint16_t* w, int64_t w_blocks, int64_t w_n, int64_t w_kblock,
                        int64_t tile, void* stream, char* err, size_t errlen) {
  // unlimited_ocr_max/kernels/dense_bf16.mojo:130-144
  if (tile < 1) return fail(err, errlen, "dense_bf16_qmv: tile must be >= 1");
  if (result_m != x_m) return fail(err, errlen, "dense_bf16_qmv: x and output disagree on M");
  if (w_n != result_n) return fail(err, errlen, "dense_bf16_qmv: w and output disagree on N");
  if (w_kblock != 16) return fail(err, errlen, "dense_bf16_qmv: w is not K-blocked by KBLOCK");
  if (w_blocks * 16 != x_kdim) return fail(err, errlen, "dense_bf16_qmv: w and x disagree on K");
  if (x_m == 0 || result_n == 0) return 0;
  GemvArgs a{};
  a.out = result;
  a.ldo = result_n;
  a.x = x;
  a.ldx = x_kdim;
  a.x_div = 1;
  a.p[0] = Proj{w, nullptr};
  a.kind = kBf16KBlocked;
  a.E = 1;
  a.N = (int)result_n;
  a.K = (int)x_kdim;
  a.gsize = kChunk;
  a.nchunks = (int)((x_kdim + kChunk - 1) / kChunk);
  a.vec = aligned16(w);
  a.batch = batch_for(a.nchunks);
  a.rows = Rows{nullptr, nullptr, nullptr, nullptr, (int)x_m};
  const hipError_t e = launch_dense(a, waves_for(a.batch), (hipStream_t)stream);
  return e == hipSuccess ? 0 : hip_fail(err, errlen, "dense_bf16_qmv", e);
}

// ------------------------------------------------------------------ the n-gram guard

int uocr_ngram_block(float* result, int64_t result_rows, int64_t result_vocab, const float* logits,
                     int64_t logits_rows, int64_t logits_vocab, const int32_t* history, int64_t hist_rows,
                     int64_t hist_len, const int32_t* ngram, int64_t ngram_len, void* stream, char* err,
                     size_t errlen) {
  // unlimited_ocr_max/kernels/ngram_block.mojo:85-99
  if (logits_rows != result_rows || logits_vocab != result_vocab)
    return fail(err, errlen, "ngram_block: logits and output disagree on shape");
  if (hist_rows != result_rows) return fail(err, errlen, "ngram_block: history and logits disagree on the row count");
  if (ngram_len != 1) return fail(err, errlen, "ngram_block: `ngram` must be a single int32");
  if (hist_len < 1) return fail(err, errlen, "ngram_block: history is empty");
  if (hist_len > kNgramMaxHistory)
    return fail(err, errlen, "ngram_block: history longer than %d ids", kNgramMaxHistory);
  if (result_rows < 0 || result_vocab < 0 || result_rows > 65535)
    return fail(err, errlen, "ngram_block: bad logits shape");
  const hipError_t e = launch_ngram_block(result, logits, result_rows, result_vocab, history, (int)hist_len, ngram,
                                          (hipStream_t)stream);
  return e == hipSuccess ? 0 : hip_fail(err, errlen, "ngram_block", e);
}

// ------------------------------------------------------------------ the decoder layer's per-row steps

int uocr_rms_norm_dense_bf16_qmv(float* result, int64_t result_m, int64_t result_n, const float* x, int64_t x_m,
                                 int64_t x_kdim, const float* residual, float* x_out, const float* gamma, float eps,
                                 const uint16_t* w, int64_t w_blocks, int64_t w_n, int64_t w_kblock, void* stream,
                                 char* err, size_t errlen) {
  const char* op = "rms_norm_dense_bf16_qmv";
  if (result_m != x_m) return fail(err, errlen, "%s: x and output disagree on M", op);
  if (w_n != result_n) return fail(err, errlen, "%s: w and output disagree on N", op);
  if (w_kblock != 16) return fail(err, errlen, "%s: w is not K-blocked by KBLOCK", op);
  if (w_blocks * 16 != x_kdim) return fail(err, errlen, "%s: w and x disagree on K", op);
  if (x_m < 0 || x_m > kDenseNarrowMaxRows || result_n < 1 || result_n >= kDenseNarrowMaxN || x_kdim < 1 ||
      x_kdim > 2048)
    return fail(err, errlen, "%s: takes at most %d rows, N < %d and K <= 2048", op, kDenseNarrowMaxRows,
                kDenseNarrowMaxN);
  if (!(eps >= 0.0f)) return fail(err, errlen, "%s: eps must be >= 0", op);
  if (x_m == 0) return 0;
  if (!result || !x || !gamma || !w || (residual && !x_out)) return fail(err, errlen, "%s: a tensor is missing", op);
  if (residual) {
    const auto overlap = [&](const void* p) {
      const char* a0 = (const char*)x_out;
      const char* b0 = (const char*)p;
      const size_t bytes = (size_t)(x_m * x_kdim) * sizeof(float);
      return a0 < b0 + bytes && b0 < a0 + bytes;
    };
    if (overlap(x) || overlap(residual))
      return fail(err, errlen, "%s: x_out must not overlap x or residual (workgroups read them while one writes)",
                  op);
  }
  GemvArgs a{};
  a.out = result;
  a.ldo = result_n;
  a.x = x;
  a.ldx = x_kdim;
  a.x_div = 1;
  a.p[0] = Proj{w, nullptr};
  a.kind = kBf16KBlocked;
  a.E = 1;
  a.N = (int)result_n;
  a.K = (int)x_kdim;
  a.gsize = kChunk;
  a.nchunks = (int)((x_kdim + kChunk - 1) / kChunk);
  a.vec = aligned16(w);
  a.batch = batch_for(a.nchunks);
  a.rows = Rows{nullptr, nullptr, nullptr, nullptr, (int)x_m};
  const hipError_t e = launch_norm_dense(a, residual, x_out, gamma, eps, (hipStream_t)stream);
  return e == hipSuccess ? 0 : hip_fail(err, errlen, op, e);
}

int uocr_rms_norm(float* out, float* x_out, const float* x, const float* residual, const float* gamma, int64_t rows,
                  int64_t dim, float eps, void* stream, char* err, size_t errlen) {
  const char* op = "rms_norm";
  if (rows < 0 || rows > INT32_MAX || dim < 1 || dim > INT32_MAX)
    return fail(err, errlen, "%s: bad shape [%lld, %lld]", op, (long long)rows, (long long)dim);
  if (!(eps >= 0.0f)) return fail(err, errlen, "%s: eps must be >= 0", op);
  if (rows == 0) return 0;
  if (!out || !x || !gamma || (residual && !x_out)) return fail(err, errlen, "%s: a tensor is missing", op);
  const hipError_t e = launch_add_rmsnorm(out, x_out, x, residual, gamma, rows, (int)dim, eps, (hipStream_t)stream);
  return e == hipSuccess ? 0 : hip_fail(err, errlen, op, e);
}

int uocr_rope(float* q_out, float* k_out, float* v_out, const float* q, const float* k, const float* v, int64_t rows,
              int64_t heads, int64_t head_dim, int64_t in_row_stride, const int32_t* positions,
              const float* cos_table, const float* sin_table, int64_t table_rows, int64_t table_dim, void* stream,
              char* err, size_t errlen) {
  const char* op = "rope";
  if (head_dim < 2 || head_dim % 2) return fail(err, errlen, "%s: head_dim must be even for RoPE", op);
  if (table_dim != head_dim)
    return fail(err, errlen, "%s: the cos/sin tables are %lld wide, not head_dim %lld", op, (long long)table_dim,
                (long long)head_dim);
  if (rows < 0 || heads < 1 || table_rows < 1 || table_rows > INT32_MAX || head_dim > INT32_MAX ||
      heads > INT32_MAX || rows * heads * head_dim > ((int64_t)1 << 31))
    return fail(err, errlen, "%s: bad shape", op);
  if (in_row_stride < heads * head_dim)
    return fail(err, errlen, "%s: input rows %lld floats apart overlap rows of %lld", op, (long long)in_row_stride,
                (long long)(heads * head_dim));
  if (rows == 0) return 0;
  if (!q || !q_out || !positions || !cos_table || !sin_table || (k && !k_out) || (v && !v_out))
    return fail(err, errlen, "%s: a tensor is missing", op);
  const hipError_t e = launch_rope(q_out, k_out, v_out, q, k, v, rows, (int)heads, (int)head_dim, in_row_stride,
                                   positions, cos_table, sin_table, (int)table_rows, (hipStream_t)stream);
  return e == hipSuccess ? 0 : hip_fail(err, errlen, op, e);
}

int uocr_swiglu(float* out, const float* gate_up, int64_t rows, int64_t ffn, void* stream, char* err,
                size_t errlen) {
  const char* op = "swiglu";
  if (rows < 0 || ffn < 1 || ffn > INT32_MAX || rows * ffn > ((int64_t)1 << 31))
    return fail(err, errlen, "%s: bad shape [%lld, %lld]", op, (long long)rows, (long long)ffn);
  if (rows == 0) return 0;
  if (!out || !gate_up) return fail(err, errlen, "%s: a tensor is missing", op);
  const hipError_t e = launch_swiglu(out, gate_up, rows, (int)ffn, (hipStream_t)stream);
  return e == hipSuccess ? 0 : hip_fail(err, errlen, op, e);
}

// ------------------------------------------------------------------ paged decode attention

// Counters of the attention's in-kernel merge of splits: per device,
// kAttnSlots slots of kAttnCounters words, allocated and zeroed by the first
// call on the device that is not under stream capture (until then calls merge
// with a second launch); each stream takes a slot when first seen (round
// robin), so streams first seen under capture need no allocation.  Every
// launch leaves its counters zero.  Launches on streams that share a slot
// must not overlap in time.
static constexpr int64_t kAttnCounters = 65536;  // (row, head) pairs
static constexpr int kAttnSlots = 16;
struct AttnCounters {
  uint32_t* words = nullptr;
  int next = 0;
  std::map<hipStream_t, int> slot;
};
static std::map<int, AttnCounters> g_attn_counters;

static uint32_t* attn_counters(hipStream_t stream, int64_t pairs) {
  if (pairs > kAttnCounters) return nullptr;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(g_ws_mu);
  AttnCounters& c = g_attn_counters[dev];
  if (c.words == nullptr) {
    if (capturing(stream)) return nullptr;
    const int64_t words = kAttnSlots * kAttnCounters;
    if (hipMalloc(&c.words, words * sizeof(uint32_t)) != hipSuccess) {
      (void)hipGetLastError();
      c.words = nullptr;
      return nullptr;
    }
    // zeroed before any stream uses a slot
    if (launch_zero_words(c.words, words, stream) != hipSuccess || hipStreamSynchronize(stream) != hipSuccess) {
      (void)hipGetLastError();
      (void)hipFree(c.words);
      c.words = nullptr;
      return nullptr;
    }
  }
  auto it = c.slot.find(stream);
  const int k = it != c.slot.end() ? it->second : (c.slot[stream] = c.next++ % kAttnSlots);
  return c.words + (int64_t)k * kAttnCounters;
}

size_t uocr_paged_attention_workspace_bytes(int64_t rows, int64_t heads, int64_t attend_max) {
  if (rows < 0 || heads < 1 || attend_max < 1 || attend_max > INT32_MAX) return 0;
  return attn_workspace_bytes(rows, (int)heads, (int)attend_max);
}

// The checks and launch of both paged attention entries.
static int paged_attention_call(const char* op, float* out, const float* q, const float* k_new, const float* v_new,
                                int64_t in_stride, const int32_t* positions, const float* cos_table,
                                const float* sin_table, int64_t table_rows, int64_t rows, int64_t heads,
                                int64_t head_dim, float* kv_blocks, int64_t pages, int64_t layers, int64_t page_size,
                                int64_t layer, const uint32_t* lookup, int64_t lookup_cols,
                                const uint32_t* attend_lengths, int64_t attend_max, const uint32_t* write_index,
                                float scale, void* workspace, size_t workspace_bytes, void* stream, char* err,
                                size_t errlen) {
  if (head_dim != 128) return fail(err, errlen, "%s: head_dim must be 128, got %lld", op, (long long)head_dim);
  if (page_size < kAttnSplitRows || page_size % kAttnSplitRows)
    return fail(err, errlen, "%s: page_size must be a positive multiple of %d", op, kAttnSplitRows);
  if (pages < 1 || layers < 1 || layer < 0 || layer >= layers)
    return fail(err, errlen, "%s: layer %lld is not in the pool's %lld layers", op, (long long)layer,
                (long long)layers);
  if (rows < 0 || rows > 65535 || heads < 1 || heads > 65535)
    return fail(err, errlen, "%s: rows must be in [0, 65535] and heads in [1, 65535]", op);
  if (lookup_cols < 1 || lookup_cols * page_size > INT32_MAX)
    return fail(err, errlen, "%s: bad lookup table width %lld", op, (long long)lookup_cols);
  if (attend_max < 1 || attend_max > lookup_cols * page_size)
    return fail(err, errlen, "%s: attend_max %lld is not in [1, %lld], the rows the lookup table addresses", op,
                (long long)attend_max, (long long)(lookup_cols * page_size));
  if (pages > INT32_MAX) return fail(err, errlen, "%s: more than 2^31 pages", op);
  if (rows == 0) return 0;
  if (!out || !q || !k_new || !v_new || !kv_blocks || !lookup || !attend_lengths || !write_index)
    return fail(err, errlen, "%s: a tensor is missing", op);
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if (!a16(out) || !a16(q) || !a16(k_new) || !a16(v_new) || !a16(kv_blocks) || !a16(workspace) || in_stride % 4)
    return fail(err, errlen, "%s: q, k_new, v_new, out, kv_blocks and workspace must be 16-byte aligned", op);
  const hipStream_t s = (hipStream_t)stream;
  void* ws = nullptr;
  if (resolve_workspace(op, workspace, workspace_bytes, attn_workspace_bytes(rows, (int)heads, (int)attend_max), s,
                        &ws, err, errlen))
    return 1;
  PagedAttention p{};
  p.out = out;
  p.q = q;
  p.k_new = k_new;
  p.v_new = v_new;
  p.kv_blocks = kv_blocks;
  p.pages = (int)pages;
  p.layers = (int)layers;
  p.page_size = (int)page_size;
  p.heads = (int)heads;
  p.head_dim = (int)head_dim;
  p.layer = (int)layer;
  p.lookup = lookup;
  p.lookup_cols = (int)lookup_cols;
  p.write_index = write_index;
  p.attend_lengths = attend_lengths;
  p.max_attend = (int)attend_max;
  p.rows = rows;
  p.scale = scale;
  p.workspace = (float*)ws;
  p.counters = attn_counters(s, rows * heads);
  p.in_stride = in_stride;
  p.positions = positions;
  p.cos_table = cos_table;
  p.sin_table = sin_table;
  p.table_rows = (int)table_rows;
  const hipError_t e = launch_paged_attention(p, s);
  return e == hipSuccess ? 0 : hip_fail(err, errlen, op, e);
}

int uocr_paged_decode_attention(float* out, const float* q, const float* k_new, const float* v_new, int64_t rows,
                                int64_t heads, int64_t head_dim, float* kv_blocks, int64_t pages, int64_t layers,
                                int64_t page_size, int64_t layer, const uint32_t* lookup, int64_t lookup_cols,
                                const uint32_t* attend_lengths, int64_t attend_max, const uint32_t* write_index,
                                float scale, void* workspace, size_t workspace_bytes, void* stream, char* err,
                                size_t errlen) {
  return paged_attention_call("paged_decode_attention", out, q, k_new, v_new, heads * head_dim, nullptr, nullptr,
                              nullptr, 0, rows, heads, head_dim, kv_blocks, pages, layers, page_size, layer, lookup,
                              lookup_cols, attend_lengths, attend_max, write_index, scale, workspace,
                              workspace_bytes, stream, err, errlen);
}

int uocr_paged_decode_attention_qkv(float* out, const float* qkv, int64_t rows, int64_t heads, int64_t head_dim,
                                    int64_t row_stride, const int32_t* positions, const float* cos_table,
                                    const float* sin_table, int64_t table_rows, int64_t table_dim, float* kv_blocks,
                                    int64_t pages, int64_t layers, int64_t page_size, int64_t layer,
                                    const uint32_t* lookup, int64_t lookup_cols, const uint32_t* attend_lengths,
                                    int64_t attend_max, const uint32_t* write_index, float scale, void* workspace,
                                    size_t workspace_bytes, void* stream, char* err, size_t errlen) {
  const char* op = "paged_decode_attention_qkv";
  if (table_dim != head_dim)
    return fail(err, errlen, "%s: the cos/sin tables are %lld wide, not head_dim %lld", op, (long long)table_dim,
                (long long)head_dim);
  if (table_rows < 1 || table_rows > INT32_MAX) return fail(err, errlen, "%s: bad cos/sin table", op);
  if (row_stride < 3 * heads * head_dim)
    return fail(err, errlen, "%s: qkv rows %lld floats apart overlap rows of %lld", op, (long long)row_stride,
                (long long)(3 * heads * head_dim));
  if (rows > 0 && (!qkv || !positions || !cos_table || !sin_table))
    return fail(err, errlen, "%s: a tensor is missing", op);
  const float* k = qkv ? qkv + heads * head_dim : nullptr;
  const float* v = qkv ? qkv + 2 * heads * head_dim : nullptr;
  return paged_attention_call(op, out, qkv, k, v, row_stride, positions, cos_table, sin_table, table_rows, rows,
                              heads, head_dim, kv_blocks, pages, layers, page_size, layer, lookup, lookup_cols,
                              attend_lengths, attend_max, write_index, scale, workspace, workspace_bytes, stream, err,
                              errlen);
}

// ------------------------------------------------------------------ the MoE block

static int check_layer(const char* op, const uocr_moe_layer* L, int64_t hidden, char* err, size_t errlen) {
  if (L == nullptr) return fail(err, errlen, "%s: no layer", op);
  if (L->num_experts < 1 || L->num_experts > 64) return fail(err, errlen, "%s: num_experts must be in [1, 64]", op);
  if (L->top_k < 1 || L->top_k > L->num_experts)
    return fail(err, errlen, "%s: top_k must be in [1, num_experts]", op);
  if (hidden != L->hidden) return fail(err, errlen, "%s: x and the layer disagree on hidden", op);
  if (L->hidden < 16 || L->hidden % 16 || L->shared_ffn < 16 || L->shared_ffn % 16 || L->ffn < 1)
    return fail(err, errlen, "%s: hidden and shared_ffn must be positive multiples of 16", op);
  if (L->int8 && (L->group < 1 || L->hidden % L->group || L->ffn % L->group))
    return fail(err, errlen, "%s: hidden and ffn must be multiples of the int8 group", op);
  if (!L->router || !L->gate_proj || !L->up_proj || !L->down_proj || !L->shared_gate || !L->shared_up ||
      !L->shared_down)
    return fail(err, errlen, "%s: a layer weight is missing", op);
  if (L->int8 && (!L->gate_proj_scales || !L->up_proj_scales || !L->down_proj_scales))
    return fail(err, errlen, "%s: an int8 layer needs its scales", op);
  return 0;
}

struct DecodeBufs {
  float* logits;
  int32_t* ids;
  float* wts;
  GroupTables g;
  float* h;
  float* hs;
  float* y;
  float* sh;
};

static DecodeBufs carve_decode(Carve& c, const uocr_moe_layer* L, int64_t B) {
  const int64_t R = B * L->top_k;
  DecodeBufs d{};
  d.logits = c.take<float>(B * L->num_experts);
  d.ids = c.take<int32_t>(R);
  d.wts = c.take<float>(R);
  d.g = carve_tables(c, (int)L->num_experts, (int)R, false, false);
  d.h = c.take<float>(R * L->ffn);
  d.hs = c.take<float>(B * L->shared_ffn);
  d.y = c.take<float>(R * L->hidden);
  d.sh = c.take<float>(B * L->hidden);
  return d;
}

// LDS per workgroup on gfx950.
constexpr size_t kMaxLds = 160 * 1024;

static bool fused_eligible(const uocr_moe_layer* L, int64_t B) {
  const char* env = std::getenv("UOCR_MOE_DECODE");
  if (env != nullptr && std::strcmp(env, "multi") == 0) return false;
  if (B < 1 || B > 8 || L->top_k > 8 || B * L->top_k > 64 || L->num_experts > 64) return false;
  for (int64_t d : {L->hidden, L->ffn, L->shared_ffn})
    if (d % 128 || d > 2048) return false;
  if (L->int8 && L->group != 128) return false;
  for (const void* p : {L->gate_proj, L->up_proj, L->down_proj, (const void*)L->shared_gate,
                        (const void*)L->shared_up, (const void*)L->shared_down})
    if (!aligned16(p)) return false;
  const FusedLayout lay = fused_layout((int)B, (int)L->num_experts, (int)L->hidden, (int)L->ffn,
                                       (int)L->shared_ffn, (int)L->top_k);
  return lay.lds_bytes <= kMaxLds;
}

// Polls per bounded wait of the persistent kernel: 2^16 (tens of milliseconds;
// healthy waits take microseconds).  UOCR_MOE_SPIN_LIMIT overrides it, so a
// test can make the waits run out and check the failure path (0: every wait
// fails at once, even one whose data is there).
static uint32_t fused_spin_limit() {
  const char* env = std::getenv("UOCR_MOE_SPIN_LIMIT");
  if (env != nullptr) {
    const long v = std::strtol(env, nullptr, 10);
    if (v >= 0 && v <= (1L << 30)) return (uint32_t)v;
  }
  return 1u << 16;
}

static FusedLayerW fused_weights(const uocr_moe_layer* L) {
  FusedLayerW w;
  w.router = L->router;
  w.gate_w = L->gate_proj;
  w.up_w = L->up_proj;
  w.down_w = L->down_proj;
  w.gate_s = L->gate_proj_scales;
  w.up_s = L->up_proj_scales;
  w.down_s = L->down_proj_scales;
  w.sh_gate = L->shared_gate;
  w.sh_up = L->shared_up;
  w.sh_down = L->shared_down;
  return w;
}

static FusedArgs fused_args(const uocr_moe_layer* L, int64_t B, const FusedLayout& lay, const FusedSlot& f) {
  FusedArgs a{};
  a.B = (int)B;
  a.E = (int)L->num_experts;
  a.H = (int)L->hidden;
  a.F = (int)L->ffn;
  a.Fs = (int)L->shared_ffn;
  a.topk = (int)L->top_k;
  a.int8 = L->int8;
  a.renorm = L->renormalize;
  a.n_layers = 1;
  a.w[0] = fused_weights(L);
  a.ctl = f.ctl;
  a.logits = f.data + lay.off_logits;
  a.h = f.data + lay.off_h;
  a.y = f.data + lay.off_y;
  a.hs = f.data + lay.off_hs;
  a.p_sgu = f.data + lay.off_psgu;
  a.p_sdn = f.data + lay.off_psdn;
  a.gh = lay.gh;
  a.gf = lay.gf;
  a.gfs = lay.gfs;
  a.sub = lay.sub;
  a.c_gu = lay.c_gu;
  a.c_dn = lay.c_dn;
  a.per_e_gu = lay.per_e_gu;
  a.per_e_dn = lay.per_e_dn;
  a.cb_fs = lay.cb_fs;
  a.cb_h = lay.cb_h;
  a.n_sgu = lay.n_sgu;
  a.n_sdn = lay.n_sdn;
  a.n_sfold = lay.n_sfold;
  a.n_comb = lay.n_comb;
  a.lds_x = lay.lds_x;
  a.lds_act = lay.lds_act;
  a.inv_gh = 1.0f / (float)lay.gh;
  a.inv_gf = 1.0f / (float)lay.gf;
  auto magic = [](int d) { return d <= 1 ? 0u : (uint32_t)((((uint64_t)1 << 32) + (uint64_t)d - 1) / (uint64_t)d); };
  a.m_2gh = magic(2 * lay.gh);
  a.m_gh = magic(lay.gh);
  a.m_gu = magic(lay.per_e_gu);
  a.m_b = magic(B);
  a.m_gfs = magic(lay.gfs);
  a.m_dn = magic(lay.per_e_dn);
  a.early_shared = B <= kFusedEarlySharedRows ? 1 : 0;
  a.defer_down = B <= kFusedEarlySharedRows ? 1 : 0;
  a.m_h = magic(a.H);
  a.spin_limit = fused_spin_limit();
  return a;
}

struct PrefillBufs {
  uint16_t* xb;  // x rounded to bf16 [T][H]
  float* logits;
  int32_t* ids;
  float* wts;
  GroupTables g;
  uint16_t* hb;
  uint16_t* hsb;
  float* y;
  float* sh;
  int32_t* hist;   // per counting workgroup: its rows per expert
};

static PrefillBufs carve_prefill(Carve& c, const uocr_moe_layer* L, int64_t T) {
  const int64_t R = T * L->top_k;
  PrefillBufs d{};
  d.xb = c.take<uint16_t>(T * L->hidden);
  d.logits = c.take<float>(T * L->num_experts);
  d.ids = c.take<int32_t>(R);
  d.wts = c.take<float>(R);
  d.g = carve_tables(c, (int)L->num_experts, (int)R, true, true);
  d.hb = c.take<uint16_t>(R * L->ffn);
  d.hsb = c.take<uint16_t>(T * L->shared_ffn);
  d.y = c.take<float>(R * L->hidden);
  d.sh = c.take<float>(2 * T * L->hidden);  // the shared experts' down sums, in up to two K ranges
  // (the T < 2048 routing's 4-token blocks outnumber the T >= 2048 one's 16-token blocks)
  d.hist = c.take<int32_t>((int64_t)fused_route_blocks((int)T) * L->num_experts);
  return d;
}

size_t uocr_moe_workspace_bytes(const uocr_moe_layer* layer, int64_t rows, int prefill) {
  if (layer == nullptr || rows < 0) return 0;
  Carve c(nullptr);
  if (prefill) {
    carve_prefill(c, layer, rows);
  } else {
    carve_decode(c, layer, rows);
  }
  return c.off + 256;
}

int uocr_moe_gate(int64_t* indices, float* weights, const float* x, int64_t seq, int64_t hidden,
                  const float* router, int64_t num_experts, int64_t top_k, int renormalize, void* workspace,
                  size_t workspace_bytes, void* stream, char* err, size_t errlen) {
  const char* op = "uocr_moe_gate";
  if (num_experts < 1 || num_experts > 64) return fail(err, errlen, "%s: num_experts must be in [1, 64]", op);
  if (top_k < 1 || top_k > num_experts) return fail(err, errlen, "%s: top_k must be in [1, num_experts]", op);
  if (seq < 0 || hidden < 1) return fail(err, errlen, "%s: bad x shape", op);
  if (seq == 0) return 0;
  const hipStream_t s = (hipStream_t)stream;
  void* ws = nullptr;
  if (resolve_workspace(op, workspace, workspace_bytes, (size_t)(seq * num_experts) * sizeof(float) + 256, s, &ws,
                        err, errlen))
    return 1;
  float* logits = static_cast<float*>(ws);
  hipError_t e = launch_logits(logits, x, hidden, router, (int)seq, (int)num_experts, (int)hidden, nullptr, s);
  if (e == hipSuccess)
    e = launch_softmax_topk(logits, (int)seq, (int)num_experts, (int)top_k, renormalize, nullptr, indices, weights,
                            s);
  return e == hipSuccess ? 0 : hip_fail(err, errlen, op, e);
}

}  // extern "C"

// The decode layer of both decode entry points.  fixed: the persistent kernel's
// control words and arena (the static scratch's); null: the stream's own slot.
static int decode_rows_impl(const char* op, float* out, const float* x, int64_t rows, int64_t hidden,
                            const uocr_moe_layer* L, int32_t* expert_ids, float* expert_weights, void* workspace,
                            size_t workspace_bytes, hipStream_t s, const FusedSlot* fixed, char* err,
                            size_t errlen) {
  if (check_layer(op, L, hidden, err, errlen)) return 1;
  if (rows < 0 || rows > 64) return fail(err, errlen, "%s: rows must be in [0, 64]", op);
  if (rows == 0) return 0;
  const int64_t B = rows, R = rows * L->top_k;
  if (fused_eligible(L, B)) {
    const FusedLayout lay = fused_layout((int)B, (int)L->num_experts, (int)L->hidden, (int)L->ffn,
                                         (int)L->shared_ffn, (int)L->top_k, fused_sub(L->int8 != 0, (int)B));
    FusedSlot slot;
    hipError_t e = hipSuccess;
    if (fixed != nullptr) {
      slot = *fixed;
    } else {
      bool need_alloc = false;
      e = fused_slot(s, &slot, &need_alloc);
      if (e == hipSuccess && need_alloc)
        return fail(err, errlen,
                    "%s: no free control slot for a new stream under capture (make a decode call on this device "
                    "outside stream capture first; it keeps a spare slot ready)",
                    op);
    }
    int grid = 0;
    if (e == hipSuccess) e = fused_grid_cached(lay.lds_bytes, &grid);
    if (e != hipSuccess) return hip_fail(err, errlen, op, e);
    if (grid < 1) return fail(err, errlen, "%s: the persistent decode kernel does not fit a CU", op);
    FusedArgs a = fused_args(L, B, lay, slot);
    // tokens per router task: every XCD computes all E x B logits on kFusedRouterWaves waves of each of its
    // workgroups
    const int64_t router_slots = (int64_t)(grid / kFusedXcds) * kFusedRouterWaves;
    const int64_t xcd_experts = L->num_experts;
    a.r_tok = 1;
    while (a.r_tok < B && xcd_experts * ((B + a.r_tok - 1) / a.r_tok) > router_slots) ++a.r_tok;
    if (grid % kFusedXcds != 0 || xcd_experts * ((B + a.r_tok - 1) / a.r_tok) > router_slots)
      return fail(err, errlen, "%s: the persistent decode kernel needs a grid of whole XCDs with room for its "
                  "router tasks", op);
    a.x = x;
    a.x_vec = aligned16(x) ? 1 : 0;
    a.out = out;
    a.ids_out = expert_ids;
    a.wts_out = expert_weights;
    if (fixed == nullptr) {
      std::lock_guard<std::mutex> lock(g_ws_mu);
      if (g_trace != nullptr && g_trace_words >= ((int64_t)lay.max_tasks + grid) * 8) {
        a.trace = g_trace;
        a.trace_wg = (int64_t)lay.max_tasks * 8;
        g_trace = nullptr;
        g_trace_grid = grid;
      }
    }
    // the static scratch's calls are not ordered (overlapping calls race, as documented)
    if (fixed != nullptr)
      e = launch_decode_fused(a, grid, lay.lds_bytes, s);
    else
      e = fused_ordered_launch(s, [&] { return launch_decode_fused(a, grid, lay.lds_bytes, s); });
    return e == hipSuccess ? 0 : hip_fail(err, errlen, op, e);
  }
  Carve dry(nullptr);
  carve_decode(dry, L, B);
  void* ws = nullptr;
  if (resolve_workspace(op, workspace, workspace_bytes, dry.off, s, &ws, err, errlen)) return 1;
  Carve c(ws);
  const DecodeBufs d = carve_decode(c, L, B);
  const int E = (int)L->num_experts, H = (int)L->hidden, F = (int)L->ffn, Fs = (int)L->shared_ffn;
  const int max_groups = (int)(E < R ? E : R);

  hipError_t e = launch_logits(d.logits, x, H, L->router, (int)B, E, H, nullptr, s);
  if (e == hipSuccess) e = launch_route_small(d.logits, (int)B, E, (int)L->top_k, L->renormalize, d.ids, d.wts, d.g, s);
  if (e != hipSuccess) return hip_fail(err, errlen, op, e);

  // gate/up (+ SwiGLU) for the routed rows and the shared experts
  GemvArgs gu{};
  gu.out = d.h;
  gu.ldo = F;
  gu.x = x;
  gu.ldx = H;
  gu.x_div = (int)L->top_k;
  gu.kind = L->int8 ? kInt8Rows : kBf16Rows;
  gu.p[0] = Proj{L->gate_proj, L->gate_proj_scales};
  gu.p[1] = Proj{L->up_proj, L->up_proj_scales};
  gu.E = E;
  gu.N = F;
  gu.K = H;
  if (L->int8) {
    gu.gsize = (int)L->group;
    gu.nchunks = H / (int)L->group;
    gu.vec = (H % 16 == 0) && (gu.gsize % 16 == 0) && aligned16(L->gate_proj) && aligned16(L->up_proj);
  } else {
    gu.gsize = kChunk;
    gu.nchunks = (H + kChunk - 1) / kChunk;
    gu.vec = (H % 8 == 0) && aligned16(L->gate_proj) && aligned16(L->up_proj);
  }
  gu.batch = batch_for(gu.nchunks);
  gu.rows = rows_of(d.g);

  GemvArgs sgu{};
  sgu.out = d.hs;
  sgu.ldo = Fs;
  sgu.x = x;
  sgu.ldx = H;
  sgu.x_div = 1;
  sgu.kind = kBf16KBlocked;
  sgu.p[0] = Proj{L->shared_gate, nullptr};
  sgu.p[1] = Proj{L->shared_up, nullptr};
  sgu.E = 1;
  sgu.N = Fs;
  sgu.K = H;
  sgu.gsize = kChunk;
  sgu.nchunks = (H + kChunk - 1) / kChunk;
  sgu.vec = aligned16(L->shared_gate) && aligned16(L->shared_up);
  sgu.batch = batch_for(sgu.nchunks);
  sgu.rows = Rows{nullptr, nullptr, nullptr, nullptr, (int)B};
  const int w1 = waves_for(gu.batch > sgu.batch ? gu.batch : sgu.batch);
  e = launch_gemv_pair(gu, max_groups, sgu, 2, w1, s);
  if (e != hipSuccess) return hip_fail(err, errlen, op, e);

  // down for the routed rows and the shared experts
  GemvArgs dn = gu;
  dn.out = d.y;
  dn.ldo = H;
  dn.x = d.h;
  dn.ldx = F;
  dn.x_div = 1;
  dn.p[0] = Proj{L->down_proj, L->down_proj_scales};
  dn.p[1] = Proj{nullptr, nullptr};
  dn.N = H;
  dn.K = F;
  if (L->int8) {
    dn.nchunks = F / (int)L->group;
    dn.vec = (F % 16 == 0) && (dn.gsize % 16 == 0) && aligned16(L->down_proj);
  } else {
    dn.nchunks = (F + kChunk - 1) / kChunk;
    dn.vec = (F % 8 == 0) && aligned16(L->down_proj);
  }
  dn.batch = batch_for(dn.nchunks);
  GemvArgs sdn = sgu;
  sdn.out = d.sh;
  sdn.ldo = H;
  sdn.x = d.hs;
  sdn.ldx = Fs;
  sdn.p[0] = Proj{L->shared_down, nullptr};
  sdn.p[1] = Proj{nullptr, nullptr};
  sdn.N = H;
  sdn.K = Fs;
  sdn.nchunks = (Fs + kChunk - 1) / kChunk;
  sdn.vec = aligned16(L->shared_down);
  sdn.batch = batch_for(sdn.nchunks);
  const int w2 = waves_for(dn.batch > sdn.batch ? dn.batch : sdn.batch);
  e = launch_gemv_pair(dn, max_groups, sdn, 1, w2, s);
  if (e == hipSuccess) e = launch_combine(out, d.y, H, d.wts, nullptr, d.sh, (int)B, H, (int)L->top_k, s);
  if (e == hipSuccess && expert_ids) e = hipMemcpyAsync(expert_ids, d.ids, R * sizeof(int32_t), hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess && expert_weights)
    e = hipMemcpyAsync(expert_weights, d.wts, R * sizeof(float), hipMemcpyDeviceToDevice, s);
  return e == hipSuccess ? 0 : hip_fail(err, errlen, op, e);
}

// The address of `scratch` on the current device, looked up once per device;
// that first call also clears the persistent kernel's region with a kernel (the
// array is zero at load; a kernel rather than a memset because this call may
// be under stream capture).
static hipError_t scratch_base(hipStream_t s, char** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(g_ws_mu);
  auto it = g_scratch.find(dev);
  if (it != g_scratch.end()) {
    *out = it->second;
    return hipSuccess;
  }
  void* p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  if (p == nullptr) return hipErrorInvalidSymbol;
  e = launch_zero_words(static_cast<uint32_t*>(p), (int64_t)(kScratchFusedBytes / 4), s);
  if (e != hipSuccess) return e;
  g_scratch[dev] = static_cast<char*>(p);
  *out = static_cast<char*>(p);
  return hipSuccess;
}

extern "C" {

int uocr_moe_decode_rows(float* out, const float* x, int64_t rows, int64_t hidden, const uocr_moe_layer* L,
                         int32_t* expert_ids, float* expert_weights, void* workspace, size_t workspace_bytes,
                         void* stream, char* err, size_t errlen) {
  return decode_rows_impl("uocr_moe_decode_rows", out, x, rows, hidden, L, expert_ids, expert_weights, workspace,
                          workspace_bytes, (hipStream_t)stream, nullptr, err, errlen);
}

int uocr_moe_decode_rows_static(float* out, const float* x, int64_t rows, int64_t hidden, const uocr_moe_layer* L,
                                int32_t* expert_ids, float* expert_weights, void* stream, char* err, size_t errlen) {
  const char* op = "uocr_moe_decode_rows_static";
  // every size check runs before the first device call
  if (check_layer(op, L, hidden, err, errlen)) return 1;
  if (rows < 0 || rows > 64) return fail(err, errlen, "%s: rows must be in [0, 64]", op);
  if (rows == 0) return 0;
  if ((size_t)kFusedCtlWords * 4 + (size_t)fused_max_words() * 8 > kScratchFusedBytes)
    return fail(err, errlen, "%s: the persistent kernel's arena does not fit the scratch", op);
  if (!fused_eligible(L, rows)) {
    Carve dry(nullptr);
    carve_decode(dry, L, rows);
    if (dry.off > kScratchBytes - kScratchFusedBytes)
      return fail(err, errlen, "%s: %lld rows of this layer need %zu bytes of scratch, more than the %zu it has", op,
                  (long long)rows, dry.off, kScratchBytes - kScratchFusedBytes);
  }
  const hipStream_t s = (hipStream_t)stream;
  char* base = nullptr;
  const hipError_t e = scratch_base(s, &base);
  if (e != hipSuccess) return hip_fail(err, errlen, op, e);
  const FusedSlot fixed{reinterpret_cast<uint32_t*>(base), reinterpret_cast<uint64_t*>(base + (size_t)kFusedCtlWords * 4)};
  return decode_rows_impl(op, out, x, rows, hidden, L, expert_ids, expert_weights, base + kScratchFusedBytes,
                          kScratchBytes - kScratchFusedBytes, s, &fixed, err, errlen);
}

int uocr_moe_decode_stack(float* out, const float* x, int64_t rows, int64_t hidden,
                          const uocr_moe_layer* const* layers, int64_t n_layers, void* stream, char* err,
                          size_t errlen) {
  const char* op = "uocr_moe_decode_stack";
  if (layers == nullptr || n_layers < 1 || n_layers > kFusedMaxLayers)
    return fail(err, errlen, "%s: n_layers must be in [1, %d]", op, kFusedMaxLayers);
  const uocr_moe_layer* L0 = layers[0];
  for (int64_t l = 0; l < n_layers; ++l) {
    const uocr_moe_layer* L = layers[l];
    if (check_layer(op, L, hidden, err, errlen)) return 1;
    if (L->num_experts != L0->num_experts || L->hidden != L0->hidden || L->ffn != L0->ffn ||
        L->shared_ffn != L0->shared_ffn || L->top_k != L0->top_k || L->int8 != L0->int8 ||
        L->group != L0->group || L->renormalize != L0->renormalize)
      return fail(err, errlen, "%s: layer %lld differs in shape or kind from layer 0", op, (long long)l);
  }
  if (rows < 0 || rows > 8) return fail(err, errlen, "%s: rows must be in [0, 8]", op);
  if (rows == 0) return 0;
  for (int64_t l = 0; l < n_layers; ++l)
    if (!fused_eligible(layers[l], rows))
      return fail(err, errlen, "%s: layer %lld does not take the persistent decode kernel (shapes, alignment or "
                  "UOCR_MOE_DECODE=multi); chain uocr_moe_decode_rows instead", op, (long long)l);
  const int64_t B = rows;
  const hipStream_t s = (hipStream_t)stream;
  const FusedLayout lay = fused_layout((int)B, (int)L0->num_experts, (int)L0->hidden, (int)L0->ffn,
                                       (int)L0->shared_ffn, (int)L0->top_k, fused_sub(L0->int8 != 0, (int)B));
  FusedSlot slot;
  bool need_alloc = false;
  hipError_t e = fused_slot(s, &slot, &need_alloc);
  uint64_t* arena = nullptr;
  if (e == hipSuccess && !need_alloc) e = fused_stack_arena(s, &arena, &need_alloc);
  if (e == hipSuccess && need_alloc)
    return fail(err, errlen, "%s: no arena for a new stream under capture (make a stacked call on this stream "
                "outside stream capture first)", op);
  int grid = 0;
  if (e == hipSuccess) e = fused_grid_cached(lay.lds_bytes, &grid);
  if (e != hipSuccess) return hip_fail(err, errlen, op, e);
  if (grid < 1) return fail(err, errlen, "%s: the persistent decode kernel does not fit a CU", op);
  // the layers' buffers in the stack arena, the control words in the stream's slot
  FusedArgs a = fused_args(L0, B, lay, FusedSlot{slot.ctl, arena});
  a.residual = 1;
  a.n_layers = (int)n_layers;
  a.layer_words = fused_max_words();
  a.xs_pairs = arena + (int64_t)kFusedMaxLayers * fused_max_words();
  for (int64_t l = 0; l < n_layers; ++l) a.w[l] = fused_weights(layers[l]);
  const int64_t router_slots = (int64_t)(grid / kFusedXcds) * kFusedRouterWaves;
  a.r_tok = 1;
  while (a.r_tok < B && L0->num_experts * ((B + a.r_tok - 1) / a.r_tok) > router_slots) ++a.r_tok;
  if (grid % kFusedXcds != 0 || L0->num_experts * ((B + a.r_tok - 1) / a.r_tok) > router_slots)
    return fail(err, errlen, "%s: the persistent decode kernel needs a grid of whole XCDs with room for its "
                "router tasks", op);
  a.x = x;
  a.x_vec = aligned16(x) ? 1 : 0;
  a.out = out;
  a.ids_out = nullptr;
  a.wts_out = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    const int64_t per_layer = (int64_t)lay.max_tasks + grid;  // records of one layer
    if (g_trace != nullptr && g_trace_words >= per_layer * n_layers * 8) {
      a.trace = g_trace;
      a.trace_wg = (int64_t)lay.max_tasks * 8;
      a.trace_layer = per_layer;
      g_trace = nullptr;
      g_trace_grid = grid;
    }
  }
  e = fused_ordered_launch(s, [&] { return launch_decode_fused(a, grid, lay.lds_bytes, s); });
  return e == hipSuccess ? 0 : hip_fail(err, errlen, op, e);
}

int uocr_moe_forward(float* out, const float* x, int64_t seq, int64_t hidden, const uocr_moe_layer* L,
                     int32_t* expert_ids, float* expert_weights, void* workspace, size_t workspace_bytes,
                     void* stream, char* err, size_t errlen) {
  const char* op = "uocr_moe_forward";
  if (check_layer(op, L, hidden, err, errlen)) return 1;
  const int BK = gemm_bk();
  if (L->hidden % BK || L->ffn % BK || L->shared_ffn % BK)
    return fail(err, errlen, "%s: hidden, ffn and shared_ffn must be multiples of %d", op, BK);
  if (L->int8 && (L->group % 64 || BK % L->group != 0 && L->group % BK != 0))
    return fail(err, errlen, "%s: the int8 group must be 64, 128 or a multiple of 128", op);
  // x is read by scalar loads; the weights by 16-byte loads when every stack is 16-byte aligned, else by
  // loads of whatever width their alignment allows (the same bits; the reference picks its load path the
  // same way, unlimited_ocr_max/kernels/loads.mojo:59-89)
  const bool vec = aligned16(L->gate_proj) && aligned16(L->up_proj) && aligned16(L->down_proj) &&
                   aligned16(L->shared_gate) && aligned16(L->shared_up) && aligned16(L->shared_down);
  if ((reinterpret_cast<uintptr_t>(x) & 3u) != 0) return fail(err, errlen, "%s: x must be 4-byte aligned", op);
  if (seq < 0 || seq * L->top_k > ((int64_t)1 << 28)) return fail(err, errlen, "%s: seq out of range", op);
  if (seq == 0) return 0;
  const hipStream_t s = (hipStream_t)stream;
  const int64_t T = seq, R = seq * L->top_k;
  const int BM = R >= 8192 && vec ? 128 : 64;  // rows per GEMM tile
  Carve dry(nullptr);
  carve_prefill(dry, L, T);
  void* ws = nullptr;
  if (resolve_workspace(op, workspace, workspace_bytes, dry.off, s, &ws, err, errlen)) return 1;
  Carve c(ws);
  const PrefillBufs d = carve_prefill(c, L, T);
  const int E = (int)L->num_experts, H = (int)L->hidden, F = (int)L->ffn, Fs = (int)L->shared_ffn;

  // routing (E <= 64 here): below 2048 tokens one launch computes the logits, the top-k and
  // per-workgroup counts; above, the logits tiles share router rows over more tokens and the
  // top-k runs in its own launch
  hipError_t e = hipSuccess;
  if (T < 2048) {
    e = launch_logits_topk_group(d.logits, d.xb, x, H, L->router, (int)T, E, H, (int)L->top_k, L->renormalize, d.ids,
                                 d.wts, BM, d.g, d.hist, s);
  } else {
    e = launch_logits(d.logits, x, H, L->router, (int)T, E, H, d.xb, s);
    if (e == hipSuccess)
      e = launch_topk_group(d.logits, (int)T, E, (int)L->top_k, L->renormalize, d.ids, d.wts, BM, d.g, d.hist, s);
  }
  if (e != hipSuccess) return hip_fail(err, errlen, op, e);
  const int max_groups = (int)(E < R ? E : R);

  GemmProblem gu{};
  gu.a = d.xb;
  gu.lda = H;
  gu.a_by_token = 1;
  gu.x_div = (int)L->top_k;
  gu.p[0] = Proj{L->gate_proj, L->gate_proj_scales};
  gu.p[1] = Proj{L->up_proj, L->up_proj_scales};
  gu.kind = L->int8 ? kInt8Rows : kBf16Rows;
  gu.N = F;
  gu.K = H;
  gu.groups = L->int8 ? (int)(H / L->group) : 1;
  gu.rows = rows_of(d.g);
  gu.tile_start = d.g.tile_start;
  gu.max_groups = max_groups;
  gu.M = (int)R;
  gu.swiglu = 1;
  gu.outb = d.hb;
  gu.ldo = F;
  gu.out_by_position = 1;

  GemmProblem sgu{};
  sgu.a = d.xb;
  sgu.lda = H;
  sgu.a_by_token = 1;
  sgu.x_div = 1;
  sgu.p[0] = Proj{L->shared_gate, nullptr};
  sgu.p[1] = Proj{L->shared_up, nullptr};
  sgu.kind = kBf16KBlocked;
  sgu.N = Fs;
  sgu.K = H;
  sgu.rows = Rows{nullptr, nullptr, nullptr, nullptr, 0};
  sgu.M = (int)T;
  sgu.swiglu = 1;
  sgu.outb = d.hsb;
  sgu.ldo = Fs;
  e = launch_gemm_pair(gu, sgu, BM, s, vec);
  if (e != hipSuccess) return hip_fail(err, errlen, op, e);

  GemmProblem dn = gu;
  dn.a = d.hb;
  dn.lda = F;
  dn.a_by_token = 0;
  dn.x_div = 1;
  dn.p[0] = Proj{L->down_proj, L->down_proj_scales};
  dn.p[1] = Proj{nullptr, nullptr};
  dn.N = H;
  dn.K = F;
  dn.groups = L->int8 ? (int)(F / L->group) : 1;
  dn.swiglu = 0;
  dn.outb = nullptr;
  dn.outf = d.y;
  dn.ldo = H;

  GemmProblem sdn = sgu;
  sdn.a = d.hsb;
  sdn.lda = Fs;
  sdn.a_by_token = 0;
  sdn.p[0] = Proj{L->shared_down, nullptr};
  sdn.p[1] = Proj{nullptr, nullptr};
  sdn.N = H;
  sdn.K = Fs;
  sdn.swiglu = 0;
  sdn.outb = nullptr;
  sdn.outf = d.sh;
  sdn.ldo = H;
  // The shared down projection in two K ranges of Fs / 2 at small T, each its own tiles (summed by the
  // combine): its K steps a tile are twice a routed down tile's, which made the shared tiles the
  // launch's longest at T = 512 (down 43 -> 35 us).
  sdn.kparts = gemm_shared_parts(dn, sdn);
  sdn.part_stride = T * H;
  e = launch_gemm_pair(dn, sdn, BM, s, vec);
  if (e == hipSuccess)
    e = launch_combine(out, d.y, H, d.wts, d.g.inv, d.sh, (int)T, H, (int)L->top_k, s, sdn.kparts);
  if (e == hipSuccess && expert_ids) e = hipMemcpyAsync(expert_ids, d.ids, R * sizeof(int32_t), hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess && expert_weights)
    e = hipMemcpyAsync(expert_weights, d.wts, R * sizeof(float), hipMemcpyDeviceToDevice, s);
  return e == hipSuccess ? 0 : hip_fail(err, errlen, op, e);
}

int uocr_moe_timing_begin(int capacity, char* err, size_t errlen) {
  if (capacity < 1) return fail(err, errlen, "uocr_moe_timing_begin: capacity must be >= 1");
  std::lock_guard<std::mutex> lock(g_timing.mu);
  while ((int)g_timing.start.size() < capacity) {
    hipEvent_t a = nullptr, b = nullptr;
    hipError_t e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&b);
    if (e != hipSuccess) return hip_fail(err, errlen, "uocr_moe_timing_begin", e);
    g_timing.start.push_back(a);
    g_timing.stop.push_back(b);
    g_timing.names.emplace_back();
  }
  g_timing.used = 0;
  g_timing.on = true;
  return 0;
}

int uocr_moe_timing_end(int capacity, float* ms, char* names, size_t name_stride, int* count, char* err,
                        size_t errlen) {
  std::lock_guard<std::mutex> lock(g_timing.mu);
  g_timing.on = false;
  const int n = (int)(g_timing.used < (size_t)capacity ? g_timing.used : (size_t)capacity);
  for (int i = 0; i < n; ++i) {
    hipError_t e = hipEventSynchronize(g_timing.stop[i]);
    float t = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&t, g_timing.start[i], g_timing.stop[i]);
    if (e != hipSuccess) return hip_fail(err, errlen, "uocr_moe_timing_end", e);
    if (ms) ms[i] = t;
    if (names && name_stride > 0) {
      std::snprintf(names + (size_t)i * name_stride, name_stride, "%s", g_timing.names[i].c_str());
    }
  }
  if (count) *count = n;
  g_timing.used = 0;
  return 0;
}

int uocr_moe_fused_trace(void* buffer, int64_t words, int* grid_waves, char* err, size_t errlen) {
  if (!fused_trace_built())
    return fail(err, errlen, "uocr_moe_fused_trace: the library was built without the decode phase trace "
                "(build with UOCR_DECODE_TRACE=1)");
  std::lock_guard<std::mutex> lock(g_ws_mu);
  if (grid_waves) *grid_waves = g_trace_grid * kFusedWaves;
  g_trace = static_cast<int64_t*>(buffer);
  g_trace_words = words;
  return 0;
}

int uocr_moe_fused_errors(void* stream, uint32_t* errors, char* err, size_t errlen) {
  const hipStream_t s = (hipStream_t)stream;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  // the stream's slot and the device's static scratch (each: control words, then the tagged arena)
  std::vector<std::pair<uint32_t*, int64_t>> areas;
  if (e == hipSuccess) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    auto it = g_fused.find(dev);
    if (it != g_fused.end()) {
      auto sl = it->second.slot.find(s);
      if (sl != it->second.slot.end()) areas.emplace_back(sl->second.ctl, (int64_t)(fused_slot_bytes() / 4));
    }
    auto sc = g_scratch.find(dev);
    if (sc != g_scratch.end()) areas.emplace_back(reinterpret_cast<uint32_t*>(sc->second), (int64_t)(kScratchFusedBytes / 4));
  }
  uint32_t v[2] = {0u, 0u};
  for (size_t i = 0; e == hipSuccess && i < areas.size(); ++i)
    e = hipMemcpyAsync(&v[i], areas[i].first + C_ERR_WORD, sizeof(uint32_t), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  // A failed launch leaves the error word set, and every later launch on the
  // slot writes NaN until it is cleared.  Only that word is cleared: the
  // failed launch still counted its arrivals and advanced the epoch, so the
  // tags it wrote (in the slot's arena and in the stream's stacked-launch
  // arena) are older than any later launch's, and no wait can take them.
  bool cleared = false;
  for (size_t i = 0; e == hipSuccess && i < areas.size(); ++i) {
    if (v[i] != 0u) {
      e = launch_zero_words(areas[i].first + C_ERR_WORD, 1, s);
      cleared = true;
    }
  }
  if (e == hipSuccess && cleared) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(err, errlen, "uocr_moe_fused_errors", e);
  if (errors) *errors = (v[0] | v[1]) != 0u ? 1u : 0u;
  return 0;
}

int uocr_moe_fused_status(uint32_t* flag, void* stream, char* err, size_t errlen) {
  const char* op = "uocr_moe_fused_status";
  if (flag == nullptr) return fail(err, errlen, "%s: no flag", op);
  const hipStream_t s = (hipStream_t)stream;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(err, errlen, op, e);
  const uint32_t* slot = nullptr;
  const uint32_t* fixed = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    auto it = g_fused.find(dev);
    if (it != g_fused.end()) {
      auto sl = it->second.slot.find(s);
      if (sl != it->second.slot.end()) slot = sl->second.ctl;
    }
    auto sc = g_scratch.find(dev);
    if (sc != g_scratch.end()) fixed = reinterpret_cast<const uint32_t*>(sc->second);
  }
  e = launch_error_status(flag, slot, fixed, s);
  return e == hipSuccess ? 0 : hip_fail(err, errlen, op, e);
}

void uocr_moe_release(void) {
  std::lock_guard<std::mutex> lock(g_ws_mu);
  for (auto& kv : g_ws)
    if (kv.second.ptr != nullptr) (void)hipFree(kv.second.ptr);
  g_ws.clear();
  for (void* p : g_retired) (void)hipFree(p);
  g_retired.clear();
  for (auto& kv : g_fused) {
    for (void* p : kv.second.chunks) (void)hipFree(p);
    if (kv.second.handoff != nullptr) (void)hipEventDestroy(kv.second.handoff);
  }
  g_fused.clear();
  g_fused_grid.clear();
  for (auto& kv : g_attn_counters)
    if (kv.second.words != nullptr) (void)hipFree(kv.second.words);
  g_attn_counters.clear();
}

}  // extern "C"
