// Paged decode attention over the KV page pool (unlimited_ocr_max/decoder.py:425-437,
// paged_decode_attention; the pool layout and row mapping of unlimited_ocr_max/kv_cache.py:1-36).
//
// Row b of a decode step has one query per head, post-RoPE q[b, h, :], and a
// new key/value row (k_new, v_new) that belongs at its write index.  It attends
// its logical rows [0, attend_len[b]), the new row included (the metadata holds
// attend_lengths = attend_len - 1, the reference's cache lengths), where logical row
// r lives in slot r % P of page lookup[b][r / P] of the pool
//   kv_blocks [pages][2 (k, v)][layers][P][heads][D]   fp32.
// out[b, h, :] = sum_r softmax_r(scale * q.k_r) v_r, fp32 throughout (the
// scale multiplies the dot product, as the reference does).
//
// k_attn_partial: workgroup (split s, head h, row b) takes kAttnSplitRows
// consecutive logical rows (one page holds them all) and issues every k and v
// load of them before any arithmetic, so a workgroup waits on memory once:
// 8 lanes per k row (a wave scores 8 rows per load instruction, 128 contiguous
// bytes a row), 32 lanes per v row (a float4 each).  It keeps (max, sum of exp,
// weighted value sum) of its rows.  The row at the write index is read from
// k_new / v_new, and split 0 also stores it into the pool (nothing else in the
// launch reads that pool row).  The splits of a (b, h) are merged by the usual
// rescaling: by the last of them to finish when the caller gives per-(b, h)
// counters, else by a second launch, k_attn_combine; a lone split writes the
// output itself.
// HBM-bound: 2 * attend_len * D * 4 bytes per (row, head).
#include "uocr_device.h"
#include "uocr_kernels.h"

namespace uocr {

namespace {

constexpr int kD = 128;          // head dim
// 8 waves: half a split's loads per thread (100 VGPRs, 4 waves a SIMD) ran
// faster than 4 waves holding all of them (170 VGPRs)
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kLanesPerRow = 8;  // 16 floats of q.k per lane: float4 sub, sub + 8, sub + 16, sub + 24
constexpr int kRowsPerPass = kThreads / kLanesPerRow;  // 64 rows scored at once by the workgroup
constexpr int kPart = kD + 4;  // floats per partial: the value sum, max, sum of exp, 2 pad (16-byte records)
constexpr int kValueGroups = kThreads / (kD / 4);      // 16 value rows at once, a float4 column per lane
constexpr int kKRows = kAttnSplitRows / kRowsPerPass;   // k rows per lane group
constexpr int kVRows = kAttnSplitRows / kValueGroups;   // v rows per lane

struct PagedArgs {
  float* pool;
  int64_t page_stride;   // floats per page: 2 * layers * P * heads * D
  int64_t kv_stride;     // floats between the k and v halves of a page: layers * P * heads * D
  int64_t layer_off;     // floats to the layer: layer * P * heads * D
  int64_t slot_stride;   // floats per slot: heads * D
  int P;
  int heads;
  int pages;     // page ids at or past this are clamped to the last page (the null page)
  int max_rows;  // lookup_cols * P: rows a lookup row can address
  const uint32_t* lookup;
  int lookup_cols;
  const uint32_t* write_index;
  const uint32_t* attend_lengths;  // attend_len - 1 per row
  int64_t in_stride;               // floats between rows of q / k_new / v_new
  const int32_t* positions;        // null: q and k_new come rotated; else RoPE them at these positions
  const float* cos_t;
  const float* sin_t;
  int table_rows;
};

// RoPE of the pair (x[d], x[d + 64]) with cos / sin rows c, s: each product
// and the sum rounded to fp32, no contraction (the bits of k_rope).
__device__ __forceinline__ void rope_pair(float& lo, float& hi, const float* c, const float* s, int d) {
#pragma clang fp contract(off)
  const float l = lo, h = hi;
  lo = l * ldg(c + d) - h * ldg(s + d);
  hi = h * ldg(c + d + kD / 2) + l * ldg(s + d + kD / 2);
}
__device__ __forceinline__ void rope_pair4(f32x4& lo, f32x4& hi, const float* c, const float* s, int d) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float l = lo[e], h = hi[e];
    rope_pair(l, h, c, s, d + e);
    lo[e] = l;
    hi[e] = h;
  }
}
// Element d of the rotated row x.
__device__ __forceinline__ float rope_elem(const float* x, const float* c, const float* s, int d) {
  float lo = ldg(x + (d % (kD / 2))), hi = ldg(x + (d % (kD / 2)) + kD / 2);
  rope_pair(lo, hi, c, s, d % (kD / 2));
  return d < kD / 2 ? lo : hi;
}

// Pointer to the k (kv = 0) or v (kv = 1) values of logical row r of batch row b, head h.
__device__ __forceinline__ float* row_ptr(const PagedArgs& a, int b, int h, int r, int kv) {
  const uint32_t page = min(ldg(a.lookup + (int64_t)b * a.lookup_cols + r / a.P), (uint32_t)(a.pages - 1));
  return a.pool + (int64_t)page * a.page_stride + kv * a.kv_stride + a.layer_off +
         (int64_t)(r % a.P) * a.slot_stride + (int64_t)h * kD;
}

// Row r0 of a split (its rows share one page: the page size is a multiple of
// the split): the k (kv = 0) or v values, rows slot_stride floats apart.
__device__ __forceinline__ const float* split_base(const PagedArgs& a, int b, int h, int r0, int kv) {
  return row_ptr(a, b, h, r0, kv);
}

// Partials cross workgroups (and XCDs, whose L2s are not coherent with one
// another) as agent-scope atomic stores and loads, which go to the memory side
// of the L2s; the counter's atomicInc comes after a wait for those stores.
__device__ __forceinline__ void publish(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float gather(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Column d of one (row, head)'s output from its `splits` partials: each split's
// value sum and sum of exp rescaled to the largest max (empty splits weigh 0).
// The partials are read kMergeChunk splits at a time, every load of a chunk
// issued before the first is used (one memory round trip per chunk).
constexpr int kMergeChunk = 8;
__device__ __forceinline__ float combine_splits(const float* p, int splits, int d) {
  constexpr float kNegInf = -__builtin_huge_valf();
  float m = kNegInf, l = 0.0f, o = 0.0f;
  for (int s0 = 0; s0 < splits; s0 += kMergeChunk) {
    float ms[kMergeChunk], ls[kMergeChunk], os[kMergeChunk];
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j) {
      const float* r = p + (int64_t)min(s0 + j, splits - 1) * kPart;  // past the last: a repeat, unused
      ms[j] = gather(r + kD);
      ls[j] = gather(r + kD + 1);
      os[j] = gather(r + d);
    }
    float mc = m;
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j)
      if (s0 + j < splits) mc = fmaxf(mc, ms[j]);
    const float keep = m == kNegInf ? 0.0f : expf(m - mc);
    l *= keep;
    o *= keep;
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j) {
      if (s0 + j < splits && ms[j] != kNegInf) {
        const float f = expf(ms[j] - mc);
        l = __builtin_fmaf(f, ls[j], l);
        o = __builtin_fmaf(f, os[j], o);
      }
    }
    m = mc;
  }
  return l > 0.0f ? o / l : 0.0f;
}

// The partial of rows [r0, r1) (r0 < r1) of (row b, head h): its value sum,
// max and sum of exp into dst, or, given `direct`, the normalised output there.
__device__ __forceinline__ void split_partial(const PagedArgs& a, const float* __restrict__ q,
                                              const float* __restrict__ k_new, const float* __restrict__ v_new,
                                              float scale, int w_idx, int64_t bh, int b, int h, int r0, int r1,
                                              float* sc, float* red, f32x4 (*vsum)[kD / 4], float* direct,
                                              float* dst) {
  const int tid = (int)threadIdx.x;
  // ---- every load of the split first: k (8 lanes per row, a load instruction covering 128 contiguous
  // bytes of a row) and v (32 lanes per row, a float4 each).  Rows past the attended ones are still in
  // the split's page (the page size is a multiple of the split), so the loads need no guard; their
  // values are masked below.
  const int n = r1 - r0;
  const int sub = tid % kLanesPerRow, rg = tid / kLanesPerRow;
  const int c = tid % (kD / 4), g = tid / (kD / 4);
  const int64_t qoff = (int64_t)b * a.in_stride + (int64_t)h * kD;  // row b, head h of q / k_new / v_new
  const float* qh = q + qoff + sub * 4;
  const float* rc = nullptr;
  const float* rs = nullptr;
  if (a.positions != nullptr) {
    const int pos = min(max(ldg(a.positions + b), 0), a.table_rows - 1);  // device data: clamped into the table
    rc = a.cos_t + (int64_t)pos * kD;
    rs = a.sin_t + (int64_t)pos * kD;
  }
  const float* kbase = split_base(a, b, h, r0, 0);
  const float* vbase = split_base(a, b, h, r0, 1);
  f32x4 qv[4], kv[kKRows][4], vv[kVRows];
#pragma unroll
  for (int u = 0; u < 4; ++u) qv[u] = *(const UOCR_GLOBAL f32x4*)(qh + 32 * u);
  if (rc != nullptr) {  // lane elements d = sub*4 + 32u + e: u = 0, 1 pair with u = 2, 3
    rope_pair4(qv[0], qv[2], rc, rs, sub * 4);
    rope_pair4(qv[1], qv[3], rc, rs, 32 + sub * 4);
  }
#pragma unroll
  for (int j = 0; j < kKRows; ++j) {
    const int i = rg + j * kRowsPerPass;
    const float* kr = (r0 + i == w_idx ? k_new + qoff : kbase + (int64_t)i * a.slot_stride) + sub * 4;
#pragma unroll
    for (int u = 0; u < 4; ++u) kv[j][u] = *(const UOCR_GLOBAL f32x4*)(kr + 32 * u);
    if (rc != nullptr && r0 + i == w_idx) {  // the new row, read unrotated
      rope_pair4(kv[j][0], kv[j][2], rc, rs, sub * 4);
      rope_pair4(kv[j][1], kv[j][3], rc, rs, 32 + sub * 4);
    }
  }
#pragma unroll
  for (int j = 0; j < kVRows; ++j) {
    const int i = g + j * kValueGroups;
    const float* vr = r0 + i == w_idx ? v_new + qoff : vbase + (int64_t)i * a.slot_stride;
    vv[j] = *(const UOCR_GLOBAL f32x4*)(vr + 4 * c);
  }
  // ---- scores
#pragma unroll
  for (int j = 0; j < kKRows; ++j) {
    float p = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      p = __builtin_fmaf(qv[u].x, kv[j][u].x, p);
      p = __builtin_fmaf(qv[u].y, kv[j][u].y, p);
      p = __builtin_fmaf(qv[u].z, kv[j][u].z, p);
      p = __builtin_fmaf(qv[u].w, kv[j][u].w, p);
    }
    // the 8 lanes of a row: a halving tree inside the 8-lane group
    p += __shfl_xor(p, 4, kWave);
    p += __shfl_xor(p, 2, kWave);
    p += __shfl_xor(p, 1, kWave);
    const int i = rg + j * kRowsPerPass;
    if (sub == 0 && i < n) sc[i] = p * scale;
  }
  __syncthreads();
  // ---- max and sum of exp over the split's rows
  float m = -__builtin_huge_valf();
  for (int i = tid; i < n; i += kThreads) m = fmaxf(m, sc[i]);
  m = tree_max(m);
  if (lane_id() == 0) red[tid / 64] = m;
  __syncthreads();
  m = red[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) m = fmaxf(m, red[i]);
  __syncthreads();
  float l = 0.0f;
  for (int i = tid; i < n; i += kThreads) {
    const float e = expf(sc[i] - m);
    sc[i] = e;
    l += e;
  }
  l = tree_sum(l);
  if (lane_id() == 0) red[tid / 64] = l;
  __syncthreads();
  static_assert(kWaves == 8, "the sum below adds 8 wave sums");
  l = ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
  // ---- value sums: thread (g, c): rows i = g mod 8, float4 column c; the 8 groups added at the end
  f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < kVRows; ++j) {
    const int i = g + j * kValueGroups;
    if (i < n) {  // rows past the attended ones may hold anything, inf and nan included
      const float w = sc[i];
      o.x = __builtin_fmaf(w, vv[j].x, o.x);
      o.y = __builtin_fmaf(w, vv[j].y, o.y);
      o.z = __builtin_fmaf(w, vv[j].z, o.z);
      o.w = __builtin_fmaf(w, vv[j].w, o.w);
    }
  }
  if (g > 0) vsum[g - 1][c] = o;
  __syncthreads();
  if (g == 0) {
#pragma unroll
    for (int j = 0; j < kValueGroups - 1; ++j) o += vsum[j][c];
    if (direct != nullptr) {  // the only split: the output itself
      *(UOCR_GLOBAL f32x4*)(direct + 4 * c) = o / l;
    } else {
      publish(dst + 4 * c, o.x);
      publish(dst + 4 * c + 1, o.y);
      publish(dst + 4 * c + 2, o.z);
      publish(dst + 4 * c + 3, o.w);
    }
  }
  if (tid == 0 && direct == nullptr) {
    publish(dst + kD, m);
    publish(dst + kD + 1, l);
  }
}

// `counters` (one per (row, head), zero between calls) lets the last split of
// a (row, head) to finish combine the splits itself: atomicInc with the limit
// splits - 1 returns splits - 1 to exactly one workgroup and leaves the counter
// at 0 again.  Without counters the partials wait for k_attn_combine.  One
// split writes the output directly.
__global__ void __launch_bounds__(kThreads) k_attn_partial(PagedArgs a, const float* __restrict__ q,
                                                           const float* __restrict__ k_new,
                                                           const float* __restrict__ v_new, float scale,
                                                           float* __restrict__ part, int splits,
                                                           uint32_t* __restrict__ counters, float* __restrict__ out) {
  __shared__ float sc[kAttnSplitRows];
  __shared__ float red[kThreads / 64];
  __shared__ f32x4 vsum[kValueGroups - 1][kD / 4];
  __shared__ uint32_t last;
  const int s = (int)blockIdx.x, h = (int)blockIdx.y, b = (int)blockIdx.z;
  const int tid = (int)threadIdx.x;
  // device metadata is clamped to what the lookup row addresses (never out of the pool)
  const int len = (int)min(ldg(a.attend_lengths + b), (uint32_t)(a.max_rows - 1)) + 1;
  const uint32_t w_raw = ldg(a.write_index + b);
  const int w_idx = w_raw < (uint32_t)a.max_rows ? (int)w_raw : -1;
  const int r0 = s * kAttnSplitRows;
  const int r1 = min(len, r0 + kAttnSplitRows);
  const int64_t bh = (int64_t)b * a.heads + h;
  float* dst = part + (bh * splits + s) * kPart;
  if (s == 0 && w_idx >= 0) {
    // the new row into the pool (its readers in this launch take it from k_new / v_new)
    const int64_t qoff = (int64_t)b * a.in_stride + (int64_t)h * kD;
    for (int i = tid; i < 2 * kD; i += kThreads) {
      const int kv = i / kD, d = i % kD;
      float v;
      if (kv == 0 && a.positions != nullptr) {
        const int pos = min(max(ldg(a.positions + b), 0), a.table_rows - 1);
        v = rope_elem(k_new + qoff, a.cos_t + (int64_t)pos * kD, a.sin_t + (int64_t)pos * kD, d);
      } else {
        v = ldg((kv ? v_new : k_new) + qoff + d);
      }
      row_ptr(a, b, h, w_idx, kv)[d] = v;
    }
  }
  if (r0 >= r1) {  // nothing to attend in this split: an empty partial
    if (tid == 0) {
      publish(dst + kD, -__builtin_huge_valf());
      publish(dst + kD + 1, 0.0f);
    }
    for (int d = tid; d < kD; d += kThreads) publish(dst + d, 0.0f);
  } else {
    split_partial(a, q, k_new, v_new, scale, w_idx, bh, b, h, r0, r1, sc, red, vsum,
                  splits == 1 ? out + bh * kD : nullptr, dst);
  }
  if (splits == 1 || counters == nullptr) return;
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores done before the count
  __syncthreads();
  if (tid == 0) last = atomicInc(counters + bh, (uint32_t)(splits - 1)) == (uint32_t)(splits - 1);
  __syncthreads();
  if (!last) return;
  if (tid < kD) out[bh * kD + tid] = combine_splits(part + bh * splits * kPart, splits, tid);
}

__global__ void __launch_bounds__(kD) k_attn_combine(const float* __restrict__ part, int splits, int heads,
                                                     float* __restrict__ out) {
  const int64_t bh = (int64_t)blockIdx.y * heads + blockIdx.x;
  out[bh * kD + threadIdx.x] = combine_splits(part + bh * splits * kPart, splits, (int)threadIdx.x);
}

}  // namespace

size_t attn_workspace_bytes(int64_t rows, int heads, int max_attend) {
  const int splits = (max_attend + kAttnSplitRows - 1) / kAttnSplitRows;
  return (size_t)rows * heads * (splits > 0 ? splits : 1) * kPart * sizeof(float);
}

hipError_t launch_paged_attention(const PagedAttention& p, hipStream_t s) {
  if (p.rows == 0) return hipSuccess;
  if (p.head_dim != kD || p.page_size % kAttnSplitRows != 0 || p.pages < 1) return hipErrorInvalidValue;
  PagedArgs a{};
  a.pool = p.kv_blocks;
  a.slot_stride = (int64_t)p.heads * kD;
  a.layer_off = (int64_t)p.layer * p.page_size * a.slot_stride;
  a.kv_stride = (int64_t)p.layers * p.page_size * a.slot_stride;
  a.page_stride = 2 * a.kv_stride;
  a.P = p.page_size;
  a.heads = p.heads;
  a.pages = p.pages;
  a.max_rows = p.lookup_cols * p.page_size;
  a.lookup = p.lookup;
  a.lookup_cols = p.lookup_cols;
  a.write_index = p.write_index;
  a.attend_lengths = p.attend_lengths;
  a.in_stride = p.in_stride > 0 ? p.in_stride : (int64_t)p.heads * kD;
  a.positions = p.positions;
  a.cos_t = p.cos_table;
  a.sin_t = p.sin_table;
  a.table_rows = p.table_rows;
  const int splits = (p.max_attend + kAttnSplitRows - 1) / kAttnSplitRows;
  const dim3 grid((unsigned)(splits > 0 ? splits : 1), (unsigned)p.heads, (unsigned)p.rows);
  UOCR_LAUNCH("attn_partial", k_attn_partial, grid, dim3(kThreads), 0, s, a, p.q, p.k_new, p.v_new, p.scale,
              p.workspace, (int)grid.x, p.counters, p.out);
  if (grid.x > 1 && p.counters == nullptr)
    UOCR_LAUNCH("attn_combine", k_attn_combine, dim3((unsigned)p.heads, (unsigned)p.rows), dim3(kD), 0, s,
                p.workspace, (int)grid.x, p.heads, p.out);
  return hipGetLastError();
}

}  // namespace uocr
