// The no-repeat-n-gram logit guard (unlimited_ocr_max/kernels/ngram_block.mojo:1-151).
//
// Row b of the result is row b of the logits with every banned id set to
// BLOCKED, a finite stand-in for -inf.  With n the n-gram size (device data)
// and h row b's history (its last window ids, the newest last), id v is
// banned when some start s in [0, len(h) - n] has h[s + n - 1] == v and
// h[s .. s + n - 2] == h[len(h) - n + 1 .. len(h) - 1]; n == 1 bans every id
// of the history; n < 1, or a history shorter than n, bans nothing.
//
// The reference checks every start for every vocabulary entry.  Here the
// banned ids come first: a workgroup stages its row's history in LDS, its
// threads test one start each against the prefix, and every match sets the
// bit of its id in an LDS bitmap of the workgroup's vocabulary chunk.  The
// chunk is then copied with the banned entries replaced, one writer per
// element (the result may alias the logits).  The copy is the whole cost:
// HBM-bound, 8 bytes per vocabulary entry and row.
#include "uocr_device.h"
#include "uocr_kernels.h"

namespace uocr {

namespace {

constexpr float kBlocked = -3.0e38f;  // ngram_block.mojo:49
constexpr int kThreads = 256;
constexpr int kPer = 4;                             // float4 per thread
constexpr int kVocabChunk = kThreads * 4 * kPer;    // vocabulary entries per workgroup

__global__ void __launch_bounds__(kThreads) k_ngram_block(float* result, const float* logits, int64_t vocab,
                                                          const int32_t* __restrict__ history, int hist_len,
                                                          const int32_t* __restrict__ ngram, int vec) {
  extern __shared__ int32_t hist[];  // [hist_len], then the chunk's bitmap
  uint32_t* bits = (uint32_t*)(hist + hist_len);
  const int row = (int)blockIdx.y;
  const int64_t c0 = (int64_t)blockIdx.x * kVocabChunk;
  const int tid = (int)threadIdx.x;
  const int n = ldg(ngram);
  const int32_t* h = history + (int64_t)row * hist_len;
  for (int i = tid; i < hist_len; i += kThreads) hist[i] = ldg(h + i);
  for (int i = tid; i < kVocabChunk / 32; i += kThreads) bits[i] = 0u;
  __syncthreads();
  if (n >= 1 && hist_len >= n) {
    const int starts = hist_len - n + 1;
    const int prefix = hist_len - n + 1;  // first id of the last n - 1
    for (int s = tid; s < starts; s += kThreads) {
      bool match = true;
      for (int j = 0; j < n - 1 && match; ++j) match = hist[s + j] == hist[prefix + j];
      const int64_t v = (int64_t)hist[s + n - 1] - c0;
      if (match && v >= 0 && v < kVocabChunk) atomicOr(&bits[v >> 5], 1u << (v & 31));
    }
  }
  __syncthreads();
  const float* src = logits + (int64_t)row * vocab + c0;
  float* dst = result + (int64_t)row * vocab + c0;
  const int64_t len = vocab - c0 < kVocabChunk ? vocab - c0 : kVocabChunk;
  if (vec) {
    // every load of the thread first, then the stores (one memory latency per chunk)
    f32x4 v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = 4 * (tid + u * kThreads);
      if (i < len) v[u] = *(const UOCR_GLOBAL f32x4*)(src + i);
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = 4 * (tid + u * kThreads);
      if (i < len) {
        const uint32_t b = bits[i >> 5] >> (i & 31);  // 4 bits: i is a multiple of 4
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if ((b >> c) & 1u) v[u][c] = kBlocked;
        *(UOCR_GLOBAL f32x4*)(dst + i) = v[u];
      }
    }
  } else {
    for (int64_t i = tid; i < len; i += kThreads) {
      const float v = src[i];
      dst[i] = ((bits[i >> 5] >> (i & 31)) & 1u) ? kBlocked : v;
    }
  }
}

}  // namespace

static size_t ngram_lds_bytes(int hist_len) { return (size_t)hist_len * 4 + kVocabChunk / 8; }

hipError_t launch_ngram_block(float* result, const float* logits, int64_t rows, int64_t vocab,
                              const int32_t* history, int hist_len, const int32_t* ngram, hipStream_t s) {
  if (rows == 0 || vocab == 0) return hipSuccess;
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  const int vec = vocab % 4 == 0 && a16(result) && a16(logits);
  const dim3 grid((unsigned)((vocab + kVocabChunk - 1) / kVocabChunk), (unsigned)rows);
  UOCR_LAUNCH("ngram_block", k_ngram_block, grid, dim3(kThreads), ngram_lds_bytes(hist_len), s, result, logits, vocab,
              history, hist_len, ngram, vec);
  return hipGetLastError();
}

}  // namespace uocr
