/*
 * CPU oracle for the DeepSeek-V2 routed-expert MoE block of unlimited-ocr-max.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP library and the timed CPU
 * baseline.  The header (oracle.h) lists what pins each function.
 *
 * Built with -ffp-contract=off: every fused multiply-add below is an explicit
 * fmaf(), every other product and sum is rounded on its own, as the function
 * comments state.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ======================================================================= */
/* scalar helpers                                                           */
/* ======================================================================= */

static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* unlimited_ocr_max/bf16.py:122-136: bias 0x7FFF plus the kept lsb, NaN to
 * the canonical quiet NaN. */
uint16_t or_bf16_rne(float f) {
  if (f != f) return 0x7FC0;
  uint32_t u = f2u(f);
  uint32_t bias = 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)((u + bias) >> 16);
}

float or_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* 2^n for n in [-126, 127] built from its exponent field. */
static inline float pow2i(int n) { return u2f((uint32_t)(n + 127) << 23); }

float or_uexp(float x) {
  if (x != x) return x;
  if (x > 88.72283f) return INFINITY;
  if (x < -103.972f) return 0.0f;
  const float log2e = 1.44269502f;           /* fp32(1/ln 2) */
  const float ln2_hi = 0.693145751953125f;   /* 16 significant bits */
  const float ln2_lo = 1.42860677e-06f;      /* fp32(ln 2 - ln2_hi) */
  float t = x * log2e;
  float n = rintf(t);
  float r = fmaf(-n, ln2_hi, x);
  r = fmaf(-n, ln2_lo, r);
  /* e^r = sum r^i / i!, i = 0..7, Horner. */
  float p = 1.98412701e-04f;                 /* 1/5040 */
  p = fmaf(p, r, 1.38888892e-03f);           /* 1/720 */
  p = fmaf(p, r, 8.33333377e-03f);           /* 1/120 */
  p = fmaf(p, r, 4.16666679e-02f);           /* 1/24 */
  p = fmaf(p, r, 1.66666672e-01f);           /* 1/6 */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ni = (int)n;
  int n1 = ni / 2;
  int n2 = ni - n1;
  return (p * pow2i(n1)) * pow2i(n2);
}

float or_silu(float g) {
  float e = or_uexp(-g);
  float d = 1.0f + e;
  return g / d;
}

void or_uexp_array(float* out, const float* x, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = or_uexp(x[i]);
}

void or_silu_array(float* out, const float* x, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = or_silu(x[i]);
}

/* ======================================================================= */
/* a persistent thread pool with dynamic chunking                          */
/* ======================================================================= */

typedef void (*task_fn)(void* ctx, int64_t begin, int64_t end);

#define MAX_WORKERS 256

static struct {
  pthread_mutex_t mu;
  pthread_cond_t go;
  pthread_cond_t done;
  int nworkers;
  uint64_t generation;
  /* the current job */
  task_fn fn;
  void* ctx;
  int64_t n, chunk;
  int active; /* workers taking part in the current job */
  atomic_llong next;
  int finished;
} pool = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER,
          PTHREAD_COND_INITIALIZER};

static void run_chunks(void) {
  for (;;) {
    int64_t b = atomic_fetch_add(&pool.next, pool.chunk);
    if (b >= pool.n) break;
    int64_t e = b + pool.chunk < pool.n ? b + pool.chunk : pool.n;
    pool.fn(pool.ctx, b, e);
  }
}

static void* worker(void* arg) {
  int id = (int)(intptr_t)arg;
  uint64_t seen = 0;
  pthread_mutex_lock(&pool.mu);
  for (;;) {
    while (pool.generation == seen) pthread_cond_wait(&pool.go, &pool.mu);
    seen = pool.generation;
    int take = id < pool.active;
    pthread_mutex_unlock(&pool.mu);
    if (take) run_chunks();
    pthread_mutex_lock(&pool.mu);
    if (take && ++pool.finished == pool.active) pthread_cond_signal(&pool.done);
  }
  return NULL;
}

static int online_cores(void) {
  long c = sysconf(_SC_NPROCESSORS_ONLN);
  return c < 1 ? 1 : (int)c;
}

int or_threads(int threads) {
  int t = threads <= 0 ? online_cores() : threads;
  if (t > MAX_WORKERS + 1) t = MAX_WORKERS + 1;
  return t;
}

static void parallel_for(int64_t n, int threads, task_fn fn, void* ctx) {
  int t = or_threads(threads);
  if (n <= 0) return;
  if (t <= 1 || n == 1) {
    fn(ctx, 0, n);
    return;
  }
  pthread_mutex_lock(&pool.mu);
  while (pool.nworkers < t - 1) {
    pthread_t th;
    if (pthread_create(&th, NULL, worker, (void*)(intptr_t)pool.nworkers) != 0)
      break;
    pthread_detach(th);
    pool.nworkers++;
  }
  pool.fn = fn;
  pool.ctx = ctx;
  pool.n = n;
  int64_t chunk = n / ((int64_t)t * 8);
  pool.chunk = chunk < 1 ? 1 : chunk;
  pool.active = t - 1 < pool.nworkers ? t - 1 : pool.nworkers;
  atomic_store(&pool.next, 0);
  pool.finished = 0;
  pool.generation++;
  pthread_cond_broadcast(&pool.go);
  pthread_mutex_unlock(&pool.mu);
  run_chunks();
  pthread_mutex_lock(&pool.mu);
  while (pool.finished < pool.active) pthread_cond_wait(&pool.done, &pool.mu);
  pthread_mutex_unlock(&pool.mu);
}

/* ======================================================================= */
/* quantiser: tools/quantize_int8.py:54-70, 298-329                         */
/* ======================================================================= */

int or_quantize_per_group(const float* w, int64_t n, int64_t k, int64_t group,
                          int8_t* q, float* scales) {
  if (group <= 0 || k % group) return -1;
  int64_t groups = k / group;
  for (int64_t row = 0; row < n; ++row) {
    for (int64_t g = 0; g < groups; ++g) {
      const float* chunk = w + row * k + g * group;
      float amax = 0.0f;
      for (int64_t i = 0; i < group; ++i) {
        float a = fabsf(chunk[i]);
        if (a > amax) amax = a;
      }
      float s = amax == 0.0f ? 1.0f : amax / 127.0f;
      scales[row * groups + g] = s;
      for (int64_t i = 0; i < group; ++i) {
        float v = rintf(chunk[i] / s);
        if (v > 127.0f) v = 127.0f;
        if (v < -127.0f) v = -127.0f;
        q[row * k + g * group + i] = (int8_t)v;
      }
    }
  }
  return 0;
}

/* ======================================================================= */
/* row grouping: unlimited_ocr_max/kernels/moe_routing.mojo:26-92          */
/* ======================================================================= */

#define FOLLOWS (-1)
#define TILE 4

static inline int64_t clamp_expert(int32_t key, int64_t E) {
  int64_t e = key;
  if (e < 0) e = 0;
  if (e >= E) e = E - 1;
  return e;
}

/* moe_routing.mojo:48-66 */
static int64_t group_tail(const int32_t* ids, int64_t row, int64_t total) {
  int32_t mine = ids[row];
  int64_t later = 0;
  for (int64_t j = 0; j < total; ++j) {
    if (ids[j] == mine) {
      if (j < row) return FOLLOWS;
      if (j > row) later++;
    }
  }
  return later;
}

/* moe_routing.mojo:69-92 */
static int next_tile(const int32_t* ids, int32_t key, int64_t total,
                     int64_t* cursor, int64_t rows[TILE]) {
  int count = 0;
  for (int r = 0; r < TILE; ++r) {
    while (*cursor < total && ids[*cursor] != key) (*cursor)++;
    if (*cursor < total) {
      rows[r] = *cursor;
      count = r + 1;
      (*cursor)++;
    }
  }
  return count;
}

/* ======================================================================= */
/* moe_int8_qmv: unlimited_ocr_max/kernels/moe_int8.mojo:101-148,181-258  */
/* ======================================================================= */

typedef struct {
  float* out;
  const float* x;
  const int32_t* ids;
  const int8_t* w;
  const float* scales;
  int64_t k, E, N, K, groups, gsize;
} int8_qmv_args;

/* _dot_rows_by: per group a scalar fma chain in kk order per row, then
 * acc = fma(scale, gsum, acc) per group (moe_int8.mojo:126-148). */
static void int8_dot_rows(const int8_qmv_args* a, int64_t e, int64_t n,
                          const int64_t* rows, int count) {
  float acc[TILE] = {0, 0, 0, 0};
  const int8_t* wrow = a->w + (e * a->N + n) * a->K;
  const float* srow = a->scales + (e * a->N + n) * a->groups;
  for (int64_t g = 0; g < a->groups; ++g) {
    float gsum[TILE] = {0, 0, 0, 0};
    int64_t base = g * a->gsize;
    for (int64_t kk = base; kk < base + a->gsize; ++kk) {
      float wv = (float)wrow[kk];
      for (int r = 0; r < count; ++r)
        gsum[r] = fmaf(wv, a->x[rows[r] * a->K + kk], gsum[r]);
    }
    float scale = srow[g];
    for (int r = 0; r < count; ++r) acc[r] = fmaf(scale, gsum[r], acc[r]);
  }
  for (int r = 0; r < count; ++r) a->out[rows[r] * a->N + n] = acc[r];
}

/* the elementwise work item (moe_int8.mojo:218-256) */
static void int8_qmv_items(void* ctx, int64_t begin, int64_t end) {
  const int8_qmv_args* a = (const int8_qmv_args*)ctx;
  for (int64_t i = begin; i < end; ++i) {
    int64_t s = i / a->N;
    int64_t n = i - s * a->N;
    int64_t later = group_tail(a->ids, s, a->k);
    if (later == FOLLOWS) continue;
    int32_t key = a->ids[s];
    int64_t e = clamp_expert(key, a->E);
    int64_t rows[TILE];
    if (later == 0) {
      rows[0] = s;
      int8_dot_rows(a, e, n, rows, 1);
      continue;
    }
    int64_t cursor = s;
    while (cursor < a->k) {
      int count = next_tile(a->ids, key, a->k, &cursor, rows);
      if (count > 0) int8_dot_rows(a, e, n, rows, count);
    }
  }
}

int or_moe_int8_qmv(float* out, const float* x, const int32_t* ids,
                    const int8_t* w, const float* scales, int64_t k,
                    int64_t E, int64_t N, int64_t K, int64_t groups,
                    int threads) {
  if (E < 1) return -1;
  if (groups < 1 || K % groups) return -2;
  int8_qmv_args a = {out, x, ids, w, scales, k, E, N, K, groups, K / groups};
  parallel_for(k * N, threads, int8_qmv_items, &a);
  return 0;
}

/* ======================================================================= */
/* moe_bf16_qmv                                                             */
/* ======================================================================= */

typedef struct {
  float* out;
  const float* x;
  const int32_t* ids;
  const uint16_t* w;
  int64_t k, E, N, K;
} bf16_qmv_args;

/* Mojo's SIMD reduce_add: halve, add lane-wise, repeat. */
static float tree_reduce(float* v, int width) {
  for (int h = width / 2; h >= 1; h /= 2)
    for (int l = 0; l < h; ++l) v[l] = v[l] + v[l + h];
  return v[0];
}

/* moe_bf16.mojo:119-148: VEC lane partials (width 16) or one scalar sum. */
static void bf16_dot_rows_ref(const bf16_qmv_args* a, int64_t e, int64_t n,
                              const int64_t* rows, int count) {
  const uint16_t* wrow = a->w + (e * a->N + n) * a->K;
  int width = (a->K % 16 == 0) ? 16 : 1;
  for (int r = 0; r < count; ++r) {
    float acc[16] = {0};
    const float* xr = a->x + rows[r] * a->K;
    for (int64_t kk = 0; kk < a->K; kk += width)
      for (int l = 0; l < width; ++l) {
        float prod = or_bf16_to_f32(wrow[kk + l]) * xr[kk + l];
        acc[l] = acc[l] + prod;
      }
    a->out[rows[r] * a->N + n] = tree_reduce(acc, width);
  }
}

/* moe_bf16.mojo:310-343 */
static void bf16_qmv_items_ref(void* ctx, int64_t begin, int64_t end) {
  const bf16_qmv_args* a = (const bf16_qmv_args*)ctx;
  for (int64_t i = begin; i < end; ++i) {
    int64_t s = i / a->N;
    int64_t n = i - s * a->N;
    int64_t later = group_tail(a->ids, s, a->k);
    if (later == FOLLOWS) continue;
    int32_t key = a->ids[s];
    int64_t e = clamp_expert(key, a->E);
    int64_t rows[TILE];
    if (later == 0) {
      rows[0] = s;
      bf16_dot_rows_ref(a, e, n, rows, 1);
      continue;
    }
    int64_t cursor = s;
    while (cursor < a->k) {
      int count = next_tile(a->ids, key, a->k, &cursor, rows);
      if (count > 0) bf16_dot_rows_ref(a, e, n, rows, count);
    }
  }
}

int or_moe_bf16_qmv_ref(float* out, const float* x, const int32_t* ids,
                        const uint16_t* w, int64_t k, int64_t E, int64_t N,
                        int64_t K, int threads) {
  if (E < 1) return -1;
  bf16_qmv_args a = {out, x, ids, w, k, E, N, K};
  parallel_for(k * N, threads, bf16_qmv_items_ref, &a);
  return 0;
}

#define CHUNK 128

/* The chunked chain of one contiguous bf16 weight row: K cut into chunks of
 * 128, each an fma chain in k order from 0, the chunk sums added in order. */
static float chunked_dot_rows(const uint16_t* wrow, const float* x, int64_t K) {
  float acc = 0.0f;
  for (int64_t c0 = 0; c0 < K; c0 += CHUNK) {
    int64_t c1 = c0 + CHUNK < K ? c0 + CHUNK : K;
    float cs = 0.0f;
    for (int64_t kk = c0; kk < c1; ++kk)
      cs = fmaf(or_bf16_to_f32(wrow[kk]), x[kk], cs);
    acc = acc + cs;
  }
  return acc;
}

static void bf16_qmv_items_chunked(void* ctx, int64_t begin, int64_t end) {
  const bf16_qmv_args* a = (const bf16_qmv_args*)ctx;
  for (int64_t i = begin; i < end; ++i) {
    int64_t s = i / a->N;
    int64_t n = i - s * a->N;
    int64_t e = clamp_expert(a->ids[s], a->E);
    a->out[i] = chunked_dot_rows(a->w + (e * a->N + n) * a->K, a->x + s * a->K,
                                 a->K);
  }
}

int or_moe_bf16_qmv_chunked(float* out, const float* x, const int32_t* ids,
                            const uint16_t* w, int64_t k, int64_t E,
                            int64_t N, int64_t K, int threads) {
  if (E < 1) return -1;
  bf16_qmv_args a = {out, x, ids, w, k, E, N, K};
  parallel_for(k * N, threads, bf16_qmv_items_chunked, &a);
  return 0;
}

/* ======================================================================= */
/* dense_bf16_qmv: unlimited_ocr_max/kernels/dense_bf16.mojo:85-158        */
/* ======================================================================= */

typedef struct {
  float* out;
  const float* x;
  const uint16_t* w; /* [K/16][N][16] */
  int64_t M, N, K, tile, tiles;
} dense_args;

/* dense_bf16.mojo:86-116: tile rows per read; padded rows read row M-1. */
static void dense_items_ref(void* ctx, int64_t begin, int64_t end) {
  const dense_args* a = (const dense_args*)ctx;
  int64_t blocks = a->K / 16;
  float acc[8][4];
  for (int64_t i = begin; i < end; ++i) {
    int64_t n = i / a->tiles;
    int64_t row0 = (i - n * a->tiles) * a->tile;
    for (int64_t r = 0; r < a->tile && r < 8; ++r)
      acc[r][0] = acc[r][1] = acc[r][2] = acc[r][3] = 0.0f;
    for (int64_t kb = 0; kb < blocks; ++kb) {
      const uint16_t* wb = a->w + (kb * a->N + n) * 16;
      float wv[16];
      for (int l = 0; l < 16; ++l) wv[l] = or_bf16_to_f32(wb[l]);
      for (int64_t r = 0; r < a->tile; ++r) {
        int64_t row = row0 + r < a->M ? row0 + r : a->M - 1;
        const float* xv = a->x + row * a->K + kb * 16;
        float p[16];
        for (int l = 0; l < 16; ++l) p[l] = wv[l] * xv[l];
        for (int l = 0; l < 8; ++l) p[l] = p[l] + p[l + 8];
        for (int l = 0; l < 4; ++l) p[l] = p[l] + p[l + 4];
        for (int l = 0; l < 4; ++l) acc[r][l] = acc[r][l] + p[l];
      }
    }
    for (int64_t r = 0; r < a->tile; ++r) {
      if (row0 + r < a->M) {
        float v[4] = {acc[r][0], acc[r][1], acc[r][2], acc[r][3]};
        a->out[(row0 + r) * a->N + n] = tree_reduce(v, 4);
      }
    }
  }
}

int or_dense_bf16_qmv_ref(float* out, const float* x, const uint16_t* w_kb,
                          int64_t M, int64_t N, int64_t K, int64_t tile,
                          int threads) {
  if (tile < 1 || tile > 8) return -1;
  if (K % 16) return -2;
  int64_t tiles = (M + tile - 1) / tile;
  dense_args a = {out, x, w_kb, M, N, K, tile, tiles};
  parallel_for(tiles * N, threads, dense_items_ref, &a);
  return 0;
}

static float chunked_dot_kblocked(const uint16_t* w_kb, int64_t N, int64_t n,
                                  const float* x, int64_t K) {
  float acc = 0.0f;
  for (int64_t c0 = 0; c0 < K; c0 += CHUNK) {
    int64_t c1 = c0 + CHUNK < K ? c0 + CHUNK : K;
    float cs = 0.0f;
    for (int64_t kk = c0; kk < c1; ++kk) {
      uint16_t b = w_kb[((kk / 16) * N + n) * 16 + (kk % 16)];
      cs = fmaf(or_bf16_to_f32(b), x[kk], cs);
    }
    acc = acc + cs;
  }
  return acc;
}

static void dense_items_chunked(void* ctx, int64_t begin, int64_t end) {
  const dense_args* a = (const dense_args*)ctx;
  for (int64_t i = begin; i < end; ++i) {
    int64_t m = i / a->N;
    int64_t n = i - m * a->N;
    a->out[i] = chunked_dot_kblocked(a->w, a->N, n, a->x + m * a->K, a->K);
  }
}

int or_dense_bf16_qmv_chunked(float* out, const float* x, const uint16_t* w_kb,
                              int64_t M, int64_t N, int64_t K, int threads) {
  if (K % 16) return -2;
  dense_args a = {out, x, w_kb, M, N, K, 1, M};
  parallel_for(M * N, threads, dense_items_chunked, &a);
  return 0;
}

/* ======================================================================= */
/* int8_dequant_expert: unlimited_ocr_max/kernels/moe_int8.mojo:303-342    */
/* ======================================================================= */

int or_int8_dequant_expert(uint16_t* out, const int8_t* w, const float* scales,
                           int32_t idx, int64_t E, int64_t N, int64_t K,
                           int64_t groups) {
  if (E < 1) return -1;
  if (groups < 1 || K % groups) return -2;
  int64_t gsize = K / groups;
  int64_t e = clamp_expert(idx, E);
  for (int64_t n = 0; n < N; ++n)
    for (int64_t kk = 0; kk < K; ++kk) {
      float v = (float)w[(e * N + n) * K + kk] *
                scales[(e * N + n) * groups + kk / gsize];
      out[n * K + kk] = or_bf16_rne(v);
    }
  return 0;
}

/* ======================================================================= */
/* gate: unlimited_ocr_max/decoder.py:500-514                               */
/* ======================================================================= */

float or_dot_tree64(const float* a, const float* b, int64_t K) {
  float p[64];
  for (int l = 0; l < 64; ++l) {
    float s = 0.0f;
    for (int64_t k = l; k < K; k += 64) s = fmaf(a[k], b[k], s);
    p[l] = s;
  }
  for (int off = 32; off >= 1; off /= 2)
    for (int l = 0; l < off; ++l) p[l] = p[l] + p[l + off];
  return p[0];
}

static void softmax_topk(const float* logits, int64_t E, int64_t topk,
                         int renorm, int32_t* ids, float* weights) {
  float m = logits[0];
  for (int64_t e = 1; e < E; ++e)
    if (logits[e] > m) m = logits[e];
  float ex[64];
  for (int l = 0; l < 64; ++l) ex[l] = l < E ? or_uexp(logits[l] - m) : 0.0f;
  float q[64];
  memcpy(q, ex, sizeof q);
  for (int off = 32; off >= 1; off /= 2)
    for (int l = 0; l < off; ++l) q[l] = q[l] + q[l + off];
  float S = q[0];
  float p[64];
  for (int64_t e = 0; e < E; ++e) p[e] = ex[e] / S;
  uint64_t taken = 0;
  for (int64_t j = 0; j < topk; ++j) {
    int64_t best = -1;
    for (int64_t e = 0; e < E; ++e) {
      if (taken >> e & 1) continue;
      if (best < 0 || p[e] > p[best]) best = e;
    }
    taken |= 1ull << best;
    ids[j] = (int32_t)best;
    weights[j] = p[best];
  }
  if (renorm) {
    float d = 0.0f;
    for (int64_t j = 0; j < topk; ++j) d = d + weights[j];
    for (int64_t j = 0; j < topk; ++j) weights[j] = weights[j] / d;
  }
}

int or_moe_gate(int32_t* ids, float* weights, const float* x, const float* wr,
                int64_t T, int64_t E, int64_t H, int64_t topk, int renorm) {
  if (E < 1 || E > 64) return -1;
  if (topk < 1 || topk > E) return -2;
  float logits[64];
  for (int64_t t = 0; t < T; ++t) {
    for (int64_t e = 0; e < E; ++e)
      logits[e] = or_dot_tree64(x + t * H, wr + e * H, H);
    softmax_topk(logits, E, topk, renorm, ids + t * topk, weights + t * topk);
  }
  return 0;
}

/* ======================================================================= */
/* the decode layer                                                          */
/* ======================================================================= */

/* exact int8 chain of one weight row (the or_moe_int8_qmv arithmetic) */
static float int8_dot_row(const int8_t* wrow, const float* srow,
                          const float* x, int64_t K, int64_t gsize) {
  float acc = 0.0f;
  for (int64_t g = 0; g < K / gsize; ++g) {
    float gs = 0.0f;
    for (int64_t kk = g * gsize; kk < (g + 1) * gsize; ++kk)
      gs = fmaf((float)wrow[kk], x[kk], gs);
    acc = fmaf(srow[g], gs, acc);
  }
  return acc;
}

static float routed_dot(const or_moe_layer* L, const void* w, const float* s,
                        int64_t e, int64_t n, int64_t N, int64_t K,
                        const float* x) {
  if (L->int8) {
    int64_t groups = K / L->group;
    return int8_dot_row((const int8_t*)w + (e * N + n) * K,
                        s + (e * N + n) * groups, x, K, L->group);
  }
  return chunked_dot_rows((const uint16_t*)w + (e * N + n) * K, x, K);
}

typedef struct {
  const or_moe_layer* L;
  const float* x;
  const int32_t* ids;
  float* h;      /* [B*k, F] */
  float* y;      /* [B*k, H] */
  float* hs;     /* [B, Fs] */
  float* sh;     /* [B, H] */
  int64_t B;
} layer_args;

static void items_gateup(void* ctx, int64_t begin, int64_t end) {
  const layer_args* a = (const layer_args*)ctx;
  const or_moe_layer* L = a->L;
  for (int64_t i = begin; i < end; ++i) {
    int64_t r = i / L->F, n = i % L->F;
    int64_t b = r / L->topk;
    int64_t e = a->ids[r];
    const float* xr = a->x + b * L->H;
    float g = routed_dot(L, L->gate_w, L->gate_s, e, n, L->F, L->H, xr);
    float u = routed_dot(L, L->up_w, L->up_s, e, n, L->F, L->H, xr);
    a->h[i] = or_silu(g) * u;
  }
}

static void items_down(void* ctx, int64_t begin, int64_t end) {
  const layer_args* a = (const layer_args*)ctx;
  const or_moe_layer* L = a->L;
  for (int64_t i = begin; i < end; ++i) {
    int64_t r = i / L->H, n = i % L->H;
    int64_t e = a->ids[r];
    a->y[i] = routed_dot(L, L->down_w, L->down_s, e, n, L->H, L->F,
                         a->h + r * L->F);
  }
}

static void items_shared_gateup(void* ctx, int64_t begin, int64_t end) {
  const layer_args* a = (const layer_args*)ctx;
  const or_moe_layer* L = a->L;
  for (int64_t i = begin; i < end; ++i) {
    int64_t b = i / L->Fs, n = i % L->Fs;
    const float* xr = a->x + b * L->H;
    float g = chunked_dot_kblocked(L->sh_gate, L->Fs, n, xr, L->H);
    float u = chunked_dot_kblocked(L->sh_up, L->Fs, n, xr, L->H);
    a->hs[i] = or_silu(g) * u;
  }
}

static void items_shared_down(void* ctx, int64_t begin, int64_t end) {
  const layer_args* a = (const layer_args*)ctx;
  const or_moe_layer* L = a->L;
  for (int64_t i = begin; i < end; ++i) {
    int64_t b = i / L->H, n = i % L->H;
    a->sh[i] = chunked_dot_kblocked(L->sh_down, L->H, n, a->hs + b * L->Fs,
                                    L->Fs);
  }
}

static int check_layer(const or_moe_layer* L) {
  if (L->E < 1 || L->E > 64) return -1;
  if (L->topk < 1 || L->topk > L->E) return -2;
  if (L->H % 16 || L->Fs % 16) return -3;
  if (L->int8 && (L->group < 1 || L->H % L->group || L->F % L->group))
    return -4;
  return 0;
}

int or_moe_decode_exact(float* out, int32_t* ids_out, float* wts_out,
                        const float* x, int64_t B, const or_moe_layer* L,
                        int threads) {
  int rc = check_layer(L);
  if (rc) return rc;
  if (B <= 0) return 0;
  int64_t R = B * L->topk;
  int32_t* ids = malloc(sizeof(int32_t) * R);
  float* wts = malloc(sizeof(float) * R);
  float* h = malloc(sizeof(float) * R * L->F);
  float* y = malloc(sizeof(float) * R * L->H);
  float* hs = malloc(sizeof(float) * B * L->Fs);
  float* sh = malloc(sizeof(float) * B * L->H);
  if (!ids || !wts || !h || !y || !hs || !sh) {
    rc = -10;
    goto done;
  }
  or_moe_gate(ids, wts, x, L->router, B, L->E, L->H, L->topk, L->renorm);
  layer_args a = {L, x, ids, h, y, hs, sh, B};
  parallel_for(R * L->F, threads, items_gateup, &a);
  parallel_for(R * L->H, threads, items_down, &a);
  parallel_for(B * L->Fs, threads, items_shared_gateup, &a);
  parallel_for(B * L->H, threads, items_shared_down, &a);
  for (int64_t b = 0; b < B; ++b)
    for (int64_t n = 0; n < L->H; ++n) {
      float acc = 0.0f;
      for (int64_t j = 0; j < L->topk; ++j)
        acc = fmaf(wts[b * L->topk + j], y[(b * L->topk + j) * L->H + n], acc);
      out[b * L->H + n] = acc + sh[b * L->H + n];
    }
  if (ids_out) memcpy(ids_out, ids, sizeof(int32_t) * R);
  if (wts_out) memcpy(wts_out, wts, sizeof(float) * R);
done:
  free(ids);
  free(wts);
  free(h);
  free(y);
  free(hs);
  free(sh);
  return rc;
}

/* decoder.py:144-163 */
static int64_t rows_per_read(int64_t rows, int64_t out_dim) {
  int64_t tiles = 1;
  for (;;) {
    int64_t tile = (rows + tiles - 1) / tiles;
    if (tile == 1 || out_dim * ((rows + tile - 1) / tile) >= 2048) return tile;
    tiles++;
  }
}

typedef struct {
  float* h;
  const float* g;
  const float* u;
} swiglu_args;

static void items_swiglu(void* ctx, int64_t begin, int64_t end) {
  const swiglu_args* a = (const swiglu_args*)ctx;
  for (int64_t i = begin; i < end; ++i) a->h[i] = or_silu(a->g[i]) * a->u[i];
}

int or_moe_decode_refdecomp(float* out, const float* x, int64_t B,
                            const or_moe_layer* L, int threads) {
  int rc = check_layer(L);
  if (rc) return rc;
  if (B <= 0) return 0;
  int64_t R = B * L->topk;
  int32_t* ids = malloc(sizeof(int32_t) * R);
  float* wts = malloc(sizeof(float) * R);
  float* xr = malloc(sizeof(float) * R * L->H);
  float* g = malloc(sizeof(float) * R * L->F);
  float* u = malloc(sizeof(float) * R * L->F);
  float* y = malloc(sizeof(float) * R * L->H);
  float* sg = malloc(sizeof(float) * B * L->Fs);
  float* su = malloc(sizeof(float) * B * L->Fs);
  float* sh = malloc(sizeof(float) * B * L->H);
  if (!ids || !wts || !xr || !g || !u || !y || !sg || !su || !sh) {
    rc = -10;
    goto done;
  }
  or_moe_gate(ids, wts, x, L->router, B, L->E, L->H, L->topk, L->renorm);
  /* _token_rows: every token row repeated k times, token-major */
  for (int64_t r = 0; r < R; ++r)
    memcpy(xr + r * L->H, x + (r / L->topk) * L->H, sizeof(float) * L->H);
  swiglu_args sw = {g, g, u};
  if (L->int8) {
    or_moe_int8_qmv(g, xr, ids, L->gate_w, L->gate_s, R, L->E, L->F, L->H,
                    L->H / L->group, threads);
    or_moe_int8_qmv(u, xr, ids, L->up_w, L->up_s, R, L->E, L->F, L->H,
                    L->H / L->group, threads);
    parallel_for(R * L->F, threads, items_swiglu, &sw);
    or_moe_int8_qmv(y, g, ids, L->down_w, L->down_s, R, L->E, L->H, L->F,
                    L->F / L->group, threads);
  } else {
    or_moe_bf16_qmv_ref(g, xr, ids, L->gate_w, R, L->E, L->F, L->H, threads);
    or_moe_bf16_qmv_ref(u, xr, ids, L->up_w, R, L->E, L->F, L->H, threads);
    parallel_for(R * L->F, threads, items_swiglu, &sw);
    or_moe_bf16_qmv_ref(y, g, ids, L->down_w, R, L->E, L->H, L->F, threads);
  }
  or_dense_bf16_qmv_ref(sg, x, L->sh_gate, B, L->Fs, L->H,
                        rows_per_read(B, L->Fs), threads);
  or_dense_bf16_qmv_ref(su, x, L->sh_up, B, L->Fs, L->H,
                        rows_per_read(B, L->Fs), threads);
  swiglu_args sws = {sg, sg, su};
  parallel_for(B * L->Fs, threads, items_swiglu, &sws);
  or_dense_bf16_qmv_ref(sh, sg, L->sh_down, B, L->H, L->Fs,
                        rows_per_read(B, L->H), threads);
  /* _mix: [1,k] @ [k,H] per token, then + shared */
  for (int64_t b = 0; b < B; ++b)
    for (int64_t n = 0; n < L->H; ++n) {
      float acc = 0.0f;
      for (int64_t j = 0; j < L->topk; ++j)
        acc = acc + wts[b * L->topk + j] * y[(b * L->topk + j) * L->H + n];
      out[b * L->H + n] = acc + sh[b * L->H + n];
    }
done:
  free(ids);
  free(wts);
  free(xr);
  free(g);
  free(u);
  free(y);
  free(sg);
  free(su);
  free(sh);
  return rc;
}
