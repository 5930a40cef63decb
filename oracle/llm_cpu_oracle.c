/*
 * CPU oracle for llmhost's Q4_32 / Q8_0 matmul path -- TEST INFRASTRUCTURE.
 *
 * A C restatement of crates/llm-quant/src/lib.rs, crates/llm-cpu/src/
 * gemv_q4.rs (+ pool.rs thread split) and crates/llm-engine/src/weights.rs
 * q8_apply.  Used only by tests (as the reference results), by the GPU smoke check and
 * as bench.py's timed CPU baseline.  The product library never links it.
 *
 * Floating-point contract: this file is compiled with -ffp-contract=off so
 * `acc += (float)idot * sw * sa` rounds exactly like the Rust source (Rust
 * never contracts a*b+c into an FMA).  The VNNI-512 kernels use explicit
 * FMA intrinsics where the Rust code does (_mm512_fmadd_ps).
 */
#define _GNU_SOURCE
#include "llm_cpu_oracle.h"

#include <cpuid.h>
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <sys/syscall.h>
#include <unistd.h>

/* ======================================================================
 * f16 <-> f32.  half 2.7.1 (Cargo.lock:210-213) f16::to_f32 is exact and
 * f16::from_f32 rounds to nearest, ties to even (IEEE 754 binary16).
 * ==================================================================== */
float oq_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: renormalise */
      int e = -1;
      do {
        man <<= 1;
        e++;
      } while ((man & 0x400u) == 0);
      man &= 0x3ffu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13) | (man ? 0x400000u : 0u);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t oq_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xff) { /* inf / nan (nan stays quiet) */
    return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u));
  }
  int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
  if (e <= 0) {                                   /* subnormal or zero */
    if (e < -10) return (uint16_t)sign;           /* below half of min subnormal */
    uint32_t m = man | 0x800000u;                 /* 24-bit significand */
    int shift = 14 - e;                           /* to 10-bit subnormal field */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t q = ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* carries into exp/inf */
  return (uint16_t)(sign | q);
}

/* ======================================================================
 * llm-quant block formats (crates/llm-quant/src/lib.rs)
 * ==================================================================== */
static float amax32(const float *src) {
  float a = 0.0f; /* fold(0.0, |acc, v| acc.max(v.abs())) */
  for (int i = 0; i < OQ_BLOCK; i++) a = fmaxf(a, fabsf(src[i]));
  return a;
}

static float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* `x.round().clamp(lo, hi) as i8` in Rust: clamp keeps NaN, and a NaN cast
 * to an integer type is 0 (saturating casts). */
static int8_t rust_round_clamp_i8(float x, float lo, float hi) {
  float r = clampf(roundf(x), lo, hi);
  return r != r ? (int8_t)0 : (int8_t)r;
}

/* lib.rs:26-37 BlockQ8_0::quantize */
void oq_q8_quantize(const float src[32], oq_block_q8 *dst) {
  float amax = amax32(src);
  uint16_t scale = oq_f32_to_f16(amax / 127.0f);
  float scale_f = oq_f16_to_f32(scale);
  float inv = scale_f == 0.0f ? 0.0f : 1.0f / scale_f;
  dst->scale = scale;
  for (int i = 0; i < OQ_BLOCK; i++) dst->qs[i] = rust_round_clamp_i8(src[i] * inv, -127.0f, 127.0f);
}

/* lib.rs:40-45 BlockQ8_0::dequantize */
void oq_q8_dequantize(const oq_block_q8 *b, float dst[32]) {
  float s = oq_f16_to_f32(b->scale);
  for (int i = 0; i < OQ_BLOCK; i++) dst[i] = (float)b->qs[i] * s;
}

/* lib.rs:63-79 BlockQ4::quantize */
void oq_q4_quantize(const float src[32], oq_block_q4 *dst) {
  float amax = amax32(src);
  uint16_t scale = oq_f32_to_f16(amax / 8.0f);
  float scale_f = oq_f16_to_f32(scale);
  float inv = scale_f == 0.0f ? 0.0f : 1.0f / scale_f;
  dst->scale = scale;
  memset(dst->qs, 0, sizeof dst->qs);
  for (int i = 0; i < OQ_BLOCK; i++) {
    int8_t q = rust_round_clamp_i8(src[i] * inv, -8.0f, 7.0f);
    uint8_t nib = (uint8_t)q & 0x0fu;
    if ((i & 1) == 0)
      dst->qs[i / 2] = nib;
    else
      dst->qs[i / 2] |= (uint8_t)(nib << 4);
  }
}

/* lib.rs:83-92 BlockQ4::nibble: two's-complement nibble, even = low. */
int8_t oq_q4_nibble(const oq_block_q4 *b, int i) {
  uint8_t packed = b->qs[i / 2];
  uint8_t nib = (i & 1) ? (uint8_t)(packed >> 4) : (uint8_t)(packed & 0x0fu);
  return (int8_t)((int8_t)(nib << 4) >> 4);
}

/* lib.rs:95-100 BlockQ4::dequantize */
void oq_q4_dequantize(const oq_block_q4 *b, float dst[32]) {
  float s = oq_f16_to_f32(b->scale);
  for (int i = 0; i < OQ_BLOCK; i++) dst[i] = (float)oq_q4_nibble(b, i) * s;
}

/* lib.rs:124-131 quantize_q4 */
int oq_quantize_q4(const float *x, size_t len, oq_block_q4 *out) {
  if (len % OQ_BLOCK) return -1;
  for (size_t b = 0; b < len / OQ_BLOCK; b++) oq_q4_quantize(x + b * OQ_BLOCK, &out[b]);
  return 0;
}

/* lib.rs:104-111 quantize_q8_0 */
int oq_quantize_q8_0(const float *x, size_t len, oq_block_q8 *out) {
  if (len % OQ_BLOCK) return -1;
  for (size_t b = 0; b < len / OQ_BLOCK; b++) oq_q8_quantize(x + b * OQ_BLOCK, &out[b]);
  return 0;
}

/* ======================================================================
 * Activation quantization: gemv_q4.rs:62-95 quantize_blocks (one row) and
 * gemv_q4.rs:747-798 quantize_batch (per token, same arithmetic).
 * ==================================================================== */
static void act_quantize_row(const float *x, size_t k, int per_row, int8_t *qs,
                             float *scales, int32_t *sums) {
  size_t nb = k / OQ_BLOCK;
  float row_scale = 0.0f;
  if (per_row) {
    float a = 0.0f;
    for (size_t i = 0; i < k; i++) a = fmaxf(a, fabsf(x[i]));
    row_scale = a / 127.0f;
  }
  for (size_t b = 0; b < nb; b++) {
    const float *src = x + b * OQ_BLOCK;
    float scale = per_row ? row_scale : amax32(src) / 127.0f;
    float inv = scale == 0.0f ? 0.0f : 1.0f / scale;
    int32_t sum = 0;
    for (int i = 0; i < OQ_BLOCK; i++) {
      int8_t q = rust_round_clamp_i8(src[i] * inv, -127.0f, 127.0f);
      qs[b * OQ_BLOCK + i] = q;
      sum += q;
    }
    scales[b] = scale;
    if (sums) sums[b] = sum;
  }
}

int oq_act_quantize(const float *x, size_t m, size_t k, int per_row, int8_t *qs,
                    float *scales, int32_t *sums) {
  if (k % OQ_BLOCK) return -1;
  size_t nb = k / OQ_BLOCK;
  for (size_t t = 0; t < m; t++)
    act_quantize_row(x + t * k, k, per_row, qs + t * k, scales + t * nb, sums ? sums + t * nb : NULL);
  return 0;
}

/* ======================================================================
 * Per-block integer dots
 * ==================================================================== */
int32_t oq_dot_q4_q8(const oq_block_q4 *b, const int8_t a[32]) {
  int32_t s = 0; /* gemv_q4.rs:959-966 */
  for (int i = 0; i < OQ_BLOCK; i++) s += (int32_t)oq_q4_nibble(b, i) * (int32_t)a[i];
  return s;
}

int32_t oq_dot_q4_q8_offset(const oq_block_q4 *b, const int8_t a[32], int32_t a_sum) {
  int32_t s = 0; /* gemv_q4.rs:1034-1050: dpbusd on unsigned s+8, minus 8*sum(a) */
  for (int i = 0; i < OQ_BLOCK; i++) s += (int32_t)(uint8_t)(oq_q4_nibble(b, i) + 8) * (int32_t)a[i];
  return s - 8 * a_sum;
}

int32_t oq_dot_q8_q8(const oq_block_q8 *b, const int8_t a[32]) {
  int32_t s = 0; /* weights.rs:206-209 */
  for (int i = 0; i < OQ_BLOCK; i++) s += (int32_t)b->qs[i] * (int32_t)a[i];
  return s;
}

/* ======================================================================
 * Packed Q4 matrix: Q4Matrix::from_blocks + pack_tile (gemv_q4.rs:128-149,
 * 212-261).  Tile (t, kb) at byte (t*bpr + kb)*320: 4 pairs x 64 bytes of
 * offset nibbles, byte[pair*64 + col*4 + j] = (s(row,8p+j)+8) |
 * (s(row,8p+4+j)+8) << 4, then 16 LE f32 scales.  Rows >= n are zero.
 * ==================================================================== */
static void pack_tile(uint8_t *out, const oq_block_q4 *blocks, size_t n, size_t bpr,
                      size_t row0, size_t kb) {
  for (int pair = 0; pair < 4; pair++) {
    int kg0 = pair * 2, kg1 = kg0 + 1;
    uint8_t *dst = out + pair * 64;
    for (int col = 0; col < OQ_TILE_N; col++) {
      size_t row = row0 + (size_t)col;
      if (row >= n) {
        memset(dst + col * 4, 0, 4);
        continue;
      }
      const oq_block_q4 *blk = &blocks[row * bpr + kb];
      for (int j = 0; j < 4; j++) {
        uint8_t lo = (uint8_t)(oq_q4_nibble(blk, kg0 * 4 + j) + 8);
        uint8_t hi = (uint8_t)(oq_q4_nibble(blk, kg1 * 4 + j) + 8);
        dst[col * 4 + j] = (uint8_t)(lo | (hi << 4));
      }
    }
  }
  float *scales = (float *)(out + OQ_TILE_QS);
  for (int col = 0; col < OQ_TILE_N; col++) {
    size_t row = row0 + (size_t)col;
    scales[col] = row < n ? oq_f16_to_f32(blocks[row * bpr + kb].scale) : 0.0f;
  }
}

static void prefault(uint8_t *p, size_t len) { /* pool.rs:302-329 */
  volatile uint8_t acc = 0;
  for (size_t i = 0; i < len; i += 4096) acc ^= p[i];
  if (len) acc ^= p[len - 1];
  (void)acc;
}

oq_q4_matrix *oq_q4_from_blocks(size_t n, size_t k, const oq_block_q4 *blocks) {
  if (k % OQ_BLOCK) return NULL;
  size_t bpr = k / OQ_BLOCK;
  oq_q4_matrix *w = calloc(1, sizeof *w);
  if (!w) return NULL;
  w->n = n;
  w->k = k;
  w->n_tiles = (n + OQ_TILE_N - 1) / OQ_TILE_N;
  size_t bytes = w->n_tiles * bpr * OQ_TILE_STRIDE;
  if (bytes == 0) return w;
  w->tiles = aligned_alloc(64, (bytes + 63) / 64 * 64);
  if (!w->tiles) {
    free(w);
    return NULL;
  }
  for (size_t t = 0; t < w->n_tiles; t++)
    for (size_t kb = 0; kb < bpr; kb++)
      pack_tile(w->tiles + (t * bpr + kb) * OQ_TILE_STRIDE, blocks, n, bpr, t * OQ_TILE_N, kb);
  prefault(w->tiles, bytes);
  return w;
}

void oq_q4_free(oq_q4_matrix *w) {
  if (!w) return;
  free(w->tiles);
  free(w);
}

/* ======================================================================
 * Pool: pool.rs semantics that matter for results and timing.  The caller is
 * tid 0; workers 1..T-1 are persistent, pinned to CPU (tid mod ncpu), and
 * spin on a job counter (parking after a long idle spin so an idle test
 * process does not burn cores); one arrival barrier per dispatch; tile range
 * of tid is [tid*n/T, (tid+1)*n/T) (pool.rs:214-221).
 * ==================================================================== */
#define OQ_MAX_THREADS 64 /* pool.rs:22 */

typedef void (*oq_job_fn)(void *ctx, size_t tid, size_t nthreads);

static struct {
  pthread_mutex_t mu;
  pthread_cond_t cv;
  int spawned;
  int sleepers;
  _Atomic uint64_t job_id;
  _Atomic uint32_t arrived;
  _Atomic uint32_t n_active;
  oq_job_fn fn;
  void *ctx;
} g_pool = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER, 1, 0, 0, 0, 1, NULL, NULL};

void oq_thread_range(size_t tid, size_t nthreads, size_t n, size_t *start, size_t *end) {
  if (nthreads == 0) {
    *start = *end = 0;
    return;
  }
  *start = tid * n / nthreads;
  *end = (tid + 1) * n / nthreads;
}

int oq_max_threads(void) { return OQ_MAX_THREADS; }

static void pin_to(size_t tid) {
  long ncpu = sysconf(_SC_NPROCESSORS_ONLN);
  if (ncpu <= 0) return;
  cpu_set_t set;
  CPU_ZERO(&set);
  CPU_SET((int)(tid % (size_t)ncpu), &set);
  pthread_setaffinity_np(pthread_self(), sizeof set, &set);
}

/* Job id each worker has already seen when it is spawned; read by the worker
 * instead of the live counter, which the dispatch that spawned it bumps. */
static uint64_t g_spawn_seen[OQ_MAX_THREADS];

static void *worker_main(void *arg) {
  size_t tid = (size_t)arg;
  pin_to(tid);
  uint64_t seen = g_spawn_seen[tid];
  for (;;) {
    uint64_t id;
    unsigned spins = 0;
    while ((id = atomic_load_explicit(&g_pool.job_id, memory_order_acquire)) == seen) {
      if (++spins < (1u << 22)) {
        _mm_pause();
        continue;
      }
      pthread_mutex_lock(&g_pool.mu);
      g_pool.sleepers++;
      while (atomic_load_explicit(&g_pool.job_id, memory_order_acquire) == seen)
        pthread_cond_wait(&g_pool.cv, &g_pool.mu);
      g_pool.sleepers--;
      pthread_mutex_unlock(&g_pool.mu);
      spins = 0;
    }
    seen = id;
    uint32_t n_active = atomic_load_explicit(&g_pool.n_active, memory_order_acquire);
    if (tid < n_active) {
      g_pool.fn(g_pool.ctx, tid, n_active);
      atomic_fetch_add_explicit(&g_pool.arrived, 1, memory_order_acq_rel);
    }
  }
  return NULL;
}

static void pool_dispatch(size_t nthreads, oq_job_fn fn, void *ctx) {
  if (nthreads > OQ_MAX_THREADS) nthreads = OQ_MAX_THREADS;
  if (nthreads <= 1) {
    fn(ctx, 0, 1);
    return;
  }
  pthread_mutex_lock(&g_pool.mu);
  while (g_pool.spawned < (int)nthreads) {
    pthread_t th;
    g_spawn_seen[g_pool.spawned] = atomic_load_explicit(&g_pool.job_id, memory_order_relaxed);
    pthread_create(&th, NULL, worker_main, (void *)(size_t)g_pool.spawned);
    pthread_detach(th);
    g_pool.spawned++;
  }
  g_pool.fn = fn;
  g_pool.ctx = ctx;
  atomic_store_explicit(&g_pool.arrived, 0, memory_order_relaxed);
  atomic_store_explicit(&g_pool.n_active, (uint32_t)nthreads, memory_order_relaxed);
  atomic_fetch_add_explicit(&g_pool.job_id, 1, memory_order_acq_rel);
  if (g_pool.sleepers) pthread_cond_broadcast(&g_pool.cv);
  pthread_mutex_unlock(&g_pool.mu);
  fn(ctx, 0, nthreads);
  while (atomic_load_explicit(&g_pool.arrived, memory_order_acquire) < nthreads - 1) _mm_pause();
}

/* pool.rs:224-241 for_ranges */
typedef void (*oq_range_fn)(void *ctx, size_t tid, size_t start, size_t end);
struct range_ctx {
  oq_range_fn f;
  void *ctx;
  size_t n_items;
};
static void range_shim(void *c, size_t tid, size_t nthreads) {
  struct range_ctx *rc = c;
  size_t s, e;
  oq_thread_range(tid, nthreads, rc->n_items, &s, &e);
  rc->f(rc->ctx, tid, s, e);
}
static void for_ranges(size_t threads, size_t n_items, oq_range_fn f, void *ctx) {
  if (threads <= 1 || n_items <= 1) {
    f(ctx, 0, 0, n_items);
    return;
  }
  struct range_ctx rc = {f, ctx, n_items};
  pool_dispatch(threads, range_shim, &rc);
}

/* ======================================================================
 * Kernel detection (gemv_q4.rs:311-333) and store_acc (gemv_q4.rs:486-497)
 * ==================================================================== */
int oq_cpu_has(const char *feature) {
  __builtin_cpu_init();
  if (!strcmp(feature, "avx2")) return __builtin_cpu_supports("avx2");
  if (!strcmp(feature, "avx512f")) return __builtin_cpu_supports("avx512f");
  if (!strcmp(feature, "avx512bw")) return __builtin_cpu_supports("avx512bw");
  if (!strcmp(feature, "avx512vnni")) return __builtin_cpu_supports("avx512vnni");
  return 0;
}

static int has_vnni512(void) {
  return oq_cpu_has("avx512vnni") && oq_cpu_has("avx512f") && oq_cpu_has("avx512bw");
}

int oq_detect_kernel(void) {
  if (has_vnni512()) return OQ_KERNEL_VNNI;
  if (oq_cpu_has("avx2")) return OQ_KERNEL_AVX2;
  return OQ_KERNEL_SCALAR;
}

static void store_acc(float *out, size_t n, size_t row0, const float acc[OQ_TILE_N], int add) {
  size_t count = row0 >= n ? 0 : (n - row0 < OQ_TILE_N ? n - row0 : OQ_TILE_N);
  for (size_t c = 0; c < count; c++) {
    if (add)
      out[row0 + c] = (float)((double)out[row0 + c] + (double)acc[c]);
    else
      out[row0 + c] = acc[c];
  }
}

static inline float tile_scale(const uint8_t *panel, int col) {
  float s;
  memcpy(&s, panel + OQ_TILE_QS + col * 4, 4);
  return s;
}

/* ======================================================================
 * GEMV tile kernels
 * ==================================================================== */
/* gemv_q4.rs:499-544 gemv_tiles_scalar: the reference operation order. */
static void gemv_tiles_scalar(const oq_q4_matrix *w, const int8_t *qs, const float *scales,
                              float *out, size_t t0, size_t t1, int add) {
  size_t bpr = w->k / OQ_BLOCK;
  for (size_t tile = t0; tile < t1; tile++) {
    float acc[OQ_TILE_N] = {0};
    for (size_t kb = 0; kb < bpr; kb++) {
      const uint8_t *panel = w->tiles + (tile * bpr + kb) * OQ_TILE_STRIDE;
      const int8_t *a = qs + kb * OQ_BLOCK;
      float sa = scales[kb];
      int32_t idot[OQ_TILE_N] = {0};
      for (int pair = 0; pair < 4; pair++) {
        int kg0 = pair * 2, kg1 = kg0 + 1;
        const uint8_t *bytes = panel + pair * 64;
        for (int col = 0; col < OQ_TILE_N; col++) {
          int32_t s = 0;
          for (int j = 0; j < 4; j++) {
            uint8_t packed = bytes[col * 4 + j];
            int32_t lo = (int32_t)(packed & 0x0f) - 8;
            int32_t hi = (int32_t)(packed >> 4) - 8;
            s += lo * a[kg0 * 4 + j];
            s += hi * a[kg1 * 4 + j];
          }
          idot[col] += s;
        }
      }
      for (int col = 0; col < OQ_TILE_N; col++) acc[col] += (float)idot[col] * tile_scale(panel, col) * sa;
    }
    store_acc(out, w->n, tile * OQ_TILE_N, acc, add);
  }
}

/* gemv_q4.rs:546-607 gemv_tiles_avx2_inner: madd_epi16 on sign-corrected
 * nibbles; integer-exact, then the same scalar f32 fold. */
__attribute__((target("avx2"))) static void gemv_tiles_avx2(const oq_q4_matrix *w, const int8_t *qs,
                                                              const float *scales, float *out, size_t t0,
                                                              size_t t1, int add) {
  size_t bpr = w->k / OQ_BLOCK;
  for (size_t tile = t0; tile < t1; tile++) {
    float acc[OQ_TILE_N] = {0};
    for (size_t kb = 0; kb < bpr; kb++) {
      const uint8_t *panel = w->tiles + (tile * bpr + kb) * OQ_TILE_STRIDE;
      const int8_t *a = qs + kb * OQ_BLOCK;
      float sa = scales[kb];
      int32_t idot[OQ_TILE_N] = {0};
      for (int pair = 0; pair < 4; pair++) {
        int kg0 = pair * 2, kg1 = kg0 + 1;
        const uint8_t *bytes = panel + pair * 64;
        int32_t a0i, a1i;
        memcpy(&a0i, a + kg0 * 4, 4);
        memcpy(&a1i, a + kg1 * 4, 4);
        __m128i aa = _mm_cvtepi8_epi16(_mm_cvtsi32_si128(a0i));
        __m128i ab = _mm_cvtepi8_epi16(_mm_cvtsi32_si128(a1i));
        for (int col = 0; col < OQ_TILE_N; col++) {
          int32_t wi;
          memcpy(&wi, bytes + col * 4, 4);
          __m128i packed = _mm_cvtsi32_si128(wi);
          __m128i lo = _mm_and_si128(packed, _mm_set1_epi8(0x0f));
          __m128i hi = _mm_and_si128(_mm_srli_epi16(packed, 4), _mm_set1_epi8(0x0f));
          __m128i eight = _mm_set1_epi8(8);
          __m128i wa = _mm_cvtepi8_epi16(_mm_sub_epi8(lo, eight));
          __m128i wb = _mm_cvtepi8_epi16(_mm_sub_epi8(hi, eight));
          __m128i sum = _mm_add_epi32(_mm_madd_epi16(wa, aa), _mm_madd_epi16(wb, ab));
          sum = _mm_add_epi32(sum, _mm_shuffle_epi32(sum, 0x31));
          idot[col] += _mm_cvtsi128_si32(sum);
        }
      }
      for (int col = 0; col < OQ_TILE_N; col++) acc[col] += (float)idot[col] * tile_scale(panel, col) * sa;
    }
    store_acc(out, w->n, tile * OQ_TILE_N, acc, add);
  }
}

/* gemv_q4.rs:622-667 gemv_tiles_vnni512_inner: 16 rows per zmm, dpbusd on
 * unsigned nibbles with the 8*sum(a) compensation recomputed per tile/kb,
 * vacc = fma(f32(isum), sw*sa, vacc). */
__attribute__((target("avx512f,avx512bw,avx512vnni"))) static void gemv_tiles_vnni512(
    const oq_q4_matrix *w, const int8_t *qs, const float *scales, float *out, size_t t0, size_t t1,
    int add) {
  size_t bpr = w->k / OQ_BLOCK;
  const __m512i off = _mm512_set1_epi8(8);
  const __m512i low_mask = _mm512_set1_epi8(0x0f);
  for (size_t tile = t0; tile < t1; tile++) {
    __m512 vacc = _mm512_setzero_ps();
    const uint8_t *tile_base = w->tiles + tile * bpr * OQ_TILE_STRIDE;
    for (size_t kb = 0; kb < bpr; kb++) {
      const uint8_t *panel = tile_base + kb * OQ_TILE_STRIDE;
      const int8_t *a_ptr = qs + kb * OQ_BLOCK;
      __m512i va[8];
      __m512i vcomp = _mm512_setzero_si512();
      for (int k = 0; k < 8; k++) {
        int32_t ai;
        memcpy(&ai, a_ptr + 4 * k, 4);
        va[k] = _mm512_set1_epi32(ai);
        vcomp = _mm512_dpbusd_epi32(vcomp, off, va[k]);
      }
      __m512i vsum = _mm512_setzero_si512();
      for (int pair = 0; pair < 4; pair++) {
        __m512i bytes = _mm512_loadu_si512((const void *)(panel + pair * 64));
        __m512i vb0 = _mm512_and_si512(bytes, low_mask);
        __m512i vb1 = _mm512_and_si512(_mm512_srli_epi16(bytes, 4), low_mask);
        vsum = _mm512_dpbusd_epi32(vsum, vb0, va[pair * 2]);
        vsum = _mm512_dpbusd_epi32(vsum, vb1, va[pair * 2 + 1]);
      }
      vsum = _mm512_sub_epi32(vsum, vcomp);
      __m512 sw = _mm512_loadu_ps((const void *)(panel + OQ_TILE_QS));
      __m512 sa = _mm512_set1_ps(scales[kb]);
      vacc = _mm512_fmadd_ps(_mm512_cvtepi32_ps(vsum), _mm512_mul_ps(sw, sa), vacc);
    }
    float acc[OQ_TILE_N];
    _mm512_storeu_ps(acc, vacc);
    store_acc(out, w->n, tile * OQ_TILE_N, acc, add);
  }
}

/* gemv_q4.rs:451-484 gemv_tiles dispatch */
static void gemv_tiles(const oq_q4_matrix *w, const int8_t *qs, const float *scales, float *out,
                       size_t t0, size_t t1, int kernel, int add) {
  if (kernel == OQ_KERNEL_VNNI && has_vnni512())
    gemv_tiles_vnni512(w, qs, scales, out, t0, t1, add);
  else if (kernel == OQ_KERNEL_AVX2 && oq_cpu_has("avx2"))
    gemv_tiles_avx2(w, qs, scales, out, t0, t1, add);
  else
    gemv_tiles_scalar(w, qs, scales, out, t0, t1, add);
}

/* Thread-local activation scratch, gemv_q4.rs:335-341 ACT_SCRATCH. */
static __thread int8_t *tl_qs;
static __thread float *tl_sc;
static __thread int32_t *tl_su;
static __thread size_t tl_cap;

static void act_scratch(size_t k) {
  if (k <= tl_cap) return;
  free(tl_qs);
  free(tl_sc);
  free(tl_su);
  tl_qs = malloc(k);
  tl_sc = malloc(k / OQ_BLOCK * sizeof(float) + 4);
  tl_su = malloc(k / OQ_BLOCK * sizeof(int32_t) + 4);
  tl_cap = k;
}

struct gemv_job {
  const oq_q4_matrix *w, *w2;
  const int8_t *qs;
  const float *scales;
  float *out, *out2;
  int kernel, add;
};

static void gemv_range(void *c, size_t tid, size_t t0, size_t t1) {
  (void)tid;
  struct gemv_job *j = c;
  gemv_tiles(j->w, j->qs, j->scales, j->out, t0, t1, j->kernel, j->add);
  if (j->w2) gemv_tiles(j->w2, j->qs, j->scales, j->out2, t0, t1, j->kernel, 0);
}

static int resolve_kernel(int kernel) { return kernel < 0 ? oq_detect_kernel() : kernel; }

/* gemv_q4.rs:366-393 gemv_q4_prep / gemv_q4_prep_add */
void oq_gemv_q4_prep(const oq_q4_matrix *w, const int8_t *qs, const float *scales, float *out,
                     int add, int kernel, int threads) {
  if (w->n == 0) return;
  struct gemv_job j = {w, NULL, qs, scales, out, NULL, resolve_kernel(kernel), add};
  for_ranges((size_t)threads, w->n_tiles, gemv_range, &j);
}

/* gemv_q4.rs:344-363 gemv_q4 / gemv_q4_add: quantize on the caller thread,
 * then one pool dispatch over tiles. */
void oq_gemv_q4(const oq_q4_matrix *w, const float *x, float *out, int add, int per_row, int kernel,
                int threads) {
  act_scratch(w->k);
  act_quantize_row(x, w->k, per_row, tl_qs, tl_sc, tl_su);
  oq_gemv_q4_prep(w, tl_qs, tl_sc, out, add, kernel, threads);
}

/* gemv_q4.rs:396-443 gemv_q4_pair: one act quant, one dispatch, each thread
 * owns the same tile range of both matrices. */
void oq_gemv_q4_pair(const oq_q4_matrix *wg, const oq_q4_matrix *wu, const float *x, float *out_g,
                     float *out_u, int per_row, int kernel, int threads) {
  act_scratch(wg->k);
  act_quantize_row(x, wg->k, per_row, tl_qs, tl_sc, tl_su);
  struct gemv_job j = {wg, wu, tl_qs, tl_sc, out_g, out_u, resolve_kernel(kernel), 0};
  for_ranges((size_t)threads, wg->n_tiles, gemv_range, &j);
}

/* ======================================================================
 * GEMM: gemm_q4_mode (gemv_q4.rs:695-722), quantize_batch (747-798),
 * gemm_tiles_scalar (822-879), gemm_tiles_vnni512_inner (881-938).
 * ==================================================================== */
struct gemm_job {
  const oq_q4_matrix *w;
  const int8_t *qs;
  const float *scales;
  float *out;
  size_t m;
  int kernel, add, per_row;
  const float *x;
  int8_t *qs_w;
  float *sc_w;
};

static void gemm_tiles_scalar(const oq_q4_matrix *w, const int8_t *qs, const float *scales, float *out,
                              size_t m, size_t t0, size_t t1, int add) {
  size_t bpr = w->k / OQ_BLOCK;
  float *acc = malloc(m * OQ_TILE_N * sizeof(float));
  for (size_t tile = t0; tile < t1; tile++) {
    memset(acc, 0, m * OQ_TILE_N * sizeof(float));
    size_t row0 = tile * OQ_TILE_N;
    for (size_t kb = 0; kb < bpr; kb++) {
      const uint8_t *panel = w->tiles + (tile * bpr + kb) * OQ_TILE_STRIDE;
      for (size_t t = 0; t < m; t++) {
        const int8_t *a = qs + t * w->k + kb * OQ_BLOCK;
        float sa = scales[t * bpr + kb];
        int32_t idot[OQ_TILE_N] = {0};
        for (int pair = 0; pair < 4; pair++) {
          int kg0 = pair * 2, kg1 = kg0 + 1;
          const uint8_t *bytes = panel + pair * 64;
          for (int col = 0; col < OQ_TILE_N; col++) {
            int32_t s = 0;
            for (int j = 0; j < 4; j++) {
              uint8_t packed = bytes[col * 4 + j];
              s += ((int32_t)(packed & 0x0f) - 8) * a[kg0 * 4 + j];
              s += ((int32_t)(packed >> 4) - 8) * a[kg1 * 4 + j];
            }
            idot[col] += s;
          }
        }
        float *dst = acc + t * OQ_TILE_N;
        for (int col = 0; col < OQ_TILE_N; col++) dst[col] += (float)idot[col] * tile_scale(panel, col) * sa;
      }
    }
    for (size_t t = 0; t < m; t++) store_acc(out + t * w->n, w->n, row0, acc + t * OQ_TILE_N, add);
  }
  free(acc);
}

__attribute__((target("avx512f,avx512bw,avx512vnni"))) static void gemm_tiles_vnni512(
    const oq_q4_matrix *w, const int8_t *qs, const float *scales, float *out, size_t m, size_t t0,
    size_t t1, int add) {
  size_t bpr = w->k / OQ_BLOCK;
  const __m512i off = _mm512_set1_epi8(8);
  const __m512i low_mask = _mm512_set1_epi8(0x0f);
  float *acc = aligned_alloc(64, (m * OQ_TILE_N * sizeof(float) + 63) / 64 * 64);
  for (size_t tile = t0; tile < t1; tile++) {
    memset(acc, 0, m * OQ_TILE_N * sizeof(float));
    size_t row0 = tile * OQ_TILE_N;
    const uint8_t *tile_base = w->tiles + tile * bpr * OQ_TILE_STRIDE;
    for (size_t kb = 0; kb < bpr; kb++) {
      const uint8_t *panel = tile_base + kb * OQ_TILE_STRIDE;
      __m512 sw = _mm512_loadu_ps((const void *)(panel + OQ_TILE_QS));
      for (size_t t = 0; t < m; t++) {
        const int8_t *a_ptr = qs + t * w->k + kb * OQ_BLOCK;
        __m512 sa = _mm512_set1_ps(scales[t * bpr + kb]);
        __m512i va[8];
        __m512i vcomp = _mm512_setzero_si512();
        for (int k = 0; k < 8; k++) {
          int32_t ai;
          memcpy(&ai, a_ptr + 4 * k, 4);
          va[k] = _mm512_set1_epi32(ai);
          vcomp = _mm512_dpbusd_epi32(vcomp, off, va[k]);
        }
        __m512i vsum = _mm512_setzero_si512();
        for (int pair = 0; pair < 4; pair++) {
          __m512i bytes = _mm512_loadu_si512((const void *)(panel + pair * 64));
          vsum = _mm512_dpbusd_epi32(vsum, _mm512_and_si512(bytes, low_mask), va[pair * 2]);
          vsum = _mm512_dpbusd_epi32(vsum, _mm512_and_si512(_mm512_srli_epi16(bytes, 4), low_mask),
                                     va[pair * 2 + 1]);
        }
        vsum = _mm512_sub_epi32(vsum, vcomp);
        __m512 vacc = _mm512_loadu_ps(acc + t * OQ_TILE_N);
        vacc = _mm512_fmadd_ps(_mm512_cvtepi32_ps(vsum), _mm512_mul_ps(sw, sa), vacc);
        _mm512_storeu_ps(acc + t * OQ_TILE_N, vacc);
      }
    }
    for (size_t t = 0; t < m; t++) store_acc(out + t * w->n, w->n, row0, acc + t * OQ_TILE_N, add);
  }
  free(acc);
}

/* ======================================================================
 * AMX-INT8 GEMM tiles: llm-cpu/src/amx.rs.  gemm_q4_mode takes them for
 * m >= 16 without add when the host can run AMX (gemv_q4.rs:711).
 * amx_ready (amx.rs:29-66): CPUID AMX-TILE and AMX-INT8, then Linux
 * arch_prctl(ARCH_REQ_XCOMP_PERM, XTILEDATA) once per process.  Palette
 * (amx.rs:79-106): tmm0/1 B panels 8 x 64 bytes (VNNI: row r holds K
 * 4r..4r+3 of each of 16 columns), tmm2/3 A 16 tokens x 32 codes, tmm4-7 C
 * 16 x 16 i32.  Per K block (amx.rs:329-518): A = the block's codes of every
 * token (zero rows to a multiple of 16); for N-tile pairs and 32-token steps,
 * C = A x B by tdpbssd, stored and folded into an f32 accumulator --
 * fma(f32(c), sw * sa, acc) for a whole 16-column tile, acc + (c * sw) * sa
 * for a partial one (fold_c / fold_c_avx512, amx.rs:264-320).
 * ==================================================================== */
static atomic_int g_amx_state; /* 0 unknown, 1 ready, 2 not available */

static int amx_probe(void) {
  unsigned a, b, c, d;
  if (!__get_cpuid_count(7, 0, &a, &b, &c, &d)) return 0;
  const int tile = (d >> 24) & 1, int8 = (d >> 25) & 1;
  if (!tile || !int8) return 0;
  /* ARCH_REQ_XCOMP_PERM = 0x1023, XFEATURE_XTILEDATA = 18 */
  return syscall(SYS_arch_prctl, 0x1023, 18) == 0;
}

int oq_amx_ready(void) {
  int st = atomic_load_explicit(&g_amx_state, memory_order_acquire);
  if (st == 0) {
    st = amx_probe() ? 1 : 2;
    atomic_store_explicit(&g_amx_state, st, memory_order_release);
  }
  return st == 1;
}

struct amx_tilecfg {
  uint8_t palette_id, start_row, reserved[14];
  uint16_t colsb[16];
  uint8_t rows[16];
} __attribute__((aligned(64)));

static __thread int t_amx_cfg_loaded;

__attribute__((target("amx-tile,amx-int8"))) static void amx_load_cfg(void) {
  if (t_amx_cfg_loaded) return;
  struct amx_tilecfg cfg;
  memset(&cfg, 0, sizeof cfg);
  cfg.palette_id = 1;
  for (int t = 0; t < 2; t++) cfg.rows[t] = 8, cfg.colsb[t] = 64;   /* B */
  for (int t = 2; t < 4; t++) cfg.rows[t] = 16, cfg.colsb[t] = 32;  /* A */
  for (int t = 4; t < 8; t++) cfg.rows[t] = 16, cfg.colsb[t] = 64;  /* C */
  _tile_loadconfig(&cfg);
  t_amx_cfg_loaded = 1;
}

/* The tile panel's nibbles as the signed int8 B panel: byte j of column c
 * in pair p (panel + 64p + 4c + j) holds K 8p+j (low nibble, row 2p) and
 * K 8p+4+j (high nibble, row 2p+1), each stored +8 (amx.rs:229-244). */
static void amx_pack_b(const uint8_t *panel, int8_t dst[8 * 64]) {
  for (int pair = 0; pair < 4; pair++)
    for (int i = 0; i < 64; i++) {
      const uint8_t b = panel[pair * 64 + i];
      dst[(2 * pair) * 64 + i] = (int8_t)((int)(b & 0x0f) - 8);
      dst[(2 * pair + 1) * 64 + i] = (int8_t)((int)(b >> 4) - 8);
    }
}

__attribute__((target("avx512f"))) static void amx_fold(const int32_t c[16 * 16], float *acc, size_t acc_stride,
                                                        size_t tok, size_t rows, size_t cols, size_t col_off,
                                                        const float sw[16], const float *scales, size_t kb,
                                                        size_t bpr) {
  if (cols == OQ_TILE_N) {
    const __m512 vsw = _mm512_loadu_ps(sw);
    for (size_t r = 0; r < rows; r++) {
      const float sa = scales[(tok + r) * bpr + kb];
      float *dst = acc + (tok + r) * acc_stride + col_off;
      const __m512 vc = _mm512_cvtepi32_ps(_mm512_loadu_si512((const void *)(c + r * 16)));
      _mm512_storeu_ps(dst, _mm512_fmadd_ps(vc, _mm512_mul_ps(vsw, _mm512_set1_ps(sa)), _mm512_loadu_ps(dst)));
    }
    return;
  }
  for (size_t r = 0; r < rows; r++) {
    const float sa = scales[(tok + r) * bpr + kb];
    float *dst = acc + (tok + r) * acc_stride + col_off;
    for (size_t col = 0; col < cols; col++) dst[col] += (float)c[r * 16 + col] * sw[col] * sa;
  }
}

__attribute__((target("amx-tile,amx-int8,avx512f"))) static void gemm_tiles_amx(
    const oq_q4_matrix *w, const int8_t *qs, const float *scales, float *out, size_t m, size_t t0, size_t t1) {
  if (t0 >= t1 || m == 0) return;
  amx_load_cfg();
  const size_t n = w->n, k = w->k, bpr = k / OQ_BLOCK;
  const size_t acc_stride = (t1 - t0) * OQ_TILE_N, m_pad = (m + 15) / 16 * 16;
  float *acc = calloc(m * acc_stride, sizeof(float));
  int8_t *a_pack = aligned_alloc(64, m_pad * 32);
  int32_t c0[16 * 16] __attribute__((aligned(64))), c1[16 * 16] __attribute__((aligned(64)));
  int8_t b0[8 * 64] __attribute__((aligned(64))), b1[8 * 64] __attribute__((aligned(64)));
  float sw0[16], sw1[16];
  for (size_t kb = 0; kb < bpr; kb++) {
    memset(a_pack, 0, m_pad * 32);
    for (size_t t = 0; t < m; t++) memcpy(a_pack + t * 32, qs + t * k + kb * OQ_BLOCK, 32);
    size_t col_base = 0;
    for (size_t tile = t0; tile < t1;) {
      const int two = tile + 1 < t1;
      const size_t row0 = tile * OQ_TILE_N;
      const size_t cols0 = n > row0 ? (n - row0 < 16 ? n - row0 : 16) : 0;
      const size_t cols1 = two ? (n > row0 + 16 ? (n - row0 - 16 < 16 ? n - row0 - 16 : 16) : 0) : 0;
      const uint8_t *p0 = w->tiles + (tile * bpr + kb) * OQ_TILE_STRIDE;
      const uint8_t *p1 = two ? w->tiles + ((tile + 1) * bpr + kb) * OQ_TILE_STRIDE : NULL;
      for (int col = 0; col < 16; col++) sw0[col] = tile_scale(p0, col);
      amx_pack_b(p0, b0);
      _tile_loadd(0, b0, 64);
      if (two) {
        for (int col = 0; col < 16; col++) sw1[col] = tile_scale(p1, col);
        amx_pack_b(p1, b1);
        _tile_loadd(1, b1, 64);
      }
      for (size_t tok = 0; tok < m; tok += 32) {
        const size_t rows0 = m - tok < 16 ? m - tok : 16;
        const size_t rows1 = m - tok > 16 ? (m - tok - 16 < 16 ? m - tok - 16 : 16) : 0;
        _tile_zero(4);
        _tile_loadd(2, a_pack + tok * 32, 32);
        _tile_dpbssd(4, 2, 0);
        _tile_stored(4, c0, 64);
        if (two) {
          _tile_zero(5);
          _tile_dpbssd(5, 2, 1);
          _tile_stored(5, c1, 64);
        }
        amx_fold(c0, acc, acc_stride, tok, rows0, cols0, col_base, sw0, scales, kb, bpr);
        if (two) amx_fold(c1, acc, acc_stride, tok, rows0, cols1, col_base + 16, sw1, scales, kb, bpr);
        if (rows1) {
          _tile_zero(6);
          _tile_loadd(3, a_pack + (tok + 16) * 32, 32);
          _tile_dpbssd(6, 3, 0);
          _tile_stored(6, c0, 64);
          if (two) {
            _tile_zero(7);
            _tile_dpbssd(7, 3, 1);
            _tile_stored(7, c1, 64);
          }
          amx_fold(c0, acc, acc_stride, tok + 16, rows1, cols0, col_base, sw0, scales, kb, bpr);
          if (two) amx_fold(c1, acc, acc_stride, tok + 16, rows1, cols1, col_base + 16, sw1, scales, kb, bpr);
        }
      }
      col_base += two ? 32 : 16;
      tile += two ? 2 : 1;
    }
  }
  for (size_t ti = 0; ti < t1 - t0; ti++) {
    const size_t row0 = (t0 + ti) * OQ_TILE_N;
    const size_t cols = n > row0 ? (n - row0 < 16 ? n - row0 : 16) : 0;
    for (size_t t = 0; t < m; t++)
      for (size_t col = 0; col < cols; col++) out[t * n + row0 + col] = acc[t * acc_stride + ti * 16 + col];
  }
  free(a_pack);
  free(acc);
}

static void gemm_range(void *c, size_t tid, size_t t0, size_t t1) {
  (void)tid;
  struct gemm_job *j = c;
  if (j->kernel == OQ_KERNEL_AMX)
    gemm_tiles_amx(j->w, j->qs, j->scales, j->out, j->m, t0, t1);
  else if (j->kernel == OQ_KERNEL_VNNI && has_vnni512())
    gemm_tiles_vnni512(j->w, j->qs, j->scales, j->out, j->m, t0, t1, j->add);
  else
    gemm_tiles_scalar(j->w, j->qs, j->scales, j->out, j->m, t0, t1, j->add);
}

static void quant_range(void *c, size_t tid, size_t t0, size_t t1) {
  (void)tid;
  struct gemm_job *j = c;
  size_t k = j->w->k, bpr = k / OQ_BLOCK;
  for (size_t t = t0; t < t1; t++)
    act_quantize_row(j->x + t * k, k, j->per_row, j->qs_w + t * k, j->sc_w + t * bpr, NULL);
}

void oq_gemm_q4(const oq_q4_matrix *w, const float *x, float *out, size_t m, int add, int per_row,
                int kernel, int threads) {
  if (m == 0 || w->n == 0) return;
  if (m == 1) {
    oq_gemv_q4(w, x, out, add, per_row, kernel, threads);
    return;
  }
  size_t k = w->k, bpr = k / OQ_BLOCK;
  int8_t *qs = malloc(m * k);
  float *sc = malloc(m * bpr * sizeof(float));
  /* gemv_q4.rs:711: AMX for m >= 16 without add on an AMX host (detected
   * kernel), or when asked for; else the tile kernels. */
  int kern = kernel;
  if ((kernel < 0 || kernel == OQ_KERNEL_AMX) && m >= 16 && !add && oq_amx_ready())
    kern = OQ_KERNEL_AMX;
  else
    kern = resolve_kernel(kernel == OQ_KERNEL_AMX ? -1 : kernel);
  struct gemm_job j = {w, qs, sc, out, m, kern, add, per_row, x, qs, sc};
  for_ranges((size_t)threads, m, quant_range, &j);
  for_ranges((size_t)threads, w->n_tiles, gemm_range, &j);
  free(qs);
  free(sc);
}

/* ======================================================================
 * Q8_0 head GEMV: llm-engine/src/weights.rs:194-227 q8_apply.  Always
 * per-block activation quant; row-parallel for_ranges(n); scalar loop;
 * tokens > 1 loops over tokens.
 * ==================================================================== */
struct q8_job {
  const oq_block_q8 *blocks;
  size_t bpr;
  const int8_t *qs;
  const float *scales;
  float *out;
};

static void q8_range(void *c, size_t tid, size_t r0, size_t r1) {
  (void)tid;
  struct q8_job *j = c;
  for (size_t row = r0; row < r1; row++) {
    float acc = 0.0f;
    const oq_block_q8 *rw = j->blocks + row * j->bpr;
    for (size_t b = 0; b < j->bpr; b++) {
      int32_t s = oq_dot_q8_q8(&rw[b], j->qs + b * OQ_BLOCK);
      acc += (float)s * oq_f16_to_f32(rw[b].scale) * j->scales[b];
    }
    j->out[row] = acc;
  }
}

void oq_q8_apply(const oq_block_q8 *blocks, size_t n, size_t k, const float *x, size_t tokens,
                 float *out, int threads) {
  size_t bpr = k / OQ_BLOCK;
  act_scratch(k);
  for (size_t t = 0; t < tokens; t++) {
    act_quantize_row(x + t * k, k, 0, tl_qs, tl_sc, tl_su);
    struct q8_job j = {blocks, bpr, tl_qs, tl_sc, out + t * n};
    for_ranges((size_t)threads, n, q8_range, &j);
  }
}

/* ======================================================================
 * Decode FFN block: rms_norm (llm-cpu/src/ops.rs:8-23), silu (ops.rs:27-36)
 * and Lfm2::ffn_residual_in (llm-engine/src/lfm2.rs:883-911).
 * ==================================================================== */
void oq_rms_norm(const float *x, const float *weight, size_t dim, size_t rows, float eps, float *out) {
  const double inv_dim = 1.0 / (double)dim;
  for (size_t r = 0; r < rows; r++) {
    const float *row = x + r * dim;
    float *dst = out + r * dim;
    double sumsq = 0.0;
    for (size_t i = 0; i < dim; i++) sumsq += (double)row[i] * (double)row[i];
    const float scale = (float)(1.0 / sqrt(sumsq * inv_dim + (double)eps));
    for (size_t i = 0; i < dim; i++) dst[i] = weight[i] * (row[i] * scale);
  }
}

void oq_silu_mul(float *g, const float *u, size_t n) {
  for (size_t i = 0; i < n; i++) {
    const float x = g[i];
    g[i] = x / (1.0f + expf(-x));
    g[i] *= u[i];
  }
}

void oq_ffn_residual(const oq_q4_matrix *w1, const oq_q4_matrix *w3, const oq_q4_matrix *w2,
                     const float *norm_w, float eps, float *hidden, size_t tokens, int per_row, int kernel,
                     int threads) {
  const size_t dim = w1->k, inter = w1->n;
  float *normed = malloc(tokens * dim * sizeof(float));
  float *g = malloc(tokens * inter * sizeof(float));
  float *u = malloc(tokens * inter * sizeof(float));
  if (norm_w)
    oq_rms_norm(hidden, norm_w, dim, tokens, eps, normed);
  else
    memcpy(normed, hidden, tokens * dim * sizeof(float));
  if (tokens == 1) {  /* apply_pair (weights.rs:106-123): the pair GEMV for one token */
    oq_gemv_q4_pair(w1, w3, normed, g, u, per_row, kernel, threads);
  } else {           /* ... else two separate apply calls */
    oq_gemm_q4(w1, normed, g, tokens, 0, per_row, kernel, threads);
    oq_gemm_q4(w3, normed, u, tokens, 0, per_row, kernel, threads);
  }
  oq_silu_mul(g, u, tokens * inter);
  if (tokens == 1)
    oq_gemv_q4(w2, g, hidden, 1, per_row, kernel, threads);
  else
    oq_gemm_q4(w2, g, hidden, tokens, 1, per_row, kernel, threads);
  free(normed);
  free(g);
  free(u);
}
