// C ABI of libllm_gpu_hip.so: contexts, weight upload/repack, and the GEMV /
// GEMM / Q8 entry points that stand in for llm-cpu's public functions
// (crates/llm-cpu/src/lib.rs:21-24) behind llm-engine's Linear / OutputHead
// seam (crates/llm-engine/src/weights.rs:75-192).
//
// Error behaviour: the reference panics on contract violations (assert_eq!
// on lengths, k % 32); here every such case returns LGH_ERR_SHAPE (or
// LGH_ERR_INVALID_ARG for null/misaligned pointers) before any work is
// enqueued, and lgh_last_error() names the violated condition.
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>

#include "lgh_internal.h"

// Fixed device scratch of lgh_q4_gemm_dev_noalloc: one copy per GPU, held
// until the process ends.  Host code never uses this name as an address (on
// the host it is a stand-in, not device memory): lgh_init looks up each
// device's copy with hipGetSymbolAddress and every call passes that pointer.
__device__ __align__(256) uint8_t scratch[LGH_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_init_err;

// Device address of `scratch` per device, looked up once per device with
// that device current.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch[kMaxDevices] = {};

int fail(lgh_ctx *ctx, int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (ctx)
    ctx->err = buf;
  else
    g_init_err = buf;
  return code;
}

int hip_fail(lgh_ctx *ctx, hipError_t e, const char *what) {
  return fail(ctx, LGH_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), static_cast<int>(e));
}

#define LGH_HIP(ctx, call)                              \
  do {                                                  \
    hipError_t e_ = (call);                             \
    if (e_ != hipSuccess) return hip_fail(ctx, e_, #call); \
  } while (0)

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

int set_device(lgh_ctx *ctx) {
  LGH_HIP(ctx, hipSetDevice(ctx->device));
  return LGH_OK;
}

// Grow-only device buffer; waits for queued work before releasing the old one.
// A stream under graph capture cannot synchronize or allocate: growing there
// fails with LGH_ERR_CAPTURE (the caller warms the shape up eagerly first, or
// uses lgh_q4_gemm_dev_noalloc).
int ensure(lgh_ctx *ctx, void **buf, size_t *cap, size_t bytes) {
  if (bytes <= *cap) return LGH_OK;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(ctx->stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
    return fail(ctx, LGH_ERR_CAPTURE,
                "a workspace must grow to %zu bytes while the stream is being captured; run the same "
                "shape once before capturing, or call lgh_q4_gemm_dev_noalloc",
                bytes);
  if (*buf) {
    LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
    LGH_HIP(ctx, hipFree(*buf));
    *buf = nullptr;
    *cap = 0;
  }
  const size_t want = align_up(bytes);
  hipError_t e = hipMalloc(buf, want);
  if (e != hipSuccess) {
    *buf = nullptr;
    return fail(ctx, LGH_ERR_OOM, "hipMalloc(%zu bytes) failed: %s", want, hipGetErrorString(e));
  }
  *cap = want;
  return LGH_OK;
}

// Free a grow-only buffer (the caller has synchronized the stream).
void release(lgh_ctx *, void **buf, size_t *cap) {
  if (*buf) (void)hipFree(*buf);
  *buf = nullptr;
  *cap = 0;
}

// The host-call staging buffer keeps its peak size between calls; after a
// weight upload that staged more than this (an fp32 matrix, e.g. 512 MB for a
// 65536 x 2048 head) it is released once the upload has completed.
constexpr size_t kStageKeepBytes = size_t(64) << 20;
void trim_stage(lgh_ctx *ctx) {
  if (ctx->stage_bytes > kStageKeepBytes) release(ctx, &ctx->stage, &ctx->stage_bytes);
}

// Carve consecutive 256-byte aligned regions out of the staging buffer.
struct Carve {
  size_t off = 0;
  size_t take(size_t bytes) {
    const size_t o = off;
    off = align_up(off + bytes);
    return o;
  }
};

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Where one call takes its device scratch (activation images, codes, split-K
// partials): the context's grow-only workspace, or -- for the entry point that
// allocates nothing -- the device's fixed scratch array, which a request larger
// than its capacity cannot grow (LGH_ERR_SHAPE).
struct Ws {
  lgh_ctx *ctx;
  char *fixed;  // non-null: the fixed scratch of ctx's device
  size_t cap;   // its size in bytes
  int get(size_t bytes, char **out) const {
    if (fixed) {
      if (bytes > cap)
        return fail(ctx, LGH_ERR_SHAPE, "the call needs %zu bytes of scratch; the fixed scratch holds %zu", bytes,
                    cap);
      *out = fixed;
      return LGH_OK;
    }
    if (int r = ensure(ctx, &ctx->ws, &ctx->ws_bytes, bytes)) return r;
    *out = static_cast<char *>(ctx->ws);
    return LGH_OK;
  }
  size_t limit() const { return fixed ? cap : SIZE_MAX; }
};

Ws grow_ws(lgh_ctx *ctx) { return Ws{ctx, nullptr, 0}; }

void set_tiles(lgh_q8 *) {}
void set_tiles(lgh_q4 *w) {
  w->nt = (w->n + 31) / 32;
  w->pp = (w->bpr + 1) / 2;
}

template <class M>
int alloc_matrix(lgh_ctx *ctx, size_t n, size_t k, size_t qs_bytes_per_block, M **out) {
  auto *w = new (std::nothrow) M();
  if (!w) return fail(ctx, LGH_ERR_OOM, "host allocation failed");
  w->device = ctx->device;
  w->n = n;
  w->k = k;
  w->bpr = k / 32;
  set_tiles(w);
  const size_t nb = n * w->bpr;
  const size_t qs_bytes = align_up(nb * qs_bytes_per_block);
  const size_t bytes = qs_bytes + align_up(nb * 2);
  void *p = nullptr;
  if (bytes) {
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
      delete w;
      return fail(ctx, LGH_ERR_OOM, "hipMalloc(%zu bytes) for weights failed: %s", bytes,
                  hipGetErrorString(e));
    }
  }
  w->qs = reinterpret_cast<decltype(w->qs)>(p);
  w->sc = reinterpret_cast<uint16_t *>(static_cast<char *>(p) + qs_bytes);
  *out = w;
  return LGH_OK;
}

void free_extra(lgh_q8 *) {}
void free_extra(lgh_q4 *w) {
  if (w->mx) (void)hipFree(w->mx);
}

template <class M>
void free_matrix(M *w) {
  if (!w) return;
  int cur = 0;
  (void)hipGetDevice(&cur);
  (void)hipSetDevice(w->device);
  if (w->qs) (void)hipFree(w->qs);
  free_extra(w);
  (void)hipSetDevice(cur);
  delete w;
}

// GEMM operand image of a Q4 matrix, built from its nibble/scale planes on
// the first call that routes the matrix to the GEMM (or by
// lgh_q4_prepare_gemm), so matrices that only ever serve decode GEMVs hold
// their 18 B per 32 weights and nothing more.  The image is a function of the
// immutable planes; the matrix's mutex makes the one-time build safe when
// contexts on several threads share the matrix, and the build waits for its
// pack kernel so every later user sees the finished image.  Matrices whose
// image would not fit 31-bit buffer offsets have none: the GEMV path serves
// them and the GEMM routes report LGH_ERR_SHAPE.
bool mx_fits(const lgh_q4 *w) {
  const size_t nt = (w->n + 31) / 32, pp = (w->bpr + 1) / 2;
  return nt * pp > 0 && (nt + 8) * pp * lgh::kMxWRec < lgh::kMxMaxBytes;
}

bool has_mx(const lgh_q4 *wc) {
  auto *w = const_cast<lgh_q4 *>(wc);
  std::lock_guard<std::mutex> lock(w->mx_mu);
  return w->mx != nullptr;
}

int ensure_mx(lgh_ctx *ctx, const lgh_q4 *wc) {
  auto *w = const_cast<lgh_q4 *>(wc);
  std::lock_guard<std::mutex> lock(w->mx_mu);
  if (w->mx) return LGH_OK;
  if (!mx_fits(w)) return fail(ctx, LGH_ERR_SHAPE, "%zu x %zu is too large for the GEMM path", w->n, w->k);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(ctx->stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
    return fail(ctx, LGH_ERR_CAPTURE,
                "the %zu x %zu matrix has no GEMM image yet and it cannot be built under stream capture; call "
                "lgh_q4_prepare_gemm first",
                w->n, w->k);
  const size_t bytes = w->nt * w->pp * lgh::kMxWRec;
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess)
    return fail(ctx, LGH_ERR_OOM, "hipMalloc(%zu bytes) for the GEMM operand image failed: %s", bytes,
                hipGetErrorString(e));
  lgh_q4 tmp;  // the pack launcher reads the shape and the destination from a matrix
  tmp.n = w->n;
  tmp.k = w->k;
  tmp.bpr = w->bpr;
  tmp.qs = w->qs;
  tmp.sc = w->sc;
  tmp.nt = w->nt;
  tmp.pp = w->pp;
  tmp.mx = static_cast<uint8_t *>(p);
  e = lgh::launch_q4_mx_pack(&tmp, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    (void)hipFree(p);
    return hip_fail(ctx, e, "GEMM image pack");
  }
  w->mx = static_cast<uint8_t *>(p);
  return LGH_OK;
}

// A matrix is used only through a context of the device that holds it.
template <class M>
int check_mat(lgh_ctx *ctx, const M *w) {
  if (!w) return fail(ctx, LGH_ERR_INVALID_ARG, "null matrix");
  if (w->device != ctx->device)
    return fail(ctx, LGH_ERR_INVALID_ARG, "the matrix is on device %d, the context on device %d", w->device,
                ctx->device);
  return LGH_OK;
}

int check_shape(lgh_ctx *ctx, const void *p, size_t n, size_t k, void *out) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (!out) return fail(ctx, LGH_ERR_INVALID_ARG, "null output handle");
  if (k % 32) return fail(ctx, LGH_ERR_SHAPE, "K=%zu is not a multiple of 32", k);
  if (n * k && !p) return fail(ctx, LGH_ERR_INVALID_ARG, "null weight pointer");
  return LGH_OK;
}

}  // namespace

extern "C" {

const char *lgh_version(void) { return "llm_gpu_hip 0.1.0 (gfx950, wave64)"; }

int lgh_init(int device, lgh_ctx **out) {
  if (!out) return fail(nullptr, LGH_ERR_INVALID_ARG, "null ctx out-pointer");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0)
    return fail(nullptr, LGH_ERR_NO_DEVICE, "no HIP device (%s)", hipGetErrorString(e));
  if (device < 0 || device >= count)
    return fail(nullptr, LGH_ERR_NO_DEVICE, "device %d out of range (count %d)", device, count);
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return fail(nullptr, LGH_ERR_HIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(nullptr, LGH_ERR_ARCH, "device %d is %s, this library is built for gfx950 only", device,
                prop.gcnArchName);
  auto *ctx = new (std::nothrow) lgh_ctx();
  if (!ctx) return fail(nullptr, LGH_ERR_OOM, "host allocation failed");
  ctx->device = device;
  ctx->cu_count = prop.multiProcessorCount;
  e = hipSetDevice(device);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return fail(nullptr, LGH_ERR_HIP, "stream creation failed: %s", hipGetErrorString(e));
  }
  ctx->stream = ctx->own_stream;
  if (device < kMaxDevices) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[device]) {
      void *p = nullptr;
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) {
        (void)hipStreamDestroy(ctx->own_stream);
        delete ctx;
        return fail(nullptr, LGH_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d failed: %s", device,
                    hipGetErrorString(e));
      }
      g_scratch[device] = p;
    }
    ctx->scratch = g_scratch[device];
  }
  *out = ctx;
  return LGH_OK;
}

void lgh_destroy(lgh_ctx *ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  if (ctx->ws) (void)hipFree(ctx->ws);
  if (ctx->stage) (void)hipFree(ctx->stage);
  if (ctx->ffn) (void)hipFree(ctx->ffn);
  if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
  delete ctx;
}

const char *lgh_last_error(const lgh_ctx *ctx) { return ctx ? ctx->err.c_str() : g_init_err.c_str(); }

int lgh_set_act_quant(lgh_ctx *ctx, int mode) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (mode != LGH_ACT_PER_BLOCK && mode != LGH_ACT_PER_ROW)
    return fail(ctx, LGH_ERR_INVALID_ARG, "unknown act-quant mode %d", mode);
  ctx->act_mode = mode;
  return LGH_OK;
}

int lgh_get_act_quant(const lgh_ctx *ctx) { return ctx ? ctx->act_mode : LGH_ERR_INVALID_ARG; }

int lgh_set_stream(lgh_ctx *ctx, void *hip_stream) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = set_device(ctx)) return r;
  // Work already queued may still read the workspaces: finish it first.
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  ctx->stream = hip_stream ? static_cast<hipStream_t>(hip_stream) : ctx->own_stream;
  return LGH_OK;
}

void *lgh_get_stream(const lgh_ctx *ctx) { return ctx ? static_cast<void *>(ctx->stream) : nullptr; }

int lgh_sync(lgh_ctx *ctx) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = set_device(ctx)) return r;
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

int lgh_trim(lgh_ctx *ctx) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = set_device(ctx)) return r;
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  release(ctx, &ctx->ws, &ctx->ws_bytes);
  release(ctx, &ctx->stage, &ctx->stage_bytes);
  release(ctx, &ctx->ffn, &ctx->ffn_bytes);
  return LGH_OK;
}

// ---- device buffers -----------------------------------------------------------
int lgh_buffer_alloc(lgh_ctx *ctx, size_t len, float **out) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (!out) return fail(ctx, LGH_ERR_INVALID_ARG, "null buffer out-pointer");
  *out = nullptr;
  if (len == 0) return LGH_OK;
  if (len > SIZE_MAX / sizeof(float)) return fail(ctx, LGH_ERR_SHAPE, "buffer of %zu floats is too large", len);
  if (int r = set_device(ctx)) return r;
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, len * sizeof(float));
  if (e != hipSuccess)
    return fail(ctx, LGH_ERR_OOM, "hipMalloc(%zu bytes) for a buffer failed: %s", len * sizeof(float),
                hipGetErrorString(e));
  e = hipMemsetAsync(p, 0, len * sizeof(float), ctx->stream);  // zeroed, as CpuBackend::alloc
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    (void)hipFree(p);
    return hip_fail(ctx, e, "buffer clear");
  }
  *out = static_cast<float *>(p);
  return LGH_OK;
}

void lgh_buffer_free(lgh_ctx *ctx, float *buf) {
  if (!ctx || !buf) return;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);  // queued work may still use it
  (void)hipFree(buf);
}

int lgh_buffer_write(lgh_ctx *ctx, float *dst_dev, const float *src, size_t len) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (len == 0) return LGH_OK;
  if (!dst_dev || !src) return fail(ctx, LGH_ERR_INVALID_ARG, "null buffer");
  if (len > SIZE_MAX / sizeof(float)) return fail(ctx, LGH_ERR_SHAPE, "buffer of %zu floats is too large", len);
  if (int r = set_device(ctx)) return r;
  LGH_HIP(ctx, hipMemcpyAsync(dst_dev, src, len * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

int lgh_buffer_read(lgh_ctx *ctx, float *dst, const float *src_dev, size_t len) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (len == 0) return LGH_OK;
  if (!dst || !src_dev) return fail(ctx, LGH_ERR_INVALID_ARG, "null buffer");
  if (len > SIZE_MAX / sizeof(float)) return fail(ctx, LGH_ERR_SHAPE, "buffer of %zu floats is too large", len);
  if (int r = set_device(ctx)) return r;
  LGH_HIP(ctx, hipMemcpyAsync(dst, src_dev, len * sizeof(float), hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

// ---- weights -------------------------------------------------------------
namespace {
// Wait for the repack of a fresh matrix (the GEMM image is built on first use).
int finish_q4(lgh_ctx *ctx, lgh_q4 *w, lgh_q4 **out) {
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    free_matrix(w);
    return hip_fail(ctx, e, "Q4 upload");
  }
  trim_stage(ctx);
  *out = w;
  return LGH_OK;
}
}  // namespace

int lgh_q4_upload_dev(lgh_ctx *ctx, const void *blocks_dev, size_t n, size_t k, lgh_q4 **out) {
  if (int r = check_shape(ctx, blocks_dev, n, k, out)) return r;
  if (int r = set_device(ctx)) return r;
  lgh_q4 *w = nullptr;
  if (int r = alloc_matrix(ctx, n, k, 16, &w)) return r;
  hipError_t e = lgh::launch_q4_repack(static_cast<const uint8_t *>(blocks_dev), n * w->bpr, w->qs, w->sc,
                                       ctx->stream);
  if (e != hipSuccess) {
    free_matrix(w);
    return hip_fail(ctx, e, "Q4 repack");
  }
  return finish_q4(ctx, w, out);
}

int lgh_q4_upload(lgh_ctx *ctx, const void *blocks, size_t n, size_t k, lgh_q4 **out) {
  if (int r = check_shape(ctx, blocks, n, k, out)) return r;
  if (int r = set_device(ctx)) return r;
  const size_t bytes = n * (k / 32) * LGH_BLOCK_Q4_BYTES;
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, bytes)) return r;
  if (bytes) LGH_HIP(ctx, hipMemcpyAsync(ctx->stage, blocks, bytes, hipMemcpyHostToDevice, ctx->stream));
  return lgh_q4_upload_dev(ctx, ctx->stage, n, k, out);
}

int lgh_q4_from_f32(lgh_ctx *ctx, const float *wf, size_t n, size_t k, lgh_q4 **out) {
  if (int r = check_shape(ctx, wf, n, k, out)) return r;
  if (int r = set_device(ctx)) return r;
  const size_t bytes = n * k * sizeof(float);
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, bytes)) return r;
  lgh_q4 *w = nullptr;
  if (int r = alloc_matrix(ctx, n, k, 16, &w)) return r;
  hipError_t e = bytes ? hipMemcpyAsync(ctx->stage, wf, bytes, hipMemcpyHostToDevice, ctx->stream) : hipSuccess;
  if (e == hipSuccess)
    e = lgh::launch_q4_quantize(static_cast<const float *>(ctx->stage), n * w->bpr, w->qs, w->sc, ctx->stream);
  if (e != hipSuccess) {
    free_matrix(w);
    return hip_fail(ctx, e, "Q4 quantize");
  }
  return finish_q4(ctx, w, out);
}

int lgh_q4_download(lgh_ctx *ctx, const lgh_q4 *w, void *blocks) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w)) return r;
  if (!blocks) return fail(ctx, LGH_ERR_INVALID_ARG, "null destination");
  if (int r = set_device(ctx)) return r;
  const size_t nb = w->n * w->bpr, bytes = nb * LGH_BLOCK_Q4_BYTES;
  if (!bytes) return LGH_OK;
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, bytes)) return r;
  LGH_HIP(ctx, lgh::launch_q4_unpack(w->qs, w->sc, nb, static_cast<uint8_t *>(ctx->stage), ctx->stream));
  LGH_HIP(ctx, hipMemcpyAsync(blocks, ctx->stage, bytes, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

// ---- device images: the matrix as it sits in HBM, for a load that is one copy ----
uint32_t lgh_image_layout(void) { return lgh::kImageLayout; }

size_t lgh_q4_image_bytes(const lgh_q4 *w, int with_gemm) {
  if (!w) return 0;
  const size_t nb = w->n * w->bpr;
  return nb * 18 + (with_gemm ? w->nt * w->pp * lgh::kMxWRec : 0);
}

int lgh_q4_export(lgh_ctx *ctx, const lgh_q4 *w, int with_gemm, void *dst, size_t bytes) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w)) return r;
  if (bytes != lgh_q4_image_bytes(w, with_gemm))
    return fail(ctx, LGH_ERR_SHAPE, "image of %zu x %zu needs %zu bytes, got %zu", w->n, w->k,
                lgh_q4_image_bytes(w, with_gemm), bytes);
  if (bytes == 0) return LGH_OK;
  if (!dst) return fail(ctx, LGH_ERR_INVALID_ARG, "null destination");
  if (int r = set_device(ctx)) return r;
  const size_t nb = w->n * w->bpr;
  char *d = static_cast<char *>(dst);
  if (with_gemm)
    if (int r = ensure_mx(ctx, w)) return r;
  LGH_HIP(ctx, hipMemcpyAsync(d, w->qs, nb * 16, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipMemcpyAsync(d + nb * 16, w->sc, nb * 2, hipMemcpyDeviceToHost, ctx->stream));
  if (with_gemm)
    LGH_HIP(ctx, hipMemcpyAsync(d + nb * 18, w->mx, w->nt * w->pp * lgh::kMxWRec, hipMemcpyDeviceToHost,
                                ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

int lgh_q4_import(lgh_ctx *ctx, const void *src, size_t bytes, size_t n, size_t k, int with_gemm, lgh_q4 **out) {
  if (int r = check_shape(ctx, src, n, k, out)) return r;
  *out = nullptr;
  if (int r = set_device(ctx)) return r;
  lgh_q4 *w = nullptr;
  if (int r = alloc_matrix(ctx, n, k, 16, &w)) return r;
  if (with_gemm && !mx_fits(w) && n * w->bpr) {
    free_matrix(w);
    return fail(ctx, LGH_ERR_SHAPE, "%zu x %zu has no GEMM image (too large for the GEMM path)", n, k);
  }
  const size_t need = lgh_q4_image_bytes(w, with_gemm), nb = n * w->bpr;
  if (bytes != need) {
    free_matrix(w);
    return fail(ctx, LGH_ERR_SHAPE, "image of %zu x %zu needs %zu bytes, got %zu", n, k, need, bytes);
  }
  const char *s = static_cast<const char *>(src);
  hipError_t e = hipSuccess;
  if (nb) e = hipMemcpyAsync(w->qs, s, nb * 16, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess && nb) e = hipMemcpyAsync(w->sc, s + nb * 16, nb * 2, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess && with_gemm && nb) {
    void *p = nullptr;
    const size_t mb = w->nt * w->pp * lgh::kMxWRec;
    e = hipMalloc(&p, mb);
    if (e == hipSuccess) {
      w->mx = static_cast<uint8_t *>(p);
      e = hipMemcpyAsync(w->mx, s + nb * 18, mb, hipMemcpyHostToDevice, ctx->stream);
    }
  }
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    free_matrix(w);
    return hip_fail(ctx, e, "Q4 image import");
  }
  *out = w;
  return LGH_OK;
}

size_t lgh_q8_image_bytes(const lgh_q8 *w) { return w ? w->n * w->bpr * LGH_BLOCK_Q8_BYTES : 0; }

int lgh_q8_export(lgh_ctx *ctx, const lgh_q8 *w, void *dst, size_t bytes) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w)) return r;
  if (bytes != lgh_q8_image_bytes(w))
    return fail(ctx, LGH_ERR_SHAPE, "image needs %zu bytes, got %zu", lgh_q8_image_bytes(w), bytes);
  if (bytes == 0) return LGH_OK;
  if (!dst) return fail(ctx, LGH_ERR_INVALID_ARG, "null destination");
  if (int r = set_device(ctx)) return r;
  const size_t nb = w->n * w->bpr;
  char *d = static_cast<char *>(dst);
  LGH_HIP(ctx, hipMemcpyAsync(d, w->qs, nb * 32, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipMemcpyAsync(d + nb * 32, w->sc, nb * 2, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

int lgh_q8_import(lgh_ctx *ctx, const void *src, size_t bytes, size_t n, size_t k, lgh_q8 **out) {
  if (int r = check_shape(ctx, src, n, k, out)) return r;
  *out = nullptr;
  const size_t nb = n * (k / 32);
  if (bytes != nb * LGH_BLOCK_Q8_BYTES)
    return fail(ctx, LGH_ERR_SHAPE, "image of %zu x %zu needs %zu bytes, got %zu", n, k, nb * LGH_BLOCK_Q8_BYTES,
                bytes);
  if (int r = set_device(ctx)) return r;
  lgh_q8 *w = nullptr;
  if (int r = alloc_matrix(ctx, n, k, 32, &w)) return r;
  const char *s = static_cast<const char *>(src);
  hipError_t e = hipSuccess;
  if (nb) e = hipMemcpyAsync(w->qs, s, nb * 32, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess && nb) e = hipMemcpyAsync(w->sc, s + nb * 32, nb * 2, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    free_matrix(w);
    return hip_fail(ctx, e, "Q8 image import");
  }
  *out = w;
  return LGH_OK;
}

int lgh_q4_prepare_gemm(lgh_ctx *ctx, const lgh_q4 *w) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w)) return r;
  if (w->n == 0 || w->bpr == 0) return LGH_OK;
  if (int r = set_device(ctx)) return r;
  return ensure_mx(ctx, w);
}

size_t lgh_q4_device_bytes(const lgh_q4 *w) {
  if (!w) return 0;
  const size_t nb = w->n * w->bpr;
  return align_up(nb * 16) + align_up(nb * 2) + (has_mx(w) ? w->nt * w->pp * lgh::kMxWRec : 0);
}

void lgh_q4_free(lgh_q4 *w) { free_matrix(w); }
size_t lgh_q4_rows(const lgh_q4 *w) { return w ? w->n : 0; }
size_t lgh_q4_cols(const lgh_q4 *w) { return w ? w->k : 0; }

int lgh_q8_upload(lgh_ctx *ctx, const void *blocks, size_t n, size_t k, lgh_q8 **out) {
  if (int r = check_shape(ctx, blocks, n, k, out)) return r;
  if (int r = set_device(ctx)) return r;
  const size_t nb = n * (k / 32), bytes = nb * LGH_BLOCK_Q8_BYTES;
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, bytes)) return r;
  lgh_q8 *w = nullptr;
  if (int r = alloc_matrix(ctx, n, k, 32, &w)) return r;
  hipError_t e = bytes ? hipMemcpyAsync(ctx->stage, blocks, bytes, hipMemcpyHostToDevice, ctx->stream) : hipSuccess;
  if (e == hipSuccess)
    e = lgh::launch_q8_repack(static_cast<const uint8_t *>(ctx->stage), nb, w->qs, w->sc, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    free_matrix(w);
    return hip_fail(ctx, e, "Q8 upload");
  }
  trim_stage(ctx);
  *out = w;
  return LGH_OK;
}

int lgh_q8_from_f32(lgh_ctx *ctx, const float *wf, size_t n, size_t k, lgh_q8 **out) {
  if (int r = check_shape(ctx, wf, n, k, out)) return r;
  if (int r = set_device(ctx)) return r;
  const size_t bytes = n * k * sizeof(float);
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, bytes)) return r;
  lgh_q8 *w = nullptr;
  if (int r = alloc_matrix(ctx, n, k, 32, &w)) return r;
  hipError_t e = bytes ? hipMemcpyAsync(ctx->stage, wf, bytes, hipMemcpyHostToDevice, ctx->stream) : hipSuccess;
  if (e == hipSuccess)
    e = lgh::launch_q8_quantize(static_cast<const float *>(ctx->stage), n * w->bpr, w->qs, w->sc, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    free_matrix(w);
    return hip_fail(ctx, e, "Q8 quantize");
  }
  trim_stage(ctx);
  *out = w;
  return LGH_OK;
}

int lgh_q8_download(lgh_ctx *ctx, const lgh_q8 *w, void *blocks) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w)) return r;
  if (!blocks) return fail(ctx, LGH_ERR_INVALID_ARG, "null destination");
  if (int r = set_device(ctx)) return r;
  const size_t nb = w->n * w->bpr, bytes = nb * LGH_BLOCK_Q8_BYTES;
  if (!bytes) return LGH_OK;
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, bytes)) return r;
  LGH_HIP(ctx, lgh::launch_q8_unpack(w->qs, w->sc, nb, static_cast<uint8_t *>(ctx->stage), ctx->stream));
  LGH_HIP(ctx, hipMemcpyAsync(blocks, ctx->stage, bytes, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

void lgh_q8_free(lgh_q8 *w) { free_matrix(w); }
size_t lgh_q8_rows(const lgh_q8 *w) { return w ? w->n : 0; }
size_t lgh_q8_cols(const lgh_q8 *w) { return w ? w->k : 0; }

// ---- device-pointer entry points -------------------------------------------
static int check_mode(lgh_ctx *ctx, int mode) {
  if (mode != LGH_ASSIGN && mode != LGH_ADD_F64 && mode != LGH_ADD_F32)
    return fail(ctx, LGH_ERR_INVALID_ARG, "unknown accumulation mode %d", mode);
  return LGH_OK;
}

// The activation rows a GEMM call quantizes: x itself, rms_norm(x, nw, eps)
// (nw not null) or silu(x) * u (u not null).  Routes whose activation image
// has a fused form build it from x directly; the others first write the rows
// to tmp ([m][k] f32; for silu tmp is x itself, overwritten in place as the
// op sequence's silu_mul does).
struct ActIn {
  const float *x;
  const float *nw = nullptr;
  float eps = 0.0f;
  const float *u = nullptr;
  float *tmp = nullptr;
};

static int gemm_multi_dev(lgh_ctx *ctx, const Ws &wsp, const lgh_q4 *const *w, int nmat, ActIn in,
                          float *const *y_dev, size_t m, int mode);
static int mma_chunked(lgh_ctx *ctx, const Ws &wsp, const lgh_q4 *const *w, int nmat, const float *x_dev,
                       const int8_t *codes_dev, const float *scales_dev, float *const *y_dev, size_t m, int mode);

static int launch_gemv(lgh_ctx *ctx, const Ws &wsp, const lgh_q4 *w0, float *y0, const lgh_q4 *w1, float *y1,
                       const float *x, int mode) {
  if (!lgh::plan_q4_gemv(w0->n, w0->bpr, w1 ? 2 : 1).ok) {
    // K longer than the GEMV covers: batched act-quant + GEMM with m = 1.
    if (int r = gemm_multi_dev(ctx, wsp, &w0, 1, ActIn{x}, &y0, 1, mode)) return r;
    return w1 ? gemm_multi_dev(ctx, wsp, &w1, 1, ActIn{x}, &y1, 1, mode) : LGH_OK;
  }
  if (int r = set_device(ctx)) return r;
  if (lgh::q4_gemv_quantize_once(w0->n, w0->bpr, w1 ? 2 : 1)) {
    Carve cv;
    const size_t oq = cv.take(w0->k), os = cv.take(w0->bpr * sizeof(float)), orow = cv.take(sizeof(float));
    char *ws = nullptr;
    if (int r = wsp.get(cv.off, &ws)) return r;
    auto *qs = reinterpret_cast<int8_t *>(ws + oq);
    auto *sc = reinterpret_cast<float *>(ws + os);
    LGH_HIP(ctx, lgh::launch_act_quant(x, 1, w0->k, ctx->act_mode, qs, sc, nullptr,
                                       reinterpret_cast<float *>(ws + orow), ctx->stream));
    LGH_HIP(ctx, lgh::launch_q4_gemv_any(w0, y0, w1, y1, nullptr, qs, sc, mode, 0, ctx->stream));
    return LGH_OK;
  }
  LGH_HIP(ctx, lgh::launch_q4_gemv(w0, y0, w1, y1, x, mode, ctx->act_mode, ctx->stream));
  return LGH_OK;
}

int lgh_q4_gemv_dev(lgh_ctx *ctx, const lgh_q4 *w, const float *x_dev, float *y_dev, int mode) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w)) return r;
  if (int r = check_mode(ctx, mode)) return r;
  if (w->n == 0) return LGH_OK;
  if (!y_dev || (w->k && !x_dev)) return fail(ctx, LGH_ERR_INVALID_ARG, "null x/y");
  if (!aligned16(x_dev)) return fail(ctx, LGH_ERR_INVALID_ARG, "x must be 16-byte aligned");
  return launch_gemv(ctx, grow_ws(ctx), w, y_dev, nullptr, nullptr, x_dev, mode);
}

int lgh_q4_gemv_pair_dev(lgh_ctx *ctx, const lgh_q4 *wg, const lgh_q4 *wu, const float *x_dev, float *yg_dev,
                         float *yu_dev) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, wg)) return r;
  if (int r = check_mat(ctx, wu)) return r;
  if (wg->k != wu->k || wg->n != wu->n)
    return fail(ctx, LGH_ERR_SHAPE, "pair needs equal shapes: gate %zux%zu, up %zux%zu", wg->n, wg->k, wu->n,
                wu->k);
  if (wg->n == 0) return LGH_OK;
  if (!yg_dev || !yu_dev || (wg->k && !x_dev)) return fail(ctx, LGH_ERR_INVALID_ARG, "null x/y");
  if (!aligned16(x_dev)) return fail(ctx, LGH_ERR_INVALID_ARG, "x must be 16-byte aligned");
  return launch_gemv(ctx, grow_ws(ctx), wg, yg_dev, wu, yu_dev, x_dev, LGH_ASSIGN);
}

// gemv_q4_prep / gemv_q4_prep_add: the GEMV kernel reads ActQ8 codes and
// block scales (either act-quant mode) instead of loading and quantizing x.
int lgh_q4_gemv_prep_dev(lgh_ctx *ctx, const lgh_q4 *w, const int8_t *qs_dev, const float *scales_dev,
                         float *y_dev, int mode) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w)) return r;
  if (int r = check_mode(ctx, mode)) return r;
  if (w->n == 0) return LGH_OK;
  if (!y_dev || (w->k && (!qs_dev || !scales_dev))) return fail(ctx, LGH_ERR_INVALID_ARG, "null codes/scales/y");
  if (!aligned16(qs_dev) || (reinterpret_cast<uintptr_t>(scales_dev) & 3u))
    return fail(ctx, LGH_ERR_INVALID_ARG, "codes must be 16-byte and scales 4-byte aligned");
  if (int r = set_device(ctx)) return r;
  if (!lgh::plan_q4_gemv(w->n, w->bpr, 1).ok) {
    // K > 32768: the codes and scales become the GEMM's activation image (one token), and the
    // GEMM folds every block as the GEMV does.
    if (!mx_fits(w)) {
      float *ys[1] = {y_dev};
      return mma_chunked(ctx, grow_ws(ctx), &w, 1, nullptr, qs_dev, scales_dev, ys, 1, mode);
    }
    if (int r = ensure_mx(ctx, w)) return r;
    const lgh_q4 *ws1[1] = {w};
    const lgh::GemmPlan plan = lgh::plan_q4_gemm(ws1, 1, 1);
    const size_t part_floats = plan.splits > 1 ? static_cast<size_t>(plan.splits) * w->n : 0;
    Carve cv;
    const size_t o_mx = cv.take(w->pp * lgh::kMxARec), o_part = cv.take(part_floats * sizeof(float));
    char *ws = nullptr;
    if (int r = grow_ws(ctx).get(cv.off, &ws)) return r;
    auto *mxa = reinterpret_cast<uint8_t *>(ws + o_mx);
    LGH_HIP(ctx, lgh::launch_act_split_mx(qs_dev, scales_dev, 1, w->k, mxa, ctx->stream));
    float *ys[1] = {y_dev};
    LGH_HIP(ctx, lgh::launch_q4_gemm(ws1, 1, mxa, ys, 1, mode, plan, reinterpret_cast<float *>(ws + o_part),
                                     part_floats, ctx->stream));
    return LGH_OK;
  }
  LGH_HIP(ctx, lgh::launch_q4_gemv_codes(w, qs_dev, scales_dev, y_dev, mode, ctx->stream));
  return LGH_OK;
}

int lgh_q4_gemv_prep(lgh_ctx *ctx, const lgh_q4 *w, const int8_t *qs, const float *scales, float *y, int mode) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w)) return r;
  if (int r = check_mode(ctx, mode)) return r;
  if (w->n == 0) return LGH_OK;
  if (!y || (w->k && (!qs || !scales))) return fail(ctx, LGH_ERR_INVALID_ARG, "null codes/scales/y");
  if (int r = set_device(ctx)) return r;
  Carve cv;
  const size_t qb = w->k, sb = w->bpr * sizeof(float), yb = w->n * sizeof(float);
  const size_t oq = cv.take(qb), os = cv.take(sb), oy = cv.take(yb);
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, cv.off)) return r;
  char *st = static_cast<char *>(ctx->stage);
  auto *qd = reinterpret_cast<int8_t *>(st + oq);
  auto *sd = reinterpret_cast<float *>(st + os);
  auto *yd = reinterpret_cast<float *>(st + oy);
  if (qb) LGH_HIP(ctx, hipMemcpyAsync(qd, qs, qb, hipMemcpyHostToDevice, ctx->stream));
  if (sb) LGH_HIP(ctx, hipMemcpyAsync(sd, scales, sb, hipMemcpyHostToDevice, ctx->stream));
  if (mode != LGH_ASSIGN) LGH_HIP(ctx, hipMemcpyAsync(yd, y, yb, hipMemcpyHostToDevice, ctx->stream));
  if (int r = lgh_q4_gemv_prep_dev(ctx, w, qd, sd, yd, mode)) return r;
  LGH_HIP(ctx, hipMemcpyAsync(y, yd, yb, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

// ActQ8::quantize_into / quantize_row_into over m rows, device to device; the
// PerRow row scales go through the GEMM workspace.
int lgh_act_quant_dev(lgh_ctx *ctx, const float *x_dev, size_t m, size_t k, int8_t *qs_dev, float *scales_dev,
                      int32_t *sums_dev) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (k % 32) return fail(ctx, LGH_ERR_SHAPE, "activation length %zu is not a multiple of 32", k);
  if (m == 0 || k == 0) return LGH_OK;
  if (!x_dev || !qs_dev || !scales_dev) return fail(ctx, LGH_ERR_INVALID_ARG, "null argument");
  if (!aligned16(x_dev) || (reinterpret_cast<uintptr_t>(qs_dev) & 3u) ||
      (reinterpret_cast<uintptr_t>(scales_dev) & 3u) || (reinterpret_cast<uintptr_t>(sums_dev) & 3u))
    return fail(ctx, LGH_ERR_INVALID_ARG, "x must be 16-byte and codes, scales, sums 4-byte aligned");
  if (int r = set_device(ctx)) return r;
  float *row_scale = nullptr;
  if (ctx->act_mode == LGH_ACT_PER_ROW) {
    if (int r = ensure(ctx, &ctx->ws, &ctx->ws_bytes, m * sizeof(float))) return r;
    row_scale = static_cast<float *>(ctx->ws);
  }
  LGH_HIP(ctx, lgh::launch_act_quant(x_dev, m, k, ctx->act_mode, qs_dev, scales_dev, sums_dev, row_scale,
                                     ctx->stream));
  return LGH_OK;
}

// Matrices whose GEMM image would not fit 31-bit buffer offsets (over 2 GiB,
// ~2.4e9 weights) have none.  Their calls that would take the GEMM (m >= 65,
// long rows at m >= 49, m == 1 with k > 32768) run the matrix-core batch
// kernel on the nibble planes instead, up to 64 tokens per launch.  With
// codes_dev / scales_dev (ActQ8 codes and block scales of the m rows) the
// image is built from them instead of from x.
static int mma_chunked(lgh_ctx *ctx, const Ws &wsp, const lgh_q4 *const *w, int nmat, const float *x_dev,
                       const int8_t *codes_dev, const float *scales_dev, float *const *y_dev, size_t m, int mode) {
  const size_t k = w[0]->k, bpr = w[0]->bpr, pq = (bpr + 3) / 4;
  struct Layout {
    size_t o_ci, o_si, o_rs, bytes;
  };
  auto layout = [&](size_t c) {
    const size_t mt = (c + 15) / 16;
    Layout l{};
    Carve cv;
    l.o_ci = cv.take(mt * pq * 2 * 1024);
    l.o_si = cv.take(mt * pq * 256);
    l.o_rs = cv.take(c * sizeof(float));
    l.bytes = cv.off;
    return l;
  };
  // 64 tokens per launch whatever the scratch: the kernel's plan (token
  // tiles, K slices) depends on the chunk, so a smaller chunk could change
  // the f32 summation order.  A fixed scratch too small for the chunk's image
  // fails in wsp.get.
  const size_t chunk = std::min<size_t>(m, 64);
  const Layout lay = layout(chunk);
  char *ws = nullptr;
  if (int r = wsp.get(lay.bytes, &ws)) return r;
  auto *ci = reinterpret_cast<uint8_t *>(ws + lay.o_ci);
  auto *si = reinterpret_cast<float *>(ws + lay.o_si);
  for (size_t m0 = 0; m0 < m; m0 += chunk) {
    const size_t mc = std::min(chunk, m - m0);
    if (codes_dev)
      LGH_HIP(ctx, lgh::launch_act_codes_mma(codes_dev + m0 * k, scales_dev + m0 * bpr, mc, k, ci, si, ctx->stream));
    else
      LGH_HIP(ctx, lgh::launch_act_quant_mma(x_dev + m0 * k, lgh::ActPrologue{}, mc, k, ctx->act_mode, ci, si,
                                             reinterpret_cast<float *>(ws + lay.o_rs), ctx->stream));
    for (int j = 0; j < nmat; j++)
      if (w[j]->n)
        LGH_HIP(ctx, lgh::launch_q4_gemv_mma(w[j], ci, si, y_dev[j] + m0 * w[j]->n, mc, mode, ctx->stream, true));
  }
  return LGH_OK;
}

// Write the transformed activation rows of `in` to in.tmp (rms_norm or silu * u,
// the op sequence's kernels) and return them; plain rows are returned as they are.
static int materialize(lgh_ctx *ctx, const ActIn &in, size_t m, size_t k, const float **rows) {
  *rows = in.x;
  if (!in.nw && !in.u) return LGH_OK;
  if (!in.tmp || (in.u && in.tmp != in.x))
    return fail(ctx, LGH_ERR_INVALID_ARG, "no buffer for the transformed activation rows");
  if (in.nw)
    LGH_HIP(ctx, lgh::launch_rms_norm(in.x, in.nw, k, m, in.eps, in.tmp, ctx->stream));
  else
    LGH_HIP(ctx, lgh::launch_silu_mul(in.tmp, in.u, m * k, ctx->stream));
  *rows = in.tmp;
  return LGH_OK;
}

// y[j] = x @ W[j]^T for 1..3 matrices with the same k, m rows of x: the
// activation quantization of each route (the MMA image, the GEMM's operand
// image) is done once and read by every matrix.  m == 1 and m <= 4 quantize
// inside their kernels, per matrix.  The rows may be rms_norm(x) or
// silu(x) * u (ActIn): the MMA and GEMM routes form them in the launch that
// writes their activation image (the normed rows are never written), the
// others after one more launch that writes them out.
static int gemm_multi_dev(lgh_ctx *ctx, const Ws &wsp, const lgh_q4 *const *w, int nmat, ActIn in,
                          float *const *y_dev, size_t m, int mode) {
  const size_t k = w[0]->k, bpr = w[0]->bpr;
  size_t nmax = 0;
  for (int j = 0; j < nmat; j++) nmax = std::max(nmax, w[j]->n);
  if (m == 0 || nmax == 0) return LGH_OK;
  if (!aligned16(in.x) || !aligned16(in.u) || !aligned16(in.nw))
    return fail(ctx, LGH_ERR_INVALID_ARG, "activation rows must be 16-byte aligned");
  // The image launch's elementwise step: silu(x) * u, or rms_norm.
  lgh::ActPrologue pro;
  pro.u = in.nw ? nullptr : in.u;
  pro.nw = in.nw;
  pro.eps = in.eps;
  const float *x_dev = in.x;
  if (m == 1 && lgh::plan_q4_gemv(nmax, bpr, 1).ok) {
    if (int r = materialize(ctx, in, m, k, &x_dev)) return r;
    for (int j = 0; j < nmat; j++)
      if (w[j]->n)
        if (int r = launch_gemv(ctx, wsp, w[j], y_dev[j], nullptr, nullptr, x_dev, mode)) return r;
    return LGH_OK;
  }
  if (int r = set_device(ctx)) return r;
  // Small batches are weight-stream bound: nibble planes, no operand image.
  if (lgh::plan_q4_batch(m, bpr).ok) {  // m <= 4: dot4 on the nibble planes
    if (int r = materialize(ctx, in, m, k, &x_dev)) return r;
    if (lgh::q4_batch_quantize_once(bpr)) {  // long rows: x quantized once, shared by every matrix
      Carve cv;
      const size_t oq = cv.take(m * k), os = cv.take(m * bpr * sizeof(float)), orow = cv.take(m * sizeof(float));
      char *ws = nullptr;
      if (int r = wsp.get(cv.off, &ws)) return r;
      auto *qs = reinterpret_cast<int8_t *>(ws + oq);
      auto *sc = reinterpret_cast<float *>(ws + os);
      LGH_HIP(ctx, lgh::launch_act_quant(x_dev, m, k, ctx->act_mode, qs, sc, nullptr,
                                         reinterpret_cast<float *>(ws + orow), ctx->stream));
      for (int j = 0; j < nmat; j++)
        LGH_HIP(ctx, lgh::launch_q4_gemv_batch(w[j], nullptr, qs, sc, y_dev[j], m, mode, 0, ctx->stream));
      return LGH_OK;
    }
    for (int j = 0; j < nmat; j++)  // x quantized inside the kernel
      LGH_HIP(ctx, lgh::launch_q4_gemv_batch(w[j], x_dev, nullptr, nullptr, y_dev[j], m, mode, ctx->act_mode,
                                             ctx->stream));
    return LGH_OK;
  }
  if (lgh::plan_q4_mma(nmax, m, bpr).ok) {  // m <= 64: activation image, then int8 MFMA per block
    const size_t mt = (m + 15) / 16, pq = (bpr + 3) / 4;
    Carve cv;
    const size_t o_ci = cv.take(mt * pq * 2 * 1024), o_si = cv.take(mt * pq * 256);
    const size_t o_rs = cv.take(m * sizeof(float));
    char *ws = nullptr;
    if (int r = wsp.get(cv.off, &ws)) return r;
    auto *ci = reinterpret_cast<uint8_t *>(ws + o_ci);
    auto *si = reinterpret_cast<float *>(ws + o_si);
    LGH_HIP(ctx, lgh::launch_act_quant_mma(x_dev, pro, m, k, ctx->act_mode, ci, si,
                                           reinterpret_cast<float *>(ws + o_rs), ctx->stream));
    for (int j = 0; j < nmat; j++)
      if (w[j]->n) LGH_HIP(ctx, lgh::launch_q4_gemv_mma(w[j], ci, si, y_dev[j], m, mode, ctx->stream));
    return LGH_OK;
  }
  for (int j = 0; j < nmat; j++)
    if (w[j]->n && !mx_fits(w[j])) {
      if (int r = materialize(ctx, in, m, k, &x_dev)) return r;
      return mma_chunked(ctx, wsp, w, nmat, x_dev, nullptr, nullptr, y_dev, m, mode);
    }
  for (int j = 0; j < nmat; j++) {
    if (!w[j]->n) continue;
    if (wsp.fixed) {  // building the image allocates
      if (!has_mx(w[j]))
        return fail(ctx, LGH_ERR_INVALID_ARG,
                    "the %zu x %zu matrix has no GEMM image; call lgh_q4_prepare_gemm before this call", w[j]->n,
                    w[j]->k);
    } else if (int r = ensure_mx(ctx, w[j])) {
      return r;
    }
  }
  // Tokens per launch: the activation image must fit 31-bit buffer offsets,
  // and the chunk's scratch (image, row scales, split-K partials) must fit
  // the fixed scratch when the call may not allocate.
  const size_t pp = (bpr + 1) / 2;
  const size_t rec_per_tile = pp * lgh::kMxARec;
  const size_t cap_tiles = lgh::kMxMaxBytes / rec_per_tile;
  if (cap_tiles <= 8) return fail(ctx, LGH_ERR_SHAPE, "K=%zu is too long for the GEMM path", k);
  size_t rows = 0;
  for (int j = 0; j < nmat; j++) rows += w[j]->n;
  // The plan (K splits and K groups) sets the order of the f32 additions, so
  // it is made once, for the token chunk the allocating path takes, and kept
  // when the fixed scratch forces smaller chunks: chunking changes only the
  // scratch footprint, never the result.
  const size_t chunk0 = std::min(m, (cap_tiles - 8) * 32);
  const lgh::GemmPlan plan = lgh::plan_q4_gemm(w, nmat, chunk0);
  const int splits = plan.splits;
  struct Layout {
    size_t part_floats, o_mx, o_rs, o_part, bytes;
  };
  auto layout = [&](size_t c) {
    Layout l{};
    l.part_floats = splits > 1 ? static_cast<size_t>(splits) * c * rows : 0;
    Carve cv;
    l.o_mx = cv.take((c + 31) / 32 * rec_per_tile);
    l.o_rs = cv.take(c * sizeof(float));
    l.o_part = cv.take(l.part_floats * sizeof(float));
    l.bytes = cv.off;
    return l;
  };
  size_t chunk = chunk0;
  Layout lay = layout(chunk);
  while (lay.bytes > wsp.limit() && chunk > 32) {  // halve, in whole 32-token tiles
    chunk = std::max<size_t>(32, (chunk / 2 + 31) / 32 * 32);
    lay = layout(chunk);
  }
  const size_t part_floats = lay.part_floats, o_mx = lay.o_mx, o_rs = lay.o_rs, o_part = lay.o_part;
  char *ws = nullptr;
  if (int r = wsp.get(lay.bytes, &ws)) return r;
  auto *mxa = reinterpret_cast<uint8_t *>(ws + o_mx);
  auto *rs = reinterpret_cast<float *>(ws + o_rs);
  auto *part = reinterpret_cast<float *>(ws + o_part);
  for (size_t m0 = 0; m0 < m; m0 += chunk) {
    const size_t mc = std::min(chunk, m - m0);
    float *yc[3] = {nullptr, nullptr, nullptr};
    for (int j = 0; j < nmat; j++) yc[j] = w[j]->n ? y_dev[j] + m0 * w[j]->n : nullptr;
    lgh::ActPrologue pc = pro;
    if (pc.u) pc.u += m0 * k;
    LGH_HIP(ctx, lgh::launch_act_quant_mx(x_dev + m0 * k, pc, mc, k, ctx->act_mode, mxa, rs, ctx->stream));
    LGH_HIP(ctx, lgh::launch_q4_gemm(w, nmat, mxa, yc, mc, mode, plan, part, part_floats, ctx->stream));
  }
  return LGH_OK;
}

int lgh_q4_gemm_dev(lgh_ctx *ctx, const lgh_q4 *w, const float *x_dev, float *y_dev, size_t m, int mode) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w)) return r;
  if (int r = check_mode(ctx, mode)) return r;
  if (m == 0 || w->n == 0) return LGH_OK;
  if (!y_dev || (w->k && !x_dev)) return fail(ctx, LGH_ERR_INVALID_ARG, "null x/y");
  return gemm_multi_dev(ctx, grow_ws(ctx), &w, 1, ActIn{x_dev}, &y_dev, m, mode);
}

// lgh_q4_gemm_dev with every scratch buffer taken from the device's fixed
// scratch array instead of the context workspace: no allocation, no free, no
// synchronisation.  On the GEMM route (65+ tokens) token chunks shrink until
// their scratch fits, with the plan of the whole call; a call that
// needs more than the array holds even for 32 tokens, or whose route takes
// its scratch in one piece (1-64 tokens), fails with LGH_ERR_SHAPE.
int lgh_q4_gemm_dev_noalloc(lgh_ctx *ctx, const lgh_q4 *w, const float *x_dev, float *y_dev, size_t m, int mode) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w)) return r;
  if (int r = check_mode(ctx, mode)) return r;
  if (m == 0 || w->n == 0) return LGH_OK;
  if (!y_dev || (w->k && !x_dev)) return fail(ctx, LGH_ERR_INVALID_ARG, "null x/y");
  if (!ctx->scratch) return fail(ctx, LGH_ERR_INVALID_ARG, "device %d has no fixed scratch", ctx->device);
  const Ws fixed{ctx, static_cast<char *>(ctx->scratch), LGH_NOALLOC_SCRATCH_BYTES};
  return gemm_multi_dev(ctx, fixed, &w, 1, ActIn{x_dev}, &y_dev, m, mode);
}

// ---- measurement probes ------------------------------------------------------------
int lgh_probe_empty_dev(lgh_ctx *ctx, int workgroups) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (workgroups < 1 || workgroups > 65535)
    return fail(ctx, LGH_ERR_INVALID_ARG, "workgroups %d outside 1..65535", workgroups);
  if (int r = set_device(ctx)) return r;
  LGH_HIP(ctx, lgh::launch_probe_empty(workgroups, ctx->stream));
  return LGH_OK;
}

size_t lgh_probe_read_outputs(size_t bytes, int per_thread) {
  if (per_thread != 1 && per_thread != 2 && per_thread != 4 && per_thread != 8) return 0;
  return lgh::probe_read_workgroups(bytes, per_thread);
}

int lgh_probe_read_dev(lgh_ctx *ctx, const void *src_dev, size_t bytes, int per_thread, float *out_dev) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (per_thread != 1 && per_thread != 2 && per_thread != 4 && per_thread != 8)
    return fail(ctx, LGH_ERR_INVALID_ARG, "per_thread %d is not 1, 2, 4 or 8", per_thread);
  if (bytes % 16) return fail(ctx, LGH_ERR_SHAPE, "%zu bytes is not a multiple of 16", bytes);
  if (bytes == 0) return LGH_OK;
  if (!src_dev || !out_dev) return fail(ctx, LGH_ERR_INVALID_ARG, "null source or output");
  if (!aligned16(src_dev) || (reinterpret_cast<uintptr_t>(out_dev) & 3u))
    return fail(ctx, LGH_ERR_INVALID_ARG, "source must be 16-byte and output 4-byte aligned");
  if (bytes >= (size_t{1} << 31)) return fail(ctx, LGH_ERR_SHAPE, "%zu bytes: the probe reads < 2 GiB", bytes);
  if (int r = set_device(ctx)) return r;
  LGH_HIP(ctx, lgh::launch_probe_read(src_dev, bytes, per_thread, out_dev, ctx->stream));
  return LGH_OK;
}

int lgh_q8_gemv_dev(lgh_ctx *ctx, const lgh_q8 *w, const float *x_dev, float *y_dev, size_t tokens) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w)) return r;
  if (tokens == 0 || w->n == 0) return LGH_OK;
  if (!y_dev || (w->k && !x_dev)) return fail(ctx, LGH_ERR_INVALID_ARG, "null x/y");
  if (!aligned16(x_dev)) return fail(ctx, LGH_ERR_INVALID_ARG, "x must be 16-byte aligned");
  if (int r = set_device(ctx)) return r;
  LGH_HIP(ctx, lgh::launch_q8_gemv(w, x_dev, y_dev, tokens, nullptr, 0.0f, ctx->stream));
  return LGH_OK;
}

int lgh_q8_norm_gemv_dev(lgh_ctx *ctx, const lgh_q8 *w, const float *norm_w_dev, float eps, const float *hidden_dev,
                         float *y_dev, size_t tokens) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w)) return r;
  if (tokens == 0 || w->n == 0) return LGH_OK;
  if (!y_dev || (w->k && !hidden_dev)) return fail(ctx, LGH_ERR_INVALID_ARG, "null hidden/y");
  if (!aligned16(hidden_dev) || !aligned16(norm_w_dev))
    return fail(ctx, LGH_ERR_INVALID_ARG, "hidden and norm weight must be 16-byte aligned");
  if (int r = set_device(ctx)) return r;
  const float *x = hidden_dev, *nw = w->k ? norm_w_dev : nullptr;
  if (nw && w->k > lgh::kQ8GemvMaxK) {  // rows longer than the prologue covers: rms_norm first
    if (int r = ensure(ctx, &ctx->ffn, &ctx->ffn_bytes, tokens * w->k * sizeof(float))) return r;
    float *nd = static_cast<float *>(ctx->ffn);
    LGH_HIP(ctx, lgh::launch_rms_norm(hidden_dev, nw, w->k, tokens, eps, nd, ctx->stream));
    x = nd;
    nw = nullptr;
  }
  LGH_HIP(ctx, lgh::launch_q8_gemv(w, x, y_dev, tokens, nw, eps, ctx->stream));
  return LGH_OK;
}

int lgh_q8_norm_gemv(lgh_ctx *ctx, const lgh_q8 *w, const float *norm_w, float eps, const float *hidden, float *y,
                     size_t tokens) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w)) return r;
  if (tokens == 0 || w->n == 0) return LGH_OK;
  if (!y || (w->k && !hidden)) return fail(ctx, LGH_ERR_INVALID_ARG, "null hidden/y");
  if (int r = set_device(ctx)) return r;
  Carve cv;
  const size_t xb = tokens * w->k * sizeof(float), nb = w->k * sizeof(float), yb = tokens * w->n * sizeof(float);
  const size_t ox = cv.take(xb), on = cv.take(norm_w ? nb : 0), oy = cv.take(yb);
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, cv.off)) return r;
  char *st = static_cast<char *>(ctx->stage);
  float *xd = reinterpret_cast<float *>(st + ox), *nd = norm_w ? reinterpret_cast<float *>(st + on) : nullptr;
  float *yd = reinterpret_cast<float *>(st + oy);
  if (xb) LGH_HIP(ctx, hipMemcpyAsync(xd, hidden, xb, hipMemcpyHostToDevice, ctx->stream));
  if (norm_w && nb) LGH_HIP(ctx, hipMemcpyAsync(nd, norm_w, nb, hipMemcpyHostToDevice, ctx->stream));
  if (int r = lgh_q8_norm_gemv_dev(ctx, w, nd, eps, xd, yd, tokens)) return r;
  LGH_HIP(ctx, hipMemcpyAsync(y, yd, yb, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

// ---- host-pointer entry points ----------------------------------------------
int lgh_q4_gemv(lgh_ctx *ctx, const lgh_q4 *w, const float *x, float *y, int mode) {
  return lgh_q4_gemm(ctx, w, x, y, 1, mode);
}

int lgh_q4_gemm(lgh_ctx *ctx, const lgh_q4 *w, const float *x, float *y, size_t m, int mode) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w)) return r;
  if (int r = check_mode(ctx, mode)) return r;
  if (m == 0 || w->n == 0) return LGH_OK;
  if (!x || !y) return fail(ctx, LGH_ERR_INVALID_ARG, "null x/y");
  if (int r = set_device(ctx)) return r;
  Carve cv;
  const size_t xb = m * w->k * sizeof(float), yb = m * w->n * sizeof(float);
  const size_t ox = cv.take(xb), oy = cv.take(yb);
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, cv.off)) return r;
  char *st = static_cast<char *>(ctx->stage);
  float *xd = reinterpret_cast<float *>(st + ox), *yd = reinterpret_cast<float *>(st + oy);
  LGH_HIP(ctx, hipMemcpyAsync(xd, x, xb, hipMemcpyHostToDevice, ctx->stream));
  if (mode != LGH_ASSIGN) LGH_HIP(ctx, hipMemcpyAsync(yd, y, yb, hipMemcpyHostToDevice, ctx->stream));
  if (int r = lgh_q4_gemm_dev(ctx, w, xd, yd, m, mode)) return r;
  LGH_HIP(ctx, hipMemcpyAsync(y, yd, yb, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

int lgh_q4_gemv_pair(lgh_ctx *ctx, const lgh_q4 *wg, const lgh_q4 *wu, const float *x, float *y_gate,
                     float *y_up) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, wg)) return r;
  if (int r = check_mat(ctx, wu)) return r;
  if (wg->k != wu->k || wg->n != wu->n)
    return fail(ctx, LGH_ERR_SHAPE, "pair needs equal shapes: gate %zux%zu, up %zux%zu", wg->n, wg->k, wu->n,
                wu->k);
  if (wg->n == 0) return LGH_OK;
  if (!x || !y_gate || !y_up) return fail(ctx, LGH_ERR_INVALID_ARG, "null x/y");
  if (int r = set_device(ctx)) return r;
  Carve cv;
  const size_t xb = wg->k * sizeof(float), yb = wg->n * sizeof(float);
  const size_t ox = cv.take(xb), og = cv.take(yb), ou = cv.take(yb);
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, cv.off)) return r;
  char *st = static_cast<char *>(ctx->stage);
  float *xd = reinterpret_cast<float *>(st + ox);
  float *gd = reinterpret_cast<float *>(st + og), *ud = reinterpret_cast<float *>(st + ou);
  LGH_HIP(ctx, hipMemcpyAsync(xd, x, xb, hipMemcpyHostToDevice, ctx->stream));
  if (int r = lgh_q4_gemv_pair_dev(ctx, wg, wu, xd, gd, ud)) return r;
  LGH_HIP(ctx, hipMemcpyAsync(y_gate, gd, yb, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipMemcpyAsync(y_up, ud, yb, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

// ---- elementwise ops and the FFN block -------------------------------------
int lgh_rms_norm_dev(lgh_ctx *ctx, const float *x_dev, const float *w_dev, size_t dim, size_t rows, float eps,
                     float *out_dev) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (dim == 0 || rows == 0) return LGH_OK;
  if (!x_dev || !w_dev || !out_dev) return fail(ctx, LGH_ERR_INVALID_ARG, "null x/weight/out");
  if (int r = set_device(ctx)) return r;
  LGH_HIP(ctx, lgh::launch_rms_norm(x_dev, w_dev, dim, rows, eps, out_dev, ctx->stream));
  return LGH_OK;
}

int lgh_rms_norm(lgh_ctx *ctx, const float *x, const float *w, size_t dim, size_t rows, float eps, float *out) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (dim == 0 || rows == 0) return LGH_OK;
  if (!x || !w || !out) return fail(ctx, LGH_ERR_INVALID_ARG, "null x/weight/out");
  if (int r = set_device(ctx)) return r;
  Carve cv;
  const size_t xb = dim * rows * sizeof(float), wb = dim * sizeof(float);
  const size_t ox = cv.take(xb), ow = cv.take(wb);
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, cv.off)) return r;
  char *st = static_cast<char *>(ctx->stage);
  float *xd = reinterpret_cast<float *>(st + ox), *wd = reinterpret_cast<float *>(st + ow);
  LGH_HIP(ctx, hipMemcpyAsync(xd, x, xb, hipMemcpyHostToDevice, ctx->stream));
  LGH_HIP(ctx, hipMemcpyAsync(wd, w, wb, hipMemcpyHostToDevice, ctx->stream));
  if (int r = lgh_rms_norm_dev(ctx, xd, wd, dim, rows, eps, xd)) return r;
  LGH_HIP(ctx, hipMemcpyAsync(out, xd, xb, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

int lgh_silu_mul_dev(lgh_ctx *ctx, float *g_dev, const float *u_dev, size_t n) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (n == 0) return LGH_OK;
  if (!g_dev || !u_dev) return fail(ctx, LGH_ERR_INVALID_ARG, "null g/u");
  if (int r = set_device(ctx)) return r;
  LGH_HIP(ctx, lgh::launch_silu_mul(g_dev, u_dev, n, ctx->stream));
  return LGH_OK;
}

int lgh_silu_mul(lgh_ctx *ctx, float *g, const float *u, size_t n) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (n == 0) return LGH_OK;
  if (!g || !u) return fail(ctx, LGH_ERR_INVALID_ARG, "null g/u");
  if (int r = set_device(ctx)) return r;
  Carve cv;
  const size_t b = n * sizeof(float);
  const size_t og = cv.take(b), ou = cv.take(b);
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, cv.off)) return r;
  char *st = static_cast<char *>(ctx->stage);
  float *gd = reinterpret_cast<float *>(st + og), *ud = reinterpret_cast<float *>(st + ou);
  LGH_HIP(ctx, hipMemcpyAsync(gd, g, b, hipMemcpyHostToDevice, ctx->stream));
  LGH_HIP(ctx, hipMemcpyAsync(ud, u, b, hipMemcpyHostToDevice, ctx->stream));
  if (int r = lgh_silu_mul_dev(ctx, gd, ud, n)) return r;
  LGH_HIP(ctx, hipMemcpyAsync(g, gd, b, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

static int check_ffn(lgh_ctx *ctx, const lgh_q4 *w1, const lgh_q4 *w3, const lgh_q4 *w2) {
  if (int r = check_mat(ctx, w1)) return r;
  if (int r = check_mat(ctx, w3)) return r;
  if (w1->k != w3->k || w1->n != w3->n)
    return fail(ctx, LGH_ERR_SHAPE, "gate/up need equal shapes: %zux%zu, %zux%zu", w1->n, w1->k, w3->n, w3->k);
  if (w2 && (w2->k != w1->n || w2->n != w1->k))
    return fail(ctx, LGH_ERR_SHAPE, "down must be %zux%zu, got %zux%zu", w1->k, w1->n, w2->n, w2->k);
  if (w1->n % 32 != 0) return fail(ctx, LGH_ERR_SHAPE, "intermediate size %zu is not a multiple of 32", w1->n);
  return LGH_OK;
}

// One token on a fused-shape FFN: two launches.
static int ffn_fused(lgh_ctx *ctx, const lgh_q4 *w1, const lgh_q4 *w3, const lgh_q4 *w2, const float *norm_w_dev,
                     float eps, float *hidden_dev) {
  const size_t n = w1->n;
  // PerBlock and a GEMV-sized W2: h leaves the gate/up kernel already
  // quantized.  Otherwise (PerRow needs all of h for its scale, or K beyond
  // the GEMV) h goes out in f32 through the regular M = 1 path.
  const bool codes = ctx->act_mode == LGH_ACT_PER_BLOCK && lgh::plan_q4_gemv(w2->n, w2->bpr, 1).ok;
  Carve cv;
  const size_t o_q = cv.take(n), o_s = cv.take(n / 32 * sizeof(float)), o_f = cv.take(codes ? 0 : n * sizeof(float));
  if (int r = ensure(ctx, &ctx->ffn, &ctx->ffn_bytes, cv.off)) return r;
  char *f = static_cast<char *>(ctx->ffn);
  auto *hq = reinterpret_cast<int8_t *>(f + o_q);
  auto *hs = reinterpret_cast<float *>(f + o_s);
  auto *hf = reinterpret_cast<float *>(f + o_f);
  LGH_HIP(ctx, lgh::launch_ffn_gate_up(w1, w3, hidden_dev, norm_w_dev, eps, ctx->act_mode, codes ? hq : nullptr, hs,
                                       codes ? nullptr : hf, nullptr, nullptr, ctx->stream));
  if (!codes) return lgh_q4_gemm_dev(ctx, w2, hf, hidden_dev, 1, LGH_ADD_F64);
  LGH_HIP(ctx, lgh::launch_q4_gemv_codes(w2, hq, hs, hidden_dev, LGH_ADD_F64, ctx->stream));
  return LGH_OK;
}

int lgh_q4_ffn_residual_dev(lgh_ctx *ctx, const lgh_q4 *w1, const lgh_q4 *w3, const lgh_q4 *w2,
                            const float *norm_w_dev, float eps, float *hidden_dev, size_t tokens) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w2)) return r;
  if (int r = check_ffn(ctx, w1, w3, w2)) return r;
  if (tokens == 0 || w1->k == 0 || w1->n == 0) return LGH_OK;  // nothing, or W2 h = 0 (hidden + 0 is hidden)
  if (!hidden_dev) return fail(ctx, LGH_ERR_INVALID_ARG, "null hidden");
  if (!aligned16(hidden_dev) || !aligned16(norm_w_dev))
    return fail(ctx, LGH_ERR_INVALID_ARG, "hidden and norm weight must be 16-byte aligned");
  if (int r = set_device(ctx)) return r;
  if (tokens == 1 && lgh::ffn_gate_up_supported(w1)) return ffn_fused(ctx, w1, w3, w2, norm_w_dev, eps, hidden_dev);
  // Several tokens (or a wide model): the reference's sequence of ops
  // (lfm2.rs:861-881) on the device, intermediates in the context.  The norm
  // and silu(g) * u are formed inside the activation-image kernels of the
  // gate/up and down GEMMs where those have a fused form (gemm_multi_dev).
  const size_t dim = w1->k, inter = w1->n;
  Carve cv;
  const size_t o_n = cv.take(norm_w_dev ? tokens * dim * sizeof(float) : 0);
  const size_t o_g = cv.take(tokens * inter * sizeof(float)), o_u = cv.take(tokens * inter * sizeof(float));
  if (int r = ensure(ctx, &ctx->ffn, &ctx->ffn_bytes, cv.off)) return r;
  char *f = static_cast<char *>(ctx->ffn);
  float *g = reinterpret_cast<float *>(f + o_g), *u = reinterpret_cast<float *>(f + o_u);
  const ActIn normed{hidden_dev, norm_w_dev, eps, nullptr, norm_w_dev ? reinterpret_cast<float *>(f + o_n) : nullptr};
  const lgh_q4 *gate_up[2] = {w1, w3};
  float *gu[2] = {g, u};
  if (int r = gemm_multi_dev(ctx, grow_ws(ctx), gate_up, 2, normed, gu, tokens, LGH_ASSIGN)) return r;
  return gemm_multi_dev(ctx, grow_ws(ctx), &w2, 1, ActIn{g, nullptr, 0.0f, u, g}, &hidden_dev, tokens, LGH_ADD_F64);
}

int lgh_q4_ffn_residual(lgh_ctx *ctx, const lgh_q4 *w1, const lgh_q4 *w3, const lgh_q4 *w2, const float *norm_w,
                        float eps, float *hidden, size_t tokens) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w2)) return r;
  if (int r = check_ffn(ctx, w1, w3, w2)) return r;
  if (tokens == 0 || w1->k == 0 || w1->n == 0) return LGH_OK;
  if (!hidden) return fail(ctx, LGH_ERR_INVALID_ARG, "null hidden");
  if (int r = set_device(ctx)) return r;
  Carve cv;
  const size_t xb = tokens * w1->k * sizeof(float), nb = w1->k * sizeof(float);
  const size_t ox = cv.take(xb), on = cv.take(norm_w ? nb : 0);
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, cv.off)) return r;
  char *st = static_cast<char *>(ctx->stage);
  float *xd = reinterpret_cast<float *>(st + ox), *nd = norm_w ? reinterpret_cast<float *>(st + on) : nullptr;
  LGH_HIP(ctx, hipMemcpyAsync(xd, hidden, xb, hipMemcpyHostToDevice, ctx->stream));
  if (norm_w) LGH_HIP(ctx, hipMemcpyAsync(nd, norm_w, nb, hipMemcpyHostToDevice, ctx->stream));
  if (int r = lgh_q4_ffn_residual_dev(ctx, w1, w3, w2, nd, eps, xd, tokens)) return r;
  LGH_HIP(ctx, hipMemcpyAsync(hidden, xd, xb, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

int lgh_q4_ffn_gate_up(lgh_ctx *ctx, const lgh_q4 *w1, const lgh_q4 *w3, const float *norm_w, float eps,
                       const float *hidden, float *g, float *u, float *h, int8_t *hq, float *hs) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_ffn(ctx, w1, w3, nullptr)) return r;
  if (w1->k == 0 || w1->n == 0) return LGH_OK;
  if (!lgh::ffn_gate_up_supported(w1))
    return fail(ctx, LGH_ERR_SHAPE, "the fused gate/up stage needs hidden size <= %zu, got %zu",
                lgh::kFfnMaxBpr * 32, w1->k);
  if (!hidden || !g || !u || !h) return fail(ctx, LGH_ERR_INVALID_ARG, "null hidden/g/u/h");
  if (int r = set_device(ctx)) return r;
  const size_t n = w1->n, xb = w1->k * sizeof(float), yb = n * sizeof(float);
  Carve cv;
  const size_t ox = cv.take(xb), on = cv.take(norm_w ? xb : 0), og = cv.take(yb), ou = cv.take(yb),
               oh = cv.take(yb), oq = cv.take(n), os = cv.take(n / 32 * sizeof(float));
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, cv.off)) return r;
  char *st = static_cast<char *>(ctx->stage);
  float *xd = reinterpret_cast<float *>(st + ox), *nd = norm_w ? reinterpret_cast<float *>(st + on) : nullptr;
  float *gd = reinterpret_cast<float *>(st + og), *ud = reinterpret_cast<float *>(st + ou);
  float *hd = reinterpret_cast<float *>(st + oh), *sd = reinterpret_cast<float *>(st + os);
  auto *qd = reinterpret_cast<int8_t *>(st + oq);
  LGH_HIP(ctx, hipMemcpyAsync(xd, hidden, xb, hipMemcpyHostToDevice, ctx->stream));
  if (norm_w) LGH_HIP(ctx, hipMemcpyAsync(nd, norm_w, xb, hipMemcpyHostToDevice, ctx->stream));
  LGH_HIP(ctx, lgh::launch_ffn_gate_up(w1, w3, xd, nd, eps, ctx->act_mode, qd, sd, hd, gd, ud, ctx->stream));
  LGH_HIP(ctx, hipMemcpyAsync(g, gd, yb, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipMemcpyAsync(u, ud, yb, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipMemcpyAsync(h, hd, yb, hipMemcpyDeviceToHost, ctx->stream));
  if (hq) LGH_HIP(ctx, hipMemcpyAsync(hq, qd, n, hipMemcpyDeviceToHost, ctx->stream));
  if (hs) LGH_HIP(ctx, hipMemcpyAsync(hs, sd, n / 32 * sizeof(float), hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

// ---- attention / conv block input side -------------------------------------
static int check_multi(lgh_ctx *ctx, size_t nmat, const lgh_q4 *const *w) {
  if (!w || nmat < 1 || nmat > 3) return fail(ctx, LGH_ERR_INVALID_ARG, "need 1 to 3 matrices, got %zu", nmat);
  for (size_t j = 0; j < nmat; j++) {
    if (!w[j]) return fail(ctx, LGH_ERR_INVALID_ARG, "null matrix %zu", j);
    if (int r = check_mat(ctx, w[j])) return r;
    if (w[j]->k != w[0]->k)
      return fail(ctx, LGH_ERR_SHAPE, "matrix %zu has k = %zu, matrix 0 k = %zu", j, w[j]->k, w[0]->k);
  }
  return LGH_OK;
}

int lgh_q4_norm_gemv_dev(lgh_ctx *ctx, size_t nmat, const lgh_q4 *const *w, const float *norm_w_dev, float eps,
                         const float *hidden_dev, float *const *y_dev, size_t tokens, int mode) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_multi(ctx, nmat, w)) return r;
  if (int r = check_mode(ctx, mode)) return r;
  const int nm = static_cast<int>(nmat);
  const size_t rows = lgh::gemv_multi_rows(w, nm), k = w[0]->k;
  if (tokens == 0 || rows == 0) return LGH_OK;
  if (!y_dev) return fail(ctx, LGH_ERR_INVALID_ARG, "null output array");
  for (size_t j = 0; j < nmat; j++)
    if (w[j]->n && !y_dev[j]) return fail(ctx, LGH_ERR_INVALID_ARG, "null output %zu", j);
  if (k && !hidden_dev) return fail(ctx, LGH_ERR_INVALID_ARG, "null hidden");
  if (!aligned16(hidden_dev) || !aligned16(norm_w_dev))
    return fail(ctx, LGH_ERR_INVALID_ARG, "hidden and norm weight must be 16-byte aligned");
  if (int r = set_device(ctx)) return r;
  // One token whose rows fit one K slice: a single launch (norm in the
  // prologue, one act-quant shared by every matrix).
  if (tokens == 1 && k > 0 && w[0]->bpr <= lgh::kFfnMaxBpr && lgh::plan_q4_gemv(rows, w[0]->bpr, 1).ok &&
      !lgh::q4_gemv_quantize_once(rows, w[0]->bpr, 1)) {
    LGH_HIP(ctx, lgh::launch_q4_gemv_multi(w, y_dev, nm, hidden_dev, nullptr, nullptr, norm_w_dev, eps, mode,
                                           ctx->act_mode, ctx->stream));
    return LGH_OK;
  }
  // Otherwise the reference's sequence (rms_norm, then one apply per matrix;
  // the matrices share each route's activation quantization, whose image
  // kernel forms the norm where it has a fused form).
  ActIn in{hidden_dev};
  if (norm_w_dev && k) {
    if (int r = ensure(ctx, &ctx->ffn, &ctx->ffn_bytes, tokens * k * sizeof(float))) return r;
    in = ActIn{hidden_dev, norm_w_dev, eps, nullptr, static_cast<float *>(ctx->ffn)};
  }
  return gemm_multi_dev(ctx, grow_ws(ctx), w, nm, in, y_dev, tokens, mode);
}

int lgh_q4_norm_gemv(lgh_ctx *ctx, size_t nmat, const lgh_q4 *const *w, const float *norm_w, float eps,
                     const float *hidden, float *const *y, size_t tokens, int mode) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_multi(ctx, nmat, w)) return r;
  if (int r = check_mode(ctx, mode)) return r;
  const size_t rows = lgh::gemv_multi_rows(w, static_cast<int>(nmat)), k = w[0]->k;
  if (tokens == 0 || rows == 0) return LGH_OK;
  if (!y) return fail(ctx, LGH_ERR_INVALID_ARG, "null output array");
  for (size_t j = 0; j < nmat; j++)
    if (w[j]->n && !y[j]) return fail(ctx, LGH_ERR_INVALID_ARG, "null output %zu", j);
  if (k && !hidden) return fail(ctx, LGH_ERR_INVALID_ARG, "null hidden");
  if (int r = set_device(ctx)) return r;
  Carve cv;
  const size_t xb = tokens * k * sizeof(float), nb = k * sizeof(float);
  const size_t ox = cv.take(xb), on = cv.take(norm_w ? nb : 0);
  size_t oy[3] = {0, 0, 0};
  for (size_t j = 0; j < nmat; j++) oy[j] = cv.take(tokens * w[j]->n * sizeof(float));
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, cv.off)) return r;
  char *st = static_cast<char *>(ctx->stage);
  float *xd = reinterpret_cast<float *>(st + ox), *nd = norm_w ? reinterpret_cast<float *>(st + on) : nullptr;
  float *yd[3] = {nullptr, nullptr, nullptr};
  if (k) LGH_HIP(ctx, hipMemcpyAsync(xd, hidden, xb, hipMemcpyHostToDevice, ctx->stream));
  if (norm_w && k) LGH_HIP(ctx, hipMemcpyAsync(nd, norm_w, nb, hipMemcpyHostToDevice, ctx->stream));
  for (size_t j = 0; j < nmat; j++) {
    yd[j] = reinterpret_cast<float *>(st + oy[j]);
    const size_t yb = tokens * w[j]->n * sizeof(float);
    if (mode != LGH_ASSIGN && yb) LGH_HIP(ctx, hipMemcpyAsync(yd[j], y[j], yb, hipMemcpyHostToDevice, ctx->stream));
  }
  if (int r = lgh_q4_norm_gemv_dev(ctx, nmat, w, nd, eps, xd, yd, tokens, mode)) return r;
  for (size_t j = 0; j < nmat; j++) {
    const size_t yb = tokens * w[j]->n * sizeof(float);
    if (yb) LGH_HIP(ctx, hipMemcpyAsync(y[j], yd[j], yb, hipMemcpyDeviceToHost, ctx->stream));
  }
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

int lgh_q8_gemv(lgh_ctx *ctx, const lgh_q8 *w, const float *x, float *y, size_t tokens) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w)) return r;
  if (tokens == 0 || w->n == 0) return LGH_OK;
  if (!x || !y) return fail(ctx, LGH_ERR_INVALID_ARG, "null x/y");
  if (int r = set_device(ctx)) return r;
  Carve cv;
  const size_t xb = tokens * w->k * sizeof(float), yb = tokens * w->n * sizeof(float);
  const size_t ox = cv.take(xb), oy = cv.take(yb);
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, cv.off)) return r;
  char *st = static_cast<char *>(ctx->stage);
  float *xd = reinterpret_cast<float *>(st + ox), *yd = reinterpret_cast<float *>(st + oy);
  LGH_HIP(ctx, hipMemcpyAsync(xd, x, xb, hipMemcpyHostToDevice, ctx->stream));
  if (int r = lgh_q8_gemv_dev(ctx, w, xd, yd, tokens)) return r;
  LGH_HIP(ctx, hipMemcpyAsync(y, yd, yb, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

// ---- test hooks ---------------------------------------------------------------
int lgh_act_quant(lgh_ctx *ctx, const float *x, size_t m, size_t k, int8_t *qs, float *scales, int32_t *sums) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (k % 32) return fail(ctx, LGH_ERR_SHAPE, "activation length %zu is not a multiple of 32", k);
  if (m == 0 || k == 0) return LGH_OK;
  if (!x || !qs || !scales) return fail(ctx, LGH_ERR_INVALID_ARG, "null argument");
  if (int r = set_device(ctx)) return r;
  const size_t bpr = k / 32;
  Carve cv;
  const size_t ox = cv.take(m * k * 4), oq = cv.take(m * k), os = cv.take(m * bpr * 4), ou = cv.take(m * bpr * 4),
               orow = cv.take(m * 4);
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, cv.off)) return r;
  char *st = static_cast<char *>(ctx->stage);
  LGH_HIP(ctx, hipMemcpyAsync(st + ox, x, m * k * 4, hipMemcpyHostToDevice, ctx->stream));
  LGH_HIP(ctx, lgh::launch_act_quant(reinterpret_cast<float *>(st + ox), m, k, ctx->act_mode,
                                     reinterpret_cast<int8_t *>(st + oq), reinterpret_cast<float *>(st + os),
                                     reinterpret_cast<int32_t *>(st + ou), reinterpret_cast<float *>(st + orow),
                                     ctx->stream));
  LGH_HIP(ctx, hipMemcpyAsync(qs, st + oq, m * k, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipMemcpyAsync(scales, st + os, m * bpr * 4, hipMemcpyDeviceToHost, ctx->stream));
  if (sums) LGH_HIP(ctx, hipMemcpyAsync(sums, st + ou, m * bpr * 4, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

int lgh_gemv_plans_uncovered(void) { return lgh::gemv_plans_uncovered(); }

int lgh_q4_block_dots(lgh_ctx *ctx, const void *blocks, const int8_t *a, size_t nblocks, int32_t *out) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (nblocks == 0) return LGH_OK;
  if (!blocks || !a || !out) return fail(ctx, LGH_ERR_INVALID_ARG, "null argument");
  if (int r = set_device(ctx)) return r;
  Carve cv;
  const size_t oraw = cv.take(nblocks * 18), oqs = cv.take(nblocks * 16), osc = cv.take(nblocks * 2),
               oa = cv.take(nblocks * 32), oo = cv.take(nblocks * 4);
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, cv.off)) return r;
  char *st = static_cast<char *>(ctx->stage);
  LGH_HIP(ctx, hipMemcpyAsync(st + oraw, blocks, nblocks * 18, hipMemcpyHostToDevice, ctx->stream));
  LGH_HIP(ctx, hipMemcpyAsync(st + oa, a, nblocks * 32, hipMemcpyHostToDevice, ctx->stream));
  LGH_HIP(ctx, lgh::launch_q4_repack(reinterpret_cast<uint8_t *>(st + oraw), nblocks,
                                     reinterpret_cast<uint8_t *>(st + oqs), reinterpret_cast<uint16_t *>(st + osc),
                                     ctx->stream));
  LGH_HIP(ctx, lgh::launch_q4_block_dots(reinterpret_cast<uint8_t *>(st + oqs), reinterpret_cast<int8_t *>(st + oa),
                                         nblocks, reinterpret_cast<int32_t *>(st + oo), ctx->stream));
  LGH_HIP(ctx, hipMemcpyAsync(out, st + oo, nblocks * 4, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

int lgh_q8_block_dots(lgh_ctx *ctx, const void *blocks, const int8_t *a, size_t nblocks, int32_t *out) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (nblocks == 0) return LGH_OK;
  if (!blocks || !a || !out) return fail(ctx, LGH_ERR_INVALID_ARG, "null argument");
  if (int r = set_device(ctx)) return r;
  Carve cv;
  const size_t oraw = cv.take(nblocks * 34), oqs = cv.take(nblocks * 32), osc = cv.take(nblocks * 2),
               oa = cv.take(nblocks * 32), oo = cv.take(nblocks * 4);
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, cv.off)) return r;
  char *st = static_cast<char *>(ctx->stage);
  LGH_HIP(ctx, hipMemcpyAsync(st + oraw, blocks, nblocks * 34, hipMemcpyHostToDevice, ctx->stream));
  LGH_HIP(ctx, hipMemcpyAsync(st + oa, a, nblocks * 32, hipMemcpyHostToDevice, ctx->stream));
  LGH_HIP(ctx, lgh::launch_q8_repack(reinterpret_cast<uint8_t *>(st + oraw), nblocks,
                                     reinterpret_cast<int8_t *>(st + oqs), reinterpret_cast<uint16_t *>(st + osc),
                                     ctx->stream));
  LGH_HIP(ctx, lgh::launch_q8_block_dots(reinterpret_cast<int8_t *>(st + oqs), reinterpret_cast<int8_t *>(st + oa),
                                         nblocks, reinterpret_cast<int32_t *>(st + oo), ctx->stream));
  LGH_HIP(ctx, hipMemcpyAsync(out, st + oo, nblocks * 4, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

int lgh_q4_mfma_block_dots(lgh_ctx *ctx, const lgh_q4 *w, const int8_t *qs, size_t m, int32_t *out) {
  if (!ctx) return LGH_ERR_INVALID_ARG;
  if (int r = check_mat(ctx, w)) return r;
  if (m == 0 || w->n == 0 || w->bpr == 0) return LGH_OK;
  if (!qs || !out) return fail(ctx, LGH_ERR_INVALID_ARG, "null argument");
  if (int r = set_device(ctx)) return r;
  if (int r = ensure_mx(ctx, w)) return r;
  const size_t ob_bytes = m * w->n * w->bpr * 4;
  const size_t mx_bytes = (m + 31) / 32 * w->pp * lgh::kMxARec;
  if (mx_bytes >= lgh::kMxMaxBytes) return fail(ctx, LGH_ERR_SHAPE, "too many tokens for one hook call");
  Carve cv;
  const size_t oq = cv.take(m * w->k), omx = cv.take(mx_bytes), oo = cv.take(ob_bytes);
  if (int r = ensure(ctx, &ctx->stage, &ctx->stage_bytes, cv.off)) return r;
  char *st = static_cast<char *>(ctx->stage);
  auto *mxa = reinterpret_cast<uint8_t *>(st + omx);
  LGH_HIP(ctx, hipMemcpyAsync(st + oq, qs, m * w->k, hipMemcpyHostToDevice, ctx->stream));
  LGH_HIP(ctx, lgh::launch_act_split_mx(reinterpret_cast<int8_t *>(st + oq), nullptr, m, w->k, mxa, ctx->stream));
  LGH_HIP(ctx, lgh::launch_q4_mfma_block_dots(w, mxa, m, reinterpret_cast<int32_t *>(st + oo), ctx->stream));
  LGH_HIP(ctx, hipMemcpyAsync(out, st + oo, ob_bytes, hipMemcpyDeviceToHost, ctx->stream));
  LGH_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return LGH_OK;
}

}  // extern "C"
