/*
 * llm_gpu_hip.h -- C ABI of the MI355X (gfx950) block-quantized matmul library.
 *
 * Drop-in for llmhost's CPU matmul seam: the functions below replace the
 * llm-cpu free functions that crates/llm-engine/src/weights.rs dispatches to
 * (Linear::apply / apply_add / apply_pair, OutputHead::apply).  Each
 * declaration cites the reference interface it replaces (paths relative to
 * the llmhost repository root).
 *
 * Conventions
 *  - Plain C: opaque handles, plain pointers and sizes; no exceptions or
 *    panics cross this boundary.  Every int-returning call returns LGH_OK (0)
 *    or a negative LGH_ERR_* code; lgh_last_error() then holds a message.
 *    The reference panics on contract violations (assert!); here the same
 *    conditions return LGH_ERR_SHAPE and write nothing.
 *  - Weight blocks are llm-quant's BlockQ4 (18 bytes: LE f16 scale + 16 bytes
 *    of two's-complement nibbles, element i in the low nibble of qs[i/2] when
 *    i is even) and BlockQ8_0 (34 bytes: LE f16 scale + 32 int8), row-major
 *    [n][k/32], consumed as-is (crates/llm-quant/src/lib.rs:17-21, 54-58).
 *  - Host-pointer calls take and return host memory and are synchronous
 *    (slice semantics of llm-cpu).  *_dev calls take device pointers, are
 *    enqueued on the context stream and return before the work completes.
 *  - One context is used by one thread at a time (llm-cpu's with_threads
 *    session lock, crates/llm-cpu/src/pool.rs:278-299).
 *  - n == 0 or m == 0 is a successful no-op, as in the reference
 *    (crates/llm-cpu/src/gemv_q4.rs:369-371, 698-700).
 */
#ifndef LLM_GPU_HIP_H
#define LLM_GPU_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LGH_OK 0
#define LGH_ERR_INVALID_ARG (-1) /* null handle/pointer or unknown enum value  */
#define LGH_ERR_SHAPE (-2)       /* k % 32 != 0, mismatched shapes             */
#define LGH_ERR_HIP (-3)         /* HIP runtime error (message has details)    */
#define LGH_ERR_ARCH (-4)        /* device is not gfx950                       */
#define LGH_ERR_NO_DEVICE (-5)   /* no such HIP device                         */
#define LGH_ERR_OOM (-6)         /* device or host allocation failed           */
#define LGH_ERR_CAPTURE (-7)     /* a workspace would have to grow while the
                                    context stream is being captured           */

/* Accumulation mode, crates/llm-cpu/src/gemv_q4.rs:445-449 AccMode, plus the
 * f32 residual add the attention and conv blocks apply after their output
 * projection (Linear::apply then add_inplace, crates/llm-cpu/src/ops.rs:48-53;
 * crates/llm-engine/src/lfm2.rs:645, 682, 749, 857). */
#define LGH_ASSIGN 0  /* out = W x                                  */
#define LGH_ADD_F64 1 /* out = (float)((double)out + (double)(W x)) */
#define LGH_ADD_F32 2 /* out = out + (float)(W x), in f32           */

/* Activation quantization, crates/llm-cpu/src/gemv_q4.rs:263-271 ActQuant. */
#define LGH_ACT_PER_BLOCK 0 /* one scale per 32-element block (default) */
#define LGH_ACT_PER_ROW 1   /* one scale per row, replicated per block  */

#define LGH_BLOCK 32
#define LGH_BLOCK_Q4_BYTES 18
#define LGH_BLOCK_Q8_BYTES 34

typedef struct lgh_ctx lgh_ctx; /* device, stream, workspaces, act-quant mode */
typedef struct lgh_q4 lgh_q4;   /* device-resident Q4 matrix [n, k]           */
typedef struct lgh_q8 lgh_q8;   /* device-resident Q8_0 matrix [n, k]         */

/* Version string; static, never freed.  Style of llmhost_version(),
 * crates/llm-capi/src/lib.rs:12-15. */
const char *lgh_version(void);

/* Open a context on HIP device `device`.  Fails with LGH_ERR_ARCH unless the
 * device is gfx950.  Replaces CpuBackend::new (crates/llm-cpu/src/lib.rs:46-57)
 * as the thing a session is bound to. */
int lgh_init(int device, lgh_ctx **out);
void lgh_destroy(lgh_ctx *ctx);
/* Message of the last failed call on ctx (or of the last failed lgh_init when
 * ctx is NULL).  Valid until the next call on ctx. */
const char *lgh_last_error(const lgh_ctx *ctx);

/* set_act_quant / current_act_quant (crates/llm-cpu/src/gemv_q4.rs:276-292),
 * per context instead of process-wide.  Affects the Q4 GEMV/GEMM; the Q8_0
 * GEMV always quantizes per block (crates/llm-engine/src/weights.rs:197). */
int lgh_set_act_quant(lgh_ctx *ctx, int mode);
int lgh_get_act_quant(const lgh_ctx *ctx);

/* Stream used by every call on ctx (a hipStream_t; NULL = the context's own
 * stream).  Lets a caller enqueue on a stream it already times or orders. */
int lgh_set_stream(lgh_ctx *ctx, void *hip_stream);
void *lgh_get_stream(const lgh_ctx *ctx);
/* Wait for all work enqueued on the context stream. */
int lgh_sync(lgh_ctx *ctx);
/* Wait for the context stream, then release the context's grow-only device
 * buffers (GEMM workspace, host-call staging, FFN intermediates); they grow
 * again on the next call that needs them.  Workspaces grow only outside
 * stream capture: a call under capture that would grow one returns
 * LGH_ERR_CAPTURE, so run each shape once before capturing.  No reference
 * counterpart (llm-cpu keeps no device buffers). */
int lgh_trim(lgh_ctx *ctx);

/* ---- device buffers ---------------------------------------------------------
 * Backend::alloc (crates/llm-core/src/backend.rs:4-13; the CPU backend's
 * Vec<f32>, crates/llm-cpu/src/lib.rs:65-75): a device buffer of `len` f32
 * elements, zero-filled, for the *_dev entry points.  len == 0 gives NULL.
 * lgh_buffer_write / lgh_buffer_read copy host <-> device (synchronous) --
 * the copy methods backend.rs:3 leaves to the first real backend.  Free with
 * lgh_buffer_free (waits for the context stream first). */
int lgh_buffer_alloc(lgh_ctx *ctx, size_t len, float **out);
void lgh_buffer_free(lgh_ctx *ctx, float *buf);
int lgh_buffer_write(lgh_ctx *ctx, float *dst_dev, const float *src, size_t len);
int lgh_buffer_read(lgh_ctx *ctx, float *dst, const float *src_dev, size_t len);

/* ---- weights ------------------------------------------------------------
 * Q4Matrix::from_blocks (crates/llm-cpu/src/gemv_q4.rs:128-149): upload
 * row-major BlockQ4[n][k/32] from host memory and repack on the device.
 * Weights are immutable afterwards. */
int lgh_q4_upload(lgh_ctx *ctx, const void *blocks, size_t n, size_t k, lgh_q4 **out);
/* Same, from device-resident BlockQ4 bytes (n*k/32*18 bytes, any alignment). */
int lgh_q4_upload_dev(lgh_ctx *ctx, const void *blocks_dev, size_t n, size_t k, lgh_q4 **out);
/* Q4Matrix::from_f32 / Linear::from_f32(.., WeightFormat::Q4_32)
 * (gemv_q4.rs:116-124, crates/llm-engine/src/weights.rs:36-43): quantize a
 * row-major fp32 [n, k] host matrix with BlockQ4::quantize
 * (crates/llm-quant/src/lib.rs:63-79) on the device. */
int lgh_q4_from_f32(lgh_ctx *ctx, const float *w, size_t n, size_t k, lgh_q4 **out);
/* Copy the device matrix back as BlockQ4[n][k/32] (18-byte blocks). */
int lgh_q4_download(lgh_ctx *ctx, const lgh_q4 *w, void *blocks);
/* Build the matrix's GEMM operand image now (28 B per 32 weights, fp6 codes
 * and f32 scales in the matrix-core layout).  An upload holds only the
 * 18 B/32 nibble and scale planes; the first call that routes the matrix to
 * the GEMM (m >= 65, long rows at m >= 49, or k > 32768) builds the image
 * itself, which allocates -- so call this before capturing such a call in a
 * graph or passing the matrix to lgh_q4_gemm_dev_noalloc.  LGH_ERR_SHAPE if
 * the image would exceed 2 GiB (about 2.4e9 weights): such a matrix never
 * has one, and the calls that would use it run the matrix-core batch kernel
 * on its nibble planes instead, 64 tokens per launch, with the same results'
 * tolerance.  No reference counterpart: llm-cpu's Q4Matrix
 * packs its tiles (and AMX panels) at load, gemv_q4.rs:116-209. */
int lgh_q4_prepare_gemm(lgh_ctx *ctx, const lgh_q4 *w);
/* Device bytes the matrix holds: the nibble and scale planes, plus the GEMM
 * image once built. */
size_t lgh_q4_device_bytes(const lgh_q4 *w);

/* ---- device images (pre-packed load format) ------------------------------------
 * The matrix exactly as it sits in HBM, so that a load is one copy with no
 * repack kernel: the Q4 image is the nibble plane (n*k/32 x 16 B, the
 * repaired nibble order), the f16 scale plane (n*k/32 x 2 B) and, with_gemm,
 * the GEMM operand image; the Q8_0 image is the code plane (n*k/32 x 32 B)
 * and the scale plane.  Export writes `bytes` (= *_image_bytes) to host
 * memory, building the GEMM image first if asked for; import allocates a
 * matrix from such an image (bytes must match n, k).  The image format is
 * this library's own (a file container around it: llmhost_amd/packfile.py);
 * it stands in for the pre-packed .lfmb container llm-quant plans
 * (ARCHITECTURE.md:101) and for Q4Matrix::from_blocks' per-load repack
 * (crates/llm-cpu/src/gemv_q4.rs:128-149).  Import copies the bytes as they
 * are: a container stores lgh_image_layout() beside its images and loads
 * them only into a library that returns the same value. */
uint32_t lgh_image_layout(void);
size_t lgh_q4_image_bytes(const lgh_q4 *w, int with_gemm);
int lgh_q4_export(lgh_ctx *ctx, const lgh_q4 *w, int with_gemm, void *dst, size_t bytes);
int lgh_q4_import(lgh_ctx *ctx, const void *src, size_t bytes, size_t n, size_t k, int with_gemm, lgh_q4 **out);
size_t lgh_q8_image_bytes(const lgh_q8 *w);
int lgh_q8_export(lgh_ctx *ctx, const lgh_q8 *w, void *dst, size_t bytes);
int lgh_q8_import(lgh_ctx *ctx, const void *src, size_t bytes, size_t n, size_t k, lgh_q8 **out);
void lgh_q4_free(lgh_q4 *w);
size_t lgh_q4_rows(const lgh_q4 *w);
size_t lgh_q4_cols(const lgh_q4 *w);

/* Q8Matrix (crates/llm-engine/src/weights.rs:126-153): BlockQ8_0[n][k/32]. */
int lgh_q8_upload(lgh_ctx *ctx, const void *blocks, size_t n, size_t k, lgh_q8 **out);
/* Q8Matrix::from_f32 with BlockQ8_0::quantize (crates/llm-quant/src/lib.rs:26-37). */
int lgh_q8_from_f32(lgh_ctx *ctx, const float *w, size_t n, size_t k, lgh_q8 **out);
int lgh_q8_download(lgh_ctx *ctx, const lgh_q8 *w, void *blocks);
void lgh_q8_free(lgh_q8 *w);
size_t lgh_q8_rows(const lgh_q8 *w);
size_t lgh_q8_cols(const lgh_q8 *w);

/* ---- Q4 GEMV, M = 1 -------------------------------------------------------
 * gemv_q4 / gemv_q4_add (crates/llm-cpu/src/gemv_q4.rs:344-363):
 * y[n] = W[n,k] @ x[k] with x quantized per ActQ8 (gemv_q4.rs:62-95); mode
 * LGH_ADD_F64 adds onto y in f64 (gemv_q4.rs:486-497). */
int lgh_q4_gemv(lgh_ctx *ctx, const lgh_q4 *w, const float *x, float *y, int mode);
int lgh_q4_gemv_dev(lgh_ctx *ctx, const lgh_q4 *w, const float *x_dev, float *y_dev, int mode);

/* gemv_q4_pair (crates/llm-cpu/src/gemv_q4.rs:396-443): SwiGLU gate and up
 * projections sharing one activation quantization, one launch.  Requires
 * equal k and equal n (gemv_q4.rs:403-417). */
int lgh_q4_gemv_pair(lgh_ctx *ctx, const lgh_q4 *w_gate, const lgh_q4 *w_up, const float *x,
                     float *y_gate, float *y_up);
int lgh_q4_gemv_pair_dev(lgh_ctx *ctx, const lgh_q4 *w_gate, const lgh_q4 *w_up,
                         const float *x_dev, float *yg_dev, float *yu_dev);

/* gemv_q4_prep / gemv_q4_prep_add (crates/llm-cpu/src/gemv_q4.rs:366-393): the
 * GEMV on activations already quantized by ActQ8 -- codes int8[k] and block
 * scales f32[k/32] as lgh_act_quant(_dev) writes them, in either act-quant
 * mode (the sums are not read).  The reference's Q4Kernel argument has no
 * counterpart (one device kernel; K > 32768 runs the GEMM on the same codes).
 * Device codes 16-byte and scales 4-byte aligned. */
int lgh_q4_gemv_prep(lgh_ctx *ctx, const lgh_q4 *w, const int8_t *qs, const float *scales, float *y, int mode);
int lgh_q4_gemv_prep_dev(lgh_ctx *ctx, const lgh_q4 *w, const int8_t *qs_dev, const float *scales_dev,
                         float *y_dev, int mode);
/* ActQ8::quantize_into / quantize_row_into (gemv_q4.rs:52-95) per row of
 * x[m,k], device to device, enqueued on the context stream and honouring the
 * context's act-quant mode: codes[m,k], scales[m,k/32], sums[m,k/32] (sums may
 * be NULL).  x 16-byte aligned, the outputs 4-byte aligned. */
int lgh_act_quant_dev(lgh_ctx *ctx, const float *x_dev, size_t m, size_t k, int8_t *qs_dev, float *scales_dev,
                      int32_t *sums_dev);

/* ---- Q4 GEMM, M >= 1 ------------------------------------------------------
 * gemm_q4 / gemm_q4_add (crates/llm-cpu/src/gemv_q4.rs:686-722):
 * y[m, n] = x[m, k] @ W[n, k]^T, activations quantized per token with
 * quantize_batch (gemv_q4.rs:747-798).  m == 1 runs the GEMV. */
int lgh_q4_gemm(lgh_ctx *ctx, const lgh_q4 *w, const float *x, float *y, size_t m, int mode);
int lgh_q4_gemm_dev(lgh_ctx *ctx, const lgh_q4 *w, const float *x_dev, float *y_dev, size_t m,
                    int mode);

/* The same product as lgh_q4_gemm_dev, for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc.  It has no counterpart in the reference.  Every
 * scratch buffer of the call (activation images and codes, split-K partials)
 * comes from one fixed device array of LGH_NOALLOC_SCRATCH_BYTES per GPU,
 * held until the process ends; the call allocates, frees and synchronizes
 * nothing.  On the GEMM route (65 or more tokens) token chunks shrink until
 * their scratch fits, keeping the whole call's plan (split-K count and K
 * groups per workgroup, which fix the f32 summation order); a call
 * whose 32-token chunk still needs more returns LGH_ERR_SHAPE.  The routes of
 * 1-64 tokens (and the 64-token chunks of a matrix too large for a GEMM
 * image) take their scratch in one piece and return LGH_ERR_SHAPE when it
 * exceeds the array (only rows of more than about 466k elements can).
 * Routes that need the matrix's GEMM image return LGH_ERR_INVALID_ARG unless
 * lgh_q4_prepare_gemm has built it.  Every context on a GPU shares that GPU's
 * array and it keeps the last call's contents: calls that overlap on one GPU
 * (several contexts or streams) race, so the caller serializes them.
 * Results equal lgh_q4_gemm_dev's bit for bit. */
#define LGH_NOALLOC_SCRATCH_BYTES (32u << 20)
int lgh_q4_gemm_dev_noalloc(lgh_ctx *ctx, const lgh_q4 *w, const float *x_dev, float *y_dev, size_t m,
                            int mode);

/* ---- measurement probes ----------------------------------------------------
 * No counterpart in the reference.  Two launches that bound what any launch
 * of the library can reach, for a benchmark to time in the same harness as
 * the matmuls (device pointers, asynchronous on the context stream):
 * lgh_probe_empty_dev launches an empty kernel of `workgroups` x 256 threads
 * (1..65535) -- the per-launch floor of dependent launches;
 * lgh_probe_read_dev reads `bytes` (a multiple of 16, below 2 GiB) at src_dev
 * (16-byte aligned) with per_thread (1, 2, 4 or 8) 128-bit streaming loads per
 * thread, all issued before any is used, and writes one f32 sum per
 * workgroup to out_dev
 * (lgh_probe_read_outputs(bytes, per_thread) floats; 0 for a bad per_thread)
 * -- a plain streaming read of that size. */
int lgh_probe_empty_dev(lgh_ctx *ctx, int workgroups);
size_t lgh_probe_read_outputs(size_t bytes, int per_thread);
int lgh_probe_read_dev(lgh_ctx *ctx, const void *src_dev, size_t bytes, int per_thread, float *out_dev);

/* ---- Q8_0 GEMV ------------------------------------------------------------
 * q8_apply (crates/llm-engine/src/weights.rs:194-227), reached through
 * OutputHead::apply (weights.rs:186-192): per token, y[n] = W[n,k] @ x[k]
 * with per-block ActQ8 activations.  Assign mode only, as in the reference.
 * Any K and any number of tokens (rows past 32768 elements are summed in
 * K ranges of 32768, added in f32). */
int lgh_q8_gemv(lgh_ctx *ctx, const lgh_q8 *w, const float *x, float *y, size_t tokens);
int lgh_q8_gemv_dev(lgh_ctx *ctx, const lgh_q8 *w, const float *x_dev, float *y_dev,
                    size_t tokens);

/* The final rms_norm of a decode or prefill step followed by the Q8_0 output
 * head (crates/llm-engine/src/lfm2.rs:559-567, 496-504): per token,
 * y = W (rms_norm(hidden, norm_w, eps)), norm_w == NULL: y = W hidden -- the
 * norm in the GEMV's prologue, one launch.  (A Q4 head takes lgh_q4_norm_gemv
 * with one matrix.)  Results equal rms_norm followed by lgh_q8_gemv. */
int lgh_q8_norm_gemv(lgh_ctx *ctx, const lgh_q8 *w, const float *norm_w, float eps, const float *hidden, float *y,
                     size_t tokens);
int lgh_q8_norm_gemv_dev(lgh_ctx *ctx, const lgh_q8 *w, const float *norm_w_dev, float eps,
                         const float *hidden_dev, float *y_dev, size_t tokens);

/* ---- elementwise ops of the FFN block ----------------------------------------
 * rms_norm (crates/llm-cpu/src/ops.rs:8-23): out[r] = w * (x[r] * scale_r)
 * over `rows` rows of `dim`, scale_r = f32(1 / sqrt(sum_sq * (1/dim) + eps))
 * with the sum of squares in f64.  out may be x. */
int lgh_rms_norm(lgh_ctx *ctx, const float *x, const float *weight, size_t dim, size_t rows, float eps,
                 float *out);
int lgh_rms_norm_dev(lgh_ctx *ctx, const float *x_dev, const float *weight_dev, size_t dim, size_t rows,
                     float eps, float *out_dev);
/* silu_inplace + the gate multiply (ops.rs:27-36, crates/llm-engine/src/
 * lfm2.rs:902-905): g[i] = (g[i] / (1 + exp(-g[i]))) * u[i]. */
int lgh_silu_mul(lgh_ctx *ctx, float *g, const float *u, size_t n);
int lgh_silu_mul_dev(lgh_ctx *ctx, float *g_dev, const float *u_dev, size_t n);

/* ---- FFN block (SwiGLU) -------------------------------------------------------
 * Lfm2::ffn_residual (crates/llm-engine/src/lfm2.rs:861-881) and, for one
 * token, Lfm2::ffn_residual_in (:883-911), over `tokens` rows of hidden:
 *   normed = rms_norm(hidden, norm_w, eps)  (norm_w == NULL: normed = hidden)
 *   g, u   = W1 normed, W3 normed           (apply_pair: gemv_q4_pair / gemm_q4)
 *   h      = silu(g) * u
 *   hidden = (float)((double)hidden + (double)(W2 h))   (gemv_q4_add / gemm_q4_add)
 * W1, W3: [inter, dim]; W2: [dim, inter].  Both activation quantizations
 * follow the context's act-quant mode.  One token with dim <= 2048 runs two
 * fused launches (the second reads h's ActQ8 codes written by the first).
 * Otherwise the ops above run on the device one after another, except that
 * for 5 or more tokens the norm and the gate/up activation image are
 * formed in one launch (the normed rows are not written) and the down
 * projection's image kernel forms silu(g) * u itself; the results equal the
 * op sequence's bit for bit.
 * No single reference function: it replaces the reference's sequence of
 * calls. */
int lgh_q4_ffn_residual(lgh_ctx *ctx, const lgh_q4 *w1, const lgh_q4 *w3, const lgh_q4 *w2,
                        const float *norm_w, float eps, float *hidden, size_t tokens);
int lgh_q4_ffn_residual_dev(lgh_ctx *ctx, const lgh_q4 *w1, const lgh_q4 *w3, const lgh_q4 *w2,
                            const float *norm_w_dev, float eps, float *hidden_dev, size_t tokens);

/* ---- attention / conv block input side ----------------------------------------
 * rms_norm, then the block's input projections, all on the same normed rows,
 * over `tokens` rows of hidden [tokens, k]:
 *   normed = rms_norm(hidden, norm_w, eps)   (norm_w == NULL: normed = hidden)
 *   y[j]   = W[j] normed  (mode as lgh_q4_gemm), j < nmat, 1 <= nmat <= 3
 * -- Lfm2::attn_decode's q_proj / k_proj / v_proj (crates/llm-engine/src/
 * lfm2.rs:784-794) and Lfm2::conv_update's in_proj (lfm2.rs:651-659); prefill
 * alike (lfm2.rs:698-711, and 609-625 when no position is padding).  Every W[j] has the same k; y[j] is
 * [tokens, W[j].n].  One token with k <= 2048 runs one launch: the norm in
 * its prologue and one activation quantization shared by all matrices (as
 * gemv_q4_pair shares one, crates/llm-cpu/src/gemv_q4.rs:396-443); otherwise
 * rms_norm then one lgh_q4_gemm per matrix (for 5 or more tokens the norm is
 * applied by the launch that writes the shared activation image).
 * Results equal that sequence. */
int lgh_q4_norm_gemv(lgh_ctx *ctx, size_t nmat, const lgh_q4 *const *w, const float *norm_w, float eps,
                     const float *hidden, float *const *y, size_t tokens, int mode);
int lgh_q4_norm_gemv_dev(lgh_ctx *ctx, size_t nmat, const lgh_q4 *const *w, const float *norm_w_dev, float eps,
                         const float *hidden_dev, float *const *y_dev, size_t tokens, int mode);

/* ---- test hooks (host pointers, synchronous) -------------------------------
 * ActQ8::quantize / quantize_row / quantize_batch (gemv_q4.rs:33-95,
 * 747-798) run by the same device code the GEMV/GEMM use, honouring the
 * context's act-quant mode: x[m,k] -> qs[m,k], scales[m,k/32], sums[m,k/32]. */
int lgh_act_quant(lgh_ctx *ctx, const float *x, size_t m, size_t k, int8_t *qs, float *scales,
                  int32_t *sums);
/* dot_q4_q8_scalar (gemv_q4.rs:959-966) for nblocks BlockQ4 against a[nblocks*32]
 * int8, using the GEMV's device unpack + dot instructions; bit-exact target. */
int lgh_q4_block_dots(lgh_ctx *ctx, const void *blocks, const int8_t *a, size_t nblocks,
                      int32_t *out);
/* The first fused launch of lgh_q4_ffn_residual (one token, dim <= 2048)
 * alone, for tests: g, u, h = silu(g) * u [inter] in f32, and h's PerBlock
 * ActQ8 codes hq [inter] and scales hs [inter/32] as the second launch
 * consumes them (hq, hs may be NULL).  hidden is not modified. */
int lgh_q4_ffn_gate_up(lgh_ctx *ctx, const lgh_q4 *w1, const lgh_q4 *w3, const float *norm_w, float eps,
                       const float *hidden, float *g, float *u, float *h, int8_t *hq, float *hs);
/* Host-only check of the kernel dispatch (no device needed): the number of
 * GEMV launch shapes the planner can choose, over a sweep of row counts
 * around every planner threshold, every K up to 32768 and 1-3 matrices, that
 * have no compiled Q4 / Q8_0 kernel, plus the ragged matrix-core kernel's
 * plans for 2-64 tokens.  0 means every plan can launch. */
int lgh_gemv_plans_uncovered(void);
/* Integer Q8_0 x Q8 block dot (crates/llm-engine/src/weights.rs:206-209). */
int lgh_q8_block_dots(lgh_ctx *ctx, const void *blocks, const int8_t *a, size_t nblocks,
                      int32_t *out);
/* Per-block integer dots through the GEMM's matrix-core path (the matrix's
 * fp6 operand image, the activations' h/l split, the scaled MFMA):
 * out[m, n, k/32] = sum over block kb of nibble(W[n]) * qs[m] (qs int8
 * [m, k]); bit-exact target dot_q4_q8_scalar (gemv_q4.rs:959-966). */
int lgh_q4_mfma_block_dots(lgh_ctx *ctx, const lgh_q4 *w, const int8_t *qs, size_t m,
                           int32_t *out);

#ifdef __cplusplus
}
#endif
#endif
