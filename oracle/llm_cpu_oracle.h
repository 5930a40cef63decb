/*
 * CPU oracle for the Q4_32 / Q8_0 block-quantized matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a C restatement of llmhost's CPU
 * algorithm (crates llm-quant and llm-cpu, plus the Q8_0 head GEMV in
 * llm-engine).  Only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py may load it, and only as the reference results or as the reported
 * CPU baseline.  The GPU library never links or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative
 * to the llmhost repository root).  Parity pins for each function are listed
 * in tests/test_oracle_*.py; nothing here is "parity unpinned".
 */
#ifndef LLM_CPU_ORACLE_H
#define LLM_CPU_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OQ_BLOCK 32       /* llm-quant/src/lib.rs:12 BLOCK_SIZE        */
#define OQ_TILE_N 16      /* llm-cpu/src/gemv_q4.rs:19 TILE_N          */
#define OQ_TILE_QS 256    /* gemv_q4.rs:21 TILE_QS                     */
#define OQ_TILE_STRIDE 320 /* gemv_q4.rs:23 TILE_STRIDE                */

/* llm-quant/src/lib.rs:54-58 BlockQ4 (natural layout: LE f16, 16 qs bytes). */
typedef struct {
  uint16_t scale;
  uint8_t qs[16];
} oq_block_q4;

/* llm-quant/src/lib.rs:17-21 BlockQ8_0 (LE f16, 32 int8). */
typedef struct {
  uint16_t scale;
  int8_t qs[32];
} oq_block_q8;

/* Kernel selector, llm-cpu/src/gemv_q4.rs:302-307 Q4Kernel. */
enum { OQ_KERNEL_SCALAR = 0, OQ_KERNEL_AVX2 = 1, OQ_KERNEL_VNNI = 2,
       OQ_KERNEL_AMX = 3 /* GEMM only: amx.rs gemm_tiles_amx (m >= 16, no add) */ };

/* ---- f16 (half 2.7.1 f16::to_f32 / from_f32: exact / round-nearest-even) */
float oq_f16_to_f32(uint16_t h);
uint16_t oq_f32_to_f16(float f);

/* ---- llm-quant block formats ------------------------------------------ */
void oq_q8_quantize(const float src[32], oq_block_q8 *dst);      /* lib.rs:26-37 */
void oq_q8_dequantize(const oq_block_q8 *b, float dst[32]);      /* lib.rs:40-45 */
void oq_q4_quantize(const float src[32], oq_block_q4 *dst);      /* lib.rs:63-79 */
int8_t oq_q4_nibble(const oq_block_q4 *b, int i);                /* lib.rs:83-92 */
void oq_q4_dequantize(const oq_block_q4 *b, float dst[32]);      /* lib.rs:95-100 */
/* lib.rs:104-141 slice helpers; return 0, or -1 when len % 32 != 0. */
int oq_quantize_q4(const float *x, size_t len, oq_block_q4 *out);
int oq_quantize_q8_0(const float *x, size_t len, oq_block_q8 *out);

/* ---- activation quantization, gemv_q4.rs:62-95 / 747-798 ------------- */
/* x[m*k] -> qs[m*k] (natural order), scales[m*k/32], sums[m*k/32].
 * per_row=0: ActQuant::PerBlock, 1: ActQuant::PerRow.  Returns -1 if k%32. */
int oq_act_quantize(const float *x, size_t m, size_t k, int per_row,
                    int8_t *qs, float *scales, int32_t *sums);

/* ---- per-block integer dots ------------------------------------------- */
int32_t oq_dot_q4_q8(const oq_block_q4 *b, const int8_t a[32]);   /* gemv_q4.rs:959-966 */
/* VNNI identity dpbusd(s+8, a) - 8*sum(a), gemv_q4.rs:1034-1050 */
int32_t oq_dot_q4_q8_offset(const oq_block_q4 *b, const int8_t a[32], int32_t a_sum);
int32_t oq_dot_q8_q8(const oq_block_q8 *b, const int8_t a[32]);   /* weights.rs:206-209 */

/* ---- packed Q4 matrix, gemv_q4.rs:97-261 ------------------------------ */
typedef struct {
  size_t n, k, n_tiles;
  uint8_t *tiles; /* n_tiles * (k/32) * 320 bytes */
} oq_q4_matrix;

oq_q4_matrix *oq_q4_from_blocks(size_t n, size_t k, const oq_block_q4 *blocks);
void oq_q4_free(oq_q4_matrix *w);

/* ---- llm-cpu entry points -------------------------------------------- */
/* kernel: OQ_KERNEL_*, or -1 for detect_q4_kernel() (gemv_q4.rs:311-322).
 * threads: session width as with_threads(threads, ..) (pool.rs:287-299).  */
int oq_detect_kernel(void);
/* gemv_q4 / gemv_q4_add (gemv_q4.rs:344-363); add=1 is AccMode::AddF64. */
void oq_gemv_q4(const oq_q4_matrix *w, const float *x, float *out, int add,
                int per_row, int kernel, int threads);
/* gemv_q4_prep on pre-quantized activations (gemv_q4.rs:366-393). */
void oq_gemv_q4_prep(const oq_q4_matrix *w, const int8_t *qs, const float *scales,
                     float *out, int add, int kernel, int threads);
/* gemv_q4_pair (gemv_q4.rs:396-443). */
void oq_gemv_q4_pair(const oq_q4_matrix *wg, const oq_q4_matrix *wu, const float *x,
                     float *out_g, float *out_u, int per_row, int kernel, int threads);
/* gemm_q4 / gemm_q4_add (gemv_q4.rs:686-722).  With kernel -1 (detected) or
 * OQ_KERNEL_AMX, m >= 16 and no add take the AMX-INT8 tiles when the host
 * can run them (amx.rs; gemv_q4.rs:711); otherwise the tile kernels. */
int oq_amx_ready(void); /* amx.rs:29-66: CPU and OS can run AMX-INT8 tiles */
void oq_gemm_q4(const oq_q4_matrix *w, const float *x, float *out, size_t m, int add,
                int per_row, int kernel, int threads);
/* q8_apply (llm-engine/src/weights.rs:194-227): blocks row-major [n][k/32]. */
void oq_q8_apply(const oq_block_q8 *blocks, size_t n, size_t k, const float *x,
                 size_t tokens, float *out, int threads);

/* ---- decode FFN block (llm-cpu/src/ops.rs, llm-engine/src/lfm2.rs) ------ */
/* rms_norm (ops.rs:8-23): rows of dim elements; f64 sequential sum of
 * squares, scale = f32(1/sqrt(sumsq*(1/dim) + eps)) in f64, out = w*(x*scale). */
void oq_rms_norm(const float *x, const float *weight, size_t dim, size_t rows, float eps, float *out);
/* silu_inplace (ops.rs:27-36) on g, then g *= u (lfm2.rs:902-905). */
void oq_silu_mul(float *g, const float *u, size_t n);
/* Lfm2::ffn_residual (lfm2.rs:861-881) / ffn_residual_in (:883-911) over
 * `tokens` rows: normed = rms_norm(hidden) (norm_w == NULL: normed = hidden),
 * g, u = apply_pair (pair GEMV for one token, two GEMMs otherwise), silu(g)*u,
 * hidden = apply_add(w2, h). */
void oq_ffn_residual(const oq_q4_matrix *w1, const oq_q4_matrix *w3, const oq_q4_matrix *w2,
                     const float *norm_w, float eps, float *hidden, size_t tokens, int per_row, int kernel,
                     int threads);

/* ---- pool (pool.rs:212-241 thread_range / for_ranges) ------------------ */
void oq_thread_range(size_t tid, size_t nthreads, size_t n, size_t *start, size_t *end);
int oq_max_threads(void); /* pool.rs:22 MAX_THREADS = 64 */
int oq_cpu_has(const char *feature); /* "avx2", "avx512f", "avx512vnni", "avx512bw" */

#ifdef __cplusplus
}
#endif
#endif
