// Internal declarations shared by the HIP sources of libllm_gpu_hip.so.
//
// Device layout of a Q4 matrix (built once at upload, immutable after):
//   qs plane: uint8 [n][bpr][16]  -- the 16 nibble bytes of each BlockQ4,
//             re-paired so that dword d (d = 0..3) of a block holds elements
//             8d..8d+3 in its low nibbles and 8d+4..8d+7 in its high nibbles
//             (still two's-complement nibbles, no offset);
//   sc plane: uint16 [n][bpr]     -- the block's f16 scale bits, unchanged.
// 16 + 2 = 18 bytes per 32 weights, exactly the BlockQ4 footprint, but every
// block's nibbles are 16-byte aligned so a lane moves a block with one
// 128-bit load.  Unpacking dword d: (d << 4) & 0xF0F0F0F0 yields elements
// 8d..8d+3 and d & 0xF0F0F0F0 yields 8d+4..8d+7, each as a signed int8
// equal to 16 x the nibble value -- natural element order, no sign fix-up.
// The factor 16 is exact and is removed once per output (x 1/16).
//
// Q8_0 matrix: qs plane int8 [n][bpr][32] (natural order) + sc plane f16.
//
// GEMM operand images (M > 1 path, fp6 matrix cores; codes defined in
// lgh_device.h).  Rows are grouped in 32-row tiles, blocks in pairs; every
// (tile, pair) record is one contiguous chunk that the GEMM copies verbatim
// into LDS:
//   weights     mx plane: [nt = ceil(n/32)][pp = ceil(bpr/2)] records of
//               kMxWRec bytes = 2 blocks x 768-byte code tile, then the 64 f32
//               block scales [block][row];
//   activations (per call, in the context workspace): [mt = ceil(m/32)][pp]
//               records of kMxARec bytes = 2 blocks x {h, l} x 768-byte code
//               tile, then 64 f32 block scales [block][token].
// A 768-byte code tile is plane0 (32 rows x 16 B: dwords 0-3 of each row)
// followed by plane1 (32 rows x 8 B: dwords 4-5).  Rows past n / m and blocks
// past bpr are zero codes with zero scales.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>

#include "../../include/llm_gpu_hip.h"

struct lgh_ctx {
  int device = 0;
  int cu_count = 0;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;
  int act_mode = LGH_ACT_PER_BLOCK;
  std::string err;
  // GEMM workspace: activation operand image, f32 row scales [m], split-K partials.
  void *ws = nullptr;
  size_t ws_bytes = 0;
  // Device staging for the host-pointer entry points.
  void *stage = nullptr;
  size_t stage_bytes = 0;
  // FFN block intermediates (h's codes / scales, or h in f32).
  void *ffn = nullptr;
  size_t ffn_bytes = 0;
  // This device's fixed scratch array (LGH_NOALLOC_SCRATCH_BYTES), shared by
  // every context on the device; looked up once per device at lgh_init.
  void *scratch = nullptr;
};

struct lgh_q4 {
  int device = 0;
  size_t n = 0, k = 0, bpr = 0;
  uint8_t *qs = nullptr;   // n*bpr*16 bytes
  uint16_t *sc = nullptr;  // n*bpr halves (same allocation as qs)
  uint8_t *mx = nullptr;   // GEMM operand image: nt*pp*kMxWRec bytes (own allocation), built on first GEMM use
  size_t nt = 0, pp = 0;   // 32-row tiles, block pairs
  std::mutex mx_mu;        // guards the one-time build of mx
};

struct lgh_q8 {
  int device = 0;
  size_t n = 0, k = 0, bpr = 0;
  int8_t *qs = nullptr;    // n*bpr*32 bytes
  uint16_t *sc = nullptr;
};

// ---- internal launchers (return hipError_t of the launch) ----------------
// All enqueue on `stream`; all pointers are device pointers.
namespace lgh {

constexpr size_t kMxTile = 768;                 // one 32-row x 32-code tile
constexpr size_t kMxWRec = 2 * kMxTile + 256;   // weights: 2 tiles + 64 f32 scales
constexpr size_t kMxARec = 4 * kMxTile + 256;   // activations: 2 x {h, l} tiles + 64 f32
// Buffer-load offsets are 32-bit: operand images must stay below this.
constexpr size_t kMxMaxBytes = size_t(1) << 31;
// Names the layout of the device images lgh_q4_export / lgh_q8_export write
// and lgh_*_import copy back without checking: the revision of the plane
// formats and the GEMM operand image (high 16 bits; raised whenever either
// changes) and the weight record size (low 16 bits).
constexpr uint32_t kImageLayout = (1u << 16) | static_cast<uint32_t>(kMxWRec);

// Weight operand image from the repacked nibble/scale planes (load time).
hipError_t launch_q4_mx_pack(const lgh_q4 *w, hipStream_t stream);
// The elementwise step an activation image launch applies to x before ActQ8:
// none, h = silu(x) * u (u [m][k]: the FFN's down-projection input, formed in
// place of the silu_mul launch) or rms_norm(x, nw, eps) (nw [k], ops.rs:8-23,
// in place of rms_norm writing the normed rows: one kernel forms each row's
// scale and writes its image).  Either way the image equals the op
// sequence's bit for bit.
struct ActPrologue {
  const float *u = nullptr;
  const float *nw = nullptr;
  float eps = 0.0f;
};
// Activation operand image: quantize the rows of x[m][k] (after the prologue)
// per ActQ8 (per_row selects the mode) straight into mt*pp records.  scratch:
// m floats (PerRow scales).
hipError_t launch_act_quant_mx(const float *x, ActPrologue pro, size_t m, size_t k, int per_row, uint8_t *mxa,
                               float *scratch, hipStream_t stream);
// Same record layout from already-quantized int8 activations aq [m][k] and
// their block scales [m][k/32] (scales null: 0).
hipError_t launch_act_split_mx(const int8_t *aq, const float *scales, size_t m, size_t k, uint8_t *mxa,
                               hipStream_t stream);

hipError_t launch_q4_repack(const uint8_t *raw_blocks, size_t nblocks, uint8_t *qs, uint16_t *sc,
                            hipStream_t stream);
hipError_t launch_q4_unpack(const uint8_t *qs, const uint16_t *sc, size_t nblocks, uint8_t *raw,
                            hipStream_t stream);
hipError_t launch_q8_repack(const uint8_t *raw_blocks, size_t nblocks, int8_t *qs, uint16_t *sc,
                            hipStream_t stream);
hipError_t launch_q8_unpack(const int8_t *qs, const uint16_t *sc, size_t nblocks, uint8_t *raw,
                            hipStream_t stream);
hipError_t launch_q4_quantize(const float *w, size_t nblocks, uint8_t *qs, uint16_t *sc,
                              hipStream_t stream);
hipError_t launch_q8_quantize(const float *w, size_t nblocks, int8_t *qs, uint16_t *sc,
                              hipStream_t stream);

// GEMV: y = W x for one or two matrices sharing x (pair).  w1 may be null.
// A workgroup of W waves covers 4*W/KW rows; each wave 4 rows x one K slice
// of 16*BPL blocks.  plan.ok is false when K is longer than one workgroup
// covers (K > 32768): the API then runs the act-quant + GEMM path with m = 1.
struct Q4GemvPlan {
  int BPL, KW, W, wgs_per_mat;
  bool ok;
};
// narrow: prefer 8-wave workgroups once that gives >= 2 per CU (Q4 rows;
// the Q8_0 head's 2x wider rows ran faster with 16 waves).
Q4GemvPlan plan_q4_gemv(size_t n, size_t bpr, int nmat, bool narrow = true);
// Plans (over a sweep of the planner's inputs) whose shape has no compiled
// Q4 / Q8_0 GEMV kernel; 0 when the dispatch tables cover the planner.
int gemv_plans_uncovered();
bool q4_gemv_quantize_once(size_t n, size_t bpr, int nmat);
hipError_t launch_q4_gemv(const lgh_q4 *w0, float *y0, const lgh_q4 *w1, float *y1, const float *x,
                          int mode, int per_row, hipStream_t stream);
// FFN gate/up stage of one decode token (lgh_ffn.hip): RMSNorm of x with
// norm_w (null: none), ActQ8 (per_row mode) of the result, g = W1 normed and
// u = W3 normed, h = silu(g) * u; writes the PerBlock ActQ8 codes hq [n] and
// scales hs [n/32] of h when hq is not null, and h / g / u in f32 to hf / g /
// u when those are not null.  W1, W3: n x k with n % 32 == 0, k <= 32 *
// kFfnMaxBpr (one workgroup holds all of x's codes).
constexpr size_t kFfnMaxBpr = 64;
bool ffn_gate_up_supported(const lgh_q4 *w1);
hipError_t launch_ffn_gate_up(const lgh_q4 *w1, const lgh_q4 *w3, const float *x, const float *norm_w, float eps,
                              int per_row, int8_t *hq, float *hs, float *hf, float *g, float *u,
                              hipStream_t stream);
// rms_norm (ops.rs:8-23) over `rows` rows of `dim`, and g = silu(g) * u
// (ops.rs:27-36, lfm2.rs:902-905); device pointers.
hipError_t launch_rms_norm(const float *x, const float *w, size_t dim, size_t rows, float eps, float *out,
                           hipStream_t stream);
hipError_t launch_silu_mul(float *g, const float *u, size_t n, hipStream_t stream);
// The same GEMV on activations already quantized per block (ActQ8 PerBlock
// codes [k] + scales [k/32], device pointers), e.g. by the FFN gate/up kernel.
hipError_t launch_q4_gemv_codes(const lgh_q4 *w, const int8_t *codes, const float *scales, float *y, int mode,
                                hipStream_t stream);
hipError_t launch_q4_gemv_any(const lgh_q4 *w0, float *y0, const lgh_q4 *w1, float *y1, const float *x,
                              const int8_t *codes, const float *scales, int mode, int per_row, hipStream_t stream);
// Up to three matrices with the same k in one launch sharing x and its
// quantization (the pair, or an attention block's q/k/v projections), with an
// optional rms_norm of x in the prologue (norm_w not null; one K slice, i.e.
// k <= 2048, and x not pre-quantized).  The plan is that of the total rows.
size_t gemv_multi_rows(const lgh_q4 *const *w, int nmat);
hipError_t launch_q4_gemv_multi(const lgh_q4 *const *w, float *const *y, int nmat, const float *x,
                                const int8_t *codes, const float *scales, const float *norm_w, float eps, int mode,
                                int per_row, hipStream_t stream);
// Batched GEMV for 2 <= m <= 4 rows of x, quantized inside the kernel
// (one launch).  ok is false when the shape does not fit.
struct Q4BatchPlan {
  int BPL, KW;
  bool ok;
};
Q4BatchPlan plan_q4_batch(size_t m, size_t bpr);
// Rows of > 64 blocks are quantized once (act_quant_kernel) and the kernel
// reads the codes: inside it, every workgroup would quantize all m rows.
bool q4_batch_quantize_once(size_t bpr);
// codes / scales (ActQ8 of the m rows, [m][k] and [m][k/32]) replace x when non-null.
hipError_t launch_q4_gemv_batch(const lgh_q4 *w, const float *x, const int8_t *codes, const float *scales, float *y,
                                size_t m, int mode, int per_row, hipStream_t stream);
// Batched GEMV on the matrix cores for 2 <= m <= 64 (TT 16-token tiles, KW
// K slices, CB-block chunks, RG 16-row groups per workgroup) on an
// activation image written by act_quant_mma, with mt = ceil(m/16) token
// tiles and pq = ceil(k/128) block quads:
//   codes  [mt][2*pq pairs][64 lanes][16 B]: lane (t, g) = token t (0..15),
//          K group g (0..3) holds codes 8g..8g+7 of the pair's two blocks
//          (the B operand of v_mfma_i32_16x16x32_i8, 8 bytes per block);
//   scales [mt][pq][16 tokens][4 blocks] f32.
// Padding tokens and blocks hold 0.
struct Q4MmaPlan {
  int TT, KW, CB, RG;
  bool ok;
};
// any_shape: a plan for every 1 <= m <= 64 and row length, also where the
// route table prefers the GEMM (for matrices that cannot hold a GEMM image).
Q4MmaPlan plan_q4_mma(size_t n, size_t m, size_t bpr, bool any_shape = false);
hipError_t launch_act_quant_mma(const float *x, ActPrologue pro, size_t m, size_t k, int per_row, uint8_t *codes,
                                float *scales, float *scratch, hipStream_t stream);
// The same image from ActQ8 codes [m][k] and block scales [m][k/32].
hipError_t launch_act_codes_mma(const int8_t *aq, const float *as, size_t m, size_t k, uint8_t *codes,
                                float *scales, hipStream_t stream);
hipError_t launch_q4_gemv_mma(const lgh_q4 *w, const uint8_t *codes, const float *scales, float *y, size_t m,
                              int mode, hipStream_t stream, bool any_shape = false);
// Q8_0 GEMV; K ranges of kQ8GemvMaxK (the Q4 GEMV plan's reach) and 65535
// tokens per launch.  With norm_w not null (k <= kQ8GemvMaxK only) each
// token's row is rms_norm'd in the prologue (eps as rms_norm).
constexpr size_t kQ8GemvMaxK = 32768;
hipError_t launch_q8_gemv(const lgh_q8 *w, const float *x, float *y, size_t tokens, const float *norm_w, float eps,
                          hipStream_t stream);

// Batched activation quantization: x[m][k] -> qs[m][k], scales[m][k/32]
// (+ sums if non-null).  row_scale: scratch of m floats (used for per_row).
hipError_t launch_act_quant(const float *x, size_t m, size_t k, int per_row, int8_t *qs,
                            float *scales, int32_t *sums, float *row_scale, hipStream_t stream);

// GEMM on an activation operand image: y[j][m][n_j] (+)= x[m][k] . W[j]^T for
// 1..3 matrices with the same k, one launch (the workgroups of all matrices
// in one grid, one split-K reduce).  plan_q4_gemm() is what a call of m
// tokens wants: the number of K splits across workgroups and of K groups
// inside one.  Both fix the f32 summation order, so the caller passes the plan
// of the whole call to every token chunk it cuts the call into.  `part` must
// hold splits * m * (sum of n) floats when splits > 1 (hipErrorInvalidValue
// otherwise, nothing launched).
struct GemmPlan {
  int splits = 1;   // K splits across workgroups, added by a reduce launch
  int kgroups = 1;  // 1, 2 or 4 (splits == 1, >= kgroups block pairs): K parts in one workgroup
};
GemmPlan plan_q4_gemm(const lgh_q4 *const *w, int nmat, size_t m);
hipError_t launch_q4_gemm(const lgh_q4 *const *w, int nmat, const uint8_t *mxa, float *const *y, size_t m, int mode,
                          GemmPlan plan, float *part, size_t part_floats, hipStream_t stream);

// Measurement probes: an empty kernel of `wgs` workgroups, and a plain read
// of `bytes` (a multiple of 16, 16-byte aligned) with per_thread (1, 2, 4, 8)
// 16-byte loads per thread, one f32 sum per workgroup into out
// [probe_read_workgroups(bytes, per_thread)].
size_t probe_read_workgroups(size_t bytes, int per_thread);
hipError_t launch_probe_empty(int wgs, hipStream_t stream);
hipError_t launch_probe_read(const void *src, size_t bytes, int per_thread, float *out, hipStream_t stream);

// Test hooks.
hipError_t launch_q4_block_dots(const uint8_t *qs, const int8_t *a, size_t nblocks, int32_t *out,
                                hipStream_t stream);
hipError_t launch_q8_block_dots(const int8_t *qs, const int8_t *a, size_t nblocks, int32_t *out,
                                hipStream_t stream);
// Exact block dots through the GEMM's operand images and matrix-core path:
// mxa from launch_act_split_mx, out[m][n][bpr].
hipError_t launch_q4_mfma_block_dots(const lgh_q4 *w, const uint8_t *mxa, size_t m, int32_t *out,
                                     hipStream_t stream);

}  // namespace lgh
