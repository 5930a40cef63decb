// M = 1 kernels for gfx950: fused activation-quant + Q4 / Q8_0 GEMV.
//
// Q4 GEMV (replaces crates/llm-cpu/src/gemv_q4.rs:344-443, 499-667):
//   * each 16-lane DPP row of a wave owns one weight row, so a wave covers 4
//     rows; a workgroup of W waves is (W/KW) row groups x KW K slices, and
//     lane c of a row walks blocks slice*16*BPL + c + 16j (j < BPL);
//   * issue order: (1) this thread's float4s of x, (2) every weight load of
//     the lane -- BPL 128-bit nibble loads + BPL f16 scale loads, all
//     branch-free raw buffer loads (out of range -> 0) -- then (3) the ActQ8
//     quantization of x into LDS, shared by the workgroup, which waits only
//     for (1), so the HBM latency of (2) overlaps the prologue;
//   * per block: 8 v_dot4_i32_i8 of the unpacked nibbles (x16) against the
//     LDS codes, acc = fma(f32(16*idot), sw*sa, acc) -- the VNNI kernel's fold
//     (gemv_q4.rs:659-661) in a different summation order;
//   * 4 DPP adds give every lane of a DPP row its row's slice sum; slice sums
//     meet in LDS and are added in slice order (deterministic), then Assign
//     or AddF64 (gemv_q4.rs:486-497) after removing the x16 (exact).
#include <algorithm>
#include <type_traits>

#include "lgh_device.h"
#include "lgh_internal.h"

namespace lgh {

// Every (BPL, KW, W) shape plan_q4_gemv() can return, for both `narrow`
// values; the Q4 and the Q8_0 dispatch tables are generated from this one
// list, and lgh_gemv_plans_uncovered() checks the planner against it.
#define LGH_GEMV_SHAPES(X)                                                                             \
  X(1, 1, 16) X(1, 1, 8) X(1, 1, 4) X(2, 1, 16) X(2, 1, 8) X(2, 1, 4) X(3, 1, 16) X(3, 1, 8) X(3, 1, 4) \
  X(4, 1, 16) X(4, 1, 8) X(4, 1, 4) X(1, 2, 4) X(2, 2, 4) X(4, 2, 16) X(2, 4, 16) X(2, 4, 8) X(2, 4, 4)  \
  X(4, 4, 16) X(2, 8, 16) X(2, 8, 8) X(4, 8, 16) X(2, 16, 16) X(4, 16, 16)

// (TT, KW, CB, RG) of every ragged MMA kernel shape plan_q4_mma can choose;
// the dispatch is generated from this list too.
#define LGH_MMA_SHAPES(X)                                                                           \
  X(1, 1, 8, 4) X(1, 2, 8, 2) X(1, 4, 8, 1) X(1, 8, 8, 1) X(2, 1, 8, 4) X(2, 2, 8, 2) X(2, 4, 8, 1) \
  X(2, 8, 8, 1) X(3, 1, 8, 4) X(3, 2, 8, 2) X(3, 4, 8, 1) X(3, 8, 8, 1) X(3, 8, 4, 1) X(4, 1, 8, 4) \
  X(4, 2, 8, 2) X(4, 4, 8, 1) X(4, 8, 8, 1)

namespace {


// Up to three matrices with the same k share one launch and one activation
// quantization (gemv_q4_pair; the q/k/v projections of an attention block):
// workgroups [0, wgs0) cover matrix 0, the next wgs1 matrix 1, the rest
// matrix 2.
struct Q4GemvArgs {
  const uint8_t *qs0;
  const uint16_t *sc0;
  float *y0;
  const uint8_t *qs1;
  const uint16_t *sc1;
  float *y1;
  const uint8_t *qs2;
  const uint16_t *sc2;
  float *y2;
  const float *x;
  const int8_t *aq;  // PREQ: ActQ8 codes [k] and scales [k/32] instead of x
  const float *as;
  const float *nw;   // NORM: rms_norm weight [k]
  double inv_k;      // NORM: 1 / k in f64, as the reference computes it (ops.rs:12)
  float eps;
  int n0, n1, n2;    // rows of each matrix
  int bpr;
  int wgs0, wgs1;
  int mode;
  int per_row;
};

// BPL blocks per lane and row, KW K slices, W waves; 4*(W/KW) rows per workgroup.
// PREQ: the activations arrive already quantized (codes + scales, written by
// the kernel that produced them), so the prologue is two short loads into
// LDS instead of loading and quantizing x.
// NORM: x is rms_norm'd first (crates/llm-cpu/src/ops.rs:8-23, as
// rms_norm_kernel): every workgroup holds all of x anyway, so it sums the
// squares in f64 (DPP tree per wave, then the wave sums in order), takes
// scale = f32(1 / sqrt(sum * (1/k) + eps)) in f64 and quantizes
// nw * (x * scale).
template <int BPL, int KW, int W, bool PREQ, bool NORM = false>
__global__ __launch_bounds__(W * kWave) void q4_gemv_kernel(Q4GemvArgs a) {
  constexpr int THREADS = W * kWave;
  constexpr int KB = 16 * BPL * KW;  // blocks covered by the workgroup (>= bpr)
  constexpr int RG = W / KW;
  // Long rows (x at least twice the workgroup's float4s) quantize in 4-lane
  // groups of 32-byte chunks (XP per thread), which halves the per-block
  // work per element; shorter rows keep 8-lane groups of float4s, which
  // spreads their few blocks over twice the waves.
  constexpr bool PAIRS = KB * 8 >= 2 * THREADS;
  constexpr int XP = (KB * 4 + THREADS - 1) / THREADS;
  constexpr int XJ = PAIRS ? 2 * XP : (KB * 8 + THREADS - 1) / THREADS;  // float4s of x per thread
  static_assert(W % KW == 0, "slices divide the waves");
  static_assert(!(PREQ && NORM), "the norm needs x");
  __shared__ __align__(16) int8_t s_qs[KB * 32];
  __shared__ float s_sa[KB];
  __shared__ float s_red[W];
  __shared__ double s_ss[NORM ? W : 1];
  __shared__ float s_part[KW > 1 ? RG * 4 * KW : 1];
  const int bpr = a.bpr;
  int wg = blockIdx.x;
  const uint8_t *qs = a.qs0;
  const uint16_t *sc = a.sc0;
  float *y = a.y0;
  int n = a.n0;
  if (wg >= a.wgs0) {
    wg -= a.wgs0;
    qs = a.qs1;
    sc = a.sc1;
    y = a.y1;
    n = a.n1;
    if (wg >= a.wgs1) {
      wg -= a.wgs1;
      qs = a.qs2;
      sc = a.sc2;
      y = a.y2;
      n = a.n2;
    }
  }
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = uniform(tid / kWave);
  const int rg = wave / KW, ks = wave % KW;
  const int row0 = (wg * RG + rg) * 4;  // first row of this wave
  const int rows = uniform(max(0, min(4, n - row0)));
  const int r = lane >> 4, c = lane & 15;
  const int kb0 = ks * 16 * BPL + c;

  // (1) x: XJ float4s per thread (XP chunk pairs with PAIRS) -- or (PREQ) the codes as 16-byte
  // chunks and the block scales.
  constexpr int QJ = PREQ ? (KB * 2 + THREADS - 1) / THREADS : 1;
  constexpr int SJ = PREQ ? (KB + THREADS - 1) / THREADS : 1;
  float4 xv[XJ];
  float4 nv[NORM ? XJ : 1];
  uint4 qv[QJ];
  float sv[SJ];
  if constexpr (PREQ) {
    const auto qr = make_rsrc(a.aq, static_cast<uint32_t>(bpr) * 32u);
    const auto ar = make_rsrc(a.as, static_cast<uint32_t>(bpr) * 4u);
#pragma unroll
    for (int j = 0; j < QJ; j++) qv[j] = buf_load16(qr, static_cast<uint32_t>(tid + j * THREADS) * 16u);
#pragma unroll
    for (int j = 0; j < SJ; j++) sv[j] = buf_load_f32(ar, static_cast<uint32_t>(tid + j * THREADS) * 4u);
  } else {
    const auto xr = make_rsrc(a.x, static_cast<uint32_t>(bpr) * 128u);
    const auto nr = make_rsrc(a.nw, NORM ? static_cast<uint32_t>(bpr) * 128u : 0u);
    if constexpr (PAIRS) {
#pragma unroll
      for (int j = 0; j < XP; j++) {
        const uint32_t c = static_cast<uint32_t>(tid + j * THREADS) * 32u;
        xv[2 * j] = buf_load_f4(xr, c);
        xv[2 * j + 1] = buf_load_f4(xr, c + 16u);
        if constexpr (NORM) {
          nv[2 * j] = buf_load_f4(nr, c);
          nv[2 * j + 1] = buf_load_f4(nr, c + 16u);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < XJ; j++) {
        xv[j] = buf_load_f4(xr, static_cast<uint32_t>(tid + j * THREADS) * 16u);
        if constexpr (NORM) nv[j] = buf_load_f4(nr, static_cast<uint32_t>(tid + j * THREADS) * 16u);
      }
    }
  }

  // (1b) x at least twice the workgroup's float4s, (PREQ) the codes, or (NORM)
  // x and the norm weight: every wave's activation requests are queued before
  // any wave's weight requests.  Without the barrier, waves that start later
  // issue them behind the earlier waves' weight loads: at K = 8192 x arrived
  // up to 1.7 us after issue (0.8 us with it); the codes GEMV of the FFN
  // block's down projection took 3.98 us against 3.78 us with it, the norm +
  // conv in_proj (K=1536, N=4608) 4.0 against 3.5 us and the norm + gate/up
  // pair 5.1 against 4.76 us (interleaved A/B).
  if constexpr (PREQ || PAIRS || NORM) {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  }

  // (2) every weight load of this lane (rows past n fall outside the resource).
  const size_t blk0 = static_cast<size_t>(row0) * bpr;
  const auto wr = make_rsrc(qs + blk0 * 16, static_cast<uint32_t>(rows * bpr) * 16u);
  const auto sr = make_rsrc(sc + blk0, static_cast<uint32_t>(rows * bpr) * 2u);
  uint4 w[BPL];
  uint16_t s[BPL];
#pragma unroll
  for (int j = 0; j < BPL; j++) {
    const int kb = kb0 + 16 * j;
    const uint32_t blk = static_cast<uint32_t>(r * bpr + kb);
    w[j] = buf_load16<kAuxNT>(wr, kb < bpr ? blk * 16u : kOOB);
    s[j] = buf_load_u16(sr, kb < bpr ? blk * 2u : kOOB);
  }

  // (2b) NORM: x = nw * (x * scale); elements past k are 0 in x and nw.
  if constexpr (NORM) rms_norm_regs<THREADS, XJ>(xv, nv, a.inv_k, a.eps, s_ss);

  // (3) x -> LDS codes (chunks and scales past the row load as 0).
  if constexpr (PREQ) {
#pragma unroll
    for (int j = 0; j < QJ; j++) {
      const int i = tid + j * THREADS;
      if (i < KB * 2) reinterpret_cast<uint4 *>(s_qs)[i] = qv[j];
    }
#pragma unroll
    for (int j = 0; j < SJ; j++) {
      const int i = tid + j * THREADS;
      if (i < KB) s_sa[i] = sv[j];
    }
    __syncthreads();
  } else if constexpr (PAIRS) {
    quantize_pairs_to_lds<THREADS, XP>(xv, bpr, a.per_row, s_qs, s_sa, s_red);
  } else {
    quantize_regs_to_lds<THREADS, XJ>(xv, bpr, a.per_row, s_qs, s_sa, s_red);
  }

  // (4) dots + fold, branch-free so every LDS read is issued before the
  // weights arrive: a block past the row has zero nibbles and a zero scale
  // (out-of-range loads) and reads block 0's codes, so it adds exactly 0.
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < BPL; j++) {
    const int kb = kb0 + 16 * j;
    const int kbc = kb < bpr ? kb : 0;
    const v4i *ap = reinterpret_cast<const v4i *>(s_qs + kbc * 32);
    const int d = dot_q4_block16(w[j], ap[0], ap[1]);
    acc = fmaf(static_cast<float>(d), h2f(s[j]) * s_sa[kbc], acc);
  }
  // (4b) AddF64 / AddF32: the old y of the row this lane stores, read now so
  // that its round trip overlaps the reductions (branch-free: the other lanes
  // read past the range).  Read after the reductions it cost 0.35 us over
  // Assign; here 0.1-0.25 us (K=8192, N=1536 AddF64 3.88 -> 3.65 us; K=1536,
  // N=8192 3.36 -> 3.24 us; interleaved A/B).  Read in the prologue instead,
  // beside the weight loads, it was slower than either (3.79 -> 4.30 us).
  float y_old = 0.0f;
  if (a.mode != LGH_ASSIGN) {  // uniform
    const int srow = KW == 1 ? (c == 0 && r < rows ? row0 + r : -1) : (ks == 0 && lane < rows ? row0 + lane : -1);
    y_old = buf_load_f32(make_rsrc(y, static_cast<uint32_t>(n) * 4u),
                         srow >= 0 ? static_cast<uint32_t>(srow) * 4u : kOOB);
  }
  // (5) 16-lane row sums (every lane of a DPP row ends with its row's sum).
  acc += dpp<0xB1>(acc);   // quad_perm [1,0,3,2]
  acc += dpp<0x4E>(acc);   // quad_perm [2,3,0,1]
  acc += dpp<0x141>(acc);  // row_half_mirror
  acc += dpp<0x140>(acc);  // row_mirror
  if constexpr (KW == 1) {
    if (c == 0 && r < rows) store_row_old(y, row0 + r, acc, a.mode, y_old);
  } else {
    if (c == 0) s_part[(rg * 4 + r) * KW + ks] = acc;
    __syncthreads();
    if (ks == 0 && lane < rows) {
      float sum = 0.0f;
#pragma unroll
      for (int k = 0; k < KW; k++) sum += s_part[(rg * 4 + lane) * KW + k];
      store_row_old(y, row0 + lane, sum, a.mode, y_old);
    }
  }
}

template <int BPL, int KW, int W, bool PREQ = false, bool NORM = false>
hipError_t launch_gemv16(const Q4GemvArgs &a, int total_wgs, hipStream_t st) {
  hipLaunchKernelGGL((q4_gemv_kernel<BPL, KW, W, PREQ, NORM>), dim3(total_wgs), dim3(W * kWave), 0, st, a);
  return hipGetLastError();
}

// The NORM prologue needs the whole row in one slice: it exists for KW = 1.
template <int BPL, int KW, int W>
hipError_t dispatch_q4(const Q4GemvArgs &a, int total_wgs, bool preq, bool norm, hipStream_t st) {
  if (preq) return launch_gemv16<BPL, KW, W, true>(a, total_wgs, st);
  if constexpr (KW == 1) {
    if (norm) return launch_gemv16<BPL, KW, W, false, true>(a, total_wgs, st);
  }
  return launch_gemv16<BPL, KW, W, false>(a, total_wgs, st);
}

// ---- batched Q4 GEMV, 2 <= M <= 4 -----------------------------------------
// Tiny ragged batches (crates/llm-cpu/src/gemv_q4.rs:686-722 with m <= 4) are
// weight-stream bound like the GEMV and need no second launch: the workgroup
// quantizes the T = 4 token rows of x in its prologue (cheap for so few
// tokens), then reads each 18-byte nibble block once and dots it against the
// T code rows in LDS: one nibble unpack, then 8 v_dot4_i32_i8 and one fold per
// token.  Row mapping, slices and DPP row sums as in q4_gemv_kernel.
struct Q4BatchArgs {
  const uint8_t *qs;
  const uint16_t *sc;
  const float *x;    // f32 [m][k]
  const int8_t *aq;  // PREQ: ActQ8 codes [m][k] and scales [m][k/32] instead of x
  const float *as;
  float *y;  // [m][n]
  int n, bpr, m, mode, per_row;
};

// PREQ: the T rows arrive already quantized (act_quant_kernel, once for
// every workgroup) instead of each workgroup quantizing all of them.
template <int T, int BPL, int KW, int W, bool PREQ>
__global__ __launch_bounds__(W * kWave) void q4_gemv_batch_kernel(Q4BatchArgs a) {
  constexpr int THREADS = W * kWave;
  constexpr int KB = 16 * BPL * KW;
  constexpr int RG = W / KW;
  constexpr int XJ = PREQ ? 1 : (KB * 8 + THREADS - 1) / THREADS;
  constexpr int QJ = PREQ ? (KB * 2 + THREADS - 1) / THREADS : 1;  // 16-byte code chunks per thread and row
  constexpr int SJ = PREQ ? (KB + THREADS - 1) / THREADS : 1;      // block scales per thread and row
  static_assert(W % KW == 0, "slices divide the waves");
  __shared__ __align__(16) int8_t s_qs[T][KB * 32];
  __shared__ float s_sa[T][KB];
  __shared__ float s_red[W];
  __shared__ float s_part[KW > 1 ? RG * 4 * KW * T : 1];
  const int bpr = a.bpr;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = uniform(tid / kWave);
  const int rg = wave / KW, ks = wave % KW;
  const int row0 = (blockIdx.x * RG + rg) * 4;
  const int rows = uniform(max(0, min(4, a.n - row0)));
  const int r = lane >> 4, c = lane & 15;
  const int kb0 = ks * 16 * BPL + c;

  // (1) the x rows -- or (PREQ) their codes and block scales -- (tokens >= m
  // read as 0), issued before the weights so that waiting for them leaves the
  // weight loads in flight.
  float4 xv[T][XJ];
  uint4 qv[T][QJ];
  float sv[T][SJ];
#pragma unroll
  for (int t = 0; t < T; t++) {
    if constexpr (PREQ) {
      const auto qr = make_rsrc(a.aq + static_cast<size_t>(t) * bpr * 32, t < a.m ? static_cast<uint32_t>(bpr) * 32u : 0u);
      const auto ar = make_rsrc(a.as + static_cast<size_t>(t) * bpr, t < a.m ? static_cast<uint32_t>(bpr) * 4u : 0u);
#pragma unroll
      for (int j = 0; j < QJ; j++) qv[t][j] = buf_load16(qr, static_cast<uint32_t>(tid + j * THREADS) * 16u);
#pragma unroll
      for (int j = 0; j < SJ; j++) sv[t][j] = buf_load_f32(ar, static_cast<uint32_t>(tid + j * THREADS) * 4u);
    } else {
      const auto xr =
          make_rsrc(a.x + static_cast<size_t>(t) * bpr * 32, t < a.m ? static_cast<uint32_t>(bpr) * 128u : 0u);
#pragma unroll
      for (int j = 0; j < XJ; j++) xv[t][j] = buf_load_f4(xr, static_cast<uint32_t>(tid + j * THREADS) * 16u);
    }
  }

  // (1b) PREQ over four or more K slices: every wave's code requests before
  // any wave's weight requests (M=2 / 4, K=8192, N=2048: 7.41 / 7.49 ->
  // 7.26 / 7.32 us; the x path at K=2048 and the codes at K=4096 measured
  // no gain or a loss, interleaved A/B).
  if constexpr (PREQ && KW >= 4) {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  }

  // (2) every weight load of this lane (rows past n read as 0).
  const size_t blk0 = static_cast<size_t>(row0) * bpr;
  const auto wr = make_rsrc(a.qs + blk0 * 16, static_cast<uint32_t>(rows * bpr) * 16u);
  const auto swr = make_rsrc(a.sc + blk0, static_cast<uint32_t>(rows * bpr) * 2u);
  uint4 w[BPL];
  uint16_t s[BPL];
#pragma unroll
  for (int j = 0; j < BPL; j++) {
    const int kb = kb0 + 16 * j;
    const uint32_t blk = static_cast<uint32_t>(r * bpr + kb);
    w[j] = buf_load16<kAuxNT>(wr, kb < bpr ? blk * 16u : kOOB);
    s[j] = buf_load_u16(swr, kb < bpr ? blk * 2u : kOOB);
  }

  // (3) codes into LDS.
  if constexpr (PREQ) {
#pragma unroll
    for (int t = 0; t < T; t++) {
#pragma unroll
      for (int j = 0; j < QJ; j++) {
        const int i = tid + j * THREADS;
        if (i < KB * 2) reinterpret_cast<uint4 *>(s_qs[t])[i] = qv[t][j];
      }
#pragma unroll
      for (int j = 0; j < SJ; j++) {
        const int i = tid + j * THREADS;
        if (i < KB) s_sa[t][i] = sv[t][j];
      }
    }
    __syncthreads();
  } else {
#pragma unroll
    for (int t = 0; t < T; t++) {
      const float rs = row_scale_of<THREADS, XJ>(xv[t], a.per_row, s_red);
      quant_regs<THREADS, XJ>(xv[t], bpr, a.per_row != 0, rs, s_qs[t], s_sa[t]);
    }
  }

  // (4) per block: one unpack, then T dots and folds.
  float acc[T];
#pragma unroll
  for (int t = 0; t < T; t++) acc[t] = 0.0f;
#pragma unroll
  for (int j = 0; j < BPL; j++) {
    const int kb = kb0 + 16 * j;
    const int kbc = kb < bpr ? kb : 0;  // past the row: zero weights and scale, adds exactly 0
    const int u[8] = {nib_lo16(w[j].x), nib_hi16(w[j].x), nib_lo16(w[j].y), nib_hi16(w[j].y),
                      nib_lo16(w[j].z), nib_hi16(w[j].z), nib_lo16(w[j].w), nib_hi16(w[j].w)};
    const float sw = h2f(s[j]);
#pragma unroll
    for (int t = 0; t < T; t++) {
      const v4i *ap = reinterpret_cast<const v4i *>(&s_qs[t][kbc * 32]);
      const v4i a0 = ap[0], a1 = ap[1];
      int d = sdot4(u[0], a0.x, 0);
      d = sdot4(u[1], a0.y, d);
      d = sdot4(u[2], a0.z, d);
      d = sdot4(u[3], a0.w, d);
      d = sdot4(u[4], a1.x, d);
      d = sdot4(u[5], a1.y, d);
      d = sdot4(u[6], a1.z, d);
      d = sdot4(u[7], a1.w, d);
      acc[t] = fmaf(static_cast<float>(d), sw * s_sa[t][kbc], acc[t]);
    }
  }
  // (5) row sums, slices in order, epilogue per token.
#pragma unroll
  for (int t = 0; t < T; t++) {
    acc[t] += dpp<0xB1>(acc[t]);
    acc[t] += dpp<0x4E>(acc[t]);
    acc[t] += dpp<0x141>(acc[t]);
    acc[t] += dpp<0x140>(acc[t]);
  }
  if constexpr (KW == 1) {
    if (c == 0 && r < rows) {
#pragma unroll
      for (int t = 0; t < T; t++)
        if (t < a.m) store_row(a.y + static_cast<size_t>(t) * a.n, row0 + r, acc[t], a.mode);
    }
  } else {
    if (c == 0) {
#pragma unroll
      for (int t = 0; t < T; t++) s_part[((rg * 4 + r) * T + t) * KW + ks] = acc[t];
    }
    __syncthreads();
    if (ks == 0 && lane < rows * T) {
      const int rr = lane / T, t = lane % T;
      if (t < a.m) {
        float sum = 0.0f;
#pragma unroll
        for (int k = 0; k < KW; k++) sum += s_part[((rg * 4 + rr) * T + t) * KW + k];
        store_row(a.y + static_cast<size_t>(t) * a.n, row0 + rr, sum, a.mode);
      }
    }
  }
}

template <int BPL, int KW, bool PREQ = false>
hipError_t launch_batch(const Q4BatchArgs &a, hipStream_t st) {
  constexpr int W = 8;
  const int rows_per_wg = 4 * W / KW;
  const unsigned wgs = static_cast<unsigned>((a.n + rows_per_wg - 1) / rows_per_wg);
  hipLaunchKernelGGL((q4_gemv_batch_kernel<4, BPL, KW, W, PREQ>), dim3(wgs), dim3(W * kWave), 0, st, a);
  return hipGetLastError();
}

// ---- batched Q4 GEMV on the matrix cores, 2 <= M <= 64 --------------------
// The same weight stream, with the block dots of 16 weight rows x 16 tokens
// on one v_mfma_i32_16x16x32_i8 per block (K = 32 = one block, so every
// MFMA result is one exact block dot; cf. tdpbssd per K-block,
// crates/llm-cpu/src/amx.rs:329-380) and the reference's per-block fold
// acc = fma(f32(dot), sw * sa, acc) (gemv_q4.rs:930-936) on the 4 results a
// lane holds.  Operands, in the MFMA's register layouts:
//   A (16 rows x 32): lane l = row l%16, elements 8g..8g+7 (g = l/16) = dword
//     g of the block's 16-byte nibble plane, unpacked x16 (the GEMV's unpack);
//   B (32 x 16 tokens): lane l = token l%16, codes 8g..8g+7 of the block --
//     8 bytes of the activation image act_quant_mma writes in this layout;
//   D: lane l = token l%16, rows 4g..4g+3.
// Weights arrive as 16-byte blocks (coalesced 64-byte runs per row) and are
// transposed to dwords through a per-wave LDS tile (row stride padded to
// avoid bank conflicts); no workgroup barrier until the K-slice reduction.
// Workgroup = 4 waves = RG row groups of 16 rows x KW K-slices.
struct Q4MmaArgs {
  const uint8_t *qs;   // nibble plane [n][bpr][16]
  const uint16_t *sc;  // f16 scales [n][bpr]
  const uint8_t *ci;   // activation codes image [mt][2 pq][64][16]
  const float *si;     // activation scales image [mt][pq][16][4]
  float *y;            // [m][n]
  int n, bpr, m, mode, mt, pq;
};

typedef int v4i32 __attribute__((ext_vector_type(4)));

// Registers of one K chunk (CB blocks) of a wave.
template <int TT, int CB>
struct MmaChunk {
  static constexpr int WL = CB / 4;  // 16-byte weight loads per lane
  static constexpr int SL = CB / 4;  // scale loads per lane
  uint4 wv[WL];
  uint16_t sv[SL];
  // One token tile forms the scale products on the matrix core (an f32
  // outer-product MFMA per block quad); two or four do them on the VALU.
  static constexpr bool kOuter = TT == 1;
  uint4 bq[TT][CB / 2];  // B operands of block pairs
  // Activation scales per block quad: of token lane % 16 and block
  // 4 quad + lane / 16 (kOuter), else of token lane % 16 and all 4 blocks.
  std::conditional_t<kOuter, float, float4> sa[TT][CB / 4];
};

// Issue every load of chunk ch: weights (piece p = 64 i + lane is row p / CB,
// block p % CB), weight scales (row lane / 4, blocks SL (lane % 4) + e), then
// each token tile's B operands and scales from the activation image (one
// contiguous 1 KB / 256 B run per instruction).  PART 1 issues only the
// weight loads (all zeros when `valid` is false), PART 2 only the
// activation loads.
template <int TT, int CB, int PART = 0>
__device__ __forceinline__ void mma_load(const Q4MmaArgs &a, __amdgpu_buffer_rsrc_t wr, __amdgpu_buffer_rsrc_t sr,
                                         __amdgpu_buffer_rsrc_t cr, __amdgpu_buffer_rsrc_t ar, int ch,
                                         MmaChunk<TT, CB> &c, bool valid = true) {
  using C = MmaChunk<TT, CB>;
  const int lane = threadIdx.x & 63, lr = lane & 15;
  const int bpr = a.bpr, kb0 = ch * CB, kb_end = valid ? bpr : 0;
  if constexpr (PART != 2) {
#pragma unroll
    for (int i = 0; i < C::WL; i++) {
      const int p = 64 * i + lane, r = p / CB, kb = kb0 + p % CB;
      c.wv[i] = buf_load16<kAuxNT>(wr, kb < kb_end ? static_cast<uint32_t>(r * bpr + kb) * 16u : kOOB);
    }
#pragma unroll
    for (int e = 0; e < C::SL; e++) {
      const int r = lane >> 2, kb = kb0 + C::SL * (lane & 3) + e;
      c.sv[e] = buf_load_u16(sr, kb < kb_end ? static_cast<uint32_t>(r * bpr + kb) * 2u : kOOB);
    }
  }
  if constexpr (PART == 1) return;
#pragma unroll
  for (int tt = 0; tt < TT; tt++) {
    const bool tile = tt < a.mt;
#pragma unroll
    for (int j = 0; j < CB / 2; j++) {
      const int pr = kb0 / 2 + j;  // block pair
      c.bq[tt][j] = buf_load16(cr, tile && pr < 2 * a.pq ? static_cast<uint32_t>((tt * 2 * a.pq + pr) * 64 + lane) * 16u
                                                          : kOOB);
    }
#pragma unroll
    for (int j = 0; j < CB / 4; j++) {
      const int qd = kb0 / 4 + j;  // block quad
      const uint32_t rec = static_cast<uint32_t>((tt * a.pq + qd) * 16 + lr) * 16u;  // token lr's 4 scales
      const bool in = tile && qd < a.pq;
      if constexpr (C::kOuter)
        c.sa[tt][j] = buf_load_f32(ar, in ? rec + 4u * static_cast<uint32_t>(lane >> 4) : kOOB);
      else
        c.sa[tt][j] = buf_load_f4(ar, in ? rec : kOOB);
    }
  }
}

// Transpose the chunk's weights and scales through this wave's LDS tile
// (the same wave writes and reads it: LDS keeps a wave's accesses in order),
// then per block one int8 MFMA and 4 folds per token tile.  The scale
// products sw[row] * sa[token]: with one token tile, one f32 MFMA per block
// quad (v_mfma_f32_16x16x1_4b_f32: block j in elements 4j..4j+3, laid out
// like the block dots -- lane l = token l%16, rows 4(l/16)..+3), which
// replaces 16 VALU multiplies (M=16, K=2048, N=8192: 8.05 -> 7.69 us); with
// two or four token tiles the extra matrix-core passes cost as much as they
// save (measured), so the VALU multiplies stay.  Blocks past the row hold
// zero weights, scales and codes and add exactly 0 (no branches).
template <int TT, int CB>
__device__ __forceinline__ void mma_compute(const MmaChunk<TT, CB> &c, uint32_t *tw, float *tsw,
                                            float (&acc)[TT][4]) {
  using C = MmaChunk<TT, CB>;
  constexpr int RS = CB * 4 + 4;  // row stride in dwords, padded against bank conflicts
  const int lane = threadIdx.x & 63, lr = lane & 15, g = lane >> 4;
#pragma unroll
  for (int i = 0; i < C::WL; i++) {
    const int p = 64 * i + lane;
    *reinterpret_cast<uint4 *>(&tw[(p / CB) * RS + (p % CB) * 4]) = c.wv[i];
  }
#pragma unroll
  for (int e = 0; e < C::SL; e++) tsw[(C::SL * (lane & 3) + e) * 16 + (lane >> 2)] = h2f(c.sv[e]);
  const v4i32 zero = {0, 0, 0, 0};
#pragma unroll
  for (int q = 0; q < CB / 4; q++) {
    long wa[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t dw = tw[lr * RS + (4 * q + j) * 4 + g];
      wa[j] = static_cast<long>(static_cast<uint32_t>(nib_lo16(dw))) |
              (static_cast<long>(static_cast<uint32_t>(nib_hi16(dw))) << 32);
    }
    if constexpr (C::kOuter) {
      const v16f zero16 = {};
      const float swq = tsw[(4 * q + g) * 16 + lr];  // row lr, block 4q + g
      const v16f P = __builtin_amdgcn_mfma_f32_16x16x1f32(swq, c.sa[0][q], zero16, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint4 bp = c.bq[0][2 * q + j / 2];
        const long wb = (j & 1) ? (static_cast<long>(bp.z) | (static_cast<long>(bp.w) << 32))
                                : (static_cast<long>(bp.x) | (static_cast<long>(bp.y) << 32));
        const v4i32 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(wa[j], wb, zero, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 4; v++) acc[0][v] = fmaf(static_cast<float>(d[v]), P[4 * j + v], acc[0][v]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int b = 4 * q + j;
        const float4 sw = *reinterpret_cast<const float4 *>(&tsw[b * 16 + 4 * g]);
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
          const uint4 bp = c.bq[tt][b / 2];
          const long wb = (b & 1) ? (static_cast<long>(bp.z) | (static_cast<long>(bp.w) << 32))
                                  : (static_cast<long>(bp.x) | (static_cast<long>(bp.y) << 32));
          const v4i32 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(wa[j], wb, zero, 0, 0, 0);
          const float4 s4 = c.sa[tt][q];
          const float s = j == 0 ? s4.x : j == 1 ? s4.y : j == 2 ? s4.z : s4.w;
          acc[tt][0] = fmaf(static_cast<float>(d[0]), sw.x * s, acc[tt][0]);
          acc[tt][1] = fmaf(static_cast<float>(d[1]), sw.y * s, acc[tt][1]);
          acc[tt][2] = fmaf(static_cast<float>(d[2]), sw.z * s, acc[tt][2]);
          acc[tt][3] = fmaf(static_cast<float>(d[3]), sw.w * s, acc[tt][3]);
        }
      }
    }
  }
}

// W = RG x KW waves: RG row groups of 16 rows, KW K slices.  The planner
// gives each wave one chunk when the row allows it, so all of a wave's loads
// are in flight at once (the GEMV's single round trip); longer rows loop.
template <int TT, int KW, int CB, int RG, bool PF = false>
__global__ __launch_bounds__(RG * KW * 64) void q4_mma_kernel(Q4MmaArgs a) {
  constexpr int W = RG * KW;
  constexpr int RS = CB * 4 + 4;
  static_assert(CB % 4 == 0 && CB <= 16, "chunk");
  __shared__ __align__(16) uint32_t s_w[W][16 * RS];
  __shared__ __align__(16) float s_sw[W][CB * 16];
  __shared__ float s_part[KW > 1 ? W * TT * 4 * 64 : 1];
  const int bpr = a.bpr;
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int rg = wave / KW, ks = wave % KW;
  const int row0 = (blockIdx.x * RG + rg) * 16;
  const int rows = uniform(max(0, min(16, a.n - row0)));
  const int lr = lane & 15, g = lane >> 4;  // A: row lr; B / D: token lr; K group g
  const int nch = (bpr + CB - 1) / CB;
  const int ch_lo = nch * ks / KW, ch_hi = nch * (ks + 1) / KW;

  const size_t blk0 = static_cast<size_t>(row0) * bpr;
  const auto wr = make_rsrc(a.qs + blk0 * 16, static_cast<uint32_t>(rows * bpr) * 16u);
  const auto sr = make_rsrc(a.sc + blk0, static_cast<uint32_t>(rows * bpr) * 2u);
  const auto cr = make_rsrc(a.ci, static_cast<uint32_t>(a.mt * 2 * a.pq) * 1024u);
  const auto ar = make_rsrc(a.si, static_cast<uint32_t>(a.mt * a.pq) * 256u);

  float acc[TT][4];
#pragma unroll
  for (int tt = 0; tt < TT; tt++)
#pragma unroll
    for (int v = 0; v < 4; v++) acc[tt][v] = 0.0f;

  // PF (one or four token tiles over three or more chunks per wave): the
  // next chunk's weights are requested right after this chunk's activation
  // operands (the fences keep that order, so waiting for the operands leaves
  // them in flight), and their HBM round trip overlaps this chunk's work.
  // Whole calls, interleaved A/B, bit-identical: M=16, K=8192, N=1536 10.7 ->
  // 10.1 us; M=12, K=16384, N=2048 17.5 -> 15.6 us; M=5, K=8192, N=4096 11.6
  // -> 11.0 us; M=64, K=8000, N=8192 36.5 -> 34.3 us; M=64, K=6144, N=4096
  // 18.0 -> 16.7 us.  Over one or two chunks per wave it cost 5-9% (M=16,
  // K=2048, N=8192; M=8, K=4096, N=8192); three token tiles lost 2-4% (M=40
  // and 48 at K=4096-8192), and two lost up to 9% on large grids (M=30,
  // K=8192, N=16384: 88 -> 170 VGPRs), so those load chunk by chunk, in a
  // kernel of their own (sharing one with the PF loop cost the one-chunk
  // launches 4%).
  if constexpr (PF) {
    MmaChunk<TT, CB> c;
    mma_load<TT, CB, 1>(a, wr, sr, cr, ar, ch_lo, c, ch_lo < ch_hi);
    for (int ch = ch_lo; ch < ch_hi; ch++) {
      mma_load<TT, CB, 2>(a, wr, sr, cr, ar, ch, c);
      __builtin_amdgcn_sched_barrier(0);
      MmaChunk<TT, CB> nx;
      mma_load<TT, CB, 1>(a, wr, sr, cr, ar, ch + 1, nx, ch + 1 < ch_hi);
      __builtin_amdgcn_sched_barrier(0);
      mma_compute<TT, CB>(c, s_w[wave], s_sw[wave], acc);
#pragma unroll
      for (int i = 0; i < MmaChunk<TT, CB>::WL; i++) c.wv[i] = nx.wv[i];
#pragma unroll
      for (int e = 0; e < MmaChunk<TT, CB>::SL; e++) c.sv[e] = nx.sv[e];
    }
  } else {
    for (int ch = ch_lo; ch < ch_hi; ch++) {
      MmaChunk<TT, CB> c;
      mma_load<TT, CB>(a, wr, sr, cr, ar, ch, c);
      mma_compute<TT, CB>(c, s_w[wave], s_sw[wave], acc);
    }
  }

  // K slices meet in LDS and are added in slice order; D layout: token
  // tt*16 + lr, rows 4g + v.
  if constexpr (KW > 1) {
#pragma unroll
    for (int tt = 0; tt < TT; tt++)
#pragma unroll
      for (int v = 0; v < 4; v++) s_part[((wave * TT + tt) * 4 + v) * 64 + lane] = acc[tt][v];
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int tt = 0; tt < TT; tt++)
#pragma unroll
      for (int v = 0; v < 4; v++) {
        float sum = 0.0f;
#pragma unroll
        for (int k = 0; k < KW; k++) sum += s_part[(((rg * KW + k) * TT + tt) * 4 + v) * 64 + lane];
        acc[tt][v] = sum;
      }
  }
#pragma unroll
  for (int tt = 0; tt < TT; tt++) {
    const int t = tt * 16 + lr;
    if (t >= a.m) continue;
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int r = 4 * g + v;
      if (r < rows) store_row(a.y + static_cast<size_t>(t) * a.n, row0 + r, acc[tt][v], a.mode);
    }
  }
}

template <int TT, int KW, int CB, int RG>
hipError_t launch_mma(const Q4MmaArgs &a, hipStream_t st) {
  const int rows_per_wg = 16 * RG;
  const unsigned wgs = static_cast<unsigned>((a.n + rows_per_wg - 1) / rows_per_wg);
  if constexpr (TT == 1 || TT == 4) {
    if ((a.bpr + CB - 1) / CB / KW >= 3) {  // every K slice has >= 3 chunks
      hipLaunchKernelGGL((q4_mma_kernel<TT, KW, CB, RG, true>), dim3(wgs), dim3(RG * KW * 64), 0, st, a);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((q4_mma_kernel<TT, KW, CB, RG>), dim3(wgs), dim3(RG * KW * 64), 0, st, a);
  return hipGetLastError();
}

// ---- Q8_0 GEMV (crates/llm-engine/src/weights.rs:194-227) ---------------
struct Q8GemvArgs {
  const int8_t *qs;    // [n][stride][32], natural order
  const uint16_t *sc;  // f16 scales [n][stride]
  const float *x;      // [tokens][xstride], this launch's K range starting at x
  float *y;            // [tokens][n]
  const float *nw;     // NORM: rms_norm weight [k]
  double inv_k;        // NORM: 1 / k in f64 (ops.rs:12)
  float eps;
  int n;
  int bpr;      // blocks of the K range this launch covers
  int stride;   // blocks per row of the matrix
  int kb_off;   // first block of the range
  int xstride;  // floats per token row of x
  int add;      // 0: y = partial; 1: y += partial in f32 (K ranges after the first)
};

// The Q4 GEMV's mapping (one weight row per 16-lane DPP row, W waves =
// W/KW row groups x KW K slices, lane c of a row walks blocks
// slice*16*BPL + c + 16j) with 32-byte int8 blocks: two 128-bit loads and
// one f16 scale per block, 8 v_dot4 against the LDS codes, and q8_apply's
// per-block term (f32(dot) * sw) * sa added to the lane's sum
// (weights.rs:206-212; the blocks are summed in a different order).  x is
// always quantized per block (weights.rs:197); token blockIdx.y.  NORM: each
// token's row is rms_norm'd in the prologue first, as q4_gemv_kernel does (the
// final norm before the output head, crates/llm-engine/src/lfm2.rs:559-567).
// HALF: lane c of a DPP row loads half c & 1 of block (c >> 1) + 8 j (16 B
// each), so a row's 16 lanes read 256 contiguous bytes per instruction; the
// two halves' integer dots meet by one DPP add, and the even lane folds the
// block.  Without it lane c loads both halves of block c + 16 j, and each
// instruction reads every other 16 bytes of 512.  Measured (interleaved A/B):
// the tied head K=1536, N=65536 19.3 -> 17.6 us; K=8192, N=1536 4.88 ->
// 4.31 us; K=4096, N=16384 14.6 -> 13.2 us; but K=N=1536 2.52 -> 2.63 us and
// K=1536, N=2048 2.65 -> 2.76 us, so small matrices keep the whole-block
// lanes.
template <int BPL, int KW, int W, bool NORM = false, bool HALF = false>
__global__ __launch_bounds__(W * kWave) void q8_gemv_kernel(Q8GemvArgs a) {
  constexpr int THREADS = W * kWave;
  constexpr int KB = 16 * BPL * KW;
  constexpr int RG = W / KW;
  constexpr bool PAIRS = KB * 8 >= 2 * THREADS;  // as in q4_gemv_kernel
  constexpr int XP = (KB * 4 + THREADS - 1) / THREADS;
  constexpr int XJ = PAIRS ? 2 * XP : (KB * 8 + THREADS - 1) / THREADS;
  static_assert(W % KW == 0, "slices divide the waves");
  __shared__ __align__(16) int8_t s_qs[KB * 32];
  __shared__ float s_sa[KB];
  __shared__ float s_red[W];
  __shared__ double s_ss[NORM ? W : 1];
  __shared__ float s_part[KW > 1 ? RG * 4 * KW : 1];
  const int bpr = a.bpr;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = uniform(tid / kWave);
  const int rg = wave / KW, ks = wave % KW;
  const int row0 = (static_cast<int>(blockIdx.x) * RG + rg) * 4;
  const int rows = uniform(max(0, min(4, a.n - row0)));
  const int r = lane >> 4, c = lane & 15;
  const int kb0 = ks * 16 * BPL + c;
  const size_t tok = blockIdx.y;

  // (1) x, then (1b) the x-before-weights barrier for long rows.
  const auto xr = make_rsrc(a.x + tok * static_cast<size_t>(a.xstride), static_cast<uint32_t>(bpr) * 128u);
  const auto nr = make_rsrc(a.nw, NORM ? static_cast<uint32_t>(bpr) * 128u : 0u);
  float4 xv[XJ];
  float4 nv[NORM ? XJ : 1];
  if constexpr (PAIRS) {
#pragma unroll
    for (int j = 0; j < XP; j++) {
      const uint32_t off = static_cast<uint32_t>(tid + j * THREADS) * 32u;
      xv[2 * j] = buf_load_f4(xr, off);
      xv[2 * j + 1] = buf_load_f4(xr, off + 16u);
      if constexpr (NORM) {
        nv[2 * j] = buf_load_f4(nr, off);
        nv[2 * j + 1] = buf_load_f4(nr, off + 16u);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  } else {
#pragma unroll
    for (int j = 0; j < XJ; j++) {
      xv[j] = buf_load_f4(xr, static_cast<uint32_t>(tid + j * THREADS) * 16u);
      if constexpr (NORM) nv[j] = buf_load_f4(nr, static_cast<uint32_t>(tid + j * THREADS) * 16u);
    }
    // No x-before-weights barrier with NORM here: the tied head (K=1536,
    // N=65536, 16-wave workgroups) measured 19.7 -> 20.2 us with one.
  }

  // (2) every weight load of this lane (rows past n fall outside the resource).
  const int stride = a.stride;
  const size_t blk0 = static_cast<size_t>(row0) * stride + a.kb_off;
  const uint32_t span = rows > 0 ? static_cast<uint32_t>((rows - 1) * stride + bpr) : 0u;
  const auto wr = make_rsrc(a.qs + blk0 * 32, span * 32u);
  const auto sr = make_rsrc(a.sc + blk0, span * 2u);
  constexpr int NL = HALF ? 2 * BPL : BPL;  // loads of 16 B per lane (x2 without HALF)
  const int hb = ks * 16 * BPL + (c >> 1), half = c & 1;
  uint4 w0[NL], w1[HALF ? 1 : BPL];
  uint16_t s[NL];
#pragma unroll
  for (int j = 0; j < NL; j++) {
    if constexpr (HALF) {
      const int kb = hb + 8 * j;
      const uint32_t blk = static_cast<uint32_t>(r * stride + kb);
      w0[j] = buf_load16<kAuxNT>(wr, kb < bpr ? blk * 32u + 16u * static_cast<uint32_t>(half) : kOOB);
      s[j] = buf_load_u16(sr, kb < bpr ? blk * 2u : kOOB);
    } else {
      const int kb = kb0 + 16 * j;
      const uint32_t blk = static_cast<uint32_t>(r * stride + kb);
      w0[j] = buf_load16<kAuxNT>(wr, kb < bpr ? blk * 32u : kOOB);
      w1[j] = buf_load16<kAuxNT>(wr, kb < bpr ? blk * 32u + 16u : kOOB);
      s[j] = buf_load_u16(sr, kb < bpr ? blk * 2u : kOOB);
    }
  }

  // (2b) NORM: x = nw * (x * scale).
  if constexpr (NORM) rms_norm_regs<THREADS, XJ>(xv, nv, a.inv_k, a.eps, s_ss);

  // (3) x -> LDS codes (per block).
  if constexpr (PAIRS)
    quantize_pairs_to_lds<THREADS, XP>(xv, bpr, 0, s_qs, s_sa, s_red);
  else
    quantize_regs_to_lds<THREADS, XJ>(xv, bpr, 0, s_qs, s_sa, s_red);

  // (4) dots and terms, branch-free: a block past the row has zero weights
  // and scale and reads block 0's codes, so its term is exactly 0.
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < NL; j++) {
    if constexpr (HALF) {
      const int kb = hb + 8 * j;
      const int kbc = kb < bpr ? kb : 0;
      const v4i ah = reinterpret_cast<const v4i *>(s_qs + kbc * 32)[half];
      int d = 0;
      d = sdot4(static_cast<int>(w0[j].x), ah.x, d);
      d = sdot4(static_cast<int>(w0[j].y), ah.y, d);
      d = sdot4(static_cast<int>(w0[j].z), ah.z, d);
      d = sdot4(static_cast<int>(w0[j].w), ah.w, d);
      d += __builtin_amdgcn_update_dpp(0, d, 0xB1, 0xf, 0xf, false);  // + the other half (lane c ^ 1)
      const float t = (static_cast<float>(d) * h2f(s[j])) * s_sa[kbc];
      acc += half ? 0.0f : t;
    } else {
      const int kb = kb0 + 16 * j;
      const int kbc = kb < bpr ? kb : 0;
      const v4i *ap = reinterpret_cast<const v4i *>(s_qs + kbc * 32);
      const int d = dot_q8_block(w0[j], w1[j], ap[0], ap[1]);
      acc += (static_cast<float>(d) * h2f(s[j])) * s_sa[kbc];
    }
  }
  // (5) 16-lane row sums, slices in order, store.
  acc += dpp<0xB1>(acc);
  acc += dpp<0x4E>(acc);
  acc += dpp<0x141>(acc);
  acc += dpp<0x140>(acc);
  float *y = a.y + tok * static_cast<size_t>(a.n);
  if constexpr (KW == 1) {
    if (c == 0 && r < rows) y[row0 + r] = a.add ? y[row0 + r] + acc : acc;
  } else {
    if (c == 0) s_part[(rg * 4 + r) * KW + ks] = acc;
    __syncthreads();
    if (ks == 0 && lane < rows) {
      float sum = 0.0f;
#pragma unroll
      for (int k = 0; k < KW; k++) sum += s_part[(rg * 4 + lane) * KW + k];
      y[row0 + lane] = a.add ? y[row0 + lane] + sum : sum;
    }
  }
}

}  // namespace

// Q4 GEMV plan: KW K slices of 64 blocks per workgroup cover the row
// (K <= 64*32*16 = 32768), then rows per wave R so the launch has >= ~4096
// waves while every lane keeps its R weight loads in registers.
Q4GemvPlan plan_q4_gemv(size_t n, size_t bpr, int nmat, bool narrow) {
  Q4GemvPlan p{};
  if (bpr <= 64) {  // one slice: 16 lanes x BPL blocks cover the row
    p.KW = 1;
    p.BPL = static_cast<int>(bpr == 0 ? 1 : (bpr + 15) / 16);
  } else {          // 2 blocks per lane, KW slices of 32 blocks (4 per lane for K > 16384)
    p.BPL = bpr > 512 ? 4 : 2;
    p.KW = 4;
    while (p.KW < 16 && static_cast<size_t>(16 * p.BPL * p.KW) < bpr) p.KW <<= 1;
  }
  p.ok = static_cast<size_t>(16 * p.BPL * p.KW) >= bpr;
  // Waves per workgroup: the largest of 16 / 8 / 4 (>= KW) that still gives
  // >= 192 workgroups; every workgroup re-quantizes all of x, so fewer and
  // larger workgroups win as long as most CUs stay busy.
  p.W = 16;
  while (p.W > 4 && p.W > p.KW && n * nmat / static_cast<size_t>(4 * p.W / p.KW) < 192) p.W >>= 1;
  // Long rows: twice the blocks per lane and half the slices (twice the rows
  // per workgroup, half the workgroups re-quantizing x) while >= 512
  // workgroups remain (K=8192: N=16384 19.9 -> 14.9 us, N=4096 6.4 -> 5.5 us;
  // K=4096: N=16384 9.4 -> 8.3 us, N=32768 16.4 -> 14.4 us).
  while (p.W == 16 && p.KW >= 4 && p.BPL < 4 && n * nmat * static_cast<size_t>(p.KW / 2) / 64 >= 512) {
    p.KW /= 2;
    p.BPL *= 2;
  }
  // One slice, `narrow`: 8 rather than 16 waves once 8 gives two or more
  // workgroups per CU (measured against 16: the Q4 N=65536 head 10.9 ->
  // 10.4 us, the gate/up pair 4.58 -> 4.41 us; the Q8_0 head 19.2 -> 19.8 us,
  // so it keeps 16).
  if (narrow && p.W == 16 && p.KW == 1 && n * nmat / 32 >= 512) p.W = 8;
  // Without `narrow` (Q8_0 rows), short rows that leave < 192 workgroups even
  // at 4 waves take two K slices (K=N=1536: 96 -> 192 workgroups, 3.43 ->
  // 2.46 us; Q4 rows of the same shape measured no change).
  if (!narrow && p.KW == 1 && p.W == 4 && bpr > 16 && n * nmat / 16 < 192) {
    p.KW = 2;
    p.BPL = static_cast<int>((bpr + 31) / 32);
  }
  const int rows_per_wg = 4 * p.W / p.KW;
  p.wgs_per_mat = static_cast<int>((n + rows_per_wg - 1) / rows_per_wg);
  return p;
}

bool mma_shape_compiled(int tt, int kw, int cb, int rg) {
#define LGH_HAS(T_, K_, C_, R_) \
  if (tt == T_ && kw == K_ && cb == C_ && rg == R_) return true;
  LGH_MMA_SHAPES(LGH_HAS)
#undef LGH_HAS
  return false;
}

bool gemv_shape_compiled(int bpl, int kw, int w) {
#define LGH_HAS(BB, KK, WW) \
  if (bpl == BB && kw == KK && w == WW) return true;
  LGH_GEMV_SHAPES(LGH_HAS)
#undef LGH_HAS
  return false;
}

// plan_q4_gemv() over every row length it accepts (1..1024 blocks), 1..3
// matrices, both `narrow` values, and total row counts on both sides of every
// threshold the planner compares against (N = n * nmat against 192 * D for
// D = 4W/KW, 3072, 4096, 8192, 16384, 32768) plus powers of two: the number
// of plans whose shape has no compiled kernel.
int gemv_plans_uncovered() {
  static const long kBreaks[] = {192, 384, 768, 1536, 3072, 6144, 12288, 4096, 8192, 16384, 32768, 65536};
  int missing = 0;
  for (int narrow = 0; narrow < 2; narrow++)
    for (int nmat = 1; nmat <= 3; nmat++)
      for (size_t bpr = 1; bpr <= 1024; bpr++) {
        auto check = [&](long n) {
          if (n < 1) return;
          const Q4GemvPlan p = plan_q4_gemv(static_cast<size_t>(n), bpr, nmat, narrow != 0);
          if (p.ok && !gemv_shape_compiled(p.BPL, p.KW, p.W)) missing++;
        };
        for (long b : kBreaks)
          for (long d = -2; d <= 2; d++) check((b + nmat - 1) / nmat + d);
        for (long n = 1; n <= (1L << 20); n *= 2) {
          check(n);
          check(3 * n);
        }
      }
  // The ragged MMA planner: every token count it takes, row lengths 1..1024
  // blocks, row counts on both sides of its 8192-row and 16384-row tests.
  for (int any = 0; any < 2; any++)
    for (size_t m = 1; m <= 65; m++)
      for (size_t bpr = 1; bpr <= 1024; bpr++)
        for (size_t n : {size_t{1}, size_t{16}, size_t{8191}, size_t{8192}, size_t{8193}, size_t{16383},
                         size_t{16384}, size_t{16385}, size_t{1} << 20}) {
          const Q4MmaPlan p = plan_q4_mma(n, m, bpr, any != 0);
          if (p.ok && !mma_shape_compiled(p.TT, p.KW, p.CB, p.RG)) missing++;
        }
  return missing;
}

// Quantize x once (act_quant_kernel) and run the codes GEMV instead when
// the workgroups would re-quantize more than ~12M elements of x between them
// (K=16384, N=8192: 19.5 -> 15.9 us; K=8192, N=16384 is even at 8.4M; a 4M
// threshold was slower at K=4096, N=16384 (9.4 -> 10.7 us) and K=8192,
// N=4096 (5.6 -> 7.5 us): the extra launch costs more).
bool q4_gemv_quantize_once(size_t n, size_t bpr, int nmat) {
  const Q4GemvPlan p = plan_q4_gemv(n, bpr, nmat);
  return p.ok && static_cast<size_t>(p.wgs_per_mat) * nmat * bpr * 32 >= (size_t{12} << 20);
}

hipError_t launch_q4_gemv(const lgh_q4 *w0, float *y0, const lgh_q4 *w1, float *y1, const float *x, int mode,
                          int per_row, hipStream_t st) {
  return launch_q4_gemv_any(w0, y0, w1, y1, x, nullptr, nullptr, mode, per_row, st);
}

hipError_t launch_q4_gemv_codes(const lgh_q4 *w, const int8_t *codes, const float *scales, float *y, int mode,
                                hipStream_t st) {
  return launch_q4_gemv_any(w, y, nullptr, nullptr, nullptr, codes, scales, mode, 0, st);
}

hipError_t launch_q4_gemv_any(const lgh_q4 *w0, float *y0, const lgh_q4 *w1, float *y1, const float *x,
                              const int8_t *codes, const float *scales, int mode, int per_row, hipStream_t st) {
  const lgh_q4 *w[2] = {w0, w1};
  float *y[2] = {y0, y1};
  return launch_q4_gemv_multi(w, y, w1 ? 2 : 1, x, codes, scales, nullptr, 0.0f, mode, per_row, st);
}

size_t gemv_multi_rows(const lgh_q4 *const *w, int nmat) {
  size_t rows = 0;
  for (int j = 0; j < nmat; j++) rows += w[j]->n;
  return rows;
}

hipError_t launch_q4_gemv_multi(const lgh_q4 *const *w, float *const *y, int nmat, const float *x,
                                const int8_t *codes, const float *scales, const float *norm_w, float eps, int mode,
                                int per_row, hipStream_t st) {
  if (nmat < 1 || nmat > 3) return hipErrorInvalidValue;
  const size_t bpr = w[0]->bpr;
  const size_t rows = gemv_multi_rows(w, nmat);
  if (rows == 0) return hipSuccess;
  // The plan depends on the total row count only, as for the pair.
  const Q4GemvPlan p = plan_q4_gemv(rows, bpr, 1);
  if (!p.ok) return hipErrorInvalidValue;  // K > 16384 * 2: the API uses the GEMM
  const bool preq = codes != nullptr, norm = norm_w != nullptr;
  if ((preq && norm) || (norm && p.KW != 1)) return hipErrorInvalidValue;  // the API routes these elsewhere
  const int rows_per_wg = 4 * p.W / p.KW;
  int wgs[3] = {0, 0, 0};
  Q4GemvArgs a{};
  const uint8_t **qsp[3] = {&a.qs0, &a.qs1, &a.qs2};
  const uint16_t **scp[3] = {&a.sc0, &a.sc1, &a.sc2};
  float **yp[3] = {&a.y0, &a.y1, &a.y2};
  int *np[3] = {&a.n0, &a.n1, &a.n2};
  for (int j = 0; j < nmat; j++) {
    *qsp[j] = w[j]->qs;
    *scp[j] = w[j]->sc;
    *yp[j] = y[j];
    *np[j] = static_cast<int>(w[j]->n);
    wgs[j] = static_cast<int>((w[j]->n + rows_per_wg - 1) / rows_per_wg);
  }
  a.x = x;
  a.aq = codes;
  a.as = scales;
  a.nw = norm_w;
  a.inv_k = 1.0 / static_cast<double>(bpr * 32);
  a.eps = eps;
  a.bpr = static_cast<int>(bpr);
  a.wgs0 = wgs[0];
  a.wgs1 = wgs[1];
  a.mode = mode;
  a.per_row = per_row;
  const int total = wgs[0] + wgs[1] + wgs[2];
  if (total == 0) return hipSuccess;
#define LGH_G16(BB, KK, WW) \
  if (p.BPL == BB && p.KW == KK && p.W == WW) return dispatch_q4<BB, KK, WW>(a, total, preq, norm, st);
  LGH_GEMV_SHAPES(LGH_G16)
#undef LGH_G16
  return hipErrorInvalidValue;
}

// m <= 4 tokens in T = 4 slots; K: one slice of BPL <= 4 blocks per lane up
// to 64 blocks, then 2 or 4 slices of 64 (the prologue quantizes 4 rows of
// up to 8192 elements).  Other shapes run the matrix-core batch kernel.
Q4BatchPlan plan_q4_batch(size_t m, size_t bpr) {
  Q4BatchPlan p{};
  if (m < 2 || m > 4 || bpr == 0) return p;
  if (bpr <= 64) {
    p.KW = 1;
    p.BPL = static_cast<int>((bpr + 15) / 16);
  } else if (bpr <= 256) {
    p.KW = bpr <= 128 ? 2 : 4;
    p.BPL = 4;
  } else {
    return p;
  }
  p.ok = true;
  return p;
}

// Rows of more than 64 blocks (two or four K slices per row group) are
// quantized once by act_quant_kernel: inside the kernel every workgroup would
// quantize all m rows, m * k elements (256 workgroups at K=8192, N=2048).
// Measured, whole call: K=8192, N=2048, M=2 / 4 9.47 / 10.05 -> 7.35 /
// 7.42 us; K=4096, N=8192 9.41 / 10.19 -> 8.70 / 8.98 us; K=3072, N=8192
// 8.25 / 8.90 -> 8.04 / 8.37 us.
bool q4_batch_quantize_once(size_t bpr) { return bpr > 64; }

hipError_t launch_q4_gemv_batch(const lgh_q4 *w, const float *x, const int8_t *codes, const float *scales, float *y,
                                size_t m, int mode, int per_row, hipStream_t st) {
  const Q4BatchPlan p = plan_q4_batch(m, w->bpr);
  if (!p.ok) return hipErrorInvalidValue;
  if (w->n == 0) return hipSuccess;
  Q4BatchArgs a{w->qs,  w->sc, x, codes, scales, y, static_cast<int>(w->n), static_cast<int>(w->bpr),
                static_cast<int>(m), mode, per_row};
  if (codes) {
    if (p.KW == 1) return hipErrorInvalidValue;
    return p.KW == 2 ? launch_batch<4, 2, true>(a, st) : launch_batch<4, 4, true>(a, st);
  }
  if (p.KW == 1) {
    switch (p.BPL) {
      case 1: return launch_batch<1, 1>(a, st);
      case 2: return launch_batch<2, 1>(a, st);
      case 3: return launch_batch<3, 1>(a, st);
      default: return launch_batch<4, 1>(a, st);
    }
  }
  return p.KW == 2 ? launch_batch<4, 2>(a, st) : launch_batch<4, 4>(a, st);
}

// Token tiles TT = ceil(m / 16) (<= 4); 8-block chunks; KW (a power of
// two <= 8) K slices per 16 rows: one chunk per wave for one or two token
// tiles, two for three or four (measured at N=8192, K=2048: more, smaller waves are
// faster while a chunk's registers stay small, then occupancy wins); RG row
// groups make the workgroup at least 4 waves.
Q4MmaPlan plan_q4_mma(size_t n, size_t m, size_t bpr, bool any_shape) {
  Q4MmaPlan p{};
  if (m < (any_shape ? 1u : 2u) || m > 64 || bpr == 0 || n == 0) return p;
  // Four token tiles over long rows: the fp6 GEMM is faster (M=64, whole
  // call: K=8192, N=1536 / 2048 / 8192 20.4 / 20.7 / 36.6 -> 18.5 / 19.3 /
  // 29.8 us; K=4096, N=16384 39.1 -> 30.9 us), but not where its grid is
  // small (K=4096, N=4096: 13.7 us here, 18.0 us on the GEMM).
  if (!any_shape && m > 48 && (bpr >= 256 || (bpr >= 128 && n >= 16384))) return p;
  p.TT = static_cast<int>((m + 15) / 16);
  p.CB = 8;
  // Three token tiles over rows of >= 48 blocks and up to 8192 rows: 4-block
  // chunks over 8 K slices (two chunks per wave, 127 VGPRs: the 4 waves per
  // SIMD of up to 512 workgroups are resident at once) instead of 8-block
  // chunks over 4.  M=40 / 48, whole call: K=1536, N=1536 / 2048 9.1 -> 7.8 /
  // 8.0 us; K=2048, N=8192 11.9 -> 11.7 / 11.6 us; K=4096, N=4096 12.2 ->
  // 11.4 us; K=8192, N=1536 17.3 -> 16.1 us.  At N=16384 (two rounds of
  // waves) it was slower: 17.9 -> 19.0 us.
  if (p.TT == 3 && bpr >= 48 && n <= 8192) p.CB = 4;
  const size_t nch = (bpr + p.CB - 1) / p.CB;
  const size_t per_wave = p.TT >= 3 ? 2 : 1;
  p.KW = 1;
  while (p.KW < 8 && static_cast<size_t>(p.KW) * per_wave < nch) p.KW *= 2;
  p.RG = p.KW >= 4 ? 1 : 4 / p.KW;
  p.ok = true;
  return p;
}

hipError_t launch_q4_gemv_mma(const lgh_q4 *w, const uint8_t *codes, const float *scales, float *y, size_t m,
                              int mode, hipStream_t st, bool any_shape) {
  const Q4MmaPlan p = plan_q4_mma(w->n, m, w->bpr, any_shape);
  if (!p.ok) return hipErrorInvalidValue;
  Q4MmaArgs a{w->qs, w->sc, codes, scales, y, static_cast<int>(w->n), static_cast<int>(w->bpr), static_cast<int>(m),
              mode, static_cast<int>((m + 15) / 16), static_cast<int>((w->bpr + 3) / 4)};
#define LGH_M(TT_, KW_, CB_, RG_) \
  if (p.TT == TT_ && p.KW == KW_ && p.CB == CB_ && p.RG == RG_) return launch_mma<TT_, KW_, CB_, RG_>(a, st);
  LGH_MMA_SHAPES(LGH_M)
#undef LGH_M
  return hipErrorInvalidValue;
}

hipError_t launch_q8_range(const lgh_q8 *w, const float *x, float *y, size_t tokens, const float *norm_w, float eps,
                           size_t b0, size_t nb, bool add, hipStream_t st);

// The Q8_0 GEMV takes the Q4 GEMV's plan (same row mapping).  Rows longer than
// one launch covers (K > 32768) run as consecutive K ranges of <= 32768,
// each adding its partial sums onto y in f32, and tokens beyond the grid's
// 65535 run as further launches.  The norm prologue needs whole rows: norm_w
// is only accepted with K <= 32768 (the API norms longer rows first).
hipError_t launch_q8_gemv(const lgh_q8 *w, const float *x, float *y, size_t tokens, const float *norm_w, float eps,
                          hipStream_t st) {
  if (w->n == 0 || tokens == 0) return hipSuccess;
  constexpr size_t kMaxBpr = kQ8GemvMaxK / 32, kMaxTok = 65535;
  if (norm_w && w->bpr > kMaxBpr) return hipErrorInvalidValue;  // the API norms first
  for (size_t t0 = 0; t0 < tokens; t0 += kMaxTok) {
    const size_t nt = std::min(kMaxTok, tokens - t0);
    for (size_t b0 = 0; b0 < w->bpr; b0 += kMaxBpr) {
      const size_t nb = std::min(kMaxBpr, w->bpr - b0);
      hipError_t e = launch_q8_range(w, x + t0 * w->k + b0 * 32, y + t0 * w->n, nt, norm_w, eps, b0, nb,
                                     b0 > 0, st);
      if (e != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

// One launch of the Q8_0 GEMV over blocks [b0, b0 + nb) of every row.
hipError_t launch_q8_range(const lgh_q8 *w, const float *x, float *y, size_t tokens, const float *norm_w, float eps,
                           size_t b0, size_t nb, bool add, hipStream_t st) {
  // Matrices of >= 2^17 blocks load contiguous half blocks (HALF); with the
  // norm prologue they also take the 8-wave plan (`narrow`): every workgroup
  // norms and quantizes x before its first dot, and with 16-wave workgroups
  // the tied head runs 4 rounds of them, one at a time per CU (norm + head
  // 20.7 -> 17.6 us; the head alone keeps 16 waves: 17.6 against 18.0 us).
  const bool half = w->n * nb >= (size_t{1} << 17);
  const bool norm = norm_w != nullptr;
  const Q4GemvPlan p = plan_q4_gemv(w->n, nb, 1, norm && half);
  if (!p.ok || tokens > 65535) return hipErrorInvalidValue;
  Q8GemvArgs a{w->qs, w->sc, x, y, norm_w, 1.0 / static_cast<double>(w->k), eps, static_cast<int>(w->n),
               static_cast<int>(nb), static_cast<int>(w->bpr), static_cast<int>(b0), static_cast<int>(w->k),
               add ? 1 : 0};
  const dim3 grid(static_cast<unsigned>(p.wgs_per_mat), static_cast<unsigned>(tokens));
#define LGH_Q8(BB, KK, WW)                                                                            \
  if (p.BPL == BB && p.KW == KK && p.W == WW) {                                                       \
    const dim3 blk(WW * kWave);                                                                       \
    if (norm && half)                                                                                 \
      hipLaunchKernelGGL((q8_gemv_kernel<BB, KK, WW, true, true>), grid, blk, 0, st, a);              \
    else if (norm)                                                                                    \
      hipLaunchKernelGGL((q8_gemv_kernel<BB, KK, WW, true, false>), grid, blk, 0, st, a);             \
    else if (half)                                                                                    \
      hipLaunchKernelGGL((q8_gemv_kernel<BB, KK, WW, false, true>), grid, blk, 0, st, a);             \
    else                                                                                              \
      hipLaunchKernelGGL((q8_gemv_kernel<BB, KK, WW, false, false>), grid, blk, 0, st, a);            \
    return hipGetLastError();                                                                         \
  }
  LGH_GEMV_SHAPES(LGH_Q8)
#undef LGH_Q8
  return hipErrorInvalidValue;
}

}  // namespace lgh
