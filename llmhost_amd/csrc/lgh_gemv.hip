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
#include "lgh_device.h"
#include "lgh_internal.h"

namespace lgh {

namespace {

constexpr int kThreads = 256;  // Q8_0 GEMV workgroup
constexpr int kWaves = kThreads / kWave;

struct Q4GemvArgs {
  const uint8_t *qs0;
  const uint16_t *sc0;
  float *y0;
  const uint8_t *qs1;
  const uint16_t *sc1;
  float *y1;
  const float *x;
  int n;
  int bpr;
  int wgs0;  // workgroups covering matrix 0; the rest cover matrix 1
  int mode;
  int per_row;
};

// Quantize the float4s held in registers (thread t holds x4[t + THREADS j])
// into LDS: s_qs (natural order) and s_sa, for blocks [0, nblk).  All
// threads must call it; it ends with a barrier.
template <int THREADS, int XJ>
__device__ __forceinline__ void quant_regs(const float4 (&xv)[XJ], int nblk, bool per_row, float row_scale,
                                           int8_t *s_qs, float *s_sa) {
  const int tid = threadIdx.x;
  const int g = tid & 7;
#pragma unroll
  for (int j = 0; j < XJ; j++) {
    const int b = (tid >> 3) + j * (THREADS / 8);
    if (b < nblk) {  // uniform across each 8-lane group
      float scale;
      int sum;
      const int q = act_quant_group8(xv[j], per_row, row_scale, scale, sum);
      reinterpret_cast<int *>(s_qs)[b * 8 + g] = q;
      if (g == 0) s_sa[b] = scale;
    }
  }
  __syncthreads();
}

// Row amax / 127 over the register-resident x (PerRow), or 0.
template <int THREADS, int XJ>
__device__ __forceinline__ float row_scale_of(const float4 (&xv)[XJ], int per_row, float *s_red) {
  if (!per_row) return 0.0f;
  float m = 0.0f;
#pragma unroll
  for (int j = 0; j < XJ; j++)
    m = fmaxf(m, fmaxf(fmaxf(fabsf(xv[j].x), fabsf(xv[j].y)), fmaxf(fabsf(xv[j].z), fabsf(xv[j].w))));
  m = wave_max(m);
  if ((threadIdx.x & (kWave - 1)) == 0) s_red[threadIdx.x / kWave] = m;
  __syncthreads();
  m = 0.0f;
  for (int w = 0; w < THREADS / kWave; w++) m = fmaxf(m, s_red[w]);
  return div127_rn(m);
}

template <int THREADS, int XJ>
__device__ __forceinline__ void quantize_regs_to_lds(const float4 (&xv)[XJ], int bpr, int per_row, int8_t *s_qs,
                                                     float *s_sa, float *s_red) {
  const float rs = row_scale_of<THREADS, XJ>(xv, per_row, s_red);
  quant_regs<THREADS, XJ>(xv, bpr, per_row != 0, rs, s_qs, s_sa);
}

__device__ __forceinline__ void store_row(float *y, int row, float acc16, int mode) {
  const float v = acc16 * 0.0625f;  // exact: undo the x16 of the nibble unpack
  if (mode == LGH_ADD_F64)
    y[row] = static_cast<float>(static_cast<double>(y[row]) + static_cast<double>(v));
  else
    y[row] = v;
}

// BPL blocks per lane and row, KW K slices, W waves; 4*(W/KW) rows per workgroup.
template <int BPL, int KW, int W>
__global__ __launch_bounds__(W * kWave) void q4_gemv_kernel(Q4GemvArgs a) {
  constexpr int THREADS = W * kWave;
  constexpr int KB = 16 * BPL * KW;  // blocks covered by the workgroup (>= bpr)
  constexpr int RG = W / KW;
  constexpr int XJ = (KB * 8 + THREADS - 1) / THREADS;
  static_assert(W % KW == 0, "slices divide the waves");
  __shared__ __align__(16) int8_t s_qs[KB * 32];
  __shared__ float s_sa[KB];
  __shared__ float s_red[W];
  __shared__ float s_part[KW > 1 ? RG * 4 * KW : 1];
  const int bpr = a.bpr;
  int wg = blockIdx.x;
  const uint8_t *qs = a.qs0;
  const uint16_t *sc = a.sc0;
  float *y = a.y0;
  if (wg >= a.wgs0) {
    wg -= a.wgs0;
    qs = a.qs1;
    sc = a.sc1;
    y = a.y1;
  }
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = uniform(tid / kWave);
  const int rg = wave / KW, ks = wave % KW;
  const int row0 = (wg * RG + rg) * 4;  // first row of this wave
  const int rows = uniform(max(0, min(4, a.n - row0)));
  const int r = lane >> 4, c = lane & 15;
  const int kb0 = ks * 16 * BPL + c;

  // (1) x: bpr*8 float4s, XJ per thread.
  const auto xr = make_rsrc(a.x, static_cast<uint32_t>(bpr) * 128u);
  float4 xv[XJ];
#pragma unroll
  for (int j = 0; j < XJ; j++) xv[j] = buf_load_f4(xr, static_cast<uint32_t>(tid + j * THREADS) * 16u);

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

  // (3) x -> LDS codes.
  quantize_regs_to_lds<THREADS, XJ>(xv, bpr, a.per_row, s_qs, s_sa, s_red);

  // (4) dots + fold.
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < BPL; j++) {
    const int kb = kb0 + 16 * j;
    if (kb < bpr) {
      const v4i *ap = reinterpret_cast<const v4i *>(s_qs + kb * 32);
      const int d = dot_q4_block16(w[j], ap[0], ap[1]);
      acc = fmaf(static_cast<float>(d), h2f(s[j]) * s_sa[kb], acc);
    }
  }
  // (5) 16-lane row sums (every lane of a DPP row ends with its row's sum).
  acc += dpp<0xB1>(acc);   // quad_perm [1,0,3,2]
  acc += dpp<0x4E>(acc);   // quad_perm [2,3,0,1]
  acc += dpp<0x141>(acc);  // row_half_mirror
  acc += dpp<0x140>(acc);  // row_mirror
  if constexpr (KW == 1) {
    if (c == 0 && r < rows) store_row(y, row0 + r, acc, a.mode);
  } else {
    if (c == 0) s_part[(rg * 4 + r) * KW + ks] = acc;
    __syncthreads();
    if (ks == 0 && lane < rows) {
      float sum = 0.0f;
#pragma unroll
      for (int k = 0; k < KW; k++) sum += s_part[(rg * 4 + lane) * KW + k];
      store_row(y, row0 + lane, sum, a.mode);
    }
  }
}

template <int BPL, int KW, int W>
hipError_t launch_gemv16(const Q4GemvArgs &a, int total_wgs, hipStream_t st) {
  hipLaunchKernelGGL((q4_gemv_kernel<BPL, KW, W>), dim3(total_wgs), dim3(W * kWave), 0, st, a);
  return hipGetLastError();
}

// ---- batched Q4 GEMV, 2 <= M <= 16 ----------------------------------------
// Small ragged batches (crates/llm-cpu/src/gemv_q4.rs:686-722 with m <= 16)
// are weight-stream bound like the GEMV, so they read the 18-byte nibble
// blocks once and dot each against T token code rows held in LDS: per block
// one nibble unpack, then 8 v_dot4_i32_i8 and one fold per token.  Same row
// mapping, slices and DPP row sums as q4_gemv_kernel.  The codes come either
// from quantizing x[T][k] in the prologue (QUANT, small T * k) or, already
// quantized by act_quant_kernel, from int8 qs[m][k] + f32 scales[m][bpr].
struct Q4BatchArgs {
  const uint8_t *qs;
  const uint16_t *sc;
  const float *x;      // QUANT: f32 [m][k]
  const int8_t *aq;    // !QUANT: int8 [m][k]
  const float *as;     // !QUANT: f32 [m][bpr]
  float *y;            // [m][n]
  int n, bpr, m, mode, per_row;
};

template <int T, int BPL, int KW, int W, bool QUANT>
__global__ __launch_bounds__(W * kWave) void q4_gemv_batch_kernel(Q4BatchArgs a) {
  constexpr int THREADS = W * kWave;
  constexpr int KB = 16 * BPL * KW;
  constexpr int RG = W / KW;
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

  // (1) activations: x rows (QUANT) or codes + scales; tokens >= m read as 0.
  constexpr int XJ = QUANT ? (KB * 8 + THREADS - 1) / THREADS : 1;
  float4 xv[T][XJ];
  if constexpr (QUANT) {
#pragma unroll
    for (int t = 0; t < T; t++) {
      const auto xr = make_rsrc(a.x + static_cast<size_t>(t) * bpr * 32, t < a.m ? static_cast<uint32_t>(bpr) * 128u : 0u);
#pragma unroll
      for (int j = 0; j < XJ; j++) xv[t][j] = buf_load_f4(xr, static_cast<uint32_t>(tid + j * THREADS) * 16u);
    }
  } else {
    const auto qr = make_rsrc(a.aq, static_cast<uint32_t>(a.m * bpr) * 32u);
    const auto sr = make_rsrc(a.as, static_cast<uint32_t>(a.m * bpr) * 4u);
    for (int i = tid; i < T * bpr * 2; i += THREADS) {  // 16-byte chunks of [T][bpr][32]
      const int t = i / (bpr * 2), rem = i % (bpr * 2);
      const uint4 v = buf_load16(qr, t < a.m ? static_cast<uint32_t>((t * bpr) * 32 + rem * 16) : kOOB);
      *reinterpret_cast<uint4 *>(&s_qs[t][rem * 16]) = v;
    }
    for (int i = tid; i < T * bpr; i += THREADS) {
      const int t = i / bpr, b = i % bpr;
      s_sa[t][b] = buf_load_f32(sr, t < a.m ? static_cast<uint32_t>(t * bpr + b) * 4u : kOOB);
    }
  }

  // (2) every weight load of this lane.
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

  // (3) codes into LDS (QUANT), one barrier.
  if constexpr (QUANT) {
#pragma unroll
    for (int t = 0; t < T; t++) {
      const float rs = row_scale_of<THREADS, XJ>(xv[t], a.per_row, s_red);
      quant_regs<THREADS, XJ>(xv[t], bpr, a.per_row != 0, rs, s_qs[t], s_sa[t]);
    }
  } else {
    __syncthreads();
  }

  // (4) per block: one unpack, then T dots and folds.
  float acc[T];
#pragma unroll
  for (int t = 0; t < T; t++) acc[t] = 0.0f;
#pragma unroll
  for (int j = 0; j < BPL; j++) {
    const int kb = kb0 + 16 * j;
    if (kb < bpr) {
      const int u[8] = {nib_lo16(w[j].x), nib_hi16(w[j].x), nib_lo16(w[j].y), nib_hi16(w[j].y),
                        nib_lo16(w[j].z), nib_hi16(w[j].z), nib_lo16(w[j].w), nib_hi16(w[j].w)};
      const float sw = h2f(s[j]);
#pragma unroll
      for (int t = 0; t < T; t++) {
        const v4i *ap = reinterpret_cast<const v4i *>(&s_qs[t][kb * 32]);
        const v4i a0 = ap[0], a1 = ap[1];
        int d = sdot4(u[0], a0.x, 0);
        d = sdot4(u[1], a0.y, d);
        d = sdot4(u[2], a0.z, d);
        d = sdot4(u[3], a0.w, d);
        d = sdot4(u[4], a1.x, d);
        d = sdot4(u[5], a1.y, d);
        d = sdot4(u[6], a1.z, d);
        d = sdot4(u[7], a1.w, d);
        acc[t] = fmaf(static_cast<float>(d), sw * s_sa[t][kb], acc[t]);
      }
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

template <int T, int BPL, int KW, bool QUANT>
hipError_t launch_batch(const Q4BatchArgs &a, hipStream_t st) {
  constexpr int W = 8;
  const int rows_per_wg = 4 * W / KW;
  const unsigned wgs = static_cast<unsigned>((a.n + rows_per_wg - 1) / rows_per_wg);
  hipLaunchKernelGGL((q4_gemv_batch_kernel<T, BPL, KW, W, QUANT>), dim3(wgs), dim3(W * kWave), 0, st, a);
  return hipGetLastError();
}

// ---- Q8_0 GEMV (crates/llm-engine/src/weights.rs:194-227) ---------------
struct Q8GemvArgs {
  const int8_t *qs;
  const uint16_t *sc;
  const float *x;
  float *y;
  int n;
  int bpr;
  int k;
};

// Same structure as the Q4 kernel: 2 x 128-bit loads per Q8_0 block, natural
// order int8 weights, always per-block activation quant (weights.rs:197).
template <int R, int S>
__global__ __launch_bounds__(kThreads) void q8_gemv_kernel(Q8GemvArgs a) {
  extern __shared__ __align__(16) char smem[];
  const int bpr = a.bpr;
  int8_t *s_qs = reinterpret_cast<int8_t *>(smem);
  float *s_sa = reinterpret_cast<float *>(smem + bpr * 32);
  float *s_red = s_sa + bpr;
  const int tok = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int row0 = (static_cast<int>(blockIdx.x) * kWaves + uniform(tid / kWave)) * R;
  const int rows = uniform(max(0, min(R, a.n - row0)));

  constexpr int XJ = 2 * S;
  const auto xr = make_rsrc(a.x + static_cast<size_t>(tok) * a.k, static_cast<uint32_t>(bpr) * 128u);
  float4 xv[XJ];
#pragma unroll
  for (int j = 0; j < XJ; j++) xv[j] = buf_load_f4(xr, static_cast<uint32_t>(tid + j * kThreads) * 16u);

  const size_t blk0 = static_cast<size_t>(row0) * bpr;
  const auto wr = make_rsrc(a.qs + blk0 * 32, static_cast<uint32_t>(rows * bpr) * 32u);
  const auto sr = make_rsrc(a.sc + blk0, static_cast<uint32_t>(rows * bpr) * 2u);
  uint4 w0[S][R], w1[S][R];
  uint16_t s[S][R];
#pragma unroll
  for (int st = 0; st < S; st++) {
    const int kb = st * kWave + lane;
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t blk = static_cast<uint32_t>(r * bpr + kb);
      w0[st][r] = buf_load16<kAuxNT>(wr, kb < bpr ? blk * 32u : kOOB);
      w1[st][r] = buf_load16<kAuxNT>(wr, kb < bpr ? blk * 32u + 16u : kOOB);
      s[st][r] = buf_load_u16(sr, kb < bpr ? blk * 2u : kOOB);
    }
  }
  quantize_regs_to_lds<kThreads, XJ>(xv, bpr, 0, s_qs, s_sa, s_red);

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) acc[r] = 0.0f;
#pragma unroll
  for (int st = 0; st < S; st++) {
    const int kb = st * kWave + lane;
    if (kb < bpr) {
      const v4i *ap = reinterpret_cast<const v4i *>(s_qs + kb * 32);
      const v4i a0 = ap[0], a1 = ap[1];
      const float sa = s_sa[kb];
#pragma unroll
      for (int r = 0; r < R; r++)
        acc[r] = fmaf(static_cast<float>(dot_q8_block(w0[st][r], w1[st][r], a0, a1)), h2f(s[st][r]) * sa, acc[r]);
    }
  }
  float *y = a.y + static_cast<size_t>(tok) * a.n;
#pragma unroll
  for (int r = 0; r < R; r++) {
    const float t = wave_sum_dpp(acc[r]);
    if (lane == 0 && r < rows) y[row0 + r] = t;
  }
}

}  // namespace

// Q4 GEMV plan: KW K slices of 64 blocks per workgroup cover the row
// (K <= 64*32*16 = 32768), then rows per wave R so the launch has >= ~4096
// waves while every lane keeps its R weight loads in registers.
Q4GemvPlan plan_q4_gemv(size_t n, size_t bpr, int nmat) {
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
  const int rows_per_wg = 4 * p.W / p.KW;
  p.wgs_per_mat = static_cast<int>((n + rows_per_wg - 1) / rows_per_wg);
  return p;
}

hipError_t launch_q4_gemv(const lgh_q4 *w0, float *y0, const lgh_q4 *w1, float *y1, const float *x, int mode,
                          int per_row, hipStream_t st) {
  if (w0->n == 0) return hipSuccess;
  const int nmat = w1 ? 2 : 1;
  const Q4GemvPlan p = plan_q4_gemv(w0->n, w0->bpr, nmat);
  if (!p.ok) return hipErrorInvalidValue;  // K > 16384 * 2: the API uses the GEMM
  Q4GemvArgs a{};
  a.qs0 = w0->qs;
  a.sc0 = w0->sc;
  a.y0 = y0;
  a.qs1 = w1 ? w1->qs : nullptr;
  a.sc1 = w1 ? w1->sc : nullptr;
  a.y1 = y1;
  a.x = x;
  a.n = static_cast<int>(w0->n);
  a.bpr = static_cast<int>(w0->bpr);
  a.wgs0 = p.wgs_per_mat;
  a.mode = mode;
  a.per_row = per_row;
  const int total = p.wgs_per_mat * nmat;
#define LGH_G16(BB, KK, WW) \
  if (p.BPL == BB && p.KW == KK && p.W == WW) return launch_gemv16<BB, KK, WW>(a, total, st)
  LGH_G16(1, 1, 16);
  LGH_G16(1, 1, 8);
  LGH_G16(1, 1, 4);
  LGH_G16(2, 1, 16);
  LGH_G16(2, 1, 8);
  LGH_G16(2, 1, 4);
  LGH_G16(3, 1, 16);
  LGH_G16(3, 1, 8);
  LGH_G16(3, 1, 4);
  LGH_G16(4, 1, 16);
  LGH_G16(4, 1, 8);
  LGH_G16(4, 1, 4);
  LGH_G16(2, 4, 16);
  LGH_G16(2, 4, 8);
  LGH_G16(2, 4, 4);
  LGH_G16(2, 8, 16);
  LGH_G16(2, 8, 8);
  LGH_G16(2, 16, 16);
  LGH_G16(4, 16, 16);
#undef LGH_G16
  return hipErrorInvalidValue;
}

Q4BatchPlan plan_q4_batch(size_t m, size_t bpr) {
  Q4BatchPlan p{};
  if (m < 2 || m > 16 || bpr == 0) return p;
  p.T = m <= 4 ? 4 : (m <= 8 ? 8 : 16);
  if (bpr <= 64) {
    p.KW = 1;
    p.BPL = static_cast<int>((bpr + 15) / 16);
  } else if (bpr <= 128) {
    p.KW = 2;
    p.BPL = 4;
  } else if (bpr <= 256) {
    p.KW = 4;
    p.BPL = 4;
  } else {
    return p;
  }
  // LDS holds T rows of codes: T * 16 * BPL * KW blocks <= 1024 (32 KB).
  p.ok = p.T * 16 * p.BPL * p.KW <= 1024;
  p.quant = p.T == 4;
  return p;
}

hipError_t launch_q4_gemv_batch(const lgh_q4 *w, const float *x, const int8_t *aq, const float *as, float *y,
                                size_t m, int mode, int per_row, hipStream_t st) {
  const Q4BatchPlan p = plan_q4_batch(m, w->bpr);
  if (!p.ok) return hipErrorInvalidValue;
  if (w->n == 0) return hipSuccess;
  Q4BatchArgs a{w->qs, w->sc, x, aq, as, y, static_cast<int>(w->n), static_cast<int>(w->bpr),
                static_cast<int>(m), mode, per_row};
#define LGH_B(TT, BB, KK, QQ) \
  if (p.T == TT && p.BPL == BB && p.KW == KK && p.quant == QQ) return launch_batch<TT, BB, KK, QQ>(a, st)
  LGH_B(4, 1, 1, true);
  LGH_B(4, 2, 1, true);
  LGH_B(4, 3, 1, true);
  LGH_B(4, 4, 1, true);
  LGH_B(4, 4, 2, true);
  LGH_B(4, 4, 4, true);
  LGH_B(8, 1, 1, false);
  LGH_B(8, 2, 1, false);
  LGH_B(8, 3, 1, false);
  LGH_B(8, 4, 1, false);
  LGH_B(8, 4, 2, false);
  LGH_B(16, 1, 1, false);
  LGH_B(16, 2, 1, false);
  LGH_B(16, 3, 1, false);
  LGH_B(16, 4, 1, false);
#undef LGH_B
  return hipErrorInvalidValue;
}

// Rows per wave for the Q8_0 GEMV.
static int pick_rows_per_wave(size_t n_total, int steps) {
  int r = 8;
  while (r > 1 && (n_total / static_cast<size_t>(r)) < 2048) r >>= 1;
  while (r > 1 && r * steps > 8) r >>= 1;
  return r;
}

hipError_t launch_q8_gemv(const lgh_q8 *w, const float *x, float *y, size_t tokens, hipStream_t st) {
  if (w->n == 0 || tokens == 0) return hipSuccess;
  Q8GemvArgs a{w->qs, w->sc, x, y, static_cast<int>(w->n), static_cast<int>(w->bpr), static_cast<int>(w->k)};
  const size_t smem = w->bpr * 36 + kWaves * sizeof(float);
  const int steps = static_cast<int>((w->bpr + kWave - 1) / kWave);
  const int R = pick_rows_per_wave(w->n * tokens, steps) >= 2 ? 2 : 1;
  const dim3 grid(static_cast<unsigned>((w->n + kWaves * R - 1) / (kWaves * R)), static_cast<unsigned>(tokens));
#define LGH_Q8(RR, SS)                                                                      \
  if (R == RR && steps == SS) {                                                             \
    hipLaunchKernelGGL((q8_gemv_kernel<RR, SS>), grid, dim3(kThreads), smem, st, a);        \
    return hipGetLastError();                                                               \
  }
  LGH_Q8(2, 1);
  LGH_Q8(1, 1);
  LGH_Q8(2, 2);
  LGH_Q8(1, 2);
  LGH_Q8(1, 3);
  LGH_Q8(1, 4);
  LGH_Q8(2, 3);
  LGH_Q8(2, 4);
  LGH_Q8(1, 5);
  LGH_Q8(1, 6);
  LGH_Q8(2, 5);
  LGH_Q8(2, 6);
#undef LGH_Q8
  return hipErrorInvalidValue;  // K > 12288: rejected by the API before launch
}

}  // namespace lgh
