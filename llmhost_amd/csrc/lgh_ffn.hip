// Decode-step SwiGLU FFN residual block for gfx950, one token (replaces
// Lfm2::ffn_residual_in, crates/llm-engine/src/lfm2.rs:883-911):
//   normed = rms_norm(hidden, ffn_norm)          crates/llm-cpu/src/ops.rs:8-23
//   g, u   = W1 normed, W3 normed                gemv_q4_pair, gemv_q4.rs:396-443
//   h      = silu(g) * u                         ops.rs:27-36, lfm2.rs:902-905
//   hidden = f32(f64(hidden) + f64(W2 h))        gemv_q4_add, gemv_q4.rs:356-363
// in two launches instead of five passes:
//   * ffn_gate_up_kernel: per workgroup, the norm of hidden (sum of squares in
//     f64, as the reference), the ActQ8 codes of `normed` in LDS, 32 rows of
//     W1 and the same 32 rows of W3 (one row of each per 16-lane DPP row),
//     then silu(g) * u for those 32 rows -- exactly one 32-element block of
//     h -- and that block's ActQ8 codes and scale;
//   * the down GEMV reading those codes (q4_gemv_kernel, PREQ), AddF64 into
//     hidden.
// The down GEMV therefore skips loading 4*inter bytes of h and quantizing it
// in every workgroup, which is the prologue that bounds the plain GEMV at
// K = 8192.
#include "lgh_device.h"
#include "lgh_internal.h"

namespace lgh {

namespace {

// Each 16-lane DPP row holds one row of W1 and the same row of W3, so a wave
// covers 4 rows of g and u and 8 waves cover one 32-row block of h: g, u and
// h = silu(g) * u meet in the lane that reduced them, and only h goes through
// LDS (to its block's quantizer).  Against 16 waves with W1 and W3 rows in
// separate waves and g / u exchanged through LDS: dim 1536, inter 8192, the
// whole block 10.0 -> 9.5 us (interleaved A/B), bit-identical.
constexpr int kFfnWaves = 8;
constexpr int kFfnThreads = kFfnWaves * kWave;

struct FfnUpArgs {
  const uint8_t *qs1, *qs3;  // W1 (gate), W3 (up): nibble planes [n][bpr][16]
  const uint16_t *sc1, *sc3;
  const float *x;   // hidden [k]
  const float *nw;  // norm weight [k], or null for no norm
  double inv_k;     // 1 / k in f64 (ops.rs:12)
  float eps;
  int bpr;        // k / 32
  int per_row;    // ActQ8 mode for `normed`
  int8_t *hq;     // ActQ8 (PerBlock) codes of h [n], or null
  float *hs;      // their scales [n / 32]
  float *hf;      // h [n], or null
  float *g_out;   // g [n], or null
  float *u_out;   // u [n], or null
};

template <int BPL>
__global__ __launch_bounds__(kFfnThreads) void ffn_gate_up_kernel(FfnUpArgs a) {
  constexpr int KB = 16 * BPL;  // blocks covered (>= bpr)
  constexpr int XJ = (KB * 8 + kFfnThreads - 1) / kFfnThreads;
  __shared__ __align__(16) int8_t s_qs[KB * 32];
  __shared__ float s_sa[KB];
  __shared__ float s_red[kFfnWaves];
  __shared__ double s_ss[kFfnWaves];
  __shared__ __align__(16) float s_h[32];
  const int bpr = a.bpr;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = uniform(tid / kWave);
  const int base = blockIdx.x * 32;
  const int row0 = base + wave * 4;
  const int r = lane >> 4, c = lane & 15;

  // (1) hidden and the norm weight (elements >= k read as 0).
  const auto xr = make_rsrc(a.x, static_cast<uint32_t>(bpr) * 128u);
  const auto nr = make_rsrc(a.nw, a.nw ? static_cast<uint32_t>(bpr) * 128u : 0u);
  float4 xv[XJ], nv[XJ];
#pragma unroll
  for (int j = 0; j < XJ; j++) {
    xv[j] = buf_load_f4(xr, static_cast<uint32_t>(tid + j * kFfnThreads) * 16u);
    nv[j] = buf_load_f4(nr, static_cast<uint32_t>(tid + j * kFfnThreads) * 16u);
  }
  // (1b) The norm and the quantization wait for every wave's hidden: queue
  // those requests before any wave's weight requests.
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);

  // (2) every weight load of this lane: its row of W1 and of W3, BPL blocks each.
  const size_t blk0 = static_cast<size_t>(row0) * bpr;
  const auto wr1 = make_rsrc(a.qs1 + blk0 * 16, static_cast<uint32_t>(4 * bpr) * 16u);
  const auto sr1 = make_rsrc(a.sc1 + blk0, static_cast<uint32_t>(4 * bpr) * 2u);
  const auto wr3 = make_rsrc(a.qs3 + blk0 * 16, static_cast<uint32_t>(4 * bpr) * 16u);
  const auto sr3 = make_rsrc(a.sc3 + blk0, static_cast<uint32_t>(4 * bpr) * 2u);
  uint4 w1[BPL], w3[BPL];
  uint16_t s1[BPL], s3[BPL];
#pragma unroll
  for (int j = 0; j < BPL; j++) {
    const int kb = c + 16 * j;
    const uint32_t blk = static_cast<uint32_t>(r * bpr + kb);
    w1[j] = buf_load16<kAuxNT>(wr1, kb < bpr ? blk * 16u : kOOB);
    s1[j] = buf_load_u16(sr1, kb < bpr ? blk * 2u : kOOB);
    w3[j] = buf_load16<kAuxNT>(wr3, kb < bpr ? blk * 16u : kOOB);
    s3[j] = buf_load_u16(sr3, kb < bpr ? blk * 2u : kOOB);
  }

  // (3) RMSNorm (ops.rs:8-23): sum of squares in f64, scale =
  // f32(1 / sqrt(sumsq * (1/dim) + eps)) in f64, normed = w * (x * scale) in
  // f32.  The f64 sum is a fixed tree instead of the reference's sequence.
  if (a.nw) {
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < XJ; j++) {
      const double x0 = xv[j].x, x1 = xv[j].y, x2 = xv[j].z, x3 = xv[j].w;
      ss += x0 * x0;
      ss += x1 * x1;
      ss += x2 * x2;
      ss += x3 * x3;
    }
    ss = wave_sum_dpp64(ss);
    if (lane == 0) s_ss[wave] = ss;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int i = 0; i < kFfnWaves; i++) tot += s_ss[i];
    const float scale = rms_scale(tot, a.inv_k, a.eps);
#pragma unroll
    for (int j = 0; j < XJ; j++) {
      xv[j].x = nv[j].x * (xv[j].x * scale);
      xv[j].y = nv[j].y * (xv[j].y * scale);
      xv[j].z = nv[j].z * (xv[j].z * scale);
      xv[j].w = nv[j].w * (xv[j].w * scale);
    }
  }

  // (4) ActQ8 of normed into LDS, shared by both matrices.
  quantize_regs_to_lds<kFfnThreads, XJ>(xv, bpr, a.per_row, s_qs, s_sa, s_red);

  // (5) dots + fold for both rows (branch-free: blocks past the row add
  // exactly 0), DPP row sums, then g, u and h of the lane's row.
  float ag = 0.0f, au = 0.0f;
#pragma unroll
  for (int j = 0; j < BPL; j++) {
    const int kb = c + 16 * j;
    const int kbc = kb < bpr ? kb : 0;
    const v4i *ap = reinterpret_cast<const v4i *>(s_qs + kbc * 32);
    const v4i a0 = ap[0], a1 = ap[1];
    const float sa = s_sa[kbc];
    ag = fmaf(static_cast<float>(dot_q4_block16(w1[j], a0, a1)), h2f(s1[j]) * sa, ag);
    au = fmaf(static_cast<float>(dot_q4_block16(w3[j], a0, a1)), h2f(s3[j]) * sa, au);
  }
  ag += dpp<0xB1>(ag);
  au += dpp<0xB1>(au);
  ag += dpp<0x4E>(ag);
  au += dpp<0x4E>(au);
  ag += dpp<0x141>(ag);
  au += dpp<0x141>(au);
  ag += dpp<0x140>(ag);
  au += dpp<0x140>(au);
  if (c == 0) {
    const int i = wave * 4 + r;
    const float g = ag * 0.0625f, u = au * 0.0625f;  // exact: undo the x16 of the unpack
    const float h = silu_mul1(g, u);
    s_h[i] = h;
    if (a.g_out) a.g_out[base + i] = g;
    if (a.u_out) a.u_out[base + i] = u;
    if (a.hf) a.hf[base + i] = h;
  }
  // (6) the block of h: its ActQ8 codes and scale (8 lanes, as
  // act_quant_kernel).
  if (!a.hq) return;  // uniform
  __syncthreads();
  if (wave == 0 && lane < 8) {
    const float4 hv = reinterpret_cast<const float4 *>(s_h)[lane];
    float scale;
    int sum;
    const int q = act_quant_group8(hv, false, 0.0f, scale, sum);
    reinterpret_cast<int *>(a.hq + base)[lane] = q;
    if (lane == 0) a.hs[blockIdx.x] = scale;
  }
}

// rms_norm over rows of dim (ops.rs:8-23): one workgroup per row, the f64
// sum of squares as a fixed tree (per-thread strided partials, DPP wave sums,
// the 4 wave sums in order), then out = w * (x * scale) in f32.
constexpr int kNormThreads = 256;

__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(const float *__restrict__ x,
                                                                const float *__restrict__ w, int dim, double inv_dim,
                                                                float eps, float *__restrict__ out) {
  __shared__ double s_ss[kNormThreads / kWave];
  const float *row = x + static_cast<size_t>(blockIdx.x) * dim;
  float *dst = out + static_cast<size_t>(blockIdx.x) * dim;
  double ss = 0.0;
  for (int i = threadIdx.x; i < dim; i += kNormThreads) {
    const double v = row[i];
    ss += v * v;
  }
  ss = wave_sum_dpp64(ss);
  if ((threadIdx.x & (kWave - 1)) == 0) s_ss[threadIdx.x / kWave] = ss;
  __syncthreads();
  double tot = 0.0;
#pragma unroll
  for (int i = 0; i < kNormThreads / kWave; i++) tot += s_ss[i];
  const float scale = rms_scale(tot, inv_dim, eps);
  for (int i = threadIdx.x; i < dim; i += kNormThreads) dst[i] = w[i] * (row[i] * scale);
}

// g = silu(g) * u (ops.rs:27-36, lfm2.rs:902-905), elementwise.
__global__ __launch_bounds__(256) void silu_mul_kernel(float *__restrict__ g, const float *__restrict__ u,
                                                       size_t n) {
  const size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  g[i] = silu_mul1(g[i], u[i]);
}

template <int BPL>
hipError_t launch_gate_up(const FfnUpArgs &a, int wgs, hipStream_t st) {
  hipLaunchKernelGGL(ffn_gate_up_kernel<BPL>, dim3(wgs), dim3(kFfnThreads), 0, st, a);
  return hipGetLastError();
}

}  // namespace

bool ffn_gate_up_supported(const lgh_q4 *w1) { return w1->bpr >= 1 && w1->bpr <= kFfnMaxBpr && w1->n % 32 == 0; }

hipError_t launch_ffn_gate_up(const lgh_q4 *w1, const lgh_q4 *w3, const float *x, const float *norm_w, float eps,
                              int per_row, int8_t *hq, float *hs, float *hf, float *g, float *u,
                              hipStream_t st) {
  if (!ffn_gate_up_supported(w1)) return hipErrorInvalidValue;
  if (w1->n == 0) return hipSuccess;
  const FfnUpArgs a{w1->qs, w3->qs, w1->sc, w3->sc, x, norm_w, 1.0 / static_cast<double>(w1->k), eps,
                    static_cast<int>(w1->bpr), per_row, hq, hs, hf, g, u};
  const int wgs = static_cast<int>(w1->n / 32);
  switch ((w1->bpr + 15) / 16) {
    case 1: return launch_gate_up<1>(a, wgs, st);
    case 2: return launch_gate_up<2>(a, wgs, st);
    case 3: return launch_gate_up<3>(a, wgs, st);
    default: return launch_gate_up<4>(a, wgs, st);
  }
}

hipError_t launch_rms_norm(const float *x, const float *w, size_t dim, size_t rows, float eps, float *out,
                           hipStream_t st) {
  if (rows == 0 || dim == 0) return hipSuccess;
  hipLaunchKernelGGL(rms_norm_kernel, dim3(static_cast<unsigned>(rows)), dim3(kNormThreads), 0, st, x, w,
                     static_cast<int>(dim), 1.0 / static_cast<double>(dim), eps, out);
  return hipGetLastError();
}

hipError_t launch_silu_mul(float *g, const float *u, size_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, st, g, u, n);
  return hipGetLastError();
}

}  // namespace lgh
