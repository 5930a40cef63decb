// M = 1 kernels for gfx950: fused activation-quant + Q4 / Q8_0 GEMV, the
// load-time repack / quantize kernels and the integer block-dot test hooks.
//
// Q4 GEMV (replaces crates/llm-cpu/src/gemv_q4.rs:344-443, 499-667):
//   * one workgroup = 4 waves; every workgroup first quantizes x into LDS
//     (ActQ8, bit-exact; 8 lanes per 32-element block), after issuing the
//     global loads of its weight rows so HBM latency overlaps the prologue;
//   * each wave owns R consecutive output rows; lane l walks the blocks
//     kb = l, l+64, ... of those rows: one 128-bit load of 32 nibbles + one
//     f16 scale per block, 8 v_dot4_i32_i8 against the LDS activations, then
//     acc = fma(f32(16*idot), sw*sa, acc) -- the VNNI kernel's fold
//     (gemv_q4.rs:659-661) in a different summation order;
//   * a wave reduction gives the row; lane 0 applies Assign or AddF64
//     (gemv_q4.rs:486-497).
// All S k-steps of a lane are loaded before the first is consumed, so a wave
// keeps R*S*16 bytes per lane in flight.
#include "lgh_device.h"
#include "lgh_internal.h"

namespace lgh {

namespace {

constexpr int kThreads = 256;
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

// Quantize x[0, 32*bpr) into LDS: s_qs (natural order) and s_sa.
__device__ __forceinline__ void quantize_x_to_lds(const float *__restrict__ x, int bpr, int per_row,
                                                  int8_t *s_qs, float *s_sa, float *s_red) {
  const int tid = threadIdx.x;
  float row_scale = 0.0f;
  if (per_row) {
    float m = 0.0f;
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    for (int i = tid; i < bpr * 8; i += kThreads) {
      float4 v = x4[i];
      m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    m = wave_max(m);
    if ((tid & (kWave - 1)) == 0) s_red[tid / kWave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    row_scale = __fdiv_rn(m, 127.0f);
  }
  const int g = tid & 7;
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  for (int b = tid >> 3; b < bpr; b += kThreads / 8) {
    float scale;
    int sum;
    int q = act_quant_group8(x4[b * 8 + g], per_row != 0, row_scale, scale, sum);
    reinterpret_cast<int *>(s_qs)[b * 8 + g] = q;
    if (g == 0) s_sa[b] = scale;
  }
  __syncthreads();
}

__device__ __forceinline__ void store_row(float *y, int row, float acc16, int mode) {
  const float v = acc16 * 0.0625f;  // exact: undo the x16 of the nibble unpack
  if (mode == LGH_ADD_F64)
    y[row] = static_cast<float>(static_cast<double>(y[row]) + static_cast<double>(v));
  else
    y[row] = v;
}

// R rows per wave, S k-steps of 64 blocks per lane (bpr <= 64*S).
template <int R, int S>
__global__ __launch_bounds__(kThreads) void q4_gemv_kernel(Q4GemvArgs a) {
  extern __shared__ __align__(16) char smem[];
  const int bpr = a.bpr;
  int8_t *s_qs = reinterpret_cast<int8_t *>(smem);
  float *s_sa = reinterpret_cast<float *>(smem + bpr * 32);
  float *s_red = s_sa + bpr;

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
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row0 = (wg * kWaves + wave) * R;

  // Issue every weight load of this lane first.
  uint4 w[S][R];
  uint16_t s[S][R];
#pragma unroll
  for (int st = 0; st < S; st++) {
    const int kb = st * kWave + lane;
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int row = row0 + r;
      if (row < a.n && kb < bpr) {
        const size_t blk = static_cast<size_t>(row) * bpr + kb;
        w[st][r] = load_nt16(reinterpret_cast<const uint4 *>(qs) + blk);
        s[st][r] = sc[blk];
      } else {
        w[st][r] = make_uint4(0, 0, 0, 0);
        s[st][r] = 0;
      }
    }
  }

  quantize_x_to_lds(a.x, bpr, a.per_row, s_qs, s_sa, s_red);

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
      for (int r = 0; r < R; r++) {
        const int d = dot_q4_block16(w[st][r], a0, a1);
        acc[r] = fmaf(static_cast<float>(d), h2f(s[st][r]) * sa, acc[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++) {
    const float t = wave_sum(acc[r]);
    if (lane == 0 && row0 + r < a.n) store_row(y, row0 + r, t, a.mode);
  }
}

// Generic fallback for any K: loops over k-steps, one step of loads at a time.
template <int R>
__global__ __launch_bounds__(kThreads) void q4_gemv_kernel_any(Q4GemvArgs a) {
  extern __shared__ __align__(16) char smem[];
  const int bpr = a.bpr;
  int8_t *s_qs = reinterpret_cast<int8_t *>(smem);
  float *s_sa = reinterpret_cast<float *>(smem + bpr * 32);
  float *s_red = s_sa + bpr;
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
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row0 = (wg * kWaves + wave) * R;
  quantize_x_to_lds(a.x, bpr, a.per_row, s_qs, s_sa, s_red);
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) acc[r] = 0.0f;
  for (int kb = lane; kb < bpr; kb += kWave) {
    const v4i *ap = reinterpret_cast<const v4i *>(s_qs + kb * 32);
    const v4i a0 = ap[0], a1 = ap[1];
    const float sa = s_sa[kb];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int row = row0 + r;
      if (row < a.n) {
        const size_t blk = static_cast<size_t>(row) * bpr + kb;
        const uint4 w = reinterpret_cast<const uint4 *>(qs)[blk];
        const int d = dot_q4_block16(w, a0, a1);
        acc[r] = fmaf(static_cast<float>(d), h2f(sc[blk]) * sa, acc[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++) {
    const float t = wave_sum(acc[r]);
    if (lane == 0 && row0 + r < a.n) store_row(y, row0 + r, t, a.mode);
  }
}

template <int R, int S>
hipError_t launch_q4_gemv_rs(const Q4GemvArgs &a, int total_wgs, size_t smem, hipStream_t st) {
  hipLaunchKernelGGL((q4_gemv_kernel<R, S>), dim3(total_wgs), dim3(kThreads), smem, st, a);
  return hipGetLastError();
}

template <int R>
hipError_t launch_q4_gemv_r(const Q4GemvArgs &a, int steps, int total_wgs, size_t smem,
                            hipStream_t st) {
  switch (steps) {
    case 1: return launch_q4_gemv_rs<R, 1>(a, total_wgs, smem, st);
    case 2: return launch_q4_gemv_rs<R, 2>(a, total_wgs, smem, st);
    case 3: return launch_q4_gemv_rs<R, 3>(a, total_wgs, smem, st);
    case 4: return launch_q4_gemv_rs<R, 4>(a, total_wgs, smem, st);
    default:
      hipLaunchKernelGGL((q4_gemv_kernel_any<R>), dim3(total_wgs), dim3(kThreads), smem, st, a);
      return hipGetLastError();
  }
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

template <int R>
__global__ __launch_bounds__(kThreads) void q8_gemv_kernel(Q8GemvArgs a) {
  extern __shared__ __align__(16) char smem[];
  const int bpr = a.bpr;
  int8_t *s_qs = reinterpret_cast<int8_t *>(smem);
  float *s_sa = reinterpret_cast<float *>(smem + bpr * 32);
  float *s_red = s_sa + bpr;
  const int tok = blockIdx.y;
  const float *x = a.x + static_cast<size_t>(tok) * a.k;
  float *y = a.y + static_cast<size_t>(tok) * a.n;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row0 = (blockIdx.x * kWaves + wave) * R;
  quantize_x_to_lds(x, bpr, 0, s_qs, s_sa, s_red);  // always per block (weights.rs:197)
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) acc[r] = 0.0f;
  for (int kb = lane; kb < bpr; kb += kWave) {
    const v4i *ap = reinterpret_cast<const v4i *>(s_qs + kb * 32);
    const v4i a0 = ap[0], a1 = ap[1];
    const float sa = s_sa[kb];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int row = row0 + r;
      if (row < a.n) {
        const size_t blk = static_cast<size_t>(row) * bpr + kb;
        const uint4 *wp = reinterpret_cast<const uint4 *>(a.qs) + blk * 2;
        const uint4 w0 = load_nt16(wp);
        const uint4 w1 = load_nt16(wp + 1);
        const int d = dot_q8_block(w0, w1, a0, a1);
        acc[r] = fmaf(static_cast<float>(d), h2f(a.sc[blk]) * sa, acc[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++) {
    const float t = wave_sum(acc[r]);
    if (lane == 0 && row0 + r < a.n) y[row0 + r] = t;
  }
}

// ---- batched activation quantization (gemv_q4.rs:747-798) -----------------
__global__ __launch_bounds__(kThreads) void row_amax_kernel(const float *__restrict__ x, int k,
                                                            float *row_scale) {
  __shared__ float s_red[kWaves];
  const float4 *x4 = reinterpret_cast<const float4 *>(x + static_cast<size_t>(blockIdx.x) * k);
  float m = 0.0f;
  for (int i = threadIdx.x; i < k / 4; i += kThreads) {
    float4 v = x4[i];
    m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  m = wave_max(m);
  if ((threadIdx.x & (kWave - 1)) == 0) s_red[threadIdx.x / kWave] = m;
  __syncthreads();
  if (threadIdx.x == 0)
    row_scale[blockIdx.x] = __fdiv_rn(fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3])), 127.0f);
}

// One 8-lane group per 32-element block; grid.x covers blocks of all rows.
__global__ __launch_bounds__(kThreads) void act_quant_kernel(const float *__restrict__ x, int m, int bpr,
                                                             int per_row, const float *row_scale,
                                                             int8_t *qs, float *scales, int32_t *sums) {
  const size_t total = static_cast<size_t>(m) * bpr;
  const size_t b = (static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x) >> 3;
  const int g = threadIdx.x & 7;
  if (b >= total) return;  // whole 8-lane groups exit together
  const size_t row = b / bpr;
  const float rs = per_row ? row_scale[row] : 0.0f;
  float scale;
  int sum;
  const float4 v = reinterpret_cast<const float4 *>(x)[b * 8 + g];
  const int q = act_quant_group8(v, per_row != 0, rs, scale, sum);
  reinterpret_cast<int *>(qs)[b * 8 + g] = q;
  if (g == 0) {
    scales[b] = scale;
    if (sums) sums[b] = sum;
  }
}

// ---- load-time kernels ----------------------------------------------------
// Raw BlockQ4 (18 bytes) -> repacked nibble block + f16 scale.
__device__ __forceinline__ uint32_t raw_nib(const uint8_t *q, int e) {
  const uint32_t b = q[e >> 1];
  return (e & 1) ? (b >> 4) : (b & 0xFu);
}

__global__ void q4_repack_kernel(const uint8_t *__restrict__ raw, size_t nblocks, uint8_t *qs,
                                 uint16_t *sc) {
  const size_t b = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const uint8_t *blk = raw + b * 18;
  uint8_t q[16];
#pragma unroll
  for (int i = 0; i < 16; i++) q[i] = blk[2 + i];
  uint32_t out[4];
#pragma unroll
  for (int d = 0; d < 4; d++) {
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t byte = raw_nib(q, 8 * d + i) | (raw_nib(q, 8 * d + 4 + i) << 4);
      v |= byte << (8 * i);
    }
    out[d] = v;
  }
  reinterpret_cast<uint4 *>(qs)[b] = make_uint4(out[0], out[1], out[2], out[3]);
  sc[b] = static_cast<uint16_t>(blk[0] | (blk[1] << 8));
}

__global__ void q4_unpack_kernel(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ sc,
                                 size_t nblocks, uint8_t *raw) {
  const size_t b = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const uint4 w = reinterpret_cast<const uint4 *>(qs)[b];
  const uint32_t d[4] = {w.x, w.y, w.z, w.w};
  uint8_t nib[32];
#pragma unroll
  for (int dd = 0; dd < 4; dd++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t byte = (d[dd] >> (8 * i)) & 0xFFu;
      nib[8 * dd + i] = byte & 0xFu;
      nib[8 * dd + 4 + i] = byte >> 4;
    }
  uint8_t *blk = raw + b * 18;
  blk[0] = sc[b] & 0xFF;
  blk[1] = sc[b] >> 8;
#pragma unroll
  for (int i = 0; i < 16; i++) blk[2 + i] = nib[2 * i] | (nib[2 * i + 1] << 4);
}

__global__ void q8_repack_kernel(const uint8_t *__restrict__ raw, size_t nblocks, int8_t *qs,
                                 uint16_t *sc) {
  const size_t b = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const uint8_t *blk = raw + b * 34;
  uint32_t out[8];
#pragma unroll
  for (int d = 0; d < 8; d++)
    out[d] = blk[2 + 4 * d] | (blk[3 + 4 * d] << 8) | (blk[4 + 4 * d] << 16) |
             (static_cast<uint32_t>(blk[5 + 4 * d]) << 24);
  uint4 *dst = reinterpret_cast<uint4 *>(qs) + 2 * b;
  dst[0] = make_uint4(out[0], out[1], out[2], out[3]);
  dst[1] = make_uint4(out[4], out[5], out[6], out[7]);
  sc[b] = static_cast<uint16_t>(blk[0] | (blk[1] << 8));
}

__global__ void q8_unpack_kernel(const int8_t *__restrict__ qs, const uint16_t *__restrict__ sc,
                                 size_t nblocks, uint8_t *raw) {
  const size_t b = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  uint8_t *blk = raw + b * 34;
  blk[0] = sc[b] & 0xFF;
  blk[1] = sc[b] >> 8;
#pragma unroll
  for (int i = 0; i < 32; i++) blk[2 + i] = static_cast<uint8_t>(qs[b * 32 + i]);
}

// BlockQ4::quantize (crates/llm-quant/src/lib.rs:63-79), one thread per block.
__global__ void q4_quantize_kernel(const float *__restrict__ w, size_t nblocks, uint8_t *qs,
                                   uint16_t *sc) {
  const size_t b = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const float *src = w + b * 32;
  float amax = 0.0f;
  for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(src[i]));
  const uint16_t sbits = f2h(__fdiv_rn(amax, 8.0f));
  const float sf = h2f(sbits);
  const float inv = sf == 0.0f ? 0.0f : __fdiv_rn(1.0f, sf);
  uint32_t nib[32];
  for (int i = 0; i < 32; i++) {
    const int q = static_cast<int>(fminf(fmaxf(roundf(src[i] * inv), -8.0f), 7.0f));
    nib[i] = static_cast<uint32_t>(q) & 0xFu;
  }
  uint32_t out[4];
  for (int d = 0; d < 4; d++) {
    uint32_t v = 0;
    for (int i = 0; i < 4; i++) v |= (nib[8 * d + i] | (nib[8 * d + 4 + i] << 4)) << (8 * i);
    out[d] = v;
  }
  reinterpret_cast<uint4 *>(qs)[b] = make_uint4(out[0], out[1], out[2], out[3]);
  sc[b] = sbits;
}

// BlockQ8_0::quantize (crates/llm-quant/src/lib.rs:26-37), one thread per block.
__global__ void q8_quantize_kernel(const float *__restrict__ w, size_t nblocks, int8_t *qs,
                                   uint16_t *sc) {
  const size_t b = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const float *src = w + b * 32;
  float amax = 0.0f;
  for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(src[i]));
  const uint16_t sbits = f2h(__fdiv_rn(amax, 127.0f));
  const float sf = h2f(sbits);
  const float inv = sf == 0.0f ? 0.0f : __fdiv_rn(1.0f, sf);
  for (int i = 0; i < 32; i++)
    qs[b * 32 + i] = static_cast<int8_t>(fminf(fmaxf(roundf(src[i] * inv), -127.0f), 127.0f));
  sc[b] = sbits;
}

// ---- test hooks -------------------------------------------------------------
__global__ void q4_block_dots_kernel(const uint8_t *__restrict__ qs, const int8_t *__restrict__ a,
                                     size_t nblocks, int32_t *out) {
  const size_t b = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const uint4 w = reinterpret_cast<const uint4 *>(qs)[b];
  const v4i *ap = reinterpret_cast<const v4i *>(a + b * 32);
  out[b] = dot_q4_block16(w, ap[0], ap[1]) >> 4;  // exact: the sum is 16 * dot
}

__global__ void q8_block_dots_kernel(const int8_t *__restrict__ qs, const int8_t *__restrict__ a,
                                     size_t nblocks, int32_t *out) {
  const size_t b = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const uint4 *wp = reinterpret_cast<const uint4 *>(qs) + 2 * b;
  const v4i *ap = reinterpret_cast<const v4i *>(a + b * 32);
  out[b] = dot_q8_block(wp[0], wp[1], ap[0], ap[1]);
}

inline unsigned blocks_for(size_t items, unsigned per) {
  return static_cast<unsigned>((items + per - 1) / per);
}

}  // namespace

hipError_t launch_q4_repack(const uint8_t *raw, size_t nblocks, uint8_t *qs, uint16_t *sc,
                            hipStream_t st) {
  if (!nblocks) return hipSuccess;
  hipLaunchKernelGGL(q4_repack_kernel, dim3(blocks_for(nblocks, 256)), dim3(256), 0, st, raw, nblocks,
                     qs, sc);
  return hipGetLastError();
}

hipError_t launch_q4_unpack(const uint8_t *qs, const uint16_t *sc, size_t nblocks, uint8_t *raw,
                            hipStream_t st) {
  if (!nblocks) return hipSuccess;
  hipLaunchKernelGGL(q4_unpack_kernel, dim3(blocks_for(nblocks, 256)), dim3(256), 0, st, qs, sc,
                     nblocks, raw);
  return hipGetLastError();
}

hipError_t launch_q8_repack(const uint8_t *raw, size_t nblocks, int8_t *qs, uint16_t *sc,
                            hipStream_t st) {
  if (!nblocks) return hipSuccess;
  hipLaunchKernelGGL(q8_repack_kernel, dim3(blocks_for(nblocks, 256)), dim3(256), 0, st, raw, nblocks,
                     qs, sc);
  return hipGetLastError();
}

hipError_t launch_q8_unpack(const int8_t *qs, const uint16_t *sc, size_t nblocks, uint8_t *raw,
                            hipStream_t st) {
  if (!nblocks) return hipSuccess;
  hipLaunchKernelGGL(q8_unpack_kernel, dim3(blocks_for(nblocks, 256)), dim3(256), 0, st, qs, sc,
                     nblocks, raw);
  return hipGetLastError();
}

hipError_t launch_q4_quantize(const float *w, size_t nblocks, uint8_t *qs, uint16_t *sc,
                              hipStream_t st) {
  if (!nblocks) return hipSuccess;
  hipLaunchKernelGGL(q4_quantize_kernel, dim3(blocks_for(nblocks, 256)), dim3(256), 0, st, w,
                     nblocks, qs, sc);
  return hipGetLastError();
}

hipError_t launch_q8_quantize(const float *w, size_t nblocks, int8_t *qs, uint16_t *sc,
                              hipStream_t st) {
  if (!nblocks) return hipSuccess;
  hipLaunchKernelGGL(q8_quantize_kernel, dim3(blocks_for(nblocks, 256)), dim3(256), 0, st, w,
                     nblocks, qs, sc);
  return hipGetLastError();
}

// Row-group size: aim for >= ~2048 waves over the launch while keeping all
// of a lane's loads (R*S) in registers.
static int pick_rows_per_wave(size_t n_total, int steps) {
  int r = 8;
  while (r > 1 && (n_total / static_cast<size_t>(r)) < 2048) r >>= 1;
  while (r > 1 && r * steps > 8) r >>= 1;
  return r;
}

hipError_t launch_q4_gemv(const lgh_q4 *w0, float *y0, const lgh_q4 *w1, float *y1, const float *x,
                          int mode, int per_row, hipStream_t st) {
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
  a.mode = mode;
  a.per_row = per_row;
  if (a.n == 0) return hipSuccess;
  const int steps = (a.bpr + kWave - 1) / kWave;
  const int nmat = w1 ? 2 : 1;
  const int R = pick_rows_per_wave(static_cast<size_t>(a.n) * nmat, steps);
  a.wgs0 = (a.n + kWaves * R - 1) / (kWaves * R);
  const int total = a.wgs0 * nmat;
  const size_t smem = static_cast<size_t>(a.bpr) * 36 + kWaves * sizeof(float);
  switch (R) {
    case 8: return launch_q4_gemv_r<8>(a, steps, total, smem, st);
    case 4: return launch_q4_gemv_r<4>(a, steps, total, smem, st);
    case 2: return launch_q4_gemv_r<2>(a, steps, total, smem, st);
    default: return launch_q4_gemv_r<1>(a, steps, total, smem, st);
  }
}

hipError_t launch_q8_gemv(const lgh_q8 *w, const float *x, float *y, size_t tokens, hipStream_t st) {
  if (w->n == 0 || tokens == 0) return hipSuccess;
  Q8GemvArgs a{w->qs, w->sc, x, y, static_cast<int>(w->n), static_cast<int>(w->bpr),
               static_cast<int>(w->k)};
  const size_t smem = w->bpr * 36 + kWaves * sizeof(float);
  constexpr int R = 2;
  const unsigned wgs = static_cast<unsigned>((w->n + kWaves * R - 1) / (kWaves * R));
  hipLaunchKernelGGL(q8_gemv_kernel<R>, dim3(wgs, static_cast<unsigned>(tokens)), dim3(kThreads), smem,
                     st, a);
  return hipGetLastError();
}

hipError_t launch_act_quant(const float *x, size_t m, size_t k, int per_row, int8_t *qs, float *scales,
                            int32_t *sums, float *row_scale, hipStream_t st) {
  if (m == 0 || k == 0) return hipSuccess;
  const size_t bpr = k / 32;
  if (per_row) {
    hipLaunchKernelGGL(row_amax_kernel, dim3(static_cast<unsigned>(m)), dim3(kThreads), 0, st, x,
                       static_cast<int>(k), row_scale);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const size_t threads = m * bpr * 8;
  hipLaunchKernelGGL(act_quant_kernel, dim3(blocks_for(threads, kThreads)), dim3(kThreads), 0, st, x,
                     static_cast<int>(m), static_cast<int>(bpr), per_row, row_scale, qs, scales, sums);
  return hipGetLastError();
}

hipError_t launch_q4_block_dots(const uint8_t *qs, const int8_t *a, size_t nblocks, int32_t *out,
                                hipStream_t st) {
  if (!nblocks) return hipSuccess;
  hipLaunchKernelGGL(q4_block_dots_kernel, dim3(blocks_for(nblocks, 256)), dim3(256), 0, st, qs, a,
                     nblocks, out);
  return hipGetLastError();
}

hipError_t launch_q8_block_dots(const int8_t *qs, const int8_t *a, size_t nblocks, int32_t *out,
                                hipStream_t st) {
  if (!nblocks) return hipSuccess;
  hipLaunchKernelGGL(q8_block_dots_kernel, dim3(blocks_for(nblocks, 256)), dim3(256), 0, st, qs, a,
                     nblocks, out);
  return hipGetLastError();
}

}  // namespace lgh
