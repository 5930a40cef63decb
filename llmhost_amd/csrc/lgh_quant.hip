// Activation quantization, load-time weight kernels and integer test hooks
// for gfx950:
//   * batched ActQ8 quantization (crates/llm-cpu/src/gemv_q4.rs:747-798),
//     bit-exact, feeding the MFMA GEMM;
//   * BlockQ4 / BlockQ8_0 repack to the device layout (and back), and the
//     device quantizers BlockQ4::quantize / BlockQ8_0::quantize
//     (crates/llm-quant/src/lib.rs:26-37, 63-79);
//   * per-block integer dots through the GEMV's unpack + v_dot4 path.
#include "lgh_device.h"
#include "lgh_internal.h"

namespace lgh {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

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
    row_scale[blockIdx.x] = div127_rn(fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3])));
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
