// Device helpers shared by the gfx950 kernels (wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/llm_gpu_hip.h"

namespace lgh {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// 128-bit streaming load (nontemporal: weights are read once per launch).
__device__ __forceinline__ uint4 load_nt16(const void *p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ---- raw buffer loads ------------------------------------------------------
// A buffer resource covers [base, base + bytes); a load whose byte offset is
// out of that range returns 0 (hardware range check), so tails and padding
// need no branches and every load of a lane can be issued back to back.
// kOOB is an offset that is always out of range.  `base` must be uniform
// across the wave (it lives in scalar registers).
constexpr uint32_t kOOB = 0x80000000u;
constexpr int kBufDword3 = 0x00020000;  // gfx9-family raw buffer: 32-bit data, no swizzle
constexpr int kAuxNT = 2;               // nontemporal (streaming) hint

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), kBufDword3);
}

template <int Aux = 0>
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, Aux);
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint2 buf_load8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(off), 0, 0);
  return make_uint2(v.x, v.y);
}

__device__ __forceinline__ float4 buf_load_f4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  // Bit-cast the whole vector: this clang reads element 0 for every
  // __builtin_bit_cast(float, v.y)-style cast of a single vector element.
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const f32x4 v = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0));
  return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint16_t buf_load_u16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(off), 0, 0);
}

__device__ __forceinline__ float buf_load_f32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(off), 0, 0));
}

// Wave-uniform value as a scalar (the compiler cannot prove threadIdx.x / 64
// uniform by itself).
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// ---- DPP wave64 sum --------------------------------------------------------
template <int Ctrl, int RowMask = 0xf>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), Ctrl, RowMask,
                                                               0xf, false));
}

// Sum over the 64 lanes, result valid in every lane: DPP within rows of 16
// (quad_perm 1032, quad_perm 2301, row_half_mirror, row_mirror), then the 4
// row partials are read as scalars and added.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror: lane i <-> 7-i within 8
  v += dpp<0x140>(v);  // row_mirror: lane i <-> 15-i within 16
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (r0 + r1) + (r2 + r3);
}

// The same wave64 sum for f64 (each DPP move is two 32-bit moves).
template <int Ctrl>
__device__ __forceinline__ double dpp64(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(b & 0xffffffffu), Ctrl, 0xf, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(b >> 32), Ctrl, 0xf, 0xf, false);
  return __builtin_bit_cast(double, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                        static_cast<uint32_t>(lo));
}

__device__ __forceinline__ double readlane64(double v, int lane) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(b & 0xffffffffu), lane));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(b >> 32), lane));
  return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ double wave_sum_dpp64(double v) {
  v += dpp64<0xB1>(v);
  v += dpp64<0x4E>(v);
  v += dpp64<0x141>(v);
  v += dpp64<0x140>(v);
  return (readlane64(v, 0) + readlane64(v, 16)) + (readlane64(v, 32) + readlane64(v, 48));
}

// f16 bits -> f32, exact (v_cvt_f32_f16; every binary16 value is a binary32
// value), matching half::f16::to_f32.
__device__ __forceinline__ float h2f(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// f32 -> f16 bits, round to nearest even (v_cvt_f16_f32 under the default
// round-to-nearest-even mode), matching half::f16::from_f32.
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Unpack one repacked nibble dword into two dwords of signed bytes, each
// byte = 16 * nibble value: lo -> elements 8d..8d+3, hi -> 8d+4..8d+7.
__device__ __forceinline__ int nib_lo16(uint32_t d) { return static_cast<int>((d << 4) & 0xF0F0F0F0u); }
__device__ __forceinline__ int nib_hi16(uint32_t d) { return static_cast<int>(d & 0xF0F0F0F0u); }

__device__ __forceinline__ int sdot4(int a, int b, int c) {
  return __builtin_amdgcn_sdot4(a, b, c, false);  // v_dot4_i32_i8, no clamp
}

// 16 x (sum over the block of nibble * a), a = 32 int8 activations in natural
// order as 8 dwords.  |result| <= 16*8*127*32 < 2^20, exact in i32 and f32.
__device__ __forceinline__ int dot_q4_block16(uint4 w, v4i a0, v4i a1) {
  int acc = 0;
  acc = sdot4(nib_lo16(w.x), a0.x, acc);
  acc = sdot4(nib_hi16(w.x), a0.y, acc);
  acc = sdot4(nib_lo16(w.y), a0.z, acc);
  acc = sdot4(nib_hi16(w.y), a0.w, acc);
  acc = sdot4(nib_lo16(w.z), a1.x, acc);
  acc = sdot4(nib_hi16(w.z), a1.y, acc);
  acc = sdot4(nib_lo16(w.w), a1.z, acc);
  acc = sdot4(nib_hi16(w.w), a1.w, acc);
  return acc;
}

// Q8_0 x Q8 block dot: 32 int8 weights (two uint4) against 32 int8 acts.
__device__ __forceinline__ int dot_q8_block(uint4 w0, uint4 w1, v4i a0, v4i a1) {
  int acc = 0;
  acc = sdot4(static_cast<int>(w0.x), a0.x, acc);
  acc = sdot4(static_cast<int>(w0.y), a0.y, acc);
  acc = sdot4(static_cast<int>(w0.z), a0.z, acc);
  acc = sdot4(static_cast<int>(w0.w), a0.w, acc);
  acc = sdot4(static_cast<int>(w1.x), a1.x, acc);
  acc = sdot4(static_cast<int>(w1.y), a1.y, acc);
  acc = sdot4(static_cast<int>(w1.z), a1.z, acc);
  acc = sdot4(static_cast<int>(w1.w), a1.w, acc);
  return acc;
}

// Unpack the 8 nibble bytes of one half block (uint2) into the 16-byte MFMA
// operand for elements 16h..16h+15 (values x16).
__device__ __forceinline__ v4i unpack_half16(uint2 w) {
  v4i r;
  r.x = nib_lo16(w.x);
  r.y = nib_hi16(w.x);
  r.z = nib_lo16(w.y);
  r.w = nib_hi16(w.y);
  return r;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// ---- exact fast divisions for ActQ8 -----------------------------------------
// RN(a / 127) for every a >= 0: q0 = a*y with y = RN(1/127), then one
// Markstein correction q = fma(fma(-q0, 127, a), y, q0), proven exhaustively
// over every finite a >= 0 (denormals included) by tests/fastquant_check.c.
// At a = +inf the correction term is inf - inf, so inf / 127 = inf is
// selected directly.
__device__ __forceinline__ float div127_rn(float a) {
  const float y = 0x1.020408p-7f;  // RN(1/127)
  const float q0 = a * y;
  const float q = fmaf(fmaf(-q0, 127.0f, a), y, q0);
  return a == __builtin_inff() ? a : q;
}

// RN(1 / s) for s > 0: v_rcp_f32 (faithful, 1 ulp) refined by one FMA Newton
// step, which tests/fastquant_check.c proves correctly rounded for either
// faithful starting value for every s in [2^-126, 2^126) except the
// all-ones significand; those and out-of-range s use the IEEE division, on a
// real branch: the division's operand passes through an empty asm inside it,
// so the compiler cannot compute the division for every lane and select.
__device__ __forceinline__ float recip_rn(float s) {
  const float y0 = __builtin_amdgcn_rcpf(s);
  float q = fmaf(fmaf(-s, y0, 1.0f), y0, y0);
  const uint32_t b = __builtin_bit_cast(uint32_t, s);
  if (b < 0x00800000u || b >= 0x7E800000u || (b & 0x7FFFFFu) == 0x7FFFFFu) {
    float t = s;
    asm volatile("" : "+v"(t));
    q = __fdiv_rn(1.0f, t);
  }
  return q;
}

// clamp(round_half_away_from_zero(v * inv), -127, 127) from a finite
// inv2 = 2 * inv: i = trunc(2y) exactly (RN(v * 2inv) = 2 RN(v * inv)), and
// for an integer i = trunc(2y), round_half_away(y) = (i + (i < 0 ? -1 : 0) + 1)
// >> 1 with an arithmetic shift (y >= 0: floor((floor(2y) + 1) / 2); y < 0:
// floor(i / 2)).  |v| <= amax keeps |v * inv2| below 256, so i never
// saturates.  NaN converts to 0, like Rust's `NaN as i8`.
__device__ __forceinline__ int quant_code(float v, float inv2) {
  const int i = static_cast<int>(v * inv2);  // v_cvt_i32_f32 truncates
  const int q = (i + (i >> 31) + 1) >> 1;
  return min(max(q, -127), 127);
}

// The reference's own arithmetic, `(v * inv).round().clamp(-127.0, 127.0) as
// i8`, for blocks whose scale is below 2^-127 (2 * inv overflows, and inv
// itself may be inf): clamp keeps NaN and a NaN cast is 0.
__device__ __forceinline__ int quant_code_ref(float v, float inv) {
  const float r = fminf(fmaxf(roundf(v * inv), -127.0f), 127.0f);
  return (v * inv) != (v * inv) ? 0 : static_cast<int>(r);
}

// ActQ8 quantization of one 32-element block by a group of 8 lanes
// (crates/llm-cpu/src/gemv_q4.rs:77-94).  Lane j of the group holds elements
// 4j..4j+3 in v.  Returns the packed int8 codes for those 4 elements; writes
// the block scale and the block sum of codes (valid in every group lane).
//   scale = amax / 127               (f32, correctly rounded)
//   inv   = scale == 0 ? 0 : 1/scale (f32, correctly rounded)
//   q     = clamp(round_half_away_from_zero(v * inv), -127, 127)
// With per_row, `row_scale` (= row amax / 127) replaces the block scale.
__device__ __forceinline__ int act_quant_group8(float4 v, bool per_row, float row_scale, float &scale,
                                                int &sum) {
  // amax folds |v| into 0.0 with Rust's f32::max, which skips NaN: each
  // lane's partial starts at 0 and is never NaN, and non-negative floats
  // order like their bit patterns, so the 8-lane max (DPP quad_perm
  // [1,0,3,2], [2,3,0,1], row_half_mirror) runs on integers.
  const float m4 = fmaxf(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))), 0.0f);
  uint32_t mb = __builtin_bit_cast(uint32_t, m4);
  mb = max(mb, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mb), 0xB1, 0xf, 0xf, false)));
  mb = max(mb, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mb), 0x4E, 0xf, 0xf, false)));
  mb = max(mb, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mb), 0x141, 0xf, 0xf, false)));
  const float amax = __builtin_bit_cast(float, mb);
  scale = per_row ? row_scale : div127_rn(amax);
  const float inv = scale == 0.0f ? 0.0f : recip_rn(scale);
  const float inv2 = 2.0f * inv;
  int q0, q1, q2, q3;
  if (inv2 <= 0x1.fffffep127f) {  // uniform per group; false only for scale < 2^-127
    q0 = quant_code(v.x, inv2);
    q1 = quant_code(v.y, inv2);
    q2 = quant_code(v.z, inv2);
    q3 = quant_code(v.w, inv2);
  } else {
    q0 = quant_code_ref(v.x, inv);
    q1 = quant_code_ref(v.y, inv);
    q2 = quant_code_ref(v.z, inv);
    q3 = quant_code_ref(v.w, inv);
  }
  int s = q0 + q1 + q2 + q3;
  s += __builtin_amdgcn_update_dpp(0, s, 0xB1, 0xf, 0xf, false);
  s += __builtin_amdgcn_update_dpp(0, s, 0x4E, 0xf, 0xf, false);
  s += __builtin_amdgcn_update_dpp(0, s, 0x141, 0xf, 0xf, false);
  sum = s;
  // low bytes of q0..q3 -> bytes 0..3 (selector 0x0c reads as zero)
  return static_cast<int>(__builtin_amdgcn_perm(q1, q0, 0x0c0c0400u) | __builtin_amdgcn_perm(q3, q2, 0x04000c0cu));
}

// The same quantization by a group of 4 lanes (a DPP quad): lane g holds
// elements 8g..8g+7 of the block in a (8g..8g+3) and b (8g+4..8g+7), so the
// per-block work (max, scale, reciprocal) is shared by 8 elements per lane
// instead of 4.  Returns the 8 codes of the lane as two dwords (element
// order); `scale` as act_quant_group8.
__device__ __forceinline__ uint2 act_quant_group4(float4 a, float4 b, bool per_row, float row_scale,
                                                  float &scale) {
  const float ma = fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w)));
  const float mb4 = fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w)));
  uint32_t mb = __builtin_bit_cast(uint32_t, fmaxf(fmaxf(ma, mb4), 0.0f));  // never NaN, see act_quant_group8
  mb = max(mb, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mb), 0xB1, 0xf, 0xf, false)));
  mb = max(mb, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mb), 0x4E, 0xf, 0xf, false)));
  const float amax = __builtin_bit_cast(float, mb);
  scale = per_row ? row_scale : div127_rn(amax);
  const float inv = scale == 0.0f ? 0.0f : recip_rn(scale);
  const float inv2 = 2.0f * inv;
  int q[8];
  const float e[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  if (inv2 <= 0x1.fffffep127f) {  // uniform per group; false only for scale < 2^-127
#pragma unroll
    for (int i = 0; i < 8; i++) q[i] = quant_code(e[i], inv2);
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) q[i] = quant_code_ref(e[i], inv);
  }
  return make_uint2(__builtin_amdgcn_perm(q[1], q[0], 0x0c0c0400u) | __builtin_amdgcn_perm(q[3], q[2], 0x04000c0cu),
                    __builtin_amdgcn_perm(q[5], q[4], 0x0c0c0400u) | __builtin_amdgcn_perm(q[7], q[6], 0x04000c0cu));
}

// silu(g) * u in f32 (crates/llm-cpu/src/ops.rs:27-36 silu, then the gate
// multiply, crates/llm-engine/src/lfm2.rs:902-905) -- one definition, so every
// kernel that forms h rounds it identically.
__device__ __forceinline__ float silu_mul1(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

// ---- rms_norm scale ------------------------------------------------------------
// scale = f32(1 / sqrt(sumsq * inv_dim + eps)) with the reference's roundings
// (crates/llm-cpu/src/ops.rs:12-17: f64 multiply, f64 add, f64 sqrt, f64
// reciprocal, then `as f32`).  The multiply and add are rounded separately
// (no contraction into an FMA).  1/sqrt(v) comes from v_rsq_f64 refined by
// two Newton steps: r lies within a few f64 ulp of the true value, as does the
// reference's RN64(1 / RN64(sqrt v)), so both round to the same f32 unless an
// f32 rounding boundary lies within 2^-40 of r (relative); then, and for v
// outside [2^-1000, 2^1000], the IEEE sqrt and division decide, on a real
// (wave-uniform) branch.
__device__ __forceinline__ float rms_scale(double sumsq, double inv_dim, float eps) {
  const double v = __dadd_rn(__dmul_rn(sumsq, inv_dim), static_cast<double>(eps));
  if (v > 0x1p-1000 && v < 0x1p1000) {
    double y = __builtin_amdgcn_rsq(v);
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const double e = __builtin_fma(-v, y * y, 1.0);
      y = __builtin_fma(0.5 * y, e, y);
    }
    const float f = static_cast<float>(y);
    const uint32_t fb = __builtin_bit_cast(uint32_t, f);
    const double fd = f;
    const double up = 0.5 * (fd + static_cast<double>(__builtin_bit_cast(float, fb + 1u)));
    const double dn = 0.5 * (fd + static_cast<double>(__builtin_bit_cast(float, fb - 1u)));
    const double tol = y * 0x1p-40;
    if (fb > 1u && fb < 0x7F7FFFFFu && __builtin_fabs(y - up) > tol && __builtin_fabs(y - dn) > tol) return f;
  }
  double t = v;
  asm volatile("" : "+v"(t));  // keep the exact path behind the branch
  return static_cast<float>(1.0 / __builtin_sqrt(t));
}

// rms_norm of the x a GEMV-style workgroup holds in registers (thread t holds
// float4s t + THREADS j; elements past k are 0 in x and in nw): the squares
// summed in f64 (per thread, DPP tree per wave, then the wave sums in order),
// scale = rms_scale(), then x = nw * (x * scale) in f32 (ops.rs:8-23).  All
// threads must call it; it contains a workgroup barrier.
template <int THREADS, int XJ>
__device__ __forceinline__ void rms_norm_regs(float4 (&xv)[XJ], const float4 (&nv)[XJ], double inv_k, float eps,
                                              double *s_ss) {
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
  if ((threadIdx.x & (kWave - 1)) == 0) s_ss[threadIdx.x / kWave] = ss;
  __syncthreads();
  double tot = 0.0;
#pragma unroll
  for (int i = 0; i < THREADS / kWave; i++) tot += s_ss[i];
  const float scale = rms_scale(tot, inv_k, eps);
#pragma unroll
  for (int j = 0; j < XJ; j++) {
    xv[j].x = nv[j].x * (xv[j].x * scale);
    xv[j].y = nv[j].y * (xv[j].y * scale);
    xv[j].z = nv[j].z * (xv[j].z * scale);
    xv[j].w = nv[j].w * (xv[j].w * scale);
  }
}

// ---- x -> LDS codes, shared by the GEMV-style kernels --------------------
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

// x -> LDS codes with 4-lane groups: thread t holds the 32-byte chunks
// t + THREADS j of x (float4s 2c and 2c + 1 of chunk c in xv[2j], xv[2j+1]),
// so quad t / 4 + (THREADS / 4) j holds one block.  All threads must call it;
// it ends with a barrier.
template <int THREADS, int XP>
__device__ __forceinline__ void quantize_pairs_to_lds(const float4 (&xv)[2 * XP], int nblk, int per_row,
                                                      int8_t *s_qs, float *s_sa, float *s_red) {
  const float rs = row_scale_of<THREADS, 2 * XP>(xv, per_row, s_red);
  const int tid = threadIdx.x;
  const int g = tid & 3;
#pragma unroll
  for (int j = 0; j < XP; j++) {
    const int b = (tid >> 2) + j * (THREADS / 4);
    if (b < nblk) {  // uniform across each quad
      float scale;
      const uint2 q = act_quant_group4(xv[2 * j], xv[2 * j + 1], per_row != 0, rs, scale);
      *reinterpret_cast<uint2 *>(s_qs + b * 32 + g * 8) = q;
      if (g == 0) s_sa[b] = scale;
    }
  }
  __syncthreads();
}

// The caller's accumulation mode applied to one output: Assign, AddF64
// (gemv_q4.rs:486-497) or the f32 residual add (ops.rs:48-53 add_inplace
// after an Assign).
__device__ __forceinline__ float apply_mode(float old, float v, int mode) {
  if (mode == LGH_ADD_F64) return static_cast<float>(static_cast<double>(old) + static_cast<double>(v));
  if (mode == LGH_ADD_F32) return old + v;
  return v;
}

__device__ __forceinline__ void store_row(float *y, int row, float acc16, int mode) {
  const float v = acc16 * 0.0625f;  // exact: undo the x16 of the nibble unpack
  y[row] = mode == LGH_ASSIGN ? v : apply_mode(y[row], v, mode);
}

// store_row with the old y[row] read earlier by the same lane.
__device__ __forceinline__ void store_row_old(float *y, int row, float acc16, int mode, float y_old) {
  const float v = acc16 * 0.0625f;
  y[row] = mode == LGH_ASSIGN ? v : apply_mode(y_old, v, mode);
}

// ---- MX-fp6 operand codes ----------------------------------------------------
// The GEMM feeds integer operands to the fp6 matrix cores as OCP MX FP6 E3M2
// codes (1 sign, 3 exponent bits with bias 3, 2 mantissa bits).  Every
// integer in [-8, 8] is exact in E3M2, so a Q4 weight (-8..7) is one code and
// an int8 activation q (-127..127) is two: q = 16 h + l with
// h = (q + 8) >> 4 in [-8, 8] and l = q - 16 h in [-8, 7].
// An MFMA operand row holds 32 codes packed densely, code t in bits
// [6t, 6t + 6) of six dwords.  Stored as two planes per 32-row tile:
// plane0 = dwords 0-3 (16 B per row), plane1 = dwords 4-5 (8 B per row).
__device__ __forceinline__ uint32_t e3m2_code(int v) {
  const uint32_t a = static_cast<uint32_t>(v < 0 ? -v : v);
  const int e = 31 - __builtin_clz(a | 1u);  // floor(log2 a) for a >= 1
  const uint32_t mag = ((static_cast<uint32_t>(e) + 3u) << 2) | (((a << 2) >> e) & 3u);
  return a == 0 ? 0u : ((v < 0 ? 0x20u : 0u) | mag);
}

__device__ __forceinline__ void split_h_l(int q, int &h, int &l) {
  h = (q + 8) >> 4;  // arithmetic shift: floor((q + 8) / 16)
  l = q - 16 * h;
}

// Dense packing across the 8 lanes of a 32-element block (lane g holds 4
// codes = 24 bits v_g): the 6 dwords of the block are, per quad of lanes,
// dword 3q + r = (v_r >> 8r) | (v_{r+1} << (24 - 8r)) for r = 0, 1, 2.
// Returns that dword in lanes with r < 3 (lane r of each quad); lane 3's
// return value is meaningless.  quad_perm [1,2,3,3] fetches v_{r+1}.
__device__ __forceinline__ uint32_t pack24_group8(uint32_t v) {
  const uint32_t nxt =
      static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xF9, 0xf, 0xf, false));
  const int r = threadIdx.x & 3;
  return (v >> (8 * r)) | (nxt << (24 - 8 * r));
}

// Four int8 codes (packed bytes) -> 24-bit E3M2 streams of their h and l parts.
__device__ __forceinline__ void codes24_hl(int q4packed, uint32_t &vh, uint32_t &vl) {
  vh = 0;
  vl = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    int h, l;
    split_h_l(static_cast<int8_t>(q4packed >> (8 * i)), h, l);
    vh |= e3m2_code(h) << (6 * i);
    vl |= e3m2_code(l) << (6 * i);
  }
}

// Byte offset of dword d (0..5) of operand row `row` within a 768-byte
// (plane0 | plane1) tile image.
__device__ __forceinline__ uint32_t mx_dword_off(int row, int d) {
  return d < 4 ? static_cast<uint32_t>(row * 16 + d * 4) : static_cast<uint32_t>(512 + row * 8 + (d - 4) * 4);
}

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

// One MFMA operand row (6 dwords): 16 bytes of plane0 at p16, 8 bytes of
// plane1 at p8.
__device__ __forceinline__ v8i mx_operand(const char *p16, const char *p8) {
  const uint4 p0 = *reinterpret_cast<const uint4 *>(p16);
  const uint2 p1 = *reinterpret_cast<const uint2 *>(p8);
  v8i r;
  r[0] = static_cast<int>(p0.x);
  r[1] = static_cast<int>(p0.y);
  r[2] = static_cast<int>(p0.z);
  r[3] = static_cast<int>(p0.w);
  r[4] = static_cast<int>(p1.x);
  r[5] = static_cast<int>(p1.y);
  r[6] = 0;
  r[7] = 0;
  return r;
}

// Row `row` of a 768-byte tile image (LDS or global): plane0 at tile + row * 16,
// plane1 at tile + 512 + row * 8.
__device__ __forceinline__ v8i mx_row(const char *tile, int row) {
  return mx_operand(tile + row * 16, tile + 512 + row * 8);
}

// The same value, opaque to the optimizer (no instruction): addresses built
// from it are not merged with addresses built from the original.
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Exact integer block dots of a 32 (weight rows) x 32 (tokens) tile for one
// 32-element block, as f32: D[i][j] = sum_k w[i][k] * q[j][k].
// A = [w | w] (K = 64, lanes 0-31 and 32-63 hold the same weight row), B =
// [h | l] (lanes 0-31 hold token j's h codes, lanes 32-63 its l codes) with
// E8M0 scale 2^4 on the h half: sum_k w*(16h) + sum_k w*l = sum_k w*q.
// Products and partial sums are integers below 2^24, so D is exact.
// Output layout: lane L, element v -> j = L % 32, i = 8*(v/4) + 4*(L/32) + v%4.
__device__ __forceinline__ v16f mx_block_dot(v8i a, v8i b) {
  const v16f zero = {};
  const int scale_b = (threadIdx.x & 32) ? 127 : 131;  // 2^0 on l, 2^4 on h
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, zero, 3, 3, 0, 127, 0, scale_b);
}

}  // namespace lgh
