// Device helpers shared by the gfx950 kernels (wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

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

// ActQ8 quantization of one 32-element block by a group of 8 lanes
// (crates/llm-cpu/src/gemv_q4.rs:77-94).  Lane j of the group holds elements
// 4j..4j+3 in v.  Returns the packed int8 codes for those 4 elements; writes
// the block scale and the block sum of codes (valid in every group lane).
//   scale = amax / 127            (f32, correctly rounded)
//   inv   = scale == 0 ? 0 : 1/scale  (f32, correctly rounded)
//   q     = clamp(round_half_away_from_zero(v * inv), -127, 127)
// With per_row, `row_scale` (= row amax / 127) replaces the block scale.
__device__ __forceinline__ int act_quant_group8(float4 v, bool per_row, float row_scale, float &scale,
                                                int &sum) {
  float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
  amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
  amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
  scale = per_row ? row_scale : __fdiv_rn(amax, 127.0f);
  const float inv = scale == 0.0f ? 0.0f : __fdiv_rn(1.0f, scale);
  const int q0 = static_cast<int>(fminf(fmaxf(roundf(v.x * inv), -127.0f), 127.0f));
  const int q1 = static_cast<int>(fminf(fmaxf(roundf(v.y * inv), -127.0f), 127.0f));
  const int q2 = static_cast<int>(fminf(fmaxf(roundf(v.z * inv), -127.0f), 127.0f));
  const int q3 = static_cast<int>(fminf(fmaxf(roundf(v.w * inv), -127.0f), 127.0f));
  int s = q0 + q1 + q2 + q3;
  s += __shfl_xor(s, 1, 8);
  s += __shfl_xor(s, 2, 8);
  s += __shfl_xor(s, 4, 8);
  sum = s;
  return (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | (static_cast<int>(static_cast<uint32_t>(q3) << 24));
}

}  // namespace lgh
