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
// h = silu(g) * u elementwise on a float4 (the op sequence's silu_mul_kernel
// arithmetic, so an image built from g and u equals one built from h).
__device__ __forceinline__ float4 silu_mul4(float4 g, float4 u) {
  return make_float4(silu_mul1(g.x, u.x), silu_mul1(g.y, u.y), silu_mul1(g.z, u.z), silu_mul1(g.w, u.w));
}

// The elementwise prologue of an image kernel on float4 f of x: h = silu(x) *
// u when u is set (uniform branch).  The norm has a kernel of its own
// (norm_image_kernel).
__device__ __forceinline__ void apply_prologue(const ActPrologue &pro, size_t f, float4 &v) {
  if (pro.u) v = silu_mul4(v, reinterpret_cast<const float4 *>(pro.u)[f]);
}

// Row amax / 127 of x, or (u not null) of silu(x) * u.
__global__ __launch_bounds__(kThreads) void row_amax_kernel(const float *__restrict__ x, const float *__restrict__ u,
                                                            int k, float *row_scale) {
  __shared__ float s_red[kWaves];
  const float4 *x4 = reinterpret_cast<const float4 *>(x + static_cast<size_t>(blockIdx.x) * k);
  const float4 *u4 = u ? reinterpret_cast<const float4 *>(u + static_cast<size_t>(blockIdx.x) * k) : nullptr;
  float m = 0.0f;
  for (int i = threadIdx.x; i < k / 4; i += kThreads) {
    float4 v = x4[i];
    if (u4) v = silu_mul4(v, u4[i]);
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

// ---- GEMM operand images ---------------------------------------------------
// Weights: one thread per (tile t, pair p, block slot s, row r).  Element e of
// a repacked nibble block sits in dword e/8, byte e%4, high nibble iff e%8 >= 4.
__global__ void q4_mx_pack_kernel(const uint8_t *__restrict__ qs, const uint16_t *__restrict__ sc, int n,
                                  int bpr, int nt, int pp, uint8_t *mx) {
  const size_t id = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (id >= static_cast<size_t>(nt) * pp * 64) return;
  const int r = static_cast<int>(id & 31), s = static_cast<int>((id >> 5) & 1);
  const size_t rec = id >> 6;  // t * pp + p
  const int t = static_cast<int>(rec / pp), p = static_cast<int>(rec % pp);
  const int row = t * 32 + r, b = 2 * p + s;
  uint32_t d[6] = {0, 0, 0, 0, 0, 0};
  float scale = 0.0f;
  if (row < n && b < bpr) {
    const size_t blk = static_cast<size_t>(row) * bpr + b;
    const uint4 w = reinterpret_cast<const uint4 *>(qs)[blk];
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 32; e++) {
      const uint32_t byte = (wd[e >> 3] >> (8 * (e & 3))) & 0xFFu;
      const uint32_t nib = (e & 4) ? (byte >> 4) : (byte & 0xFu);
      const int v = static_cast<int>(nib ^ 8u) - 8;  // sign-extend 4 bits
      const uint32_t code = e3m2_code(v);
      const int bit = 6 * e;
      d[bit >> 5] |= code << (bit & 31);
      if ((bit & 31) > 26) d[(bit >> 5) + 1] |= code >> (32 - (bit & 31));
    }
    scale = h2f(sc[blk]);
  }
  uint8_t *tile = mx + rec * kMxWRec + s * kMxTile;
  *reinterpret_cast<uint4 *>(tile + r * 16) = make_uint4(d[0], d[1], d[2], d[3]);
  *reinterpret_cast<uint2 *>(tile + 512 + r * 8) = make_uint2(d[4], d[5]);
  reinterpret_cast<float *>(mx + rec * kMxWRec + 2 * kMxTile)[s * 32 + r] = scale;
}

// Store the h and l code dwords of one (token, block) group: dword 3*quad + r
// of the block comes from lane r < 3 of each quad (pack24_group8).
__device__ __forceinline__ void store_hl_group8(uint8_t *rec, int s, int tok, uint32_t vh, uint32_t vl) {
  const uint32_t dh = pack24_group8(vh);
  const uint32_t dl = pack24_group8(vl);
  const int g = threadIdx.x & 7, r = g & 3;
  if (r < 3) {
    const uint32_t off = mx_dword_off(tok, 3 * (g >> 2) + r);
    *reinterpret_cast<uint32_t *>(rec + (2 * s) * kMxTile + off) = dh;
    *reinterpret_cast<uint32_t *>(rec + (2 * s + 1) * kMxTile + off) = dl;
  }
}

// The h / l E3M2 codes of every int8 code q, indexed by q + 128:
// code(h) | code(l) << 6, read from this table into LDS by each workgroup
// (a lookup in place of ~25 VALU per code).
struct HlTable {
  uint16_t v[256];
};
constexpr uint16_t e3m2_const(int v) {
  int a = v < 0 ? -v : v, e = 0;
  while ((2 << e) <= a) e++;
  return static_cast<uint16_t>(a == 0 ? 0 : ((v < 0 ? 0x20 : 0) | ((e + 3) << 2) | (((a << 2) >> e) & 3)));
}
constexpr HlTable make_hl_table() {
  HlTable t{};
  for (int i = 0; i < 256; i++) {
    const int q = i - 128, h = (q + 8) >> 4, l = q - 16 * h;  // split_h_l
    t.v[i] = static_cast<uint16_t>(e3m2_const(h) | (e3m2_const(l) << 6));
  }
  return t;
}
__constant__ HlTable kHlTable = make_hl_table();

// Activations -> the GEMM's operand image, one record (r = token tile * pp +
// block pair: 32 tokens x 2 blocks) per workgroup.  The 64 four-lane groups
// each quantize one (token, block): group G = tid / 4 takes token G % 32 of
// the tile and block G / 32 of the pair, lane g = tid % 4 elements 8g..8g+7
// (two float4s; act_quant_group4 shares the block's max, scale and
// reciprocal among 8 elements per lane).  Lane g's 8 codes are bits [48g,
// 48g + 48) of the block's 192-bit h and l streams.  The record is assembled
// in LDS and written with 16-byte stores, so every line of the image is
// written whole by one workgroup.  Against one half-record per workgroup
// with 8-lane groups and the table computed per workgroup (same image, bit
// for bit; kernel trace): M=512, K=10752 7.96 -> 7.44 us, M=2048, K=10752
// 25.0 -> 19.7 us, M=512, K=2048 unchanged (5.2 us); whole GEMM calls
// 1.3-3.8% faster (interleaved A/B).
__global__ __launch_bounds__(kThreads) void act_quant_mx_kernel(const float *__restrict__ x, ActPrologue pro, int m,
                                                                int bpr, int pp, int per_row, const float *row_scale,
                                                                uint32_t recs, uint8_t *mxa) {
  __shared__ uint16_t s_hl[256];
  __shared__ __align__(16) uint8_t s_rec[kMxARec];
  static_assert(kThreads == 256, "one table entry per thread, 64 groups = 32 tokens x 2 blocks");
  const int tid = threadIdx.x, g = tid & 3, grp = tid >> 2, i = grp & 31, s = grp >> 5;
  const uint32_t r = blockIdx.x;
  const int t = static_cast<int>(r / static_cast<uint32_t>(pp)) * 32 + i;
  const int blk = 2 * static_cast<int>(r % static_cast<uint32_t>(pp)) + s;
  const bool ok = r < recs && t < m && blk < bpr;
  float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), b = a;
  if (ok) {
    const size_t f = (static_cast<size_t>(t) * bpr + blk) * 8 + 2 * g;
    const float4 *src = reinterpret_cast<const float4 *>(x) + f;
    a = src[0];
    b = src[1];
    apply_prologue(pro, f, a);
    apply_prologue(pro, f + 1, b);
  }
  s_hl[tid] = kHlTable.v[tid];
  __syncthreads();  // the table
  const bool pr = ok && per_row;
  const float rs = pr ? row_scale[t] : 0.0f;
  float scale;
  const uint2 q = act_quant_group4(a, b, pr, rs, scale);
  // The 48-bit h and l streams of the lane's 8 codes (code e at bit 6e).
  uint32_t hlo = 0, hhi = 0, llo = 0, lhi = 0;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const uint32_t byte = ((e < 4 ? q.x : q.y) >> (8 * (e & 3))) & 0xFFu;
    const uint32_t hl = s_hl[byte ^ 0x80u];
    const uint32_t ch = hl & 63u, cl = hl >> 6;
    const int bit = 6 * e;
    if (bit < 32) {
      hlo |= ch << bit;
      llo |= cl << bit;
    }
    if (bit + 6 > 32) {  // code 5 straddles the two words
      hhi |= bit >= 32 ? ch << (bit - 32) : ch >> (32 - bit);
      lhi |= bit >= 32 ? cl << (bit - 32) : cl >> (32 - bit);
    }
  }
  // Dwords of the block's operand row: lane 0 -> 0, 1; lane 1 -> 2; lane 2
  // -> 3, 4; lane 3 -> 5 (quad_perm [1,2,3,3] fetches lane g + 1's low word).
  const uint32_t nh = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(hlo), 0xF9, 0xf, 0xf, false));
  const uint32_t nl = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(llo), 0xF9, 0xf, 0xf, false));
  uint8_t *th = s_rec + (2 * s) * kMxTile, *tl = th + kMxTile;
  if ((g & 1) == 0) {
    const int d = 3 * (g >> 1);
    *reinterpret_cast<uint32_t *>(th + mx_dword_off(i, d)) = hlo;
    *reinterpret_cast<uint32_t *>(tl + mx_dword_off(i, d)) = llo;
    *reinterpret_cast<uint32_t *>(th + mx_dword_off(i, d + 1)) = hhi | (nh << 16);
    *reinterpret_cast<uint32_t *>(tl + mx_dword_off(i, d + 1)) = lhi | (nl << 16);
  } else {
    const int d = 3 * (g >> 1) + 2;
    *reinterpret_cast<uint32_t *>(th + mx_dword_off(i, d)) = (hlo >> 16) | (hhi << 16);
    *reinterpret_cast<uint32_t *>(tl + mx_dword_off(i, d)) = (llo >> 16) | (lhi << 16);
  }
  if (g == 0) reinterpret_cast<float *>(s_rec + 4 * kMxTile)[s * 32 + i] = ok ? scale : 0.0f;
  __syncthreads();
  constexpr int kChunks = static_cast<int>(kMxARec / 16);  // 208 16-byte chunks
  if (tid < kChunks && r < recs)
    reinterpret_cast<uint4 *>(mxa + static_cast<size_t>(r) * kMxARec)[tid] = reinterpret_cast<const uint4 *>(s_rec)[tid];
}

__global__ __launch_bounds__(kThreads) void act_split_mx_kernel(const int8_t *__restrict__ aq,
                                                                const float *__restrict__ as, int m, int bpr,
                                                                int pp, size_t groups, uint8_t *mxa) {
  const size_t gi = (static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x) >> 3;
  if (gi >= groups) return;
  const int g = threadIdx.x & 7;
  const int t = static_cast<int>(gi / (2 * pp)), b = static_cast<int>(gi % (2 * pp));
  int q = 0;
  if (t < m && b < bpr) q = reinterpret_cast<const int *>(aq)[(static_cast<size_t>(t) * bpr + b) * 8 + g];
  uint32_t vh, vl;
  codes24_hl(q, vh, vl);
  uint8_t *rec = mxa + (static_cast<size_t>(t >> 5) * pp + (b >> 1)) * kMxARec;
  store_hl_group8(rec, b & 1, t & 31, vh, vl);
  if (g == 0) {
    const float sa = (as && t < m && b < bpr) ? as[static_cast<size_t>(t) * bpr + b] : 0.0f;
    reinterpret_cast<float *>(rec + 4 * kMxTile)[(b & 1) * 32 + (t & 31)] = sa;
  }
}

// Activations for the matrix-core batch GEMV, in its MFMA register layouts
// (lgh_internal.h): one 8-lane group per (token, block) over the padded
// ranges [0, 16*mt) x [0, 4*pq); padding gets code 0 and scale 0.
__global__ __launch_bounds__(kThreads) void act_quant_mma_kernel(const float *__restrict__ x, ActPrologue pro, int m,
                                                                 int bpr, int pq, int per_row, const float *row_scale,
                                                                 size_t groups, uint8_t *codes, float *scales) {
  const size_t gi = (static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x) >> 3;
  if (gi >= groups) return;  // whole 8-lane groups exit together
  const int g8 = threadIdx.x & 7;
  const int t = static_cast<int>(gi / (4 * pq)), b = static_cast<int>(gi % (4 * pq));
  const bool ok = t < m && b < bpr;
  float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (ok) {
    const size_t f = (static_cast<size_t>(t) * bpr + b) * 8 + g8;
    v = reinterpret_cast<const float4 *>(x)[f];
    apply_prologue(pro, f, v);
  }
  const bool pr = ok && per_row;
  const float rs = pr ? row_scale[t] : 0.0f;
  float scale;
  int sum;
  const int q = act_quant_group8(v, pr, rs, scale, sum);
  // Codes 4 g8 .. 4 g8 + 3 of block b: lane (t % 16) + 16 (g8 / 2) of the
  // block pair b / 2, bytes 8 (b % 2) + 4 (g8 % 2).
  const size_t pair = static_cast<size_t>(t >> 4) * (2 * pq) + (b >> 1);
  const int lane = (t & 15) + 16 * (g8 >> 1);
  *reinterpret_cast<int *>(codes + (pair * 64 + lane) * 16 + (b & 1) * 8 + (g8 & 1) * 4) = q;
  if (g8 == 0) scales[((static_cast<size_t>(t >> 4) * pq + (b >> 2)) * 16 + (t & 15)) * 4 + (b & 3)] = ok ? scale : 0.0f;
}

// The same image from ActQ8 codes and block scales already computed (the
// prepared-activation GEMV of a matrix without a GEMM image).
__global__ __launch_bounds__(kThreads) void act_codes_mma_kernel(const int8_t *__restrict__ aq,
                                                                 const float *__restrict__ as, int m, int bpr,
                                                                 int pq, size_t groups, uint8_t *codes,
                                                                 float *scales) {
  const size_t gi = (static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x) >> 3;
  if (gi >= groups) return;
  const int g8 = threadIdx.x & 7;
  const int t = static_cast<int>(gi / (4 * pq)), b = static_cast<int>(gi % (4 * pq));
  const bool ok = t < m && b < bpr;
  const size_t blk = static_cast<size_t>(t) * bpr + b;
  const int q = ok ? reinterpret_cast<const int *>(aq)[blk * 8 + g8] : 0;
  const size_t pair = static_cast<size_t>(t >> 4) * (2 * pq) + (b >> 1);
  const int lane = (t & 15) + 16 * (g8 >> 1);
  *reinterpret_cast<int *>(codes + (pair * 64 + lane) * 16 + (b & 1) * 8 + (g8 & 1) * 4) = q;
  if (g8 == 0) scales[((static_cast<size_t>(t >> 4) * pq + (b >> 2)) * 16 + (t & 15)) * 4 + (b & 3)] = ok ? as[blk] : 0.0f;
}

// ---- rms_norm in the activation images ---------------------------------------
// rms_norm (ops.rs:8-23) and an activation image in one launch, one
// workgroup per token row of the padded token range.  The sum of squares is
// formed exactly as rms_norm_kernel forms it (thread i adds the f64 squares
// of elements i, i + 256, ... in turn; DPP wave trees; the 4 wave sums in
// order), so the scale and every normed value nw * (x * scale) equal the op
// sequence's bit for bit.  The normed row is then quantized by 8-lane groups
// (act_quant_group8: the codes and scales of the image kernels' quantizers)
// and written to the row's places in the image: the GEMM's operand records
// (MX, 32-token tiles) or the matrix-core batch layout (16-token tiles).
// Rows past m and blocks past bpr get code 0 and scale 0, as the image
// kernels write them.  Workgroups are dealt round robin to the 8 XCDs, so
// workgroup b takes token (b / 8) % TT of tile 8 (b / (8 TT)) + b % 8: the
// rows of one tile, which share the image's cache lines, are written through
// one XCD's L2.
template <bool MX>
__global__ __launch_bounds__(kThreads) void norm_image_kernel(const float *__restrict__ x,
                                                              const float *__restrict__ nw, double inv_k, float eps,
                                                              int m, int bpr, int nblk, int mt, int per_row,
                                                              uint8_t *__restrict__ img, float *__restrict__ scales) {
  constexpr int TT = MX ? 32 : 16;
  constexpr int kRound = kThreads / 8;  // blocks per round of 8-lane groups
  constexpr int kPre = 4;               // rounds whose loads are in flight together
  const int wg = static_cast<int>(blockIdx.x);
  const int tile = 8 * (wg / (8 * TT)) + (wg & 7);
  if (tile >= mt) return;  // whole workgroups
  const int t = tile * TT + (wg >> 3) % TT;
  const bool live = t < m;  // uniform
  const int k = bpr * 32;
  const uint32_t row_bytes = static_cast<uint32_t>(k) * 4u;
  // Rows past m read as zeros (a resource of size 0) and are stored as zeros.
  const auto xr = make_rsrc(x + static_cast<size_t>(live ? t : 0) * k, live ? row_bytes : 0u);
  const auto nr = make_rsrc(nw, row_bytes);
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int g8 = tid & 7, grp = tid >> 3;
  // The first rounds' float4s of x and nw (blocks past bpr read 0), requested
  // before the sum of squares so they arrive while it is formed.
  float4 xa[kPre], wa[kPre];
  auto load_rounds = [&](int b0) {
#pragma unroll
    for (int u = 0; u < kPre; u++) {
      const uint32_t off = static_cast<uint32_t>((b0 + kRound * u + grp) * 8 + g8) * 16u;
      xa[u] = buf_load_f4(xr, off);
      wa[u] = buf_load_f4(nr, off);
    }
  };
  load_rounds(0);
  // Thread i: the squares of elements i, i + 256, ... in order, 8 loads in
  // flight; elements past k read 0 and add +0.0, which changes no sum.
  double ss = 0.0;
  for (int i0 = 0; i0 < k; i0 += kThreads * 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) v[u] = buf_load_f32(xr, static_cast<uint32_t>(i0 + tid + kThreads * u) * 4u);
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const double d = v[u];
      ss += d * d;
    }
  }
  __shared__ double s_ss[kWaves];
  __shared__ float s_mx[kWaves];
  ss = wave_sum_dpp64(ss);
  if (lane == 0) s_ss[wave] = ss;
  __syncthreads();
  double tot = 0.0;
#pragma unroll
  for (int i = 0; i < kWaves; i++) tot += s_ss[i];
  const float scale = rms_scale(tot, inv_k, eps);
  float rs = 0.0f;
  if (per_row) {  // amax(nw * (x * scale)) / 127, as row_amax_kernel over the normed rows
    float mx = 0.0f;
    for (int f = tid; f < k / 4; f += kThreads) {
      const float4 a = buf_load_f4(xr, static_cast<uint32_t>(f) * 16u);
      const float4 w = buf_load_f4(nr, static_cast<uint32_t>(f) * 16u);
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(w.x * (a.x * scale)), fabsf(w.y * (a.y * scale))),
                           fmaxf(fabsf(w.z * (a.z * scale)), fabsf(w.w * (a.w * scale)))));
    }
    mx = wave_max(mx);
    if (lane == 0) s_mx[wave] = mx;
    __syncthreads();
    rs = div127_rn(fmaxf(fmaxf(s_mx[0], s_mx[1]), fmaxf(s_mx[2], s_mx[3])));
  }
  for (int b0 = 0; b0 < nblk; b0 += kRound * kPre) {
    if (b0 > 0) load_rounds(b0);
#pragma unroll
    for (int u = 0; u < kPre; u++) {
      const int blk = b0 + kRound * u + grp;
      const bool ok = live && blk < bpr;
      const float4 a = xa[u], w = wa[u];
      const float4 v = ok ? make_float4(w.x * (a.x * scale), w.y * (a.y * scale), w.z * (a.z * scale),
                                        w.w * (a.w * scale))
                          : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      float sc;
      int sum;
      const int q = act_quant_group8(v, ok && per_row, rs, sc, sum);
      if (blk >= nblk) continue;  // whole 8-lane groups
      if constexpr (MX) {
        uint32_t vh, vl;
        codes24_hl(q, vh, vl);
        uint8_t *rec = img + (static_cast<size_t>(tile) * (nblk / 2) + (blk >> 1)) * kMxARec;
        store_hl_group8(rec, blk & 1, t & 31, vh, vl);
        if (g8 == 0) reinterpret_cast<float *>(rec + 4 * kMxTile)[(blk & 1) * 32 + (t & 31)] = ok ? sc : 0.0f;
      } else {
        const int pq = nblk / 4;
        const size_t pair = static_cast<size_t>(tile) * (2 * pq) + (blk >> 1);
        const int ln = (t & 15) + 16 * (g8 >> 1);
        *reinterpret_cast<int *>(img + (pair * 64 + ln) * 16 + (blk & 1) * 8 + (g8 & 1) * 4) = q;
        if (g8 == 0)
          scales[((static_cast<size_t>(tile) * pq + (blk >> 2)) * 16 + (t & 15)) * 4 + (blk & 3)] = ok ? sc : 0.0f;
      }
    }
  }
}

template <bool MX>
hipError_t launch_norm_image(const float *x, const ActPrologue &pro, size_t m, size_t k, int per_row, int nblk,
                             uint8_t *img, float *scales, hipStream_t st) {
  constexpr size_t TT = MX ? 32 : 16;
  const size_t mt = (m + TT - 1) / TT;
  const size_t wgs = (mt + 7) / 8 * 8 * TT;
  hipLaunchKernelGGL(norm_image_kernel<MX>, dim3(static_cast<unsigned>(wgs)), dim3(kThreads), 0, st, x, pro.nw,
                     1.0 / static_cast<double>(k), pro.eps, static_cast<int>(m), static_cast<int>(k / 32), nblk,
                     static_cast<int>(mt), per_row, img, scales);
  return hipGetLastError();
}

inline unsigned blocks_for(size_t items, unsigned per) {
  return static_cast<unsigned>((items + per - 1) / per);
}

}  // namespace

hipError_t launch_q4_mx_pack(const lgh_q4 *w, hipStream_t st) {
  const size_t threads = w->nt * w->pp * 64;
  if (!threads) return hipSuccess;
  hipLaunchKernelGGL(q4_mx_pack_kernel, dim3(blocks_for(threads, 256)), dim3(256), 0, st, w->qs, w->sc,
                     static_cast<int>(w->n), static_cast<int>(w->bpr), static_cast<int>(w->nt),
                     static_cast<int>(w->pp), w->mx);
  return hipGetLastError();
}

// The PerRow scale an image kernel needs before it starts (row_amax_kernel
// over x or silu(x) * u).  scratch: m floats.
hipError_t row_stats(const float *x, const ActPrologue &pro, size_t m, size_t k, int per_row, float *scratch,
                     const float **row_scale, hipStream_t st) {
  *row_scale = per_row ? scratch : nullptr;
  if (!per_row) return hipSuccess;
  hipLaunchKernelGGL(row_amax_kernel, dim3(static_cast<unsigned>(m)), dim3(kThreads), 0, st, x, pro.u,
                     static_cast<int>(k), scratch);
  return hipGetLastError();
}

hipError_t launch_act_quant_mx(const float *x, ActPrologue pro, size_t m, size_t k, int per_row, uint8_t *mxa,
                               float *scratch, hipStream_t st) {
  const size_t bpr = k / 32, pp = (bpr + 1) / 2, mt = (m + 31) / 32;
  if (m == 0 || bpr == 0) return hipSuccess;
  if (pro.nw) return launch_norm_image<true>(x, pro, m, k, per_row, static_cast<int>(2 * pp), mxa, nullptr, st);
  const float *rs = nullptr;
  if (hipError_t e = row_stats(x, pro, m, k, per_row, scratch, &rs, st)) return e;
  const size_t recs = mt * pp;  // < 2^31: the image is below kMxMaxBytes
  hipLaunchKernelGGL(act_quant_mx_kernel, dim3(static_cast<unsigned>(recs)), dim3(kThreads), 0, st, x, pro,
                     static_cast<int>(m), static_cast<int>(bpr), static_cast<int>(pp), per_row, rs,
                     static_cast<uint32_t>(recs), mxa);
  return hipGetLastError();
}

hipError_t launch_act_quant_mma(const float *x, ActPrologue pro, size_t m, size_t k, int per_row, uint8_t *codes,
                                float *scales, float *scratch, hipStream_t st) {
  const size_t bpr = k / 32, pq = (bpr + 3) / 4, mt = (m + 15) / 16;
  if (m == 0 || bpr == 0) return hipSuccess;
  if (pro.nw) return launch_norm_image<false>(x, pro, m, k, per_row, static_cast<int>(4 * pq), codes, scales, st);
  const float *rs = nullptr;
  if (hipError_t e = row_stats(x, pro, m, k, per_row, scratch, &rs, st)) return e;
  const size_t groups = mt * 16 * pq * 4;
  hipLaunchKernelGGL(act_quant_mma_kernel, dim3(blocks_for(groups * 8, kThreads)), dim3(kThreads), 0, st, x, pro,
                     static_cast<int>(m), static_cast<int>(bpr), static_cast<int>(pq), per_row, rs, groups, codes,
                     scales);
  return hipGetLastError();
}

hipError_t launch_act_codes_mma(const int8_t *aq, const float *as, size_t m, size_t k, uint8_t *codes,
                                float *scales, hipStream_t st) {
  const size_t bpr = k / 32, pq = (bpr + 3) / 4, mt = (m + 15) / 16;
  if (m == 0 || bpr == 0) return hipSuccess;
  const size_t groups = mt * 16 * pq * 4;
  hipLaunchKernelGGL(act_codes_mma_kernel, dim3(blocks_for(groups * 8, kThreads)), dim3(kThreads), 0, st, aq, as,
                     static_cast<int>(m), static_cast<int>(bpr), static_cast<int>(pq), groups, codes, scales);
  return hipGetLastError();
}

hipError_t launch_act_split_mx(const int8_t *aq, const float *scales, size_t m, size_t k, uint8_t *mxa,
                               hipStream_t st) {
  const size_t bpr = k / 32, pp = (bpr + 1) / 2, mt = (m + 31) / 32;
  if (m == 0 || bpr == 0) return hipSuccess;
  const size_t groups = mt * 32 * pp * 2;
  hipLaunchKernelGGL(act_split_mx_kernel, dim3(blocks_for(groups * 8, kThreads)), dim3(kThreads), 0, st, aq,
                     scales, static_cast<int>(m), static_cast<int>(bpr), static_cast<int>(pp), groups, mxa);
  return hipGetLastError();
}

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
    hipLaunchKernelGGL(row_amax_kernel, dim3(static_cast<unsigned>(m)), dim3(kThreads), 0, st, x, nullptr,
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
