// M > 1 kernels for gfx950: Q4 x int8 GEMM on v_mfma_i32_32x32x32_i8 with a
// per-32-block scale fold (replaces crates/llm-cpu/src/gemv_q4.rs:686-952 and
// the AMX tiles of crates/llm-cpu/src/amx.rs:329-518).
//
// One 32-element K block is exactly one MFMA K step, so each MFMA yields the
// exact integer block dots of a 32x32 (weight rows n) x (tokens m) tile --
// the analogue of amx.rs's tdpbssd + tilestored -- and the fold
//   acc[n][m] = fma(f32(16*c), sw[n,kb] * sa[m,kb], acc[n][m])
// is the analogue of fold_c (amx.rs:263-320).  A operand = unpacked weight
// nibbles (16 x value, see lgh_internal.h), B operand = quantized activations;
// the x16 is removed once at the store.
//
// Workgroup = 4 waves in a WN x WM grid; each wave owns TN x TM MFMA tiles.
// K is staged through LDS in chunks of KC blocks with a register prefetch of
// the next chunk.  LDS planes are [block q][half h][row][bytes] so every MFMA
// operand read is a contiguous, conflict-free ds_read.
#include "lgh_device.h"
#include "lgh_internal.h"

namespace lgh {

namespace {

constexpr int kThreads = 256;
constexpr int KC = 4;  // K blocks per LDS chunk

struct GemmArgs {
  const uint8_t *qs;   // weights: [n][bpr][16]
  const uint16_t *sc;  // [n][bpr]
  const int8_t *aq;    // activations: [m][k]
  const float *sa;     // [m][bpr]
  float *y;            // [m][n]
  int n, m, k, bpr, mode;
};

template <int WN, int WM, int TN, int TM>
struct Cfg {
  static constexpr int BN = WN * TN * 32;
  static constexpr int BM = WM * TM * 32;
  // LDS plane strides (bytes), padded by 16 so the 2*KC planes start on
  // different banks for the staging writes.
  static constexpr int W_PLANE = BN * 8 + 16;
  static constexpr int A_PLANE = BM * 16 + 16;
  static constexpr int W_BYTES = KC * 2 * W_PLANE;
  static constexpr int A_BYTES = KC * 2 * A_PLANE;
  static constexpr int SW_BYTES = KC * BN * 4;
  static constexpr int SA_BYTES = KC * BM * 4;
  static constexpr int LDS = W_BYTES + A_BYTES + SW_BYTES + SA_BYTES;
  // Per-thread staging counts.
  static constexpr int W_LD = (BN * KC + kThreads - 1) / kThreads;      // uint4 blocks
  static constexpr int A_LD = (BM * KC * 2 + kThreads - 1) / kThreads;  // uint4 halves
  static constexpr int SW_LD = (BN * KC + kThreads - 1) / kThreads;
  static constexpr int SA_LD = (BM * KC + kThreads - 1) / kThreads;
  static_assert(WN * WM * 64 == kThreads, "4 waves per workgroup");
};

template <class C>
struct Stage {
  uint4 w[C::W_LD];
  uint4 a[C::A_LD];
  uint16_t sw[C::SW_LD];  // f16 bits; converted when written to LDS
  float sa[C::SA_LD];
};

// Issue every global load of one K chunk, all branch-free raw buffer loads.
// The resources cover this workgroup's operand panels: rows beyond n / m fall
// outside them and load as 0; blocks beyond bpr get kOOB offsets.  They are
// rebuilt from scalars here (kernel arguments and blockIdx) so the compiler
// keeps them in SGPRs.
template <class C>
__device__ __forceinline__ void load_chunk(const GemmArgs &g, int n0, int m0, int kb0, Stage<C> &s) {
  const int tid = threadIdx.x;
  // readfirstlane: the clamps select to VALU med3, which would otherwise put
  // the resource sizes in VGPRs (and every load in a waterfall loop).
  const uint32_t rn = static_cast<uint32_t>(uniform(max(0, min(C::BN, g.n - n0))));
  const uint32_t rm = static_cast<uint32_t>(uniform(max(0, min(C::BM, g.m - m0))));
  const size_t wb = static_cast<size_t>(n0) * g.bpr, ab = static_cast<size_t>(m0);
  const auto pw = make_rsrc(g.qs + wb * 16, rn * g.bpr * 16u);
  const auto psw = make_rsrc(g.sc + wb, rn * g.bpr * 2u);
  const auto pa = make_rsrc(g.aq + ab * g.k, rm * static_cast<uint32_t>(g.k));
  const auto psa = make_rsrc(g.sa + ab * g.bpr, rm * g.bpr * 4u);
#pragma unroll
  for (int i = 0; i < C::W_LD; i++) {
    const int c = tid + i * kThreads;  // c -> (row, q): 4 threads cover a row's 64 B
    const int row = c / KC, kb = kb0 + c % KC;
    const bool ok = c < C::BN * KC && kb < g.bpr;
    s.w[i] = buf_load16<kAuxNT>(pw, ok ? static_cast<uint32_t>(row * g.bpr + kb) * 16u : kOOB);
  }
#pragma unroll
  for (int i = 0; i < C::SW_LD; i++) {
    const int c = tid + i * kThreads;
    const int row = c / KC, kb = kb0 + c % KC;
    const bool ok = c < C::BN * KC && kb < g.bpr;
    s.sw[i] = buf_load_u16(psw, ok ? static_cast<uint32_t>(row * g.bpr + kb) * 2u : kOOB);
  }
#pragma unroll
  for (int i = 0; i < C::A_LD; i++) {
    const int c = tid + i * kThreads;  // c -> (row, q, h): 8 threads cover a row's 128 B
    const int row = c / (KC * 2), qh = c % (KC * 2);
    const bool ok = c < C::BM * KC * 2 && kb0 + qh / 2 < g.bpr;
    s.a[i] = buf_load16(pa, ok ? static_cast<uint32_t>(row * g.k + kb0 * 32 + qh * 16) : kOOB);
  }
#pragma unroll
  for (int i = 0; i < C::SA_LD; i++) {
    const int c = tid + i * kThreads;
    const int row = c / KC, kb = kb0 + c % KC;
    const bool ok = c < C::BM * KC && kb < g.bpr;
    s.sa[i] = buf_load_f32(psa, ok ? static_cast<uint32_t>(row * g.bpr + kb) * 4u : kOOB);
  }
}

template <class C>
__device__ __forceinline__ void store_chunk(char *lds, const Stage<C> &s) {
  const int tid = threadIdx.x;
  char *s_w = lds;
  char *s_a = lds + C::W_BYTES;
  float *s_sw = reinterpret_cast<float *>(lds + C::W_BYTES + C::A_BYTES);
  float *s_sa = s_sw + KC * C::BN;
#pragma unroll
  for (int i = 0; i < C::W_LD; i++) {
    const int c = tid + i * kThreads;
    if (c < C::BN * KC) {
      const int row = c / KC, q = c % KC;
      *reinterpret_cast<uint2 *>(s_w + (2 * q) * C::W_PLANE + row * 8) = make_uint2(s.w[i].x, s.w[i].y);
      *reinterpret_cast<uint2 *>(s_w + (2 * q + 1) * C::W_PLANE + row * 8) = make_uint2(s.w[i].z, s.w[i].w);
    }
  }
#pragma unroll
  for (int i = 0; i < C::SW_LD; i++) {
    const int c = tid + i * kThreads;
    if (c < C::BN * KC) s_sw[(c % KC) * C::BN + c / KC] = h2f(s.sw[i]);
  }
#pragma unroll
  for (int i = 0; i < C::A_LD; i++) {
    const int c = tid + i * kThreads;
    if (c < C::BM * KC * 2) {
      const int row = c / (KC * 2), qh = c % (KC * 2);
      *reinterpret_cast<uint4 *>(s_a + qh * C::A_PLANE + row * 16) = s.a[i];
    }
  }
#pragma unroll
  for (int i = 0; i < C::SA_LD; i++) {
    const int c = tid + i * kThreads;
    if (c < C::BM * KC) s_sa[(c % KC) * C::BM + c / KC] = s.sa[i];
  }
}

template <int WN, int WM, int TN, int TM>
__global__ __launch_bounds__(kThreads) void q4_gemm_mfma_kernel(GemmArgs g) {
  using C = Cfg<WN, WM, TN, TM>;
  extern __shared__ __align__(16) char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wn = wave % WN, wm = wave / WN;
  const int col = lane & 31, h = lane >> 5;
  const int n0 = blockIdx.x * C::BN;
  const int m0 = blockIdx.y * C::BM;

  const char *s_w = lds;
  const char *s_a = lds + C::W_BYTES;
  const float *s_sw = reinterpret_cast<const float *>(lds + C::W_BYTES + C::A_BYTES);
  const float *s_sa = s_sw + KC * C::BN;

  float acc[TN][TM][16];
#pragma unroll
  for (int tn = 0; tn < TN; tn++)
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[tn][tm][v] = 0.0f;

  const int nchunks = (g.bpr + KC - 1) / KC;
  Stage<C> st;
  load_chunk<C>(g, n0, m0, 0, st);
  store_chunk<C>(lds, st);
  __syncthreads();

  for (int ch = 0; ch < nchunks; ch++) {
    if (ch + 1 < nchunks) load_chunk<C>(g, n0, m0, (ch + 1) * KC, st);
    // Not unrolled: unrolling lets the scheduler hoist all KC*TN*TM MFMAs and
    // keep their 16-register results live at once (register spills).
#pragma unroll 1
    for (int q = 0; q < KC; q++) {
      v4i A[TN], B[TM];
#pragma unroll
      for (int tn = 0; tn < TN; tn++) {
        const int nl = (wn * TN + tn) * 32 + col;
        A[tn] = unpack_half16(*reinterpret_cast<const uint2 *>(s_w + (2 * q + h) * C::W_PLANE + nl * 8));
      }
#pragma unroll
      for (int tm = 0; tm < TM; tm++) {
        const int ml = (wm * TM + tm) * 32 + col;
        B[tm] = *reinterpret_cast<const v4i *>(s_a + (2 * q + h) * C::A_PLANE + ml * 16);
      }
      float sa[TM];
#pragma unroll
      for (int tm = 0; tm < TM; tm++) sa[tm] = s_sa[q * C::BM + (wm * TM + tm) * 32 + col];
#pragma unroll
      for (int tn = 0; tn < TN; tn++) {
        float sw[16];
#pragma unroll
        for (int gq = 0; gq < 4; gq++) {
          const float4 f = *reinterpret_cast<const float4 *>(s_sw + q * C::BN + (wn * TN + tn) * 32 + 8 * gq + 4 * h);
          sw[4 * gq + 0] = f.x;
          sw[4 * gq + 1] = f.y;
          sw[4 * gq + 2] = f.z;
          sw[4 * gq + 3] = f.w;
        }
#pragma unroll
        for (int tm = 0; tm < TM; tm++) {
          const v16i zero = {};
          const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[tn], B[tm], zero, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 16; v++)
            acc[tn][tm][v] = fmaf(static_cast<float>(c[v]), sw[v] * sa[tm], acc[tn][tm][v]);
        }
      }
    }
    __syncthreads();
    if (ch + 1 < nchunks) {
      store_chunk<C>(lds, st);
      __syncthreads();
    }
  }

  // D[i][j] of a 32x32 MFMA tile: lane l, element v -> j = l % 32,
  // i = 8*(v/4) + 4*(l/32) + v%4.  Here i = weight row n, j = token m.
#pragma unroll
  for (int tn = 0; tn < TN; tn++)
#pragma unroll
    for (int tm = 0; tm < TM; tm++) {
      const int m = m0 + (wm * TM + tm) * 32 + col;
      if (m >= g.m) continue;
      float *yrow = g.y + static_cast<size_t>(m) * g.n;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int n = n0 + (wn * TN + tn) * 32 + 8 * (v / 4) + 4 * h + (v % 4);
        if (n < g.n) {
          const float val = acc[tn][tm][v] * 0.0625f;
          if (g.mode == LGH_ADD_F64)
            yrow[n] = static_cast<float>(static_cast<double>(yrow[n]) + static_cast<double>(val));
          else
            yrow[n] = val;
        }
      }
    }
}

// Integer block dots through the MFMA operand path: one wave per
// (32 weight rows, 32 tokens, block kb); out[m][n][kb] = c / 16.
__global__ __launch_bounds__(64) void q4_mfma_block_dots_kernel(const uint8_t *__restrict__ qs,
                                                                const int8_t *__restrict__ aq, int n,
                                                                int m, int k, int bpr, int32_t *out) {
  const int lane = threadIdx.x, col = lane & 31, h = lane >> 5;
  const int n0 = blockIdx.x * 32, m0 = blockIdx.y * 32, kb = blockIdx.z;
  const int nr = n0 + col, mr = m0 + col;
  uint2 w = make_uint2(0, 0);
  if (nr < n) w = *reinterpret_cast<const uint2 *>(qs + (static_cast<size_t>(nr) * bpr + kb) * 16 + 8 * h);
  v4i b = {0, 0, 0, 0};
  if (mr < m) b = *reinterpret_cast<const v4i *>(aq + static_cast<size_t>(mr) * k + kb * 32 + 16 * h);
  const v16i zero = {};
  const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(unpack_half16(w), b, zero, 0, 0, 0);
  for (int v = 0; v < 16; v++) {
    const int i = n0 + 8 * (v / 4) + 4 * h + (v % 4);
    const int j = m0 + col;
    if (i < n && j < m) out[(static_cast<size_t>(j) * n + i) * bpr + kb] = c[v] >> 4;
  }
}

template <int WN, int WM, int TN, int TM>
hipError_t launch_cfg(const GemmArgs &g, hipStream_t st) {
  using C = Cfg<WN, WM, TN, TM>;
  const dim3 grid((g.n + C::BN - 1) / C::BN, (g.m + C::BM - 1) / C::BM);
  hipLaunchKernelGGL((q4_gemm_mfma_kernel<WN, WM, TN, TM>), grid, dim3(kThreads), C::LDS, st, g);
  return hipGetLastError();
}

inline long tiles(long n, long m, int bn, int bm) { return ((n + bn - 1) / bn) * ((m + bm - 1) / bm); }

}  // namespace

hipError_t launch_q4_gemm(const lgh_q4 *w, const int8_t *aq, const float *sa, float *y, size_t m, int mode,
                          hipStream_t st) {
  GemmArgs g{w->qs, w->sc, aq, sa, y, static_cast<int>(w->n), static_cast<int>(m), static_cast<int>(w->k),
             static_cast<int>(w->bpr), mode};
  if (g.n == 0 || g.m == 0) return hipSuccess;
  if (m <= 32) return launch_cfg<4, 1, 1, 1>(g, st);  // 128 n x 32 m
  if (tiles(g.n, g.m, 128, 128) >= 240) return launch_cfg<2, 2, 2, 2>(g, st);
  return launch_cfg<2, 2, 1, 1>(g, st);  // 64 x 64
}

hipError_t launch_q4_mfma_block_dots(const lgh_q4 *w, const int8_t *aq, size_t m, int32_t *out,
                                     hipStream_t st) {
  if (w->n == 0 || m == 0 || w->bpr == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((w->n + 31) / 32), static_cast<unsigned>((m + 31) / 32),
                  static_cast<unsigned>(w->bpr));
  hipLaunchKernelGGL(q4_mfma_block_dots_kernel, grid, dim3(64), 0, st, w->qs, aq, static_cast<int>(w->n),
                     static_cast<int>(m), static_cast<int>(w->k), static_cast<int>(w->bpr), out);
  return hipGetLastError();
}

}  // namespace lgh
