// M > 1 kernels for gfx950: the Q4 x ActQ8 GEMM (replaces
// crates/llm-cpu/src/gemv_q4.rs:686-952 and the AMX tiles of
// crates/llm-cpu/src/amx.rs:329-518).
//
// Per 32-element block the reference computes the exact integer dot of a
// weight row and a token, then folds it in f32:
//   acc[n][m] = fma(f32(dot), sw[n,kb] * sa[m,kb], acc[n][m])   (gemv_q4.rs:930-936)
// On the matrix cores this becomes, for a 32 x 32 (rows x tokens) tile:
//   * the block dots: one scaled fp6 MFMA (mx_block_dot, lgh_device.h) whose
//     f32 result is the exact integer dot -- the analogue of tdpbssd +
//     tilestored (amx.rs:329-380), with no int->float conversion;
//   * the scale products sw[n] * sa[m] of two consecutive blocks: one f32
//     32x32x1_2b MFMA outer product, laid out exactly like the block dots
//     (block b in elements 16b..16b+15);
//   * the fold: one v_fma_f32 per element and block -- the only VALU work of
//     the inner loop (fold_c, amx.rs:263-320).
// (With int8 MFMA the fold costs a convert, a multiply and an FMA per
// element: three VALU ops per 32-deep MFMA result, which caps the GEMM near
// one sixth of the int8 matrix peak.  Here it is one.)
//
// Workgroup = 4 waves in a WN x WM grid, each owning TN x TM 32x32 tiles.
// K advances one block pair per stage.  A stage is the verbatim concatenation
// of NS weight records and MS activation records (lgh_internal.h), copied
// global -> LDS by buffer_load ... lds (DMA: no registers, no VALU) into one
// of NB LDS buffers; stages p+1 .. p+NB-1 are in flight while stage p is
// computed, one barrier per stage.
#include "lgh_device.h"
#include "lgh_internal.h"

namespace lgh {

namespace {

constexpr int kThreads = 256;
constexpr int kWRec = static_cast<int>(kMxWRec);
constexpr int kARec = static_cast<int>(kMxARec);
constexpr int kTile = static_cast<int>(kMxTile);
constexpr long kSplitTarget = 512;  // two workgroups per CU (M=512, K=10752, N=2048: 61.5 -> 48.6 us vs one)
constexpr size_t kSplitMinPairs = 64;  // K >= 4096
constexpr size_t kSplitPairs = 16;     // K >= 1024 per split
constexpr long kWideWgs = 640;  // 128 x 64 workgroup tiles from this many of them (2.5 per CU), no split K
constexpr long kKgTiles = 512;  // two K groups per workgroup below this many 128 x 32 tiles (no split K)
constexpr long kKg4Tiles = 256;  // four below this many
constexpr size_t kKgSplitPairs = 128;  // two K groups replace a split in two up to this many block pairs

struct GemmArgs {
  const uint8_t *wmx;  // weight operand image [nt][pp]
  const uint8_t *amx;  // activation operand image [mt][pp]
  float *y;            // [m][n]
  float *part;         // split-K partials [splits][m][n] (splits > 1)
  int n, m, nt, mt, pp, mode, vec4, splits;
  uint32_t w_bytes, a_bytes;
};

// Up to three matrices with the same k on the same activation image in one
// launch (the q / k / v or gate / up projections of one input): grid.x runs
// over the N tiles of matrix 0, then of matrix 1, then of matrix 2.
struct GemmMulti {
  GemmArgs g[3];
  int gx0, gx1;  // N-tile groups of matrices 0 and 1
};

template <int WN, int WM, int TN, int TM>
struct Cfg {
  static constexpr int NS = WN * TN;  // 32-row weight tiles per workgroup
  static constexpr int MS = WM * TM;  // 32-token tiles per workgroup
  static constexpr int W_CH = NS * kWRec / 16;  // 16-byte chunks per stage
  static constexpr int A_CH = MS * kARec / 16;
  // A stage is copied by "wave loads" of 64 chunks (1 KB, one DMA
  // instruction of a wave); every wave issues WPW of them per stage, the
  // ones past the data load zeros into the padding.
  static constexpr int WL_W = W_CH / 64;                       // weight wave loads
  static constexpr int WL = WL_W + (A_CH + 63) / 64;           // all wave loads
  static constexpr int WPW = (WL + kThreads / 64 - 1) / (kThreads / 64);
  static constexpr int A_LDS = NS * kWRec;  // activation records start here in a stage
  static constexpr int STAGE = WPW * (kThreads / 64) * 1024;
  static_assert(WN * WM * 64 == kThreads, "4 waves per workgroup");
  static_assert(W_CH % 64 == 0, "weight records fill whole wave loads (NS % 4 == 0)");
  static_assert(kWRec % 16 == 0 && kARec % 16 == 0, "records are 16-byte chunks");
};

// Byte offsets (stage 0) of this lane's chunk in each of its wave's loads,
// kOOB for padding loads.  Tiles past nt / mt land past the image end and
// load as zeros through the buffer range check.
template <class C>
struct Slots {
  uint32_t off[C::WPW];
};

template <class C>
__device__ __forceinline__ void init_slots(const GemmArgs &g, int wave, int nt0, int mt0, Slots<C> &s) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < C::WPW; i++) {
    const int j = wave + 4 * i;  // wave load index within the stage
    if (j < C::WL_W) {
      const int c = 64 * j + lane;
      s.off[i] = static_cast<uint32_t>((nt0 + c / (kWRec / 16)) * g.pp) * kWRec + (c % (kWRec / 16)) * 16;
    } else {
      const int c = 64 * (j - C::WL_W) + lane;
      s.off[i] = c < C::A_CH
                     ? static_cast<uint32_t>((mt0 + c / (kARec / 16)) * g.pp) * kARec + (c % (kARec / 16)) * 16
                     : kOOB;
    }
  }
}

typedef __attribute__((address_space(3))) void lds_void;
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Raw buffer resource (SGPR quad) for an image of `bytes` bytes: out-of-range
// offsets read as 0.
__device__ __forceinline__ i32x4 sgpr_rsrc(const void *base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = uniform(static_cast<int>(a & 0xffffffffu));
  r[1] = uniform(static_cast<int>((a >> 32) & 0xffffu));  // stride 0
  r[2] = uniform(static_cast<int>(bytes));
  r[3] = kBufDword3;
  return r;
}

// One wave load: lane l's 16 bytes from rsrc + voff + soff land at LDS byte
// address lds + 16 l (buffer_load_dwordx4 ... lds, address base in M0).
// Issued as inline asm so that the compiler does not see an LDS write it
// would have to fence conservatively; the pipeline waits for it explicitly
// (vmcnt).  voff must stay live (loop-invariant): a VMEM instruction may read
// its address VGPR after issue.  An LDS DMA that reads M0 right after an SALU
// write of M0 needs one wait state on this GPU family (the s_nop; the
// compiler inserts none inside inline asm).
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(soff), "s"(lds)
               : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_addr(const char *p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_void *)p));
}

// DMA stage p of this workgroup's operand records into `buf` (global ->
// LDS, no registers): wave load j lands at buf + 1 KB * j.  Record p sits at
// a uniform offset p * record size from record 0, passed as soffset.  The
// hardware range check is only guaranteed on the VGPR offset, so every
// address is kept inside the image by construction: record-0 offsets of
// tiles past the image and of padding slots are >= 2^31 (out of range ->
// zeros), and a stage p >= plive (prefetched past the end of the range and
// never computed, or a stage a K group runs only to keep its barriers in step
// with the other groups') loads zeros: its loads go through a resource of
// size 0 (every offset out of range) with soffset 0.  Either way the stage
// issues its WPW loads, so the vmcnt waits keep counting stages, and the
// VGPR offsets stay the loop-invariant ones.
template <class C>
__device__ __forceinline__ void dma_stage(const GemmArgs &g, const Slots<C> &s, int wave, int p, int plive,
                                          const char *buf) {
  const i32x4 rw = sgpr_rsrc(g.wmx, g.w_bytes);
  const i32x4 ra = sgpr_rsrc(g.amx, g.a_bytes);
  const i32x4 rz = sgpr_rsrc(g.wmx, 0u);
  const uint32_t base = lds_addr(buf);
  const bool live = p < plive;  // wave-uniform
  const int q = uniform(live ? p : 0);
  const uint32_t sw = static_cast<uint32_t>(q * kWRec), sa = static_cast<uint32_t>(q * kARec);
#pragma unroll
  for (int i = 0; i < C::WPW; i++) {
    const int j = wave + 4 * i;  // wave-uniform: the selects below are scalar
    const bool wt = j < C::WL_W;
    dma16(live ? (wt ? rw : ra) : rz, s.off[i], wt ? sw : sa, base + 1024u * static_cast<uint32_t>(j));
  }
}

// Per-thread LDS byte offsets (from a stage buffer's start) of a wave's
// operand reads, built once and kept opaque: every read is then one base
// VGPR plus a constant (buffer, tile, block), so the whole pipeline holds 10
// address VGPRs instead of one per buffer and read.  Blocks 0 and 1 have
// bases of their own, so the compiler does not pair their reads into one
// ds_read2 whose result would then be split into the two operands by v_mov.
struct StageOffs {
  int a16[2], a8[2];  // weight operand rows (plane0, plane1) of blocks 0 and 1, tile tn = 0
  int b16[2], b8[2];  // activation operand rows (h or l half) of blocks 0 and 1, tile tm = 0
  int ws, as;         // weight / activation scale arrays
};

template <class C, int TN, int TM>
__device__ __forceinline__ StageOffs stage_offsets(int wn, int wm) {
  const int lane = threadIdx.x & 63, row = lane & 31, half = lane >> 5;
  const int wrec = wn * TN * kWRec, arec = C::A_LDS + wm * TM * kARec;
  StageOffs o;
#pragma unroll
  for (int b = 0; b < 2; b++) {
    o.a16[b] = opaque(wrec + b * kTile + row * 16);
    o.a8[b] = opaque(wrec + b * kTile + 512 + row * 8);
    o.b16[b] = opaque(arec + (2 * b + half) * kTile + row * 16);
    o.b8[b] = opaque(arec + (2 * b + half) * kTile + 512 + row * 8);
  }
  o.ws = opaque(wrec + 2 * kTile + lane * 4);
  o.as = opaque(arec + 4 * kTile + lane * 4);
  return o;
}

// One stage of the inner loop for a wave's TN x TM tiles: per tile, the
// outer product of the two blocks' scales, the two blocks' exact dots, and
// 32 FMAs folding them into the accumulators (block order as in the reference).
template <class C, int TN, int TM>
__device__ __forceinline__ void compute_stage(const char *buf, const StageOffs &o, float (&acc)[TN][TM][16]) {
  const v32f zero32 = {};
  if constexpr (TN * TM > 1) {
    // Several tiles per wave: all operands first (LDS reads), then per tile
    // its scales' outer product, its two block dots and its folds, so one
    // tile's products are live at a time (same per-element arithmetic and
    // block order as below).
    float xs[TN], ys[TM];
    v8i A[2][TN], B[2][TM];
#pragma unroll
    for (int tn = 0; tn < TN; tn++) xs[tn] = *reinterpret_cast<const float *>(buf + o.ws + tn * kWRec);
#pragma unroll
    for (int tm = 0; tm < TM; tm++) ys[tm] = *reinterpret_cast<const float *>(buf + o.as + tm * kARec);
#pragma unroll
    for (int b = 0; b < 2; b++) {
#pragma unroll
      for (int tn = 0; tn < TN; tn++) A[b][tn] = mx_operand(buf + o.a16[b] + tn * kWRec, buf + o.a8[b] + tn * kWRec);
#pragma unroll
      for (int tm = 0; tm < TM; tm++) B[b][tm] = mx_operand(buf + o.b16[b] + tm * kARec, buf + o.b8[b] + tm * kARec);
    }
#pragma unroll
    for (int tn = 0; tn < TN; tn++)
#pragma unroll
      for (int tm = 0; tm < TM; tm++) {
        const v32f P = __builtin_amdgcn_mfma_f32_32x32x1f32(xs[tn], ys[tm], zero32, 0, 0, 0);
        const v16f c0 = mx_block_dot(A[0][tn], B[0][tm]);
        const v16f c1 = mx_block_dot(A[1][tn], B[1][tm]);
        float t0[16];
#pragma unroll
        for (int v = 0; v < 16; v++) t0[v] = fmaf(c0[v], P[v], acc[tn][tm][v]);
#pragma unroll
        for (int v = 0; v < 16; v++) acc[tn][tm][v] = fmaf(c1[v], P[16 + v], t0[v]);
      }
    __builtin_amdgcn_sched_group_barrier(0x100, 5 * (TN + TM), 0);  // DS reads
#pragma unroll
    for (int t = 0; t < TN * TM; t++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);   // outer product + block dots
      __builtin_amdgcn_sched_group_barrier(0x002, 32, 0);  // folds
    }
    return;
  }
  // The scale outer products go first: lane L holds block L/32, row or token
  // L%32 of the record's f32 scale array [block][row] (read linearly).  Their
  // 16-pass MFMA runs while the dot operands arrive from LDS, and their
  // result is ready when the first block's dots are.
  float xs[TN], ys[TM];
  v8i A[2][TN], B[2][TM];
#pragma unroll
  for (int tn = 0; tn < TN; tn++) xs[tn] = *reinterpret_cast<const float *>(buf + o.ws + tn * kWRec);
#pragma unroll
  for (int tm = 0; tm < TM; tm++) ys[tm] = *reinterpret_cast<const float *>(buf + o.as + tm * kARec);
  v32f P[TN][TM];
#pragma unroll
  for (int tn = 0; tn < TN; tn++)
#pragma unroll
    for (int tm = 0; tm < TM; tm++) P[tn][tm] = __builtin_amdgcn_mfma_f32_32x32x1f32(xs[tn], ys[tm], zero32, 0, 0, 0);
#pragma unroll
  for (int b = 0; b < 2; b++) {
#pragma unroll
    for (int tn = 0; tn < TN; tn++) A[b][tn] = mx_operand(buf + o.a16[b] + tn * kWRec, buf + o.a8[b] + tn * kWRec);
#pragma unroll
    for (int tm = 0; tm < TM; tm++) B[b][tm] = mx_operand(buf + o.b16[b] + tm * kARec, buf + o.b8[b] + tm * kARec);
  }
#pragma unroll
  for (int tn = 0; tn < TN; tn++)
#pragma unroll
    for (int tm = 0; tm < TM; tm++) {
      const v16f c0 = mx_block_dot(A[0][tn], B[0][tm]);
      const v16f c1 = mx_block_dot(A[1][tn], B[1][tm]);
      // Per element the blocks are added in order.
      float t0[16];
#pragma unroll
      for (int v = 0; v < 16; v++) t0[v] = fmaf(c0[v], P[tn][tm][v], acc[tn][tm][v]);
#pragma unroll
      for (int v = 0; v < 16; v++) acc[tn][tm][v] = fmaf(c1[v], P[tn][tm][16 + v], t0[v]);
    }
  __builtin_amdgcn_sched_group_barrier(0x100, TN + TM, 0);        // DS reads of the scales
  __builtin_amdgcn_sched_group_barrier(0x008, TN * TM, 0);        // outer products
  __builtin_amdgcn_sched_group_barrier(0x100, 4 * (TN + TM), 0);  // DS reads of the operands
#pragma unroll
  for (int t = 0; t < TN * TM; t++) {
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);   // block dots
    __builtin_amdgcn_sched_group_barrier(0x002, 32, 0);  // folds
  }
}

// Wait until at most N of this wave's vector-memory operations are in
// flight and its LDS operations are done, then meet the workgroup.  The
// "memory" clobber keeps every LDS access on its side of the barrier.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

// Stage p, held in `cur`; `nxt` (read during stage p-1) receives stage
// p+NB-1.  The wait leaves only stages p+1..p+NB-2's DMAs of this wave in
// flight; after the barrier every wave's DMAs of stage p are complete and
// every wave is done reading `nxt`.
template <class C, int TN, int TM, int NB>
__device__ __forceinline__ void pipeline_step(const GemmArgs &g, const Slots<C> &slots, int wave, int p, int plive,
                                              const char *cur, char *nxt, const StageOffs &o,
                                              float (&acc)[TN][TM][16]) {
  wait_vm_barrier<(NB - 2) * C::WPW>();
  dma_stage<C>(g, slots, wave, p + NB - 1, plive, nxt);
  compute_stage<C, TN, TM>(cur, o, acc);
  // Keep each stage's MFMAs and folds inside the stage: interleaving them
  // with the next stage's only lengthens register lifetimes.
  __builtin_amdgcn_sched_barrier(0);
}

// NB stage buffers (prefetch distance NB - 1); WPE waves per SIMD.  KG K
// groups of 4 waves: group k runs its own pipeline over the k-th part of the
// workgroup's block pairs (every group the same number of stages, the last
// ones possibly of zeros), and the groups' sums are added in a fixed tree at
// the end -- KG times the waves for a launch whose tiles alone leave the
// SIMDs with less than one wave each, with no second launch to add partials.
template <int WN, int WM, int TN, int TM, int NB, int WPE, int KG = 1>
__global__ __launch_bounds__(kThreads * KG) __attribute__((amdgpu_waves_per_eu(WPE))) void q4_gemm_mx_kernel(
    GemmMulti gm) {
  using C = Cfg<WN, WM, TN, TM>;
  // NB stage buffers per K group in one array, indexed by compile-time
  // constants only (and the group): a buffer's reads are the per-thread
  // offsets plus a constant.
  __shared__ __align__(1024) char lds[KG][NB][C::STAGE];
  const int wave_g = uniform(threadIdx.x >> 6);
  const int kg = KG > 1 ? wave_g >> 2 : 0, wave = wave_g & 3;
  const int wn = wave % WN, wm = wave / WN;
  int bx = blockIdx.x, mat = 0;
  if (bx >= gm.gx0) {
    bx -= gm.gx0;
    mat = 1;
    if (bx >= gm.gx1) {
      bx -= gm.gx1;
      mat = 2;
    }
  }
  const GemmArgs &g = gm.g[uniform(mat)];
  const int nt0 = bx * C::NS, mt0 = blockIdx.y * C::MS;
  const int lane = threadIdx.x & 63, row = lane & 31, half = lane >> 5;

  float acc[TN][TM][16];
#pragma unroll
  for (int tn = 0; tn < TN; tn++)
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[tn][tm][v] = 0.0f;

  Slots<C> slots;
  init_slots<C>(g, wave, nt0, mt0, slots);
  const StageOffs offs = stage_offsets<C, TN, TM>(wn, wm);
  // Split z of the K range: block pairs [p0, pend); K group kg: n stages from q0, those from
  // qlive on of zeros.
  const int z = blockIdx.z;
  const int p0 = static_cast<int>(static_cast<long>(g.pp) * z / g.splits);
  const int pend = static_cast<int>(static_cast<long>(g.pp) * (z + 1) / g.splits);
  const int n = (pend - p0 + KG - 1) / KG;
  const int q0 = p0 + kg * n, qend = q0 + n, qlive = min(qend, pend);
  char (&buf)[NB][C::STAGE] = lds[kg];
#pragma unroll
  for (int u = 0; u < NB - 1; u++) dma_stage<C>(g, slots, wave, q0 + u, qlive, buf[u]);
  // Unrolled by NB so every stage's buffer roles are static.
  int p = q0;
  for (; p + NB - 1 < qend; p += NB) {
#pragma unroll
    for (int u = 0; u < NB; u++)
      pipeline_step<C, TN, TM, NB>(g, slots, wave, p + u, qlive, buf[u], buf[(u + NB - 1) % NB], offs, acc);
  }
#pragma unroll
  for (int u = 0; u < NB - 1; u++)
    if (p + u < qend)
      pipeline_step<C, TN, TM, NB>(g, slots, wave, p + u, qlive, buf[u], buf[(u + NB - 1) % NB], offs, acc);
  // Drain the prefetches of stages past the range before the workgroup can
  // exit (their LDS must not be written after it is released).
  asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
  if constexpr (KG > 1) {
    // The groups' sums through the (now idle) stage buffers, a tree in group
    // order: at level h group kg + h's sums are added to group kg's (kg < h),
    // so four groups give (g0 + g2) + (g1 + g3).  Every wave takes every
    // barrier; only group 0 goes on to the stores.
    constexpr int kSlot = 4 * TN * TM * 16 * 64;
    static_assert((KG / 2) * kSlot * sizeof(float) <= sizeof(lds), "exchange fits the stage buffers");
    float *xch = reinterpret_cast<float *>(&lds[0][0][0]);
#pragma unroll
    for (int h = KG / 2; h >= 1; h /= 2) {
      __syncthreads();
      if (kg >= h && kg < 2 * h) {
        float *slot = xch + (kg - h) * kSlot;
#pragma unroll
        for (int tn = 0; tn < TN; tn++)
#pragma unroll
          for (int tm = 0; tm < TM; tm++)
#pragma unroll
            for (int v = 0; v < 16; v++) slot[(((wave * TN + tn) * TM + tm) * 16 + v) * 64 + lane] = acc[tn][tm][v];
      }
      __syncthreads();
      if (kg < h) {
        const float *slot = xch + kg * kSlot;
#pragma unroll
        for (int tn = 0; tn < TN; tn++)
#pragma unroll
          for (int tm = 0; tm < TM; tm++)
#pragma unroll
            for (int v = 0; v < 16; v++)
              acc[tn][tm][v] = acc[tn][tm][v] + slot[(((wave * TN + tn) * TM + tm) * 16 + v) * 64 + lane];
      }
    }
    if (kg != 0) return;
  }

  // With split K the partial sums go to part[z] (assign); a second kernel
  // adds the splits in order and applies the caller's mode.
  const bool split = g.splits > 1;
  float *const out = split ? g.part + static_cast<size_t>(z) * g.m * g.n : g.y;
  const int mode = split ? LGH_ASSIGN : g.mode;
  const bool vec4 = split ? (g.n % 4 == 0) : (g.vec4 != 0);

  // Element v of a lane: token j = L % 32, weight row i = 8*(v/4) + 4*(L/32) + v%4,
  // so each group of 4 elements is 4 consecutive outputs of one token.
#pragma unroll
  for (int tn = 0; tn < TN; tn++)
#pragma unroll
    for (int tm = 0; tm < TM; tm++) {
      const int j = (mt0 + wm * TM + tm) * 32 + row;
      if (j >= g.m) continue;
      float *yrow = out + static_cast<size_t>(j) * g.n;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int i0 = (nt0 + wn * TN + tn) * 32 + 8 * q + 4 * half;
        float v[4] = {acc[tn][tm][4 * q], acc[tn][tm][4 * q + 1], acc[tn][tm][4 * q + 2], acc[tn][tm][4 * q + 3]};
        if (vec4 && i0 + 3 < g.n) {
          float4 *dst = reinterpret_cast<float4 *>(yrow + i0);
          if (mode != LGH_ASSIGN) {
            const float4 o = *dst;
            v[0] = apply_mode(o.x, v[0], mode);
            v[1] = apply_mode(o.y, v[1], mode);
            v[2] = apply_mode(o.z, v[2], mode);
            v[3] = apply_mode(o.w, v[3], mode);
          }
          *dst = make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; e++) {
            if (i0 + e >= g.n) continue;
            yrow[i0 + e] = mode == LGH_ASSIGN ? v[e] : apply_mode(yrow[i0 + e], v[e], mode);
          }
        }
      }
    }
}

// Exact block dots through the same operand images and MFMA: one wave per
// (32-row tile, 32-token tile, block kb); out[m][n][kb] = dot.
__global__ __launch_bounds__(64) void q4_mx_block_dots_kernel(const uint8_t *__restrict__ wmx,
                                                              const uint8_t *__restrict__ amx, int n, int m,
                                                              int bpr, int pp, int32_t *out) {
  const int lane = threadIdx.x, row = lane & 31, half = lane >> 5;
  const int t = blockIdx.x, u = blockIdx.y, kb = blockIdx.z;
  const char *wrec = reinterpret_cast<const char *>(wmx) + (static_cast<size_t>(t) * pp + kb / 2) * kMxWRec;
  const char *arec = reinterpret_cast<const char *>(amx) + (static_cast<size_t>(u) * pp + kb / 2) * kMxARec;
  const v8i a = mx_row(wrec + (kb & 1) * kTile, row);
  const v8i b = mx_row(arec + (2 * (kb & 1) + half) * kTile, row);
  const v16f c = mx_block_dot(a, b);
  for (int v = 0; v < 16; v++) {
    const int i = t * 32 + 8 * (v / 4) + 4 * half + (v % 4);
    const int j = u * 32 + row;
    if (i < n && j < m) out[(static_cast<size_t>(j) * n + i) * bpr + kb] = static_cast<int32_t>(c[v]);
  }
}

// y = sum over splits of part[z] (z ascending), then the caller's mode, for
// the outputs of a launch over up to three matrices: element i of their
// concatenation belongs to matrix j = the first with i < end[j].
struct ReduceMulti {
  const float *part[3];
  float *y[3];
  size_t end[3];  // cumulative m * n
  int splits, mode;
};

// Four outputs per thread, when every matrix's m * n is a multiple of 4 and
// every y is 16-byte aligned (partials always are): no float4 straddles two
// matrices.  The same additions in the same order as the scalar kernel
// (M=512, K=8192, N=1536: 35.3 -> 33.6 us; M=65, K=8192, N=8192: 34.6 ->
// 33.1 us; M=130, K=8192, N=8192: 46.8 -> 44.5 us; interleaved A/B).
__global__ __launch_bounds__(256) void splitk_reduce_multi4_kernel(ReduceMulti r) {
  const size_t i = (static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i >= r.end[2]) return;
  int j = 0;
  size_t begin = 0;
  if (i >= r.end[0]) {
    j = 1;
    begin = r.end[0];
    if (i >= r.end[1]) {
      j = 2;
      begin = r.end[1];
    }
  }
  const size_t total = r.end[j] - begin, e = i - begin;
  const float *part = r.part[j];
  float4 v = *reinterpret_cast<const float4 *>(part + e);
  for (int z = 1; z < r.splits; z++) {
    const float4 p = *reinterpret_cast<const float4 *>(part + static_cast<size_t>(z) * total + e);
    v.x += p.x;
    v.y += p.y;
    v.z += p.z;
    v.w += p.w;
  }
  float4 *y = reinterpret_cast<float4 *>(r.y[j] + e);
  if (r.mode != LGH_ASSIGN) {
    const float4 o = *y;
    v.x = apply_mode(o.x, v.x, r.mode);
    v.y = apply_mode(o.y, v.y, r.mode);
    v.z = apply_mode(o.z, v.z, r.mode);
    v.w = apply_mode(o.w, v.w, r.mode);
  }
  *y = v;
}

__global__ __launch_bounds__(256) void splitk_reduce_multi_kernel(ReduceMulti r) {
  size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= r.end[2]) return;
  int j = 0;
  size_t begin = 0;
  if (i >= r.end[0]) {
    j = 1;
    begin = r.end[0];
    if (i >= r.end[1]) {
      j = 2;
      begin = r.end[1];
    }
  }
  const size_t total = r.end[j] - begin, e = i - begin;
  const float *part = r.part[j];
  float v = part[e];
  for (int z = 1; z < r.splits; z++) v += part[static_cast<size_t>(z) * total + e];
  float *y = r.y[j];
  y[e] = r.mode == LGH_ASSIGN ? v : apply_mode(y[e], v, r.mode);
}

// Split K when the tiles alone leave CUs idle (aim for >= kSplitTarget
// workgroups), but only rows of >= kSplitMinPairs block pairs, and keep >=
// kSplitPairs per split: a split's fixed costs (pipeline fill, the store of
// its partial tile, the reduce launch) outweigh the extra workgroups on
// shorter ones.  Measured (whole call): K=2048, N=8192, M=65 / 128 / 192:
// 20.4 / 23.1 / 28.1 -> 15.1 / 16.0 / 19.6 us unsplit (the former rule split
// down to 8 pairs); M=512, K=1536, N=2560 25.5 -> 17.2 us; K=8192, N=1536,
// M=65 / 128: 20.9 / 23.3 -> 19.1 / 20.6 us with >= 16 pairs per split.
template <int WN, int WM, int TN, int TM>
int splits_for_tiles(long tiles, size_t pp) {
  int splits = 1;
  if (pp < kSplitMinPairs) return splits;
  while (tiles * splits < kSplitTarget && pp / (2 * splits) >= kSplitPairs) splits *= 2;
  return splits;
}

template <int WN, int WM, int TN, int TM, int NB, int WPE, int KG = 1>
hipError_t launch_cfg(GemmMulti gm, int nmat, int splits, hipStream_t st) {
  using C = Cfg<WN, WM, TN, TM>;
  int gx[3] = {0, 0, 0};
  for (int j = 0; j < nmat; j++) {
    gm.g[j].splits = splits;
    gx[j] = (gm.g[j].nt + C::NS - 1) / C::NS;
  }
  gm.gx0 = gx[0];
  gm.gx1 = gx[1];
  const dim3 grid(static_cast<unsigned>(gx[0] + gx[1] + gx[2]), (gm.g[0].mt + C::MS - 1) / C::MS, splits);
  hipLaunchKernelGGL((q4_gemm_mx_kernel<WN, WM, TN, TM, NB, WPE, KG>), grid, dim3(kThreads * KG), 0, st, gm);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  ReduceMulti r{};
  size_t end = 0;
  for (int j = 0; j < 3; j++) {
    if (j < nmat) {
      r.part[j] = gm.g[j].part;
      r.y[j] = gm.g[j].y;
      end += static_cast<size_t>(gm.g[j].m) * gm.g[j].n;
    }
    r.end[j] = end;
  }
  r.splits = splits;
  r.mode = gm.g[0].mode;
  bool vec = true;
  for (int j = 0; j < nmat; j++)
    vec = vec && (static_cast<size_t>(gm.g[j].m) * gm.g[j].n) % 4 == 0 &&
          (reinterpret_cast<uintptr_t>(gm.g[j].y) & 15u) == 0;
  if (vec)
    hipLaunchKernelGGL(splitk_reduce_multi4_kernel, dim3(static_cast<unsigned>((end / 4 + 255) / 256)), dim3(256), 0,
                       st, r);
  else
    hipLaunchKernelGGL(splitk_reduce_multi_kernel, dim3(static_cast<unsigned>((end + 255) / 256)), dim3(256), 0, st,
                       r);
  return hipGetLastError();
}

}  // namespace

// Workgroups of a launch with workgroup tiles of NS 32-row x MS 32-token
// tiles, summed over the matrices of one call.
template <int NS, int MS>
static long gemm_tiles(const lgh_q4 *const *w, int nmat, size_t m) {
  long tiles = 0;
  for (int j = 0; j < nmat; j++) tiles += static_cast<long>((w[j]->nt + NS - 1) / NS);
  return tiles * static_cast<long>(((m + 31) / 32 + MS - 1) / MS);
}

GemmPlan plan_q4_gemm(const lgh_q4 *const *w, int nmat, size_t m) {
  GemmPlan plan;
  const long tiles = gemm_tiles<4, 1>(w, nmat, m);
  const size_t pp = w[0]->pp;
  plan.splits = splits_for_tiles<4, 1, 1, 1>(tiles, pp);
  // Two K groups instead of two splits on rows of <= 128 block pairs: the
  // same waves, no partials and no reduce launch.  Whole calls, interleaved
  // A/B: K=4096, N=4096, M=256 25.7 -> 22.2 us; K=8192, N=8192, M=128 37.4 ->
  // 35.4 us.  On longer rows the split stays ahead (K=10752, N=2048, M=512
  // 47.9 against 48.6 us, bit-identical: the halves are the same), and in
  // place of one of four or more splits the groups lose (K=8192, N=1536,
  // M=512: 4 splits 33.5 us, 2 groups x 2 splits 35.0 us).
  if (plan.splits == 2 && pp <= kKgSplitPairs) plan.splits = 1;
  if (plan.splits == 1 && tiles < kKg4Tiles && pp >= 4)
    plan.kgroups = 4;
  else if (plan.splits == 1 && tiles < kKgTiles && pp >= 2)
    plan.kgroups = 2;
  return plan;
}

hipError_t launch_q4_gemm(const lgh_q4 *const *w, int nmat, const uint8_t *mxa, float *const *y, size_t m, int mode,
                          GemmPlan plan, float *part, size_t part_floats, hipStream_t st) {
  if (m == 0 || nmat < 1 || nmat > 3) return m == 0 ? hipSuccess : hipErrorInvalidValue;
  size_t rows = 0;
  for (int j = 0; j < nmat; j++) rows += w[j]->n;
  if (rows == 0) return hipSuccess;
  const int splits = plan.splits;
  if (splits < 1 || (splits > 1 && (!part || static_cast<size_t>(splits) * m * rows > part_floats)))
    return hipErrorInvalidValue;
  if (plan.kgroups != 1 && ((plan.kgroups != 2 && plan.kgroups != 4) || splits != 1 ||
                            w[0]->pp < static_cast<size_t>(plan.kgroups)))
    return hipErrorInvalidValue;
  const size_t mt = (m + 31) / 32;
  GemmMulti gm{};
  size_t off = 0;
  for (int j = 0; j < nmat; j++) {
    gm.g[j] = GemmArgs{w[j]->mx,
                       mxa,
                       y[j],
                       splits > 1 ? part + static_cast<size_t>(splits) * m * off : nullptr,
                       static_cast<int>(w[j]->n),
                       static_cast<int>(m),
                       static_cast<int>(w[j]->nt),
                       static_cast<int>(mt),
                       static_cast<int>(w[j]->pp),
                       mode,
                       (w[j]->n % 4 == 0 && (reinterpret_cast<uintptr_t>(y[j]) & 15u) == 0) ? 1 : 0,
                       1,
                       static_cast<uint32_t>(w[j]->nt * w[j]->pp * kMxWRec),
                       static_cast<uint32_t>(mt * w[j]->pp * kMxARec)};
    off += w[j]->n;
  }
  // Without split K and with >= 640 of them: 128-row x 64-token workgroup
  // tiles (each wave 32 rows x 64 tokens: 156 VGPRs, 3 waves per SIMD, 48 KB
  // of LDS), 35% fewer operand bytes through L2 and LDS per MAC than 128 x 32.
  // Whole calls, against 128 x 32: M=512, K=2048, N=10752 (672 workgroups)
  // 41.3 -> 38.8 us; M=768 / 1024, same K and N, 53.8 -> 52.2 / 71.0 -> 68.6
  // us; M=2048, K=2048, N=10752 141.7 -> 128.8 us (and against the two-buffer
  // 5-wave form of 128 x 32, 134-137 us); M=2048, K=1536, N=8192 79.2 -> 74.8
  // us; M=4096, K=2048, N=10752 316 -> 291 us.  Fewer workgroups leave CUs
  // idle: M=512, K=2048, N=8192 (512) 32.2 -> 32.5 us, M=256, N=10752 (336)
  // 25.8 -> 29.3 us, M=1024, K=10752, N=2048 (256; split K otherwise) 82.6
  // -> 94.4 us.
  // Few tiles and no split K (planned for the whole call: the two groups' sums
  // are added at the end, another f32 order): K groups per workgroup; two: 8
  // waves, 72 KB of LDS.  Whole calls, against one group: K=2048, N=8192, M=65
  // / 128 / 192: 17.1 / 17.8 / 20.3 -> 14.4 / 15.3 / 19.4 us; N=10752, M=65
  // 18.3 -> 15.6 us; K=1536, N=8192, M=65 13.7 -> 12.1 us; K=2048, N=2048,
  // M=512 17.3 -> 16.2 us; N=2048, K=1536, M=128 12.6 -> 11.7 us.  Below 256
  // tiles four groups (16 waves, 144 KB of LDS), against two: N=1536, K=2048,
  // M=65 / 128 / 256 13.3 / 13.5 / 14.1 -> 12.7 / 12.7 / 13.5 us; N=2048,
  // K=1536, M=65 11.7 -> 11.4 us; N=2048, K=2048, M=256 14.2 -> 13.6 us; equal
  // at N=8192 (192 tiles at M=65).
  if (plan.kgroups == 4) return launch_cfg<4, 1, 1, 1, 3, 4, 4>(gm, nmat, 1, st);
  if (plan.kgroups == 2) return launch_cfg<4, 1, 1, 1, 3, 4, 2>(gm, nmat, 1, st);
  if (splits == 1 && gemm_tiles<4, 2>(w, nmat, m) >= kWideWgs) return launch_cfg<4, 1, 1, 2, 3, 3>(gm, nmat, 1, st);
  // Otherwise 128 x 32 (4 waves, one 32 x 32 tile each, 108 VGPRs, 4 waves
  // per SIMD): the most workgroups resident to cover the stage loads.
  return launch_cfg<4, 1, 1, 1, 3, 4>(gm, nmat, splits, st);
}

hipError_t launch_q4_mfma_block_dots(const lgh_q4 *w, const uint8_t *mxa, size_t m, int32_t *out,
                                     hipStream_t st) {
  if (w->n == 0 || m == 0 || w->bpr == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(w->nt), static_cast<unsigned>((m + 31) / 32),
                  static_cast<unsigned>(w->bpr));
  hipLaunchKernelGGL(q4_mx_block_dots_kernel, grid, dim3(64), 0, st, w->mx, mxa, static_cast<int>(w->n),
                     static_cast<int>(m), static_cast<int>(w->bpr), static_cast<int>(w->pp), out);
  return hipGetLastError();
}

}  // namespace lgh
