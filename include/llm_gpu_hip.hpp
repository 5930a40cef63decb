/*
 * llm_gpu_hip.hpp -- C++17 host interface over the C ABI (llm_gpu_hip.h),
 * header-only.
 *
 * It mirrors, with the reference's names and contracts, the host side a
 * llmhost user calls (paths relative to the llmhost repository root):
 *   - llm-quant's block formats            crates/llm-quant/src/lib.rs:17-101
 *   - llm-cpu's matmul functions           crates/llm-cpu/src/lib.rs:21-24,
 *                                          crates/llm-cpu/src/gemv_q4.rs:25-443, 686-722
 *   - llm-engine's matmul seam             crates/llm-engine/src/weights.rs:11-227
 *   - llm-core's Backend / Block traits    crates/llm-core/src/backend.rs:4-13,
 *                                          crates/llm-core/src/block.rs:6-14
 * Where the reference panics on a contract violation (assert_eq! on slice
 * lengths, k % 32), these functions throw ShapeError before any work is
 * enqueued; the C ABI's other failures throw Error with lgh_last_error()'s
 * message.  Loading errors (Linear::from_f32) throw LoadError, the
 * reference's Result::Err.  Host-pointer calls are synchronous, with the
 * reference's slice semantics.  Matrices are move-only owners of their device
 * planes.
 */
#ifndef LLM_GPU_HIP_HPP
#define LLM_GPU_HIP_HPP

#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "llm_gpu_hip.h"

namespace llm_gpu_hip {

constexpr std::size_t BLOCK_SIZE = LGH_BLOCK;  // crates/llm-quant/src/lib.rs:12

// BlockQ4 / BlockQ8_0 as stored: little-endian f16 scale bits, then the
// codes (crates/llm-quant/src/lib.rs:17-21, 54-58).
struct BlockQ4 {
  uint16_t scale;     // f16 bits
  uint8_t qs[16];     // element i in the low nibble of qs[i/2] when i is even
  // Signed 4-bit code of element i, -8..7 (lib.rs:83-92).
  int nibble(std::size_t i) const {
    const int b = qs[i / 2];
    const int v = (i & 1) ? (b >> 4) : (b & 0xF);
    return v >= 8 ? v - 16 : v;
  }
};
struct BlockQ8_0 {
  uint16_t scale;  // f16 bits
  int8_t qs[32];
};
static_assert(sizeof(BlockQ4) == LGH_BLOCK_Q4_BYTES, "BlockQ4 is 18 bytes");
static_assert(sizeof(BlockQ8_0) == LGH_BLOCK_Q8_BYTES, "BlockQ8_0 is 34 bytes");

// f16 bits -> f32, exact (every binary16 value is a binary32 value), as
// half::f16::to_f32 at crates/llm-quant/src/lib.rs:41, 96.
inline float f16_to_f32(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0x1Fu) {
    bits = sign | 0x7F800000u | (man << 13);  // inf / NaN
  } else if (exp != 0) {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  } else if (man == 0) {
    bits = sign;  // +-0
  } else {        // subnormal: normalise
    int e = -1;
    uint32_t m = man;
    do {
      m <<= 1;
      e++;
    } while ((m & 0x400u) == 0);
    bits = sign | ((112u - static_cast<uint32_t>(e)) << 23) | ((m & 0x3FFu) << 13);
  }
  float f;
  static_assert(sizeof(f) == sizeof(bits), "binary32");
  __builtin_memcpy(&f, &bits, sizeof f);
  return f;
}

class Error : public std::runtime_error {
 public:
  Error(int code, const std::string &msg) : std::runtime_error(msg), code_(code) {}
  int code() const { return code_; }

 private:
  int code_;
};

// A violated contract the reference asserts (it would panic).
class ShapeError : public Error {
 public:
  using Error::Error;
};

// LoadError::Message (crates/llm-engine/src/load.rs).
class LoadError : public std::runtime_error {
 public:
  using std::runtime_error::runtime_error;
};

inline void check(const lgh_ctx *ctx, int rc) {
  if (rc == LGH_OK) return;
  const std::string msg = "[" + std::to_string(rc) + "] " + lgh_last_error(ctx);
  if (rc == LGH_ERR_SHAPE) throw ShapeError(rc, msg);
  throw Error(rc, msg);
}

inline void require(bool ok, const char *what) {
  if (!ok) throw ShapeError(LGH_ERR_SHAPE, what);
}

// ActQuant (crates/llm-cpu/src/gemv_q4.rs:263-271).
enum class ActQuant { PerBlock = LGH_ACT_PER_BLOCK, PerRow = LGH_ACT_PER_ROW };

// One device, one stream, the workspaces and the act-quant mode: what a
// session binds to (CpuBackend::new, crates/llm-cpu/src/lib.rs:46-57).
class Context {
 public:
  explicit Context(int device = 0) { check(nullptr, lgh_init(device, &h_)); }
  ~Context() { lgh_destroy(h_); }
  Context(const Context &) = delete;
  Context &operator=(const Context &) = delete;

  // set_act_quant / current_act_quant (gemv_q4.rs:276-299), per context.
  void set_act_quant(ActQuant mode) { check(h_, lgh_set_act_quant(h_, static_cast<int>(mode))); }
  ActQuant current_act_quant() const { return static_cast<ActQuant>(lgh_get_act_quant(h_)); }
  void sync() { check(h_, lgh_sync(h_)); }
  void trim() { check(h_, lgh_trim(h_)); }
  lgh_ctx *native() const { return h_; }

 private:
  lgh_ctx *h_ = nullptr;
};

// Q4Matrix (crates/llm-cpu/src/gemv_q4.rs:97-209): the device planes of an
// n x k Q4 matrix.
class Q4Matrix {
 public:
  // Q4Matrix::from_blocks (gemv_q4.rs:116-149): blocks row-major [n][k/32].
  static Q4Matrix from_blocks(Context &ctx, std::size_t n, std::size_t k, const BlockQ4 *blocks) {
    lgh_q4 *w = nullptr;
    check(ctx.native(), lgh_q4_upload(ctx.native(), blocks, n, k, &w));
    return Q4Matrix(ctx, w);
  }
  static Q4Matrix from_blocks(Context &ctx, std::size_t n, std::size_t k, const std::vector<BlockQ4> &blocks) {
    require(blocks.size() == n * (k / BLOCK_SIZE) && k % BLOCK_SIZE == 0, "Q4Matrix::from_blocks: block count");
    return from_blocks(ctx, n, k, blocks.data());
  }
  // Q4Matrix::from_f32 (gemv_q4.rs:128-149): quantize_q4 on the device.
  static Q4Matrix from_f32(Context &ctx, const float *w, std::size_t n, std::size_t k) {
    lgh_q4 *m = nullptr;
    check(ctx.native(), lgh_q4_from_f32(ctx.native(), w, n, k, &m));
    return Q4Matrix(ctx, m);
  }
  static Q4Matrix from_f32(Context &ctx, const std::vector<float> &w, std::size_t n, std::size_t k) {
    require(w.size() == n * k, "Q4Matrix::from_f32: weight length");
    return from_f32(ctx, w.data(), n, k);
  }

  Q4Matrix(Q4Matrix &&o) noexcept : ctx_(o.ctx_), w_(std::exchange(o.w_, nullptr)) {}
  Q4Matrix &operator=(Q4Matrix &&o) noexcept {
    if (this != &o) {
      lgh_q4_free(w_);
      ctx_ = o.ctx_;
      w_ = std::exchange(o.w_, nullptr);
    }
    return *this;
  }
  Q4Matrix(const Q4Matrix &) = delete;
  Q4Matrix &operator=(const Q4Matrix &) = delete;
  ~Q4Matrix() { lgh_q4_free(w_); }

  std::size_t n() const { return lgh_q4_rows(w_); }
  std::size_t k() const { return lgh_q4_cols(w_); }
  // The blocks back, as uploaded or as from_f32 quantized them.
  std::vector<BlockQ4> blocks() const {
    std::vector<BlockQ4> b(n() * (k() / BLOCK_SIZE));
    check(ctx_->native(), lgh_q4_download(ctx_->native(), w_, b.data()));
    return b;
  }
  // Build the GEMM operand image now (it is otherwise built on first GEMM use).
  void prepare_gemm() const { check(ctx_->native(), lgh_q4_prepare_gemm(ctx_->native(), w_)); }
  Context &context() const { return *ctx_; }
  const lgh_q4 *native() const { return w_; }

 private:
  Q4Matrix(Context &ctx, lgh_q4 *w) : ctx_(&ctx), w_(w) {}
  Context *ctx_;
  lgh_q4 *w_;
};

// Q8Matrix (crates/llm-engine/src/weights.rs:126-153).
class Q8Matrix {
 public:
  static Q8Matrix from_blocks(Context &ctx, std::size_t n, std::size_t k, const BlockQ8_0 *blocks) {
    lgh_q8 *w = nullptr;
    check(ctx.native(), lgh_q8_upload(ctx.native(), blocks, n, k, &w));
    return Q8Matrix(ctx, w);
  }
  // quantize_q8_0 of a row-major fp32 [n][k] (weights.rs:133-146), on the device.
  static Q8Matrix from_f32(Context &ctx, const float *w, std::size_t n, std::size_t k) {
    lgh_q8 *m = nullptr;
    check(ctx.native(), lgh_q8_from_f32(ctx.native(), w, n, k, &m));
    return Q8Matrix(ctx, m);
  }
  Q8Matrix(Q8Matrix &&o) noexcept : ctx_(o.ctx_), w_(std::exchange(o.w_, nullptr)) {}
  Q8Matrix &operator=(Q8Matrix &&o) noexcept {
    if (this != &o) {
      lgh_q8_free(w_);
      ctx_ = o.ctx_;
      w_ = std::exchange(o.w_, nullptr);
    }
    return *this;
  }
  Q8Matrix(const Q8Matrix &) = delete;
  Q8Matrix &operator=(const Q8Matrix &) = delete;
  ~Q8Matrix() { lgh_q8_free(w_); }

  std::size_t n() const { return lgh_q8_rows(w_); }
  std::size_t k() const { return lgh_q8_cols(w_); }
  std::vector<BlockQ8_0> blocks() const {
    std::vector<BlockQ8_0> b(n() * (k() / BLOCK_SIZE));
    check(ctx_->native(), lgh_q8_download(ctx_->native(), w_, b.data()));
    return b;
  }
  Context &context() const { return *ctx_; }
  const lgh_q8 *native() const { return w_; }

 private:
  Q8Matrix(Context &ctx, lgh_q8 *w) : ctx_(&ctx), w_(w) {}
  Context *ctx_;
  lgh_q8 *w_;
};

// ActQ8 (crates/llm-cpu/src/gemv_q4.rs:25-95): per 32-block int8 codes,
// f32 scales and code sums of one activation row, in the context's mode.
struct ActQ8 {
  std::vector<int8_t> qs;
  std::vector<float> scales;
  std::vector<int32_t> sums;

  static ActQ8 quantize(Context &ctx, const std::vector<float> &x) {
    require(x.size() % BLOCK_SIZE == 0, "ActQ8::quantize: len % 32 != 0");
    ActQ8 a;
    a.qs.resize(x.size());
    a.scales.resize(x.size() / BLOCK_SIZE);
    a.sums.resize(x.size() / BLOCK_SIZE);
    if (!x.empty())
      check(ctx.native(),
            lgh_act_quant(ctx.native(), x.data(), 1, x.size(), a.qs.data(), a.scales.data(), a.sums.data()));
    return a;
  }
};

// ---- llm-cpu's matmul functions (crates/llm-cpu/src/lib.rs:21-24) ----------

// gemv_q4 (gemv_q4.rs:344-353): out[n] = W x.  Asserts x.len() == k and
// out.len() == n.
inline void gemv_q4(const Q4Matrix &w, const std::vector<float> &x, std::vector<float> &out) {
  require(x.size() == w.k() && out.size() == w.n(), "gemv_q4: x.len() == k and out.len() == n");
  check(w.context().native(), lgh_q4_gemv(w.context().native(), w.native(), x.data(), out.data(), LGH_ASSIGN));
}

// gemv_q4_add (gemv_q4.rs:355-364): dst += W x in f64.
inline void gemv_q4_add(const Q4Matrix &w, const std::vector<float> &x, std::vector<float> &dst) {
  require(x.size() == w.k() && dst.size() == w.n(), "gemv_q4_add: x.len() == k and dst.len() == n");
  check(w.context().native(), lgh_q4_gemv(w.context().native(), w.native(), x.data(), dst.data(), LGH_ADD_F64));
}

// gemv_q4_prep (gemv_q4.rs:366-393): the GEMV on activations already
// quantized by ActQ8::quantize.
inline void gemv_q4_prep(const Q4Matrix &w, const ActQ8 &a, std::vector<float> &out) {
  require(a.qs.size() == w.k() && a.scales.size() == w.k() / BLOCK_SIZE && out.size() == w.n(),
          "gemv_q4_prep: acts and out lengths");
  check(w.context().native(), lgh_q4_gemv_prep(w.context().native(), w.native(), a.qs.data(), a.scales.data(),
                                                out.data(), LGH_ASSIGN));
}

// gemv_q4_pair (gemv_q4.rs:396-443): gate and up on one activation.  The
// reference asserts equal k and equal 16-row tile counts and stores both
// outputs with the gate's n (:417-441), which is only well defined for equal
// n; equal shapes are required here.
inline void gemv_q4_pair(const Q4Matrix &wg, const Q4Matrix &wu, const std::vector<float> &x,
                         std::vector<float> &out_gate, std::vector<float> &out_up) {
  require(wg.k() == wu.k() && wg.n() == wu.n(), "gemv_q4_pair: equal shapes");
  require(x.size() == wg.k() && out_gate.size() == wg.n() && out_up.size() == wu.n(),
          "gemv_q4_pair: x / out lengths");
  check(wg.context().native(), lgh_q4_gemv_pair(wg.context().native(), wg.native(), wu.native(), x.data(),
                                                 out_gate.data(), out_up.data()));
}

// gemm_q4 (gemv_q4.rs:686-688, 696-722): out[m][n] = x[m][k] W^T.
inline void gemm_q4(const Q4Matrix &w, const std::vector<float> &x, std::vector<float> &out, std::size_t m) {
  require(x.size() == m * w.k() && out.size() == m * w.n(), "gemm_q4: x.len() == m*k and out.len() == m*n");
  check(w.context().native(), lgh_q4_gemm(w.context().native(), w.native(), x.data(), out.data(), m, LGH_ASSIGN));
}

// gemm_q4_add (gemv_q4.rs:690-693): out += x W^T in f64.
inline void gemm_q4_add(const Q4Matrix &w, const std::vector<float> &x, std::vector<float> &out, std::size_t m) {
  require(x.size() == m * w.k() && out.size() == m * w.n(), "gemm_q4_add: x.len() == m*k and out.len() == m*n");
  check(w.context().native(), lgh_q4_gemm(w.context().native(), w.native(), x.data(), out.data(), m, LGH_ADD_F64));
}

// q8_apply (crates/llm-engine/src/weights.rs:194-227): the Q8_0 GEMV, token by token.
inline void q8_apply(const Q8Matrix &w, const std::vector<float> &x, std::size_t tokens, std::vector<float> &out) {
  require(x.size() == tokens * w.k() && out.size() == tokens * w.n(), "q8_apply: x / out lengths");
  check(w.context().native(), lgh_q8_gemv(w.context().native(), w.native(), x.data(), out.data(), tokens));
}

// ---- llm-engine's seam (crates/llm-engine/src/weights.rs) ------------------

// WeightFormat (crates/llm-quant/src/formats.rs:9-57): the tags of this path.
enum class WeightFormat { F32, Q8_0, Q4_32 };

// Linear (weights.rs:11-103) in its Q4 variant: Y = X W^T with W [rows, cols].
// The fp32 variant of the reference is not part of the block-quantized path.
class Linear {
 public:
  explicit Linear(Q4Matrix m) : m_(std::move(m)) {}

  // Linear::from_f32 (weights.rs:22-48).
  static Linear from_f32(Context &ctx, const std::vector<float> &weight, std::size_t rows, std::size_t cols,
                         WeightFormat format) {
    if (weight.size() != rows * cols)
      throw LoadError("linear weight length " + std::to_string(weight.size()) + " != " + std::to_string(rows) +
                      "*" + std::to_string(cols));
    if (format != WeightFormat::Q4_32) throw LoadError("unsupported linear weight format on the device path");
    if (cols % BLOCK_SIZE)
      throw LoadError("Q4 linear K=" + std::to_string(cols) + " is not a multiple of " + std::to_string(BLOCK_SIZE));
    return Linear(Q4Matrix::from_f32(ctx, weight, rows, cols));
  }

  std::size_t rows() const { return m_.n(); }
  std::size_t cols() const { return m_.k(); }
  const Q4Matrix &matrix() const { return m_; }

  // out[tokens, rows] = x[tokens, cols] W^T (weights.rs:75-88).
  void apply(const std::vector<float> &x, std::size_t tokens, std::vector<float> &out) const {
    require(x.size() == tokens * cols() && out.size() == tokens * rows(), "Linear::apply: x / out lengths");
    if (tokens == 1)
      gemv_q4(m_, x, out);
    else
      gemm_q4(m_, x, out, tokens);
  }

  // dst[tokens, rows] += x W^T with the f64 residual add (weights.rs:91-102).
  void apply_add(const std::vector<float> &x, std::size_t tokens, std::vector<float> &dst) const {
    require(x.size() == tokens * cols() && dst.size() == tokens * rows(), "Linear::apply_add: x / dst lengths");
    if (tokens == 1)
      gemv_q4_add(m_, x, dst);
    else
      gemm_q4_add(m_, x, dst, tokens);
  }

 private:
  Q4Matrix m_;
};

// apply_pair (weights.rs:106-123): gemv_q4_pair for one token (which
// requires w1 and w3 of one shape), two applies otherwise.
inline void apply_pair(const Linear &w1, const Linear &w3, const std::vector<float> &x, std::size_t tokens,
                       std::vector<float> &out1, std::vector<float> &out3) {
  if (tokens == 1) {
    gemv_q4_pair(w1.matrix(), w3.matrix(), x, out1, out3);
  } else {
    w1.apply(x, tokens, out1);
    w3.apply(x, tokens, out3);
  }
}

// OutputHead (weights.rs:156-192): the Q8_0 tied head, or a Linear.
class OutputHead {
 public:
  explicit OutputHead(Q8Matrix q8) : q8_(std::make_unique<Q8Matrix>(std::move(q8))) {}
  explicit OutputHead(Linear lin) : lin_(std::make_unique<Linear>(std::move(lin))) {}
  std::size_t rows() const { return q8_ ? q8_->n() : lin_->rows(); }
  // logits[tokens, rows] = x W^T (weights.rs:186-191).
  void apply(const std::vector<float> &x, std::size_t tokens, std::vector<float> &out) const {
    if (q8_)
      q8_apply(*q8_, x, tokens, out);
    else
      lin_->apply(x, tokens, out);
  }

 private:
  std::unique_ptr<Q8Matrix> q8_;
  std::unique_ptr<Linear> lin_;
};

// ---- llm-core's Backend / Block traits -------------------------------------

// Backend::Buffer (crates/llm-core/src/backend.rs:4-13): a zeroed device f32
// allocation of `len` elements.
class HipBuffer {
 public:
  HipBuffer(Context &ctx, std::size_t len) : ctx_(&ctx), len_(len) {
    check(ctx.native(), lgh_buffer_alloc(ctx.native(), len, &p_));
  }
  HipBuffer(HipBuffer &&o) noexcept
      : ctx_(o.ctx_), len_(std::exchange(o.len_, 0)), p_(std::exchange(o.p_, nullptr)) {}
  HipBuffer(const HipBuffer &) = delete;
  HipBuffer &operator=(const HipBuffer &) = delete;
  ~HipBuffer() { lgh_buffer_free(ctx_->native(), p_); }
  std::size_t len() const { return len_; }
  float *device_ptr() const { return p_; }
  void write(const std::vector<float> &src) {
    require(src.size() == len_, "HipBuffer::write: length");
    check(ctx_->native(), lgh_buffer_write(ctx_->native(), p_, src.data(), len_));
  }
  std::vector<float> read() const {
    std::vector<float> out(len_);
    check(ctx_->native(), lgh_buffer_read(ctx_->native(), out.data(), p_, len_));
    return out;
  }

 private:
  Context *ctx_;
  std::size_t len_;
  float *p_ = nullptr;
};

// Backend (backend.rs:4-13): name() and alloc(len).
class HipBackend {
 public:
  explicit HipBackend(Context &ctx) : ctx_(&ctx) {}
  const char *name() const { return "hip"; }
  HipBuffer alloc(std::size_t len) const { return HipBuffer(*ctx_, len); }

 private:
  Context *ctx_;
};

// LayerKind / Block (crates/llm-core/src/block.rs:6-14) for the FFN block of
// one layer: forward(input, output) writes output = input + W2
// (silu(W1 n) * W3 n), n = rms_norm(input) (crates/llm-engine/src/lfm2.rs:883-911).
enum class LayerKind { Attention, Conv, Ffn };

class HipFfnBlock {
 public:
  HipFfnBlock(const Q4Matrix &w1, const Q4Matrix &w3, const Q4Matrix &w2, std::vector<float> norm_w, float eps)
      : w1_(&w1), w3_(&w3), w2_(&w2), norm_w_(std::move(norm_w)), eps_(eps) {
    require(w1.k() == w3.k() && w1.n() == w3.n() && w2.k() == w1.n() && w2.n() == w1.k() &&
                norm_w_.size() == w1.k(),
            "HipFfnBlock: w1/w3 [inter, dim], w2 [dim, inter], norm [dim]");
  }
  LayerKind kind() const { return LayerKind::Ffn; }
  // output[tokens, dim] = input + FFN(input).
  void forward(const std::vector<float> &input, std::vector<float> &output) const {
    const std::size_t dim = w1_->k();
    require(input.size() % dim == 0 && output.size() == input.size(), "HipFfnBlock::forward: lengths");
    output = input;
    if (input.empty()) return;
    Context &c = w1_->context();
    check(c.native(), lgh_q4_ffn_residual(c.native(), w1_->native(), w3_->native(), w2_->native(), norm_w_.data(),
                                          eps_, output.data(), input.size() / dim));
  }

 private:
  const Q4Matrix *w1_, *w3_, *w2_;
  std::vector<float> norm_w_;
  float eps_;
};

}  // namespace llm_gpu_hip

#endif  // LLM_GPU_HIP_HPP
