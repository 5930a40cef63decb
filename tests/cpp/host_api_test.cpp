// Tests of the C++ host interface (include/llm_gpu_hip.hpp) on the GPU, in
// the shape of the reference's own unit tests for the same functions:
//   crates/llm-quant/src/lib.rs:143-222   (block round trips, zero blocks, slices)
//   crates/llm-cpu/src/gemv_q4.rs:1071-1249 (block dots, GEMV kernels agree,
//     grid / thread independence, GEMM == per-token GEMV, GEMV == block dots)
//   crates/llm-engine/src/weights.rs:11-227 (Linear, apply_pair, OutputHead)
//   crates/llm-core/src/backend.rs:4-13, block.rs:6-14 (Backend, Block)
// with the same formula-generated inputs.  The expected values a test needs
// are computed here from the definitions, as the reference tests compute
// theirs.  Build: tests/cpp/build_cpp.py; run by tests/test_gpu_cpp_host.py.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <string>
#include <vector>

#include "llm_gpu_hip.hpp"

using namespace llm_gpu_hip;

namespace {

int g_failed = 0;

#define EXPECT(cond, ...)                                                \
  do {                                                                   \
    if (!(cond)) {                                                       \
      std::fprintf(stderr, "  FAILED %s:%d: ", __FILE__, __LINE__);      \
      std::fprintf(stderr, __VA_ARGS__);                                 \
      std::fprintf(stderr, "\n");                                        \
      throw std::runtime_error("expectation failed");                    \
    }                                                                    \
  } while (0)

template <class E, class F>
bool throws(F f) {
  try {
    f();
  } catch (const E &) {
    return true;
  }
  return false;
}

void run(const char *name, const std::function<void()> &body) {
  std::printf("[test] %s\n", name);
  std::fflush(stdout);
  try {
    body();
    std::printf("[ok] %s\n", name);
  } catch (const std::exception &e) {
    std::printf("[FAIL] %s: %s\n", name, e.what());
    g_failed++;
  }
  std::fflush(stdout);
}

float dequant(const BlockQ4 &b, std::size_t i) { return static_cast<float>(b.nibble(i)) * f16_to_f32(b.scale); }
float dequant(const BlockQ8_0 &b, std::size_t i) { return static_cast<float>(b.qs[i]) * f16_to_f32(b.scale); }

// lib.rs:149-159
std::vector<float> pattern() {
  std::vector<float> src(BLOCK_SIZE);
  for (std::size_t i = 0; i < BLOCK_SIZE; i++) src[i] = static_cast<float>(i) * 0.37f - 5.1f;
  src[0] = -6.0f;
  src[1] = 6.0f;
  src[2] = 0.0f;
  return src;
}

float amax_of(const std::vector<float> &v) {
  float m = 0.0f;
  for (float x : v) m = std::fmax(m, std::fabs(x));
  return m;
}

// dot_q4_q8_scalar (gemv_q4.rs:959-966): the exact integer block dot.
int32_t dot_q4_q8(const BlockQ4 &b, const int8_t *a) {
  int32_t s = 0;
  for (std::size_t i = 0; i < BLOCK_SIZE; i++) s += b.nibble(i) * static_cast<int32_t>(a[i]);
  return s;
}

// gemv_q4.rs:1080-1088
void pattern_block(int seed, std::vector<float> &w, std::vector<int8_t> &a) {
  w.resize(BLOCK_SIZE);
  a.resize(BLOCK_SIZE);
  for (int i = 0; i < static_cast<int>(BLOCK_SIZE); i++) {
    w[i] = static_cast<float>((i * 17 + seed) % 21 - 10) * 0.25f;
    a[i] = static_cast<int8_t>((i * 9 + seed) % 25 - 12);
  }
}

std::vector<float> gen(std::size_t len, int mul, int mod, int off, float step) {
  std::vector<float> v(len);
  for (std::size_t i = 0; i < len; i++)
    v[i] = static_cast<float>((static_cast<int>(i) * mul) % mod - off) * step;
  return v;
}

// The packed GEMV's expected value from block dots, in the reference's
// operation order (gemv_q4.rs:1212-1222): acc += idot * sw * sa, no FMA.
std::vector<float> block_dot_gemv(const std::vector<BlockQ4> &blocks, std::size_t n, std::size_t k,
                                  const ActQ8 &acts) {
  const std::size_t bpr = k / BLOCK_SIZE;
  std::vector<float> out(n);
  for (std::size_t row = 0; row < n; row++) {
    float acc = 0.0f;
    for (std::size_t b = 0; b < bpr; b++) {
      const BlockQ4 &blk = blocks[row * bpr + b];
      const int32_t idot = dot_q4_q8(blk, &acts.qs[b * BLOCK_SIZE]);
      const float t = static_cast<float>(idot) * f16_to_f32(blk.scale);
      acc = acc + t * acts.scales[b];
    }
    out[row] = acc;
  }
  return out;
}

void expect_close(const std::vector<float> &got, const std::vector<float> &want, double rel, const char *what) {
  EXPECT(got.size() == want.size(), "%s: sizes %zu vs %zu", what, got.size(), want.size());
  for (std::size_t i = 0; i < got.size(); i++)
    EXPECT(std::fabs(static_cast<double>(got[i]) - want[i]) <= rel * (1.0 + std::fabs(static_cast<double>(want[i]))),
           "%s: element %zu: %.9g vs %.9g", what, i, got[i], want[i]);
}

}  // namespace

int main() {
  Context ctx(0);

  // ---- crates/llm-quant/src/lib.rs tests -----------------------------------
  run("q8_0_roundtrip", [&] {
    const auto src = pattern();
    const auto blk = Q8Matrix::from_f32(ctx, src.data(), 1, BLOCK_SIZE).blocks().at(0);
    const float bound = amax_of(src) / 127.0f + 1e-3f;
    for (std::size_t i = 0; i < BLOCK_SIZE; i++)
      EXPECT(std::fabs(src[i] - dequant(blk, i)) <= bound, "element %zu", i);
  });
  run("q4_roundtrip", [&] {
    const auto src = pattern();
    const auto blk = Q4Matrix::from_f32(ctx, src, 1, BLOCK_SIZE).blocks().at(0);
    const float bound = amax_of(src) / 8.0f + 1e-3f;
    for (std::size_t i = 0; i < BLOCK_SIZE; i++) {
      EXPECT(std::fabs(src[i] - dequant(blk, i)) <= bound, "element %zu", i);
      EXPECT(blk.nibble(i) >= -8 && blk.nibble(i) <= 7, "nibble %zu out of range", i);
    }
  });
  run("q8_0_and_q4_zero_block", [&] {
    const std::vector<float> zero(BLOCK_SIZE, 0.0f);
    const auto b8 = Q8Matrix::from_f32(ctx, zero.data(), 1, BLOCK_SIZE).blocks().at(0);
    const auto b4 = Q4Matrix::from_f32(ctx, zero, 1, BLOCK_SIZE).blocks().at(0);
    for (std::size_t i = 0; i < BLOCK_SIZE; i++) {
      EXPECT(dequant(b8, i) == 0.0f, "q8 %zu", i);
      EXPECT(dequant(b4, i) == 0.0f, "q4 %zu", i);
    }
  });
  run("slice_helpers_roundtrip", [&] {
    std::vector<float> src(3 * BLOCK_SIZE);
    for (std::size_t i = 0; i < src.size(); i++) src[i] = std::sin(static_cast<float>(i)) * 3.0f;
    const auto b8 = Q8Matrix::from_f32(ctx, src.data(), 1, src.size()).blocks();
    const auto b4 = Q4Matrix::from_f32(ctx, src, 1, src.size()).blocks();
    float e8 = 0.0f, e4 = 0.0f;
    for (std::size_t i = 0; i < src.size(); i++) {
      e8 = std::fmax(e8, std::fabs(src[i] - dequant(b8[i / BLOCK_SIZE], i % BLOCK_SIZE)));
      e4 = std::fmax(e4, std::fabs(src[i] - dequant(b4[i / BLOCK_SIZE], i % BLOCK_SIZE)));
    }
    EXPECT(e8 < 0.05f, "slice Q8_0 err %g", e8);
    EXPECT(e4 < 0.5f, "slice Q4 err %g", e4);
  });

  // ---- crates/llm-cpu/src/gemv_q4.rs tests ---------------------------------
  run("block_dots_match_scalar_dot", [&] {  // vnni_and_avx2_match_scalar_dot
    for (int seed = 0; seed < 16; seed++) {
      std::vector<float> w;
      std::vector<int8_t> a;
      pattern_block(seed, w, a);
      const BlockQ4 blk = Q4Matrix::from_f32(ctx, w, 1, BLOCK_SIZE).blocks().at(0);
      int32_t dev = 0;
      check(ctx.native(), lgh_q4_block_dots(ctx.native(), &blk, a.data(), 1, &dev));
      EXPECT(dev == dot_q4_q8(blk, a.data()), "seed %d: %d vs %d", seed, dev, dot_q4_q8(blk, a.data()));
    }
  });
  run("gemv_kernels_agree", [&] {
    const std::size_t n = 17, k = 64;
    const auto w = gen(n * k, 13, 19, 9, 0.15f), x = gen(k, 7, 15, 7, 0.2f);
    const auto mat = Q4Matrix::from_f32(ctx, w, n, k);
    const auto acts = ActQ8::quantize(ctx, x);
    std::vector<float> prep(n), gemv(n);
    gemv_q4_prep(mat, acts, prep);
    gemv_q4(mat, x, gemv);
    const auto scalar = block_dot_gemv(mat.blocks(), n, k, acts);
    expect_close(prep, scalar, 1e-6, "prep vs scalar");
    expect_close(gemv, scalar, 1e-6, "gemv vs scalar");
  });
  run("gemv_grid_independent", [&] {  // gemv_pool_matches_serial: the split of rows changes nothing
    const std::size_t n = 128, k = 64;
    const auto w = gen(n * k, 3, 17, 8, 0.1f), x = gen(k, 5, 11, 5, 0.2f);
    const auto whole = Q4Matrix::from_f32(ctx, w, n, k);
    const auto blocks = whole.blocks();
    const std::size_t half = n / 2, bpr = k / BLOCK_SIZE;
    const auto top = Q4Matrix::from_blocks(ctx, half, k, blocks.data());
    const auto bottom = Q4Matrix::from_blocks(ctx, n - half, k, blocks.data() + half * bpr);
    std::vector<float> all(n), a(half), b(n - half);
    gemv_q4(whole, x, all);
    gemv_q4(top, x, a);
    gemv_q4(bottom, x, b);
    for (std::size_t i = 0; i < n; i++) {
      const float part = i < half ? a[i] : b[i - half];
      EXPECT(all[i] == part, "row %zu: %.9g vs %.9g", i, all[i], part);
    }
  });
  run("gemm_matches_per_token_gemv", [&] {
    const std::size_t n = 48, k = 64, m = 20;
    const auto w = gen(n * k, 3, 17, 8, 0.1f), x = gen(m * k, 5, 11, 5, 0.2f);
    const auto mat = Q4Matrix::from_f32(ctx, w, n, k);
    std::vector<float> gemm(m * n), gemv(m * n), xt(k), yt(n);
    gemm_q4(mat, x, gemm, m);
    for (std::size_t t = 0; t < m; t++) {
      std::copy(x.begin() + t * k, x.begin() + (t + 1) * k, xt.begin());
      gemv_q4(mat, xt, yt);
      std::copy(yt.begin(), yt.end(), gemv.begin() + t * n);
    }
    expect_close(gemm, gemv, 1e-5, "gemm vs gemv");
  });
  run("packed_gemv_matches_block_dots", [&] {
    const std::size_t n = 17, k = 64;
    const auto w = gen(n * k, 13, 19, 9, 0.15f), x = gen(k, 7, 15, 7, 0.2f);
    const auto blocks = Q4Matrix::from_f32(ctx, w, n, k).blocks();  // quantize_q4
    const auto acts = ActQ8::quantize(ctx, x);
    const auto expected = block_dot_gemv(blocks, n, k, acts);
    const auto mat = Q4Matrix::from_blocks(ctx, n, k, blocks);
    std::vector<float> got(n);
    gemv_q4_prep(mat, acts, got);
    expect_close(got, expected, 1e-6, "packed vs block dots");
  });
  run("contract_violations_throw", [&] {  // the reference's assert_eq!s
    const auto mat = Q4Matrix::from_f32(ctx, gen(8 * 64, 3, 17, 8, 0.1f), 8, 64);
    std::vector<float> x(63), y(8), x2(64), y2(7);
    EXPECT(throws<ShapeError>([&] { gemv_q4(mat, x, y); }), "short x");
    EXPECT(throws<ShapeError>([&] { gemv_q4(mat, x2, y2); }), "short out");
    std::vector<float> xm(3 * 64), ym(3 * 8 - 1);
    EXPECT(throws<ShapeError>([&] { gemm_q4(mat, xm, ym, 3); }), "short gemm out");
    EXPECT(throws<Error>([&] { Q4Matrix::from_f32(ctx, gen(8 * 48, 3, 17, 8, 0.1f), 8, 48); }), "k % 32");
  });

  // ---- crates/llm-engine/src/weights.rs: the seam ---------------------------
  run("linear_from_f32_errors", [&] {
    EXPECT(throws<LoadError>([&] { Linear::from_f32(ctx, std::vector<float>(10), 3, 4, WeightFormat::Q4_32); }),
           "length");
    EXPECT(throws<LoadError>([&] { Linear::from_f32(ctx, std::vector<float>(4 * 48), 4, 48, WeightFormat::Q4_32); }),
           "K % 32");
    EXPECT(throws<LoadError>([&] { Linear::from_f32(ctx, std::vector<float>(4 * 64), 4, 64, WeightFormat::F32); }),
           "format");
  });
  run("linear_apply_add_pair", [&] {
    const std::size_t rows = 40, cols = 96, tokens = 3;
    const auto w1 = gen(rows * cols, 7, 23, 11, 0.05f), w3 = gen(rows * cols, 11, 29, 14, 0.04f);
    const Linear l1 = Linear::from_f32(ctx, w1, rows, cols, WeightFormat::Q4_32);
    const Linear l3 = Linear::from_f32(ctx, w3, rows, cols, WeightFormat::Q4_32);
    const auto x1 = gen(cols, 5, 13, 6, 0.3f), xm = gen(tokens * cols, 3, 19, 9, 0.25f);
    // apply with one token is gemv_q4, with several gemm_q4.
    std::vector<float> y(rows), ref(rows), ym(tokens * rows), refm(tokens * rows);
    l1.apply(x1, 1, y);
    gemv_q4(l1.matrix(), x1, ref);
    EXPECT(y == ref, "apply(1) == gemv_q4");
    l1.apply(xm, tokens, ym);
    gemm_q4(l1.matrix(), xm, refm, tokens);
    EXPECT(ym == refm, "apply(3) == gemm_q4");
    // apply_add adds in f64 onto dst.
    std::vector<float> dst(rows), base = gen(rows, 3, 7, 3, 0.5f);
    dst = base;
    l1.apply_add(x1, 1, dst);
    for (std::size_t i = 0; i < rows; i++)
      EXPECT(dst[i] == static_cast<float>(static_cast<double>(base[i]) + static_cast<double>(ref[i])), "add %zu", i);
    // apply_pair == two applies.
    std::vector<float> o1(rows), o3(rows), r1(rows), r3(rows);
    apply_pair(l1, l3, x1, 1, o1, o3);
    l1.apply(x1, 1, r1);
    l3.apply(x1, 1, r3);
    EXPECT(o1 == r1 && o3 == r3, "pair(1) == two applies");
    std::vector<float> p1(tokens * rows), p3(tokens * rows), s1(tokens * rows), s3(tokens * rows);
    apply_pair(l1, l3, xm, tokens, p1, p3);
    l1.apply(xm, tokens, s1);
    l3.apply(xm, tokens, s3);
    EXPECT(p1 == s1 && p3 == s3, "pair(3) == two applies");
    EXPECT(throws<ShapeError>([&] { l1.apply(xm, 2, ym); }), "apply length assert");
  });
  run("output_head_q8", [&] {  // q8_apply, weights.rs:194-227
    const std::size_t n = 24, k = 64, tokens = 2;
    const auto w = gen(n * k, 7, 31, 15, 0.06f), x = gen(tokens * k, 5, 17, 8, 0.2f);
    Q8Matrix q8 = Q8Matrix::from_f32(ctx, w.data(), n, k);
    const auto blocks = q8.blocks();
    const OutputHead head(std::move(q8));
    std::vector<float> got(tokens * n);
    head.apply(x, tokens, got);
    // Expected: per token ActQ8 (always per block), then per row and block
    // acc = acc + ((f32(sum wq*aq) * f32(scale)) * sa) (weights.rs:200-215).
    const std::size_t bpr = k / BLOCK_SIZE;
    for (std::size_t t = 0; t < tokens; t++) {
      const ActQ8 a = ActQ8::quantize(ctx, std::vector<float>(x.begin() + t * k, x.begin() + (t + 1) * k));
      for (std::size_t r = 0; r < n; r++) {
        float acc = 0.0f;
        for (std::size_t b = 0; b < bpr; b++) {
          int32_t d = 0;
          for (std::size_t i = 0; i < BLOCK_SIZE; i++)
            d += static_cast<int32_t>(blocks[r * bpr + b].qs[i]) * a.qs[b * BLOCK_SIZE + i];
          const float t1 = static_cast<float>(d) * f16_to_f32(blocks[r * bpr + b].scale);
          acc = acc + t1 * a.scales[b];
        }
        const float g = got[t * n + r];
        EXPECT(std::fabs(static_cast<double>(g) - acc) <= 1e-4 + 1e-5 * std::fabs(acc), "token %zu row %zu: %.9g vs %.9g",
               t, r, g, acc);
      }
    }
  });

  // ---- crates/llm-core: Backend and Block ----------------------------------
  run("backend_alloc_write_read", [&] {
    const HipBackend be(ctx);
    EXPECT(std::string(be.name()) == "hip", "name");
    HipBuffer buf = be.alloc(1000);
    EXPECT(buf.len() == 1000, "len");
    const auto zero = buf.read();
    for (float v : zero) EXPECT(v == 0.0f, "zeroed");
    const auto src = gen(1000, 7, 101, 50, 0.01f);
    buf.write(src);
    EXPECT(buf.read() == src, "round trip");
  });
  run("ffn_block_forward", [&] {
    const std::size_t dim = 64, inter = 128, tokens = 2;
    const auto w1 = Q4Matrix::from_f32(ctx, gen(inter * dim, 7, 23, 11, 0.05f), inter, dim);
    const auto w3 = Q4Matrix::from_f32(ctx, gen(inter * dim, 11, 29, 14, 0.04f), inter, dim);
    const auto w2zero = Q4Matrix::from_f32(ctx, std::vector<float>(dim * inter, 0.0f), dim, inter);
    const auto w2 = Q4Matrix::from_f32(ctx, gen(dim * inter, 5, 19, 9, 0.03f), dim, inter);
    const std::vector<float> norm(dim, 1.0f);
    const HipFfnBlock zero_block(w1, w3, w2zero, norm, 1e-5f);
    EXPECT(zero_block.kind() == LayerKind::Ffn, "kind");
    const auto in = gen(tokens * dim, 3, 37, 18, 0.1f);
    std::vector<float> out(in.size());
    zero_block.forward(in, out);
    EXPECT(out == in, "W2 = 0 leaves the residual stream unchanged");
    const HipFfnBlock block(w1, w3, w2, norm, 1e-5f);
    block.forward(in, out);
    bool changed = false;
    for (std::size_t i = 0; i < out.size(); i++) {
      EXPECT(std::isfinite(out[i]), "finite %zu", i);
      changed = changed || out[i] != in[i];
    }
    EXPECT(changed, "the FFN adds to the residual stream");
    std::vector<float> bad(in.size() + 1);
    EXPECT(throws<ShapeError>([&] { block.forward(in, bad); }), "forward length assert");
  });

  std::printf("%s: %d failed\n", g_failed ? "FAILED" : "PASSED", g_failed);
  return g_failed ? 1 : 0;
}
