/*
 * Exhaustive CPU proof of the two fast divisions used by the device ActQ8
 * quantizer (llmhost_amd/csrc/lgh_device.h, act_quant_group8):
 *
 *   div127(a)  = fma(fma(-q0, 127, a), y, q0),  q0 = a * y,  y = RN(1/127)
 *                must equal RN(a / 127) for every finite a >= 0;
 *   recip(s)   = fma(fma(-s, y0, 1), y0, y0)    for y0 either faithful
 *                neighbour of 1/s (what a 1-ulp v_rcp_f32 may return)
 *                must equal RN(1 / s) for every s in [2^-126, 2^126).
 *
 * Correct rounding is decided exactly: with q a candidate, the remainders
 * a - 127*q (resp. 1 - s*q) of q and of its two float neighbours are exact
 * in double, so RN is the neighbour with the smallest |remainder| (ties to
 * the even significand).  Built and run by tests/test_fastquant.py.
 * Prints "ok <count>" or the first failing input.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float f_of(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static uint32_t b_of(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* Is q = RN(num / den)?  Exact remainders: num, den, q are floats, so
 * den*q fits in 48 bits and num - den*q is exact in double when q is
 * within a few ulps of num/den (checked by the caller's construction). */
static int is_rn_quot(double num, double den, float q) {
  float lo = nextafterf(q, 0.0f), hi = nextafterf(q, INFINITY);
  double r = fabs(num - den * (double)q);
  double rl = fabs(num - den * (double)lo);
  double rh = fabs(num - den * (double)hi);
  if (q == 0.0f) rl = INFINITY;
  if (r < rl && r < rh) return 1;
  if (r > rl || r > rh) return 0;
  return (b_of(q) & 1u) == 0; /* tie: the even one wins */
}

int main(void) {
  const float y = 1.0f / 127.0f;
  if (b_of(y) != 0x3C010204u) { printf("RN(1/127) bits %08x\n", b_of(y)); return 1; }
  int64_t bad_div = -1, bad_rcp = -1;
  /* div127 over every finite a >= 0 (bits 0x00000000 .. 0x7F7FFFFF). */
#pragma omp parallel for schedule(static, 1 << 20) reduction(max : bad_div)
  for (int64_t bb = 0; bb <= 0x7F7FFFFF; bb++) {
    float a = f_of((uint32_t)bb);
    float q0 = a * y;
    float r = fmaf(-q0, 127.0f, a);
    float q = fmaf(r, y, q0);
    if (!is_rn_quot((double)a, 127.0, q) && bb > bad_div) bad_div = bb;
  }
  if (bad_div >= 0) {
    printf("div127 fails at a=%a (bits %08llx)\n", f_of((uint32_t)bad_div), (long long)bad_div);
    return 1;
  }
  /* recip over normal s with 1/s normal: [2^-126, 2^126), except the
   * all-ones significand, which the device routes to the IEEE division
   * (the Newton step from the lower neighbour lands exactly on a tie there). */
#pragma omp parallel for schedule(static, 1 << 20) reduction(max : bad_rcp)
  for (int64_t bb = 0x00800000; bb < 0x7E800000; bb++) {
    uint32_t b = (uint32_t)bb;
    if ((b & 0x7FFFFFu) == 0x7FFFFFu) continue;
    float s = f_of(b);
    double inv = 1.0 / (double)s;           /* only to find the two faithful neighbours */
    float c = (float)inv;
    float cand[2];
    if ((double)c > inv) { cand[0] = nextafterf(c, 0.0f); cand[1] = c; }
    else if ((double)c < inv) { cand[0] = c; cand[1] = nextafterf(c, INFINITY); }
    else { cand[0] = c; cand[1] = c; }      /* 1/s exact: a 1-ulp rcp returns it */
    for (int k = 0; k < 2; k++) {
      float y0 = cand[k];
      float e = fmaf(-s, y0, 1.0f);
      float q = fmaf(e, y0, y0);
      if (!is_rn_quot(1.0, (double)s, q) && bb > bad_rcp) bad_rcp = bb;
    }
  }
  if (bad_rcp >= 0) {
    printf("recip fails at s=%a (bits %08llx)\n", f_of((uint32_t)bad_rcp), (long long)bad_rcp);
    return 1;
  }
  /* quant_code's rounding: for every float y with |y| <= 130, i = trunc(2y)
   * (2y is exact) and (i + (i >> 31) + 1) >> 1 == roundf(y) (C's roundf
   * rounds half away from zero, like Rust's f32::round). */
  int64_t bad_rnd = -1;
#pragma omp parallel for schedule(static, 1 << 20) reduction(max : bad_rnd)
  for (int64_t bb = 0; bb <= 0x43020000; bb++) { /* 0x43020000 = 130.0f */
    for (int sgn = 0; sgn < 2; sgn++) {
      float yv = f_of((uint32_t)bb | (sgn ? 0x80000000u : 0u));
      int i = (int)(2.0f * yv);
      int q = (i + (i >> 31) + 1) >> 1;
      if ((float)q != roundf(yv) && bb > bad_rnd) bad_rnd = bb;
    }
  }
  if (bad_rnd >= 0) {
    printf("rounding fails at |y|=%a\n", f_of((uint32_t)bad_rnd));
    return 1;
  }
  printf("ok\n");
  return 0;
}
