/* CPU check of the quantize kernel's division-free int8 code (test
 * infrastructure, built and run by tests/test_quant_codes_cpu.py).
 *
 * Reference: rint(x / s) with an IEEE float32 division, as the reference's
 * quantize_rows computes it (torch.round(x / scale), _int8.py:87-97).
 * Kernel form (mode 1), on v = PRE * x with PRE = 1 or 16 (the butterfly's
 * factor), y = fl(1 / s) / PRE and sp = PRE * s:
 *   q = v * y;  r = fmaf(-q, sp, v);  code = rint(fmaf(r, y, q))
 * Mode 0 drops the correction (code = rint(q)) and mode 2 uses s instead of
 * sp in the residual: both are plausible mistakes and must report mismatches.
 *
 * Cases: row scales s = max(amax / 127, 1e-30) for amax over many binades,
 * exact multiples of 1/16 and random bit patterns; per scale, random x in
 * [-amax, amax], +-amax, and x within 3 ulps of (k + 1/2) s for every code k
 * (the quotients next to a rounding boundary). fmaf is the C library's, which
 * rounds once. Usage: markstein_check <scales> <mode>; prints the counts and
 * exits 1 on any code mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint64_t st = 88172645463325252ull;
static uint64_t rnd(void) {
  st ^= st << 13;
  st ^= st >> 7;
  st ^= st << 17;
  return st;
}
static float u01(void) { return (float)((rnd() >> 40) * (1.0 / 16777216.0)); }

static long tested = 0, bad = 0;
static int mode = 1;

static void check(float x, float s, int pre) {
  if (!isfinite(x * (float)pre)) return; /* outside the kernel's domain */
  volatile float xs = x, ss = s;
  const float ref = rintf(xs / ss);
  const float y = (1.0f / ss) * (1.0f / (float)pre), sp = s * (float)pre;
  const float v = x * (float)pre;
  const float q = v * y;
  float code;
  if (mode == 0) code = rintf(q);
  else if (mode == 2) code = rintf(fmaf(fmaf(-q, s, v), y, q));
  else code = rintf(fmaf(fmaf(-q, sp, v), y, q));
  ++tested;
  if (code != ref && !(code == 0.0f && ref == 0.0f)) {
    if (bad < 5) printf("mismatch: x=%a s=%a pre=%d ref=%g got=%g\n", x, s, pre, ref, code);
    ++bad;
  }
}

int main(int argc, char** argv) {
  const long n_s = argc > 1 ? atol(argv[1]) : 20000;
  mode = argc > 2 ? atoi(argv[2]) : 1;
  for (long i = 0; i < n_s; ++i) {
    float amax;
    switch (i % 4) {
      case 0: amax = u01() * 10.0f; break;
      case 1: amax = ldexpf(1.0f + u01(), (int)(rnd() % 200) - 100); break;
      case 2: amax = (float)(1 + rnd() % 254) / 16.0f; break;
      default: {
        const uint32_t b = (uint32_t)(rnd() & 0x7fffffffu);
        memcpy(&amax, &b, 4);
        if (!isfinite(amax)) amax = 1.0f;
      }
    }
    float s = amax / 127.0f;
    if (s < 1e-30f) s = 1e-30f;
    for (int pre = 1; pre <= 16; pre += 15) {
      for (int j = 0; j < 200; ++j) check((2.0f * u01() - 1.0f) * amax, s, pre);
      check(amax, s, pre);
      check(-amax, s, pre);
      for (int k = -128; k < 128; ++k) {
        const float x0 = ((float)k + 0.5f) * s;
        for (int d = -3; d <= 3; ++d) {
          float x = x0;
          for (int t = 0; t < abs(d); ++t) x = nextafterf(x, d > 0 ? INFINITY : -INFINITY);
          if (fabsf(x) <= amax) check(x, s, pre);
        }
      }
    }
  }
  printf("tested %ld code mismatches %ld\n", tested, bad);
  return bad != 0;
}
