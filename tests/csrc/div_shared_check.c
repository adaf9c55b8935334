/* CPU check of the division the row kernels use for x / scale:
 *   y = x * r;  e = fma(y, s, -x);  q = fma(-e, r, y),  r = RN(1/s)
 * must equal the IEEE quotient x / s for every x with |x| <= amax,
 * s = RN(amax / 448), whenever the quotient is large enough to change an
 * e4m3 code (|x / s| >= 2^-12; smaller quotients all encode to a signed zero),
 * and must carry the quotient's sign always (x = -0 gives -0).
 * x and amax are bf16 values (the rows are bf16 before quantisation).
 * Usage: div_shared_check N SEED -> prints "n=<checked> bad=<mismatches>". */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint64_t st;
static uint64_t next(void) { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return st; }
static float bf16(uint32_t bits) { uint32_t u = bits << 16; float f; memcpy(&f, &u, 4); return f; }

int main(int argc, char** argv) {
  long n = argc > 1 ? atol(argv[1]) : 10000000;
  st = argc > 2 ? strtoull(argv[2], 0, 10) : 88172645463325252ull;
  long bad = 0, checked = 0;
  for (long i = 0; i < n; ++i) {
    float x = bf16(next() & 0xFFFF), a = bf16(next() & 0x7FFF);
    if (!isfinite(x) || !isfinite(a)) continue;
    if (fabsf(x) > a) a = fabsf(x);
    if (a < 1e-12f) a = 1e-12f;
    float s = a / 448.0f;
    float r = 1.0f / s;
    float y = x * r;
    float e = fmaf(y, s, -x);
    float q = fmaf(-e, r, y);
    float t = x / s;
    ++checked;
    if (fabsf(t) >= 0x1p-12f && memcmp(&q, &t, 4) != 0) ++bad;
    if (signbit(q) != signbit(t)) ++bad;
  }
  printf("n=%ld bad=%ld\n", checked, bad);
  return bad != 0;
}
