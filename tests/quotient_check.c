/* Exhaustive check of the FP8 quantiser's quotient (musa-aiter_amd/csrc/kv_hip_common.h, quot_fast).
 *
 * For x with B significant bits (bf16: 8, fp16: 11, or any B <= 12) and s a float32 in [1, 2), the
 * kernel computes r = RN(1/s), q0 = RN(x*r), q1 = RN(q0 + RN_fma(x - s*q0)*r) and uses q1 as RN(x/s).
 * This program compares q1 with the correctly rounded quotient derived from exact integer division,
 * for every x significand in [2^(B-1), 2^B) and every s significand (or every `stride`-th one), and
 * prints the number of mismatches.  Scaling x and s by powers of two scales both sides exactly while
 * every intermediate stays normal, which the kernel guarantees by its [2^-60, 2^60] range check.
 *
 * usage: quotient_check <B> [stride]
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* RN(X / S * 2^(23 - (B - 1))) for integers X in [2^(B-1), 2^B), S in [2^23, 2^24), as a float. */
static float exact_quotient(uint64_t X, uint64_t S, int B) {
  const int up = 64 - B;                      /* quotient keeps 25+ significant bits */
  const unsigned __int128 n = (unsigned __int128)X << up;
  const unsigned __int128 q = n / S, rem = n % S;
  int len = 0;
  for (unsigned __int128 t = q; t; t >>= 1) ++len;
  const int drop = len - 24;
  uint64_t m = (uint64_t)(q >> drop);
  const int guard = (int)((q >> (drop - 1)) & 1);
  const int sticky = rem != 0 || (q & (((unsigned __int128)1 << (drop - 1)) - 1)) != 0;
  if (guard && (sticky || (m & 1))) ++m;     /* round half to even */
  return ldexpf((float)m, drop - up + 23 - (B - 1));
}

int main(int argc, char** argv) {
  const int B = argc > 1 ? atoi(argv[1]) : 8;
  const uint32_t stride = argc > 2 ? (uint32_t)atoi(argv[2]) : 1u;
  if (B < 1 || B > 12 || stride < 1) return 2;
  uint64_t total = 0, one_step_bad = 0, no_correction_bad = 0;
#pragma omp parallel for reduction(+ : total, one_step_bad, no_correction_bad) schedule(dynamic, 4)
  for (uint32_t xm = 0; xm < (1u << (B - 1)); ++xm) {
    const uint64_t X = (1ull << (B - 1)) | xm;
    const float x = ldexpf((float)X, -(B - 1));
    for (uint32_t sm = (xm * 2654435761u) % stride; sm < (1u << 23); sm += stride) {
      const uint64_t S = (1ull << 23) | sm;
      float s;
      const uint32_t sb = 0x3F800000u | sm;
      memcpy(&s, &sb, 4);
      const float want = exact_quotient(X, S, B);
      const float r = 1.0f / s;
      const float q0 = x * r;
      const float q1 = fmaf(fmaf(-s, q0, x), r, q0);
      ++total;
      one_step_bad += bits_of(q1) != bits_of(want);
      no_correction_bad += bits_of(q0) != bits_of(want);
    }
  }
  printf("bits=%d stride=%u cases=%llu one_step_mismatches=%llu no_correction_mismatches=%llu\n", B, stride,
         (unsigned long long)total, (unsigned long long)one_step_bad, (unsigned long long)no_correction_bad);
  return 0;
}
