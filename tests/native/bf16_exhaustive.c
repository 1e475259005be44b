/* Test helper (not product code): counts the float bit patterns, of all
 * 2^32, on which a given float -> bf16 conversion differs from
 * round-to-nearest-even stated from its definition - the bf16 neighbour
 * nearer in exact (double) arithmetic, ties to the even mantissa, NaN kept
 * a quiet NaN with its sign and upper payload bits, overflow past the
 * largest finite bf16 rounding to infinity as IEEE does. */
#include <math.h>
#include <stdint.h>
#include <string.h>

typedef uint16_t (*conv_fn)(float);

static double bits_to_double(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return (double)f;
}

static uint16_t rne_by_definition(uint32_t u) {
  if ((u & 0x7f800000u) == 0x7f800000u) {                /* inf or NaN */
    if (u & 0x007fffffu) return (uint16_t)((u >> 16) | 0x0040u);
    return (uint16_t)(u >> 16);
  }
  const uint32_t lo = u & 0xffff0000u;                   /* truncation toward zero */
  const uint32_t hi = lo + 0x10000u;                     /* next bf16 away from zero */
  const double x = fabs(bits_to_double(u));
  const double flo = fabs(bits_to_double(lo));
  /* hi may be the infinity pattern: its distance is then measured to
   * 2^128, the value the exponent step would reach (IEEE overflow rule). */
  const double fhi = ((hi & 0x7f800000u) == 0x7f800000u) ? ldexp(1.0, 128) : fabs(bits_to_double(hi));
  const double dlo = x - flo, dhi = fhi - x;
  if (dhi < dlo || (dhi == dlo && ((lo >> 16) & 1u))) return (uint16_t)(hi >> 16);
  return (uint16_t)(lo >> 16);
}

/* Mismatches of f over the patterns [first, first + count). */
int64_t bf16_mismatches(conv_fn f, uint64_t first, uint64_t count) {
  int64_t bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
  for (int64_t i = 0; i < (int64_t)count; ++i) {
    const uint32_t u = (uint32_t)(first + (uint64_t)i);
    float x;
    memcpy(&x, &u, 4);
    if (f(x) != rne_by_definition(u)) ++bad;
  }
  return bad;
}
