/* Exhaustive-in-the-divisor check of the quotient method of the append
 * quantizers (div_by_norm in kaplumba_amd/csrc/tq_append.h): for every f32
 * divisor significand d in [1, 2) and a sample of dividends x in [0.5, 2),
 *   r = RN(1/d), q = RN(x r), u = RN(q + RN_exact(x - q d) r)   (two fmas)
 * must equal the IEEE quotient RN(x / d) bit for bit.  Scaling x and d by
 * powers of two does not change the rounding while nothing leaves the normal
 * range, so this covers every normal quotient the kernels form.  It also
 * counts the plain RN(x r) mismatches, which must not be zero (the check
 * would otherwise be vacuous).  Prints "<pairs> <fma-refined mismatches>
 * <plain mismatches>".  Build: cc -O2 -mfma -ffp-contract=off -pthread. */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#define NTHREADS 8
#define PER_DIVISOR 64

static float bits_to_float(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t float_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

typedef struct { uint32_t m0, m1; long refined_bad, plain_bad; } span_t;

static void* run(void* arg) {
  span_t* s = (span_t*)arg;
  uint64_t state = 0x9e3779b97f4a7c15ull ^ s->m0;
  for (uint32_t m = s->m0; m < s->m1; ++m) {
    const float d = bits_to_float(0x3f800000u | m);
    const float r = 1.0f / d;
    for (int k = 0; k < PER_DIVISOR; ++k) {
      state ^= state << 13; state ^= state >> 7; state ^= state << 17;
      float x = bits_to_float(0x3f800000u | (uint32_t)(state & 0x7fffffu));
      if (k & 1) x *= 0.5f;
      const float want = x / d;
      const float q = x * r;
      const float u = fmaf(fmaf(-q, d, x), r, q);
      if (float_to_bits(u) != float_to_bits(want)) s->refined_bad++;
      if (float_to_bits(q) != float_to_bits(want)) s->plain_bad++;
    }
  }
  return 0;
}

int main(void) {
  pthread_t th[NTHREADS];
  span_t sp[NTHREADS];
  const uint32_t step = (1u << 23) / NTHREADS;
  for (int i = 0; i < NTHREADS; ++i) {
    sp[i].m0 = i * step;
    sp[i].m1 = (i + 1) * step;
    sp[i].refined_bad = sp[i].plain_bad = 0;
    pthread_create(&th[i], 0, run, &sp[i]);
  }
  long refined = 0, plain = 0;
  for (int i = 0; i < NTHREADS; ++i) {
    pthread_join(th[i], 0);
    refined += sp[i].refined_bad;
    plain += sp[i].plain_bad;
  }
  printf("%llu %ld %ld\n", (unsigned long long)(1u << 23) * PER_DIVISOR, refined, plain);
  return 0;
}
