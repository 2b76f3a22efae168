/* Exhaustive check behind the division-free e4m3 quantisation of the GPU
 * kernels (quot_abs and quot_signed in flashvsr-sm89-ops_amd/csrc/common.h).
 *
 * For every finite bf16 v (both signs) and every bf16 amax >= |v| (from +0 to
 * +inf), with s = fl(max(amax, 1e-12) / 448) and r = fl(1 / s):
 *   q0 = fl(|v| * r),  e = fma(-q0, min(s, FLT_MAX), |v|),  q1 = fma(e, r, q0)
 * and the code e4m3(q1) with v's sign bit or-ed in must equal the e4m3 code of
 * the IEEE quotient fl(v / s) (clamped to +-448), the quantisation contract.
 * The signed form (quot_signed in common.h) is checked on the same pairs:
 *   p0 = fl(v * r),  t = fma(p0, min(s, FLT_MAX), -v),  q = fma(t, -r, p0)
 * and e4m3(q), sign included, must equal the same code.
 * The one NaN case (v = +-inf with amax = inf) compares as NaN either way: the
 * sign of a NaN made by inf / inf differs between processors (x86 sets it).
 *
 * usage: fma_quotient_check [stride [offset]] -- amax patterns offset,
 * offset+stride, ... (stride 1 = exhaustive, ~1.07e9 pairs).  Prints the pair
 * count and the number of mismatches; exit status 1 on any mismatch. */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

uint8_t orc_e4m3_one(float f); /* oracle/fvsr_oracle.c */

static float bf16(uint32_t h) {
  uint32_t u = h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint8_t code_of(float q) {
  if (q == q) q = fminf(fmaxf(q, -448.0f), 448.0f);
  return orc_e4m3_one(q);
}

int main(int argc, char** argv) {
  const uint32_t stride = argc > 1 ? (uint32_t)atoi(argv[1]) : 1u;
  const uint32_t offset = argc > 2 ? (uint32_t)atoi(argv[2]) : 0u;
  long long pairs = 0, bad = 0;
  for (uint32_t ha = offset; ha <= 0x7f80u; ha += stride) {
    const float amax = bf16(ha);
    volatile float am = fmaxf(amax, 1e-12f);
    volatile float s = am / 448.0f;
    volatile float r = 1.0f / s;
    const float sc = fminf(s, FLT_MAX);
    for (uint32_t hv = 0; hv <= ha; ++hv) {
      const float a = bf16(hv);
      const float q0 = a * r;
      const float e = fmaf(-q0, sc, a);
      const float q1 = fmaf(e, r, q0);
      const uint8_t c = code_of(q1);
      for (uint32_t sg = 0; sg < 2; ++sg) {
        const float v = bf16(hv | (sg << 15));
        const uint8_t want = code_of(v / s), got = (uint8_t)(c | (sg << 7));
        /* quot_signed: the quotient on the signed value, the sign from the
         * conversion itself */
        const float p0 = v * r;
        const float t = fmaf(p0, sc, -v);
        const uint8_t got_signed = code_of(fmaf(t, -r, p0));
        ++pairs;
        const int both_nan = (want & 0x7f) == 0x7f && (got & 0x7f) == 0x7f;
        const int both_nan_signed = (want & 0x7f) == 0x7f && (got_signed & 0x7f) == 0x7f;
        if ((want != got && !both_nan) || (want != got_signed && !both_nan_signed)) {
          if (bad < 8)
            printf("mismatch amax=%a v=%a want=%02x got=%02x signed=%02x\n", amax, v, want, got,
                   got_signed);
          ++bad;
        }
      }
    }
  }
  printf("pairs %lld mismatches %lld\n", pairs, bad);
  return bad != 0;
}
