/* Host check of the pooled-gradient division used by the dQ and dK/dV
 * epilogues (div_by_count in simple-vsa_amd/csrc/vsa_device.h): for every
 * finite bf16 value x, every finite fp16 value x (the two input dtypes of the
 * MFMA kernels) and every count c in [1, 1024], q0 = x * RN(1/c) followed by
 * one FMA residual correction must equal the correctly rounded x / c bit for
 * bit (zeros compare by value).  Prints the mismatch count per dtype and exits
 * non-zero on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float bf16_bits_to_float(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* IEEE binary16 bits -> float (exact: every fp16 value is an fp32 value). */
static float f16_bits_to_float(uint16_t h) {
  const int sign = h >> 15, exp = (h >> 10) & 31, man = h & 1023;
  float v;
  if (exp == 0) v = ldexpf((float)man, -24);                 /* zero / subnormal */
  else if (exp == 31) v = man ? NAN : INFINITY;
  else v = ldexpf((float)(man | 1024), exp - 25);
  return sign ? -v : v;
}

static int check(const char* name, float (*to_float)(uint16_t)) {
  long checked = 0, bad = 0;
  for (int c = 1; c <= 1024; ++c) {
    volatile float vc = (float)c;
    const float cf = vc;
    const float r = 1.0f / vc;
    for (uint32_t h = 0; h < 65536; ++h) {
      volatile float vx = to_float((uint16_t)h);
      const float x = vx;
      if (!isfinite(x)) continue;
      const float ref = vx / vc;
      const float q0 = x * r;
      const float q = fmaf(fmaf(-q0, cf, x), r, q0);
      ++checked;
      if (memcmp(&ref, &q, 4) != 0 && !(ref == 0.0f && q == 0.0f)) {
        if (bad < 5) printf("%s mismatch x=%a c=%d div=%a fma=%a\n", name, x, c, ref, q);
        ++bad;
      }
    }
  }
  printf("%s checked %ld mismatches %ld\n", name, checked, bad);
  return bad != 0;
}

int main(void) {
  const int bad_bf16 = check("bf16", bf16_bits_to_float);
  const int bad_f16 = check("fp16", f16_bits_to_float);
  return bad_bf16 || bad_f16;
}
