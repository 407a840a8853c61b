/* Host check of the pooled-gradient division used by the dQ and dK/dV
 * epilogues (div_by_count in simple-vsa_amd/csrc/vsa_device.h): for every
 * finite bf16 value x and every count c in [1, 1024], q0 = x * RN(1/c)
 * followed by one FMA residual correction must equal the correctly rounded
 * x / c bit for bit (zeros compare by value).  Prints the mismatch count and
 * exits non-zero on any mismatch. */
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

int main(void) {
  long checked = 0, bad = 0;
  for (int c = 1; c <= 1024; ++c) {
    volatile float vc = (float)c;
    const float cf = vc;
    const float r = 1.0f / vc;
    for (uint32_t h = 0; h < 65536; ++h) {
      volatile float vx = bf16_bits_to_float((uint16_t)h);
      const float x = vx;
      if (!isfinite(x)) continue;
      const float ref = vx / vc;
      const float q0 = x * r;
      const float q = fmaf(fmaf(-q0, cf, x), r, q0);
      ++checked;
      if (memcmp(&ref, &q, 4) != 0 && !(ref == 0.0f && q == 0.0f)) {
        if (bad < 5) printf("mismatch x=%a c=%d div=%a fma=%a\n", x, c, ref, q);
        ++bad;
      }
    }
  }
  printf("checked %ld mismatches %ld\n", checked, bad);
  return bad != 0;
}
