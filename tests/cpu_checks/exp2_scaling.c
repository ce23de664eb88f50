/* exp2_scaling.c -- the softmax kernels' exp2 polynomials (mx_common.hpp:
 * exp2_poly / exp2_poly_neg, exp2_poly_aie / exp2_poly_aie_neg) scale their
 * result by 2^k with ldexp instead of a multiply by 2^k built in the exponent
 * field. This checks that both give the same bits for floats x in [-120, 0]
 * (every STRIDE-th bit pattern; STRIDE 1 is every float there), in the fused
 * form (fmaf Horner) and the unfused one (a rounded multiply, then a rounded
 * add). Usage: exp2_scaling STRIDE. Prints the count checked; exit 1 on the
 * first difference. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
/* volatile: each operation rounded on its own, as the device's mul_rn and add_rn */
static float mul_rn(float a, float b) { volatile float r = a * b; return r; }
static float add_rn(float a, float b) { volatile float r = a + b; return r; }

static const float C[8] = {1.5483275463e-05f, 1.5669833174e-04f, 1.3331825236e-03f,
                           9.6164605538e-03f, 5.5504156855e-02f, 2.4022684109e-01f,
                           6.9314717694e-01f, 9.9999998955e-01f};

static float poly(float f, int fused) {
  float p = C[0];
  for (int i = 1; i < 8; ++i) p = fused ? fmaf(p, f, C[i]) : add_rn(mul_rn(p, f), C[i]);
  return p;
}

int main(int argc, char **argv) {
  const uint32_t stride = argc > 1 ? (uint32_t)strtoul(argv[1], NULL, 10) : 1u;
  const uint32_t hi = f2u(120.0f);
  unsigned long long n = 0;
  for (int fused = 0; fused < 2; ++fused) {
    for (uint32_t m = 0; m <= hi; m += stride) {
      const float x = u2f(0x80000000u | m);
      const int k = (int)x;
      const float f = fused ? x - (float)k : add_rn(x, -(float)k);
      const float p = poly(f, fused);
      const float bits = mul_rn(p, u2f((uint32_t)(k + 127) << 23));
      const float ld = ldexpf(p, k);
      if (f2u(bits) != f2u(ld)) {
        printf("differ: %s x=%a bits=%a ldexp=%a\n", fused ? "fused" : "unfused", x, bits, ld);
        return 1;
      }
      ++n;
    }
  }
  printf("%llu\n", n);
  return 0;
}
