/* Exhaustive check of the quotient the quantisation kernels use instead of a division
 * (quant_div in comfyui-kirei-vdn-h3_amd/csrc/common.h):
 *
 *   s = max(amax / qmax, 1e-12), r = 1 / s, q0 = x * r, q = copysign(fma(fma(-s, q0, x), r, q0), x)
 *
 * For every finite positive bf16 amax and every bf16 x with |x| <= amax, both signs, the int8
 * code clamp(rne(q), +-127) (qmax = 127) and the e4m3fn code of clamp(q, +-448) (qmax = 448) must
 * equal those of the correctly rounded x / s. The codes follow the reference's quantisation
 * (vdn_h3/fp8.py:41-54 `_quantize_rows_kernel`, :99-105).
 *
 *   quant_division_check [amax_stride [uncorrected]]
 *
 * amax_stride 1 (the default) visits all 32,639 amax values, 1.07e9 pairs per qmax (a few
 * minutes on one core); a larger stride visits every stride-th amax plus the largest one.
 * "uncorrected" checks the bare product x * r instead, which must show mismatches (the check's
 * own control).
 * Prints the counts and exits 1 on any mismatch. Build with -ffp-contract=off so that x * r and
 * the divisions stay single roundings. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* OCP e4m3fn code of a finite |x| <= 448, round to nearest even */
static uint32_t e4m3_code(float x) {
  const uint32_t sign = (to_bits(x) >> 24) & 0x80u;
  const float a = fabsf(x);
  if (a < 0.015625f) return sign | (uint32_t)rintf(a * 512.f); /* multiples of 2^-9 */
  uint32_t ua = to_bits(a);
  ua += 0x7ffffu + ((ua >> 20) & 1u);
  return sign | (((ua >> 23) - 120u) << 3) | ((ua >> 20) & 7u);
}

static uint32_t i8_code(float x) { return (uint32_t)(int32_t)fminf(fmaxf(rintf(x), -127.f), 127.f) & 0xffu; }

static uint32_t code_of(float qmax, float q) {
  return qmax == 127.f ? i8_code(q) : e4m3_code(fminf(fmaxf(q, -448.f), 448.f));
}

int main(int argc, char **argv) {
  const long stride = argc > 1 ? atol(argv[1]) : 1;
  const int uncorrected = argc > 2 && strcmp(argv[2], "uncorrected") == 0;
  if (stride < 1) {
    fprintf(stderr, "amax_stride must be >= 1\n");
    return 2;
  }
  const float qmaxes[2] = {127.f, 448.f};
  long long bad = 0;
  for (int k = 0; k < 2; ++k) {
    long long pairs = 0, mismatches = 0;
    for (uint32_t ab = 1;; ab = ab + stride < 0x7f7fu ? ab + stride : 0x7f7fu) {
      const float amax = from_bits(ab << 16);
      const float s = fmaxf(amax / qmaxes[k], 1e-12f), r = 1.f / s;
      for (uint32_t xb = 0; xb <= ab; ++xb) {
        for (int neg = 0; neg < 2; ++neg) {
          const float x = neg ? -from_bits(xb << 16) : from_bits(xb << 16);
          const float q0 = x * r;
          const float q = uncorrected ? q0 : copysignf(fmaf(fmaf(-s, q0, x), r, q0), x);
          ++pairs;
          if (code_of(qmaxes[k], q) != code_of(qmaxes[k], x / s)) {
            if (mismatches < 5) printf("  mismatch: qmax %g amax %a x %a\n", qmaxes[k], amax, x);
            ++mismatches;
          }
        }
      }
      if (ab == 0x7f7fu) break;
    }
    printf("qmax %g: %lld pairs, %lld code mismatches\n", qmaxes[k], pairs, mismatches);
    bad += mismatches;
  }
  return bad ? 1 : 0;
}
