/*
 * C restatement of the reference's torch-free INT4 workload.  TEST
 * INFRASTRUCTURE ONLY: linked by tests/ and the native check harness as the
 * checker, never by the product library.
 *
 *   kfo_lcg_*          csrc/micro/sanitize_gemm.cu:21-25 (LCG, uniform())
 *   kfo_lcg_workload   csrc/micro/sanitize_gemm.cu:36-50 (draw order, q, scales, x)
 *   kfo_pack           csrc/micro/sanitize_gemm.cu:44-47 (host packer, kNibbleK)
 *   kfo_unpack         kernelforge/quantize.py:88-97
 *   kfo_dequant_fp16   kernelforge/quantize.py:112-113 (fp16(q * s), one RNE)
 *   kfo_ref_f64        csrc/micro/sanitize_gemm.cu:58-66 (double-precision sum)
 *   kfo_max_rel_err_f16 tests/test_gemm.py:36-45 (pass rule; the native check's)
 *   kfo_f32_to_f16     IEEE 754 binary32 -> binary16, round to nearest even,
 *                      written from the format definition (no library call)
 *
 * Pinned by tests/test_oracle.py against the numpy oracle (an independent
 * restatement), exhaustive fp16 conversion checks and the reference's KATs.
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, so no FMA contraction
 * changes the fp32 arithmetic of uniform() and the scale formula).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

static const int kNibbleK[8] = {0, 2, 4, 6, 1, 3, 5, 7}; /* k offset stored at nibble i */

uint16_t kfo_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exp = (x >> 23) & 0xFFu;
  const uint32_t man = x & 0x7FFFFFu;
  if (exp == 0xFFu) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u : 0u));
  const int e = (int)exp - 127 + 15; /* biased fp16 exponent */
  if (e >= 31) return (uint16_t)(sign | 0x7C00u);
  if (e >= 1) {
    uint32_t res = ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (res & 1u))) ++res; /* carry may reach inf: correct */
    return (uint16_t)(sign | res);
  }
  /* fp16 subnormal: count units of 2^-24.  value = sig * 2^(exp-150), sig 24 bits. */
  const int s = 14 - e;
  if (s > 25 || exp == 0) return (uint16_t)sign;
  const uint32_t sig = man | 0x800000u;
  uint32_t res = sig >> s;
  const uint32_t rem = sig & ((1u << s) - 1u);
  const uint32_t half = 1u << (s - 1);
  if (rem > half || (rem == half && (res & 1u))) ++res;
  return (uint16_t)(sign | res);
}

float kfo_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const int e = (h >> 10) & 0x1F;
  const uint32_t man = h & 0x3FFu;
  float v;
  if (e == 0)
    v = ldexpf((float)man, -24);
  else if (e == 31)
    v = man ? NAN : INFINITY;
  else
    v = ldexpf((float)(man | 0x400u), e - 25);
  uint32_t bits;
  memcpy(&bits, &v, 4);
  bits |= sign;
  memcpy(&v, &bits, 4);
  return v;
}

uint32_t kfo_lcg_next(uint32_t* s) { return *s = *s * 1664525u + 1013904223u; }

float kfo_lcg_uniform(uint32_t* s) { return ((float)(kfo_lcg_next(s) >> 8) / 16777216.f) * 2.f - 1.f; }

void kfo_pack(const int8_t* q, int n, int k, int32_t* packed) {
  for (int r = 0; r < n; ++r)
    for (int w = 0; w < k / 8; ++w) {
      uint32_t word = 0;
      for (int i = 0; i < 8; ++i)
        word |= (uint32_t)(q[(size_t)r * k + 8 * w + kNibbleK[i]] + 8) << (4 * i);
      packed[(size_t)r * (k / 8) + w] = (int32_t)word;
    }
}

void kfo_unpack(const int32_t* packed, int n, int k, int8_t* q) {
  for (int r = 0; r < n; ++r)
    for (int w = 0; w < k / 8; ++w) {
      const uint32_t word = (uint32_t)packed[(size_t)r * (k / 8) + w];
      for (int i = 0; i < 8; ++i)
        q[(size_t)r * k + 8 * w + kNibbleK[i]] = (int8_t)((int)((word >> (4 * i)) & 0xFu) - 8);
    }
}

/* Draw order of sanitize_gemm.cu: q (N*K), scales (N*K/G), then x for each M in ms.
 * x_concat receives the x matrices one after another (sum(ms) * K values). */
void kfo_lcg_workload(int group, int n, int k, const int* ms, int nms, int8_t* q, uint16_t* scales,
                      int32_t* packed, uint16_t* x_concat) {
  uint32_t s = (uint32_t)group;
  for (size_t i = 0; i < (size_t)n * k; ++i) q[i] = (int8_t)((int)(kfo_lcg_next(&s) >> 28) - 8);
  for (size_t i = 0; i < (size_t)n * (k / group); ++i)
    scales[i] = kfo_f32_to_f16(0.01f + 0.02f * fabsf(kfo_lcg_uniform(&s)));
  kfo_pack(q, n, k, packed);
  size_t off = 0;
  for (int j = 0; j < nms; ++j)
    for (size_t i = 0; i < (size_t)ms[j] * k; ++i) x_concat[off++] = kfo_f32_to_f16(kfo_lcg_uniform(&s));
}

void kfo_dequant_fp16(const int32_t* packed, const uint16_t* scales, int n, int k, int group, uint16_t* out) {
  for (int r = 0; r < n; ++r)
    for (int w = 0; w < k / 8; ++w) {
      const uint32_t word = (uint32_t)packed[(size_t)r * (k / 8) + w];
      const float s = kfo_f16_to_f32(scales[(size_t)r * (k / group) + (8 * w) / group]);
      for (int i = 0; i < 8; ++i) {
        const int q = (int)((word >> (4 * i)) & 0xFu) - 8;
        /* q * s is exact in fp32 (4-bit times 11-bit significand): one rounding to fp16. */
        out[(size_t)r * k + 8 * w + kNibbleK[i]] = kfo_f32_to_f16((float)q * s);
      }
    }
}

/* The pass rule of tests/test_gemm.py:36-45 (and sanitize_gemm.cu:84-86) on fp16 outputs:
 * max|y - ref| / max|ref| over all n elements, so that "result <= tol" decides as the
 * reference's "err <= tol * scale" does.  A NaN in y or ref gives NaN (fails every <= test;
 * fmax would drop it), an all-zero ref gives 0 for a zero error and +inf otherwise, n == 0
 * gives 0. */
double kfo_max_rel_err_f16(const uint16_t* y, const double* ref, size_t n) {
  double num = 0.0, den = 0.0;
  for (size_t i = 0; i < n; ++i) {
    const double d = fabs((double)kfo_f16_to_f32(y[i]) - ref[i]);
    const double a = fabs(ref[i]);
    if (isnan(d) || isnan(a)) return NAN;
    if (d > num) num = d;
    if (a > den) den = a;
  }
  if (den == 0.0) return num == 0.0 ? 0.0 : INFINITY;
  return num / den;
}

void kfo_ref_f64(const uint16_t* x, const int32_t* packed, const uint16_t* scales, int m, int n, int k,
                 int group, double* y) {
  for (int i = 0; i < m; ++i)
    for (int r = 0; r < n; ++r) {
      double acc = 0.0;
      for (int w = 0; w < k / 8; ++w) {
        const uint32_t word = (uint32_t)packed[(size_t)r * (k / 8) + w];
        const double s = (double)kfo_f16_to_f32(scales[(size_t)r * (k / group) + (8 * w) / group]);
        for (int p = 0; p < 8; ++p) {
          const int kk = 8 * w + kNibbleK[p];
          const int q = (int)((word >> (4 * p)) & 0xFu) - 8;
          acc += (double)kfo_f16_to_f32(x[(size_t)i * k + kk]) * q * s;
        }
      }
      y[(size_t)i * n + r] = acc;
    }
}
