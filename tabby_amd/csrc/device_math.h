// Device-side arithmetic shared by the sampler kernels: orderable keys for f32 logits and
// the f64 exp that the sampling tail uses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tabby {

// ---------------------------------------------------------------------------------------
// Orderable keys. key(a) > key(b) exactly when a > b for non-NaN f32, with -0 mapped onto
// +0 first (x + 0.0f is +0 for x = -0 and x otherwise), because the reference's comparator
// (src/engine/sampler.ts:28) treats the two zeros as equal and falls back to the index.
// -inf maps to kNegInfKey, the smallest key any logit can have; padding lanes use it too.
// ---------------------------------------------------------------------------------------
constexpr uint32_t kNegInfKey = 0x007FFFFFu;

__device__ __forceinline__ uint32_t key_of(float x) {
  const uint32_t b = __float_as_uint(x + 0.0f);
  return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}

__device__ __forceinline__ float value_of(uint32_t k) {
  return __uint_as_float(k ^ (~(uint32_t)((int32_t)k >> 31) | 0x80000000u));
}

// Composite sort key: value key in the high word, ~index in the low word, so a larger
// composite is a larger value or, for equal values, a lower index. Every composite of a row
// is distinct, which is what makes the selection exact without a separate tie pass.
__device__ __forceinline__ uint64_t composite(uint32_t key, uint32_t index) {
  return ((uint64_t)key << 32) | (uint32_t)~index;
}
__device__ __forceinline__ uint32_t composite_index(uint64_t c) { return ~(uint32_t)c; }
__device__ __forceinline__ uint32_t composite_key(uint64_t c) { return (uint32_t)(c >> 32); }

// ---------------------------------------------------------------------------------------
// exp(x) in f64 by the method of Sun fdlibm's e_exp.c (Copyright (C) 1993 Sun Microsystems;
// freely distributable) -- the method V8 ships as Math.exp, which the reference's
// sampleFromTopK calls (src/engine/sampler.ts:156,170). x = k*ln2 + r with ln2 split into a
// high part with 32 significant bits (so k*ln2_hi is exact) and a low part; a degree-5 Remez
// polynomial gives R(r^2) ~ r*(e^r+1)/(e^r-1); then exp(r) = 1 + 2r/(R - r) and an exact
// scaling by 2^k. Contraction is off: each operation must round once, in this order, to
// reproduce V8 to the last bit.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ double fdlibm_exp_inline(double x) {
#pragma clang fp contract(off)
  const double ln2_hi = 6.93147180369123816490e-01;
  const double ln2_lo = 1.90821492927058770002e-10;
  const double inv_ln2 = 1.44269504088896338700e+00;
  const double p1 = 1.66666666666666019037e-01;
  const double p2 = -2.77777777770155933842e-03;
  const double p3 = 6.61375632143793436117e-05;
  const double p4 = -1.65339022054652515390e-06;
  const double p5 = 4.13813679705723846039e-08;

  const uint64_t bits = (uint64_t)__double_as_longlong(x);
  uint32_t hx = (uint32_t)(bits >> 32);
  const bool negative = (hx >> 31) != 0;
  hx &= 0x7fffffffu;

  if (hx >= 0x40862e42u) {  // |x| >= 709.78
    if (hx >= 0x7ff00000u) {
      if (((hx & 0xfffffu) | (uint32_t)bits) != 0u) return x + x;  // NaN
      return negative ? 0.0 : x;                                    // exp(+-inf)
    }
    if (x > 7.09782712893383973096e+02) return __longlong_as_double(0x7ff0000000000000LL);
    if (x < -7.45133219101941108420e+02) return 0.0;
  }

  double hi = 0.0, lo = 0.0;
  int k = 0;
  if (hx > 0x3fd62e42u) {    // |x| > ln2/2
    if (hx < 0x3ff0a2b2u) {  // |x| < 1.5 ln2
      if (x == 1.0) return 2.718281828459045;
      if (negative) {
        hi = x + ln2_hi;
        lo = -ln2_lo;
        k = -1;
      } else {
        hi = x - ln2_hi;
        lo = ln2_lo;
        k = 1;
      }
    } else {
      k = (int)(inv_ln2 * x + (negative ? -0.5 : 0.5));
      const double t = (double)k;
      hi = x - t * ln2_hi;
      lo = t * ln2_lo;
    }
    x = hi - lo;
  } else if (hx < 0x3e300000u) {  // |x| < 2^-28
    return 1.0 + x;
  }

  const double t = x * x;
  const double c = x - t * (p1 + t * (p2 + t * (p3 + t * (p4 + t * p5))));
  if (k == 0) return 1.0 - ((x * c) / (c - 2.0) - x);
  const double y = 1.0 - ((lo - (x * c) / (2.0 - c)) - hi);
  if (k >= -1021) {
    if (k == 1024) return y * 2.0 * 8.98846567431157953865e+307;
    return y * __longlong_as_double((long long)((uint64_t)(0x3ff00000u + ((uint32_t)k << 20)) << 32));
  }
  return y * __longlong_as_double(
                 (long long)((uint64_t)(0x3ff00000u + ((uint32_t)(k + 1000) << 20)) << 32)) *
         9.33263618503218878990e-302;
}

// exp(x) for x <= 0 to within a few ulp, without branches: x = k*ln2 + r with the Cody-Waite
// split of ln2 above (k*ln2_hi exact), e^r by its Taylor series to degree 12 evaluated in
// Estrin's form (|r| <= ln2/2, truncation below 2^-52 relative), then an exact scaling by 2^k
// (ldexp, gradual underflow). Not V8's bits: for sums and probabilities whose bits the
// callers do not need, or that they check against a margin.
__device__ __forceinline__ double exp_nonpos(double x) {
  x = fmax(x, -746.0);  // exp(-746) rounds to 0; -inf too
  const double k = __builtin_rint(x * 1.44269504088896338700e+00);
  double r = __builtin_fma(-k, 6.93147180369123816490e-01, x);
  r = __builtin_fma(-k, 1.90821492927058770002e-10, r);
  const double r2 = r * r, r4 = r2 * r2, r8 = r4 * r4;
  const double p01 = 1.0 + r;
  const double p23 = __builtin_fma(r, 1.66666666666666666667e-01, 5.0e-01);
  const double p45 = __builtin_fma(r, 8.33333333333333333333e-03, 4.16666666666666666667e-02);
  const double p67 = __builtin_fma(r, 1.98412698412698412698e-04, 1.38888888888888888889e-03);
  const double p89 = __builtin_fma(r, 2.75573192239858906526e-06, 2.48015873015873015873e-05);
  const double pab = __builtin_fma(r, 2.50521083854417187751e-08, 2.75573192239858906526e-07);
  const double q0 = __builtin_fma(r2, p23, p01);
  const double q1 = __builtin_fma(r2, p67, p45);
  const double q2 = __builtin_fma(r2, pab, p89);
  const double q3 = 2.08767569878680989792e-09;  // 1/12!
  const double s0 = __builtin_fma(r4, q1, q0);
  const double s1 = __builtin_fma(r4, q3, q2);
  return __builtin_ldexp(__builtin_fma(r8, s1, s0), (int)k);
}

// fround(Math.exp(x)) for x <= 0 (or NaN): V8's exp rounded to f32, the exps of the reference's
// f32 softmax (src/reference/cpu.ts:253). exp_nonpos gives e^x within a few f64 ulps, and
// V8's fdlibm exp is within one; both round to the same f32 unless e^x lies within their
// combined error of a rounding boundary of f32 (the midpoint between two neighbours). So the
// fast value is kept when its distance to that boundary exceeds 2^-44 of it -- thousands of
// times either error bound -- and otherwise (about one argument in 2^20) fdlibm_exp decides.
__device__ __forceinline__ float exp_to_f32(float x) {
  if (x != x) return x;
  const double r = exp_nonpos((double)x);
  const float y = (float)r;
  const double res = r - (double)y;  // exact: r and y are within half an f32 ulp
  const uint32_t yb = __float_as_uint(y);
  const int e = (int)(yb >> 23);
  double half = __builtin_ldexp(1.0, (e > 1 ? e : 1) - 151);  // half the f32 ulp above y
  if (res < 0.0 && (yb & 0x7fffffu) == 0u && e > 1) half *= 0.5;  // below a power of two
  if (__builtin_fabs(res) < half - r * 0x1p-44) return y;
  return (float)fdlibm_exp_inline((double)x);
}

// Out-of-line form for call sites where code size matters more than the call.
__device__ __noinline__ double fdlibm_exp(double x) { return fdlibm_exp_inline(x); }

}  // namespace tabby
