// Cosine of an fp32 argument for the fused time encoding.
//
// cos(x) = cos(2 pi f) with f the signed fractional part of x / (2 pi), f in
// [-1/2, 1/2], computed in float64 by rev_frac.  The device then evaluates
// cos(2 pi f) with v_cos_f32, whose argument is in revolutions (max abs error
// 1.3e-7 measured on gfx950 over every fp32 |f| <= 1/2).
//
//  * |x| < 2^29 (rev_frac_small): u = x * (1/(2 pi)) rounded once in float64, so
//    |u - x/(2 pi)| <= 2 |u| 2^-53 < 2e-8 revolutions; f = u - rint(u) exactly.
//  * |x| >= 2^29: x = M 2^E with an integer |M| < 2^24 and E in [6, 104], so
//    frac(x / (2 pi)) = frac(M F_E) with F_E = frac(2^E / (2 pi)) held as a
//    double-double hi + lo (tgx_rev_table.h, generated from a 400-bit pi).
//    p = M hi and its rounding error e = fma(M, hi, -p) are exact, so
//    f = (p - rint(p)) + (e + M lo) is within ~2^-80 of the true fraction.
//  * non-finite x gives NaN.
//
// Worst case on the device: 2e-8 rev (reduction) + 2^-27 rev (f rounded to fp32)
// + 1.3e-7 (v_cos_f32), i.e. below 3.5e-7 absolute.  rev_frac is plain float64
// arithmetic and also builds for the host, where the CPU tests compare
// cos(2 pi f) with libm's cos(x).
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "tgx_rev_table.h"

namespace tgx {

constexpr double kInv2Pi = 0.15915494309189535;
constexpr float kRevArg = 536870912.0f;  // 2^29

__host__ __device__ inline double rev_frac_small(float x) {
  const double u = static_cast<double>(x) * kInv2Pi;
  return u - rint(u);
}

// tab: an array initialised with TGX_REV_TABLE_ROWS
__host__ __device__ inline double rev_frac(float x, const double (*tab)[2]) {
  if (fabsf(x) < kRevArg) return rev_frac_small(x);
  const uint32_t bits = __builtin_bit_cast(uint32_t, x);
  const int ex = static_cast<int>((bits >> 23) & 0xffu);
  if (ex == 0xff) return static_cast<double>(x - x);  // inf or NaN -> NaN
  const int E = ex - 150;                             // x = M * 2^E
  double M = static_cast<double>(static_cast<int32_t>((bits & 0x7fffffu) | 0x800000u));
  if (bits >> 31) M = -M;
  const double hi = tab[E - TGX_REV_TABLE_MIN_EXP][0];
  const double lo = tab[E - TGX_REV_TABLE_MIN_EXP][1];
  const double p = M * hi;
  const double e = fma(M, hi, -p);
  const double f = (p - rint(p)) + fma(M, lo, e);
  return f - rint(f);
}

}  // namespace tgx
