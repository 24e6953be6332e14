// cos of an fp32 argument, evaluated in float64 (time-encoding hot loop).
//
// Reduction x = k*pi + r with k = rint(x/pi) obtained by adding 1.5*2^52 (the
// low mantissa bit of the sum is k's parity), r by Cody-Waite with a two-term
// pi (error ~1e-16 for |x| < 2^40), then cos(r) on |r| <= pi/2 by a degree-5
// polynomial in r^2 and cos(x) = (-1)^k cos(r).  The coefficients are a
// near-minimax fit computed for this library (iterated reweighted least
// squares on Chebyshev nodes, max error 2.2e-10 on |r| <= pi/2 * 1.0001).
// Callers route |x| >= 2^40 to cos_slow.  The same source compiles for the
// host, which is how the CPU tests check it against float64 cos.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

namespace tgx {

constexpr double kInvPi = 0.3183098861837907;
constexpr double kPiHi = 3.141592653589793;
constexpr double kPiLo = 1.2246467991473532e-16;
constexpr double kRoundMagic = 6755399441055744.0;  // 1.5 * 2^52
constexpr double kA0 = 0.999999999780424;
constexpr double kA1 = -0.49999999357852726;
constexpr double kA2 = 0.0416666362342501;
constexpr double kA3 = -0.0013888361089159438;
constexpr double kA4 = 2.4760145078500364e-05;
constexpr double kA5 = -2.605120135781943e-07;
constexpr float kBigArg = 1099511627776.0f;  // 2^40

__host__ __device__ inline float cos_fast(float x) {
  const double xd = static_cast<double>(x);
  const double t = fma(xd, kInvPi, kRoundMagic);
  const double k = t - kRoundMagic;
  const uint32_t parity = static_cast<uint32_t>(__builtin_bit_cast(uint64_t, t)) << 31;
  double r = fma(-k, kPiHi, xd);
  r = fma(-k, kPiLo, r);
  const double z = r * r;
  double p = fma(z, kA5, kA4);
  p = fma(p, z, kA3);
  p = fma(p, z, kA2);
  p = fma(p, z, kA1);
  p = fma(p, z, kA0);
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, static_cast<float>(p)) ^ parity);
}

__host__ __device__ inline float cos_slow(float x) {
  return static_cast<float>(cos(static_cast<double>(x)));
}

__host__ __device__ inline float cos_any(float x) {
  return fabsf(x) < kBigArg ? cos_fast(x) : cos_slow(x);
}

}  // namespace tgx
