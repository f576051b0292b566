// Exact modular arithmetic for primes p < 2^50 on the gfx950 FP64 pipeline.
//
// Residues live in HBM as canonical uint64 in [0, p).  Inside kernels they are held as
// FP64 values that are exact integers ("signed-lazy" form): every value x satisfies
// |x| <= 2^52 and x is congruent to the residue.  FP64 FMA runs at full rate on gfx950
// (one wave64 instruction per SIMD every 4 cycles), while 64-bit integer multiplies are
// built from several 32-bit VALU multiplies; a lazy FP64 modular multiply measured 3.2x
// the throughput of a 32-bit-op Shoup multiply on MI355X, both bit-exact.
//
// Multiplication by a constant w in [0, p) with wp = fl(w / p):
//   q = rint(a * wp),  h = fl(a * w),  l = fma(a, w, -h)   (exact low part of a*w)
//   r = fma(-q, p, h) + l
// For |a| <= 2^52:  |fl(a*wp) - a*w/p| <= |a| 2^-52 <= 1, so |a*w - q*p| <= 1.5 p;
// |a*w| < 2^102 gives |l| <= 2^49, hence |h - q*p| <= 1.5p + 2^49 < 2^53 and the FMA is
// exact; the final sum is the exact integer a*w - q*p, so r == a*w (mod p), |r| <= 1.5 p.
// For |a| <= 2^51 the same argument gives |r| <= p.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hck {

constexpr int kLogN = 16;
constexpr int kN = 1 << kLogN;
constexpr double kTwo52 = 4503599627370496.0;  // 2^52

struct TwPair {
  double w;   // residue in [0, p) as an exact double
  double wp;  // fl(w / p)
};

__device__ __forceinline__ double u2d(uint64_t x) {
  // x < 2^52: place x in the mantissa of 2^52 and subtract 2^52 (exact).
  return __longlong_as_double((long long)(x | 0x4330000000000000ULL)) - kTwo52;
}

__device__ __forceinline__ uint64_t d2u(double x) {
  // x an integer in [0, 2^52): 2^52 + x has x as its mantissa field.
  return (uint64_t)__double_as_longlong(x + kTwo52) & 0x000FFFFFFFFFFFFFULL;
}

// a * w mod p, signed-lazy result (|r| <= 1.5 p for |a| <= 2^52, <= p for |a| <= 2^51).
__device__ __forceinline__ double mulc(double a, double w, double wp, double p) {
  const double q = __builtin_rint(a * wp);
  const double h = a * w;
  const double l = __builtin_fma(a, w, -h);
  return __builtin_fma(-q, p, h) + l;
}

__device__ __forceinline__ double mulc(double a, const TwPair& t, double p) {
  return mulc(a, t.w, t.wp, p);
}

// x mod p into [-p/2 - 1, p/2 + 1] for exact |x| <= 2^53 (pinv = fl(1/p)).
__device__ __forceinline__ double reduce(double x, double p, double pinv) {
  const double q = __builtin_rint(x * pinv);
  return __builtin_fma(-q, p, x);
}

// x mod p into [0, p) for exact |x| <= 2^53.
__device__ __forceinline__ double canon(double x, double p, double pinv) {
  const double q = __builtin_floor(x * pinv);
  double r = __builtin_fma(-q, p, x);
  r = r < 0.0 ? r + p : r;
  r = r >= p ? r - p : r;
  return r;
}

// a * b mod p for a residue b in [0, p) without a stored companion: the quotient is estimated
// from the product itself, q = rint(fl(a * b) * pinv).  fl(fl(a b) pinv) is within three
// roundings of X = a b / p, so |q - X| <= 0.5 + |X| 3 2^-53, and with |X| < |a| = A p,
//   |r| <= (0.5 + 0.375 A) p   (p < 2^50),
// the bound of mulc.  For |a| <= 2^52 (A <= 4): |h - q p| <= 2p + 2^49 < 2^53, so the FMA is
// exact and r == a b (mod p).  Twiddle tables store only w (8 bytes), and the product doubles as
// the quotient's input: 6 FP64 operations.
__device__ __forceinline__ double mulv(double a, double b, double p, double pinv) {
  const double h = a * b;
  const double q = __builtin_rint(h * pinv);
  const double l = __builtin_fma(a, b, -h);
  return __builtin_fma(-q, p, h) + l;
}

// Round half away from zero (llround semantics), written out: the library round() of this
// toolchain does not send negative ties away from zero.  trunc, one exact subtraction and two
// comparisons: no product to contract, so the result is the same in every translation unit.
__device__ __forceinline__ double round_away(double x) {
  double r = __builtin_trunc(x);
  const double d = x - r;  // exact
  if (d >= 0.5) r += 1.0;
  else if (d <= -0.5) r -= 1.0;
  return r;
}

}  // namespace hck
