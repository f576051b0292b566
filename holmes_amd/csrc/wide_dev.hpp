// Device arithmetic of the wide-prime path (64-bit canonical residues, primes below 2^61), shared by
// wide.hip (the separate-launch kernels) and wide_fused.hip (the fused key switch).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "modarith64.hpp"
#include "wide.hpp"

namespace hck {

__device__ __forceinline__ uint64_t wadd(uint64_t a, uint64_t b, uint64_t p) {
  const uint64_t s = a + b;
  return s >= p ? s - p : s;
}
__device__ __forceinline__ uint64_t wsub(uint64_t a, uint64_t b, uint64_t p) { return a >= b ? a - b : a + p - b; }
// a * w mod p, canonical, for any 64-bit a (Shoup: the lazy result lies in [0, 2p)).
__device__ __forceinline__ uint64_t wmulc(uint64_t a, uint64_t w, uint64_t ws, uint64_t p) {
  const uint64_t r = mulshoup_lazy(a, w, ws, p);
  return r >= p ? r - p : r;
}
__device__ __forceinline__ Barrett64 wbar(const WideTables& T, int pi) { return Barrett64{T.p[pi], T.mu[pi], T.w[pi]}; }
// canonical representative of a lazy word below 2p / below 4p
__device__ __forceinline__ uint64_t wcanon2(uint64_t x, uint64_t p) { return x >= p ? x - p : x; }
__device__ __forceinline__ uint64_t wcanon4(uint64_t x, uint64_t p) { return wcanon2(x >= 2 * p ? x - 2 * p : x, p); }
__device__ __forceinline__ uint64_t wcanon8(uint64_t x, uint64_t p) { return wcanon4(x >= 4 * p ? x - 4 * p : x, p); }

// x k 2^-64 mod p below 2p, for x k < 2^64 p (Montgomery; mneg = -p^-1 mod 2^64): t + m p is a
// multiple of 2^64 for m = t mneg, and its low words add up to 2^64 exactly when t's low word is not 0.
// Sums of such products are brought back by one product with 2^64 mod p (WideTables::r64).
__device__ __forceinline__ uint64_t wmont(uint64_t x, uint64_t k, uint64_t p, uint64_t mneg) {
  const u128_t t = (u128_t)x * k;
  const uint64_t tl = (uint64_t)t, th = (uint64_t)(t >> 64);
  const uint64_t m = tl * mneg;
  return th + (uint64_t)(((u128_t)m * p) >> 64) + (tl != 0 ? 1 : 0);
}

// t mod p for t < p 2^64: Montgomery's reduction (t 2^-64, below 2p), then the product with 2^64 mod p
// (r = 2^64 mod p, rs its Shoup companion); canonical result.
__device__ __forceinline__ uint64_t wfold128(u128_t t, uint64_t p, uint64_t mneg, uint64_t r, uint64_t rs) {
  const uint64_t tl = (uint64_t)t, th = (uint64_t)(t >> 64);
  const uint64_t m = tl * mneg;
  const uint64_t u = th + (uint64_t)(((u128_t)m * p) >> 64) + (tl != 0 ? 1 : 0);
  return wmulc(u, r, rs, p);
}

// The int8 matrix-core base conversion's operands and fold (wide.hip: wk_mconv, wide_fused.hip).
// Each source residue is centered (|ybar| < b / 2 < 2^60) and written as the 64-bit word of its eight
// balanced base-256 digits (byte a = d_a + 128 of ybar + 0x80..80; the XOR turns each byte into d_a as
// int8).  One v_mfma_i32_16x16x64_i8 per output digit c gives the byte-position sums C_c of the
// conversion (|C_c| <= 64 * 128^2 = 2^20); wfold combines the eight of one target into its residue.
typedef int wv4i __attribute__((ext_vector_type(4)));
constexpr uint64_t kDigitBias = 0x8080808080808080ULL;

__device__ __forceinline__ uint64_t wdigits(uint64_t v, uint64_t b) {
  const long long y = 2 * v > b ? (long long)v - (long long)b : (long long)v;  // centered
  return ((uint64_t)y + kDigitBias) ^ kDigitBias;
}

__device__ __forceinline__ uint64_t wfold(const wv4i (&a)[8], int r, uint64_t t, double tinv) {
  // byte-position pairs (|.| < 2^29), x = p0 + p1 2^16 + p2 2^32 + p3 2^48 with |x| < 2^76.01
  const int p0 = a[0][r] + a[1][r] * 256, p1 = a[2][r] + a[3][r] * 256;
  const int p2 = a[4][r] + a[5][r] * 256, p3 = a[6][r] + a[7][r] * 256;
  // the quotient from a double estimate of x (absolute error < 2^25, so |x / t - qq| < 0.5 + 2^-20 for
  // t > 2^46), the remainder x - qq t exactly in wrapping 64-bit arithmetic: it lies in (-t, t)
  const double xd = __builtin_fma(__builtin_fma(__builtin_fma((double)p3, 65536.0, (double)p2), 65536.0, (double)p1),
                                  65536.0, (double)p0);
  const long long qq = (long long)__builtin_rint(xd * tinv);
  const uint64_t xl = (uint64_t)(long long)p0 + ((uint64_t)(long long)p1 << 16) + ((uint64_t)(long long)p2 << 32) +
                      ((uint64_t)(long long)p3 << 48);
  long long v = (long long)(xl - (uint64_t)qq * t);
  if (v < 0) v += (long long)t;
  return (uint64_t)v;
}

// wfold of the conversion sum plus a signed term z (|z| < 2^60): the sum x + z, |x + z| < 2^76.02, is
// estimated in double with an absolute error below 2^26, so the quotient estimate still leaves the
// remainder in (-t, t) for t > 2^46.
__device__ __forceinline__ uint64_t wfold_add(const wv4i (&a)[8], int r, uint64_t t, double tinv, long long z) {
  const int p0 = a[0][r] + a[1][r] * 256, p1 = a[2][r] + a[3][r] * 256;
  const int p2 = a[4][r] + a[5][r] * 256, p3 = a[6][r] + a[7][r] * 256;
  const double xd = __builtin_fma(__builtin_fma(__builtin_fma((double)p3, 65536.0, (double)p2), 65536.0, (double)p1),
                                  65536.0, (double)p0) +
                    (double)z;
  const long long qq = (long long)__builtin_rint(xd * tinv);
  const uint64_t xl = (uint64_t)(long long)p0 + ((uint64_t)(long long)p1 << 16) + ((uint64_t)(long long)p2 << 32) +
                      ((uint64_t)(long long)p3 << 48) + (uint64_t)z;
  long long v = (long long)(xl - (uint64_t)qq * t);
  if (v < 0) v += (long long)t;
  return (uint64_t)v;
}

}  // namespace hck
