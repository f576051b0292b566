// Exact 64-bit integer modular arithmetic for primes 2^31 < p < 2^62 (host and device).
//
// The FP64 arithmetic of modarith.hpp is exact only below 2^50; wider primes (the reference's 59/60-bit
// chains) are reduced with Barrett's method on 64-bit words:
//   w = bit length of p, mu = floor(2^(2w) / p)  (2^w < mu <= 2^(w+1) < 2^63 for w <= 62);
//   for x < p^2:  q = floor(floor(x / 2^(w-1)) * mu / 2^(w+1)),  r = x - q p,  0 <= r < 3p
// (Menezes, van Oorschot, Vanstone, Handbook of Applied Cryptography, algorithm 14.42), then at
// most two subtractions of p.  r < 3p < 2^64, so r is computed from the low words alone.
// Products use the compiler's 64 x 64 -> 128-bit multiply (unsigned __int128 multiplication; no
// 128-bit division is needed anywhere).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hck {

typedef unsigned __int128 u128_t;

struct Barrett64 {
  uint64_t p;
  uint64_t mu;
  int w;
};

__host__ __device__ __forceinline__ int bit_length64(uint64_t x) {
  int n = 0;
  while (x) {
    ++n;
    x >>= 1;
  }
  return n;
}

// mu = floor(2^(2w) / p) by restoring long division: 2^(2w) has one set bit, so every later
// dividend bit is zero and the running remainder (< p < 2^62) doubles each step.
__host__ __device__ __forceinline__ Barrett64 barrett_make(uint64_t p) {
  Barrett64 b;
  b.p = p;
  b.w = bit_length64(p);
  uint64_t rem = 1, mu = 0;
  for (int i = 2 * b.w - 1; i >= 0; --i) {
    rem <<= 1;
    mu <<= 1;
    if (rem >= p) {
      rem -= p;
      mu |= 1;
    }
  }
  b.mu = mu;
  return b;
}

// x mod p for x < p^2.
__host__ __device__ __forceinline__ uint64_t barrett_reduce(u128_t x, const Barrett64& b) {
  const uint64_t q1 = (uint64_t)(x >> (b.w - 1));
  const uint64_t q3 = (uint64_t)(((u128_t)q1 * b.mu) >> (b.w + 1));
  uint64_t r = (uint64_t)x - q3 * b.p;
  if (r >= b.p) r -= b.p;
  if (r >= b.p) r -= b.p;
  return r;
}

// a * c mod p for residues a, c < p.
__host__ __device__ __forceinline__ uint64_t mulmod64(uint64_t a, uint64_t c, const Barrett64& b) {
  return barrett_reduce((u128_t)a * c, b);
}

__host__ __device__ __forceinline__ uint64_t addmod64(uint64_t a, uint64_t c, uint64_t p) {
  const uint64_t s = a + c;
  return s >= p ? s - p : s;
}

__host__ __device__ __forceinline__ uint64_t submod64(uint64_t a, uint64_t c, uint64_t p) {
  return a >= c ? a - c : a + p - c;
}

// Shoup's companion of a constant c < p: floor(c 2^64 / p).  Host only (one 128-bit division).
inline uint64_t shoup_companion(uint64_t c, uint64_t p) { return (uint64_t)(((u128_t)c << 64) / p); }

// a * c mod p in [0, 2p) with c's companion (Shoup): q = floor(a c' / 2^64), r = a c - q p.
__host__ __device__ __forceinline__ uint64_t mulshoup_lazy(uint64_t a, uint64_t c, uint64_t cs, uint64_t p) {
  const uint64_t q = (uint64_t)(((u128_t)a * cs) >> 64);
  return a * c - q * p;
}

}  // namespace hck
