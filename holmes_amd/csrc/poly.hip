// Elementwise limb kernels: automorphism (NTT-domain permutation), add/sub/mul/neg, scalar
// multiplication and addition, X^(N/2) multiplication, signed-integer reduction.  All are HBM-streaming kernels: one thread per
// coefficient, 256 threads per workgroup, grid (N / 256, limbs, polys).
#include <hip/hip_runtime.h>

#include "../../include/holmes_ckks.h"
#include "internal.hpp"
#include "wide.hpp"

namespace hck {
namespace {

struct PrimeMap {
  uint8_t prime[kMaxPrimes];
};
struct ScalarMap {
  TwPair s[kMaxPrimes];
};

__device__ __forceinline__ uint32_t brv16(uint32_t x) { return __brev(x) >> 16; }

// out[k] = in[k'] with 2 brv(k') + 1 = g (2 brv(k) + 1) mod 2N (slot k holds the evaluation at
// psi^(2 brv(k) + 1); sigma_g maps it to the evaluation at psi^(g (2 brv(k) + 1))).
__global__ __launch_bounds__(256) void k_automorph(const uint64_t* __restrict__ in, uint64_t* __restrict__ out,
                                                   long long in_stride, long long out_stride,
                                                   uint32_t g) {
  const uint32_t k = blockIdx.x * 256 + threadIdx.x;
  const uint32_t e = ((2u * brv16(k) + 1u) * g) & (2u * kN - 1u);
  const uint32_t src = brv16((e - 1u) >> 1);
  const long long limb = blockIdx.y;
  out[(long long)blockIdx.z * out_stride + limb * kN + k] = in[(long long)blockIdx.z * in_stride + limb * kN + src];
}

template <int OP>
__global__ __launch_bounds__(256) void k_poly_op(uint64_t* out, const uint64_t* a, const uint64_t* b,
                                                 long long out_stride, long long a_stride,
                                                 long long b_stride, PrimeMap pm, ScalarMap sm,
                                                 DevTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int limb = blockIdx.y;
  const int pi = pm.prime[limb];
  const double p = T.p[pi], pinv = T.pinv[pi];
  const long long lo = (long long)limb * kN + k;
  const long long z = blockIdx.z;
  const double x = u2d(a[z * a_stride + lo]);
  double r;
  if constexpr (OP == HCK_OP_ADD) {
    r = x + u2d(b[z * b_stride + lo]);
    r = r >= p ? r - p : r;
  } else if constexpr (OP == HCK_OP_SUB) {
    r = x - u2d(b[z * b_stride + lo]);
    r = r < 0.0 ? r + p : r;
  } else if constexpr (OP == HCK_OP_NEG) {
    r = x == 0.0 ? 0.0 : p - x;
  } else if constexpr (OP == HCK_OP_MUL) {
    r = canon(mulv(x, u2d(b[z * b_stride + lo]), p, pinv), p, pinv);
  } else if constexpr (OP == HCK_OP_MAC) {
    const double acc = u2d(out[z * out_stride + lo]);
    r = canon(acc + mulv(x, u2d(b[z * b_stride + lo]), p, pinv), p, pinv);
  } else if constexpr (OP == HCK_OP_MUL_SCALAR) {
    r = canon(mulc(x, sm.s[limb], p), p, pinv);
  } else if constexpr (OP == HCK_OP_ADD_SCALAR) {
    r = x + sm.s[limb].w;  // a constant polynomial is the same value at every evaluation point
    r = r >= p ? r - p : r;
  } else {  // HCK_OP_MUL_XHALF: X^(N/2) evaluates to zeta4 at slots k < N/2 and -zeta4 above
    const double m = mulc(x, T.zeta4[pi], p);
    r = canon(k < kN / 2 ? m : -m, p, pinv);
  }
  out[z * out_stride + lo] = d2u(r);
}

__global__ __launch_bounds__(256) void k_from_signed(const int64_t* __restrict__ in, uint64_t* __restrict__ out,
                                                     long long in_stride, long long out_stride,
                                                     PrimeMap pm, const uint64_t* __restrict__ pu) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int limb = blockIdx.y;
  const uint64_t q = pu[pm.prime[limb]];
  const int64_t v = in[(long long)blockIdx.z * in_stride + k];
  // |v| may exceed q: take the magnitude modulo q (integer remainder), then negate.
  const uint64_t mag = v >= 0 ? (uint64_t)v : (uint64_t)(-(v + 1)) + 1u;
  uint64_t r = mag % q;
  if (v < 0 && r) r = q - r;
  out[(long long)blockIdx.z * out_stride + (long long)limb * kN + k] = r;
}

}  // namespace
}  // namespace hck

extern "C" int hck_automorphism(const hck_context* ctx, const uint64_t* in, uint64_t* out, int polys,
                                int64_t in_stride, int64_t out_stride, int limbs, uint32_t galois,
                                void* stream) {
  if (!ctx || !in || !out || polys < 0 || limbs < 0 || polys > 65535 || limbs > 65535) return HCK_ERR_ARG;
  if ((galois & 1u) == 0 || galois >= 2u * hck::kN) return HCK_ERR_ARG;
  if (in == out) return HCK_ERR_ARG;
  if (polys == 0 || limbs == 0) return HCK_OK;
  hck::k_automorph<<<dim3(hck::kN / 256, limbs, polys), 256, 0, (hipStream_t)stream>>>(
      in, out, in_stride, out_stride, galois);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

extern "C" int hck_poly_op(const hck_context* ctx, int op, uint64_t* out, const uint64_t* a,
                           const uint64_t* b, int polys, int64_t out_stride, int64_t a_stride,
                           int64_t b_stride, int limbs, const int* prime_idx, const uint64_t* scalar,
                           void* stream) {
  if (!ctx || !out || !a || !prime_idx || polys < 0 || polys > 65535) return HCK_ERR_ARG;
  if (limbs < 0 || limbs > hck::kMaxPrimes) return HCK_ERR_ARG;
  if (op < HCK_OP_ADD || op > HCK_OP_ADD_SCALAR) return HCK_ERR_ARG;
  const bool binary = op == HCK_OP_ADD || op == HCK_OP_SUB || op == HCK_OP_MUL || op == HCK_OP_MAC;
  if (binary && !b) return HCK_ERR_ARG;
  const bool with_scalar = op == HCK_OP_MUL_SCALAR || op == HCK_OP_ADD_SCALAR;
  if (with_scalar && !scalar) return HCK_ERR_ARG;
  hck::PrimeMap pm{};
  hck::ScalarMap sm{};
  for (int i = 0; i < limbs; ++i) {
    if (prime_idx[i] < 0 || prime_idx[i] >= ctx->np) return HCK_ERR_ARG;
    pm.prime[i] = (uint8_t)prime_idx[i];
    if (with_scalar) {
      const uint64_t q = ctx->primes[prime_idx[i]];
      if (scalar[i] >= q) return HCK_ERR_ARG;
      sm.s[i] = hck::TwPair{(double)scalar[i], (double)scalar[i] / (double)q};
    }
  }
  if (polys == 0 || limbs == 0) return HCK_OK;
  if (ctx->wide)
    return hck::wide_poly_op(ctx, op, out, a, b, polys, out_stride, a_stride, b_stride, limbs, prime_idx, scalar,
                             (hipStream_t)stream);
  const dim3 grid(hck::kN / 256, limbs, polys);
  hipStream_t s = (hipStream_t)stream;
  switch (op) {
    case HCK_OP_ADD: hck::k_poly_op<HCK_OP_ADD><<<grid, 256, 0, s>>>(out, a, b, out_stride, a_stride, b_stride, pm, sm, ctx->dev); break;
    case HCK_OP_SUB: hck::k_poly_op<HCK_OP_SUB><<<grid, 256, 0, s>>>(out, a, b, out_stride, a_stride, b_stride, pm, sm, ctx->dev); break;
    case HCK_OP_MUL: hck::k_poly_op<HCK_OP_MUL><<<grid, 256, 0, s>>>(out, a, b, out_stride, a_stride, b_stride, pm, sm, ctx->dev); break;
    case HCK_OP_NEG: hck::k_poly_op<HCK_OP_NEG><<<grid, 256, 0, s>>>(out, a, b, out_stride, a_stride, b_stride, pm, sm, ctx->dev); break;
    case HCK_OP_MUL_SCALAR: hck::k_poly_op<HCK_OP_MUL_SCALAR><<<grid, 256, 0, s>>>(out, a, b, out_stride, a_stride, b_stride, pm, sm, ctx->dev); break;
    case HCK_OP_MUL_XHALF: hck::k_poly_op<HCK_OP_MUL_XHALF><<<grid, 256, 0, s>>>(out, a, b, out_stride, a_stride, b_stride, pm, sm, ctx->dev); break;
    case HCK_OP_MAC: hck::k_poly_op<HCK_OP_MAC><<<grid, 256, 0, s>>>(out, a, b, out_stride, a_stride, b_stride, pm, sm, ctx->dev); break;
    case HCK_OP_ADD_SCALAR: hck::k_poly_op<HCK_OP_ADD_SCALAR><<<grid, 256, 0, s>>>(out, a, b, out_stride, a_stride, b_stride, pm, sm, ctx->dev); break;
    default: return HCK_ERR_ARG;
  }
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

extern "C" int hck_poly_from_signed(const hck_context* ctx, const int64_t* in, uint64_t* out, int polys,
                                    int64_t in_stride, int64_t out_stride, int limbs,
                                    const int* prime_idx, void* stream) {
  if (!ctx || !in || !out || !prime_idx || polys < 0 || polys > 65535) return HCK_ERR_ARG;
  if (limbs < 0 || limbs > hck::kMaxPrimes) return HCK_ERR_ARG;
  hck::PrimeMap pm{};
  for (int i = 0; i < limbs; ++i) {
    if (prime_idx[i] < 0 || prime_idx[i] >= ctx->np) return HCK_ERR_ARG;
    pm.prime[i] = (uint8_t)prime_idx[i];
  }
  if (polys == 0 || limbs == 0) return HCK_OK;
  hck::k_from_signed<<<dim3(hck::kN / 256, limbs, polys), 256, 0, (hipStream_t)stream>>>(
      in, out, in_stride, out_stride, pm, ctx->d_primes_u64);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}
