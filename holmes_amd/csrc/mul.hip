// Ciphertext x ciphertext multiplication: tensor product, relinearisation (a key switch of the
// degree-2 component with the s^2 -> s key, its result added to the degree-0/1 components inside
// the key switch's last kernel), and the grouped scalar-weighted sum the polynomial evaluators use.
// Algorithm: the CKKS multiply EasyFHE runs for fhe.homo_mul_no_relin / homo_relinearize /
// homo_mul_relin (llama3fhe/operators/attention/prefill/qk.py:460-464,
// llama3fhe/operators/attention/kernel_helpers.py:146-152,
// llama3fhe/operators/nonlinear/polynomial.py:140-190) and grouped_scalar_weighted_acc
// (polynomial.py:256-300).
#include <hip/hip_runtime.h>

#include "../../include/holmes_ckks.h"
#include "internal.hpp"
#include "wide.hpp"

namespace hck {
namespace {

constexpr int kMaxBatchM = 64;  // items per key-switch launch sequence

// d0 = a0 b0, d1 = a0 b1 + a1 b0, d2 = a1 b1 (mod q_limb), canonical.  Grid (N / 256, limbs, batch).
__global__ __launch_bounds__(256) void k_tensor(const uint64_t* __restrict__ a0, const uint64_t* __restrict__ a1,
                                                long long a_stride, const uint64_t* __restrict__ b0,
                                                const uint64_t* __restrict__ b1, long long b_stride,
                                                uint64_t* __restrict__ d0, uint64_t* __restrict__ d1,
                                                uint64_t* __restrict__ d2, long long d_stride, DevTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int i = blockIdx.y;
  const long long z = blockIdx.z;
  const double p = T.p[i], pinv = T.pinv[i];
  const long long lo = (long long)i * kN + k;
  const double x0 = u2d(a0[z * a_stride + lo]), x1 = u2d(a1[z * a_stride + lo]);
  const double y0 = u2d(b0[z * b_stride + lo]), y1 = u2d(b1[z * b_stride + lo]);
  // canonical operands: each product is within 0.875 p, the cross sum within 1.75 p
  d0[z * d_stride + lo] = d2u(canon(mulv(x0, y0, p, pinv), p, pinv));
  d1[z * d_stride + lo] = d2u(canon(mulv(x0, y1, p, pinv) + mulv(x1, y0, p, pinv), p, pinv));
  d2[z * d_stride + lo] = d2u(canon(mulv(x1, y1, p, pinv), p, pinv));
}

// The tensor terms the fused rescaled product reads from memory: d2 = a1 b1 on every limb, d0 and d1
// on the last limb only (the finish forms them for the other limbs from a and b).
// Grid (N / 256, limbs, batch).
__global__ __launch_bounds__(256) void k_tensor_d2(const uint64_t* __restrict__ a0, const uint64_t* __restrict__ a1,
                                                   long long a_stride, const uint64_t* __restrict__ b0,
                                                   const uint64_t* __restrict__ b1, long long b_stride,
                                                   uint64_t* __restrict__ d0, uint64_t* __restrict__ d1,
                                                   uint64_t* __restrict__ d2, long long d_stride, int ell, DevTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int i = blockIdx.y;
  const long long z = blockIdx.z;
  const double p = T.p[i], pinv = T.pinv[i];
  const long long lo = (long long)i * kN + k;
  const double x1 = u2d(a1[z * a_stride + lo]), y1 = u2d(b1[z * b_stride + lo]);
  d2[z * d_stride + lo] = d2u(canon(mulv(x1, y1, p, pinv), p, pinv));
  if (i == ell - 1) {
    const double x0 = u2d(a0[z * a_stride + lo]), y0 = u2d(b0[z * b_stride + lo]);
    d0[z * d_stride + lo] = d2u(canon(mulv(x0, y0, p, pinv), p, pinv));
    d1[z * d_stride + lo] = d2u(canon(mulv(x0, y1, p, pinv) + mulv(x1, y0, p, pinv), p, pinv));
  }
}

// out[g][l][k] = sum_j w[g][j][l] * in[j][l][k] (mod q_l), canonical.  Grid (N / 256, limbs, groups).
__global__ __launch_bounds__(256) void k_weighted_sum(const uint64_t* __restrict__ in, long long in_stride, int n,
                                                      const uint64_t* __restrict__ w, uint64_t* __restrict__ out,
                                                      long long out_stride, int limbs, DevTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int i = blockIdx.y;
  const long long g = blockIdx.z;
  const double p = T.p[i], pinv = T.pinv[i];
  const uint64_t* wg = w + g * (long long)n * limbs + i;
  const uint64_t* x = in + (long long)i * kN + k;
  double acc = 0.0;
  for (int j = 0; j < n; ++j) {
    acc += mulv(u2d(x[(long long)j * in_stride]), u2d(wg[(long long)j * limbs]), p, pinv);  // |term| <= 0.875 p
    if ((j & 7) == 7) acc = reduce(acc, p, pinv);  // <= p/2 + 8 * 0.875 p < 8 p between reductions
  }
  out[g * out_stride + (long long)i * kN + k] = d2u(canon(acc, p, pinv));
}

// Linear combinations over pointer lists: out[g][l][k] = sum_t w[t][l] * x[g * terms + t][l][k] (mod q_l),
// canonical; w == null: unit weights (canonical inputs).  Each operand is one [limbs][N] polynomial at
// its own address, so ciphertexts of different levels and allocations combine without copies.
// Grid (N / 256, limbs, groups).  Reduced every 7 terms: |acc| <= p/2 + 7 p < 2^53 stays exact.
constexpr int kLcMaxPtrs = 256;
constexpr int kLcMaxGroups = 64;
struct LcPtrs {
  const uint64_t* x[kLcMaxPtrs];
  uint64_t* out[kLcMaxGroups];
};

__global__ __launch_bounds__(256) void k_lincomb(const LcPtrs P, int terms, const uint64_t* __restrict__ w, int limbs,
                                                DevTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int i = blockIdx.y, g = blockIdx.z;
  const double p = T.p[i], pinv = T.pinv[i];
  const long long off = (long long)i * kN + k;
  double acc = 0.0;
  for (int t = 0; t < terms; ++t) {
    const double x = u2d(P.x[g * terms + t][off]);
    acc += w ? mulv(x, u2d(w[(long long)t * limbs + i]), p, pinv) : x;  // |term| < p
    if (t % 7 == 6) acc = reduce(acc, p, pinv);
  }
  P.out[g][off] = d2u(canon(acc, p, pinv));
}

int launch_tensor(const hck_context* c, int ell, int batch, const uint64_t* a0, const uint64_t* a1, long long a_stride,
                  const uint64_t* b0, const uint64_t* b1, long long b_stride, uint64_t* d0, uint64_t* d1,
                  uint64_t* d2, long long d_stride, hipStream_t s) {
  if (c->wide) return wide_tensor(c, ell, batch, a0, a1, a_stride, b0, b1, b_stride, d0, d1, d2, d_stride, s);
  k_tensor<<<dim3(kN / 256, ell, batch), 256, 0, s>>>(a0, a1, a_stride, b0, b1, b_stride, d0, d1, d2, d_stride,
                                                      c->dev);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

bool valid_level(const hck_context* c, int ell) { return c && ell >= 1 && ell <= c->L; }

}  // namespace
}  // namespace hck

extern "C" int hck_tensor(const hck_context* ctx, int level_limbs, int batch, const uint64_t* a0, const uint64_t* a1,
                          int64_t a_stride, const uint64_t* b0, const uint64_t* b1, int64_t b_stride, uint64_t* d0,
                          uint64_t* d1, uint64_t* d2, int64_t d_stride, void* stream) {
  if (!hck::valid_level(ctx, level_limbs) || batch < 0 || batch > 65535) return HCK_ERR_ARG;
  if (!a0 || !a1 || !b0 || !b1 || !d0 || !d1 || !d2) return HCK_ERR_ARG;
  if (batch == 0) return HCK_OK;
  return hck::launch_tensor(ctx, level_limbs, batch, a0, a1, a_stride, b0, b1, b_stride, d0, d1, d2, d_stride,
                            (hipStream_t)stream);
}

extern "C" size_t hck_relinearize_workspace_bytes(const hck_context* ctx, int level_limbs, int batch) {
  return hck_keyswitch_workspace_bytes(ctx, level_limbs, batch);
}

extern "C" int hck_relinearize(const hck_context* ctx, int level_limbs, int batch, const uint64_t* d0,
                               const uint64_t* d1, const uint64_t* d2, int64_t in_stride, const uint64_t* relin_ksk,
                               uint64_t* out0, uint64_t* out1, int64_t out_stride, void* workspace,
                               size_t workspace_bytes, void* stream) {
  if (!hck::valid_level(ctx, level_limbs) || batch < 0) return HCK_ERR_ARG;
  if (!d0 || !d1 || !d2 || !relin_ksk || !out0 || !out1) return HCK_ERR_ARG;
  // d2 is read by two kernels while the outputs are written; d0 / d1 are read where they are written
  if (out0 == d2 || out1 == d2 || out0 == out1) return HCK_ERR_ARG;
  if (batch == 0) return HCK_OK;
  const int chunk = batch < hck::kMaxBatchM ? batch : hck::kMaxBatchM;
  if (!workspace || workspace_bytes < hck::ks_fused_bytes(ctx, level_limbs, chunk)) return HCK_ERR_WORKSPACE;
  const uint64_t* keys[hck::kMaxBatchM];
  for (int b = 0; b < chunk; ++b) keys[b] = relin_ksk;
  for (int i0 = 0; i0 < batch; i0 += chunk) {
    const int nb = batch - i0 < chunk ? batch - i0 : chunk;
    const long long ii = (long long)i0 * in_stride, oi = (long long)i0 * out_stride;
    int rc = hck::ks_fused(ctx, level_limbs, nb, d2 + ii, in_stride, 1u, keys, nullptr, 0, d0 + ii, d1 + ii,
                           in_stride, out0 + oi, out1 + oi, out_stride, (char*)workspace, (hipStream_t)stream);
    if (rc) return rc;
  }
  return HCK_OK;
}

extern "C" size_t hck_mul_relin_workspace_bytes(const hck_context* ctx, int level_limbs, int batch) {
  if (!hck::valid_level(ctx, level_limbs) || batch < 0) return 0;
  const int chunk = batch < hck::kMaxBatchM ? batch : hck::kMaxBatchM;
  return hck::ks_fused_bytes(ctx, level_limbs, chunk) + (size_t)3 * chunk * level_limbs * hck::kN * 8;
}

extern "C" int hck_mul_relin(const hck_context* ctx, int level_limbs, int batch, const uint64_t* a0,
                             const uint64_t* a1, int64_t a_stride, const uint64_t* b0, const uint64_t* b1,
                             int64_t b_stride, const uint64_t* relin_ksk, uint64_t* out0, uint64_t* out1,
                             int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream) {
  if (!hck::valid_level(ctx, level_limbs) || batch < 0) return HCK_ERR_ARG;
  if (!a0 || !a1 || !b0 || !b1 || !relin_ksk || !out0 || !out1 || out0 == out1) return HCK_ERR_ARG;
  if (batch == 0) return HCK_OK;
  if (!workspace || workspace_bytes < hck_mul_relin_workspace_bytes(ctx, level_limbs, batch)) return HCK_ERR_WORKSPACE;
  const int chunk = batch < hck::kMaxBatchM ? batch : hck::kMaxBatchM;
  const long long poly = (long long)level_limbs * hck::kN;
  char* ks_ws = (char*)workspace;
  uint64_t* d = (uint64_t*)(ks_ws + hck::ks_fused_bytes(ctx, level_limbs, chunk));  // [3][chunk][limbs][N]
  const uint64_t* keys[hck::kMaxBatchM];
  for (int b = 0; b < chunk; ++b) keys[b] = relin_ksk;
  hipStream_t s = (hipStream_t)stream;
  for (int i0 = 0; i0 < batch; i0 += chunk) {
    const int nb = batch - i0 < chunk ? batch - i0 : chunk;
    uint64_t* d0 = d;
    uint64_t* d1 = d + (long long)chunk * poly;
    uint64_t* d2 = d + 2LL * chunk * poly;
    int rc = hck::launch_tensor(ctx, level_limbs, nb, a0 + (long long)i0 * a_stride, a1 + (long long)i0 * a_stride,
                                a_stride, b0 + (long long)i0 * b_stride, b1 + (long long)i0 * b_stride, b_stride, d0,
                                d1, d2, poly, s);
    if (rc) return rc;
    const long long oi = (long long)i0 * out_stride;
    rc = hck::ks_fused(ctx, level_limbs, nb, d2, poly, 1u, keys, nullptr, 0, d0, d1, poly, out0 + oi, out1 + oi,
                       out_stride, ks_ws, s);
    if (rc) return rc;
  }
  return HCK_OK;
}

// The product rescaled: on the matrix-core conversion engine the relinearisation's ModDown and the
// rescale share one pass (ks_rescaled); otherwise hck_mul_relin into the workspace, then the
// rescale.  Both give the same residues.
static bool relin_rescale_fused(const hck_context* ctx, int ell) {
  if (ctx->wide) return ell >= 2 && hck::wide_fused_ok(ctx);
  return ctx->conv_engine == 1 && ell >= 2 && ctx->alpha <= hck::kMaxAlpha && ctx->K <= hck::kMaxSpecial;
}

extern "C" size_t hck_mul_relin_rescale_workspace_bytes(const hck_context* ctx, int level_limbs, int batch) {
  if (!hck::valid_level(ctx, level_limbs) || level_limbs < 2 || batch < 0) return 0;
  const int chunk = batch < hck::kMaxBatchM ? batch : hck::kMaxBatchM;
  const size_t poly = (size_t)level_limbs * hck::kN * 8;
  if (relin_rescale_fused(ctx, level_limbs)) return hck::ks_rs_bytes(ctx, level_limbs, chunk) + 3 * chunk * poly;
  const size_t ks = hck::ks_fused_bytes(ctx, level_limbs, chunk), rs = hck::rescale_bytes(ctx, level_limbs, 2 * chunk);
  return (ks > rs ? ks : rs) + 5 * chunk * poly;
}

namespace {

// The rescaled product with its post-ops: out = (twice ? 2 : 1) * rescale(a * b) - sub (+ scalar on
// out0); sub0 / sub1 and scalar nullable.
int mul_relin_rescale_post(const hck_context* ctx, int level_limbs, int batch, const uint64_t* a0,
                           const uint64_t* a1, int64_t a_stride, const uint64_t* b0, const uint64_t* b1,
                           int64_t b_stride, const uint64_t* relin_ksk, int twice, const uint64_t* sub0,
                           const uint64_t* sub1, int64_t sub_stride, const uint64_t* scalar, uint64_t* out0,
                           uint64_t* out1, int64_t out_stride, void* workspace, size_t workspace_bytes,
                           hipStream_t s) {
  if (!hck::valid_level(ctx, level_limbs) || level_limbs < 2 || batch < 0) return HCK_ERR_ARG;
  if (!a0 || !a1 || !b0 || !b1 || !relin_ksk || !out0 || !out1 || out0 == out1) return HCK_ERR_ARG;
  if ((sub0 == nullptr) != (sub1 == nullptr)) return HCK_ERR_ARG;
  {
    // The outputs may not overlap the operands or each other: the matrix-core engine's finish
    // re-reads a0, a1, b0, b1 after it has stored the first output component, and tiles of
    // different items are in flight together.
    const int64_t in_len = (int64_t)level_limbs * hck::kN, out_len = (int64_t)(level_limbs - 1) * hck::kN;
    const uint64_t* outs[2] = {out0, out1};
    const uint64_t* ins[4] = {a0, a1, b0, b1};
    const int64_t in_stride[4] = {a_stride, a_stride, b_stride, b_stride};
    for (const uint64_t* o : outs)
      for (int k = 0; k < 4; ++k)
        if (hck::batches_overlap(o, out_stride, out_len, ins[k], in_stride[k], in_len, batch)) return HCK_ERR_ARG;
    if (hck::batches_overlap(out0, out_stride, out_len, out1, out_stride, out_len, batch)) return HCK_ERR_ARG;
  }
  if (scalar)
    for (int i = 0; i < level_limbs - 1; ++i)
      if (scalar[i] >= ctx->primes[i]) return HCK_ERR_ARG;
  if (batch == 0) return HCK_OK;
  if (!workspace || workspace_bytes < hck_mul_relin_rescale_workspace_bytes(ctx, level_limbs, batch))
    return HCK_ERR_WORKSPACE;
  const int ell = level_limbs;
  const bool fused = relin_rescale_fused(ctx, ell);
  const int chunk = batch < hck::kMaxBatchM ? batch : hck::kMaxBatchM;
  const long long poly = (long long)ell * hck::kN;
  const size_t ks_bytes = fused ? hck::ks_rs_bytes(ctx, ell, chunk) : [&] {
    const size_t ks = hck::ks_fused_bytes(ctx, ell, chunk), rs = hck::rescale_bytes(ctx, ell, 2 * chunk);
    return ks > rs ? ks : rs;
  }();
  char* ks_ws = (char*)workspace;
  uint64_t* d = (uint64_t*)(ks_ws + ks_bytes);  // [3][chunk][ell][N], then (unfused) [2][chunk][ell][N]
  const uint64_t* keys[hck::kMaxBatchM];
  for (int b = 0; b < chunk; ++b) keys[b] = relin_ksk;
  int prime_idx[hck::kMaxPrimes];
  for (int i = 0; i < ell - 1; ++i) prime_idx[i] = i;
  for (int i0 = 0; i0 < batch; i0 += chunk) {
    const int nb = batch - i0 < chunk ? batch - i0 : chunk;
    uint64_t* d0 = d;
    uint64_t* d1 = d + (long long)chunk * poly;
    uint64_t* d2 = d + 2LL * chunk * poly;
    const long long ai = (long long)i0 * a_stride, bi = (long long)i0 * b_stride;
    const long long oi = (long long)i0 * out_stride, si = (long long)i0 * sub_stride;
    int rc;
    if (fused) {
      // d2 everywhere and d0 / d1 on the last limb; the finish forms d0 / d1 of the other limbs
      if (ctx->wide) {
        rc = hck::wide_tensor_d2(ctx, ell, nb, a0 + ai, a1 + ai, a_stride, b0 + bi, b1 + bi, b_stride, d0, d1, d2, poly,
                                 s);
        if (rc) return rc;
      } else {
        hck::k_tensor_d2<<<dim3(hck::kN / 256, ell, nb), 256, 0, s>>>(a0 + ai, a1 + ai, a_stride, b0 + bi, b1 + bi,
                                                                     b_stride, d0, d1, d2, poly, ell, ctx->dev);
        HCK_CHECK_LAUNCH();
      }
      const uint64_t* ab[4] = {a0 + ai, a1 + ai, b0 + bi, b1 + bi};
      rc = hck::ks_rescaled(ctx, ell, nb, d2, poly, 1u, keys, nullptr, 0, d0, d1, poly, out0 + oi, out1 + oi,
                            out_stride, ks_ws, s, twice, sub0 ? sub0 + si : nullptr, sub1 ? sub1 + si : nullptr,
                            sub_stride, scalar, ab, a_stride, b_stride);
      if (rc) return rc;
      continue;
    }
    rc = hck::launch_tensor(ctx, ell, nb, a0 + ai, a1 + ai, a_stride, b0 + bi, b1 + bi, b_stride, d0, d1, d2, poly, s);
    if (rc) return rc;
    uint64_t* mid = d + 3LL * chunk * poly;  // [2][nb][ell][N]: the relinearised product
    rc = hck::ks_fused(ctx, ell, nb, d2, poly, 1u, keys, nullptr, 0, d0, d1, poly, mid, mid + (long long)nb * poly,
                       poly, ks_ws, s);
    if (rc) return rc;
    uint64_t* outs[2] = {out0 + oi, out1 + oi};
    const uint64_t* subs[2] = {sub0 ? sub0 + si : nullptr, sub1 ? sub1 + si : nullptr};
    for (int c = 0; c < 2; ++c) {
      rc = hck::rescale_fused(ctx, ell, nb, mid + (long long)c * nb * poly, poly, outs[c], out_stride, ks_ws, s);
      if (rc) return rc;
      if (twice) {
        rc = hck_poly_op(ctx, HCK_OP_ADD, outs[c], outs[c], outs[c], nb, out_stride, out_stride, out_stride, ell - 1,
                         prime_idx, nullptr, s);
        if (rc) return rc;
      }
      if (subs[c]) {
        rc = hck_poly_op(ctx, HCK_OP_SUB, outs[c], outs[c], subs[c], nb, out_stride, out_stride, sub_stride, ell - 1,
                         prime_idx, nullptr, s);
        if (rc) return rc;
      }
      if (scalar && c == 0) {
        rc = hck_poly_op(ctx, HCK_OP_ADD_SCALAR, outs[c], outs[c], nullptr, nb, out_stride, out_stride, 0, ell - 1,
                         prime_idx, scalar, s);
        if (rc) return rc;
      }
    }
  }
  return HCK_OK;
}

}  // namespace

extern "C" int hck_mul_relin_rescale(const hck_context* ctx, int level_limbs, int batch, const uint64_t* a0,
                                     const uint64_t* a1, int64_t a_stride, const uint64_t* b0, const uint64_t* b1,
                                     int64_t b_stride, const uint64_t* relin_ksk, uint64_t* out0, uint64_t* out1,
                                     int64_t out_stride, void* workspace, size_t workspace_bytes, void* stream) {
  return mul_relin_rescale_post(ctx, level_limbs, batch, a0, a1, a_stride, b0, b1, b_stride, relin_ksk, 0, nullptr,
                                nullptr, 0, nullptr, out0, out1, out_stride, workspace, workspace_bytes,
                                (hipStream_t)stream);
}

extern "C" int hck_mul_relin_rescale_postop(const hck_context* ctx, int level_limbs, int batch, const uint64_t* a0,
                                            const uint64_t* a1, int64_t a_stride, const uint64_t* b0,
                                            const uint64_t* b1, int64_t b_stride, const uint64_t* relin_ksk,
                                            int apply_double, const uint64_t* sub0, const uint64_t* sub1,
                                            int64_t sub_stride, const uint64_t* scalar, uint64_t* out0,
                                            uint64_t* out1, int64_t out_stride, void* workspace,
                                            size_t workspace_bytes, void* stream) {
  if (sub0 && (sub0 == out0 || sub0 == out1 || sub1 == out0 || sub1 == out1)) return HCK_ERR_ARG;
  return mul_relin_rescale_post(ctx, level_limbs, batch, a0, a1, a_stride, b0, b1, b_stride, relin_ksk,
                                apply_double ? 1 : 0, sub0, sub1, sub_stride, scalar, out0, out1, out_stride, workspace,
                                workspace_bytes, (hipStream_t)stream);
}

extern "C" int hck_weighted_sum(const hck_context* ctx, int limbs, int n, int groups, const uint64_t* in,
                                int64_t in_stride, const uint64_t* weights, uint64_t* out, int64_t out_stride,
                                void* stream) {
  if (!ctx || !in || !weights || !out || limbs < 1 || limbs > ctx->L || n < 1 || groups < 0 || groups > 65535)
    return HCK_ERR_ARG;
  if (groups == 0) return HCK_OK;
  if (ctx->wide) return hck::wide_weighted_sum(ctx, limbs, n, groups, in, in_stride, weights, out, out_stride, (hipStream_t)stream);
  hck::k_weighted_sum<<<dim3(hck::kN / 256, limbs, groups), 256, 0, (hipStream_t)stream>>>(
      in, in_stride, n, weights, out, out_stride, limbs, ctx->dev);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

extern "C" size_t hck_lincomb_rescale_workspace_bytes(const hck_context* ctx, int level_limbs, int groups) {
  if (!ctx || level_limbs < 2 || level_limbs > ctx->L || groups < 0) return 0;
  if (!ctx->wide) return hck::lincomb_rescale_bytes(ctx, level_limbs, groups);
  // the fused wide kernels form the sums where they are used; the separate-launch ones run the two
  // steps: the combination [groups][ell][N], then one rescale at a time
  if (hck::wide_fused_ok(ctx)) return hck::wide_fused_rescale_bytes(ctx, level_limbs, groups);
  return (size_t)groups * level_limbs * hck::kN * 8 + hck::rescale_bytes(ctx, level_limbs, 1);
}

extern "C" int hck_lincomb_rescale(const hck_context* ctx, int level_limbs, int groups, int terms,
                                   const uint64_t* const* x, const uint64_t* weights, uint64_t* const* out,
                                   const uint64_t* add, uint64_t add_mask, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  const int ell = level_limbs;
  if (!ctx || !x || !out || !weights || ell < 2 || ell > ctx->L || groups < 0 || terms < 1) return HCK_ERR_ARG;
  if (groups > hck::kLcRsGroups || (long long)groups * terms > hck::kLcRsPtrs) return HCK_ERR_ARG;
  if (groups == 0) return HCK_OK;
  for (int j = 0; j < groups * terms; ++j)
    if (!x[j]) return HCK_ERR_ARG;
  for (int g = 0; g < groups; ++g)
    if (!out[g]) return HCK_ERR_ARG;
  // outputs must not be inputs: the fused path forms the combination and its rescale in one pass,
  // so an output written over any group's input would be read back by another tile
  for (int g = 0; g < groups; ++g)
    for (int j = 0; j < groups * terms; ++j)
      if (hck::batches_overlap(out[g], 0, (int64_t)(ell - 1) * hck::kN, x[j], 0, (int64_t)ell * hck::kN, 1))
        return HCK_ERR_ARG;
  if (add)
    for (int i = 0; i < ell - 1; ++i)
      if (add[i] >= ctx->primes[i]) return HCK_ERR_ARG;
  if (!workspace || workspace_bytes < hck_lincomb_rescale_workspace_bytes(ctx, ell, groups)) return HCK_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  if (!ctx->wide)
    return hck::lincomb_rescale(ctx, ell, groups, terms, x, weights, out, add, add_mask, (char*)workspace, s);
  if (hck::wide_fused_ok(ctx))
    return hck::wide_lincomb_rescale_fused(ctx, ell, groups, terms, x, weights, out, add, add_mask, (char*)workspace, s);
  const long long poly = (long long)ell * hck::kN;
  uint64_t* tmp = (uint64_t*)workspace;
  char* rs_ws = (char*)(tmp + groups * poly);
  uint64_t* tptr[hck::kLcRsGroups];
  for (int g = 0; g < groups; ++g) tptr[g] = tmp + g * poly;
  int rc = hck_lincomb(ctx, ell, groups, terms, x, weights, tptr, stream);
  if (rc) return rc;
  int prime_idx[hck::kMaxPrimes];
  for (int i = 0; i < ell - 1; ++i) prime_idx[i] = i;
  for (int g = 0; g < groups; ++g) {
    rc = hck::rescale_fused(ctx, ell, 1, tptr[g], poly, out[g], (long long)(ell - 1) * hck::kN, rs_ws, s);
    if (rc) return rc;
    if (add && ((add_mask >> g) & 1ull)) {
      rc = hck_poly_op(ctx, HCK_OP_ADD_SCALAR, out[g], out[g], nullptr, 1, 0, 0, 0, ell - 1, prime_idx, add, stream);
      if (rc) return rc;
    }
  }
  return HCK_OK;
}

extern "C" int hck_lincomb(const hck_context* ctx, int limbs, int groups, int terms, const uint64_t* const* x,
                           const uint64_t* weights, uint64_t* const* out, void* stream) {
  if (!ctx || !x || !out || limbs < 1 || limbs > ctx->L || groups < 0 || terms < 1) return HCK_ERR_ARG;
  if (groups > hck::kLcMaxGroups || (long long)groups * terms > hck::kLcMaxPtrs) return HCK_ERR_ARG;
  if (groups == 0) return HCK_OK;
  hck::LcPtrs P{};
  for (int j = 0; j < groups * terms; ++j) {
    if (!x[j]) return HCK_ERR_ARG;
    P.x[j] = x[j];
  }
  for (int g = 0; g < groups; ++g) {
    if (!out[g]) return HCK_ERR_ARG;
    P.out[g] = out[g];
  }
  if (ctx->wide) return hck::wide_lincomb(ctx, limbs, groups, terms, x, weights, out, (hipStream_t)stream);
  hck::k_lincomb<<<dim3(hck::kN / 256, limbs, groups), 256, 0, (hipStream_t)stream>>>(P, terms, weights, limbs,
                                                                                     ctx->dev);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}
