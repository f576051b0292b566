// Hybrid key switching (ModUp -> key inner product -> ModDown), rotation and rescale.
//
// Pipeline for a batch of B polynomials d at ell limbs (beta = ceil(ell / alpha) digits):
//   1. INTT(d)                                   -> coef   [B][ell][N]          (lazy doubles)
//   2. ModUp base conversion, digit j           -> ext_j  [B][beta][ell+K][N]  (targets only)
//   3. NTT of every ext target limb
//   4. inner product with the key, both comps   -> acc    [B][2][ell+K][N]
//   5. INTT of acc's P limbs
//   6. ModDown base conversion P -> Q            -> conv   [B][2][ell][N]
//   7. NTT(conv)
//   8. out_c = (acc_c - conv_c) * P^-1 (+ addend)  canonical uint64
// Digit j's own limbs never leave the input: step 4 reads them from d directly.  Every
// intermediate is an exact-integer double (modarith.hpp); only the outputs are canonicalised.
// Algorithm: the key-switch kernels EasyFHE runs for fhe.homo_rotate (F.cv_modup,
// F.cv_innerproduct_*, F.cv_moddown; bench/cmp/report.py:26-30) with the key laid out as in
// llama3fhe/parallel/prefill/keys.py:105-117 ([2][beta][limbs + K][N]).
#include <hip/hip_runtime.h>

#include "../../include/holmes_ckks.h"
#include "internal.hpp"

namespace hck {
namespace {

constexpr int kMaxBatch = 64;
struct KeyPtrs {
  const uint64_t* k[kMaxBatch];
};

template <Fmt F>
__device__ __forceinline__ double ldx(const void* base, long long i) {
  if constexpr (F == kU64) return u2d(((const uint64_t*)base)[i]);
  else return ((const double*)base)[i];
}

// Fast base conversion, one thread per coefficient.  Group (z, y): sources at
// src + z * src_zs + y * src_ys + (src_off0 + y * src_off_y + s) * N, targets at
// dst + z * dst_zs + y * dst_ys + cc.dst_slot[t] * N, constants cc_base[y * cc_y].
template <Fmt IN>
__global__ __launch_bounds__(256) void k_conv(const void* __restrict__ src, long long src_zs, long long src_ys,
                                              int src_off0, int src_off_y, double* __restrict__ dst,
                                              long long dst_zs, long long dst_ys,
                                              const ConvConsts* __restrict__ cc_base, int cc_y, DevTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int y = blockIdx.y;
  const long long z = blockIdx.z;
  const ConvConsts& C = cc_base[y * cc_y];
  const int ns = C.ns, nt = C.nt;
  const char* s = (const char*)src + (z * src_zs + y * src_ys) * 8;
  double* d = dst + z * dst_zs + y * dst_ys;
  const int off0 = src_off0 + y * src_off_y;
  double ys[kMaxAlpha];
#pragma unroll
  for (int i = 0; i < kMaxAlpha; ++i) {
    if (i < ns) {
      const int pi = C.src_prime[i];
      const double p = T.p[pi], pinv = T.pinv[pi];
      const double x = ldx<IN>(s, (long long)(off0 + i) * kN + k);
      // centered representative in (-p/2, p/2]: part of the definition (zero-mean lift)
      const double y = canon(mulc(x, C.hinv[i], p), p, pinv);
      ys[i] = y > 0.5 * p ? y - p : y;
    }
  }
  for (int t = 0; t < nt; ++t) {
    const int pt = C.dst_prime[t];
    const double p = T.p[pt], pinv = T.pinv[pt];
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < kMaxAlpha; ++i) {
      if (i < ns) {
        acc += mulc(ys[i], C.hmod[i][t], p);       // |term| <= 0.75 p for |ys| < 2^50
        if ((i & 7) == 7) acc = reduce(acc, p, pinv);
      }
    }
    d[(long long)C.dst_slot[t] * kN + k] = reduce(acc, p, pinv);
  }
}

// Inner product with the key: acc[b][c][e] = sum_j ext_j[e] * key_b[c][j][prime(e)].
__global__ __launch_bounds__(256) void k_inner_product(const uint64_t* __restrict__ d, long long d_stride,
                                                       const double* __restrict__ ext, double* __restrict__ acc,
                                                       KeyPtrs keys, int ell, int beta, DevTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int e = blockIdx.y;
  const int b = blockIdx.z;
  const int L = T.L, K = T.K, alpha = T.alpha;
  const int ext_l = ell + K;
  const int pi = e < ell ? e : L + (e - ell);
  const double p = T.p[pi], pinv = T.pinv[pi];
  const int beta_max = (L + alpha - 1) / alpha;
  const long long comp_stride = (long long)beta_max * (L + K) * kN;
  const uint64_t* key = keys.k[b];
  const int own = e < ell ? e / alpha : -1;  // digit whose own limb this is (read from d)
  double sb = 0.0, sa = 0.0;
  for (int j = 0; j < beta; ++j) {
    const double x = (j == own) ? u2d(d[(long long)b * d_stride + (long long)e * kN + k])
                                : ext[(((long long)b * beta + j) * ext_l + e) * kN + k];
    const long long ko = ((long long)j * (L + K) + pi) * kN + k;
    sb += mulv(x, u2d(key[ko]), p, pinv);                // |x| <= 3p: |term| <= 2p
    sa += mulv(x, u2d(key[comp_stride + ko]), p, pinv);
    if ((j & 3) == 3) { sb = reduce(sb, p, pinv); sa = reduce(sa, p, pinv); }
  }
  double* o = acc + ((long long)b * 2 * ext_l + e) * kN + k;
  o[0] = reduce(sb, p, pinv);
  o[(long long)ext_l * kN] = reduce(sa, p, pinv);
}

// out_c[b][i] = (acc_c[b][i] - conv_c[b][i]) * P^-1 mod q_i  (+ add[b][i] for c = 0).
__global__ __launch_bounds__(256) void k_moddown_combine(const double* __restrict__ acc, const double* __restrict__ conv,
                                                         const uint64_t* __restrict__ add, long long add_stride,
                                                         uint64_t* __restrict__ out_b, uint64_t* __restrict__ out_a,
                                                         long long out_stride, int ell,
                                                         const LevelConsts* __restrict__ lc, DevTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int i = blockIdx.y;
  const int b = blockIdx.z >> 1, c = blockIdx.z & 1;
  const int ext_l = ell + T.K;
  const double p = T.p[i], pinv = T.pinv[i];
  const double a = acc[(((long long)b * 2 + c) * ext_l + i) * kN + k];
  const double v = conv[(((long long)b * 2 + c) * ell + i) * kN + k];
  double r = mulc(a - v, lc->p_inv[i], p);
  if (c == 0 && add) r += u2d(add[(long long)b * add_stride + (long long)i * kN + k]);
  uint64_t* o = c == 0 ? out_b : out_a;
  o[(long long)b * out_stride + (long long)i * kN + k] = d2u(canon(r, p, pinv));
}

// Rescale helpers: spread the last limb's coefficients, as centered (-q_last/2, q_last/2]
// values, to every lower prime, then combine (x_i - NTT(spread_i)) * q_last^-1 = round(X / q_last).
__global__ __launch_bounds__(256) void k_rescale_spread(const uint64_t* __restrict__ last, double* __restrict__ spread,
                                                        int ell, DevTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int i = blockIdx.y;
  const long long z = blockIdx.z;
  const double x = u2d(last[z * kN + k]);
  const double p = T.p[i], ql = T.p[ell - 1];
  // x in (q_last/2, q_last) stands for x - q_last; q_last < 2 q_i keeps both cases in [0, q_i)
  spread[(z * (ell - 1) + i) * kN + k] = x > 0.5 * ql ? x - ql + p : (x >= p ? x - p : x);
}

__global__ __launch_bounds__(256) void k_rescale_combine(const uint64_t* __restrict__ in, long long in_stride,
                                                         const double* __restrict__ spread, uint64_t* __restrict__ out,
                                                         long long out_stride, int ell,
                                                         const LevelConsts* __restrict__ lc, DevTables T) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  const int i = blockIdx.y;
  const long long z = blockIdx.z;
  const double p = T.p[i], pinv = T.pinv[i];
  const double x = u2d(in[z * in_stride + (long long)i * kN + k]);
  const double v = spread[(z * (ell - 1) + i) * kN + k];
  out[z * out_stride + (long long)i * kN + k] = d2u(canon(mulc(x - v, lc->qlast_inv[i], p), p, pinv));
}

struct KsLayout {
  size_t coef, ext, acc, total;  // byte offsets
};

KsLayout ks_layout(const hck_context* c, int ell, int batch) {
  const size_t n = kN, beta = beta_of(c, ell), ext_l = ell + c->K;
  KsLayout L;
  L.coef = 0;                                                    // [B][2][ell][N] (coef, later conv)
  L.ext = L.coef + (size_t)batch * 2 * ell * n * 8;              // [B][beta][ell+K][N]
  L.acc = L.ext + (size_t)batch * beta * ext_l * n * 8;          // [B][2][ell+K][N]
  L.total = L.acc + (size_t)batch * 2 * ext_l * n * 8;
  return L;
}

int keyswitch_chunk(const hck_context* c, int ell, int batch, const uint64_t* d, long long d_stride,
                    const uint64_t* const* ksk, const uint64_t* add, long long add_stride, uint64_t* out_b,
                    uint64_t* out_a, long long out_stride, char* ws, hipStream_t s) {
  const int K = c->K, beta = beta_of(c, ell), ext_l = ell + K;
  const KsLayout lay = ks_layout(c, ell, batch);
  double* coef = (double*)(ws + lay.coef);
  double* ext = (double*)(ws + lay.ext);
  double* acc = (double*)(ws + lay.acc);
  const long long n = kN;
  int rc;
  // 1. INTT(d)
  LimbList lq;
  lq.n = ell;
  for (int i = 0; i < ell; ++i) { lq.off[i] = (uint16_t)i; lq.prime[i] = (uint8_t)i; }
  if ((rc = launch_ntt_inv(c, d, kU64, coef, kF64, batch, d_stride, 2LL * ell * n, lq, s))) return rc;
  // 2. ModUp base conversion per digit
  k_conv<kF64><<<dim3(kN / 256, beta, batch), 256, 0, s>>>(
      coef, 2LL * ell * n, 0, 0, c->alpha, ext, (long long)beta * ext_l * n, (long long)ext_l * n,
      modup_consts(c, ell, 0), 1, c->dev);
  HCK_CHECK_LAUNCH();
  // 3. NTT of the extended targets
  LimbList lt;
  lt.n = 0;
  for (int j = 0; j < beta; ++j) {
    const int lo = j * c->alpha, hi = lo + c->alpha < ell ? lo + c->alpha : ell;
    for (int e = 0; e < ext_l; ++e) {
      if (e >= lo && e < hi) continue;
      if (lt.n >= kMaxList) return HCK_ERR_UNSUPPORTED;
      lt.off[lt.n] = (uint16_t)(j * ext_l + e);
      lt.prime[lt.n] = (uint8_t)prime_of_ext(c, ell, e);
      ++lt.n;
    }
  }
  if ((rc = launch_ntt_fwd(c, ext, kF64, ext, kF64, batch, (long long)beta * ext_l * n,
                           (long long)beta * ext_l * n, lt, s)))
    return rc;
  // 4. inner product
  KeyPtrs kp{};
  for (int b = 0; b < batch; ++b) kp.k[b] = ksk[b];
  k_inner_product<<<dim3(kN / 256, ext_l, batch), 256, 0, s>>>(d, d_stride, ext, acc, kp, ell, beta, c->dev);
  HCK_CHECK_LAUNCH();
  // 5. INTT of the P limbs of both components
  LimbList lp;
  lp.n = 2 * K;
  for (int comp = 0; comp < 2; ++comp)
    for (int k = 0; k < K; ++k) {
      lp.off[comp * K + k] = (uint16_t)(comp * ext_l + ell + k);
      lp.prime[comp * K + k] = (uint8_t)(c->L + k);
    }
  if ((rc = launch_ntt_inv(c, acc, kF64, acc, kF64, batch, 2LL * ext_l * n, 2LL * ext_l * n, lp, s))) return rc;
  // 6. ModDown base conversion P -> Q (conv reuses the coef region)
  double* conv = coef;
  k_conv<kF64><<<dim3(kN / 256, 2, batch), 256, 0, s>>>(
      acc, 2LL * ext_l * n, (long long)ext_l * n, ell, 0, conv, 2LL * ell * n, (long long)ell * n,
      c->d_moddown + ell, 0, c->dev);
  HCK_CHECK_LAUNCH();
  // 7. NTT(conv)
  LimbList lc2;
  lc2.n = 2 * ell;
  for (int comp = 0; comp < 2; ++comp)
    for (int i = 0; i < ell; ++i) {
      lc2.off[comp * ell + i] = (uint16_t)(comp * ell + i);
      lc2.prime[comp * ell + i] = (uint8_t)i;
    }
  if ((rc = launch_ntt_fwd(c, conv, kF64, conv, kF64, batch, 2LL * ell * n, 2LL * ell * n, lc2, s))) return rc;
  // 8. combine
  k_moddown_combine<<<dim3(kN / 256, ell, 2 * batch), 256, 0, s>>>(
      acc, conv, add, add_stride, out_b, out_a, out_stride, ell, c->d_level + ell, c->dev);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

}  // namespace
}  // namespace hck

extern "C" size_t hck_keyswitch_workspace_bytes(const hck_context* ctx, int level_limbs, int batch) {
  if (!ctx || level_limbs < 1 || level_limbs > ctx->L || batch < 0) return 0;
  const int chunk = batch < hck::kMaxBatch ? batch : hck::kMaxBatch;
  return hck::ks_layout(ctx, level_limbs, chunk).total;
}

extern "C" int hck_keyswitch(const hck_context* ctx, int level_limbs, int batch, const uint64_t* d,
                             int64_t d_stride, const uint64_t* const* ksk, const uint64_t* add_b,
                             int64_t add_stride, uint64_t* out_b, uint64_t* out_a, int64_t out_stride,
                             void* workspace, size_t workspace_bytes, void* stream) {
  if (!ctx || !d || !ksk || !out_b || !out_a || batch < 0) return HCK_ERR_ARG;
  if (level_limbs < 1 || level_limbs > ctx->L) return HCK_ERR_ARG;
  if (batch == 0) return HCK_OK;
  for (int b = 0; b < batch; ++b) if (!ksk[b]) return HCK_ERR_ARG;
  const int chunk = batch < hck::kMaxBatch ? batch : hck::kMaxBatch;
  if (!workspace || workspace_bytes < hck::ks_layout(ctx, level_limbs, chunk).total) return HCK_ERR_WORKSPACE;
  for (int b0 = 0; b0 < batch; b0 += chunk) {
    const int nb = batch - b0 < chunk ? batch - b0 : chunk;
    int rc = hck::keyswitch_chunk(ctx, level_limbs, nb, d + (long long)b0 * d_stride, d_stride, ksk + b0,
                                  add_b ? add_b + (long long)b0 * add_stride : nullptr, add_stride,
                                  out_b + (long long)b0 * out_stride, out_a + (long long)b0 * out_stride,
                                  out_stride, (char*)workspace, (hipStream_t)stream);
    if (rc) return rc;
  }
  return HCK_OK;
}

extern "C" size_t hck_rotate_workspace_bytes(const hck_context* ctx, int level_limbs, int batch) {
  if (!ctx || level_limbs < 1 || level_limbs > ctx->L || batch < 0) return 0;
  const int chunk = batch < hck::kMaxBatch ? batch : hck::kMaxBatch;
  return hck::ks_layout(ctx, level_limbs, chunk).total + (size_t)2 * batch * level_limbs * hck::kN * 8;
}

extern "C" int hck_rotate(const hck_context* ctx, int level_limbs, int batch, uint32_t galois,
                          const uint64_t* c0, const uint64_t* c1, int64_t in_stride,
                          const uint64_t* const* ksk, uint64_t* out0, uint64_t* out1, int64_t out_stride,
                          void* workspace, size_t workspace_bytes, void* stream) {
  if (!ctx || !c0 || !c1 || !ksk || !out0 || !out1 || batch < 0) return HCK_ERR_ARG;
  if (level_limbs < 1 || level_limbs > ctx->L) return HCK_ERR_ARG;
  if (batch == 0) return HCK_OK;
  if (!workspace || workspace_bytes < hck_rotate_workspace_bytes(ctx, level_limbs, batch)) return HCK_ERR_WORKSPACE;
  const long long ln = (long long)level_limbs * hck::kN;
  uint64_t* r0 = (uint64_t*)workspace;
  uint64_t* r1 = r0 + (long long)batch * ln;
  char* ks_ws = (char*)(r1 + (long long)batch * ln);
  int rc = hck_automorphism(ctx, c0, r0, batch, in_stride, ln, level_limbs, galois, stream);
  if (rc) return rc;
  if ((rc = hck_automorphism(ctx, c1, r1, batch, in_stride, ln, level_limbs, galois, stream))) return rc;
  return hck_keyswitch(ctx, level_limbs, batch, r1, ln, ksk, r0, ln, out0, out1, out_stride, ks_ws,
                       workspace_bytes - (size_t)((char*)ks_ws - (char*)workspace), stream);
}

extern "C" size_t hck_rescale_workspace_bytes(const hck_context* ctx, int level_limbs, int polys) {
  if (!ctx || level_limbs < 2 || level_limbs > ctx->L || polys < 0) return 0;
  return (size_t)polys * hck::kN * 8 * (1 + (size_t)(level_limbs - 1));
}

extern "C" int hck_rescale(const hck_context* ctx, int level_limbs, int polys, const uint64_t* in,
                           int64_t in_stride, uint64_t* out, int64_t out_stride, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (!ctx || !in || !out || polys < 0 || polys > 65535) return HCK_ERR_ARG;
  if (level_limbs < 2 || level_limbs > ctx->L) return HCK_ERR_ARG;
  if (polys == 0) return HCK_OK;
  if (!workspace || workspace_bytes < hck_rescale_workspace_bytes(ctx, level_limbs, polys)) return HCK_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  const int ell = level_limbs;
  uint64_t* last = (uint64_t*)workspace;                    // [polys][N]
  double* spread = (double*)(last + (size_t)polys * hck::kN);  // [polys][ell-1][N]
  hck::LimbList l1;
  l1.n = 1;
  l1.off[0] = 0;
  l1.prime[0] = (uint8_t)(ell - 1);
  int rc = hck::launch_ntt_inv(ctx, in + (long long)(ell - 1) * hck::kN, hck::kU64, last, hck::kU64, polys,
                               in_stride, hck::kN, l1, s);
  if (rc) return rc;
  hck::k_rescale_spread<<<dim3(hck::kN / 256, ell - 1, polys), 256, 0, s>>>(last, spread, ell, ctx->dev);
  HCK_CHECK_LAUNCH();
  hck::LimbList lq;
  lq.n = ell - 1;
  for (int i = 0; i < ell - 1; ++i) { lq.off[i] = (uint16_t)i; lq.prime[i] = (uint8_t)i; }
  if ((rc = hck::launch_ntt_fwd(ctx, spread, hck::kF64, spread, hck::kF64, polys, (long long)(ell - 1) * hck::kN,
                                (long long)(ell - 1) * hck::kN, lq, s)))
    return rc;
  hck::k_rescale_combine<<<dim3(hck::kN / 256, ell - 1, polys), 256, 0, s>>>(
      in, in_stride, spread, out, out_stride, ell, ctx->d_level + ell, ctx->dev);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}
