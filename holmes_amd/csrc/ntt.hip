// Negacyclic NTT / INTT for N = 2^16 on gfx950: two LDS-staged passes of 8 stages each.
//
// Transform convention (bench/cmp/kernels/holmes_encode.cu:75-78): forward stage l (0..15) pairs
// n and n + 2^(15-l) with root psi_rev[2^l + (n >> (16 - l))], Cooley-Tukey butterflies,
// bit-reversed evaluation order out.  The inverse runs the stages in reverse order with
// Gentleman-Sande butterflies on psi^-1 powers and folds N^-1 into its last stage.
//
// View a limb as a 256 x 256 row-major matrix (row r = n >> 8, column c = n & 255).
//   pass "cols" = stages 0..7: butterflies stay inside a column; every column uses the same 255
//                 roots (index 2^l + (r >> (8 - l))), so those loads are wave-uniform.
//   pass "rows" = stages 8..15: butterflies stay inside a contiguous 256-word row.
// A workgroup of 256 threads (4 wave64) owns 16 columns (or 16 rows) = 4096 words; each thread
// holds 16 words in registers and runs 4 stages as a radix-16 step, exchanges through LDS, and
// runs the next 4.  Global loads and stores are 128-byte coalesced: 16 consecutive lanes touch 16
// consecutive words.  Between the passes the limb is kept in HBM as signed-lazy doubles
// (modarith.hpp), so only the final pass canonicalises.
//
// Lazy-reduction bounds (p < 2^50, mulv error model of modarith.hpp): forward stages reduce the
// sum operand on even stages only; with B_e, B_o the bounds (in units of p) after even and odd
// stages, B_e = 1 + 0.375 B_o and B_o = 0.5 + 1.375 B_e, so values stay below 2.45 p and 3.9 p
// (< 2^52).  Inverse stages reduce every sum: values stay below 2 p.
#include <hip/hip_runtime.h>

#include "../../include/holmes_ckks.h"
#include "internal.hpp"
#include "wide.hpp"

namespace hck {
namespace {

constexpr int kThreads = 256;
// cols: element (row r, column cl) at (r + (r >> 4)) * 16 + cl; rows: element (row rb, col c) at
// rb * 272 + c + (c >> 4).  Both keep 16- and 32-lane groups of every exchange conflict-free.
constexpr int kLds = 16 * 272;

__device__ __forceinline__ int cidx(int r, int cl) { return (r + (r >> 4)) * 16 + cl; }
__device__ __forceinline__ int ridx(int rb, int c) { return rb * 272 + c + (c >> 4); }

template <bool RED>
__device__ __forceinline__ void ct(double& u, double& v, const double w, double p, double pinv) {
  const double m = mulv(v, w, p, pinv);
  const double a = RED ? reduce(u, p, pinv) : u;
  u = a + m;
  v = a - m;
}

__device__ __forceinline__ void gs(double& u, double& v, const double w, double p, double pinv) {
  const double s = u + v, d = u - v;
  u = reduce(s, p, pinv);
  v = mulv(d, w, p, pinv);
}

template <Fmt F>
__device__ __forceinline__ double ld(const void* base, long long i) {
  if constexpr (F == kU64) return u2d(((const uint64_t*)base)[i]);
  else return ((const double*)base)[i];
}

template <Fmt F>
__device__ __forceinline__ void st(void* base, long long i, double x, double p, double pinv) {
  if constexpr (F == kU64) ((uint64_t*)base)[i] = d2u(canon(x, p, pinv));
  else ((double*)base)[i] = x;
}

// ---------------------------------------------------------------------------- forward, cols
template <Fmt IN>
__global__ __launch_bounds__(kThreads) void k_fwd_cols(const void* __restrict__ src, void* dst,
                                                       long long src_stride, long long dst_stride,
                                                       LimbList list, DevTables T) {
  __shared__ double sh[kLds];
  const int e = blockIdx.y;
  const int pi = list.prime[e];
  const double p = T.p[pi], pinv = T.pinv[pi];
  const double* __restrict__ tw = T.tw_fwd + (size_t)pi * kN;
  const long long lo = (long long)list.off[e] * kN;
  const char* s = (const char*)src + ((long long)blockIdx.z * src_stride + lo) * 8;
  char* d = (char*)dst + ((long long)blockIdx.z * dst_stride + lo) * 8;
  const int tid = threadIdx.x, cl = tid & 15, j = tid >> 4, c = blockIdx.x * 16 + cl;
  double x[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = ld<IN>(s, (long long)(j + 16 * k) * 256 + c);
  // stages 0..3: rows j + 16k, pair distance 2^(3-l) in k, root 2^l + (k >> (4 - l))
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    const int h = 8 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      const double w = tw[(1 << l) + (k >> (4 - l))];
      if (l & 1) ct<false>(x[k], x[k + h], w, p, pinv);
      else ct<true>(x[k], x[k + h], w, p, pinv);
    }
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) sh[cidx(j + 16 * k, cl)] = x[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = sh[cidx(16 * j + k, cl)];
  // stages 4..7: rows 16j + k, pair distance 2^(7-l), root 2^l + (j << (l - 4)) + (k >> (8 - l))
#pragma unroll
  for (int l = 4; l < 8; ++l) {
    const int h = 128 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      const double w = tw[(1 << l) + (j << (l - 4)) + (k >> (8 - l))];
      if (l & 1) ct<false>(x[k], x[k + h], w, p, pinv);
      else ct<true>(x[k], x[k + h], w, p, pinv);
    }
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) ((double*)d)[(long long)(16 * j + k) * 256 + c] = x[k];
}

// ---------------------------------------------------------------------------- forward, rows
template <Fmt OUT>
__global__ __launch_bounds__(kThreads) void k_fwd_rows(void* data, long long stride, LimbList list,
                                                       DevTables T) {
  __shared__ double sh[kLds];
  const int e = blockIdx.y;
  const int pi = list.prime[e];
  const double p = T.p[pi], pinv = T.pinv[pi];
  const double* __restrict__ tw = T.tw_fwd + (size_t)pi * kN;
  char* base = (char*)data + ((long long)blockIdx.z * stride + (long long)list.off[e] * kN) * 8;
  const int tid = threadIdx.x, j = tid & 15, rb = tid >> 4, b = blockIdx.x * 16 + rb;
  double* row = (double*)base + (long long)b * 256;
  double x[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = row[j + 16 * k];
  // stages 8..11: c = j + 16k, pair distance 2^(11-l) in k, root 2^l + (b << (l-8)) + (k >> (12-l))
#pragma unroll
  for (int l = 8; l < 12; ++l) {
    const int h = 2048 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      const double w = tw[(1 << l) + (b << (l - 8)) + (k >> (12 - l))];
      if (l & 1) ct<false>(x[k], x[k + h], w, p, pinv);
      else ct<true>(x[k], x[k + h], w, p, pinv);
    }
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) sh[ridx(rb, j + 16 * k)] = x[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = sh[ridx(rb, 16 * j + k)];
  // stages 12..15: c = 16j + k, root 2^l + (b << (l-8)) + (j << (l-12)) + (k >> (16-l))
#pragma unroll
  for (int l = 12; l < 16; ++l) {
    const int h = 32768 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      const double w = tw[(1 << l) + (b << (l - 8)) + (j << (l - 12)) + (k >> (16 - l))];
      if (l & 1) ct<false>(x[k], x[k + h], w, p, pinv);
      else ct<true>(x[k], x[k + h], w, p, pinv);
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) sh[ridx(rb, 16 * j + k)] = x[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) st<OUT>(row, j + 16 * k, sh[ridx(rb, j + 16 * k)], p, pinv);
}

// ---------------------------------------------------------------------------- inverse, rows
template <Fmt IN>
__global__ __launch_bounds__(kThreads) void k_inv_rows(const void* __restrict__ src, void* dst,
                                                       long long src_stride, long long dst_stride,
                                                       LimbList list, DevTables T) {
  __shared__ double sh[kLds];
  const int e = blockIdx.y;
  const int pi = list.prime[e];
  const double p = T.p[pi], pinv = T.pinv[pi];
  const double* __restrict__ tw = T.tw_inv + (size_t)pi * kN;
  const long long lo = (long long)list.off[e] * kN;
  const char* s = (const char*)src + ((long long)blockIdx.z * src_stride + lo) * 8;
  char* d = (char*)dst + ((long long)blockIdx.z * dst_stride + lo) * 8;
  const int tid = threadIdx.x, j = tid & 15, rb = tid >> 4, b = blockIdx.x * 16 + rb;
  double x[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) sh[ridx(rb, j + 16 * k)] = ld<IN>(s, (long long)b * 256 + j + 16 * k);
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = sh[ridx(rb, 16 * j + k)];
  // stages 15..12 on c = 16j + k
#pragma unroll
  for (int l = 15; l >= 12; --l) {
    const int h = 32768 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      gs(x[k], x[k + h], tw[(1 << l) + (b << (l - 8)) + (j << (l - 12)) + (k >> (16 - l))], p, pinv);
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) sh[ridx(rb, 16 * j + k)] = x[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = sh[ridx(rb, j + 16 * k)];
  // stages 11..8 on c = j + 16k
#pragma unroll
  for (int l = 11; l >= 8; --l) {
    const int h = 2048 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      gs(x[k], x[k + h], tw[(1 << l) + (b << (l - 8)) + (k >> (12 - l))], p, pinv);
    }
  }
  double* row = (double*)d + (long long)b * 256;
#pragma unroll
  for (int k = 0; k < 16; ++k) row[j + 16 * k] = x[k];
}

// ---------------------------------------------------------------------------- inverse, cols
template <Fmt OUT>
__global__ __launch_bounds__(kThreads) void k_inv_cols(void* data, long long stride, LimbList list,
                                                       DevTables T) {
  __shared__ double sh[kLds];
  const int e = blockIdx.y;
  const int pi = list.prime[e];
  const double p = T.p[pi], pinv = T.pinv[pi];
  const double* __restrict__ tw = T.tw_inv + (size_t)pi * kN;
  char* base = (char*)data + ((long long)blockIdx.z * stride + (long long)list.off[e] * kN) * 8;
  double* m = (double*)base;
  const int tid = threadIdx.x, cl = tid & 15, j = tid >> 4, c = blockIdx.x * 16 + cl;
  double x[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = m[(long long)(16 * j + k) * 256 + c];
  // stages 7..4 on rows 16j + k
#pragma unroll
  for (int l = 7; l >= 4; --l) {
    const int h = 128 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      gs(x[k], x[k + h], tw[(1 << l) + (j << (l - 4)) + (k >> (8 - l))], p, pinv);
    }
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) sh[cidx(16 * j + k, cl)] = x[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = sh[cidx(j + 16 * k, cl)];
  // stages 3..1 on rows j + 16k
#pragma unroll
  for (int l = 3; l >= 1; --l) {
    const int h = 8 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      gs(x[k], x[k + h], tw[(1 << l) + (k >> (4 - l))], p, pinv);
    }
  }
  // stage 0 with N^-1 folded in: (u, v) -> ((u + v) N^-1, (u - v) psi_inv_rev[1] N^-1)
  const TwPair n0 = T.ninv[pi], n1 = T.ninv_w1[pi];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const double s0 = x[k] + x[k + 8], d0 = x[k] - x[k + 8];
    x[k] = mulc(s0, n0, p);
    x[k + 8] = mulc(d0, n1, p);
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) st<OUT>(m, (long long)(j + 16 * k) * 256 + c, x[k], p, pinv);
}

// ---------------------------------------------------------------------------- encode + cols
// The encoder's last step fused with the column pass: the block of 16 columns of one plaintext row
// loads each coefficient once (the special IFFT output gathered in bit-reversed order, * 1/n,
// * scale, rounded half away from zero: coefficient n < N/2 from the real part of slot brev(n),
// n >= N/2 from the imaginary part of slot brev(n - N/2)), then for each of its limbs (lpb of them
// from blockIdx.y lpb: a launch of few rows still fills the chip) takes the residue in [0, p) and
// runs stages 0..7 exactly as k_fwd_cols<kU64> does on stored residues, so the result is
// bit-identical to rounding, storing every limb and transforming.  The residues of all limbs never
// reach HBM.  Grid (16, limb chunks, rows).
// Encoder cap: |coefficient| < 2^61, the reference's MAX_ENCODED_BITS
// (llama3fhe/operators/attention/prefill/softmax.py:559).  A rounded coefficient is an exact double
// (at and above 2^53 every double is an integer), and canon() reduces it exactly: q = floor(x / p)
// is then below 2^12 and the residue x - q p (|.| < 2p) is the exact result of one FMA.
constexpr double kEncodeCap = 2305843009213693952.0;  // 2^61

__global__ __launch_bounds__(kThreads) void k_encode_cols(const double* __restrict__ vre,
                                                          const double* __restrict__ vim, double scale,
                                                          double* __restrict__ out, long long out_stride,
                                                          LimbList list, int lpb, int* __restrict__ overflow,
                                                          DevTables T) {
  __shared__ double sh[kLds];
  const long long row = blockIdx.z;
  const int tid = threadIdx.x, cl = tid & 15, j = tid >> 4, c = blockIdx.x * 16 + cl;
  const double* re = vre + row * (kN / 2);
  const double* im = vim + row * (kN / 2);
  double a[16];
  bool big = false;
  {
#pragma clang fp contract(off)
    const double inv_n = 1.0 / (double)(kN / 2);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int n = (j + 16 * k) * 256 + c;
      const int h = n >= kN / 2;
      const int slot = (int)(__brev((unsigned)(n - h * (kN / 2))) >> (32 - (kLogN - 1)));
      const double w = (h ? im : re)[slot] * inv_n;
      a[k] = round_away(w * scale);
      big |= fabs(a[k]) >= kEncodeCap;
    }
  }
  if (big) overflow[row] = 1;
  double* d = out + row * out_stride;
  const int e_end = min(list.n, ((int)blockIdx.y + 1) * lpb);  // this block: limbs [blockIdx.y lpb, e_end)
  for (int e = (int)blockIdx.y * lpb; e < e_end; ++e) {
    const int pi = list.prime[e];
    const double p = T.p[pi], pinv = T.pinv[pi];
    const double* __restrict__ tw = T.tw_fwd + (size_t)pi * kN;
    double x[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) x[k] = canon(a[k], p, pinv);
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const int hh = 8 >> l;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        if (k & hh) continue;
        const double w = tw[(1 << l) + (k >> (4 - l))];
        if (l & 1) ct<false>(x[k], x[k + hh], w, p, pinv);
        else ct<true>(x[k], x[k + hh], w, p, pinv);
      }
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) sh[cidx(j + 16 * k, cl)] = x[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) x[k] = sh[cidx(16 * j + k, cl)];
    __syncthreads();  // the next limb rewrites sh
#pragma unroll
    for (int l = 4; l < 8; ++l) {
      const int hh = 128 >> l;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        if (k & hh) continue;
        const double w = tw[(1 << l) + (j << (l - 4)) + (k >> (8 - l))];
        if (l & 1) ct<false>(x[k], x[k + hh], w, p, pinv);
        else ct<true>(x[k], x[k + hh], w, p, pinv);
      }
    }
    double* dl = d + (long long)list.off[e] * kN;
#pragma unroll
    for (int k = 0; k < 16; ++k) dl[(long long)(16 * j + k) * 256 + c] = x[k];
  }
}

}  // namespace

int launch_ntt_fwd(const hck_context* c, const void* src, Fmt in, void* dst, Fmt out, int groups,
                   long long src_stride, long long dst_stride, const LimbList& list, hipStream_t s) {
  if (c->wide) {
    if (in != kU64 || out != kU64) return HCK_ERR_UNSUPPORTED;
    return wide_ntt(c, (const uint64_t*)src, (uint64_t*)dst, groups, src_stride, dst_stride, list, false, s);
  }
  if (list.n <= 0 || groups <= 0) return HCK_OK;
  if (list.n > kMaxList || groups > 65535) return HCK_ERR_ARG;
  const dim3 grid(16, list.n, groups);
  if (in == kU64)
    k_fwd_cols<kU64><<<grid, kThreads, 0, s>>>(src, dst, src_stride, dst_stride, list, c->dev);
  else
    k_fwd_cols<kF64><<<grid, kThreads, 0, s>>>(src, dst, src_stride, dst_stride, list, c->dev);
  if (out == kU64)
    k_fwd_rows<kU64><<<grid, kThreads, 0, s>>>(dst, dst_stride, list, c->dev);
  else
    k_fwd_rows<kF64><<<grid, kThreads, 0, s>>>(dst, dst_stride, list, c->dev);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

int launch_encode_ntt(const hck_context* c, const double* vre, const double* vim, double scale, uint64_t* out,
                      long long out_stride, int rows, int* overflow, const LimbList& list, hipStream_t s) {
  if (c->wide) return wide_encode_ntt(c, vre, vim, scale, out, out_stride, rows, overflow, list, s);
  if (list.n <= 0 || rows <= 0) return HCK_OK;
  if (list.n > kMaxList || rows > 65535) return HCK_ERR_ARG;
  // limbs split over blockIdx.y so that a launch of few rows still fills the chip (each block rounds
  // its coefficients again: the IFFT output is read from L2)
  const int lpb = encode_limbs_per_block(list.n, rows);
  k_encode_cols<<<dim3(16, (list.n + lpb - 1) / lpb, rows), kThreads, 0, s>>>(vre, vim, scale, (double*)out,
                                                                            out_stride, list, lpb, overflow, c->dev);
  k_fwd_rows<kU64><<<dim3(16, list.n, rows), kThreads, 0, s>>>(out, out_stride, list, c->dev);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

int launch_ntt_inv(const hck_context* c, const void* src, Fmt in, void* dst, Fmt out, int groups,
                   long long src_stride, long long dst_stride, const LimbList& list, hipStream_t s) {
  if (c->wide) {
    if (in != kU64 || out != kU64) return HCK_ERR_UNSUPPORTED;
    return wide_ntt(c, (const uint64_t*)src, (uint64_t*)dst, groups, src_stride, dst_stride, list, true, s);
  }
  if (list.n <= 0 || groups <= 0) return HCK_OK;
  if (list.n > kMaxList || groups > 65535) return HCK_ERR_ARG;
  const dim3 grid(16, list.n, groups);
  if (in == kU64)
    k_inv_rows<kU64><<<grid, kThreads, 0, s>>>(src, dst, src_stride, dst_stride, list, c->dev);
  else
    k_inv_rows<kF64><<<grid, kThreads, 0, s>>>(src, dst, src_stride, dst_stride, list, c->dev);
  if (out == kU64)
    k_inv_cols<kU64><<<grid, kThreads, 0, s>>>(dst, dst_stride, list, c->dev);
  else
    k_inv_cols<kF64><<<grid, kThreads, 0, s>>>(dst, dst_stride, list, c->dev);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

}  // namespace hck

namespace {
int make_list(const hck_context* ctx, int limbs, const int* prime_idx, hck::LimbList& L) {
  if (limbs < 0 || limbs > hck::kMaxList || !prime_idx) return HCK_ERR_ARG;
  L.n = limbs;
  for (int i = 0; i < limbs; ++i) {
    if (prime_idx[i] < 0 || prime_idx[i] >= ctx->np) return HCK_ERR_ARG;
    L.off[i] = (uint16_t)i;
    L.prime[i] = (uint8_t)prime_idx[i];
  }
  return HCK_OK;
}
}  // namespace

extern "C" int hck_ntt_forward(const hck_context* ctx, const uint64_t* src, uint64_t* dst, int polys,
                               int64_t src_stride, int64_t dst_stride, int limbs,
                               const int* prime_idx, void* stream) {
  if (!ctx || !src || !dst || polys < 0) return HCK_ERR_ARG;
  hck::LimbList L;
  int rc = make_list(ctx, limbs, prime_idx, L);
  if (rc) return rc;
  return hck::launch_ntt_fwd(ctx, src, hck::kU64, dst, hck::kU64, polys, src_stride, dst_stride, L,
                             (hipStream_t)stream);
}

extern "C" int hck_ntt_inverse(const hck_context* ctx, const uint64_t* src, uint64_t* dst, int polys,
                               int64_t src_stride, int64_t dst_stride, int limbs,
                               const int* prime_idx, void* stream) {
  if (!ctx || !src || !dst || polys < 0) return HCK_ERR_ARG;
  hck::LimbList L;
  int rc = make_list(ctx, limbs, prime_idx, L);
  if (rc) return rc;
  return hck::launch_ntt_inv(ctx, src, hck::kU64, dst, hck::kU64, polys, src_stride, dst_stride, L,
                             (hipStream_t)stream);
}
