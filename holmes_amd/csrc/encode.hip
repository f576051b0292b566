// CKKS plaintext encode on the GPU (full packing, slots = N/2) and BSGS diagonal packing.
//
//   k_pack_diagonals   weight rows of one BSGS chunk (llama3fhe/operators/linear/weight.py:122-154)
//   k_sifft_cols       special inverse FFT stages with half-width 16384 .. 128 (column pass)
//   k_sifft_rows       stages 64 .. 1 (row pass)
//   k_encode_cols      (ntt.hip) bit-reversed gather, * 1/n, * scale, round half away from zero
//                      (Re -> coefficient k, Im -> coefficient k + n: the interleave of
//                      bench/cmp/kernels/holmes_encode.cu:108-111), then per limb the residue and
//                      the forward NTT's column pass; k_fwd_rows finishes the NTT.
//
// The special IFFT is the textbook CKKS encoder over the rotation group; the butterfly, complex
// product and rounding are the exact IEEE operation sequence of the oracle (floating-point
// contraction is off in this file), so encoded residues are bit-identical to it.  View the
// n = 2^15 slots as a 256 x 128 matrix (k = 128 r + c): stages with half-width >= 128 pair rows of
// a column, the rest stay inside a row.  Coefficients must stay below 2^61 in magnitude (the
// reference's encoder cap); a row that overflows sets its flag and is reported to the caller.
#pragma clang fp contract(off)
#include <hip/hip_runtime.h>

#include "../../include/holmes_ckks.h"
#include "internal.hpp"
#include "wide.hpp"

namespace hck {
namespace {

constexpr int kSlots = kN / 2;  // 32768

struct Cx {
  double re, im;
};

// (u, v) -> (u + v, (u - v) * w), same operation order as the oracle
__device__ __forceinline__ void sbf(Cx& u, Cx& v, double wr, double wi) {
  const double ur = u.re + v.re, ui = u.im + v.im;
  const double dr = u.re - v.re, di = u.im - v.im;
  u.re = ur;
  u.im = ui;
  v.re = dr * wr - di * wi;
  v.im = dr * wi + di * wr;
}

__global__ __launch_bounds__(256) void k_pack_diagonals(const double* __restrict__ W, int D, int lanes,
                                                        int lane_shift, int baby_steps, int giant_base,
                                                        double* __restrict__ out) {
  const int s = blockIdx.x * 256 + threadIdx.x;
  const int row = blockIdx.y;
  const int gr = row / baby_steps, b = row % baby_steps;
  const long long g = giant_base + gr;
  const long long f = s / lanes, lane = s % lanes;
  long long o = (f - g * baby_steps) % D;
  if (o < 0) o += D;
  const long long in = (f + b + (long long)lane_shift * lane) % D;
  out[(long long)row * kSlots + s] = W[o * D + in];
}

// Column pass: block = 16 columns x 256 rows of one row-vector; thread (cl, j) holds rows j + 16k
// (stages 16384 .. 2048) then rows 16j + k (stages 1024 .. 128).  Input: real parts, and
// imaginary parts when vals_im is given (else 0).
__global__ __launch_bounds__(256) void k_sifft_cols(const double* __restrict__ vals,
                                                    const double* __restrict__ vals_im, double* __restrict__ vre,
                                                    double* __restrict__ vim, const double* __restrict__ twr,
                                                    const double* __restrict__ twi) {
  __shared__ double S[16 * 272];
  const long long row = blockIdx.y;
  const double* v = vals + row * kSlots;
  const double* vi = vals_im ? vals_im + row * kSlots : nullptr;
  const int t = threadIdx.x, cl = t & 15, j = t >> 4, c = blockIdx.x * 16 + cl;
  Cx x[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int at = (j + 16 * k) * 128 + c;
    x[k] = Cx{v[at], vi ? vi[at] : 0.0};
  }
  // rows r = j + 16k: half-width 128 * 2^tt pairs r and r + 2^tt, tt = 7 .. 4 (k bits 3 .. 0)
#pragma unroll
  for (int tt = 7; tt >= 4; --tt) {
    const int h = 128 << tt, kd = 1 << (tt - 4);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & kd) continue;
      const int r = j + 16 * k;
      const int jj = 128 * (r & ((1 << tt) - 1)) + c;  // position inside the butterfly block
      sbf(x[k], x[k + kd], twr[h - 1 + jj], twi[h - 1 + jj]);
    }
  }
  // exchange rows j + 16k -> rows 16j + k (real parts, then imaginary parts)
#pragma unroll
  for (int part = 0; part < 2; ++part) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int r = j + 16 * k;
      S[cl * 272 + r + (r >> 4)] = part ? x[k].im : x[k].re;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int r = 16 * j + k;
      const double y = S[cl * 272 + r + (r >> 4)];
      if (part) x[k].im = y; else x[k].re = y;
    }
    __syncthreads();
  }
  // rows r = 16j + k: tt = 3 .. 0 (k bits 3 .. 0)
#pragma unroll
  for (int tt = 3; tt >= 0; --tt) {
    const int h = 128 << tt, kd = 1 << tt;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & kd) continue;
      const int r = 16 * j + k;
      const int jj = 128 * (r & ((1 << tt) - 1)) + c;
      sbf(x[k], x[k + kd], twr[h - 1 + jj], twi[h - 1 + jj]);
    }
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const long long idx = row * kSlots + (long long)(16 * j + k) * 128 + c;
    vre[idx] = x[k].re;
    vim[idx] = x[k].im;
  }
}

// Row pass: block = 32 rows of 128; thread (rr, j), j < 8, holds c = j + 8k (half-widths 64 .. 8)
// then c = 16j + k (half-widths 4 .. 1).  In place.
__global__ __launch_bounds__(256) void k_sifft_rows(double* __restrict__ vre, double* __restrict__ vim,
                                                    const double* __restrict__ twr, const double* __restrict__ twi) {
  __shared__ double S[32 * 136];
  const long long row = blockIdx.y;
  const int t = threadIdx.x, j = t & 7, rr = t >> 3, r = blockIdx.x * 32 + rr;
  double* re = vre + row * kSlots + (long long)r * 128;
  double* im = vim + row * kSlots + (long long)r * 128;
  Cx x[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) x[k] = Cx{re[j + 8 * k], im[j + 8 * k]};
  // c = j + 8k: half-width h = 8 * 2^tt pairs k and k + 2^tt, tt = 3 .. 0; position c mod h
#pragma unroll
  for (int tt = 3; tt >= 0; --tt) {
    const int h = 8 << tt, kd = 1 << tt;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & kd) continue;
      const int cc = (j + 8 * k) & (h - 1);
      sbf(x[k], x[k + kd], twr[h - 1 + cc], twi[h - 1 + cc]);
    }
  }
#pragma unroll
  for (int part = 0; part < 2; ++part) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int cc = j + 8 * k;
      S[rr * 136 + cc + (cc >> 4)] = part ? x[k].im : x[k].re;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int cc = 16 * j + k;
      const double y = S[rr * 136 + cc + (cc >> 4)];
      if (part) x[k].im = y; else x[k].re = y;
    }
    __syncthreads();
  }
  // c = 16j + k: half-widths 4, 2, 1 (k bits 2 .. 0)
#pragma unroll
  for (int tt = 2; tt >= 0; --tt) {
    const int h = 1 << tt;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      const int cc = (16 * j + k) & (h - 1);
      sbf(x[k], x[k + h], twr[h - 1 + cc], twi[h - 1 + cc]);
    }
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    re[16 * j + k] = x[k].re;
    im[16 * j + k] = x[k].im;
  }
}

}  // namespace
}  // namespace hck

extern "C" int hck_pack_diagonals(const hck_context* ctx, const double* weight, int dimension, int lanes,
                                  int lane_shift, int baby_steps, int giant_base, int giant_count,
                                  double* out, void* stream) {
  if (!ctx || !weight || !out || dimension < 1 || lanes < 1 || lane_shift < 0 || baby_steps < 1 ||
      giant_base < 0 || giant_count < 1)
    return HCK_ERR_ARG;
  const long long rows = (long long)giant_count * baby_steps;
  if (rows > 65535) return HCK_ERR_ARG;
  hck::k_pack_diagonals<<<dim3(hck::kSlots / 256, (unsigned)rows), 256, 0, (hipStream_t)stream>>>(
      weight, dimension, lanes, lane_shift, baby_steps, giant_base, out);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

extern "C" size_t hck_encode_workspace_bytes(const hck_context* ctx, int rows) {
  if (!ctx || rows < 0) return 0;
  return (size_t)rows * hck::kSlots * 2 * sizeof(double) + (size_t)rows * sizeof(int) + 256;
}

extern "C" int hck_encode(const hck_context* ctx, const double* values, const double* values_im, int rows,
                          double scale, int limbs, const int* prime_idx, uint64_t* out, int64_t out_row_stride,
                          void* workspace, size_t workspace_bytes, int* overflow_flags, void* stream) {
  if (!ctx || !values || !out || !prime_idx || !overflow_flags || rows < 0 || rows > 65535) return HCK_ERR_ARG;
  if (limbs < 1 || limbs > hck::kMaxPrimes || !(scale > 0.0)) return HCK_ERR_ARG;
  if (rows == 0) return HCK_OK;
  if (!workspace || workspace_bytes < hck_encode_workspace_bytes(ctx, rows)) return HCK_ERR_WORKSPACE;
  hck::LimbList L;
  L.n = limbs;
  for (int l = 0; l < limbs; ++l) {
    if (prime_idx[l] < 0 || prime_idx[l] >= ctx->np) return HCK_ERR_ARG;
    L.off[l] = (uint16_t)l;
    L.prime[l] = (uint8_t)prime_idx[l];
  }
  hipStream_t s = (hipStream_t)stream;
  double* vre = (double*)workspace;
  double* vim = vre + (size_t)rows * hck::kSlots;
  hck::k_sifft_cols<<<dim3(128 / 16, rows), 256, 0, s>>>(values, values_im, vre, vim, ctx->d_enc_twr,
                                                          ctx->d_enc_twi);
  HCK_CHECK_LAUNCH();
  hck::k_sifft_rows<<<dim3(256 / 32, rows), 256, 0, s>>>(vre, vim, ctx->d_enc_twr, ctx->d_enc_twi);
  HCK_CHECK_LAUNCH();
  // rounding, residues and the NTT's column pass in one kernel, then the row pass
  return hck::launch_encode_ntt(ctx, vre, vim, scale, out, out_row_stride, rows, overflow_flags, L, s);
}

// The reference's encode sidecar entry point with its argument list (bench/cmp/kernels/
// holmes_encode.cu:240-285, bound by bench/cmp/holmes_fast_stage2.py:37).  The per-limb Barrett
// tables (diffs, ratios, ks) and the launch-shape knobs (limbs_per_block, parts bit 2) belong to the
// sidecar's own kernels and are accepted but not read: residues are reduced exactly by `primes`.
extern "C" int holmes_encode_stage2(void* out, const void* in, long long in_stride, int rows, double sf, int limbs,
                                    const void* primes, const void* diffs, const void* ratios, const void* ks,
                                    const void* roots, const void* roots_shoup, void* stream, int rows_per_launch,
                                    int parts, int limbs_per_block) {
  (void)diffs;
  (void)ratios;
  (void)ks;
  (void)limbs_per_block;
  return hck::encode_stage2((uint64_t*)out, (const double*)in, in_stride, rows, sf, limbs, (const uint64_t*)primes,
                            (const uint64_t*)roots, (const uint64_t*)roots_shoup, rows_per_launch, parts,
                            (hipStream_t)stream);
}
