// Fused hybrid key switch: five kernels per batch, extended-basis limbs cross HBM once.
//
// A limb (N = 2^16 words) is a 256 x 256 matrix, n = 256 r + c.  The forward NTT runs stages
// 0..7 inside columns ("cols" pass) and 8..15 inside rows ("rows" pass); the inverse runs rows
// (15..8) then cols (7..0).  The workspace keeps limbs tile-major (tile_layout.hpp): the
// memory-bound rows kernels get the contiguous side; the VALU-bound cols kernels the strided one.
//
//   K1 ks_intt_rows   sigma_g(d) (natural, u64) --INTT rows-->                T1 (workspace)
//   K2 ks_cols_conv   T1 --INTT cols--> coefficients --ModUp conversion (LDS)--> NTT cols --> T2
//   K3 ks_rows_ip     P limbs: T2 --NTT rows--> x_j;  acc = sum_j x_j * key_j --INTT rows--> ACCP
//   K4 ks_cols_conv   ACCP --INTT cols--> ModDown conversion P -> Q --NTT cols--> T4
//   K5 ks_rows_ipq    Q limbs: acc = sum_j x_j * key_j as in K3 (d itself for the digit's own limbs);
//                     T4 --NTT rows--> v;  out = (acc - v) * P^-1 (+ sigma_g(addend)) (+ acc_in),
//                     canonical u64.  The Q-limb inner product never goes to HBM.
//
// A rotation passes its Galois element g: the NTT-domain automorphism sigma_g is a permutation of
// each limb, so K1 (and K3 for a digit's own limbs) read d = c1 and K5 reads the addend c0 through
// it, and no permuted copy of the input is written.  The optional per-component accumulators
// (acc_b, acc_a) fold a following ciphertext addition (the Horner giant step of a BSGS product)
// into the same store.
// Per ciphertext at ell = 24, K = 8, dnum 3 this moves 352 MiB (key 96 MiB) instead of the
// 648 MiB of separate transform / conversion / product kernels.  Arithmetic: modarith.hpp.
// Algorithm: the key-switch EasyFHE runs for fhe.homo_rotate (F.cv_modup, F.cv_innerproduct_*,
// F.cv_moddown; bench/cmp/report.py:26-30); key layout llama3fhe/parallel/prefill/keys.py:105-117.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "../../include/holmes_ckks.h"
#include "internal.hpp"
#include "tile_layout.hpp"
#include "wide.hpp"

namespace hck {
namespace {

constexpr int kT = 256;          // threads per workgroup
constexpr int kMaxBatchF = 64;   // ciphertexts per launch (key pointers passed by value)
constexpr int kSrcMax = 8;       // source limbs of one conversion held in LDS
constexpr int kYStride = 272;    // LDS stride of one (source, column) run of 256 values

struct KeyPtrsF {
  const uint64_t* k[kMaxBatchF];
};

// Galois element per ciphertext of a launch (a batch of rotations by different amounts), or one for
// all (then the batch may exceed kMaxBatchF).  The value is uniform over a workgroup.
struct GalF {
  int per_item;
  uint32_t uniform;
  uint32_t g[kMaxBatchF];
};
__device__ __forceinline__ uint32_t gal_of(const GalF& G, int b) { return G.per_item ? G.g[b] : G.uniform; }
inline GalF gal_uniform(uint32_t g) {
  GalF G{};
  G.per_item = 0;
  G.uniform = g;
  return G;
}

template <bool RED>
__device__ __forceinline__ void ct_bf(double& u, double& v, const double w, double p, double pinv) {
  const double m = mulv(v, w, p, pinv);
  const double a = RED ? reduce(u, p, pinv) : u;
  u = a + m;
  v = a - m;
}

__device__ __forceinline__ void gs_bf(double& u, double& v, const double w, double p, double pinv) {
  const double s = u + v, d = u - v;
  u = reduce(s, p, pinv);
  v = mulv(d, w, p, pinv);
}

// ----------------------------------------------------------------- column transforms (16 threads)
// forward stages 0..3 on layout A.  Inputs already within p/2 + 1 (REDUCED) skip the reduction
// of stage 0; the bounds after stage 1 are then those of the reducing schedule (<= 2.15 p).
template <bool REDUCED = false>
__device__ __forceinline__ void col_fwd_lo(double (&x)[16], const double* __restrict__ tw, double p, double pinv) {
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    const int h = 8 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      const double w = tw[(1 << l) + (k >> (4 - l))];
      if ((l & 1) || (REDUCED && l == 0)) ct_bf<false>(x[k], x[k + h], w, p, pinv);
      else ct_bf<true>(x[k], x[k + h], w, p, pinv);
    }
  }
}

// forward stages 4..7 on layout B
__device__ __forceinline__ void col_fwd_hi(double (&x)[16], int j, const double* __restrict__ tw, double p,
                                           double pinv) {
#pragma unroll
  for (int l = 4; l < 8; ++l) {
    const int h = 128 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      const double w = tw[(1 << l) + (j << (l - 4)) + (k >> (8 - l))];
      if (l & 1) ct_bf<false>(x[k], x[k + h], w, p, pinv);
      else ct_bf<true>(x[k], x[k + h], w, p, pinv);
    }
  }
}

// inverse stages 7..4 on layout B
__device__ __forceinline__ void col_inv_hi(double (&x)[16], int j, const double* __restrict__ tw, double p,
                                           double pinv) {
#pragma unroll
  for (int l = 7; l >= 4; --l) {
    const int h = 128 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      gs_bf(x[k], x[k + h], tw[(1 << l) + (j << (l - 4)) + (k >> (8 - l))], p, pinv);
    }
  }
}

// inverse stages 3..0 on layout A, N^-1 folded into stage 0
__device__ __forceinline__ void col_inv_lo(double (&x)[16], const double* __restrict__ tw, TwPair n0, TwPair n1,
                                           double p, double pinv) {
#pragma unroll
  for (int l = 3; l >= 1; --l) {
    const int h = 8 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      gs_bf(x[k], x[k + h], tw[(1 << l) + (k >> (4 - l))], p, pinv);
    }
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const double s = x[k] + x[k + 8], d = x[k] - x[k + 8];
    x[k] = mulc(s, n0, p);
    x[k + 8] = mulc(d, n1, p);
  }
}

// ----------------------------------------------------------------- row transforms (256 threads)
// forward stages 8..11 on layout A for row b
__device__ __forceinline__ void row_fwd_lo(double (&x)[16], int b, const double* __restrict__ tw, double p,
                                           double pinv) {
#pragma unroll
  for (int l = 8; l < 12; ++l) {
    const int h = 2048 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      const double w = tw[(1 << l) + (b << (l - 8)) + (k >> (12 - l))];
      if (l & 1) ct_bf<false>(x[k], x[k + h], w, p, pinv);
      else ct_bf<true>(x[k], x[k + h], w, p, pinv);
    }
  }
}

// forward stages 12..15 on layout B
__device__ __forceinline__ void row_fwd_hi(double (&x)[16], int b, int j, const double* __restrict__ tw, double p,
                                           double pinv) {
#pragma unroll
  for (int l = 12; l < 16; ++l) {
    const int h = 32768 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      const double w = tw[(1 << l) + (b << (l - 8)) + (j << (l - 12)) + (k >> (16 - l))];
      if (l & 1) ct_bf<false>(x[k], x[k + h], w, p, pinv);
      else ct_bf<true>(x[k], x[k + h], w, p, pinv);
    }
  }
}

// inverse stages 15..12 on layout B
__device__ __forceinline__ void row_inv_hi(double (&x)[16], int b, int j, const double* __restrict__ tw, double p,
                                           double pinv) {
#pragma unroll
  for (int l = 15; l >= 12; --l) {
    const int h = 32768 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      gs_bf(x[k], x[k + h], tw[(1 << l) + (b << (l - 8)) + (j << (l - 12)) + (k >> (16 - l))], p, pinv);
    }
  }
}

// inverse stages 11..8 on layout A
__device__ __forceinline__ void row_inv_lo(double (&x)[16], int b, const double* __restrict__ tw, double p,
                                           double pinv) {
#pragma unroll
  for (int l = 11; l >= 8; --l) {
    const int h = 2048 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      gs_bf(x[k], x[k + h], tw[(1 << l) + (b << (l - 8)) + (k >> (12 - l))], p, pinv);
    }
  }
}

// 16 words of one natural-layout limb for the thread at natural offset na (+16k), read through
// sigma_g (g == 1: the identity, plain coalesced loads).
__device__ __forceinline__ void load_gal(double (&x)[16], const uint64_t* __restrict__ limb, long long na,
                                         uint32_t g) {
  if (g == 1u) {
#pragma unroll
    for (int k = 0; k < 16; ++k) x[k] = u2d(limb[na + 16 * k]);
  } else {
#pragma unroll
    for (int k = 0; k < 16; ++k) x[k] = u2d(limb[gal_src(na + 16 * k, g)]);
  }
}

// NTT rows pass of row group g, x loaded by load_t (map T, layout A); returns layout A under map N
// (thread owns natural words nat_a(g) + 16k).
__device__ __forceinline__ void rows_fwd_t(double (&x)[16], int g, double* S, const double* __restrict__ tw,
                                           double p, double pinv) {
  const RowMap mt = map_t(), mn = map_n();
  row_fwd_lo(x, g + 16 * mt.rb, tw, p, pinv);
  row_xchg<true, false>(x, S, mt, mn);
  row_fwd_hi(x, g + 16 * mn.rb, mn.j, tw, p, pinv);
  row_xchg<false, true>(x, S, mn, mn);
}

// INTT rows pass of row group g held in layout A under map N; stores the result to the workspace.
__device__ __forceinline__ void rows_inv_to_t(double (&x)[16], double* __restrict__ dst_t, int g, double* S,
                                              const double* __restrict__ tw, double p, double pinv) {
  const RowMap mt = map_t(), mn = map_n();
  row_xchg<true, false>(x, S, mn, mn);
  row_inv_hi(x, g + 16 * mn.rb, mn.j, tw, p, pinv);
  row_xchg<false, true>(x, S, mn, mt);
  row_inv_lo(x, g + 16 * mt.rb, tw, p, pinv);
#pragma unroll
  for (int k = 0; k < 16; ++k) dst_t[ws_a(g, k)] = x[k];
}

// ----------------------------------------------------------------- K1: INTT rows of d
// Limb i (< limbs) of poly b reads input limb limb0 + i under prime prime0 + i and writes output
// limb i of a `limbs`-limb workspace poly.  1-D grid over (poly, limb, row group) tiles, decoded so
// that the polys of one tile run on one XCD back to back (the XCDs take workgroups round-robin):
// each row group's twiddles are then fetched into one XCD's L2, not into all eight.
__device__ __forceinline__ void intt_rows_body(const uint64_t* __restrict__ d, long long d_stride, const GalF& G,
                                               int limb0, int prime0, double* __restrict__ t1, int limbs, int batch,
                                               const DevTables& T, int lin, double* S, int koff = 0) {
  const int xcd = lin % kXcds, q = lin / kXcds;
  const int tile = (q / batch) * kXcds + xcd, b = q % batch;
  if (tile >= 16 * limbs) return;
  const int i = tile >> 4, rg = tile & 15;
  const int pi = prime0 + i;
  const double p = T.p[pi], pinv = T.pinv[pi];
  const double* __restrict__ tw = T.tw_inv + (size_t)pi * kN;
  double x[16];
  load_gal(x, d + (long long)b * d_stride + (long long)(limb0 + i) * kN, nat_a(rg), gal_of(G, koff + b));
  rows_inv_to_t(x, t1 + ((long long)b * limbs + i) * kN, rg, S, tw, p, pinv);
}

__global__ __launch_bounds__(kT) void k_ks_intt_rows(const uint64_t* __restrict__ d, long long d_stride,
                                                     const GalF G, int limb0, int prime0, double* __restrict__ t1,
                                                     int limbs, int batch, DevTables T) {
  __shared__ double S[kRowLds];
  intt_rows_body(d, d_stride, G, limb0, prime0, t1, limbs, batch, T, blockIdx.x, S);
}

// ----------------------------------------------------------------- K2 / K4: cols + conversion
// Block: two columns (c0, c0 + 1) of one conversion group; 16 slots of 16 threads.  LDS holds 16 runs
// of kYStride doubles (Y).
// Phase 1: slot sigma owns (source s = sigma >> 1, column sigma & 1): it loads the column straight
// into layout B, runs the INTT col stages with run sigma as its exchange buffer (the last stage also
// multiplies by hinv_s, folded into N^-1), and leaves y_s = centered [x_s * hinv_s] in run sigma.
// Phase 2: thread j of slot sigma owns rows j + 16k of column sigma & 1 for the targets
// tg = 8 r + (sigma >> 1), r = 0 .. rounds - 1: they share that column, so each y value read from LDS
// feeds up to kRoundsFused targets at once.  Then NTT col stages per target, stored straight from
// layout B.  Without SEPX (at most kRoundsFused rounds) the exchanges reuse the Y runs after a
// barrier that follows the last read of Y; SEPX keeps separate exchange runs for more targets.
constexpr int kRoundsFused = 3;                 // targets per thread held in registers
constexpr int kTgtFused = 8 * kRoundsFused;     // targets a conversion group may have without SEPX

// The conversion kernel's arguments: source group (z, y) at src + z src_zs + y src_ys + y src_off_y
// limbs, destination group at dst + z dst_zs + y dst_ys, constants cc_base[y cc_y].
struct ConvArgs {
  const double* src;
  long long src_zs, src_ys;
  int src_off_y;
  double* dst;
  long long dst_zs, dst_ys;
  const ConvConsts* cc_base;
  int cc_y;
  const double* zsrc;  // the ModDown-rescale's extra source limb (group (z, y) at zsrc + z src_zs + y src_ys)
};

template <bool SEPX>
__device__ __forceinline__ void cols_conv_body(const ConvArgs& A, int bx, int y, long long z, double* Y, double* X,
                                               TwPair* H, const DevTables& T) {
  const double* __restrict__ src = A.src;
  double* __restrict__ dst = A.dst;
  const long long src_zs = A.src_zs, src_ys = A.src_ys, dst_zs = A.dst_zs, dst_ys = A.dst_ys;
  const int src_off_y = A.src_off_y;
  const ConvConsts* __restrict__ cc_base = A.cc_base;
  const int cc_y = A.cc_y;
  const int t = threadIdx.x, sigma = t >> 4, j = t & 15;
  const int c0 = bx * 2;
  const ConvConsts& C = cc_base[y * cc_y];
  const int ns = C.ns, nt = C.nt;
  for (int q = t; q < ns * nt; q += kT) H[q] = C.hmod[q / nt][q % nt];
  const int cl = sigma & 1;
  double* R = Y + sigma * kYStride;
  // phase 1 (ns <= 8: one task per slot)
  {
    const int s = sigma >> 1;
    const bool act = s < ns;
    const int sp = C.src_prime[act ? s : 0];
    const double p = T.p[sp], pinv = T.pinv[sp];
    const double* __restrict__ tw = T.tw_inv + (size_t)sp * kN;
    double x[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) x[k] = 0.0;
    if (act) {
      const double* col = src + z * src_zs + y * src_ys + (long long)(y * src_off_y + s) * kN +
                          (long long)(c0 + cl) * 16;
#pragma unroll
      for (int k = 0; k < 16; ++k) x[k] = col[4096 * k + j];  // rows 16 j + k: wpos = 4096 k + 16 c + j
      col_inv_hi(x, j, tw, p, pinv);
    }
    col_b_to_a(x, R, j);
    if (act) {
      col_inv_lo(x, tw, C.inv_n0[s], C.inv_n1[s], p, pinv);
      // centered lift (zero-mean): |x| <= 1.5 p, so fl(x pinv) is within 3 2^-53 of x / p while
      // x / p is at least 1 / (2p) > 4 2^-53 away from a half-integer (p odd, p < 2^50): the
      // rounding picks the nearest multiple of p and the result is the unique representative in
      // [-(p-1)/2, (p-1)/2]
#pragma unroll
      for (int k = 0; k < 16; ++k) R[j + 16 * k] = reduce(x[k], p, pinv);
    }
  }
  __syncthreads();
  // phase 2
  const int rounds = (nt + 7) / 8;
  double* dbase = dst + z * dst_zs + y * dst_ys + (long long)(c0 + cl) * 16;
  double* RX = SEPX ? X + sigma * kYStride : R;
  for (int r0 = 0; r0 < rounds; r0 += kRoundsFused) {
    double x[kRoundsFused][16];
    int tg[kRoundsFused];
    double p[kRoundsFused], pinv[kRoundsFused];
#pragma unroll
    for (int u = 0; u < kRoundsFused; ++u) {
      const int tt = 8 * (r0 + u) + (sigma >> 1);
      tg[u] = tt < nt ? tt : -1;
      const int tp = C.dst_prime[tt < nt ? tt : 0];
      p[u] = T.p[tp];
      pinv[u] = T.pinv[tp];
#pragma unroll
      for (int k = 0; k < 16; ++k) x[u][k] = 0.0;
    }
    for (int s = 0; s < ns; ++s) {
      const double* Yr = Y + (s * 2 + cl) * kYStride;
      TwPair h[kRoundsFused];
#pragma unroll
      for (int u = 0; u < kRoundsFused; ++u) h[u] = H[s * nt + (tg[u] < 0 ? 0 : tg[u])];
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const double v = Yr[j + 16 * k];
#pragma unroll
        for (int u = 0; u < kRoundsFused; ++u) x[u][k] += mulc(v, h[u], p[u]);  // |term| <= 0.69 p
      }
    }
    if (!SEPX) __syncthreads();  // every slot is done reading Y before the runs become exchange buffers
#pragma unroll
    for (int u = 0; u < kRoundsFused; ++u) {
      if (r0 + u < rounds) {  // uniform across the block
        const bool act = tg[u] >= 0;
        const double* __restrict__ tw = T.tw_fwd + (size_t)C.dst_prime[act ? tg[u] : 0] * kN;
        if (act) {
#pragma unroll
          for (int k = 0; k < 16; ++k) x[u][k] = reduce(x[u][k], p[u], pinv[u]);
          col_fwd_lo<true>(x[u], tw, p[u], pinv[u]);
        }
        col_a_to_b(x[u], RX, j);
        if (act) {
          col_fwd_hi(x[u], j, tw, p[u], pinv[u]);
          double* col = dbase + (long long)C.dst_slot[tg[u]] * kN;
#pragma unroll
          for (int k = 0; k < 16; ++k) col[4096 * k + j] = x[u][k];
        }
      }
    }
  }
}

template <bool SEPX>
__global__ __launch_bounds__(kT) void k_ks_cols_conv(const ConvArgs A, DevTables T) {
  __shared__ double Y[16 * kYStride];
  __shared__ double X[SEPX ? 16 * kYStride : 1];
  __shared__ TwPair H[kSrcMax * (SEPX ? kMaxPrimes : kTgtFused)];  // H[s * nt + tg] = hmod[s][tg]
  cols_conv_body<SEPX>(A, blockIdx.x, blockIdx.y, blockIdx.z, Y, X, H, T);
}

// ----------------------------------------------------------------- K2 / K4 on the matrix cores
// The same transform as cols_conv_body, with the conversion sums on the int8 matrix cores.
// Phase 1 is unchanged except that each centered source residue y (|y| < 2^49) is stored as the
// 64-bit word of its balanced base-256 digits d_0..d_6 (byte a = d_a as int8, byte 7 zero).  The
// table ConvConsts::dig_off holds, per target t, the digits e_c of K_{s,a,t} = hmod[s][t] 256^a mod
// t (centered), so that out_t = sum_c 256^c C_c (mod t) with C_c = sum_{s,a} d_{s,a} e_{s,a,t,c}:
// for every 16 coefficients one v_mfma_i32_16x16x64_i8 per digit c computes C_c for 16 target rows
// (K = 8 sources x 8 digit bytes), |C_c| <= 56 * 128^2 < 2^20.
// Phase 2 mapping: wave w takes column w >> 1 and half w & 1 of its targets; quarter-wave g (the
// 16 lanes that form a column slot) owns MI (kMItems) targets, MFMA rows 4 g + r.  A lane's MFMA
// operand rows / columns are its lane index mod 16: the constants of row j, the digits of the
// coefficient 16 k + j of tile k; its output rows 4 g + r at column j, i.e. rows j + 16 k of its
// quarter's targets over the 16 tiles: the NTT cols pass's layout A, so the sums go straight into
// the forward transform.  (Operand layout measured: lane l supplies A row l % 16 and B column
// l % 16 with K bytes 16 (l / 16) .. +15; D row 4 (l / 16) + r, column l % 16 in register r.)
typedef int v4i __attribute__((ext_vector_type(4)));
constexpr int kMItems = 3;               // targets per quarter-wave per pass
constexpr int kMPass = 8 * kMItems;      // targets of one column per pass (two waves x 4 quarters)

// Balanced base-256 digits of an integer-valued y, |y| < 2^49: v = y + M lies in [0, 2^56) for
// M = 0x0080808080808080, and byte a of v, minus 128, is digit a (byte 7 stays 0); subtracting
// 128 from each byte is the XOR with M.  y + 1.5 2^52 puts y, offset, in the mantissa.
__device__ __forceinline__ uint64_t digit_word(double y) {
  constexpr uint64_t M = 0x0080808080808080ULL;
  const double t = y + 6755399441055744.0;  // bits(t) = 0x4338000000000000 + y
  return ((uint64_t)__double_as_longlong(t) + (M - 0x4338000000000000ULL)) ^ M;
}

// sum_c C_c 256^c mod p into [-p/2 - 1, p/2 + 1] (|C_c| < 2^20): lo = C_0..C_3 part (|lo| < 2^45),
// hi = C_4..C_6 part (|hi| < 2^37), value lo + 2^32 hi.  hi 2^32 is exact; q = rint(hi 2^32 / p)
// leaves |hi 2^32 - q p| <= 1.5 p (exact FMA), the sum with lo stays below 2^52, and reduce()
// centers it.
// The pairs a = C_0 + 256 C_1, b = C_2 + 256 C_3, d = C_4 + 256 C_5 and C_6 (each |.| < 2^29).
__device__ __forceinline__ double mconv_fold(int a, int b, int d, int c6, double p, double pinv) {
  const double lo = __builtin_fma(65536.0, (double)b, (double)a);
  const double hi = __builtin_fma(65536.0, (double)c6, (double)d);
  const double q = __builtin_rint(hi * (4294967296.0 * pinv));
  const double r = __builtin_fma(-q, p, hi * 4294967296.0) + lo;
  return reduce(r, p, pinv);
}

// mconv_fold with an integer addend r (|r| < 2^49) in the low part: |lo + r| < 2^50, and the
// fold's final sum stays below 2^52.
__device__ __forceinline__ double mconv_fold_add(int a, int b, int d, int c6, double r, double p, double pinv) {
  const double lo = __builtin_fma(65536.0, (double)b, (double)a) + r;
  const double hi = __builtin_fma(65536.0, (double)c6, (double)d);
  const double q = __builtin_rint(hi * (4294967296.0 * pinv));
  const double v = __builtin_fma(-q, p, hi * 4294967296.0) + lo;
  return reduce(v, p, pinv);
}

template <bool SEPX, int MI = kMItems>
__device__ __forceinline__ void cols_mconv_body(const ConvArgs& A, int bx, int y, long long z, double* Y, double* X,
                                                const DevTables& T) {
  const double* __restrict__ src = A.src;
  double* __restrict__ dst = A.dst;
  const ConvConsts& C = A.cc_base[y * A.cc_y];
  const int ns = C.ns, nt = C.nt;
  const int t = threadIdx.x, sigma = t >> 4, j = t & 15;
  const int c0 = bx * 2;
  uint64_t* D = reinterpret_cast<uint64_t*>(Y);
  // phase 1: slot sigma = (source sigma >> 1, column sigma & 1), as in cols_conv_body
  {
    const int s = sigma >> 1, cl = sigma & 1;
    const bool act = s < ns;
    const int sp = C.src_prime[act ? s : 0];
    const double p = T.p[sp], pinv = T.pinv[sp];
    const double* __restrict__ tw = T.tw_inv + (size_t)sp * kN;
    double x[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) x[k] = 0.0;
    if (act) {
      const double* col = src + z * A.src_zs + y * A.src_ys + (long long)(y * A.src_off_y + s) * kN +
                          (long long)(c0 + cl) * 16;
#pragma unroll
      for (int k = 0; k < 16; ++k) x[k] = col[4096 * k + j];
      col_inv_hi(x, j, tw, p, pinv);
    }
    double* R = Y + sigma * kYStride;
    col_b_to_a(x, R, j);
    if (act) col_inv_lo(x, tw, C.inv_n0[s], C.inv_n1[s], p, pinv);
    // centered lift as in cols_conv_body, then the digit word (an idle source stores zero digits)
#pragma unroll
    for (int k = 0; k < 16; ++k) D[sigma * kYStride + j + 16 * k] = act ? digit_word(reduce(x[k], p, pinv)) : 0ULL;
  }
  __syncthreads();
  // phase 2
  const int w = t >> 6, g = (t >> 4) & 3;
  const int cl = w >> 1, h = w & 1;
  const uint8_t* __restrict__ dig = T.conv_dig + C.dig_off;
  const uint64_t* B0 = D + (4 * g + cl) * kYStride + j;      // source 2 g, column cl
  const uint64_t* B1 = D + (4 * g + 2 + cl) * kYStride + j;  // source 2 g + 1
  double* RX = (SEPX ? X : Y) + sigma * kYStride;
  double* dbase = dst + z * A.dst_zs + y * A.dst_ys + (long long)(c0 + cl) * 16;
  for (int base = 0; base < nt;) {
    // mi targets per quarter in this pass (at most MI): the last pass spreads what is left over
    // every quarter, so that no wave idles while another transforms three targets
    const int mi = min(MI, (nt - base + 7) / 8);
    // constants of MFMA row j: target of quarter j >> 2, item j & 3
    const int ta = base + (4 * h + (j >> 2)) * mi + (j & 3);
    const bool arow = (j & 3) < mi && ta < nt;
    v4i av[kConvDigits];
#pragma unroll
    for (int c = 0; c < kConvDigits; ++c)
      av[c] = arow ? *reinterpret_cast<const v4i*>(dig + ((size_t)ta * kConvDigits + c) * 64 + 16 * g) : v4i{0, 0, 0, 0};
    int to[MI];
    double p[MI], pinv[MI];
#pragma unroll
    for (int r = 0; r < MI; ++r) {
      to[r] = r < mi ? base + (4 * h + g) * mi + r : nt;
      const int tp = C.dst_prime[to[r] < nt ? to[r] : 0];
      p[r] = T.p[tp];
      pinv[r] = T.pinv[tp];
    }
    double x[MI][16];
    // the next tile's digit words are read while this tile's sums are folded
    uint64_t w0 = B0[0], w1 = B1[0];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const v4i bv = {(int)(uint32_t)w0, (int)(uint32_t)(w0 >> 32), (int)(uint32_t)w1, (int)(uint32_t)(w1 >> 32)};
      v4i acc[kConvDigits];
#pragma unroll
      for (int c = 0; c < kConvDigits; ++c)
        acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[c], bv, v4i{0, 0, 0, 0}, 0, 0, 0);
      if (k < 15) {
        w0 = B0[16 * (k + 1)];
        w1 = B1[16 * (k + 1)];
      }
#pragma unroll
      for (int r = 0; r < MI; ++r) {
        x[r][k] = r < mi ? mconv_fold(acc[0][r] + (int)((uint32_t)acc[1][r] << 8),
                                      acc[2][r] + (int)((uint32_t)acc[3][r] << 8),
                                      acc[4][r] + (int)((uint32_t)acc[5][r] << 8), acc[6][r], p[r], pinv[r])
                         : 0.0;
        // the fold happens here, in its tile: sunk to its use in the transform, every tile's
        // accumulators would stay live at once
        asm volatile("" : "+v"(x[r][k]));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (!SEPX) __syncthreads();  // every wave is done reading D before its runs become exchange buffers
#pragma unroll
    for (int r = 0; r < MI; ++r) {
      if (r >= mi) break;  // uniform over the block
      const bool act = to[r] < nt;
      const double* __restrict__ tw = T.tw_fwd + (size_t)C.dst_prime[act ? to[r] : 0] * kN;
      if (act) col_fwd_lo<true>(x[r], tw, p[r], pinv[r]);
      col_a_to_b(x[r], RX, j);
      if (act) {
        col_fwd_hi(x[r], j, tw, p[r], pinv[r]);
        double* col = dbase + (long long)C.dst_slot[to[r]] * kN;
#pragma unroll
        for (int k = 0; k < 16; ++k) col[4096 * k + j] = x[r][k];
      }
    }
    base += 8 * mi;
  }
}

// MI: targets per quarter-wave per pass (kMItems, or 2 for conversions of at most 16 targets: fewer
// registers, three waves per SIMD).
template <bool SEPX, int MI = kMItems>
__global__ __launch_bounds__(kT, 2) void k_ks_cols_mconv(const ConvArgs A, DevTables T) {
  __shared__ double Y[16 * kYStride];
  __shared__ double X[SEPX ? 16 * kYStride : 1];
  cols_mconv_body<SEPX, MI>(A, blockIdx.x, blockIdx.y, blockIdx.z, Y, X, T);
}

// ----------------------------------------------------------------- K4 of the ModDown fused with the rescale
// cols_mconv_body with one more source limb, Z = the q_{ell-1} limb of P * acc + IP (ConvConsts
// of d_mdrs).  After phase 1, slots 0 and 1 run Z's INTT cols (P^-1 folded into its last stage, via
// two extra LDS runs); phase 1c forms, for every coefficient of the two columns, the rescale's
// centered residue r = [Z P^-1 - sum_s y_s hmod[s][nt]]_{q_{ell-1}}, i.e. the q_{ell-1} limb of the
// ModDown output in the coefficient domain; phase 2 adds r to every stored target's conversion sum
// (whose tables carry P^-1) before the NTT cols.  With the finish of k_ks_rows_ipq_rs this yields
//   out_i = ((IP_i - NTT(conv_i)) P^-1 + acc_i - NTT(r)) q_{ell-1}^-1,
// the ModDown followed by the rescale, exactly.
__device__ __forceinline__ double undigit(uint64_t w) {
  constexpr uint64_t M = 0x0080808080808080ULL;
  return __longlong_as_double((long long)((w ^ M) - M + 0x4338000000000000ULL)) - 6755399441055744.0;
}

template <bool SEPX, int MI = kMItems>
__device__ __forceinline__ void cols_mconv_rs_body(const ConvArgs& A, int bx, int y, long long z, double* Y, double* X,
                                                   double* Z, const DevTables& T) {
  const double* __restrict__ src = A.src;
  double* __restrict__ dst = A.dst;
  const ConvConsts& C = A.cc_base[y * A.cc_y];
  const int ns = C.ns, nt = C.nt;
  const int t = threadIdx.x, sigma = t >> 4, j = t & 15;
  const int c0 = bx * 2;
  uint64_t* D = reinterpret_cast<uint64_t*>(Y);
  // phase 1: the P sources, as in cols_mconv_body
  {
    const int s = sigma >> 1, cl = sigma & 1;
    const bool act = s < ns;
    const int sp = C.src_prime[act ? s : 0];
    const double p = T.p[sp], pinv = T.pinv[sp];
    const double* __restrict__ tw = T.tw_inv + (size_t)sp * kN;
    double x[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) x[k] = 0.0;
    if (act) {
      const double* col = src + z * A.src_zs + y * A.src_ys + (long long)s * kN + (long long)(c0 + cl) * 16;
#pragma unroll
      for (int k = 0; k < 16; ++k) x[k] = col[4096 * k + j];
      col_inv_hi(x, j, tw, p, pinv);
    }
    double* R = Y + sigma * kYStride;
    col_b_to_a(x, R, j);
    if (act) col_inv_lo(x, tw, C.inv_n0[s], C.inv_n1[s], p, pinv);
#pragma unroll
    for (int k = 0; k < 16; ++k) D[sigma * kYStride + j + 16 * k] = act ? digit_word(reduce(x[k], p, pinv)) : 0ULL;
    // phase 1b: Z's columns on slots 0 and 1 (one wave), Z P^-1 centered into run cl of Z
    if (sigma < 2) {
      const int zp = C.dst_prime[nt];
      const double pz = T.p[zp], pzinv = T.pinv[zp];
      const double* __restrict__ twz = T.tw_inv + (size_t)zp * kN;
      const double* col = A.zsrc + z * A.src_zs + y * A.src_ys + (long long)(c0 + cl) * 16;
#pragma unroll
      for (int k = 0; k < 16; ++k) x[k] = col[4096 * k + j];
      col_inv_hi(x, j, twz, pz, pzinv);
      double* RZ = Z + cl * kYStride;
      col_b_to_a(x, RZ, j);
      col_inv_lo(x, twz, C.z_n0, C.z_n1, pz, pzinv);
#pragma unroll
      for (int k = 0; k < 16; ++k) RZ[j + 16 * k] = reduce(x[k], pz, pzinv);
    }
  }
  __syncthreads();
  // phase 1c: r for the 512 coefficients of the two columns, two per thread
  {
    const int zp = C.dst_prime[nt];
    const double pz = T.p[zp], pzinv = T.pinv[zp];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int q = t + 256 * u, cl = q >> 8, pos = q & 255;
      double acc = 0.0;
      for (int s = 0; s < ns; ++s)  // |y_s| < 2^49: |term| <= p, the sum within 8 p
        acc += mulc(undigit(D[(2 * s + cl) * kYStride + pos]), C.hmod[s][nt], pz);
      // |Z - acc| <= p + 2 once acc is reduced: reduce() returns the exact centered residue
      const double v = Z[cl * kYStride + pos] - reduce(acc, pz, pzinv);
      Z[cl * kYStride + pos] = reduce(v, pz, pzinv);
    }
  }
  __syncthreads();
  // phase 2: as cols_mconv_body, r added to every conversion sum
  const int w = t >> 6, g = (t >> 4) & 3;
  const int cl = w >> 1, h = w & 1;
  const uint8_t* __restrict__ dig = T.conv_dig + C.dig_off;
  const uint64_t* B0 = D + (4 * g + cl) * kYStride + j;      // source 2 g, column cl
  const uint64_t* B1 = D + (4 * g + 2 + cl) * kYStride + j;  // source 2 g + 1
  const double* RZ = Z + cl * kYStride + j;
  double* RX = (SEPX ? X : Y) + sigma * kYStride;
  double* dbase = dst + z * A.dst_zs + y * A.dst_ys + (long long)(c0 + cl) * 16;
  for (int base = 0; base < nt;) {
    const int mi = min(MI, (nt - base + 7) / 8);  // as in cols_mconv_body
    const int ta = base + (4 * h + (j >> 2)) * mi + (j & 3);
    const bool arow = (j & 3) < mi && ta < nt;
    v4i av[kConvDigits];
#pragma unroll
    for (int c = 0; c < kConvDigits; ++c)
      av[c] = arow ? *reinterpret_cast<const v4i*>(dig + ((size_t)ta * kConvDigits + c) * 64 + 16 * g) : v4i{0, 0, 0, 0};
    int to[MI];
    double p[MI], pinv[MI];
#pragma unroll
    for (int r = 0; r < MI; ++r) {
      to[r] = r < mi ? base + (4 * h + g) * mi + r : nt;
      const int tp = C.dst_prime[to[r] < nt ? to[r] : 0];
      p[r] = T.p[tp];
      pinv[r] = T.pinv[tp];
    }
    double x[MI][16];
    uint64_t w0 = B0[0], w1 = B1[0];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const double rz = RZ[16 * k];
      const v4i bv = {(int)(uint32_t)w0, (int)(uint32_t)(w0 >> 32), (int)(uint32_t)w1, (int)(uint32_t)(w1 >> 32)};
      v4i acc[kConvDigits];
#pragma unroll
      for (int c = 0; c < kConvDigits; ++c)
        acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[c], bv, v4i{0, 0, 0, 0}, 0, 0, 0);
      if (k < 15) {
        w0 = B0[16 * (k + 1)];
        w1 = B1[16 * (k + 1)];
      }
#pragma unroll
      for (int r = 0; r < MI; ++r) {
        x[r][k] = r < mi ? mconv_fold_add(acc[0][r] + (int)((uint32_t)acc[1][r] << 8),
                                          acc[2][r] + (int)((uint32_t)acc[3][r] << 8),
                                          acc[4][r] + (int)((uint32_t)acc[5][r] << 8), acc[6][r], rz, p[r], pinv[r])
                         : 0.0;
        asm volatile("" : "+v"(x[r][k]));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (!SEPX) __syncthreads();
#pragma unroll
    for (int r = 0; r < MI; ++r) {
      if (r >= mi) break;  // uniform over the block
      const bool act = to[r] < nt;
      const double* __restrict__ tw = T.tw_fwd + (size_t)C.dst_prime[act ? to[r] : 0] * kN;
      if (act) col_fwd_lo<true>(x[r], tw, p[r], pinv[r]);
      col_a_to_b(x[r], RX, j);
      if (act) {
        col_fwd_hi(x[r], j, tw, p[r], pinv[r]);
        double* col = dbase + (long long)C.dst_slot[to[r]] * kN;
#pragma unroll
        for (int k = 0; k < 16; ++k) col[4096 * k + j] = x[r][k];
      }
    }
    base += 8 * mi;
  }
}

template <bool SEPX, int MI = kMItems>
__global__ __launch_bounds__(kT, 2) void k_ks_cols_mconv_rs(const ConvArgs A, DevTables T) {
  __shared__ double Y[16 * kYStride];
  __shared__ double X[SEPX ? 16 * kYStride : 1];
  __shared__ double Z[2 * kYStride];
  cols_mconv_rs_body<SEPX, MI>(A, blockIdx.x, blockIdx.y, blockIdx.z, Y, X, Z, T);
}

// Launches a ModUp / ModDown conversion (grid (128, groups, items)) on the engine the context
// selects; nt_max is the largest target count over the groups.
void launch_conv(const hck_context* c, const ConvArgs& A, dim3 grid, int nt_max, hipStream_t s) {
  if (c->conv_engine == 1) {
    auto k = nt_max <= 16 ? k_ks_cols_mconv<false, 2> : nt_max <= kMPass ? k_ks_cols_mconv<false> : k_ks_cols_mconv<true>;
    k<<<grid, kT, 0, s>>>(A, c->dev);
  } else {
    auto k = nt_max <= kTgtFused ? k_ks_cols_conv<false> : k_ks_cols_conv<true>;
    k<<<grid, kT, 0, s>>>(A, c->dev);
  }
}

// ----------------------------------------------------------------- forward row twiddles in LDS
// The tile kernels keep the forward twiddles of their 16 rows in LDS, so that no global load sits
// between a tile's data loads and its transform (loads retire in order: a twiddle load issued
// behind a key load would wait for it).  Row rb (row b = g + 16 rb) owns a 256-entry run at
// TW + rb * kTwRow; stage l (8..15) uses entries [2^(l-8), 2^(l-7)) of the run:
//   stages 8..11 (map T, index uniform per row): entry 2^(l-8) + t holds tw[2^l + (b << (l-8)) + t];
//   stages 12..15 (map N, lane j): entry 2^(l-8) + 16 k' + j holds tw[2^l + (b << (l-8)) + (j << (l-12)) + k'],
// so the 16 lanes of a row read 16 consecutive entries.  The odd run stride spreads the 16 rows of
// map T over distinct banks.
constexpr int kTwRow = 257;
constexpr int kTwLds = 16 * kTwRow;

__device__ __forceinline__ int tw_heap_src(int b, int m) {
  // m in [1, 256): stage l = 8 + floor(log2 m), t = m - 2^(l-8); returns the table index for entry m
  const int lv = 31 - __clz(m);  // l - 8
  int t = m - (1 << lv);
  if (lv >= 4) {                 // stored transposed: t = 16 k' + j  <->  (j << (lv-4)) + k'
    const int j = t & 15, kk = t >> 4;
    t = (j << (lv - 4)) + kk;
  }
  return (1 << (lv + 8)) + (b << lv) + t;
}

// Loads the forward twiddles of row group rg (prime table tw) into TW: issue (registers), then store.
struct TwStage {
  double v[16];
};
__device__ __forceinline__ void tw_issue(TwStage& st, const double* __restrict__ tw, int rg) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int idx = threadIdx.x + kT * i, rb = idx >> 8, m = idx & 255;
    st.v[i] = m ? tw[tw_heap_src(rg + 16 * rb, m)] : 0.0;
  }
}
__device__ __forceinline__ void tw_store(const TwStage& st, double* TW) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int idx = threadIdx.x + kT * i;
    TW[(idx >> 8) * kTwRow + (idx & 255)] = st.v[i];
  }
}

// forward stages 8..11 on layout A (map T) with the row's twiddle run R
__device__ __forceinline__ void row_fwd_lo_lds(double (&x)[16], const double* R, double p, double pinv) {
#pragma unroll
  for (int l = 8; l < 12; ++l) {
    const int h = 2048 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      const double w = R[(1 << (l - 8)) + (k >> (12 - l))];
      if (l & 1) ct_bf<false>(x[k], x[k + h], w, p, pinv);
      else ct_bf<true>(x[k], x[k + h], w, p, pinv);
    }
  }
}

// forward stages 12..15 on layout B (map N, lane j) with the row's twiddle run R
__device__ __forceinline__ void row_fwd_hi_lds(double (&x)[16], const double* R, int j, double p, double pinv) {
#pragma unroll
  for (int l = 12; l < 16; ++l) {
    const int h = 32768 >> l;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k & h) continue;
      const double w = R[(1 << (l - 8)) + 16 * (k >> (16 - l)) + j];
      if (l & 1) ct_bf<false>(x[k], x[k + h], w, p, pinv);
      else ct_bf<true>(x[k], x[k + h], w, p, pinv);
    }
  }
}

// NTT rows pass of x (map T, layout A, as load_t returns it).  The result stays in S: thread (map N)
// finds its natural words nat_a(g) + 16 k at S[s_out(k)].  S may be read until the next rows_fwd_lds,
// which starts with a barrier.
__device__ __forceinline__ int s_out(int k) {
  const RowMap mn = map_n();
  return ridx(mn.rb, mn.j + 16 * k);
}
__device__ __forceinline__ void rows_fwd_lds(double (&x)[16], double* S, const double* TW, double p, double pinv) {
  const RowMap mt = map_t(), mn = map_n();
  row_fwd_lo_lds(x, TW + mt.rb * kTwRow, p, pinv);
  __syncthreads();  // earlier readers of S are done
  row_xchg<true, false>(x, S, mt, mn);
  row_fwd_hi_lds(x, TW + mn.rb * kTwRow, mn.j, p, pinv);
#pragma unroll
  for (int k = 0; k < 16; ++k) S[ridx(mn.rb, 16 * mn.j + k)] = x[k];
  __syncthreads();
}

// ----------------------------------------------------------------- inner product of one tile
// sb / sa = sum_j x_j * key_j[comp] over the digits j of ciphertext b, extended limb e (prime pi),
// row group rg: x_j is the NTT rows pass of the ModUp output T2 (or, for the digit that contains
// limb e, d itself read through sigma_g).  The digit containing e goes first; each later digit's
// tile load is issued as soon as the previous transform has left its result in S, behind that
// digit's key loads, so the tile lands while the inner product runs.  After the last digit, `after`
// (a workspace limb, or null) is loaded into x for the caller.  TW must hold the forward twiddles
// (visible).  With ``zero`` false the products are added to sb / sa (|sb|, |sa| <= p/2 + 1 on entry:
// the grouped kernel's running sums).  Returns |sb|, |sa| <= p/2 + 1.
// Hoisted digits (HoistSrc::digits non-null): the extended digits of every input were materialised
// once in the full NTT domain (natural layout, canonical u64, [input][beta][ell + K] limbs, the own
// digit's limbs unused), and item b rotates input (src0 + b) mod inputs: each digit is then read
// through sigma_g like d itself, with no row transform (ModUp commutes with sigma_g).
struct HoistSrc {
  const uint64_t* digits;
  int inputs, src0;
};
template <bool HOIST>
__device__ __forceinline__ int hoist_input(const HoistSrc& H, int b) { return HOIST ? (H.src0 + b) % H.inputs : b; }

// Where tile_ip reads its operands: the own digit's limb e (d through sigma_g), the keys of digit jd,
// the ModUp output tile of T2 digit jd (or, hoisted, the materialised digit).
struct IpSrc {
  const uint64_t* d;
  long long d_stride;
  const double* t2b;      // T2 digit j at t2b + j * ext_l * kN
  const uint64_t* key;
  long long comp_stride;  // the key's a component follows its b component at this distance
  int L, K, ext_l, beta, own, nt2, pi, src;
  long long na;
  __device__ __forceinline__ int t2digit(int n) const { return (own >= 0 && n >= own) ? n + 1 : n; }
  __device__ __forceinline__ void keys(uint64_t (&kb)[16], uint64_t (&ka)[16], int jd) const {
    const uint64_t* kp = key + ((long long)jd * (L + K) + pi) * kN + na;
#pragma unroll
    for (int k = 0; k < 16; ++k) { kb[k] = kp[16 * k]; ka[k] = kp[comp_stride + 16 * k]; }
  }
};

template <bool HOIST>
__device__ __forceinline__ IpSrc ip_src(const uint64_t* __restrict__ d, long long d_stride,
                                        const double* __restrict__ t2, const uint64_t* __restrict__ key, int b, int e,
                                        int pi, int rg, int ell, int beta, const DevTables& T, const HoistSrc& H) {
  IpSrc I;
  I.d = d;
  I.d_stride = d_stride;
  I.key = key;
  I.L = T.L;
  I.K = T.K;
  I.ext_l = ell + T.K;
  I.beta = beta;
  const int beta_max = (T.L + T.alpha - 1) / T.alpha;
  I.comp_stride = (long long)beta_max * (T.L + T.K) * kN;
  I.own = e < ell ? e / T.alpha : -1;
  I.nt2 = beta - (I.own >= 0 ? 1 : 0);
  I.pi = pi;
  I.na = nat_a(rg);
  I.src = hoist_input<HOIST>(H, b);
  I.t2b = t2 ? t2 + ((long long)b * beta * I.ext_l + e) * kN : nullptr;
  return I;
}

// The loads of tile_ip's first step: the own digit (raw words into xr) and its keys; without an own
// digit the first T2 tile (x only), or, hoisted, the first materialised digit (xr) and its keys.  The
// tile kernels issue them before their twiddle staging, so that the data is in flight across the
// staging barrier, and call tile_ip_body with ``pre`` set.  OWN_ALWAYS: the caller's limb is a Q
// limb (an own digit exists), so no other load path joins the own digit's (a join would make the
// compiler wait for the staged twiddles before these loads).
template <bool HOIST, bool OWN_ALWAYS = false>
__device__ __forceinline__ void tile_ip_first(uint64_t (&xr)[16], double (&x)[16], uint64_t (&kb)[16],
                                              uint64_t (&ka)[16], const IpSrc& I, int e, int rg, uint32_t g,
                                              const HoistSrc& H, const double* __restrict__ after) {
  if (OWN_ALWAYS || I.own >= 0) {
    load_gal_raw(xr, I.d + (long long)I.src * I.d_stride + (long long)e * kN, I.na, g);
    I.keys(kb, ka, I.own);
  } else if constexpr (HOIST) {
    if (I.nt2 > 0) {
      const int jd = I.t2digit(0);
      load_gal_raw(xr, H.digits + ((long long)(I.src * I.beta + jd) * I.ext_l + e) * kN, I.na, g);
      I.keys(kb, ka, jd);
    }
  } else {
    const double* first = I.nt2 > 0 ? I.t2b + (long long)I.t2digit(0) * I.ext_l * kN : after;
    if (first) load_t(x, first, rg);
  }
}

template <bool HOIST, bool OWN_ALWAYS = false>
__device__ __forceinline__ void tile_ip_body(double (&sb)[16], double (&sa)[16], double (&x)[16], uint64_t (&xr)[16],
                                             uint64_t (&kb)[16], uint64_t (&ka)[16], const IpSrc& I, int e, int rg,
                                             uint32_t g, double* S, const double* TW, const double* __restrict__ after,
                                             double p, double pinv, bool zero, const HoistSrc& H, bool pre) {
  if (zero) {
#pragma unroll
    for (int k = 0; k < 16; ++k) { sb[k] = 0.0; sa[k] = 0.0; }
  }
  if (OWN_ALWAYS || I.own >= 0) {
    if (!pre) tile_ip_first<HOIST, OWN_ALWAYS>(xr, x, kb, ka, I, e, rg, g, H, after);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const double v = u2d(xr[k]);
      sb[k] += mulv(v, u2d(kb[k]), p, pinv);  // |v| < p: |term| <= 0.9p
      sa[k] += mulv(v, u2d(ka[k]), p, pinv);
    }
  }
  if constexpr (HOIST) {
    // canonical digits read through sigma_g: |term| <= 0.9p; a reduction every three digits keeps
    // the sums below p/2 + 1 + 0.9p + 3 * 0.9p < 8p <= 2^53
    for (int n = 0; n < I.nt2; ++n) {
      const int jd = I.t2digit(n);
      if (n > 0 || OWN_ALWAYS || I.own >= 0 || !pre) {
        load_gal_raw(xr, H.digits + ((long long)(I.src * I.beta + jd) * I.ext_l + e) * kN, I.na, g);
        I.keys(kb, ka, jd);
      }
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const double v = u2d(xr[k]);
        sb[k] += mulv(v, u2d(kb[k]), p, pinv);
        sa[k] += mulv(v, u2d(ka[k]), p, pinv);
      }
      if (n % 3 == 2) {
#pragma unroll
        for (int k = 0; k < 16; ++k) { sb[k] = reduce(sb[k], p, pinv); sa[k] = reduce(sa[k], p, pinv); }
      }
    }
    if (after) load_t(x, after, rg);
#pragma unroll
    for (int k = 0; k < 16; ++k) { sb[k] = reduce(sb[k], p, pinv); sa[k] = reduce(sa[k], p, pinv); }
    return;
  }
  if (OWN_ALWAYS || I.own >= 0 || !pre) {
    const double* first = I.nt2 > 0 ? I.t2b + (long long)I.t2digit(0) * I.ext_l * kN : after;
    if (first) load_t(x, first, rg);
  }
  for (int n = 0; n < I.nt2; ++n) {
    rows_fwd_lds(x, S, TW, p, pinv);
    // the keys, then the next tile: the inner product waits for the keys only, the tile lands
    // behind it.  (Keys issued before the transform would overlap it too, but with the tile, both
    // accumulators and the transform live they do not fit in 256 VGPRs.)
    I.keys(kb, ka, I.t2digit(n));
    const double* next = n + 1 < I.nt2 ? I.t2b + (long long)I.t2digit(n + 1) * I.ext_l * kN : after;
    if (next) load_t(x, next, rg);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const double v = S[s_out(k)];
      sb[k] += mulv(v, u2d(kb[k]), p, pinv);  // |v| <= 3.9p: |term| <= 2p
      sa[k] += mulv(v, u2d(ka[k]), p, pinv);
    }
    if (n % 3 == 2) {  // <= p/2 + 1 + 3 * 2p (+ 0.9p for the own digit) < 8p <= 2^53 between reductions
#pragma unroll
      for (int k = 0; k < 16; ++k) { sb[k] = reduce(sb[k], p, pinv); sa[k] = reduce(sa[k], p, pinv); }
    }
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) { sb[k] = reduce(sb[k], p, pinv); sa[k] = reduce(sa[k], p, pinv); }
}

template <bool HOIST = false>
__device__ __forceinline__ void tile_ip(double (&sb)[16], double (&sa)[16], double (&x)[16],
                                        const uint64_t* __restrict__ d, long long d_stride, uint32_t g,
                                        const double* __restrict__ t2, const uint64_t* __restrict__ key, int b,
                                        int e, int pi, int rg, int ell, int beta, double* S, const double* TW,
                                        const double* __restrict__ after, double p, double pinv,
                                        const DevTables& T, bool zero = true, HoistSrc H = HoistSrc{nullptr, 1, 0}) {
  uint64_t xr[16], kb[16], ka[16];
  const IpSrc I = ip_src<HOIST>(d, d_stride, t2, key, b, e, pi, rg, ell, beta, T, H);
  tile_ip_body<HOIST>(sb, sa, x, xr, kb, ka, I, e, rg, g, S, TW, after, p, pinv, zero, H, false);
}

// ----------------------------------------------------------------- K3: inner product, P limbs / ext
// Tile = (row group, extended limb e0 + tile / 16).  Without ext_b the kernel covers the K special
// limbs (e0 = ell): the inner product's INTT rows pass goes to ACCP (workspace layout) for the
// ModDown conversion.  With ext_b it covers all ell + K limbs (e0 = 0) and ends the key switch in the
// extended basis: it writes (P * sigma(add) + IP_b, IP_a) over Q u P as canonical NTT-domain residues
// to ext_b / ext_a ([ell + K] limbs per ciphertext, Q limbs first), plus the extended-basis
// accumulators acc_b / acc_a when given (which ext_b / ext_a may alias).
template <bool HOIST = false>
__device__ __forceinline__ void rows_ip_body(const uint64_t* __restrict__ d, long long d_stride, const GalF& G,
                                             const double* __restrict__ t2, const KeyPtrsF& keys, int ell, int beta,
                                             int batch, int tiles, int e0, double* __restrict__ accp,
                                             const uint64_t* __restrict__ add, long long add_stride, uint64_t* ext_b,
                                             uint64_t* ext_a, long long ext_stride, const uint64_t* acc_b,
                                             const uint64_t* acc_a, long long acc_stride, const DevTables& T, int lin,
                                             double* S, double* TW, int koff = 0, HoistSrc H = HoistSrc{nullptr, 1, 0}) {
  const TileId id = decode_tile(batch, lin);
  if (id.tile >= tiles) return;
  const int b = id.b, e = e0 + (id.tile >> 4), rg = id.tile & 15;
  const uint32_t g = gal_of(G, koff + b);
  const int L = T.L, K = T.K;
  const int pi = e < ell ? e : L + (e - ell);
  const double p = T.p[pi], pinv = T.pinv[pi];
  double sb[16], sa[16], x[16];
  uint64_t xr[16], kb[16], ka[16];
  const IpSrc I = ip_src<HOIST>(d, d_stride, t2, keys.k[koff + b], b, e, pi, rg, ell, beta, T, H);
  {
    TwStage st;
    tw_issue(st, T.tw_fwd + (size_t)pi * kN, rg);
    tile_ip_first<HOIST>(xr, x, kb, ka, I, e, rg, g, H, nullptr);  // in flight across the staging barrier
    tw_store(st, TW);
    __syncthreads();
  }
  tile_ip_body<HOIST>(sb, sa, x, xr, kb, ka, I, e, rg, g, S, TW, nullptr, p, pinv, true, H, true);
  const long long na = nat_a(rg);
  if (ext_b) {
    if (e < ell && add) {
      double ad[16];
      load_gal(ad, add + (long long)hoist_input<HOIST>(H, b) * add_stride + (long long)e * kN, na, g);
      const TwPair pm = T.pmodq[pi];
#pragma unroll
      for (int k = 0; k < 16; ++k) sb[k] += mulc(ad[k], pm, p);  // |sb| <= 1.5 p
    }
    if (acc_b) {
      double ab[16], aa[16];
      load_gal(ab, acc_b + (long long)b * acc_stride + (long long)e * kN, na, 1u);
      load_gal(aa, acc_a + (long long)b * acc_stride + (long long)e * kN, na, 1u);
#pragma unroll
      for (int k = 0; k < 16; ++k) { sb[k] += ab[k]; sa[k] += aa[k]; }  // |sb| <= 2.5 p
    }
    uint64_t* ob = ext_b + (long long)b * ext_stride + (long long)e * kN + na;
    uint64_t* oa = ext_a + (long long)b * ext_stride + (long long)e * kN + na;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      ob[16 * k] = d2u(canon(sb[k], p, pinv));
      oa[16 * k] = d2u(canon(sa[k], p, pinv));
    }
    return;
  }
  // P limb: INTT rows of both components, stored to the workspace for the ModDown cols kernel.
  // ACCP holds tiles / 16 limbs per component from e0 on: the K special limbs, or (ModDown fused
  // with the rescale, e0 = ell - 1) the q_{ell-1} limb first, as Z = P * acc + IP.
  const int k1 = tiles >> 4;
  if (e < ell && (add || acc_b)) {  // Z = IP + P (sigma(add) + acc): |sb| <= p/2 + 1 + 3 p before the reduction
    const TwPair pm = T.pmodq[pi];
    double t[16];
    if (add) {
      load_gal(t, add + (long long)hoist_input<HOIST>(H, b) * add_stride + (long long)e * kN, na, g);
#pragma unroll
      for (int k = 0; k < 16; ++k) sb[k] += mulc(t[k], pm, p);
    }
    if (acc_b) {
      load_gal(t, acc_b + (long long)b * acc_stride + (long long)e * kN, na, 1u);
#pragma unroll
      for (int k = 0; k < 16; ++k) sb[k] += mulc(t[k], pm, p);
      load_gal(t, acc_a + (long long)b * acc_stride + (long long)e * kN, na, 1u);
#pragma unroll
      for (int k = 0; k < 16; ++k) sa[k] += mulc(t[k], pm, p);
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) { sb[k] = reduce(sb[k], p, pinv); sa[k] = reduce(sa[k], p, pinv); }
  }
  const double* __restrict__ twi = T.tw_inv + (size_t)pi * kN;
  double* o = accp + ((long long)b * 2 * k1 + (e - e0)) * kN;
  __syncthreads();  // the inner product's reads of S are done before the exchanges rewrite it
  rows_inv_to_t(sb, o, rg, S, twi, p, pinv);
  rows_inv_to_t(sa, o + (long long)k1 * kN, rg, S, twi, p, pinv);
}

__global__ __launch_bounds__(kT, 2) void k_ks_rows_ip(const uint64_t* __restrict__ d, long long d_stride, const GalF G,
                                                   const double* __restrict__ t2, KeyPtrsF keys, int ell,
                                                   int beta, int batch, int tiles, int e0, double* __restrict__ accp,
                                                   const uint64_t* __restrict__ add, long long add_stride,
                                                   uint64_t* ext_b, uint64_t* ext_a, long long ext_stride,
                                                   const uint64_t* acc_b, const uint64_t* acc_a,
                                                   long long acc_stride, DevTables T) {
  __shared__ double S[kRowLds];
  __shared__ double TW[kTwLds];
  rows_ip_body(d, d_stride, G, t2, keys, ell, beta, batch, tiles, e0, accp, add, add_stride, ext_b, ext_a, ext_stride,
               acc_b, acc_a, acc_stride, T, blockIdx.x, S, TW);
}

// K3 of hoisted rotations (P limbs only): the digits come from HoistSrc, item b rotates input
// (H.src0 + b) mod H.inputs.
__global__ __launch_bounds__(kT, 2) void k_ks_rows_ip_h(const uint64_t* __restrict__ d, long long d_stride,
                                                     const GalF G, KeyPtrsF keys, int ell, int beta, int batch,
                                                     double* __restrict__ accp, DevTables T, HoistSrc H) {
  __shared__ double S[kRowLds];
  __shared__ double TW[kTwLds];
  rows_ip_body<true>(d, d_stride, G, nullptr, keys, ell, beta, batch, 16 * T.K, ell, accp, nullptr, 0, nullptr,
                     nullptr, 0, nullptr, nullptr, 0, T, blockIdx.x, S, TW, 0, H);
}

// One component of the ModDown finish, its T4 tile loaded in x (map T): ip <- (ip - NTT rows(v)) * P^-1,
// plus the addends, canonical store.  `next` (or nothing) is loaded into x once the transform is done.
__device__ __forceinline__ void ipq_finish(double (&ip)[16], double (&x)[16], const double* __restrict__ next,
                                           const uint64_t* __restrict__ add_limb, uint32_t g,
                                           const uint64_t* __restrict__ acc_limb, uint64_t* __restrict__ o,
                                           long long na, int rg, double* S, const double* TW, TwPair pinv_P,
                                           double p, double pinv) {
  rows_fwd_lds(x, S, TW, p, pinv);
  if (next) load_t(x, next, rg);
  double ad[16];
  if (add_limb) load_gal(ad, add_limb, na, g);
#pragma unroll
  for (int k = 0; k < 16; ++k) ip[k] = mulc(ip[k] - S[s_out(k)], pinv_P, p);  // |ip - v| <= 4.5 p: |r| <= 2.2 p
  if (add_limb) {
#pragma unroll
    for (int k = 0; k < 16; ++k) ip[k] += ad[k];
  }
  if (acc_limb) {
    load_gal(ad, acc_limb, na, 1u);
#pragma unroll
    for (int k = 0; k < 16; ++k) ip[k] += ad[k];  // |r| <= 4.2 p
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) o[16 * k] = d2u(canon(ip[k], p, pinv));
}

// ipq_finish of the ModDown fused with the rescale:
//   r <- (ip P^-1 - NTT rows(v) + sigma_g(add) + acc) q_{ell-1}^-1   (add, acc nullable),
// then the post-ops of RsPost: r <- (twice ? 2 r : r) - sub + scalar   (sub nullable, scalar 0).
__device__ __forceinline__ void ipq_finish_rs(double (&ip)[16], double (&x)[16], const double* __restrict__ next,
                                              const uint64_t* __restrict__ add_limb, uint32_t g,
                                              const uint64_t* __restrict__ acc_limb, uint64_t* __restrict__ o,
                                              long long na, int rg, double* S, const double* TW, TwPair pinv_P,
                                              TwPair ql_inv, double p, double pinv,
                                              const uint64_t* __restrict__ sub_limb = nullptr, bool twice = false,
                                              double scalar = 0.0, const uint64_t* __restrict__ px1 = nullptr,
                                              const uint64_t* __restrict__ py1 = nullptr,
                                              const uint64_t* __restrict__ px2 = nullptr,
                                              const uint64_t* __restrict__ py2 = nullptr) {
  rows_fwd_lds(x, S, TW, p, pinv);
  if (next) load_t(x, next, rg);
#pragma unroll
  for (int k = 0; k < 16; ++k) ip[k] = mulc(ip[k], pinv_P, p) - S[s_out(k)];  // |.| <= p + 3.9 p
  double ad[16];
  if (px1) {  // the tensor term formed here: x1 y1 (+ x2 y2), each product within 0.875 p
    double t[16];
    load_gal(ad, px1, na, 1u);
    load_gal(t, py1, na, 1u);
#pragma unroll
    for (int k = 0; k < 16; ++k) ip[k] += mulv(ad[k], t[k], p, pinv);
    if (px2) {
      load_gal(ad, px2, na, 1u);
      load_gal(t, py2, na, 1u);
#pragma unroll
      for (int k = 0; k < 16; ++k) ip[k] += mulv(ad[k], t[k], p, pinv);
    }
  }
  if (add_limb) {
    load_gal(ad, add_limb, na, g);
#pragma unroll
    for (int k = 0; k < 16; ++k) ip[k] += ad[k];
  }
  if (acc_limb) {
    load_gal(ad, acc_limb, na, 1u);
#pragma unroll
    for (int k = 0; k < 16; ++k) ip[k] += ad[k];  // |.| <= 6.9 p
  }
  if (!sub_limb && !twice && scalar == 0.0) {
#pragma unroll
    for (int k = 0; k < 16; ++k) o[16 * k] = d2u(canon(mulc(ip[k], ql_inv, p), p, pinv));
    return;
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) {  // |r| <= 1.5 p: |2 r - sub + scalar| <= 5 p
    const double r = mulc(ip[k], ql_inv, p);
    ip[k] = (twice ? 2.0 * r : r) + scalar;
  }
  if (sub_limb) {
    load_gal(ad, sub_limb, na, 1u);
#pragma unroll
    for (int k = 0; k < 16; ++k) ip[k] -= ad[k];
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) o[16 * k] = d2u(canon(ip[k], p, pinv));
}

// Post-ops of a rescaled product (the Chebyshev step of fhe.homo_mul_relin_rescale_postop):
// out <- (twice ? 2 out : out) - sub (+ scalar[i] on the b component).
struct RsPost {
  const uint64_t* sub_b;
  const uint64_t* sub_a;
  long long sub_stride;
  int twice, has_scalar;
  uint64_t scalar[kMaxPrimes];
  // the product's degree-0/1 terms formed in the finish instead of read as accumulators:
  // acc_b = a0 b0, acc_a = a0 b1 + a1 b0 on limbs < ell - 1 (a*, b* nullable)
  const uint64_t *a0, *a1, *b0, *b1;
  long long a_stride, b_stride;
};

// ----------------------------------------------------------------- K5: Q limbs: inner product + ModDown
// Tile = (row group, Q limb i): the inner product of limb i (as in K3) is combined with the NTT rows
// pass v of the ModDown conversion T4 right away, so the Q-limb inner product never goes to HBM:
//   out_b = (IP_b - v_b) * P^-1 + sigma_g(add) (+ acc_b),   out_a = (IP_a - v_a) * P^-1 (+ acc_a),
// canonical u64.
template <bool HOIST = false, bool RS = false>
__device__ __forceinline__ void rows_ipq_body(const uint64_t* __restrict__ d, long long d_stride, const GalF& G,
                                              const double* __restrict__ t2, const KeyPtrsF& keys, int ell, int beta,
                                              int batch, const double* __restrict__ t4,
                                              const uint64_t* __restrict__ add, long long add_stride,
                                              const uint64_t* __restrict__ acc_b, const uint64_t* __restrict__ acc_a,
                                              long long acc_stride, uint64_t* __restrict__ out_b,
                                              uint64_t* __restrict__ out_a, long long out_stride,
                                              const LevelConsts* __restrict__ lc, const DevTables& T, int lin,
                                              double* S, double* TW, int koff = 0,
                                              HoistSrc H = HoistSrc{nullptr, 1, 0}, const RsPost* post = nullptr) {
  const int nq = RS ? ell - 1 : ell;  // output limbs (the rescale drops q_{ell-1})
  const TileId id = decode_tile(batch, lin);
  if (id.tile >= 16 * nq) return;
  const int b = id.b, i = id.tile >> 4, rg = id.tile & 15;
  const uint32_t g = gal_of(G, koff + b);
  const double p = T.p[i], pinv = T.pinv[i];
  const double* v_b = t4 + ((long long)b * 2 * nq + i) * kN;
  const double* v_a = v_b + (long long)nq * kN;
  double sb[16], sa[16], x[16];
  uint64_t xr[16], kb[16], ka[16];
  const IpSrc I = ip_src<HOIST>(d, d_stride, t2, keys.k[koff + b], b, i, i, rg, ell, beta, T, H);
  {
    TwStage st;
    tw_issue(st, T.tw_fwd + (size_t)i * kN, rg);
    tile_ip_first<HOIST, true>(xr, x, kb, ka, I, i, rg, g, H, v_b);  // in flight across the staging barrier
    tw_store(st, TW);
    __syncthreads();
  }
  tile_ip_body<HOIST, true>(sb, sa, x, xr, kb, ka, I, i, rg, g, S, TW, v_b, p, pinv, true, H, true);
  const long long na = nat_a(rg);
  const TwPair pinv_P = lc->p_inv[i];
  if constexpr (RS) {
    // out = (IP P^-1 - v + sigma(add) + acc) q_{ell-1}^-1, v = NTT rows of (conv P^-1 + r)
    const TwPair ql_inv = lc->qlast_inv[i];
    const long long so = (long long)b * post->sub_stride + (long long)i * kN;
    const bool prod = post->a0 != nullptr;
    const long long ao = (long long)b * post->a_stride + (long long)i * kN;
    const long long bo = (long long)b * post->b_stride + (long long)i * kN;
    ipq_finish_rs(sb, x, v_a, add ? add + (long long)b * add_stride + (long long)i * kN : nullptr, g,
                  acc_b && !prod ? acc_b + (long long)b * acc_stride + (long long)i * kN : nullptr,
                  out_b + (long long)b * out_stride + (long long)i * kN + na, na, rg, S, TW, pinv_P, ql_inv, p, pinv,
                  post->sub_b ? post->sub_b + so : nullptr, post->twice != 0,
                  post->has_scalar ? u2d(post->scalar[i]) : 0.0, prod ? post->a0 + ao : nullptr,
                  prod ? post->b0 + bo : nullptr);
    ipq_finish_rs(sa, x, nullptr, nullptr, 1u,
                  acc_a && !prod ? acc_a + (long long)b * acc_stride + (long long)i * kN : nullptr,
                  out_a + (long long)b * out_stride + (long long)i * kN + na, na, rg, S, TW, pinv_P, ql_inv, p, pinv,
                  post->sub_a ? post->sub_a + so : nullptr, post->twice != 0, 0.0, prod ? post->a0 + ao : nullptr,
                  prod ? post->b1 + bo : nullptr, prod ? post->a1 + ao : nullptr, prod ? post->b0 + bo : nullptr);
    return;
  }
  ipq_finish(sb, x, v_a, add ? add + (long long)hoist_input<HOIST>(H, b) * add_stride + (long long)i * kN : nullptr, g,
             acc_b ? acc_b + (long long)b * acc_stride + (long long)i * kN : nullptr,
             out_b + (long long)b * out_stride + (long long)i * kN + na, na, rg, S, TW, pinv_P, p, pinv);
  ipq_finish(sa, x, nullptr, nullptr, 1u, acc_a ? acc_a + (long long)b * acc_stride + (long long)i * kN : nullptr,
             out_a + (long long)b * out_stride + (long long)i * kN + na, na, rg, S, TW, pinv_P, p, pinv);
}

// K3 for grouped extended-basis rotations: output o (one tile of it per workgroup) is
//   acc[o] + sum_m (P * sigma_m(add[b]) + IP_b(sigma_m(d[b])), IP_a(sigma_m(d[b])))   over b = m * outputs + o,
// the members m < group each with their own Galois element and key (the giant steps of one BSGS
// chunk for every input: the running sum stays in registers, so the extended accumulator is read
// and written once per group instead of once per member).  All outputs of a tile are dealt to one
// XCD, so a member's key tile is fetched from HBM once and shared from L2.  ext may alias acc.
__global__ __launch_bounds__(kT, 2) void k_ks_rows_ip_sum(const uint64_t* __restrict__ d, long long d_stride,
                                                       const GalF G, const double* __restrict__ t2, KeyPtrsF keys,
                                                       int ell, int beta, int outputs, int group, int tiles,
                                                       const uint64_t* __restrict__ add, long long add_stride,
                                                       uint64_t* ext_b, uint64_t* ext_a, long long ext_stride,
                                                       const uint64_t* acc_b, const uint64_t* acc_a,
                                                       long long acc_stride, DevTables T) {
  __shared__ double S[kRowLds];
  __shared__ double TW[kTwLds];
  const TileId id = decode_tile(outputs, blockIdx.x);
  if (id.tile >= tiles) return;
  const int o = id.b, e = id.tile >> 4, rg = id.tile & 15;
  const int L = T.L;
  const int pi = e < ell ? e : L + (e - ell);
  const double p = T.p[pi], pinv = T.pinv[pi];
  {
    TwStage st;
    tw_issue(st, T.tw_fwd + (size_t)pi * kN, rg);
    tw_store(st, TW);
    __syncthreads();
  }
  const long long na = nat_a(rg);
  double sb[16], sa[16], x[16];
  for (int m = 0; m < group; ++m) {
    const int b = m * outputs + o;
    const uint32_t g = gal_of(G, b);
    tile_ip(sb, sa, x, d, d_stride, g, t2, keys.k[b], b, e, pi, rg, ell, beta, S, TW, nullptr, p, pinv, T, m == 0);
    if (e < ell && add) {
      double ad[16];
      load_gal(ad, add + (long long)b * add_stride + (long long)e * kN, na, g);
      const TwPair pm = T.pmodq[pi];
#pragma unroll
      for (int k = 0; k < 16; ++k) sb[k] = reduce(sb[k] + mulc(ad[k], pm, p), p, pinv);  // back to p/2 + 1
    }
  }
  if (acc_b) {
    double ab[16], aa[16];
    load_gal(ab, acc_b + (long long)o * acc_stride + (long long)e * kN, na, 1u);
    load_gal(aa, acc_a + (long long)o * acc_stride + (long long)e * kN, na, 1u);
#pragma unroll
    for (int k = 0; k < 16; ++k) { sb[k] += ab[k]; sa[k] += aa[k]; }  // |sb| <= 1.5 p + 1
  }
  uint64_t* ob = ext_b + (long long)o * ext_stride + (long long)e * kN + na;
  uint64_t* oa = ext_a + (long long)o * ext_stride + (long long)e * kN + na;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    ob[16 * k] = d2u(canon(sb[k], p, pinv));
    oa[16 * k] = d2u(canon(sa[k], p, pinv));
  }
}

__global__ __launch_bounds__(kT, 2) void k_ks_rows_ipq(const uint64_t* __restrict__ d, long long d_stride, const GalF G,
                                                    const double* __restrict__ t2, KeyPtrsF keys, int ell, int beta,
                                                    int batch, const double* __restrict__ t4,
                                                    const uint64_t* __restrict__ add, long long add_stride,
                                                    const uint64_t* __restrict__ acc_b,
                                                    const uint64_t* __restrict__ acc_a, long long acc_stride,
                                                    uint64_t* __restrict__ out_b, uint64_t* __restrict__ out_a,
                                                    long long out_stride, const LevelConsts* __restrict__ lc,
                                                    DevTables T) {
  __shared__ double S[kRowLds];
  __shared__ double TW[kTwLds];
  rows_ipq_body(d, d_stride, G, t2, keys, ell, beta, batch, t4, add, add_stride, acc_b, acc_a, acc_stride, out_b, out_a,
                out_stride, lc, T, blockIdx.x, S, TW);
}

// K5 of the relinearisation fused with the rescale: Q limbs 0 .. ell - 2 (ipq_finish_rs).
__global__ __launch_bounds__(kT, 2) void k_ks_rows_ipq_rs(const uint64_t* __restrict__ d, long long d_stride,
                                                       const GalF G, const double* __restrict__ t2, KeyPtrsF keys,
                                                       int ell, int beta,
                                                       int batch, const double* __restrict__ t4,
                                                       const uint64_t* __restrict__ add, long long add_stride,
                                                       const uint64_t* __restrict__ acc_b,
                                                       const uint64_t* __restrict__ acc_a, long long acc_stride,
                                                       uint64_t* __restrict__ out_b, uint64_t* __restrict__ out_a,
                                                       long long out_stride, const LevelConsts* __restrict__ lc,
                                                       DevTables T, RsPost post) {
  __shared__ double S[kRowLds];
  __shared__ double TW[kTwLds];
  rows_ipq_body<false, true>(d, d_stride, G, t2, keys, ell, beta, batch, t4, add, add_stride, acc_b, acc_a,
                             acc_stride, out_b, out_a, out_stride, lc, T, blockIdx.x, S, TW, 0,
                             HoistSrc{nullptr, 1, 0}, &post);
}

// K5 of hoisted rotations: as k_ks_rows_ipq with the digits and inputs of HoistSrc.
__global__ __launch_bounds__(kT, 2) void k_ks_rows_ipq_h(const uint64_t* __restrict__ d, long long d_stride,
                                                      const GalF G, KeyPtrsF keys, int ell, int beta, int batch,
                                                      const double* __restrict__ t4, const uint64_t* __restrict__ add,
                                                      long long add_stride, uint64_t* __restrict__ out_b,
                                                      uint64_t* __restrict__ out_a, long long out_stride,
                                                      const LevelConsts* __restrict__ lc, DevTables T, HoistSrc H) {
  __shared__ double S[kRowLds];
  __shared__ double TW[kTwLds];
  rows_ipq_body<true>(d, d_stride, G, nullptr, keys, ell, beta, batch, t4, add, add_stride, nullptr, nullptr, 0, out_b,
                      out_a, out_stride, lc, T, blockIdx.x, S, TW, 0, H);
}

// The hoisted digits: the NTT rows pass of every ModUp output tile of T2, stored canonical in the
// natural layout at digits[b][j][e] (the own digit's limbs of digit j are skipped: d itself serves
// them).  Grid (16 (ell + K), beta, batch).
__global__ __launch_bounds__(kT) void k_ks_hoist_store(const double* __restrict__ t2, int ell, int beta,
                                                       uint64_t* __restrict__ digits, DevTables T) {
  __shared__ double S[kRowLds];
  const int e = blockIdx.x >> 4, rg = blockIdx.x & 15, j = blockIdx.y, b = blockIdx.z;
  if (e < ell && e / T.alpha == j) return;
  const int ext_l = ell + T.K;
  const int pi = e < ell ? e : T.L + (e - ell);
  const double p = T.p[pi], pinv = T.pinv[pi];
  const long long off = ((long long)(b * beta + j) * ext_l + e) * kN;
  double x[16];
  load_t(x, t2 + off, rg);
  rows_fwd_t(x, rg, S, T.tw_fwd + (size_t)pi * kN, p, pinv);
  uint64_t* o = digits + off + nat_a(rg);
#pragma unroll
  for (int k = 0; k < 16; ++k) o[16 * k] = d2u(canon(x[k], p, pinv));
}

// ----------------------------------------------------------------- ModDown / rescale finish
// Poly p = blockIdx.x: v = NTT rows of T4[p] (ell limbs); out = (x[p] - v) * inv[i] with x canonical
// u64: inv = P^-1 (ModDown of an extended-basis input) or q_last^-1 (rescale).
__global__ __launch_bounds__(kT) void k_ks_rows_finish(const double* __restrict__ t4, const uint64_t* __restrict__ xq,
                                                       long long xq_pstride, uint64_t* __restrict__ out,
                                                       long long out_pstride, int ell,
                                                       const TwPair* __restrict__ inv, DevTables T) {
  __shared__ double S[kRowLds];
  const int i = blockIdx.z, rg = blockIdx.y, pl = blockIdx.x;
  const double p = T.p[i], pinv = T.pinv[i];
  const double* __restrict__ tw = T.tw_fwd + (size_t)i * kN;
  const long long na = nat_a(rg);
  double a[16], x[16];
  const uint64_t* ap = xq + (long long)pl * xq_pstride + (long long)i * kN + na;
#pragma unroll
  for (int k = 0; k < 16; ++k) a[k] = u2d(ap[16 * k]);
  load_t(x, t4 + ((long long)pl * ell + i) * kN, rg);
  rows_fwd_t(x, rg, S, tw, p, pinv);
  const TwPair pi_ = inv[i];
  uint64_t* o = out + (long long)pl * out_pstride + (long long)i * kN + na;
#pragma unroll
  for (int k = 0; k < 16; ++k) o[16 * k] = d2u(canon(mulc(a[k] - x[k], pi_, p), p, pinv));  // |a - x| <= 4.9 p
}

// ----------------------------------------------------------------- NTT rows + canonical store
// Poly p = blockIdx.x, limb i = blockIdx.z of an ell-limb workspace poly: out limb (limb0 + i) of
// poly p = canonical NTT rows pass of T4[p][i] under prime prime0 + i.
__global__ __launch_bounds__(kT) void k_ks_rows_store(const double* __restrict__ t4, int ell,
                                                      uint64_t* __restrict__ out, long long out_pstride, int limb0,
                                                      int prime0, DevTables T) {
  __shared__ double S[kRowLds];
  const int i = blockIdx.z, rg = blockIdx.y, pl = blockIdx.x;
  const int pi = prime0 + i;
  const double p = T.p[pi], pinv = T.pinv[pi];
  const double* __restrict__ tw = T.tw_fwd + (size_t)pi * kN;
  const long long na = nat_a(rg);
  double x[16];
  load_t(x, t4 + ((long long)pl * ell + i) * kN, rg);
  rows_fwd_t(x, rg, S, tw, p, pinv);
  uint64_t* o = out + (long long)pl * out_pstride + (long long)(limb0 + i) * kN + na;
#pragma unroll
  for (int k = 0; k < 16; ++k) o[16 * k] = d2u(canon(x[k], p, pinv));
}

}  // namespace

// Workspace (doubles, per ciphertext): R1 = T1 / T4 [2 ell limbs], T2 [beta (ell + K)], ACCP [2 K].
size_t ks_fused_bytes(const hck_context* c, int ell, int batch) {
  if (c->wide) return wide_ks_bytes(c, ell, batch);
  const size_t beta = beta_of(c, ell), ext_l = ell + c->K;
  return (size_t)batch * kN * 8 * (2 * ell + beta * ext_l + 2 * c->K);
}

int ks_fused(const hck_context* c, int ell, int batch, const uint64_t* d, long long d_stride, uint32_t galois,
             const uint64_t* const* ksk, const uint64_t* add, long long add_stride, const uint64_t* acc_b,
             const uint64_t* acc_a, long long acc_stride, uint64_t* out_b, uint64_t* out_a, long long out_stride,
             char* ws, hipStream_t s, uint64_t* ext_b, uint64_t* ext_a, long long ext_stride,
             const uint32_t* galois_items) {
  if (c->wide)
    return wide_ks(c, ell, batch, d, d_stride, galois, ksk, add, add_stride, acc_b, acc_a, acc_stride, out_b, out_a,
                   out_stride, ws, s, ext_b, ext_a, ext_stride, galois_items);
  if (c->alpha > kSrcMax || c->K > kSrcMax) return HCK_ERR_UNSUPPORTED;
  if (batch > kMaxBatchF) return HCK_ERR_ARG;
  GalF G = gal_uniform(galois);
  if (galois_items) {
    G.per_item = 1;
    for (int b = 0; b < batch; ++b) G.g[b] = galois_items[b];
  }
  const int K = c->K, beta = beta_of(c, ell), ext_l = ell + K;
  const long long n = kN;
  double* r1 = (double*)ws;
  double* t2 = r1 + (long long)batch * 2 * ell * n;
  double* accp = t2 + (long long)batch * beta * ext_l * n;
  // Targets of digit j: ext_l minus the digit's own limbs; the last digit is the smallest.
  const int last_digit = ell - c->alpha * (beta - 1);
  KeyPtrsF kp{};
  for (int b = 0; b < batch; ++b) kp.k[b] = ksk[b];
  // K1
  k_ks_intt_rows<<<dim3(((16 * ell + kXcds - 1) / kXcds) * kXcds * batch), kT, 0, s>>>(d, d_stride, G, 0, 0,
                                                                                    r1, ell, batch, c->dev);
  HCK_CHECK_LAUNCH();
  // K2: ModUp, one block per (column pair, digit, ciphertext)
  launch_conv(c,
              ConvArgs{r1, (long long)ell * n, 0, c->alpha, t2, (long long)beta * ext_l * n, (long long)ext_l * n,
                       modup_consts(c, ell, 0), 1},
              dim3(128, beta, batch), ext_l - last_digit, s);
  HCK_CHECK_LAUNCH();
  if (ext_b) {
    // K3 over every extended limb, ending in the extended basis
    const int tiles = 16 * ext_l, groups = (tiles + kXcds - 1) / kXcds;
    k_ks_rows_ip<<<dim3(groups * kXcds * batch), kT, 0, s>>>(d, d_stride, G, t2, kp, ell, beta, batch, tiles,
                                                            0, nullptr, add, add_stride, ext_b, ext_a, ext_stride,
                                                            acc_b, acc_a, acc_stride, c->dev);
    HCK_CHECK_LAUNCH();
    return HCK_OK;
  }
  // K3 over the K special limbs
  {
    const int tiles = 16 * K, groups = (tiles + kXcds - 1) / kXcds;
    k_ks_rows_ip<<<dim3(groups * kXcds * batch), kT, 0, s>>>(d, d_stride, G, t2, kp, ell, beta, batch, tiles,
                                                            ell, accp, nullptr, 0, nullptr, nullptr, 0, nullptr,
                                                            nullptr, 0, c->dev);
    HCK_CHECK_LAUNCH();
  }
  // K4: ModDown conversion, one block per (column pair, component, ciphertext); T4 reuses R1
  double* t4 = r1;
  launch_conv(c,
              ConvArgs{accp, 2LL * K * n, (long long)K * n, 0, t4, 2LL * ell * n, (long long)ell * n,
                       c->d_moddown + ell, 0},
              dim3(128, 2, batch), ell, s);
  HCK_CHECK_LAUNCH();
  // K5: Q limbs
  {
    const int tiles = 16 * ell, groups = (tiles + kXcds - 1) / kXcds;
    k_ks_rows_ipq<<<dim3(groups * kXcds * batch), kT, 0, s>>>(d, d_stride, G, t2, kp, ell, beta, batch, t4,
                                                             add, add_stride, acc_b, acc_a, acc_stride, out_b,
                                                             out_a, out_stride, c->d_level + ell, c->dev);
    HCK_CHECK_LAUNCH();
  }
  return HCK_OK;
}

size_t ks_rs_bytes(const hck_context* c, int ell, int batch) {
  if (c->wide) return wide_fused_rs_bytes(c, ell, batch);
  const size_t beta = beta_of(c, ell), ext_l = ell + c->K;
  return (size_t)batch * kN * 8 * (2 * ell + beta * ext_l + 2 * (c->K + 1));
}

int ks_rescaled(const hck_context* c, int ell, int batch, const uint64_t* d, long long d_stride, uint32_t galois,
                const uint64_t* const* ksk, const uint64_t* add, long long add_stride, const uint64_t* acc_b,
                const uint64_t* acc_a, long long acc_stride, uint64_t* out_b, uint64_t* out_a, long long out_stride,
                char* ws, hipStream_t s, int twice, const uint64_t* sub_b, const uint64_t* sub_a,
                long long sub_stride, const uint64_t* scalar, const uint64_t* const* prod_ab, long long a_stride,
                long long b_stride) {
  if (c->wide)
    return wide_ks_rescaled(c, ell, batch, d, d_stride, galois, ksk, add, add_stride, acc_b, acc_a, acc_stride, out_b,
                            out_a, out_stride, ws, s, twice, sub_b, sub_a, sub_stride, scalar, prod_ab, a_stride,
                            b_stride);
  if (c->conv_engine != 1 || ell < 2) return HCK_ERR_UNSUPPORTED;
  if (c->alpha > kSrcMax || c->K > kSrcMax) return HCK_ERR_UNSUPPORTED;
  if (batch < 1 || batch > kMaxBatchF || (acc_b == nullptr) != (acc_a == nullptr)) return HCK_ERR_ARG;
  const GalF G = gal_uniform(galois);
  const int K = c->K, beta = beta_of(c, ell), ext_l = ell + K, nq = ell - 1;
  const long long n = kN;
  double* r1 = (double*)ws;
  double* t2 = r1 + (long long)batch * 2 * ell * n;
  double* accp = t2 + (long long)batch * beta * ext_l * n;  // [batch][2][K + 1]: q_{ell-1}, then P
  const int last_digit = ell - c->alpha * (beta - 1);
  KeyPtrsF kp{};
  for (int b = 0; b < batch; ++b) kp.k[b] = ksk[b];
  // K1, K2 as in ks_fused
  k_ks_intt_rows<<<dim3(((16 * ell + kXcds - 1) / kXcds) * kXcds * batch), kT, 0, s>>>(d, d_stride, G, 0, 0,
                                                                                    r1, ell, batch, c->dev);
  HCK_CHECK_LAUNCH();
  launch_conv(c,
              ConvArgs{r1, (long long)ell * n, 0, c->alpha, t2, (long long)beta * ext_l * n, (long long)ext_l * n,
                       modup_consts(c, ell, 0), 1},
              dim3(128, beta, batch), ext_l - last_digit, s);
  HCK_CHECK_LAUNCH();
  // K3 over q_{ell-1} and the K special limbs
  {
    const int tiles = 16 * (K + 1), groups = (tiles + kXcds - 1) / kXcds;
    k_ks_rows_ip<<<dim3(groups * kXcds * batch), kT, 0, s>>>(d, d_stride, G, t2, kp, ell, beta, batch, tiles,
                                                            ell - 1, accp, add, add_stride, nullptr, nullptr, 0, acc_b,
                                                            acc_a, acc_stride, c->dev);
    HCK_CHECK_LAUNCH();
  }
  // K4: ModDown + rescale conversion to the ell - 1 lower limbs; T4 reuses R1
  double* t4 = r1;
  {
    const ConvArgs A{accp + n, 2LL * (K + 1) * n, (long long)(K + 1) * n, 0, t4, 2LL * nq * n, (long long)nq * n,
                     c->d_mdrs + ell, 0, accp};
    if (nq <= 16) k_ks_cols_mconv_rs<false, 2><<<dim3(128, 2, batch), kT, 0, s>>>(A, c->dev);
    else if (nq <= kMPass) k_ks_cols_mconv_rs<false><<<dim3(128, 2, batch), kT, 0, s>>>(A, c->dev);
    else k_ks_cols_mconv_rs<true><<<dim3(128, 2, batch), kT, 0, s>>>(A, c->dev);
    HCK_CHECK_LAUNCH();
  }
  // K5: Q limbs 0 .. ell - 2
  {
    const int tiles = 16 * nq, groups = (tiles + kXcds - 1) / kXcds;
    RsPost post{};
    post.sub_b = sub_b;
    post.sub_a = sub_a;
    post.sub_stride = sub_stride;
    post.twice = twice;
    post.has_scalar = scalar != nullptr;
    for (int i = 0; scalar && i < nq; ++i) post.scalar[i] = scalar[i];
    if (prod_ab) {
      post.a0 = prod_ab[0];
      post.a1 = prod_ab[1];
      post.b0 = prod_ab[2];
      post.b1 = prod_ab[3];
      post.a_stride = a_stride;
      post.b_stride = b_stride;
    }
    k_ks_rows_ipq_rs<<<dim3(groups * kXcds * batch), kT, 0, s>>>(d, d_stride, G, t2, kp, ell, beta, batch, t4,
                                                                add, add_stride, acc_b, acc_a, acc_stride, out_b,
                                                                out_a, out_stride, c->d_level + ell, c->dev, post);
    HCK_CHECK_LAUNCH();
  }
  return HCK_OK;
}

// Grouped extended-basis rotations (k_ks_rows_ip_sum): item b = m * outputs + o of d / add (Galois
// element galois_items[b], key ksk[b]) is member m of output o.  K1 and K2 run over every item, as
// in ks_fused; the workspace is ks_fused_bytes(c, ell, outputs * group).
int ks_fused_sum(const hck_context* c, int ell, int outputs, int group, const uint64_t* d, long long d_stride,
                 const uint32_t* galois_items, const uint64_t* const* ksk, const uint64_t* add, long long add_stride,
                 const uint64_t* acc_b, const uint64_t* acc_a, long long acc_stride, uint64_t* ext_b,
                 uint64_t* ext_a, long long ext_stride, char* ws, hipStream_t s) {
  const int batch = outputs * group;
  if (outputs < 1 || group < 1 || batch > kMaxBatchF) return HCK_ERR_ARG;
  if (c->wide && wide_fused_ok(c))
    return wide_ks_fused_sum(c, ell, outputs, group, d, d_stride, galois_items, ksk, add, add_stride, acc_b, acc_a,
                             acc_stride, ext_b, ext_a, ext_stride, ws, s);
  if (c->wide) {
    // one member at a time, each accumulated into the extended outputs (same residues)
    for (int m = 0; m < group; ++m) {
      const uint64_t* keys[kMaxBatchF];
      uint32_t gals[kMaxBatchF];
      for (int o = 0; o < outputs; ++o) {
        keys[o] = ksk[m * outputs + o];
        gals[o] = galois_items[m * outputs + o];
      }
      const long long off = (long long)m * outputs;
      const int rc = wide_ks(c, ell, outputs, d + off * d_stride, d_stride, 1u, keys,
                             add ? add + off * add_stride : nullptr, add_stride, m ? ext_b : acc_b, m ? ext_a : acc_a,
                             m ? ext_stride : acc_stride, nullptr, nullptr, 0, ws, s, ext_b, ext_a, ext_stride, gals);
      if (rc) return rc;
    }
    return HCK_OK;
  }
  if (c->alpha > kSrcMax || c->K > kSrcMax) return HCK_ERR_UNSUPPORTED;
  GalF G{};
  G.per_item = 1;
  KeyPtrsF kp{};
  for (int b = 0; b < batch; ++b) {
    G.g[b] = galois_items[b];
    kp.k[b] = ksk[b];
  }
  const int K = c->K, beta = beta_of(c, ell), ext_l = ell + K;
  const long long n = kN;
  double* r1 = (double*)ws;
  double* t2 = r1 + (long long)batch * 2 * ell * n;
  const int last_digit = ell - c->alpha * (beta - 1);
  k_ks_intt_rows<<<dim3(((16 * ell + kXcds - 1) / kXcds) * kXcds * batch), kT, 0, s>>>(d, d_stride, G, 0, 0,
                                                                                    r1, ell, batch, c->dev);
  HCK_CHECK_LAUNCH();
  launch_conv(c,
              ConvArgs{r1, (long long)ell * n, 0, c->alpha, t2, (long long)beta * ext_l * n, (long long)ext_l * n,
                       modup_consts(c, ell, 0), 1},
              dim3(128, beta, batch), ext_l - last_digit, s);
  HCK_CHECK_LAUNCH();
  const int tiles = 16 * ext_l, groups = (tiles + kXcds - 1) / kXcds;
  k_ks_rows_ip_sum<<<dim3(groups * kXcds * outputs), kT, 0, s>>>(d, d_stride, G, t2, kp, ell, beta, outputs, group,
                                                                tiles, add, add_stride, ext_b, ext_a, ext_stride,
                                                                acc_b, acc_a, acc_stride, c->dev);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

// ----------------------------------------------------------------- hoisted rotations
// ks_hoist: the extended digits of `inputs` polynomials d (NTT domain, no automorphism) in the full
// NTT domain, canonical u64 [inputs][beta][ell + K] limbs (the own digit's limbs of each digit are
// left unwritten); workspace T1 + T2 as in ks_fused.
size_t ks_hoist_bytes(const hck_context* c, int ell, int inputs) {
  if (c->wide) return wide_hoist_bytes(c, ell, inputs);
  const size_t beta = beta_of(c, ell), ext_l = ell + c->K;
  const size_t per = inputs < kMaxBatchF ? inputs : kMaxBatchF;
  return per * kN * 8 * (ell + beta * ext_l);
}

int ks_hoist(const hck_context* c, int ell, int inputs, const uint64_t* d, long long d_stride, uint64_t* digits,
             char* ws, hipStream_t s) {
  if (c->wide) return wide_hoist(c, ell, inputs, d, d_stride, digits, ws, s);
  if (c->alpha > kSrcMax || c->K > kSrcMax) return HCK_ERR_UNSUPPORTED;
  const int K = c->K, beta = beta_of(c, ell), ext_l = ell + K;
  const long long n = kN;
  const int per = inputs < kMaxBatchF ? inputs : kMaxBatchF;
  double* t1 = (double*)ws;
  double* t2 = t1 + (long long)per * ell * n;
  const int last_digit = ell - c->alpha * (beta - 1);
  for (int b0 = 0; b0 < inputs; b0 += kMaxBatchF) {
    const int nb = inputs - b0 < kMaxBatchF ? inputs - b0 : kMaxBatchF;
    k_ks_intt_rows<<<dim3(((16 * ell + kXcds - 1) / kXcds) * kXcds * nb), kT, 0, s>>>(
        d + (long long)b0 * d_stride, d_stride, gal_uniform(1u), 0, 0, t1, ell, nb, c->dev);
    HCK_CHECK_LAUNCH();
    launch_conv(c,
                ConvArgs{t1, (long long)ell * n, 0, c->alpha, t2, (long long)beta * ext_l * n, (long long)ext_l * n,
                         modup_consts(c, ell, 0), 1},
                dim3(128, beta, nb), ext_l - last_digit, s);
    HCK_CHECK_LAUNCH();
    k_ks_hoist_store<<<dim3(16 * ext_l, beta, nb), kT, 0, s>>>(t2, ell, beta,
                                                                digits + (long long)b0 * beta * ext_l * n, c->dev);
    HCK_CHECK_LAUNCH();
  }
  return HCK_OK;
}

// ks_hoisted: item i (< items) = rotation of input i % inputs by galois[i] with key ksk[i], from its
// hoisted digits: (sigma(c0) + KS_b(sigma(c1)), KS_a(sigma(c1))) over ell limbs, bit-identical to
// ks_fused with that Galois element (ModUp commutes with sigma).  Workspace T4 + ACCP per item of
// a launch (at most kMaxBatchF items each).
size_t ks_hoisted_bytes(const hck_context* c, int ell, int items) {
  if (c->wide) return wide_hoisted_bytes(c, ell, items);
  const int per = items < kMaxBatchF ? items : kMaxBatchF;
  return (size_t)per * kN * 8 * (2 * ell + 2 * c->K);
}

int ks_hoisted(const hck_context* c, int ell, int inputs, int items, const uint32_t* galois,
               const uint64_t* const* ksk, const uint64_t* c0, const uint64_t* c1, long long in_stride,
               const uint64_t* digits, uint64_t* out_b, uint64_t* out_a, long long out_stride, char* ws,
               hipStream_t s) {
  if (c->wide)
    return wide_hoisted(c, ell, inputs, items, galois, ksk, c0, c1, in_stride, digits, out_b, out_a, out_stride, ws,
                        s);
  if (c->alpha > kSrcMax || c->K > kSrcMax) return HCK_ERR_UNSUPPORTED;
  const int K = c->K, beta = beta_of(c, ell);
  const long long n = kN;
  for (int i0 = 0; i0 < items; i0 += kMaxBatchF) {
    const int nb = items - i0 < kMaxBatchF ? items - i0 : kMaxBatchF;
    GalF G{};
    G.per_item = 1;
    KeyPtrsF kp{};
    for (int b = 0; b < nb; ++b) {
      G.g[b] = galois[i0 + b];
      kp.k[b] = ksk[i0 + b];
    }
    const HoistSrc H{digits, inputs, i0 % inputs};
    double* t4 = (double*)ws;
    double* accp = t4 + (long long)nb * 2 * ell * n;
    {
      const int tiles = 16 * K, groups = (tiles + kXcds - 1) / kXcds;
      k_ks_rows_ip_h<<<dim3(groups * kXcds * nb), kT, 0, s>>>(c1, in_stride, G, kp, ell, beta, nb, accp, c->dev, H);
      HCK_CHECK_LAUNCH();
    }
    launch_conv(c,
                ConvArgs{accp, 2LL * K * n, (long long)K * n, 0, t4, 2LL * ell * n, (long long)ell * n,
                         c->d_moddown + ell, 0},
                dim3(128, 2, nb), ell, s);
    HCK_CHECK_LAUNCH();
    {
      const int tiles = 16 * ell, groups = (tiles + kXcds - 1) / kXcds;
      k_ks_rows_ipq_h<<<dim3(groups * kXcds * nb), kT, 0, s>>>(c1, in_stride, G, kp, ell, beta, nb, t4, c0, in_stride,
                                                             out_b + (long long)i0 * out_stride,
                                                             out_a + (long long)i0 * out_stride, out_stride,
                                                             c->d_level + ell, c->dev, H);
      HCK_CHECK_LAUNCH();
    }
  }
  return HCK_OK;
}

size_t moddown_bytes(const hck_context* c, int ell, int polys) {
  if (c->wide) return wide_moddown_bytes(c, ell, polys);
  return (size_t)polys * kN * 8 * (size_t)(c->K + ell);
}

// ModDown of extended-basis polys in[p] ([ell + K] canonical NTT-domain limbs, Q first):
// out[p] = (x_Q - NTT(conv(INTT(x_P)))) * P^-1 over the ell Q primes.
int moddown_ext(const hck_context* c, int ell, int polys, const uint64_t* in, long long in_stride, uint64_t* out,
                long long out_stride, char* ws, hipStream_t s) {
  if (c->wide) return wide_moddown(c, ell, polys, in, in_stride, out, out_stride, ws, s);
  if (c->K > kSrcMax) return HCK_ERR_UNSUPPORTED;
  const int K = c->K;
  const long long n = kN;
  double* tp = (double*)ws;                       // [polys][K] workspace layout
  double* t4 = tp + (long long)polys * K * n;     // [polys][ell] workspace layout
  k_ks_intt_rows<<<dim3(((16 * K + kXcds - 1) / kXcds) * kXcds * polys), kT, 0, s>>>(in, in_stride, gal_uniform(1u), ell, c->L,
                                                                                   tp, K, polys, c->dev);
  HCK_CHECK_LAUNCH();
  launch_conv(c, ConvArgs{tp, (long long)K * n, 0, 0, t4, (long long)ell * n, 0, c->d_moddown + ell, 0},
              dim3(128, 1, polys), ell, s);
  HCK_CHECK_LAUNCH();
  k_ks_rows_finish<<<dim3(polys, 16, ell), kT, 0, s>>>(t4, in, in_stride, out, out_stride, ell,
                                                       (c->d_level + ell)->p_inv, c->dev);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

size_t rescale_bytes(const hck_context* c, int ell, int polys) {
  if (c->wide) return wide_rescale_bytes(c, ell, polys);
  return (size_t)polys * kN * 8 * (size_t)ell;
}

// Rescale = ModDown with q_{ell-1} as the one special prime: INTT rows of the last limb, then the
// cols kernel (INTT cols, centered lift, spread to the ell - 1 lower primes, NTT cols), then the
// finish kernel with q_{ell-1}^-1.  The spread limbs cross HBM once (the two-pass NTT of a separate
// spread would move them three times).
int rescale_fused(const hck_context* c, int ell, int polys, const uint64_t* in, long long in_stride, uint64_t* out,
                  long long out_stride, char* ws, hipStream_t s) {
  if (c->wide) return wide_rescale(c, ell, polys, in, in_stride, out, out_stride, ws, s);
  const long long n = kN;
  const int nt = ell - 1;
  double* tl = (double*)ws;                       // [polys][1] workspace layout
  double* t4 = tl + (long long)polys * n;         // [polys][ell - 1] workspace layout
  k_ks_intt_rows<<<dim3(((16 + kXcds - 1) / kXcds) * kXcds * polys), kT, 0, s>>>(in, in_stride, gal_uniform(1u), ell - 1,
                                                                                ell - 1, tl, 1, polys, c->dev);
  HCK_CHECK_LAUNCH();
  auto conv = nt <= kTgtFused ? k_ks_cols_conv<false> : k_ks_cols_conv<true>;
  conv<<<dim3(128, 1, polys), kT, 0, s>>>(ConvArgs{tl, n, 0, 0, t4, (long long)nt * n, 0, c->d_rescale + ell, 0},
                                          c->dev);
  HCK_CHECK_LAUNCH();
  k_ks_rows_finish<<<dim3(polys, 16, nt), kT, 0, s>>>(t4, in, in_stride, out, out_stride, nt,
                                                      (c->d_level + ell)->qlast_inv, c->dev);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

// ----------------------------------------------------------------- linear combination + rescale
// out[g] = rescale(sum_t w[t] x[g][t]) (+ the residues add[] on the groups of add_mask), the
// Paterson-Stockmeyer step "c0 + sum c_j T_j, rescaled": the combination is formed in the two
// kernels that read it (the last limb's INTT rows, and the finish over the other limbs), so it is
// never stored.  The residues equal hck_lincomb followed by hck_rescale and a scalar add.
struct LcRsArgs {
  const uint64_t* x[kLcRsPtrs];  // group-major: x[g * terms + t], limb i at x + i N
  uint64_t* out[kLcRsGroups];    // limb i < ell - 1 at out + i N
  uint64_t add[kMaxPrimes];      // per output limb
};

// the combination of limb `limb` of group g's terms for row group rg, natural layout (reduced to
// within p/2 + 1): weights w[t][limb] ([terms][ell]), reduced every 7 terms (|acc| < 8 p)
__device__ __forceinline__ void lc_tile(double (&acc)[16], const LcRsArgs& A, int g, int terms,
                                        const uint64_t* __restrict__ w, int ell, int limb, long long na, double p,
                                        double pinv) {
#pragma unroll
  for (int k = 0; k < 16; ++k) acc[k] = 0.0;
  for (int t = 0; t < terms; ++t) {
    const uint64_t* xl = A.x[g * terms + t] + (long long)limb * kN + na;
    const double wt = u2d(w[(long long)t * ell + limb]);
#pragma unroll
    for (int k = 0; k < 16; ++k) acc[k] += mulv(u2d(xl[16 * k]), wt, p, pinv);  // |term| <= 0.875 p
    if (t % 7 == 6) {
#pragma unroll
      for (int k = 0; k < 16; ++k) acc[k] = reduce(acc[k], p, pinv);
    }
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) acc[k] = reduce(acc[k], p, pinv);
}

// INTT rows of the combination's last limb (ell - 1) of every group, to the workspace layout.
// Grid (16, groups).
__global__ __launch_bounds__(kT) void k_lc_intt_last(const LcRsArgs A, int terms, const uint64_t* __restrict__ w,
                                                     int ell, double* __restrict__ tl, DevTables T) {
  __shared__ double S[kRowLds];
  const int rg = blockIdx.x, g = blockIdx.y, pi = ell - 1;
  const double p = T.p[pi], pinv = T.pinv[pi];
  double x[16];
  lc_tile(x, A, g, terms, w, ell, pi, nat_a(rg), p, pinv);
  // lc_tile reads the natural layout; rows_inv_to_t takes the values in map N, which nat_a indexes
  rows_inv_to_t(x, tl + (long long)g * kN, rg, S, T.tw_inv + (size_t)pi * kN, p, pinv);
}

// The finish: out[g][i] = (sum_t w[t][i] x[g][t][i] - NTT rows(T4[g][i])) q_{ell-1}^-1 (+ add[i]).
// Grid (groups, 16, ell - 1).
__global__ __launch_bounds__(kT) void k_lc_finish(const LcRsArgs A, int terms, const uint64_t* __restrict__ w,
                                                  int ell, const double* __restrict__ t4, uint64_t add_mask,
                                                  const TwPair* __restrict__ ql_inv, DevTables T) {
  __shared__ double S[kRowLds];
  const int g = blockIdx.x, rg = blockIdx.y, i = blockIdx.z, nt = ell - 1;
  const double p = T.p[i], pinv = T.pinv[i];
  const long long na = nat_a(rg);
  double a[16], x[16];
  load_t(x, t4 + ((long long)g * nt + i) * kN, rg);
  lc_tile(a, A, g, terms, w, ell, i, na, p, pinv);
  rows_fwd_t(x, rg, S, T.tw_fwd + (size_t)i * kN, p, pinv);
  const TwPair qi = ql_inv[i];
  const double ad = ((add_mask >> g) & 1ull) ? u2d(A.add[i]) : 0.0;
  uint64_t* o = A.out[g] + (long long)i * kN + na;
#pragma unroll
  for (int k = 0; k < 16; ++k) o[16 * k] = d2u(canon(mulc(a[k] - x[k], qi, p) + ad, p, pinv));  // |a - x| <= 4.9 p
}

size_t lincomb_rescale_bytes(const hck_context* c, int ell, int groups) {
  (void)c;
  return (size_t)groups * kN * 8 * (size_t)ell;
}

int lincomb_rescale(const hck_context* c, int ell, int groups, int terms, const uint64_t* const* x,
                    const uint64_t* w, uint64_t* const* out, const uint64_t* add, uint64_t add_mask, char* ws,
                    hipStream_t s) {
  if (c->wide) return HCK_ERR_UNSUPPORTED;
  if (ell < 2 || groups < 1 || groups > kLcRsGroups || terms < 1 || groups * terms > kLcRsPtrs || !w)
    return HCK_ERR_ARG;
  LcRsArgs A{};
  for (int j = 0; j < groups * terms; ++j) A.x[j] = x[j];
  for (int g = 0; g < groups; ++g) A.out[g] = out[g];
  for (int i = 0; i < ell - 1; ++i) A.add[i] = add ? add[i] : 0;
  if (!add) add_mask = 0;
  const long long n = kN;
  double* tl = (double*)ws;                    // [groups][1] workspace layout
  double* t4 = tl + (long long)groups * n;     // [groups][ell - 1] workspace layout
  k_lc_intt_last<<<dim3(16, groups), kT, 0, s>>>(A, terms, w, ell, tl, c->dev);
  HCK_CHECK_LAUNCH();
  const int nt = ell - 1;
  auto conv = nt <= kTgtFused ? k_ks_cols_conv<false> : k_ks_cols_conv<true>;
  conv<<<dim3(128, 1, groups), kT, 0, s>>>(ConvArgs{tl, n, 0, 0, t4, (long long)nt * n, 0, c->d_rescale + ell, 0},
                                           c->dev);
  HCK_CHECK_LAUNCH();
  k_lc_finish<<<dim3(groups, 16, nt), kT, 0, s>>>(A, terms, w, ell, t4, add_mask, (c->d_level + ell)->qlast_inv,
                                                  c->dev);
  HCK_CHECK_LAUNCH();
  return HCK_OK;
}

size_t modraise_bytes(const hck_context* c, int to, int polys) {
  if (c->wide) return wide_modraise_bytes(c, to, polys);
  return (size_t)polys * kN * 8 * (size_t)to;
}

// ModRaise on the conversion kernels: INTT rows of limb 0, the cols kernel (INTT cols, centered
// lift, spread to q_1 .. q_{to-1}, NTT cols), NTT rows with a canonical store; limb 0 itself is
// unchanged (the lift is congruent to it modulo q_0) and copied.
int modraise_fused(const hck_context* c, int to, int polys, const uint64_t* in, long long in_stride, uint64_t* out,
                   long long out_stride, char* ws, hipStream_t s) {
  if (c->wide) return wide_modraise(c, to, polys, in, in_stride, out, out_stride, ws, s);
  const long long n = kN;
  const int nt = to - 1;
  double* tl = (double*)ws;                       // [polys][1] workspace layout
  double* t4 = tl + (long long)polys * n;         // [polys][to - 1] workspace layout
  k_ks_intt_rows<<<dim3(((16 + kXcds - 1) / kXcds) * kXcds * polys), kT, 0, s>>>(in, in_stride, gal_uniform(1u), 0, 0, tl, 1,
                                                                                polys, c->dev);
  HCK_CHECK_LAUNCH();
  auto conv = nt <= kTgtFused ? k_ks_cols_conv<false> : k_ks_cols_conv<true>;
  conv<<<dim3(128, 1, polys), kT, 0, s>>>(ConvArgs{tl, n, 0, 0, t4, (long long)nt * n, 0, c->d_raise + to, 0},
                                          c->dev);
  HCK_CHECK_LAUNCH();
  k_ks_rows_store<<<dim3(polys, 16, nt), kT, 0, s>>>(t4, nt, out, out_stride, 1, 1, c->dev);
  HCK_CHECK_LAUNCH();
  // a single poly may come with any item stride (0 included): its pitch is then the row itself
  const size_t row = (size_t)n * 8;
  const size_t dp = polys > 1 ? (size_t)out_stride * 8 : row, sp = polys > 1 ? (size_t)in_stride * 8 : row;
  hipError_t e = hipMemcpy2DAsync(out, dp, in, sp, row, polys, hipMemcpyDeviceToDevice, s);
  return e == hipSuccess ? HCK_OK : (int)e;
}

}  // namespace hck
